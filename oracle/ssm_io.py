"""CPU restatement of the SSM block's input / output stages around the scan.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Follows modules/ssm.py (SSM.forward :98-152, SSM.step :156-204) and
inference/ssm_cache.py (build_conv_ctx :8-36, update :38-43):

* prologue (:116-118): silu, then nn.Conv1d(groups=channels, padding=K-1)
  sliced to seq_len -- a causal depthwise conv over zero history:
      xBC[b,t,c] = bias[c] + sum_j w[c,j] silu(hBC[b, t-K+1+j, c]);
  then the split into x, B, C (:120-125);
* epilogue (:144-150): out = (y + D x) silu(gate);
* decode (:173-182, ssm_cache.py:38-43): roll the (b, channels, K) context
  left, write the new raw row last, out = bias + sum_j w[:,j] silu(ctx[:,:,j]).

The backward formulas are written out by hand (the reference gets them from
torch autograd).  Tensors here are (b, L, channels), the reference's layout
before its transpose to (b, channels, L) for Conv1d.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def silu(z):
    return z * torch.sigmoid(z)


def dsilu(z):
    s = torch.sigmoid(z)
    return s * (1 + z * (1 - s))


def conv_forward(hbc, w, bias=None, dtype=torch.float64):
    """xBC (b, L, channels) in `dtype`.  w (channels, K) or (channels, 1, K)."""
    w = w.reshape(w.shape[0], w.shape[-1]).to(dtype)
    K = w.shape[1]
    s = silu(hbc.to(dtype))
    b, L, ch = s.shape
    pad = torch.cat([torch.zeros(b, K - 1, ch, dtype=dtype), s], dim=1)   # zero history
    out = torch.zeros(b, L, ch, dtype=dtype)
    for j in range(K):
        out = out + w[:, j] * pad[:, j:j + L]                             # row t + j of pad = t-K+1+j
    if bias is not None:
        out = out + bias.to(dtype)
    return out


def split(xbc, x_dim, bc_dim):
    return xbc[..., :x_dim], xbc[..., x_dim:x_dim + bc_dim], xbc[..., x_dim + bc_dim:]


def conv_backward(hbc, w, g, dtype=torch.float64):
    """(dhbc, dw (channels, K), dbias) for the upstream gradient g = d xBC."""
    w = w.reshape(w.shape[0], w.shape[-1]).to(dtype)
    K = w.shape[1]
    h = hbc.to(dtype)
    g = g.to(dtype)
    b, L, ch = h.shape
    s = silu(h)
    gpad = torch.cat([g, torch.zeros(b, K - 1, ch, dtype=dtype)], dim=1)   # g[s + K - 1 - j]
    acc = torch.zeros(b, L, ch, dtype=dtype)
    for j in range(K):
        acc = acc + w[:, j] * gpad[:, K - 1 - j:K - 1 - j + L]
    dh = acc * dsilu(h)
    spad = torch.cat([torch.zeros(b, K - 1, ch, dtype=dtype), s], dim=1)
    dw = torch.stack([(g * spad[:, j:j + L]).sum((0, 1)) for j in range(K)], dim=1)
    db = g.sum((0, 1))
    return dh, dw, db


def build_conv_ctx(hbc, lengths, K, dtype=None):
    """(b, channels, K): hbc[b, len_b - K + j] where 0 <= len_b - K + j < len_b,
    else 0 (index clamped to [0, L-1] as the reference's gather does)."""
    b, L, ch = hbc.shape
    lens = torch.full((b,), L, dtype=torch.int64) if lengths is None else lengths.to(torch.int64)
    ctx = torch.zeros(b, ch, K, dtype=dtype or hbc.dtype)
    for i in range(b):
        for j in range(K):
            src = int(lens[i]) - K + j
            if 0 <= src < int(lens[i]) and L > 0:
                ctx[i, :, j] = hbc[i, min(src, L - 1)].to(ctx.dtype)
    return ctx


def conv_step(hbc_t, ctx, w, bias=None, dtype=torch.float64):
    """(out (b, channels), new ctx (b, channels, K)); ctx is not modified."""
    w = w.reshape(w.shape[0], w.shape[-1]).to(dtype)
    new = torch.roll(ctx, shifts=-1, dims=-1).clone()
    new[:, :, -1] = hbc_t.to(new.dtype)
    out = (silu(new.to(dtype)) * w).sum(-1)
    if bias is not None:
        out = out + bias.to(dtype)
    return out, new


def gate_forward(y, x, D, gate, dtype=torch.float64):
    return (y.to(dtype) + D.to(dtype) * x.to(dtype)) * silu(gate.to(dtype))


def gate_backward(dout, y, x, D, gate, dtype=torch.float64):
    """(dy, dx, dD, dgate) of gate_forward."""
    do, y, x, D, g = (t.to(dtype) for t in (dout, y, x, D, gate))
    dy = do * silu(g)
    dx = D * dy
    dD = (dy * x).reshape(-1, x.shape[-1]).sum(0)
    dg = do * (y + D * x) * dsilu(g)
    return dy, dx, dD, dg


def conv_forward_torch(hbc, w, bias=None, dtype=torch.float64):
    """The reference's own composition (modules/ssm.py:112-118): transpose,
    F.silu, depthwise F.conv1d with padding K-1, slice to seq_len, transpose
    back.  Used to pin conv_forward's causal indexing."""
    b, L, ch = hbc.shape
    w3 = w.reshape(ch, 1, w.shape[-1]).to(dtype)
    K = w3.shape[-1]
    z = F.silu(hbc.to(dtype).transpose(1, 2))
    out = F.conv1d(z, w3, None if bias is None else bias.to(dtype), padding=K - 1, groups=ch)
    return out[:, :, :L].transpose(1, 2)
