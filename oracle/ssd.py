"""CPU restatement of the reference SSD chunked scan (forward + backward).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): used by tests/ as the
parity checker and by bench.py's cpu_baseline leg as the timed CPU path.

Every function follows one reference kernel, cited file:line relative to
/root/reference/src/selective_attention/triton_kernels/.  Computation runs in
`dtype` (float64 for pinning, float32 for the timed baseline) on whatever
device the inputs live on (the CPU in every use).  Shapes follow the
reference:
  u (b,L,H,P)  A (H,)  B,C (b,L,G,N)  delta_raw (b,L,H)  delta_bias (H,)
  h_init (b,H,P,N)  length (b,) int64
Internal chunk tensors: dt, dc (b,H,nc,Lc); states (b,nc,H,P,N);
CB (b,nc,G,Lc,Lc).

Reference behaviours reproduced on purpose:
  * softplus is log(exp(z)+1) below the threshold 20 (softplus.py:8);
  * dt is clamped to delta_limit, then zeroed at t >= length
    (ssd_scan/forward_kernel.py:63-80); a length above seq_len is clamped to
    seq_len (the reference would read out of bounds);
  * exp(min(x, 0)) decay clamps (forward_kernel.py:178, :438);
  * y is computed (non-zero) at t >= length; dy is ignored there and every
    gradient row at t >= length is zero (backward_kernel.py:69-70, :245);
  * x_B enters the exclusive decay-cumsum only for tau < lim-1
    (backward_kernel.py:427-430, backward.py:217);
  * ddc_last[0] = 0 without h_init (backward_kernel.py:163-167).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

Tensor = torch.Tensor


def softplus20(z: Tensor) -> Tensor:
    """softplus.py:5-8 + forward_kernel.py:77: log(exp(z)+1) if z <= 20 else z."""
    return torch.where(z <= 20.0, torch.log(torch.exp(z) + 1.0), z)


def _pad_seq(x: Tensor, Lp: int) -> Tensor:
    """Zero-pad dim 1 (sequence) to Lp."""
    L = x.shape[1]
    if L == Lp:
        return x
    pad = torch.zeros((x.shape[0], Lp - L) + tuple(x.shape[2:]), dtype=x.dtype, device=x.device)
    return torch.cat([x, pad], dim=1)


def _time_mask(length: Tensor, L: int, Lp: int, device) -> Tensor:
    """(b, Lp) bool: t < min(length, L)."""
    t = torch.arange(Lp, device=device)
    lens = length.to(device=device, dtype=torch.int64).clamp(min=0, max=L)
    return t[None, :] < lens[:, None]


def _heads(x: Tensor, hpg: int, dim: int) -> Tensor:
    """Expand a group axis to heads (head h uses group h // hpg)."""
    return x.repeat_interleave(hpg, dim=dim) if hpg > 1 else x


def make_dt(delta_raw: Tensor, delta_bias: Optional[Tensor], use_softplus: bool,
            delta_limit: Tuple[float, float], dtype) -> Tensor:
    """dt before the length mask: clamp(softplus20(delta_raw + bias))."""
    z = delta_raw.to(dtype)
    if delta_bias is not None:
        z = z + delta_bias.to(dtype)
    d = softplus20(z) if use_softplus else z
    return torch.clamp(d, min=float(delta_limit[0]), max=float(delta_limit[1]))


def chunk_cumsum_forward(A, delta_raw, delta_bias, length, chunk_size, use_softplus,
                         delta_limit, dtype=torch.float64):
    """ssd_scan/forward.py:14-56, kernel forward_kernel.py:20-87.

    Returns dt, dc: (b, H, nc, Lc); dc = inclusive cumsum of dt*A per chunk.
    """
    b, L, H = delta_raw.shape
    nc = math.ceil(L / chunk_size)
    Lp = nc * chunk_size
    d = make_dt(delta_raw, delta_bias, use_softplus, delta_limit, dtype)
    d = _pad_seq(d, Lp)
    m = _time_mask(length, L, Lp, d.device)
    d = torch.where(m[:, :, None], d, torch.zeros((), dtype=dtype, device=d.device))
    dt = d.view(b, nc, chunk_size, H).permute(0, 3, 1, 2).contiguous()
    dc = torch.cumsum(dt * A.to(dtype)[None, :, None, None], dim=-1)
    return dt, dc


def chunk_state_forward(u, B, dt, dc, dtype=torch.float64):
    """ssd_scan/forward.py:62-96, kernel forward_kernel.py:108-185.

    S_c[p,n] = sum_tau exp(min(dc_last - dc_tau, 0)) * dt_tau * u[tau,p] * B[tau,n]
    """
    b, L, H, P = u.shape
    G, N = B.shape[2], B.shape[3]
    _, _, nc, Lc = dt.shape
    Lp = nc * Lc
    uc = _pad_seq(u.to(dtype), Lp).view(b, nc, Lc, H, P)
    Bc = _heads(_pad_seq(B.to(dtype), Lp).view(b, nc, Lc, G, N), H // G, 3)
    w = torch.exp(torch.clamp(dc[..., -1:] - dc, max=0.0)) * dt          # (b,H,nc,Lc)
    w = w.permute(0, 2, 3, 1)                                             # (b,nc,Lc,H)
    return torch.einsum("bclhp,bclhn->bchpn", uc * w[..., None], Bc)


def state_passing_forward(states, h_init, dc_last):
    """ssd_scan/forward.py:102-133, kernel forward_kernel.py:203-250.

    states (b,nc,H,P,N) -> H_in (b,nc,H,P,N) (state entering each chunk), h_last.
    """
    b, nc, H, P, N = states.shape
    prev = (h_init.to(states.dtype).clone() if h_init is not None
            else torch.zeros((b, H, P, N), dtype=states.dtype, device=states.device))
    H_in = torch.empty_like(states)
    for c in range(nc):
        H_in[:, c] = prev
        prev = torch.exp(dc_last[:, :, c])[:, :, None, None] * prev + states[:, c]
    return H_in, prev


def bmm_chunk_forward(B, C, chunk_size, dtype=torch.float64):
    """ssd_scan/forward.py:139-169, kernel forward_kernel.py:271-328.

    CB[b,c,g,tau,sigma] = C[tau] . B[sigma] (full square; only tau >= sigma is used).
    """
    b, L, G, N = B.shape
    nc = math.ceil(L / chunk_size)
    Lp = nc * chunk_size
    Bc = _pad_seq(B.to(dtype), Lp).view(b, nc, chunk_size, G, N)
    Cc = _pad_seq(C.to(dtype), Lp).view(b, nc, chunk_size, G, N)
    return torch.einsum("bclgn,bcsgn->bcgls", Cc, Bc)


def chunk_scan_forward(u, dt, dc, C, H_in, CB, dtype=torch.float64):
    """ssd_scan/forward.py:175-217, kernel forward_kernel.py:351-455 (IS_CAUSAL=True).

    y[tau,p] = exp(dc_tau) * C_tau . H_in[p,:]
             + sum_{sigma <= tau} CB[tau,sigma] * exp(min(dc_tau - dc_sigma, 0)) * dt_sigma * u[sigma,p]
    """
    b, L, H, P = u.shape
    G, N = C.shape[2], C.shape[3]
    _, _, nc, Lc = dt.shape
    Lp = nc * Lc
    hpg = H // G
    uc = _pad_seq(u.to(dtype), Lp).view(b, nc, Lc, H, P)
    Ch = _heads(_pad_seq(C.to(dtype), Lp).view(b, nc, Lc, G, N), hpg, 3)
    edc = torch.exp(dc).permute(0, 2, 3, 1)                                # (b,nc,Lc,H)
    y = torch.einsum("bclhn,bchpn->bclhp", Ch, H_in) * edc[..., None]
    tri = torch.tril(torch.ones(Lc, Lc, dtype=torch.bool, device=u.device))
    dcp = dc.permute(0, 2, 1, 3)                                          # (b,nc,H,Lc)
    dtp = dt.permute(0, 2, 1, 3)
    decay = torch.exp(torch.clamp(dcp[..., :, None] - dcp[..., None, :], max=0.0))
    M = _heads(CB, hpg, 2) * decay * dtp[..., None, :]
    M = torch.where(tri, M, torch.zeros((), dtype=dtype, device=u.device))
    y = y + torch.einsum("bchls,bcshp->bclhp", M, uc)
    return y.reshape(b, Lp, H, P)[:, :L]


def ssd_scan_forward(u, A, B, C, delta_raw, delta_bias=None, h_init=None, length=None,
                     chunk_size=256, use_delta_softplus=True,
                     delta_limit=(0.0, float("inf")), dtype=torch.float64,
                     return_intermediates=False):
    """ssd_scan/forward.py:223-276 (and the op ops/ssd_scan.py:67-73).

    Returns y (b,L,H,P) and h_last (b,H,P,N) in `dtype`.
    """
    b, L, H, P = u.shape
    if length is None:
        length = torch.full((b,), L, dtype=torch.int64)
    dt, dc = chunk_cumsum_forward(A, delta_raw, delta_bias, length, chunk_size,
                                  use_delta_softplus, delta_limit, dtype)
    S = chunk_state_forward(u, B, dt, dc, dtype)
    H_in, h_last = state_passing_forward(S, None if h_init is None else h_init.to(dtype),
                                         dc[..., -1])
    CB = bmm_chunk_forward(B, C, chunk_size, dtype)
    y = chunk_scan_forward(u, dt, dc, C, H_in, CB, dtype)
    if return_intermediates:
        return y, h_last, dict(dt=dt, dc=dc, states=S, H_in=H_in, CB=CB)
    return y, h_last


def ssd_scan_backward(u, A, B, C, delta_raw, delta_bias, h_init, y_grad, h_last_grad, length,
                      chunk_size=256, use_delta_softplus=True,
                      delta_limit=(0.0, float("inf")), dtype=torch.float64):
    """Manual backward, ssd_scan/backward.py:467-555, kernels backward_kernel.py.

    Returns (u_grad, A_grad, B_grad, C_grad, delta_raw_grad, delta_bias_grad,
    h_init_grad) in `dtype` (the op casts to the input dtypes).
    """
    b, L, H, P = u.shape
    G, N = B.shape[2], B.shape[3]
    hpg = H // G
    if length is None:
        length = torch.full((b,), L, dtype=torch.int64)
    dev = u.device
    zero = torch.zeros((), dtype=dtype, device=dev)

    # recompute (backward.py:507-519)
    y, h_last, it = ssd_scan_forward(u, A, B, C, delta_raw, delta_bias, h_init, length,
                                     chunk_size, use_delta_softplus, delta_limit, dtype, True)
    dt, dc, H_in, CB = it["dt"], it["dc"], it["H_in"], it["CB"]
    _, _, nc, Lc = dt.shape
    Lp = nc * Lc
    m = _time_mask(length, L, Lp, dev).view(b, nc, Lc)                    # tau < lim
    mh = m[:, :, :, None]                                                 # (b,nc,Lc,1)

    uc = _pad_seq(u.to(dtype), Lp).view(b, nc, Lc, H, P)
    Bc = _pad_seq(B.to(dtype), Lp).view(b, nc, Lc, G, N)
    Cc = _pad_seq(C.to(dtype), Lp).view(b, nc, Lc, G, N)
    Bh, Ch = _heads(Bc, hpg, 3), _heads(Cc, hpg, 3)
    dyc = _pad_seq(y_grad.to(dtype), Lp).view(b, nc, Lc, H, P)
    dyc = torch.where(mh[..., None], dyc, zero)                           # dy' (ignored at t >= len)
    um = torch.where(mh[..., None], uc, zero)

    dcp = dc.permute(0, 2, 3, 1)                                          # (b,nc,Lc,H)
    dtp = dt.permute(0, 2, 3, 1)
    dc_last = dc[..., -1]                                                 # (b,H,nc)

    # chunk_scan_backward_h: dH_intra = sum_tau dy'_tau exp(dc_tau) (x) C_tau  (backward_kernel.py:73-89)
    dH_intra = torch.einsum("bclhp,bclhn->bchpn", dyc * torch.exp(dcp)[..., None], Ch)

    # state_passing_backward (backward_kernel.py:151-167)
    Gr = (h_last_grad.to(dtype).clone() if h_last_grad is not None
          else torch.zeros((b, H, P, N), dtype=dtype, device=dev))
    dS = torch.empty_like(dH_intra)
    ddc_last = torch.zeros((b, H, nc), dtype=dtype, device=dev)
    for c in range(nc - 1, -1, -1):
        scale = torch.exp(dc_last[:, :, c])
        ddc_last[:, :, c] = (H_in[:, c] * Gr).sum(dim=(-1, -2)) * scale
        dS[:, c] = Gr
        Gr = scale[:, :, None, None] * Gr + dH_intra[:, c]
    h_init_grad = Gr if h_init is not None else None
    if h_init is None:
        ddc_last[:, :, 0] = 0.0

    # chunk_scan_chunk_state_backward_u (backward_kernel.py:244-317)
    sc = torch.exp(torch.clamp(dcp[:, :, -1:, :] - dcp, max=0.0))        # (b,nc,Lc,H)
    Bhm = torch.where(mh[..., None], Bh, zero)
    acc = torch.einsum("bclhn,bchpn->bclhp", Bhm, dS) * sc[..., None]
    dcH = dc.permute(0, 2, 1, 3)                                          # (b,nc,H,Lc)
    decT = torch.exp(torch.clamp(dcH[..., None, :] - dcH[..., :, None], max=0.0))  # [l,s]=e^{min(dc_s-dc_l,0)}
    upper = torch.triu(torch.ones(Lc, Lc, dtype=torch.bool, device=dev))  # s >= l
    CBT = _heads(CB, hpg, 2).transpose(-1, -2)                            # [l,s] = CB[s,l]
    M2 = torch.where(upper, CBT * decT, zero)
    acc = acc + torch.einsum("bchls,bcshp->bclhp", M2, dyc)
    acc = torch.where(mh[..., None], acc, zero)
    u_grad = (acc * dtp[..., None]).reshape(b, Lp, H, P)[:, :L]
    ddt_direct = (acc * um).sum(-1)                                       # (b,nc,Lc,H)

    # chunk_state_backward_B (backward_kernel.py:392-441)
    w = torch.where(mh, torch.exp(torch.clamp(dcp[:, :, -1:, :] - dcp, max=0.0)) * dtp, zero)
    contribB = torch.einsum("bclhp,bchpn->bclhn", um, dS) * w[..., None]
    dB = contribB.view(b, nc, Lc, G, hpg, N).sum(4)
    xB = (contribB * Bhm).sum(-1)                                         # (b,nc,Lc,H)
    pos = torch.arange(Lc, device=dev)
    lim = (length.to(dev).clamp(0, L)[:, None] - torch.arange(nc, device=dev)[None, :] * Lc)
    xB = torch.where((pos[None, None, :] < lim[:, :, None] - 1)[..., None], xB, zero)
    dA_B = torch.cumsum(xB, dim=2) - xB                                   # exclusive prefix

    # chunk_scan_backward_C (backward_kernel.py:510-551)
    contribC = torch.einsum("bclhp,bchpn->bclhn", dyc, H_in) * torch.exp(dcp)[..., None]
    dC = contribC.view(b, nc, Lc, G, hpg, N).sum(4)
    Chm = torch.where(mh[..., None], Ch, zero)
    xC = (contribC * Chm).sum(-1)                                         # (b,nc,Lc,H)

    # chunk_scan_backward_CB (backward_kernel.py:615-668): W_h[l,s] for l >= s
    dy_u = torch.einsum("bclhp,bcshp->bchls", dyc, um)
    decS = torch.exp(torch.clamp(dcH[..., :, None] - dcH[..., None, :], max=0.0))  # [l,s]=e^{min(dc_l-dc_s,0)}
    lower = torch.tril(torch.ones(Lc, Lc, dtype=torch.bool, device=dev))
    dtH = dt.permute(0, 2, 1, 3)                                          # (b,nc,H,Lc)
    W = torch.where(lower, dy_u * dtH[..., None, :] * decS, zero)         # (b,nc,H,Lc,Lc)
    dCB = W.view(b, nc, G, hpg, Lc, Lc).sum(3)

    # bmm_chunk_backward x2 (backward_kernel.py:729-765, backward.py:541-542)
    dB = dB + torch.einsum("bcgls,bclgn->bcsgn", dCB, Cc * m[..., None, None])
    dC = dC + torch.einsum("bcgls,bcsgn->bclgn", dCB, Bc * m[..., None, None])
    dB = torch.where(m[..., None, None], dB, zero)
    dC = torch.where(m[..., None, None], dC, zero)

    # chunk_scan_backward_decay_cumsum (backward_kernel.py:834-911)
    strict = torch.tril(torch.ones(Lc, Lc, dtype=torch.bool, device=dev), diagonal=-1)
    Q = torch.where(strict, W * _heads(CB, hpg, 2), zero)                 # (b,nc,H,l,s)
    R = torch.cumsum(Q, dim=-1) - Q                                       # R[l,k] = sum_{s<k} Q[l,s]
    geq = torch.triu(torch.ones(Lc, Lc, dtype=torch.bool, device=dev))   # [k,l]: l >= k
    dA_intra = torch.einsum("bchlk,kl->bchk", R, geq.to(dtype))          # sum_{l>=k} R[l,k]

    # host glue backward.py:544-548
    xC = xC.permute(0, 3, 1, 2).clone()                                   # (b,H,nc,Lc)
    xC[..., -1] = xC[..., -1] + ddc_last
    dA_C = torch.flip(torch.cumsum(torch.flip(xC, [-1]), dim=-1), [-1])
    da = dA_intra.permute(0, 2, 1, 3) + dA_B.permute(0, 3, 1, 2) + dA_C  # (b,H,nc,Lc)

    # chunk_cumsum_backward (backward_kernel.py:973-1039)
    Af = A.to(dtype)
    ddt = da * Af[None, :, None, None] + ddt_direct.permute(0, 3, 1, 2)
    z = delta_raw.to(dtype)
    if delta_bias is not None:
        z = z + delta_bias.to(dtype)
    z = _pad_seq(z, Lp).view(b, nc, Lc, H).permute(0, 3, 1, 2)            # (b,H,nc,Lc)
    dsp = softplus20(z) if use_delta_softplus else z
    lo, hi = float(delta_limit[0]), float(delta_limit[1])
    clamped = (dsp < lo) | (dsp > hi)
    dtv = torch.clamp(dsp, min=lo, max=hi)
    mH = m[:, None, :, :]                                                 # (b,1,nc,Lc)
    ddt = torch.where(clamped & mH, zero, ddt)
    if use_delta_softplus:
        ddt = torch.where(z <= 20.0, ddt * torch.sigmoid(z), ddt)
    ddt = torch.where(mH, ddt, zero)
    daa = torch.where(mH, da, zero)
    A_grad = (daa * dtv).sum(dim=(0, 2, 3))
    delta_bias_grad = ddt.sum(dim=(0, 2, 3)) if delta_bias is not None else None
    delta_raw_grad = ddt.permute(0, 2, 3, 1).reshape(b, Lp, H)[:, :L]

    B_grad = dB.reshape(b, Lp, G, N)[:, :L]
    C_grad = dC.reshape(b, Lp, G, N)[:, :L]
    return u_grad, A_grad, B_grad, C_grad, delta_raw_grad, delta_bias_grad, h_init_grad


# ---------------------------------------------------------------------------
# independent closed form (pins the chunked restatement)
# ---------------------------------------------------------------------------
def ssd_sequential(u, A, B, C, delta_raw, delta_bias=None, h_init=None, length=None,
                   use_delta_softplus=True, delta_limit=(0.0, float("inf")),
                   dtype=torch.float64):
    """Token-by-token recurrence S_t = exp(A dt_t) S_{t-1} + dt_t u_t (x) B_t, y_t = S_t C_t.

    dt_t = 0 for t >= length (state frozen), matching the op's length semantics.
    Differentiable (used for autograd cross-checks).  Returns y, h_last.
    """
    b, L, H, P = u.shape
    G, N = B.shape[2], B.shape[3]
    hpg = H // G
    if length is None:
        length = torch.full((b,), L, dtype=torch.int64)
    d = make_dt(delta_raw, delta_bias, use_delta_softplus, delta_limit, dtype)
    m = _time_mask(length, L, L, d.device)
    d = torch.where(m[:, :, None], d, torch.zeros((), dtype=dtype, device=d.device))
    Bh = _heads(B.to(dtype), hpg, 2)
    Ch = _heads(C.to(dtype), hpg, 2)
    uf = u.to(dtype)
    S = (h_init.to(dtype) if h_init is not None
         else torch.zeros((b, H, P, N), dtype=dtype, device=u.device))
    Af = A.to(dtype)
    ys = []
    for t in range(L):
        a = torch.exp(Af[None, :] * d[:, t])                              # (b,H)
        S = a[:, :, None, None] * S + (d[:, t, :, None] * uf[:, t])[..., None] * Bh[:, t, :, None, :]
        ys.append((S * Ch[:, t, :, None, :]).sum(-1))
    return torch.stack(ys, dim=1), S
