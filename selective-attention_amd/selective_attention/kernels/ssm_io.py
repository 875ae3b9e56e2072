"""Launchers of the SSM block's input / output stages around the scan.

Prologue (reference modules/ssm.py:116-125): xBC = Conv1d_K(silu(hBC)) + bias,
causal with zero history, split into x, B, C.  Decode (modules/ssm.py:173-182,
inference/ssm_cache.py:38-43): the context window of the last K raw rows is
shifted and the same conv applied to it.  Prefill context
(inference/ssm_cache.py:8-36).  Epilogue (modules/ssm.py:144-150):
out = (y + D x) silu(gate).  Every launch goes to libsa_hip.so.
"""
from __future__ import annotations

import torch

from .. import _lib
from .common import act_dtype_code, as_dtype, require_device


def _conv_weight(weight: torch.Tensor) -> torch.Tensor:
    """(channels, K) float32 from a Conv1d weight (channels, 1, K) or (channels, K)."""
    w = weight.reshape(weight.shape[0], weight.shape[-1]) if weight.dim() == 3 else weight
    if w.dim() != 2:
        raise ValueError(f"conv weight must be (channels, 1, K) or (channels, K), got {tuple(weight.shape)}")
    return as_dtype(w, torch.float32).contiguous()


def _bias(bias: torch.Tensor | None) -> torch.Tensor | None:
    return None if bias is None else as_dtype(bias, torch.float32).contiguous()


def ssm_conv_forward(hbc, weight, bias, x_dim, bc_dim, lengths=None, with_ctx=False,
                     ctx_only=False):
    """hbc (b, L, channels) -> x (b, L, x_dim), B, C (b, L, bc_dim) and, with
    with_ctx, the decode context (b, channels, K) of raw hbc rows (ctx_only:
    the context alone; x, B, C are None)."""
    require_device(hbc, weight, bias, lengths)
    b, L, ch = hbc.shape
    w = _conv_weight(weight)
    if w.shape[0] != ch:
        raise ValueError(f"conv weight has {w.shape[0]} channels, input has {ch}")
    K = w.shape[1]
    hbc = hbc.contiguous()
    if ctx_only:
        x = Bo = Co = None
    else:
        x = torch.empty(b, L, x_dim, dtype=hbc.dtype, device=hbc.device)
        Bo = torch.empty(b, L, bc_dim, dtype=hbc.dtype, device=hbc.device)
        Co = torch.empty(b, L, bc_dim, dtype=hbc.dtype, device=hbc.device)
    with_ctx = with_ctx or ctx_only
    ctx = torch.empty(b, ch, K, dtype=hbc.dtype, device=hbc.device) if with_ctx else None
    lens = None if lengths is None else as_dtype(lengths, torch.int64).contiguous()
    bs = _bias(bias)
    _lib.call("sa_ssm_conv_fwd", act_dtype_code(hbc.dtype), _lib.ptr(hbc), _lib.ptr(w), _lib.ptr(bs),
              b, L, ch, K, x_dim, bc_dim, _lib.ptr(x), _lib.ptr(Bo), _lib.ptr(Co), _lib.ptr(lens),
              _lib.ptr(ctx), _lib.stream_of(hbc))
    return x, Bo, Co, ctx


def ssm_conv_backward(hbc, weight, dx, dB, dC, x_dim, bc_dim, with_bias=True):
    """Gradients of hbc, the conv weight (channels, K) float32 and bias."""
    b, L, ch = hbc.shape
    w = _conv_weight(weight)
    K = w.shape[1]
    dt_ = hbc.dtype
    dx = as_dtype(dx, dt_).contiguous()
    dB = as_dtype(dB, dt_).contiguous()
    dC = as_dtype(dC, dt_).contiguous()
    dhbc = torch.empty_like(hbc)
    dw = torch.empty(ch, K, dtype=torch.float32, device=hbc.device)
    db = torch.empty(ch, dtype=torch.float32, device=hbc.device) if with_bias else None
    nbytes = _lib.load().sa_ssm_conv_bwd_workspace_size(b, L, ch, K)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=hbc.device)
    _lib.call("sa_ssm_conv_bwd", act_dtype_code(dt_), _lib.ptr(hbc), _lib.ptr(w), _lib.ptr(dx),
              _lib.ptr(dB), _lib.ptr(dC), b, L, ch, K, x_dim, bc_dim, _lib.ptr(dhbc), _lib.ptr(dw),
              _lib.ptr(db), _lib.ptr(ws), nbytes, _lib.stream_of(hbc))
    return dhbc, dw, db


def ssm_conv_step(hbc_t, conv_ctx, weight, bias, x_dim, bc_dim):
    """One decode step: conv_ctx (b, channels, K) is shifted in place."""
    require_device(hbc_t, conv_ctx, weight, bias)
    b, ch = hbc_t.shape
    w = _conv_weight(weight)
    K = w.shape[1]
    if tuple(conv_ctx.shape) != (b, ch, K) or not conv_ctx.is_contiguous():
        raise ValueError(f"conv_ctx must be a contiguous ({b}, {ch}, {K}) tensor, got {tuple(conv_ctx.shape)}")
    if conv_ctx.dtype != hbc_t.dtype:
        raise ValueError(f"conv_ctx dtype {conv_ctx.dtype} != input dtype {hbc_t.dtype}")
    hbc_t = hbc_t.contiguous()
    x = torch.empty(b, x_dim, dtype=hbc_t.dtype, device=hbc_t.device)
    Bo = torch.empty(b, bc_dim, dtype=hbc_t.dtype, device=hbc_t.device)
    Co = torch.empty(b, bc_dim, dtype=hbc_t.dtype, device=hbc_t.device)
    bs = _bias(bias)
    _lib.call("sa_ssm_conv_step", act_dtype_code(hbc_t.dtype), _lib.ptr(hbc_t), _lib.ptr(conv_ctx),
              _lib.ptr(w), _lib.ptr(bs), b, ch, K, x_dim, bc_dim, _lib.ptr(x), _lib.ptr(Bo),
              _lib.ptr(Co), _lib.stream_of(hbc_t))
    return x, Bo, Co


def ssm_gate_forward(y, x, D, gate):
    """out = (y + D x) silu(gate), dtype of x; y float32 (..., dim)."""
    require_device(y, x, D, gate)
    dim = x.shape[-1]
    rows = x.numel() // dim if dim else 0
    y32 = as_dtype(y, torch.float32).contiguous()
    x = x.contiguous()
    gate = as_dtype(gate, x.dtype).contiguous()
    D32 = as_dtype(D, torch.float32).contiguous()
    out = torch.empty_like(x)
    _lib.call("sa_ssm_gate_fwd", act_dtype_code(x.dtype), _lib.ptr(y32), _lib.ptr(x), _lib.ptr(D32),
              _lib.ptr(gate), rows, dim, _lib.ptr(out), _lib.stream_of(x))
    return out


def ssm_gate_backward(dout, y, x, D, gate, y_is_yd=False):
    """(dy float32, dx, dD float32, dgate) of ssm_gate_forward.  With y_is_yd,
    y is yd = y + D x in the dtype of x (saved by the fused scan epilogue)."""
    dim = x.shape[-1]
    rows = x.numel() // dim if dim else 0
    dout = as_dtype(dout, x.dtype).contiguous()
    y32 = as_dtype(y, x.dtype if y_is_yd else torch.float32).contiguous()
    x = x.contiguous()
    gate = as_dtype(gate, x.dtype).contiguous()
    D32 = as_dtype(D, torch.float32).contiguous()
    dy = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    dx = torch.empty_like(x)
    dgate = torch.empty_like(x)
    dD = torch.empty(dim, dtype=torch.float32, device=x.device)
    nbytes = _lib.load().sa_ssm_gate_bwd_workspace_size(rows, dim)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
    _lib.call("sa_ssm_gate_bwd", act_dtype_code(x.dtype), _lib.ptr(dout), _lib.ptr(y32),
              1 if y_is_yd else 0, _lib.ptr(x), _lib.ptr(D32), _lib.ptr(gate), rows, dim,
              _lib.ptr(dy), _lib.ptr(dx), _lib.ptr(dgate), _lib.ptr(dD), _lib.ptr(ws), nbytes,
              _lib.stream_of(x))
    return dy, dx, dD, dgate
