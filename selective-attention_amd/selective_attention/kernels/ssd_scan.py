"""Launchers of the SSD chunked scan (forward and backward).

Mirror ssd_scan_forward / ssd_scan_backward
(triton_kernels/ssd_scan/forward.py:223-276, backward.py:467-555).  The
forward also returns the chunk intermediates (dt, dc and the per-chunk entry
states) so that the backward reuses them instead of recomputing four
kernels; the reference's ctx saves inputs only and recomputes.
"""
from __future__ import annotations

import math
from typing import Tuple

import torch

from .. import _lib
from .common import act_dtype_code, as_dtype, limits, require_device


def _f32_aligned(t: torch.Tensor | None) -> torch.Tensor | None:
    """float32, contiguous, 16-byte aligned (vectorised state loads)."""
    if t is None:
        return None
    t = as_dtype(t, torch.float32).contiguous()
    if t.data_ptr() % 16 != 0:
        t = t.clone()
    return t


def _prep(u, A, B, C, delta_raw, delta_bias, h_init, length):
    require_device(u, A, B, C, delta_raw, delta_bias, h_init, length)
    b, L, H, P = u.shape
    code = act_dtype_code(u.dtype)
    B = as_dtype(B, u.dtype).contiguous()
    C = as_dtype(C, u.dtype).contiguous()
    delta_raw = as_dtype(delta_raw, u.dtype).contiguous()
    A32 = as_dtype(A, torch.float32).contiguous()
    bias32 = None if delta_bias is None else as_dtype(delta_bias, torch.float32).contiguous()
    h0 = _f32_aligned(h_init)
    if length is not None:   # None: full rows (the C-ABI's NULL length)
        length = as_dtype(length, torch.int64).contiguous()
    return code, u.contiguous(), A32, B, C, delta_raw, bias32, h0, length


def ssd_scan_forward(
    u: torch.Tensor,
    A: torch.Tensor,
    B: torch.Tensor,
    C: torch.Tensor,
    delta_raw: torch.Tensor,
    delta_bias: torch.Tensor | None,
    h_init: torch.Tensor | None,
    length: torch.Tensor | None,
    chunk_size: int,
    use_delta_softplus: bool = True,
    delta_limit: Tuple = (0.0, float("inf")),
    is_causal: bool = True,
    return_saved: bool = False,
):
    """
    Args:
        u: (batch_size, seq_len, num_heads, head_dim)
        A: (num_heads,)
        B, C: (batch_size, seq_len, num_groups, state_dim)
        delta_raw: (batch_size, seq_len, num_heads)
        delta_bias: (num_heads,)
        h_init: (batch_size, num_heads, head_dim, state_dim)
        length: (batch_size,) int64

    Returns:
        y: (batch_size, seq_len, num_heads, head_dim) float32
        h_last: (batch_size, num_heads, head_dim, state_dim) float32
        [saved: (dt, dc, states) when return_saved]

    `is_causal` is accepted for signature parity; the reference's scan is
    always causal (chunk_scan hard-codes IS_CAUSAL=True, forward.py:213).
    """
    code, u, A32, B, C, delta_raw, bias32, h0, length = _prep(
        u, A, B, C, delta_raw, delta_bias, h_init, length)
    b, L, H, P = u.shape
    G, N = B.shape[2], B.shape[3]
    nc = max(1, math.ceil(L / chunk_size))
    dev = u.device
    f32 = torch.float32
    y = torch.empty((b, L, H, P), dtype=f32, device=dev)
    h_last = torch.empty((b, H, P, N), dtype=f32, device=dev)
    dt = torch.empty((b, H, nc, chunk_size), dtype=f32, device=dev)
    dc = torch.empty((b, H, nc, chunk_size), dtype=f32, device=dev)
    states = torch.empty((b, nc, H, P, N), dtype=f32, device=dev)
    lo, hi = limits(delta_limit)
    if L == 0:
        h_last.copy_(h0 if h0 is not None else torch.zeros_like(h_last))
    else:
        _lib.call(
            "sa_ssd_fwd", code, _lib.ptr(u), _lib.ptr(A32), _lib.ptr(B), _lib.ptr(C),
            _lib.ptr(delta_raw), _lib.ptr(bias32), _lib.ptr(h0), _lib.ptr(length),
            b, L, H, P, G, N, int(chunk_size), 1 if use_delta_softplus else 0, lo, hi,
            _lib.ptr(y), _lib.ptr(h_last), _lib.ptr(dt), _lib.ptr(dc), _lib.ptr(states),
            _lib.stream_of(u))
    if return_saved:
        return y, h_last, (dt, dc, states)
    return y, h_last


def ssd_scan_forward_gated(u, A, B, C, delta_raw, delta_bias, h_init, length, chunk_size,
                           use_delta_softplus, delta_limit, D, gate):
    """ssd_scan_forward with the SSM epilogue (modules/ssm.py:144-150) fused into
    the chunk scan's output stage.  bf16 only (check gated_supported first).

    Args: as ssd_scan_forward, plus D (H*P,) and gate (b, L, H, P).
    Returns: out = (y + D u) silu(gate) and yd = y + D u, both (b, L, H, P)
    bf16, h_last, and saved (dt, dc, states).
    """
    code, u, A32, B, C, delta_raw, bias32, h0, length = _prep(
        u, A, B, C, delta_raw, delta_bias, h_init, length)
    b, L, H, P = u.shape
    G, N = B.shape[2], B.shape[3]
    nc = max(1, math.ceil(L / chunk_size))
    dev = u.device
    f32 = torch.float32
    D32 = _f32_aligned(D)
    gate = as_dtype(gate, u.dtype).contiguous()
    out = torch.empty((b, L, H, P), dtype=u.dtype, device=dev)
    yd = torch.empty((b, L, H, P), dtype=u.dtype, device=dev)
    h_last = torch.empty((b, H, P, N), dtype=f32, device=dev)
    dt = torch.empty((b, H, nc, chunk_size), dtype=f32, device=dev)
    dc = torch.empty((b, H, nc, chunk_size), dtype=f32, device=dev)
    states = torch.empty((b, nc, H, P, N), dtype=f32, device=dev)
    lo, hi = limits(delta_limit)
    if L == 0:
        h_last.copy_(h0 if h0 is not None else torch.zeros_like(h_last))
    else:
        _lib.call(
            "sa_ssd_fwd_gated", code, _lib.ptr(u), _lib.ptr(A32), _lib.ptr(B), _lib.ptr(C),
            _lib.ptr(delta_raw), _lib.ptr(bias32), _lib.ptr(h0), _lib.ptr(length),
            b, L, H, P, G, N, int(chunk_size), 1 if use_delta_softplus else 0, lo, hi,
            _lib.ptr(D32), _lib.ptr(gate), _lib.ptr(out), _lib.ptr(yd),
            _lib.ptr(h_last), _lib.ptr(dt), _lib.ptr(dc), _lib.ptr(states), _lib.stream_of(u))
    return out, yd, h_last, (dt, dc, states)


def gated_supported(dtype: torch.dtype, head_dim: int, state_dim: int) -> bool:
    """Whether ssd_scan_forward_gated handles these sizes."""
    code = act_dtype_code(dtype)
    return bool(_lib.load().sa_ssd_fwd_gated_supported(code, head_dim, state_dim))


def ssd_scan_backward(u, A, B, C, delta_raw, delta_bias, h_init, y_grad, h_last_grad, length,
                      chunk_size, use_delta_softplus=True, delta_limit=(0.0, float("inf")),
                      is_causal=True, saved=None):
    """
    Args: as ssd_scan_forward, plus
        y_grad: (batch_size, seq_len, num_heads, head_dim) or None
        h_last_grad: (batch_size, num_heads, head_dim, state_dim) or None
        saved: (dt, dc, states) returned by ssd_scan_forward(return_saved=True);
               recomputed when None

    Returns:
        u_grad, A_grad, B_grad, C_grad, delta_raw_grad, delta_bias_grad, h_init_grad
        in the dtypes of the corresponding inputs (None for absent optionals).
        Gradients are zero at t >= length and dy is ignored there
        (backward_kernel.py:69-70, :245).
    """
    dtypes = dict(u=u.dtype, A=A.dtype, B=B.dtype, C=C.dtype, delta_raw=delta_raw.dtype,
                  bias=None if delta_bias is None else delta_bias.dtype,
                  h=None if h_init is None else h_init.dtype)
    if saved is None:
        _, _, saved = ssd_scan_forward(u, A, B, C, delta_raw, delta_bias, h_init, length,
                                       chunk_size, use_delta_softplus, delta_limit, is_causal,
                                       return_saved=True)
    code, u, A32, B, C, delta_raw, bias32, h0, length = _prep(
        u, A, B, C, delta_raw, delta_bias, h_init, length)
    dt, dc, states = saved
    b, L, H, P = u.shape
    G, N = B.shape[2], B.shape[3]
    dev = u.device
    f32 = torch.float32
    if y_grad is None:
        dy = torch.zeros((b, L, H, P), dtype=f32, device=dev)
    else:
        dy = _f32_aligned(y_grad)
    dh_last = _f32_aligned(h_last_grad)

    du = torch.empty_like(u)
    dB = torch.empty_like(B)
    dC = torch.empty_like(C)
    ddr = torch.empty_like(delta_raw)
    dA = torch.empty((H,), dtype=f32, device=dev)
    dbias = None if delta_bias is None else torch.empty((H,), dtype=f32, device=dev)
    dh0 = None if h_init is None else torch.empty((b, H, P, N), dtype=f32, device=dev)
    if L == 0:
        du.zero_(); dB.zero_(); dC.zero_(); ddr.zero_(); dA.zero_()
        if dbias is not None:
            dbias.zero_()
        if dh0 is not None:
            dh0.copy_(dh_last if dh_last is not None else torch.zeros_like(dh0))
    else:
        lib = _lib.load()
        nbytes = lib.sa_ssd_bwd_workspace_size(code, b, L, H, P, G, N, int(chunk_size))
        if nbytes == 0:
            raise RuntimeError(f"sa_ssd_bwd_workspace_size: {lib.sa_last_error().decode()}")
        ws = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
        lo, hi = limits(delta_limit)
        _lib.call(
            "sa_ssd_bwd", code, _lib.ptr(u), _lib.ptr(A32), _lib.ptr(B), _lib.ptr(C),
            _lib.ptr(delta_raw), _lib.ptr(bias32), _lib.ptr(length), _lib.ptr(dy),
            _lib.ptr(dh_last), _lib.ptr(dt), _lib.ptr(dc), _lib.ptr(states),
            b, L, H, P, G, N, int(chunk_size), 1 if use_delta_softplus else 0, lo, hi,
            0 if h_init is None else 1,
            _lib.ptr(du), _lib.ptr(dA), _lib.ptr(dB), _lib.ptr(dC), _lib.ptr(ddr),
            _lib.ptr(dbias), _lib.ptr(dh0), _lib.ptr(ws), nbytes, _lib.stream_of(u))
    return (as_dtype(du, dtypes["u"]), as_dtype(dA, dtypes["A"]), as_dtype(dB, dtypes["B"]),
            as_dtype(dC, dtypes["C"]), as_dtype(ddr, dtypes["delta_raw"]),
            None if dbias is None else as_dtype(dbias, dtypes["bias"]),
            None if dh0 is None else as_dtype(dh0, dtypes["h"]))
