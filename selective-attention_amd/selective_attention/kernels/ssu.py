"""Launcher of the single-step selective state update.

Mirrors ssu_forward (triton_kernels/ssu/forward.py:7-63): y = empty_like(u),
one kernel launch that updates the fp32 state h in place and writes y in the
dtype of u.
"""
from __future__ import annotations

from typing import Tuple

import torch

from .. import _lib
from .common import act_dtype_code, as_dtype, limits, require_device


def ssu_forward(
    u: torch.Tensor,
    A: torch.Tensor,
    B: torch.Tensor,
    C: torch.Tensor,
    delta_raw: torch.Tensor,
    delta_bias: torch.Tensor | None,
    h: torch.Tensor,
    use_delta_softplus: bool = True,
    delta_limit: Tuple = (0.0, float("inf")),
):
    """
    Args:
        u: (batch_size, num_heads, head_dim)
        A: (num_heads,)
        B, C: (batch_size, num_groups, state_dim)
        delta_raw: (batch_size, num_heads)
        delta_bias: (num_heads,)
        h: (batch_size, num_heads, head_dim, state_dim), updated in place

    Returns:
        y: (batch_size, num_heads, head_dim), dtype of u
        h: the updated state (the same tensor object)
    """
    require_device(u, A, B, C, delta_raw, delta_bias, h)
    batch_size, num_heads, head_dim = u.shape
    _, num_groups, state_dim = B.shape
    code = act_dtype_code(u.dtype)
    B = as_dtype(B, u.dtype).contiguous()
    C = as_dtype(C, u.dtype).contiguous()
    delta_raw = as_dtype(delta_raw, u.dtype).contiguous()
    A32 = as_dtype(A, torch.float32).contiguous()
    bias32 = None if delta_bias is None else as_dtype(delta_bias, torch.float32).contiguous()

    # the kernel keeps the state in fp32; other state dtypes round-trip
    h_work = h if h.dtype == torch.float32 else h.float()

    y = torch.empty_like(u)
    lo, hi = limits(delta_limit)
    _lib.call(
        "sa_ssu_fwd", code, _lib.ptr(u), _lib.ptr(A32), _lib.ptr(B), _lib.ptr(C),
        _lib.ptr(delta_raw), _lib.ptr(bias32), _lib.ptr(h_work), _lib.ptr(y),
        batch_size, num_heads, head_dim, num_groups, state_dim,
        1 if use_delta_softplus else 0, lo, hi, _lib.stream_of(u))
    if h_work is not h:
        h.copy_(h_work)
    return y, h


def ssu_gated_forward(u, A, B, C, delta_raw, delta_bias, h, D, gate,
                      use_delta_softplus: bool = True, delta_limit: Tuple = (0.0, float("inf"))):
    """ssu_forward and the SSM block's decode epilogue in one kernel:
    returns out (batch, heads, head_dim) = (y + D u) * silu(gate) in the
    dtype of u, y rounded to that dtype first; h (float32) is updated in
    place.  D (heads * head_dim,), gate (batch, heads, head_dim)."""
    require_device(u, A, B, C, delta_raw, delta_bias, h, D, gate)
    batch_size, num_heads, head_dim = u.shape
    _, num_groups, state_dim = B.shape
    if h.dtype != torch.float32 or not h.is_contiguous():
        raise ValueError("ssu_gated_forward: h must be a contiguous float32 tensor")
    if D.numel() != num_heads * head_dim or tuple(gate.shape) != tuple(u.shape):
        raise ValueError(f"ssu_gated_forward: D {tuple(D.shape)} / gate {tuple(gate.shape)} "
                         f"do not match u {tuple(u.shape)}")
    code = act_dtype_code(u.dtype)
    u = u.contiguous()
    B = as_dtype(B, u.dtype).contiguous()
    C = as_dtype(C, u.dtype).contiguous()
    delta_raw = as_dtype(delta_raw, u.dtype).contiguous()
    gate = as_dtype(gate, u.dtype).contiguous()
    A32 = as_dtype(A, torch.float32).contiguous()
    D32 = as_dtype(D, torch.float32).contiguous()
    bias32 = None if delta_bias is None else as_dtype(delta_bias, torch.float32).contiguous()
    out = torch.empty_like(u)
    lo, hi = limits(delta_limit)
    _lib.call(
        "sa_ssu_fwd_gated", code, _lib.ptr(u), _lib.ptr(A32), _lib.ptr(B), _lib.ptr(C),
        _lib.ptr(delta_raw), _lib.ptr(bias32), _lib.ptr(h), _lib.ptr(D32), _lib.ptr(gate),
        _lib.ptr(out), batch_size, num_heads, head_dim, num_groups, state_dim,
        1 if use_delta_softplus else 0, lo, hi, _lib.stream_of(u))
    return out
