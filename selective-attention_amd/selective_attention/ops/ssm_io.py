"""The SSM block's input / output stages around the scan, on gfx950.

New ops (no reference op signature: the reference runs these steps as torch
ops inside SSM.forward / SSM.step); they follow the reference conventions
(tensors in and out, ValueError on bad shapes before any launch).

* SSMConvFn.apply(hBC, conv_weight, conv_bias, x_dim, bc_dim) -> (x, B, C):
  modules/ssm.py:116-125 -- F.silu, the depthwise causal Conv1d
  (padding K-1, sliced to seq_len) and the split, with x (b, L, x_dim) and
  B, C (b, L, bc_dim) returned as contiguous tensors (the scan takes them
  without a copy).  Backward through the same conv.
* build_conv_ctx(hBC, lengths, K): SSMCache.build_conv_ctx
  (inference/ssm_cache.py:8-36), (b, channels, K) raw rows.
* ssm_conv_step(hBC_t, conv_ctx, conv_weight, conv_bias, x_dim, bc_dim):
  SSMCache.update (inference/ssm_cache.py:38-43) plus the conv of SSM.step
  (modules/ssm.py:173-182); conv_ctx is updated in place.
* SSMGateFn.apply(y, x, D, gate) -> (y + D x) silu(gate):
  modules/ssm.py:144-150 (and :200-202), in the dtype of x.
* SSDScanGatedFn.apply(u, A, B, C, delta_raw, delta_bias, h_init, length,
  chunk_size, use_delta_softplus, delta_limit, D, gate) -> (out, h_last):
  the scan and the epilogue in one op (modules/ssm.py:136-150), fused into
  the chunk scan's output stage for bf16.
"""
from __future__ import annotations

import torch

from ..kernels.ssm_io import (ssm_conv_backward, ssm_conv_forward, ssm_conv_step as _conv_step,
                              ssm_gate_backward, ssm_gate_forward)
from ..utils import check_ndim, check_shape


def _check_conv(hBC, weight, bias, x_dim, bc_dim, seq_dims):
    check_ndim(hBC, seq_dims, name="hBC")
    channels = hBC.shape[-1]
    if weight.dim() == 3:
        check_shape(weight, (channels, 1, weight.shape[-1]), name="conv_weight")
    else:
        check_ndim(weight, 2, name="conv_weight")
        check_shape(weight, (channels, weight.shape[-1]), name="conv_weight")
    check_ndim(bias, 1, name="conv_bias", optional=True)
    if bias is not None:
        check_shape(bias, (channels,), name="conv_bias")
    if x_dim < 0 or bc_dim < 0 or x_dim + 2 * bc_dim != channels:
        raise ValueError(f"x_dim ({x_dim}) + 2 * bc_dim ({bc_dim}) must equal the {channels} channels")
    if not 1 <= weight.shape[-1] <= 8:
        raise ValueError(f"conv kernel size {weight.shape[-1]} outside [1, 8]")


class SSMConvFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hBC, conv_weight, conv_bias, x_dim: int, bc_dim: int):
        """
        Args:
            hBC: (batch_size, seq_len, x_dim + 2 * bc_dim)
            conv_weight: (channels, 1, K) or (channels, K)
            conv_bias: (channels,) or None
        Returns:
            x: (batch_size, seq_len, x_dim); B, C: (batch_size, seq_len, bc_dim)
        """
        _check_conv(hBC, conv_weight, conv_bias, x_dim, bc_dim, 3)
        x, B, C, _ = ssm_conv_forward(hBC, conv_weight, conv_bias, x_dim, bc_dim)
        ctx.save_for_backward(hBC, conv_weight, conv_bias)
        ctx.dims = (x_dim, bc_dim)
        return x, B, C

    @staticmethod
    def backward(ctx, dx, dB, dC):
        hBC, weight, bias = ctx.saved_tensors
        x_dim, bc_dim = ctx.dims
        b, L, _ = hBC.shape
        z = lambda n: torch.zeros(b, L, n, dtype=hBC.dtype, device=hBC.device)
        dx = z(x_dim) if dx is None else dx
        dB = z(bc_dim) if dB is None else dB
        dC = z(bc_dim) if dC is None else dC
        dhbc, dw, db = ssm_conv_backward(hBC, weight, dx, dB, dC, x_dim, bc_dim, bias is not None)
        dw = dw.reshape(weight.shape).to(weight.dtype)
        db = None if db is None else db.to(bias.dtype)
        return dhbc, dw, db, None, None


@torch.inference_mode()
def build_conv_ctx(hBC: torch.Tensor, lengths: torch.Tensor | None, cache_size: int) -> torch.Tensor:
    """(batch_size, channels, cache_size) decode context of raw hBC rows.

    hBC is (batch_size, seq_len, channels) here (the reference transposes it to
    (batch_size, channels, seq_len) first).
    """
    check_ndim(hBC, 3, name="hBC")
    check_ndim(lengths, 1, name="lengths", optional=True)
    b, L, ch = hBC.shape
    w = torch.zeros(ch, cache_size, dtype=torch.float32, device=hBC.device)
    _, _, _, ctx = ssm_conv_forward(hBC, w, None, ch, 0, lengths=lengths, ctx_only=True)
    return ctx


@torch.inference_mode()
def ssm_conv_step(hBC_t, conv_ctx, conv_weight, conv_bias, x_dim: int, bc_dim: int):
    """One decode step.  hBC_t (batch_size, channels); conv_ctx
    (batch_size, channels, K), contiguous, updated in place.  Returns x
    (batch_size, x_dim), B and C (batch_size, bc_dim)."""
    _check_conv(hBC_t, conv_weight, conv_bias, x_dim, bc_dim, 2)
    check_ndim(conv_ctx, 3, name="conv_ctx")
    return _conv_step(hBC_t, conv_ctx, conv_weight, conv_bias, x_dim, bc_dim)


class SSMGateFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, y, x, D, gate):
        """
        Args:
            y: (..., dim) float32 scan output; x, gate: (..., dim); D: (dim,)
        Returns:
            (y + D x) silu(gate), dtype of x
        """
        check_shape(y, tuple(x.shape), name="y")
        check_shape(gate, tuple(x.shape), name="gate")
        check_ndim(D, 1, name="D")
        check_shape(D, (x.shape[-1],), name="D")
        out = ssm_gate_forward(y, x, D, gate)
        ctx.save_for_backward(y, x, D, gate)
        return out

    @staticmethod
    def backward(ctx, dout):
        y, x, D, gate = ctx.saved_tensors
        dy, dx, dD, dgate = ssm_gate_backward(dout, y, x, D, gate)
        return dy.to(y.dtype), dx, dD.to(D.dtype), dgate.to(gate.dtype)


class SSDScanGatedFn(torch.autograd.Function):
    """SSDScanFn followed by the SSM epilogue, as SSM.forward runs them
    (modules/ssm.py:136-150): out = (y + D u) silu(gate), h_last.

    For bf16 activations (head_dim % 8 == 0, state_dim a multiple of 32 up to
    256) the epilogue is fused into the chunk scan's output stage: the fp32 y
    is never written; the scan saves yd = y + D u (bf16) for the gate's
    backward instead.  Other inputs run the scan and SSMGateFn's kernel in
    turn.  u is used twice (scan input and D skip); its gradient is the sum.
    """

    @staticmethod
    def forward(ctx, u, A, B, C, delta_raw, delta_bias, h_init, length, chunk_size: int,
                use_delta_softplus: bool, delta_limit, D, gate):
        """
        Args: as SSDScanFn (u (batch_size, seq_len, num_heads, head_dim), ...), plus
            D: (num_heads * head_dim,); gate: (batch_size, seq_len, num_heads, head_dim)
        Returns:
            out: (batch_size, seq_len, num_heads, head_dim), dtype of u
            h_last: (batch_size, num_heads, head_dim, state_dim) float32
        """
        from ..kernels.ssd_scan import gated_supported, ssd_scan_forward, ssd_scan_forward_gated
        from .ssd_scan import check_scan_args
        u, A, B, C, delta_raw, delta_bias, h_init, length = check_scan_args(
            u, A, B, C, delta_raw, delta_bias, h_init, length)
        b, L, H, P = u.shape
        check_ndim(D, 1, name="D")
        check_shape(D, (H * P,), name="D")
        check_shape(gate, (b, L, H, P), name="gate")
        gate = gate.contiguous()
        fused = gated_supported(u.dtype, P, B.shape[3])
        if fused:
            out, ysave, h_last, saved = ssd_scan_forward_gated(
                u, A, B, C, delta_raw, delta_bias, h_init, length, chunk_size,
                use_delta_softplus, delta_limit, D, gate)
        else:
            y, h_last, saved = ssd_scan_forward(u, A, B, C, delta_raw, delta_bias, h_init, length,
                                                chunk_size, use_delta_softplus, delta_limit, True,
                                                return_saved=True)
            out = ssm_gate_forward(y.view(b, L, H * P), u.view(b, L, H * P), D,
                                   gate.view(b, L, H * P)).view(b, L, H, P)
            ysave = y
        ctx.save_for_backward(u, A, B, C, delta_raw, delta_bias, h_init, length, D, gate, ysave,
                              *saved)
        ctx.fused = fused
        ctx.cfg = (chunk_size, use_delta_softplus, delta_limit)
        ctx.set_materialize_grads(False)   # an unused h_last arrives as None (read as zero)
        return out, h_last

    @staticmethod
    def backward(ctx, dout, h_last_grad):
        from ..kernels.ssd_scan import ssd_scan_backward
        u, A, B, C, delta_raw, delta_bias, h_init, length, D, gate, ysave, dt, dc, states = \
            ctx.saved_tensors
        chunk_size, sp, limit = ctx.cfg
        if dout is None:
            dout = torch.zeros_like(u)
        P = u.shape[-1]
        dy, d_skip, dD, dgate = ssm_gate_backward(
            dout.reshape(*u.shape[:2], -1), ysave.reshape(*u.shape[:2], -1),
            u.reshape(*u.shape[:2], -1), D, gate.reshape(*u.shape[:2], -1), y_is_yd=ctx.fused)
        grads = ssd_scan_backward(u, A, B, C, delta_raw, delta_bias, h_init, dy.view(u.shape),
                                  h_last_grad, length, chunk_size, sp, limit, True,
                                  saved=(dt, dc, states))
        du, dA, dB, dC, ddr, dbias, dh0 = grads
        du = du + d_skip.view(u.shape)
        return (du, dA, dB, dC, ddr, dbias, dh0, None, None, None, None,
                dD.to(D.dtype), dgate.view(u.shape).to(gate.dtype))
