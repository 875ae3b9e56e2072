"""SSDScanFn: the chunked SSD scan op (training / prefill).

Drop-in for the reference's SSDScanFn (ops/ssd_scan.py:7-96): a
torch.autograd.Function with the same forward signature and defaults, the
same ndim/shape validation (ValueError before any launch), contiguity
handling, an absent `length` meaning the full sequence,
fp32 outputs y and h_last, and a backward that returns
(u_grad, A_grad, B_grad, C_grad, delta_raw_grad, delta_bias_grad,
h_init_grad, None x5).  Caller: SSM.forward (modules/ssm.py:136-139).

Difference kept on purpose: the forward saves the chunk intermediates
(dt, dc, chunk entry states) for the backward instead of recomputing them.
"""
from __future__ import annotations

from typing import Tuple

import torch

from ..kernels.ssd_scan import ssd_scan_backward, ssd_scan_forward
from ..utils import check_ndim, check_shape, to_contiguous


class SSDScanFn(torch.autograd.Function):
    @staticmethod
    def forward(
        ctx,
        u: torch.Tensor,
        A: torch.Tensor,
        B: torch.Tensor,
        C: torch.Tensor,
        delta_raw: torch.Tensor,
        delta_bias: torch.Tensor | None = None,
        h_init: torch.Tensor | None = None,
        length: torch.Tensor | None = None,
        chunk_size: int = 256,
        use_delta_softplus: bool = True,
        delta_limit: Tuple[float, float] = (0.0, float("inf")),
        is_causal: bool = True,
    ):
        """
        Args:
            u: (batch_size, seq_len, num_heads, head_dim)
            A: (num_heads,)
            B, C: (batch_size, seq_len, num_groups, state_dim)
            delta_raw: (batch_size, seq_len, num_heads)
            delta_bias: (num_heads,)
            h_init: (batch_size, num_heads, head_dim, state_dim)
            length: (batch_size,)

        Returns:
            y: (batch_size, seq_len, num_heads, head_dim)
            h_last: (batch_size, num_heads, head_dim, state_dim)
        """
        u, A, B, C, delta_raw, delta_bias, h_init, length = check_scan_args(
            u, A, B, C, delta_raw, delta_bias, h_init, length)

        y, h_last, saved = ssd_scan_forward(
            u, A, B, C, delta_raw, delta_bias, h_init, length,
            chunk_size, use_delta_softplus, delta_limit, is_causal, return_saved=True,
        )

        dt, dc, states = saved
        ctx.save_for_backward(u, A, B, C, delta_raw, delta_bias, h_init, length, dt, dc, states)
        # an output that takes no gradient arrives as None rather than as a
        # materialised zero tensor (the backward reads None as zero)
        ctx.set_materialize_grads(False)
        ctx.chunk_size = chunk_size
        ctx.use_delta_softplus = use_delta_softplus
        ctx.delta_limit = delta_limit
        ctx.is_causal = is_causal

        return y, h_last

    @staticmethod
    def backward(ctx, y_grad, h_last_grad):
        u, A, B, C, delta_raw, delta_bias, h_init, length, dt, dc, states = ctx.saved_tensors

        grads = ssd_scan_backward(
            u, A, B, C, delta_raw, delta_bias, h_init, y_grad, h_last_grad, length,
            ctx.chunk_size, ctx.use_delta_softplus, ctx.delta_limit, ctx.is_causal,
            saved=(dt, dc, states),
        )
        u_grad, A_grad, B_grad, C_grad, delta_raw_grad, delta_bias_grad, h_init_grad = grads
        return (u_grad, A_grad, B_grad, C_grad, delta_raw_grad, delta_bias_grad, h_init_grad,
                None, None, None, None, None)


def check_scan_args(u, A, B, C, delta_raw, delta_bias, h_init, length):
    """The reference's validation and contiguity handling (ops/ssd_scan.py:38-68):
    ValueError on a bad ndim / shape before any launch, contiguous copies;
    an absent `length` means the full sequence."""
    check_ndim(u, 4, name="u")
    check_ndim(A, 1, name="A")
    check_ndim(B, 4, name="B")
    check_ndim(C, 4, name="C")
    check_ndim(delta_raw, 3, name="delta_raw")
    check_ndim(delta_bias, 1, name="delta_bias", optional=True)
    check_ndim(h_init, 4, name="h_init", optional=True)
    check_ndim(length, 1, name="length", optional=True)

    batch_size, seq_len, num_heads, head_dim = u.shape
    num_groups, state_dim = B.shape[2], B.shape[3]

    check_shape(A, (num_heads,), name="A")
    check_shape(B, (batch_size, seq_len, num_groups, state_dim), name="B")
    check_shape(C, (batch_size, seq_len, num_groups, state_dim), name="C")
    check_shape(delta_raw, (batch_size, seq_len, num_heads), name="delta_raw")
    check_shape(delta_bias, (num_heads,), name="delta_bias", optional=True)
    check_shape(h_init, (batch_size, num_heads, head_dim, state_dim), name="h_init",
                optional=True)
    check_shape(length, (batch_size,), name="length", optional=True)
    if num_heads % num_groups != 0:
        raise ValueError(f"num_heads ({num_heads}) must be a multiple of num_groups ({num_groups})")

    u = to_contiguous(u)
    A = to_contiguous(A)
    B = to_contiguous(B)
    C = to_contiguous(C)
    delta_raw = to_contiguous(delta_raw)
    delta_bias = to_contiguous(delta_bias)
    h_init = to_contiguous(h_init)
    length = to_contiguous(length)
    # an absent length stays None: the kernels take it as every row full,
    # where the reference materialises torch.full((batch,), seq_len)
    return u, A, B, C, delta_raw, delta_bias, h_init, length
