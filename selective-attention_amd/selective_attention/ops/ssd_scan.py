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
        """Chunked scan of every (batch row, head) over the sequence.

        Shapes (b = batch, L = seq_len, H = heads, P = head_dim, G = groups,
        N = state_dim): u (b, L, H, P); A (H,); B and C (b, L, G, N);
        delta_raw (b, L, H); delta_bias (H,) or None; h_init (b, H, P, N) or
        None (zero state); length (b,) int64 or None (every row full).

        Returns (y, h_last): y (b, L, H, P) and the state after the last
        valid token h_last (b, H, P, N), both fp32.
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
    first every tensor's ndim, then every shape against the sizes u and B
    give, each a ValueError raised before any launch, in the reference's
    order; then contiguous copies where needed.  An absent `length` stays
    None: the kernels read it as every row full (the reference builds
    torch.full((batch,), seq_len) on the device instead)."""
    args = dict(u=u, A=A, B=B, C=C, delta_raw=delta_raw, delta_bias=delta_bias,
                h_init=h_init, length=length)
    optional = ("delta_bias", "h_init", "length")
    ndims = dict(u=4, A=1, B=4, C=4, delta_raw=3, delta_bias=1, h_init=4, length=1)
    for name, nd in ndims.items():
        check_ndim(args[name], nd, name=name, optional=name in optional)

    b, L, H, P = u.shape
    G, N = B.shape[2], B.shape[3]
    shapes = dict(A=(H,), B=(b, L, G, N), C=(b, L, G, N), delta_raw=(b, L, H),
                  delta_bias=(H,), h_init=(b, H, P, N), length=(b,))
    for name, shape in shapes.items():
        check_shape(args[name], shape, name=name, optional=name in optional)
    if H % G != 0:
        raise ValueError(f"num_heads ({H}) must be a multiple of num_groups ({G})")

    return tuple(to_contiguous(args[name]) for name in ndims)
