"""SSUFn: the decode-step state update op.

Drop-in for the reference's SSUFn (ops/ssu.py:8-63): an nn.Module subclass
with a static forward under torch.inference_mode, the same argument order and
defaults, the same ndim/shape validation (ValueError before any launch), and
the same in-place update of a contiguous h.  Caller: SSM.step
(modules/ssm.py:195-197).
"""
from __future__ import annotations

from typing import Tuple

import torch
import torch.nn as nn

from ..kernels.ssu import ssu_forward
from ..utils import check_ndim, check_shape, to_contiguous


class SSUFn(nn.Module):
    @staticmethod
    @torch.inference_mode()
    def forward(
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
        """One recurrence step of every (batch row, head) state.

        Shapes (b = batch, H = heads, P = head_dim, G = groups, N = state_dim):
        u (b, H, P); A (H,); B and C (b, G, N); delta_raw (b, H);
        delta_bias (H,) or None; h (b, H, P, N), fp32 state.

        Returns (y, h): y (b, H, P) in the dtype of u, and the state after the
        step -- the caller's tensor itself, updated in place, when it is a
        contiguous fp32 tensor.
        """
        u, A, B, C, delta_raw, delta_bias, h = check_step_args(u, A, B, C, delta_raw,
                                                               delta_bias, h)
        return ssu_forward(u, A, B, C, delta_raw, delta_bias, h, use_delta_softplus, delta_limit)


def check_step_args(u, A, B, C, delta_raw, delta_bias, h):
    """The reference's validation of a state-update call (ops/ssu.py:38-61):
    ValueError on a wrong ndim, then on a shape that disagrees with u and B,
    before any launch; every tensor made contiguous."""
    expected_ndim = dict(u=3, A=1, B=3, C=3, delta_raw=2, h=4)
    args = dict(u=u, A=A, B=B, C=C, delta_raw=delta_raw, h=h)
    for name, t in args.items():
        check_ndim(t, expected_ndim[name], name=name)
        if name == "delta_raw":
            check_ndim(delta_bias, 1, name="delta_bias", optional=True)

    b, nh, p = u.shape
    ng, n = B.shape[1], B.shape[2]
    expected_shape = dict(A=(nh,), B=(b, ng, n), C=(b, ng, n), delta_raw=(b, nh),
                          h=(b, nh, p, n))
    for name, shape in expected_shape.items():
        check_shape(args[name], shape, name=name)
        if name == "delta_raw":
            check_shape(delta_bias, (nh,), name="delta_bias", optional=True)
    if nh % ng != 0:
        raise ValueError(f"num_heads ({nh}) must be a multiple of num_groups ({ng})")

    return tuple(to_contiguous(t) for t in (u, A, B, C, delta_raw, delta_bias, h))
