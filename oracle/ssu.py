"""CPU restatement of the single-step selective state update.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Follows triton_kernels/ssu/forward_kernel.py:59-78 (launcher
ssu/forward.py:7-63): no length mask, state update then readout.
"""
from __future__ import annotations

import torch

from .ssd import make_dt


def ssu_forward(u, A, B, C, delta_raw, delta_bias, h, use_delta_softplus=True,
                delta_limit=(0.0, float("inf")), dtype=torch.float64):
    """Returns (y, h_new) in `dtype`; h is not modified.

    u (b,H,P), A (H,), B,C (b,G,N), delta_raw (b,H), delta_bias (H,), h (b,H,P,N).
    """
    b, H, P = u.shape
    G = B.shape[1]
    hpg = H // G
    dt = make_dt(delta_raw, delta_bias, use_delta_softplus, delta_limit, dtype)   # (b,H)
    Bh = B.to(dtype).repeat_interleave(hpg, dim=1)                               # (b,H,N)
    Ch = C.to(dtype).repeat_interleave(hpg, dim=1)
    decay = torch.exp(A.to(dtype)[None, :] * dt)                                 # (b,H)
    h_new = (h.to(dtype) * decay[:, :, None, None]
             + (dt[:, :, None] * u.to(dtype))[..., None] * Bh[:, :, None, :])
    y = (h_new * Ch[:, :, None, :]).sum(-1)
    return y, h_new
