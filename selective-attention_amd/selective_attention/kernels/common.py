"""Host-side helpers shared by the kernel launchers."""
from __future__ import annotations

import torch

from .. import _lib

_ACT_DTYPES = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16}


def act_dtype_code(dtype: torch.dtype) -> int:
    """Kernel dtype code for activations (u, B, C, delta_raw, q/k/v)."""
    try:
        return _ACT_DTYPES[dtype]
    except KeyError:
        raise TypeError(f"unsupported activation dtype {dtype}; expected float32 or bfloat16")


def as_dtype(t: torch.Tensor | None, dtype: torch.dtype) -> torch.Tensor | None:
    if t is None or t.dtype == dtype:
        return t
    return t.to(dtype)


def require_device(*tensors: torch.Tensor | None) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(
                f"tensor on {t.device}: the HIP kernels need device tensors (no CPU path)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def limits(delta_limit) -> tuple[float, float]:
    lo, hi = float(delta_limit[0]), float(delta_limit[1])
    return lo, hi
