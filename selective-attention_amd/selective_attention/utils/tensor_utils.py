"""Input validation shared by the ops.

Same names, arguments and error type as the reference's validators
(utils/tensor_utils.py:5-45): a mismatch raises ValueError before any kernel
launch.  The messages carry the tensor name as a "[name] " prefix (the
reference builds that prefix inverted in two places, :13 and :32/36; the
exception type and the condition are what callers rely on).
"""
from __future__ import annotations

from typing import Tuple

import torch


def _prefix(name: str | None) -> str:
    return f"[{name}] " if name else ""


def check_ndim(tensor: torch.Tensor | None, ndim: int, name: str | None = None,
               optional: bool = False) -> None:
    if tensor is None:
        if not optional:
            raise ValueError(f"{_prefix(name)}Expected tensor with ndim {ndim}, but got None")
        return
    if tensor.ndim != ndim:
        raise ValueError(
            f"{_prefix(name)}Dim mismatch: expected ndim={ndim}, got ndim={tensor.ndim}, "
            f"shape={tuple(tensor.shape)}")


def check_shape(tensor: torch.Tensor | None, shape: Tuple[int, ...], name: str | None = None,
                optional: bool = False) -> None:
    if tensor is None:
        if not optional:
            raise ValueError(f"{_prefix(name)}Expected tensor with shape {shape}, but got None")
    elif tuple(tensor.shape) != tuple(shape):
        raise ValueError(
            f"{_prefix(name)}Shape mismatch: expected {tuple(shape)}, got {tuple(tensor.shape)}")


def to_contiguous(tensor: torch.Tensor | None) -> torch.Tensor | None:
    if tensor is None:
        return tensor
    if not tensor.is_contiguous():
        return tensor.contiguous()
    return tensor
