"""Library layers of the LMs, as the reference defines them: RMSNorm
(modules/rms_norm.py:4-44), RoPE (modules/rope.py:9-64), SwiGLU
(modules/feed_forward.py:4-11).  In inference RMSNorm and the rotation of q
and k run as single fused kernels (kernels/lm_ops.py); with autograd (the
SSM blocks can train) RMSNorm keeps its torch composite."""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..kernels.lm_ops import (add_rms_norm, add_rms_norm_supported, gemv, gemv_multi,
                              gemv_supported, rms_norm, rope_qk, silu_mul)


def _gemv_ok(x: torch.Tensor, lin: nn.Linear) -> bool:
    return (gemv_supported(x, lin.weight)
            and (lin.bias is None or lin.bias.dtype == torch.bfloat16)
            and not (torch.is_grad_enabled() and (x.requires_grad or lin.weight.requires_grad)))


class Linear(nn.Linear):
    """nn.Linear (same parameters and state-dict names) whose inference
    forward on at most 8 bf16 rows, the decode steps' shape, runs the
    small-batch GEMV kernel instead of a GEMM."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if _gemv_ok(x, self):
            return gemv(x, self.weight, self.bias)
        return super().forward(x)

    def split_forward(self, x: torch.Tensor, sizes) -> list:
        """torch.split(self(x), sizes, dim=-1).  On the decode shape the
        weight's row blocks go to one multi-GEMV launch that writes each
        piece as its own contiguous tensor (no copies of split views)."""
        bs = [None] * len(sizes) if self.bias is None else torch.split(self.bias, sizes)
        if _gemv_ok(x, self) and len(sizes) <= 4:
            return gemv_multi(x, torch.split(self.weight, sizes), bs)
        if x.is_cuda and not torch.is_grad_enabled():
            # one GEMM per row block: contiguous pieces, no copies of split views later
            return [F.linear(x, w, bb) for w, bb in zip(torch.split(self.weight, sizes), bs)]
        return list(torch.split(self(x), sizes, dim=-1))


def project(x: torch.Tensor, linears, xscale: torch.Tensor | None = None) -> list:
    """[lin(x * xscale if xscale is given else x) for lin in linears]: one
    multi-GEMV launch on the decode shape (at most 4 layers), where the
    product x * xscale is taken in bf16 as torch does."""
    if len(linears) <= 4 and all(_gemv_ok(x, lin) for lin in linears):
        return gemv_multi(x, [lin.weight for lin in linears], [lin.bias for lin in linears], xscale)
    xs = x if xscale is None else x * xscale
    return [lin(xs) for lin in linears]


class RMSNorm(nn.Module):
    """x * rsqrt(mean(x^2) + eps) * (1 + weight), computed in fp32 and
    returned in the dtype of x; the weight starts at 0 (modules/rms_norm.py)."""

    def __init__(self, dim: int, num_groups: int | None = None, eps: float = 1e-6,
                 elementwise_affine: bool = True):
        super().__init__()
        self.eps = eps
        self.num_groups = num_groups
        self.elementwise_affine = elementwise_affine
        if elementwise_affine:
            shape = (dim,) if num_groups is None else (num_groups, dim)
            self.weight = nn.Parameter(torch.zeros(shape))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if (self.elementwise_affine and x.is_cuda and x.is_contiguous()
                and x.dtype in (torch.float32, torch.bfloat16)
                and not (torch.is_grad_enabled() and (x.requires_grad or self.weight.requires_grad))):
            return rms_norm(x, self.weight, self.eps)     # one fused kernel (inference)
        xf = x.float()
        out = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        if self.elementwise_affine:
            out = out * (1.0 + self.weight.float())
        return out.type_as(x)

    def add_forward(self, x: torch.Tensor, y: torch.Tensor):
        """(x + y, self(x + y)): a pre-norm block's residual add and its next
        norm, in one kernel in inference for bf16 rows of 512k <= 4096 elements."""
        if (self.elementwise_affine and add_rms_norm_supported(x, self.weight)
                and not (torch.is_grad_enabled()
                         and (x.requires_grad or y.requires_grad or self.weight.requires_grad))):
            return add_rms_norm(x, y, self.weight, self.eps)
        s = x + y
        return s, self(s)


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


class RoPE(nn.Module):
    """Rotary embedding with inverse frequencies base^(-i / (dim/2)) and the
    angle table [theta, theta] over the head dimension (modules/rope.py)."""

    def __init__(self, dim: int, base: float = 10000):
        super().__init__()
        assert dim % 2 == 0
        self.dim, self.base = dim, base
        half = dim // 2
        inv_freq = 1.0 / (base ** (torch.arange(0, half, dtype=torch.float32) / half))
        self.register_buffer("inv_freq", inv_freq, persistent=False)
        # fp32 copy kept outside Module.to(): casting the model to bf16 casts
        # the buffer too, and bf16 frequencies put the angle off by radians at
        # positions in the thousands
        self._inv_fp32 = {}

    def freqs(self, device) -> torch.Tensor:
        """The inverse frequencies in fp32 on `device` (computed once per device)."""
        key = str(device)
        if key not in self._inv_fp32:
            half = self.dim // 2
            f = 1.0 / (self.base ** (torch.arange(0, half, dtype=torch.float32) / half))
            self._inv_fp32[key] = f.to(device)
        return self._inv_fp32[key]

    def cos_sin(self, positions: torch.Tensor):
        ang = positions.to(torch.float32).unsqueeze(-1) * self.freqs(positions.device).unsqueeze(0)
        ang = torch.cat([ang, ang], dim=-1)
        return torch.cos(ang), torch.sin(ang)

    def forward(self, q: torch.Tensor, k: torch.Tensor, positions: torch.Tensor, mode: str = "seq"):
        """mode "seq": q, k (batch, heads, seq_len, head_dim), positions (seq_len,);
        mode "pos": q, k (batch, heads, head_dim), positions (batch,)."""
        cos, sin = self.cos_sin(positions)
        if mode == "seq":
            cos, sin = cos[None, None], sin[None, None]
        else:
            cos, sin = cos[:, None], sin[:, None]
        return q * cos + _rotate_half(q) * sin, k * cos + _rotate_half(k) * sin

    def rotate_qk(self, q: torch.Tensor, k: torch.Tensor, positions: torch.Tensor | None,
                  period: int):
        """q, k (..., heads, head_dim) on the GPU, rotated in one fused kernel
        and returned in bf16; row r of the leading dimensions at
        positions[r % period], or at r % period when positions is None."""
        return rope_qk(q, k, self.freqs(q.device), positions, period)


class SwiGLU(nn.Module):
    """out(w1(x) * silu(w2(x))) (modules/feed_forward.py)."""

    def __init__(self, dim: int, hidden_dim: int):
        super().__init__()
        self.w1 = Linear(dim, hidden_dim)
        self.w2 = Linear(dim, hidden_dim)
        self.out = Linear(hidden_dim, dim)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        a, c = project(x, [self.w1, self.w2])
        if (a.is_cuda and a.dtype == torch.bfloat16 and c.dtype == torch.bfloat16
                and a.numel() % 8 == 0
                and not (torch.is_grad_enabled() and (a.requires_grad or c.requires_grad))):
            return self.out(silu_mul(a, c))          # one fused kernel (inference)
        return self.out(a * F.silu(c))
