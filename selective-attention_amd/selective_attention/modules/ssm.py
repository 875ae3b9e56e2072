"""The SSM block (modules/ssm.py:10-204) on the gfx950 ops.

Parameters, their initialisation and the forward / step interfaces follow
the reference.  The compute between in_proj and out_proj runs in the
kernels: SSMConvFn (SiLU + causal depthwise conv + split; with the decode
context in the same pass at prefill), SSDScanGatedFn (the chunked scan with
the D-skip / SiLU-gate epilogue fused for bf16), and at decode ssm_conv_step
and the state update with the same epilogue in one kernel (ssu_gated_forward;
SSUFn then SSMGateFn when autograd is recording).
"""
from __future__ import annotations

import math
from typing import Tuple

import torch
import torch.nn as nn

from ..kernels.ssm_io import ssm_conv_forward
from ..kernels.ssu import ssu_gated_forward
from .layers import Linear
from ..ops import SSDScanGatedFn, SSMConvFn, SSMGateFn, SSUFn, ssm_conv_step


class SSM(nn.Module):
    def __init__(self, layer_idx: int, model_dim: int = 512, state_dim: int = 128,
                 conv_kernel_size: int = 4, head_dim: int = 64, num_groups: int = 1,
                 expansion_factor: int = 2, chunk_size: int = 256,
                 delta_limit: Tuple[float, float] = (0.0, float("inf")),
                 A_init_range: Tuple[float, float] = (1, 16),
                 delta_init_limit: Tuple[float, float] = (0.001, 0.1),
                 delta_init_floor: float = 1e-4, dropout_rate: float = 0.15, device="cuda"):
        super().__init__()
        self.layer_idx = layer_idx
        self.model_dim = model_dim
        self.state_dim = state_dim
        self.inner_dim = expansion_factor * model_dim
        assert self.inner_dim % head_dim == 0
        self.conv_kernel_size = conv_kernel_size
        self.head_dim = head_dim
        self.num_heads = self.inner_dim // head_dim
        self.num_groups = num_groups
        assert self.num_heads % num_groups == 0
        self.chunk_size = chunk_size
        self.delta_limit = delta_limit
        self.bc_dim = num_groups * state_dim

        self.in_proj = Linear(model_dim, 2 * self.inner_dim + 2 * self.bc_dim + self.num_heads)
        conv_dim = self.inner_dim + 2 * self.bc_dim
        self.conv = nn.Conv1d(conv_dim, conv_dim, conv_kernel_size, groups=conv_dim,
                              padding=conv_kernel_size - 1)

        # delta_bias = softplus^-1(dt0), dt0 log-uniform in delta_init_limit, floored
        lo, hi = math.log(delta_init_limit[0]), math.log(delta_init_limit[1])
        dt0 = torch.exp(torch.rand(self.num_heads, dtype=torch.float32) * (hi - lo) + lo)
        dt0 = dt0.clamp(min=delta_init_floor)
        self.delta_bias = nn.Parameter(dt0 + torch.log(-torch.expm1(-dt0)))
        self.delta_bias._no_weight_decay = True
        A = torch.empty(self.num_heads, dtype=torch.float32).uniform_(*A_init_range)
        self.A_log = nn.Parameter(torch.log(A))
        self.A_log._no_weight_decay = True
        self.D = nn.Parameter(torch.ones(self.inner_dim))
        self.D._no_weight_decay = True

        self.out_proj = Linear(self.inner_dim, model_dim)
        self.dropout = nn.Dropout(dropout_rate)

    def _A(self) -> torch.Tensor:
        """A = -exp(A_log) in fp32; in inference computed once per value of
        A_log (the decode step then launches nothing for it)."""
        if torch.is_grad_enabled() and self.A_log.requires_grad:
            return -torch.exp(self.A_log.float())
        key = (self.A_log.data_ptr(), self.A_log._version, self.A_log.device)
        if getattr(self, "_A_key", None) != key:
            self._A_val = -torch.exp(self.A_log.detach().float())
            self._A_key = key
        return self._A_val

    def _split(self, proj: torch.Tensor):
        return torch.split(proj, [self.inner_dim + 2 * self.bc_dim, self.inner_dim, self.num_heads],
                           dim=-1)

    def forward(self, hidden_states: torch.Tensor, lengths: torch.Tensor | None = None,
                ssm_hiddens: torch.Tensor | None = None, cache=None):
        """
        Args:
            hidden_states: (batch_size, seq_len, model_dim)
            lengths: (batch_size,)
            ssm_hiddens: (batch_size, num_heads, head_dim, state_dim)
        Returns:
            hidden_states: (batch_size, seq_len, model_dim)
            last_ssm_hiddens: (batch_size, num_heads, head_dim, state_dim) float32
        """
        b, L, _ = hidden_states.shape
        hBC, gate, delta_raw = self.in_proj.split_forward(
            hidden_states, [self.inner_dim + 2 * self.bc_dim, self.inner_dim, self.num_heads])
        A = self._A()
        if cache is not None and not self.training:
            # prefill: the decode context (raw rows before SiLU) from the conv's own pass
            x, B, C, ctx = ssm_conv_forward(hBC, self.conv.weight, self.conv.bias, self.inner_dim,
                                            self.bc_dim, lengths=lengths, with_ctx=True)
            cache.conv_ctx = ctx
        else:
            x, B, C = SSMConvFn.apply(hBC, self.conv.weight, self.conv.bias, self.inner_dim,
                                      self.bc_dim)
        H, P, G, N = self.num_heads, self.head_dim, self.num_groups, self.state_dim
        out, h_last = SSDScanGatedFn.apply(
            x.view(b, L, H, P), A, B.view(b, L, G, N), C.view(b, L, G, N), delta_raw,
            self.delta_bias, ssm_hiddens, lengths, self.chunk_size, True, self.delta_limit,
            self.D, gate.reshape(b, L, H, P))
        if cache is not None and not self.training:
            cache.h = h_last
        return self.out_proj(out.view(b, L, self.inner_dim)), h_last

    def step(self, hidden_states: torch.Tensor, cache) -> torch.Tensor:
        """hidden_states (batch_size, model_dim) -> (batch_size, model_dim);
        cache.conv_ctx and cache.h are updated in place."""
        b = hidden_states.shape[0]
        hBC, gate, delta_raw = self.in_proj.split_forward(
            hidden_states, [self.inner_dim + 2 * self.bc_dim, self.inner_dim, self.num_heads])
        x, B, C = ssm_conv_step(hBC, cache.conv_ctx, self.conv.weight, self.conv.bias,
                                self.inner_dim, self.bc_dim)
        A = self._A()
        H, P, G, N = self.num_heads, self.head_dim, self.num_groups, self.state_dim
        if (not torch.is_grad_enabled() and cache.h.dtype == torch.float32
                and cache.h.is_contiguous() and gate.dtype == x.dtype):
            # state update, y + D x and the SiLU gate in one kernel
            out = ssu_gated_forward(x.view(b, H, P), A, B.view(b, G, N), C.view(b, G, N),
                                    delta_raw, self.delta_bias, cache.h, self.D,
                                    gate.reshape(b, H, P)).view(b, self.inner_dim)
            return self.out_proj(out)
        y, cache.h = SSUFn.forward(x.view(b, H, P), A, B.view(b, G, N), C.view(b, G, N),
                                   delta_raw, self.delta_bias, cache.h)
        out = SSMGateFn.apply(y.reshape(b, self.inner_dim), x, self.D, gate)
        return self.out_proj(out)
