"""CausalBlock (modules/causal_block.py:13-139): pre-norm residual block of
SSM, SelectiveMHA and SwiGLU, with the reference's constructor arguments and
forward / step interfaces.  Each residual add inside the block runs with the
next norm (RMSNorm.add_forward: one kernel in inference)."""
from __future__ import annotations

import torch
import torch.nn as nn

from .layers import RMSNorm, SwiGLU
from .selective_attention import SelectiveMHA
from .ssm import SSM


class CausalBlock(nn.Module):
    def __init__(self, layer_idx: int, model_dim: int = 512, head_dim: int = 64,
                 attn_log_gate_penalty: float = 2.0, ssm_state_dim: int = 128,
                 ssm_conv_kernel_size: int = 4, ssm_num_groups: int = 1,
                 ssm_chunk_size: int = 256, dropout_rate: float = 0.15, device="cuda"):
        super().__init__()
        self.layer_idx = layer_idx
        self.norm1 = RMSNorm(model_dim)
        self.norm2 = RMSNorm(model_dim)
        self.norm3 = RMSNorm(model_dim)
        self.ssm = SSM(layer_idx=layer_idx, model_dim=model_dim, state_dim=ssm_state_dim,
                       conv_kernel_size=ssm_conv_kernel_size, head_dim=head_dim,
                       num_groups=ssm_num_groups, chunk_size=ssm_chunk_size,
                       dropout_rate=dropout_rate, device=device)
        self.mha = SelectiveMHA(layer_idx=layer_idx, dim=model_dim, head_dim=head_dim,
                                log_gate_penalty=attn_log_gate_penalty, is_causal=True)
        self.ffn = SwiGLU(model_dim, model_dim * 4)
        self.dropout = nn.Dropout(dropout_rate)

    def forward(self, hidden_states: torch.Tensor, lengths: torch.Tensor | None = None,
                attn_gate_threshold=None, cache=None, analysis_cfg=None, stats=None):
        """(batch, seq_len, model_dim) -> (hidden_states, last_ssm_hiddens)."""
        h, last = self.ssm(self.norm1(hidden_states), lengths=lengths,
                           cache=cache.ssm_cache if cache is not None else None)
        hidden_states, n = self.norm2.add_forward(hidden_states, self.dropout(h))
        h = self.mha(n, lengths=lengths, attn_gate_threshold=attn_gate_threshold,
                     cache=cache.attn_cache if cache is not None else None)
        hidden_states, n = self.norm3.add_forward(hidden_states, self.dropout(h))
        hidden_states = hidden_states + self.dropout(self.ffn(n))
        return hidden_states, last

    def step(self, hidden_states: torch.Tensor, cache, state, gen_cfg, analysis_cfg=None,
             stats=None, pending=None, defer_add: bool = False):
        """(batch, model_dim) -> (batch, model_dim).  A model stepping its
        blocks may leave each block's last residual add to the next: `pending`
        is added to hidden_states first (with norm1, one kernel), and with
        defer_add the block returns (hidden_states, ffn output) unsummed."""
        if pending is None:
            n = self.norm1(hidden_states)
        else:
            hidden_states, n = self.norm1.add_forward(hidden_states, pending)
        h = self.ssm.step(n, cache.ssm_cache)
        hidden_states, n = self.norm2.add_forward(hidden_states, self.dropout(h))
        h = self.mha.step(n, cache.attn_cache, state, gen_cfg)
        hidden_states, n = self.norm3.add_forward(hidden_states, self.dropout(h))
        f = self.dropout(self.ffn(n))
        return (hidden_states, f) if defer_add else hidden_states + f
