"""The encoder and decoder blocks of the seq2seq LM: BiBlock
(modules/bi_block.py:10-94: SSM, bidirectional SelectiveMHA, SwiGLU) and
CrossBlock (modules/cross_block.py:10-173: SSM seeded with the encoder's
state, causal SelectiveMHA, CrossSelectiveMHA, SwiGLU), pre-norm residual,
with the reference's constructor arguments and forward / step interfaces."""
from __future__ import annotations

import torch
import torch.nn as nn

from .cross_selective_attention import CrossSelectiveMHA
from .layers import RMSNorm, SwiGLU
from .selective_attention import SelectiveMHA
from .ssm import SSM


def _ssm(layer_idx, model_dim, head_dim, state_dim, conv, groups, chunk, dropout, device):
    return SSM(layer_idx=layer_idx, model_dim=model_dim, state_dim=state_dim,
               conv_kernel_size=conv, head_dim=head_dim, num_groups=groups, chunk_size=chunk,
               dropout_rate=dropout, device=device)


class BiBlock(nn.Module):
    def __init__(self, layer_idx: int, model_dim: int = 512, head_dim: int = 64,
                 attn_log_gate_penalty: float = 2, ssm_state_dim: int = 128,
                 ssm_conv_kernel_size: int = 4, ssm_num_groups: int = 1,
                 ssm_chunk_size: int = 256, dropout_rate: float = 0.15, device="cuda"):
        super().__init__()
        self.layer_idx = layer_idx
        self.norm1, self.norm2, self.norm3 = RMSNorm(model_dim), RMSNorm(model_dim), RMSNorm(model_dim)
        self.ssm = _ssm(layer_idx, model_dim, head_dim, ssm_state_dim, ssm_conv_kernel_size,
                        ssm_num_groups, ssm_chunk_size, dropout_rate, device)
        self.mha = SelectiveMHA(layer_idx=layer_idx, dim=model_dim, head_dim=head_dim,
                                log_gate_penalty=attn_log_gate_penalty, is_causal=False)
        self.ffn = SwiGLU(model_dim, model_dim * 4)
        self.dropout = nn.Dropout(dropout_rate)

    def forward(self, hidden_states: torch.Tensor, lengths: torch.Tensor | None = None,
                attn_gate_threshold=None, analysis_cfg=None, stats=None):
        """(batch, seq_len, model_dim) -> (hidden_states, last_ssm_hiddens)."""
        h, last = self.ssm(self.norm1(hidden_states), lengths=lengths)
        hidden_states, n = self.norm2.add_forward(hidden_states, self.dropout(h))
        h = self.mha(n, lengths=lengths, attn_gate_threshold=attn_gate_threshold)
        hidden_states, n = self.norm3.add_forward(hidden_states, self.dropout(h))
        hidden_states = hidden_states + self.dropout(self.ffn(n))
        return hidden_states, last


class CrossBlock(nn.Module):
    def __init__(self, layer_idx: int, model_dim: int = 512, head_dim: int = 64,
                 attn_log_gate_penalty: float = 2, ssm_state_dim: int = 128,
                 ssm_conv_kernel_size: int = 4, ssm_num_groups: int = 1,
                 ssm_chunk_size: int = 256, dropout_rate: float = 0.15, device="cuda"):
        super().__init__()
        self.layer_idx = layer_idx
        self.norm1, self.norm2 = RMSNorm(model_dim), RMSNorm(model_dim)
        self.norm3, self.norm4 = RMSNorm(model_dim), RMSNorm(model_dim)
        self.ssm = _ssm(layer_idx, model_dim, head_dim, ssm_state_dim, ssm_conv_kernel_size,
                        ssm_num_groups, ssm_chunk_size, dropout_rate, device)
        self.mha = SelectiveMHA(layer_idx=layer_idx, dim=model_dim, head_dim=head_dim,
                                log_gate_penalty=attn_log_gate_penalty, is_causal=True)
        self.cross_mha = CrossSelectiveMHA(layer_idx=layer_idx, dim=model_dim, head_dim=head_dim,
                                           log_gate_penalty=attn_log_gate_penalty)
        self.ffn = SwiGLU(model_dim, model_dim * 4)
        self.dropout = nn.Dropout(dropout_rate)

    def forward(self, hidden_states: torch.Tensor, context: torch.Tensor,
                context_lengths: torch.Tensor, ssm_hiddens: torch.Tensor,
                self_attn_gate_threshold=None, cross_attn_gate_threshold=None, cache=None,
                analysis_cfg=None, stats=None):
        """(batch, seq_len, model_dim) -> (batch, seq_len, model_dim)."""
        h, _ = self.ssm(self.norm1(hidden_states), ssm_hiddens=ssm_hiddens,
                        cache=cache.ssm_cache if cache is not None else None)
        hidden_states, n = self.norm2.add_forward(hidden_states, self.dropout(h))
        h = self.mha(n, attn_gate_threshold=self_attn_gate_threshold,
                     cache=cache.attn_cache if cache is not None else None)
        hidden_states, n = self.norm3.add_forward(hidden_states, self.dropout(h))
        h = self.cross_mha(n, context=context, context_lengths=context_lengths,
                           attn_gate_threshold=cross_attn_gate_threshold,
                           cache=cache.cross_attn_cache if cache is not None else None)
        hidden_states, n = self.norm4.add_forward(hidden_states, self.dropout(h))
        return hidden_states + self.dropout(self.ffn(n))

    def step(self, hidden_states: torch.Tensor, cache, state, gen_cfg, analysis_cfg=None,
             stats=None, pending=None, defer_add: bool = False):
        """(batch, model_dim) -> (batch, model_dim); pending / defer_add as in
        CausalBlock.step (the last residual add left to the next block)."""
        if pending is None:
            n = self.norm1(hidden_states)
        else:
            hidden_states, n = self.norm1.add_forward(hidden_states, pending)
        h = self.ssm.step(n, cache.ssm_cache)
        hidden_states, n = self.norm2.add_forward(hidden_states, self.dropout(h))
        h = self.mha.step(n, cache.attn_cache, state, gen_cfg)
        hidden_states, n = self.norm3.add_forward(hidden_states, self.dropout(h))
        h = self.cross_mha.step(n, cache.cross_attn_cache, gen_cfg)
        hidden_states, n = self.norm4.add_forward(hidden_states, self.dropout(h))
        f = self.dropout(self.ffn(n))
        return (hidden_states, f) if defer_add else hidden_states + f
