"""CrossSelectiveMHA (modules/cross_selective_attention.py:35-258), inference,
on the cross mode of the attention kernel.

Decoder queries attend every key of their row's context, each key with
log(gate) * score_std_ema * penalty as its bias, except the context's key 0,
which carries none (_gated_softmax :8-32, step :233-236).  At prefill (a
cache is given) key 0's gate is 1, padding and keys below the threshold are
dropped (:102-118: the reference compresses them away; here they carry bias
-inf); without a cache the reference applies no threshold (:119-125), and
neither does this module.  The context keys, values and biases are kept in
the cache for the decode steps, which run the same kernel with one query per
row.  No RoPE, as in the reference.  Training raises NotImplementedError (no
attention backward kernel).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from ..ops.attention import attn_varlen
from .selective_attention import _threshold


class CrossSelectiveMHA(nn.Module):
    def __init__(self, layer_idx: int, dim: int, head_dim: int, log_gate_penalty: float):
        super().__init__()
        self.layer_idx = layer_idx
        assert dim % head_dim == 0
        self.dim = dim
        self.num_heads = dim // head_dim
        self.head_dim = head_dim
        self.scale = head_dim ** -0.5
        self.log_gate_penalty = log_gate_penalty
        self.q_proj = nn.Linear(dim, dim, bias=False)
        self.k_proj = nn.Linear(dim, dim, bias=False)
        self.v_proj = nn.Linear(dim, dim)
        self.out_proj = nn.Linear(dim, dim)
        self.select_gate_proj = nn.Linear(dim, self.num_heads)
        self.register_buffer("score_std_ema", torch.zeros(self.num_heads))
        nn.init.constant_(self.select_gate_proj.bias, 2.0)

    def _context(self, context, context_lengths, threshold, prefill):
        """Keys and values as (b * Lc, H, D) bf16 rows, the bias as (H, b * Lc)
        float32 and the key offsets (b + 1,) int32."""
        b, Lc, _ = context.shape
        dev = context.device
        H, D = self.num_heads, self.head_dim
        gate = torch.sigmoid(self.select_gate_proj(context)).float().transpose(1, 2)   # (b, H, Lc)
        first = torch.arange(Lc, device=dev) == 0
        if prefill:
            gate = torch.where(first[None, None, :], torch.ones_like(gate), gate)
        kept = gate > 0.0
        if context_lengths is not None:
            kept &= (torch.arange(Lc, device=dev)[None, :] < context_lengths.to(dev)[:, None])[:, None, :]
        thr = _threshold(threshold, H, dev) if prefill else None
        if thr is not None:
            kept &= (gate >= thr[None, :, None]) | first[None, None, :]
        lg = torch.log(gate) * self.score_std_ema.float()[None, :, None] * self.log_gate_penalty
        lg = torch.where(kept, lg, torch.full_like(lg, float("-inf")))
        k = self.k_proj(context).to(torch.bfloat16).reshape(b * Lc, H, D)
        v = self.v_proj(context).to(torch.bfloat16).reshape(b * Lc, H, D)
        cu_k = torch.arange(b + 1, dtype=torch.int32, device=dev) * Lc
        return k, v, lg.transpose(0, 1).reshape(H, b * Lc).contiguous(), cu_k

    def forward(self, hidden_states: torch.Tensor, context: torch.Tensor,
                context_lengths: torch.Tensor | None = None, attn_gate_threshold=None, cache=None,
                analysis_cfg=None, stats=None):
        """
        Args:
            hidden_states: (batch_size, seq_len, dim); context: (batch_size, context_len, dim)
            context_lengths: (batch_size,); attn_gate_threshold: (num_heads,) or a float
            cache: CrossSelectiveAttnCache filled for decoding, or None
        Returns:
            hidden_states: (batch_size, seq_len, dim)
        """
        if self.training:
            raise NotImplementedError(
                "CrossSelectiveMHA: the training forward needs an attention backward kernel, "
                "which is not built; use eval() for inference")
        b, L, _ = hidden_states.shape
        H, D = self.num_heads, self.head_dim
        k, v, bias, cu_k = self._context(context, context_lengths, attn_gate_threshold,
                                         cache is not None)
        q = self.q_proj(hidden_states).to(torch.bfloat16).reshape(b * L, H, D)
        cu_q = torch.arange(b + 1, dtype=torch.int32, device=q.device) * L
        out = attn_varlen(q, k, v, cu_q, "cross", cu_k, key_bias=bias)
        if cache is not None:
            cache.k, cache.v, cache.key_bias, cache.cu_k = k, v, bias, cu_k
        return self.out_proj(out.view(b, L, self.dim).to(hidden_states.dtype))

    def step(self, hidden_states: torch.Tensor, cache, gen_cfg, analysis_cfg=None, stats=None):
        """hidden_states (batch_size, dim) -> (batch_size, dim)."""
        b = hidden_states.shape[0]
        H, D = self.num_heads, self.head_dim
        q = self.q_proj(hidden_states).to(torch.bfloat16).reshape(b, H, D)
        cu_q = torch.arange(b + 1, dtype=torch.int32, device=q.device)
        out = attn_varlen(q, cache.k, cache.v, cu_q, "cross", cache.cu_k, key_bias=cache.key_bias)
        return self.out_proj(out.view(b, self.dim).to(hidden_states.dtype))
