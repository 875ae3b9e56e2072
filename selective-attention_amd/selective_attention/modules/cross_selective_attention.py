"""CrossSelectiveMHA (modules/cross_selective_attention.py:35-258) on the
cross mode of the attention kernel.

Decoder queries attend every key of their row's context, each key with
log(gate) * score_std_ema * penalty as its bias, except the context's key 0,
which carries none (_gated_softmax :8-32, step :233-236).  At prefill (a
cache is given) key 0's gate is 1, padding and keys below the threshold are
dropped (:102-118: the reference compresses them away; here they carry bias
-inf); without a cache the reference applies no threshold (:119-125), and
neither does this module.  The context keys, values and biases are kept in
the cache for the decode steps, as pages for the split-KV paged decode
kernel (one query per row over the whole context spreads over every CU).
No RoPE, as in the reference.  Training (:88-161): the per-head std of the
valid scores (every query, keys inside the context length) comes from the
in-kernel statistics (ScoreStdFn), score_std_ema takes the running average,
and the gated softmax (key 0 unbiased, padded keys at -inf) runs densely in
torch under autograd (no attention backward kernel here).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from ..ops.attention import attn_varlen, paged_decode_attn
from ..ops.selective_mha import ScoreStdFn, cross_attention_train
from .layers import Linear
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
        self.q_proj = Linear(dim, dim, bias=False)
        self.k_proj = Linear(dim, dim, bias=False)
        self.v_proj = Linear(dim, dim)
        self.out_proj = Linear(dim, dim)
        self.select_gate_proj = Linear(dim, self.num_heads)
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
            return self._train_forward(hidden_states, context, context_lengths)
        b, L, _ = hidden_states.shape
        H, D = self.num_heads, self.head_dim
        k, v, bias, cu_k = self._context(context, context_lengths, attn_gate_threshold,
                                         cache is not None)
        q = self.q_proj(hidden_states).to(torch.bfloat16).reshape(b * L, H, D)
        cu_q = torch.arange(b + 1, dtype=torch.int32, device=q.device) * L
        out = attn_varlen(q, k, v, cu_q, "cross", cu_k, key_bias=bias)
        if cache is not None:
            cache.k, cache.v, cache.key_bias, cache.cu_k = k, v, bias, cu_k
            cache.pages = self._pages(k, v, bias, b, context.shape[1])
        return self.out_proj(out.view(b, L, self.dim).to(hidden_states.dtype))

    def _train_forward(self, hidden_states, context, context_lengths):
        """The reference's training forward (:88-161): the current batch's
        score std in the log-gate (its gradient included), no threshold."""
        b, L, _ = hidden_states.shape
        Lc = context.shape[1]
        dev = hidden_states.device
        H, D = self.num_heads, self.head_dim
        gate = torch.sigmoid(self.select_gate_proj(context)).transpose(1, 2)   # (b, H, Lc)
        q = self.q_proj(hidden_states).view(b, L, H, D).transpose(1, 2)
        k = self.k_proj(context).view(b, Lc, H, D).transpose(1, 2)
        v = self.v_proj(context).view(b, Lc, H, D).transpose(1, 2)
        lens = None if context_lengths is None else context_lengths.to(dev)
        std = ScoreStdFn.apply(q.contiguous(), k.contiguous(), None, lens, False)
        with torch.no_grad():
            self.score_std_ema.mul_(0.9).add_(std.detach().to(self.score_std_ema.dtype), alpha=0.1)
        log_gate = torch.log(gate.float()) * std[None, :, None] * self.log_gate_penalty
        out = cross_attention_train(q, k, v, log_gate, lens)
        return self.out_proj(out.transpose(1, 2).reshape(b, L, self.dim).to(hidden_states.dtype))

    def _pages(self, k, v, bias, b, Lc, ps=64):
        """The context as decode pages for the stream-K paged kernel: per row,
        keys 1 .. Lc-1, then padding (bias -inf), then key 0 in the row's last
        slot, the slot that kernel leaves unbiased (key 0's bias is 0 here
        anyway, so its exemption changes nothing)."""
        H, D = self.num_heads, self.head_dim
        dev = k.device
        npg = (Lc + ps - 1) // ps
        Lp = npg * ps
        kk = torch.zeros(b, Lp, H, D, dtype=torch.bfloat16, device=dev)
        vv = torch.zeros_like(kk)
        bb = torch.full((b, Lp, H), float("-inf"), dtype=torch.float32, device=dev)
        k3, v3 = k.view(b, Lc, H, D), v.view(b, Lc, H, D)
        b3 = bias.view(H, b, Lc).permute(1, 2, 0)
        kk[:, :Lc - 1], vv[:, :Lc - 1], bb[:, :Lc - 1] = k3[:, 1:], v3[:, 1:], b3[:, 1:]
        kk[:, Lp - 1], vv[:, Lp - 1], bb[:, Lp - 1] = k3[:, 0], v3[:, 0], b3[:, 0]
        k_pages = kk.view(b, npg, ps, H, D).permute(0, 1, 3, 2, 4).reshape(b * npg, H, ps, D).contiguous()
        v_pages = vv.view(b, npg, ps, H, D).permute(0, 1, 3, 4, 2).reshape(b * npg, H, D, ps).contiguous()
        g_pages = bb.view(b, npg, ps, H).permute(0, 1, 3, 2).reshape(b * npg, H, ps).contiguous()
        table = torch.arange(b * npg, dtype=torch.int32, device=dev).view(b, npg)
        lens = torch.full((b,), Lp, dtype=torch.int32, device=dev)
        return k_pages, v_pages, table, lens, g_pages

    def step(self, hidden_states: torch.Tensor, cache, gen_cfg, analysis_cfg=None, stats=None):
        """hidden_states (batch_size, dim) -> (batch_size, dim): one query per
        row over the context pages (split-KV paged decode kernel)."""
        b = hidden_states.shape[0]
        H, D = self.num_heads, self.head_dim
        q = self.q_proj(hidden_states).to(torch.bfloat16).reshape(b, H, D)
        k_pages, v_pages, table, lens, g_pages = cache.pages
        out = paged_decode_attn(q, k_pages, v_pages, table, lens, None, g_pages)
        return self.out_proj(out.reshape(b, self.dim).to(hidden_states.dtype))
