"""SelectiveMHA (modules/selective_attention.py:146-446) on the gfx950
attention ops.

Parameters and interfaces follow the reference.  Prefill runs
selective_mha_prefill (the block-sparse kernel over every causal block with
the log-gate as key bias) and fills the paged cache; step appends to the
paged cache and runs the paged decode kernel.  A key whose gate is zeroed
(below the threshold, or past a length) enters as key bias -inf: the
reference's compression of the cache (its compressed branch, :63-83) drops
exactly those keys.  Writing the drop as -inf directly, instead of
log(0) * score_std * penalty, also keeps a zero score_std_ema (its value
before any training step) from turning dropped keys into NaN.

With is_causal=False (the encoder's BiBlock) every key of the sequence is
visible, the query's own key again exempt (the reference's self column /
self mask, :84-86); that variant has no decode step.

Training (:197-277): the per-head std of the valid scores comes from the
in-kernel statistics (ScoreStdFn: count, sum and sum of squares reduced
without a score matrix, differentiable), score_std_ema takes the running
average, the log-gate is log(gate) * std * penalty, and the gated softmax
runs densely in torch under autograd (this package has no attention
backward kernel).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from ..kernels.lm_ops import mha_gates
from ..ops.attention import attn_varlen
from ..ops.selective_mha import ScoreStdFn, gated_attention_train, selective_mha_prefill
from .layers import Linear, RoPE, project


def _threshold(thr, num_heads: int, device):
    if thr is None:
        return None
    if isinstance(thr, (int, float)):
        return torch.full((num_heads,), float(thr), device=device)
    return torch.as_tensor(thr, device=device).reshape(num_heads)


class SelectiveMHA(nn.Module):
    def __init__(self, layer_idx: int, dim: int, head_dim: int, log_gate_penalty: float,
                 is_causal: bool = True):
        super().__init__()
        self.layer_idx = layer_idx
        assert dim % head_dim == 0
        self.dim = dim
        self.num_heads = dim // head_dim
        self.head_dim = head_dim
        self.is_causal = is_causal
        self.scale = head_dim ** -0.5
        self.log_gate_penalty = log_gate_penalty

        self.gate_proj = Linear(dim, self.num_heads + dim)
        self.rope = RoPE(head_dim)
        self.q_proj = Linear(dim, dim, bias=False)
        self.k_proj = Linear(dim, dim, bias=False)
        self.v_proj = Linear(dim, dim)
        self.out_proj = Linear(dim, dim)
        self.register_buffer("score_std_ema", torch.zeros(self.num_heads))
        nn.init.constant_(self.gate_proj.bias, 2.0)

    def _gates(self, hidden_states):
        gate = torch.sigmoid(self.gate_proj(hidden_states))
        return torch.split(gate, [self.num_heads, self.dim], dim=-1)

    def _log_gate(self, select_gate, kept):
        """log(gate) * score_std_ema * penalty where kept, -inf elsewhere;
        select_gate (batch, heads[, seq_len]) -> float32."""
        std = self.score_std_ema.float()
        std = std[None, :, None] if select_gate.dim() == 3 else std[None, :]
        lg = torch.log(select_gate.float()) * std * self.log_gate_penalty
        return torch.where(kept, lg, torch.full_like(lg, float("-inf")))

    def forward(self, hidden_states: torch.Tensor, lengths: torch.Tensor | None = None,
                attn_gate_threshold: torch.Tensor | None = None, cache=None,
                analysis_cfg=None, stats=None):
        """
        Args:
            hidden_states: (batch_size, seq_len, dim)
            lengths: (batch_size,)
            attn_gate_threshold: (num_heads,) or a float
            cache: SelectiveAttnCache filled for decoding, or None
        Returns:
            hidden_states: (batch_size, seq_len, dim)
        """
        if self.training:
            return self._train_forward(hidden_states, lengths)
        b, L, _ = hidden_states.shape
        dev = hidden_states.device
        H, D = self.num_heads, self.head_dim
        select_gate, out_gate = self._gates(hidden_states)
        select_gate = select_gate.transpose(1, 2)                     # (b, H, L)
        thr = _threshold(attn_gate_threshold, H, dev)
        kept = select_gate > 0.0
        if thr is not None:
            kept &= select_gate >= thr[None, :, None]
        if lengths is not None:
            lens = lengths.to(dev)
            kept &= (torch.arange(L, device=dev)[None, :] < lens[:, None])[:, None, :]
        v = self.v_proj(hidden_states)
        if not bool(kept.any()):
            # every key dropped: each query attends only itself (:208-209)
            return self.out_proj(v * out_gate)
        q, k = self.rope.rotate_qk(self.q_proj(hidden_states).view(b, L, H, D),
                                   self.k_proj(hidden_states).view(b, L, H, D), None, L)
        q, k = q.transpose(1, 2), k.transpose(1, 2)                   # (b, H, L, D) views
        vh = v.view(b, L, H, D).to(torch.bfloat16).transpose(1, 2)
        log_gate = self._log_gate(select_gate, kept)
        if self.is_causal:
            out = selective_mha_prefill(q, k, vh, log_gate, lengths)
            if cache is not None:
                cache.build_kv(k, vh, log_gate, lengths)
            out = out.transpose(1, 2).reshape(b, L, self.dim)
        else:
            out = self._bidirectional(q, k, vh, log_gate, lengths)
        return self.out_proj(out.to(hidden_states.dtype) * out_gate)

    def _train_forward(self, hidden_states, lengths):
        """The reference's training forward (:197-277): no threshold, the
        current batch's score std in the log-gate (its gradient included),
        padded keys at -inf, the diagonal exempt."""
        b, L, _ = hidden_states.shape
        dev = hidden_states.device
        H, D = self.num_heads, self.head_dim
        select_gate, out_gate = self._gates(hidden_states)
        select_gate = select_gate.transpose(1, 2)                     # (b, H, L)
        v = self.v_proj(hidden_states)
        q = self.q_proj(hidden_states).view(b, L, H, D).transpose(1, 2)
        k = self.k_proj(hidden_states).view(b, L, H, D).transpose(1, 2)
        vh = v.view(b, L, H, D).transpose(1, 2)
        q_rot, k_rot = self.rope(q, k, torch.arange(L, device=dev), mode="seq")
        lens = None if lengths is None else lengths.to(dev)
        std = ScoreStdFn.apply(q_rot.contiguous(), k_rot.contiguous(), lens, lens, self.is_causal)
        with torch.no_grad():
            self.score_std_ema.mul_(0.9).add_(std.detach().to(self.score_std_ema.dtype), alpha=0.1)
        log_gate = torch.log(select_gate.float()) * std[None, :, None] * self.log_gate_penalty
        if lens is not None:
            pad = torch.arange(L, device=dev)[None, :] >= lens[:, None]
            log_gate = log_gate.masked_fill(pad[:, None, :], float("-inf"))
        out = gated_attention_train(q_rot, k_rot, vh, log_gate, self.is_causal)
        out = out.transpose(1, 2).reshape(b, L, self.dim).to(hidden_states.dtype)
        return self.out_proj(out * out_gate)

    def _bidirectional(self, q, k, v, log_gate, lengths):
        """Every key of the row (dropped and padded ones at -inf), the query's
        own key unbiased; q, k, v (b, H, L, D) views of (b, L, H, D) memory.
        Returns (b, L, dim) with rows past a length set to 0."""
        b, H, L, D = q.shape
        dev = q.device
        rows = lambda x: x.transpose(1, 2).contiguous().view(b * L, H, D)
        cu = torch.arange(b + 1, dtype=torch.int32, device=dev) * L
        bias = log_gate.transpose(0, 1).reshape(H, b * L)
        out = attn_varlen(rows(q), rows(k), rows(v), cu, "full", key_bias=bias).view(b, L, H * D)
        if lengths is not None:
            pad = torch.arange(L, device=dev)[None, :] >= lengths.to(dev)[:, None]
            out = out.masked_fill(pad[:, :, None], 0.0)
        return out

    def step(self, hidden_states: torch.Tensor, cache, state, gen_cfg, analysis_cfg=None,
             stats=None):
        """hidden_states (batch_size, dim) -> (batch_size, dim).  The new key
        always gets a slot; when no head of any row keeps it, its gate is -inf
        everywhere and it takes no weight in later steps, which is what the
        reference's write_idx rollback (:414-415) achieves."""
        if not self.is_causal:
            raise NotImplementedError("SelectiveMHA.step: the bidirectional variant has no decode step")
        b = hidden_states.shape[0]
        dev = hidden_states.device
        H, D = self.num_heads, self.head_dim
        thr = None
        if gen_cfg.attn_gate_thresholds is not None:
            thr = _threshold(gen_cfg.attn_gate_thresholds[self.layer_idx], H, dev)
        if state.step % gen_cfg.cache_update_interval == 0:
            cache.compact()
        g, q, k, v = project(hidden_states, [self.gate_proj, self.q_proj, self.k_proj, self.v_proj])
        if g.is_cuda and g.dtype == torch.bfloat16:
            # sigmoid, split, threshold and log-gate in one kernel
            log_gate, out_gate = mha_gates(g, thr, self.score_std_ema, self.log_gate_penalty, H)
        else:
            select_gate, out_gate = torch.split(torch.sigmoid(g), [H, self.dim], dim=-1)
            kept = select_gate > 0.0
            if thr is not None:
                kept &= select_gate >= thr[None, :]
            log_gate = self._log_gate(select_gate, kept)
        q, k, v = q.view(b, H, D), k.view(b, H, D), v.view(b, H, D)
        q, k = self.rope.rotate_qk(q, k, state.lengths.to(dev), b)
        cache.update_kv(k, v.to(torch.bfloat16), log_gate)
        out = cache.attend(q).reshape(b, self.dim).to(hidden_states.dtype)
        return project(out, [self.out_proj], xscale=out_gate)[0]
