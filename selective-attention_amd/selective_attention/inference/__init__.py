"""Inference state of the causal LM: the same containers as the reference's
`selective_attention.inference` (ssm_cache.py:3-43, selective_attn_cache.py:3-42,
causal_block_cache.py, infer_state.py:4-14, generation_config.py:5-14), with
SelectiveMHA's KV cache kept in pages (PagedSelectiveAttnCache) instead of
dense per-head compacted tensors.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List

import torch

from ..ops.selective_mha import PagedSelectiveAttnCache
from ..ops.ssm_io import build_conv_ctx as _build_conv_ctx


class SSMCache:
    """inference/ssm_cache.py:3-43: the conv context (batch, channels, K) of
    raw in_proj rows and the SSM state h (batch, heads, head_dim, state_dim)."""

    def __init__(self):
        self.h = None
        self.conv_ctx = None

    def build_conv_ctx(self, x: torch.Tensor, lengths: torch.Tensor | None, cache_size: int):
        """x (batch, channels, seq_len) as in the reference (a transposed view
        of (batch, seq_len, channels) memory is read in place)."""
        self.conv_ctx = _build_conv_ctx(x.transpose(1, 2), lengths, cache_size)

    def update(self, x: torch.Tensor):
        """Shift the context and append x (batch, channels).  SSM.step does
        this inside the conv-step kernel; this method is for callers that
        keep the reference's two-call sequence."""
        self.conv_ctx = torch.roll(self.conv_ctx, shifts=-1, dims=-1)
        self.conv_ctx[:, :, -1] = x


class SelectiveAttnCache:
    """inference/selective_attn_cache.py:3-42 on pages.

    build_kv / update_kv keep the reference's names.  Keys are never
    compacted: a key whose gate is dropped keeps its slot with a -inf gate,
    and compact() (the reference's _reset_cache, modules/selective_attention.py:
    11-25) frees pages whose keys every head has dropped.  `reserve` is the
    number of decode tokens the pages are sized for beyond the prefill; the
    pool doubles when it runs out.
    """

    def __init__(self, reserve: int = 256, page_size: int = 64):
        self.reserve = reserve
        self.page_size = page_size
        self.pages: PagedSelectiveAttnCache | None = None

    def _make(self, b, H, D, tokens, device):
        self.pages = PagedSelectiveAttnCache(b, H, D, tokens + self.reserve + 1, device,
                                             page_size=self.page_size, grow=True)

    def build_kv(self, k_rot, v, log_gate, lengths=None):
        """k_rot, v (batch, heads, seq_len, head_dim); log_gate (batch, heads, seq_len)."""
        b, H, L, D = k_rot.shape
        self._make(b, H, D, L, k_rot.device)
        self.pages.build(k_rot, v, log_gate, lengths)

    def update_kv(self, k_rot, v, log_gate):
        """k_rot, v (batch, heads, head_dim); log_gate (batch, heads)."""
        if self.pages is None:
            b, H, D = k_rot.shape
            self._make(b, H, D, 0, k_rot.device)
        self.pages.append(k_rot, v, log_gate)

    def attend(self, q_rot):
        return self.pages.attend(q_rot)

    def prepare_decode(self, steps: int, like: torch.Tensor | None = None):
        """Fix the pages for `steps` more tokens and keep lengths on the device
        (PagedSelectiveAttnCache.enter_device_mode) so that decode steps can be
        captured in a graph.  `like` (batch, heads, head_dim) sizes a cache that
        prefill did not build."""
        if self.pages is None:
            b, H, D = like.shape
            self._make(b, H, D, 0, like.device)
        self.pages.enter_device_mode(steps)

    def compact(self) -> int:
        return 0 if self.pages is None else self.pages.drop_evicted_pages()

    @property
    def write_idx(self) -> int:
        """Tokens held by the longest row (the reference's cache length)."""
        if self.pages is None:
            return 0
        if self.pages.lens_dev is not None:
            return int(self.pages.lens_dev.max())
        return max(self.pages.lens)


class CrossSelectiveAttnCache:
    """inference/cross_selective_attn_cache.py: the context's keys and values
    for the decoder's cross-attention, here as (batch * context_len, heads,
    head_dim) bf16 rows with the per-key bias (heads, batch * context_len)
    and the key offsets cu_k (batch + 1,), and the same context as decode
    pages.  Filled at prefill, read-only while decoding."""

    def __init__(self):
        self.k = None
        self.v = None
        self.key_bias = None
        self.cu_k = None
        self.pages = None   # (k_pages, v_pages, page_table, seq_lens, gate_pages) for decode


class CrossBlockCache:
    """inference/cross_block_cache.py: SSM, self-attention and cross-attention caches."""

    def __init__(self, reserve: int = 256):
        self.ssm_cache = SSMCache()
        self.attn_cache = SelectiveAttnCache(reserve)
        self.cross_attn_cache = CrossSelectiveAttnCache()


class CausalBlockCache:
    """inference/causal_block_cache.py: one SSM cache and one attention cache per block."""

    def __init__(self, reserve: int = 256):
        self.ssm_cache = SSMCache()
        self.attn_cache = SelectiveAttnCache(reserve)


class InferenceState:
    """inference/infer_state.py:4-14: decode step counter and per-row lengths."""

    def __init__(self, lengths: torch.Tensor):
        self.step = 0
        self.lengths = lengths

    def update(self):
        self.step += 1
        self.lengths += 1


@dataclass
class GenerationConfig:
    """inference/generation_config.py:5-14."""
    bos_token_id: int
    eos_token_id: int
    pad_token_id: int
    max_new_tokens: int = 256
    attn_gate_thresholds: torch.Tensor | List | None = None    # (num_layers, num_heads)
    cross_attn_gate_thresholds: torch.Tensor | List | None = None
    enc_attn_gate_thresholds: torch.Tensor | List | None = None
    cache_update_interval: int = 100


__all__ = ["SSMCache", "SelectiveAttnCache", "CrossSelectiveAttnCache", "CausalBlockCache",
           "CrossBlockCache", "InferenceState", "GenerationConfig"]
