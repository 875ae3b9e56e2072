"""Attention ops: varlen block-sparse prefill and paged GQA decode.

New ops (the reference computes attention densely in torch inside
SelectiveMHA, modules/selective_attention.py:177-446, with no kernel
boundary).  Validation follows the reference's op conventions: ndim/shape
errors raise ValueError before any launch.
"""
from __future__ import annotations

import torch

from ..kernels import attention as _k
from ..utils import check_ndim, check_shape


def sparse_attn_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       cu_seqlens: torch.Tensor, block_idx: torch.Tensor, block_size: int = 64,
                       softmax_scale: float | None = None,
                       key_bias: torch.Tensor | None = None) -> torch.Tensor:
    check_ndim(q, 3, name="q")
    T, H, D = q.shape
    check_shape(k, (T, H, D), name="k")
    check_shape(v, (T, H, D), name="v")
    check_ndim(cu_seqlens, 1, name="cu_seqlens")
    check_ndim(block_idx, 3, name="block_idx")
    if block_idx.shape[0] != H:
        raise ValueError(f"[block_idx] Shape mismatch: expected {H} heads, got {block_idx.shape[0]}")
    check_shape(key_bias, (H, T), name="key_bias", optional=True)
    return _k.sparse_attn_varlen(q, k, v, cu_seqlens, block_idx, block_size, softmax_scale,
                                 key_bias)


def paged_decode_attn(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                      page_table: torch.Tensor, seq_lens: torch.Tensor,
                      softmax_scale: float | None = None,
                      key_bias: torch.Tensor | None = None) -> torch.Tensor:
    check_ndim(q, 3, name="q")
    check_ndim(k_pages, 4, name="k_pages")
    npages, hkv, ps, hd = k_pages.shape
    check_shape(v_pages, (npages, hkv, hd, ps), name="v_pages")
    b = q.shape[0]
    check_ndim(page_table, 2, name="page_table")
    if page_table.shape[0] != b:
        raise ValueError(f"[page_table] Shape mismatch: expected batch {b}, got {page_table.shape[0]}")
    check_shape(seq_lens, (b,), name="seq_lens")
    if q.shape[1] % k_pages.shape[1] != 0:
        raise ValueError("num_q_heads must be a multiple of num_kv_heads")
    check_shape(key_bias, tuple(k_pages.shape[:3]), name="key_bias", optional=True)
    return _k.paged_decode_attn(q, k_pages, v_pages, page_table, seq_lens, softmax_scale, key_bias)
