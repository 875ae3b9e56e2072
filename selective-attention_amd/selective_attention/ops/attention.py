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


def attn_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_q: torch.Tensor,
                mode: str = "causal", cu_seqlens_k: torch.Tensor | None = None,
                key_bias: torch.Tensor | None = None,
                softmax_scale: float | None = None) -> torch.Tensor:
    """Dense varlen attention: causal or bidirectional self-attention of
    packed sequences, or cross-attention of packed queries over packed key
    sequences, with the gate's log as a per-key bias (see
    kernels.attention.attn_varlen)."""
    check_ndim(q, 3, name="q")
    Tq, H, D = q.shape
    check_ndim(k, 3, name="k")
    Tk = k.shape[0]
    check_shape(k, (Tk, H, D), name="k")
    check_shape(v, (Tk, H, D), name="v")
    check_ndim(cu_seqlens_q, 1, name="cu_seqlens_q")
    if mode == "cross":
        check_ndim(cu_seqlens_k, 1, name="cu_seqlens_k")
        check_shape(cu_seqlens_k, tuple(cu_seqlens_q.shape), name="cu_seqlens_k")
    elif Tk != Tq:
        raise ValueError(f"[k] self-attention needs as many keys as queries ({Tk} != {Tq})")
    check_shape(key_bias, (H, Tk), name="key_bias", optional=True)
    return _k.attn_varlen(q, k, v, cu_seqlens_q, mode, cu_seqlens_k, key_bias, softmax_scale)


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
