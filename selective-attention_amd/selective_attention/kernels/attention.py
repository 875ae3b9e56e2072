"""Launchers of the attention ops (no counterpart kernel in the reference).

sparse_attn_varlen: varlen block-sparse causal self-attention over packed
sequences.  paged_decode_attn: split-KV paged GQA decode
attention.  Semantics follow the reference's gated
softmax (modules/selective_attention.py:99-144): an optional per-key bias
(the log-gate) is added to every score except the query's own position
(prefill) / the newest key (decode).
"""
from __future__ import annotations

import math

import torch

from .. import _lib
from .common import require_device


def _i32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.int32 and t.is_contiguous() else t.to(torch.int32).contiguous()


def sparse_attn_varlen(q, k, v, cu_seqlens, block_idx, block_size=64, softmax_scale=None,
                       key_bias=None):
    """
    Args:
        q, k, v: (total_tokens, num_heads, head_dim) bfloat16, sequences packed
        cu_seqlens: (num_seqs + 1,) int32 offsets of the sequences
        block_idx: (num_heads, n_qblk, max_blocks) int32.  Query blocks are the
            64-token blocks of each sequence, numbered sequence by sequence;
            entries are key-block indices local to the query's sequence
            (block j = positions [64j, 64j+64)), -1 for unused slots.
            Blocks after the query block and out-of-range entries are ignored;
            a row is a set (an id repeated in it is attended once).  Query
            blocks past the last row select nothing (zero outputs); rows past
            the packing's query blocks are never read.
        key_bias: (num_heads, total_tokens) float32 or None: added to the score
            of key j for every query except j itself.

    Returns:
        o: (total_tokens, num_heads, head_dim), dtype of q.  A query with no
        admissible key (its diagonal block not selected, nothing else either)
        gets zeros.
    """
    require_device(q, k, v, cu_seqlens, block_idx, key_bias)
    T, H, D = q.shape
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise TypeError("sparse_attn_varlen: q, k, v must be bfloat16")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    cu = _i32(cu_seqlens)
    idx = _i32(block_idx)
    bias = None if key_bias is None else key_bias.to(torch.float32).contiguous()
    o = torch.empty_like(q)
    scale = -1.0 if softmax_scale is None else float(softmax_scale)
    _lib.call("sa_sparse_attn_fwd", _lib.DTYPE_BF16, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v),
              _lib.ptr(cu), cu.shape[0] - 1, _lib.ptr(idx), idx.shape[1], idx.shape[2],
              int(block_size), _lib.ptr(bias), T, H, D, scale, _lib.ptr(o), _lib.stream_of(q))
    return o


ATTN_MODES = {"causal": 0, "full": 1, "cross": 2}


def attn_varlen(q, k, v, cu_seqlens_q, mode="causal", cu_seqlens_k=None, key_bias=None,
                softmax_scale=None):
    """
    Dense varlen attention over packed sequences (sa_attn_varlen_fwd).

    Args:
        q: (total_q, num_heads, head_dim) bfloat16; k, v: (total_k, num_heads, head_dim)
        cu_seqlens_q: (num_seqs + 1,) int32 query offsets
        mode: "causal" (keys j <= i of the own sequence), "full" (every key
            of the own sequence) or "cross" (every key of the sequence's range
            in cu_seqlens_k)
        key_bias: (num_heads, total_k) float32 or None, added to every score
            except the query's own key ("causal", "full") or key 0 of the key
            sequence ("cross")

    Returns:
        o: (total_q, num_heads, head_dim) bfloat16; a query with no key gets zeros.
    """
    require_device(q, k, v, cu_seqlens_q, cu_seqlens_k, key_bias)
    if mode not in ATTN_MODES:
        raise ValueError(f"attn_varlen: mode {mode!r} not in {sorted(ATTN_MODES)}")
    Tq, H, D = q.shape
    Tk = k.shape[0]
    for t in (q, k, v):
        if t.dtype != torch.bfloat16:
            raise TypeError("attn_varlen: q, k, v must be bfloat16")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    cu_q = _i32(cu_seqlens_q)
    cu_k = None if cu_seqlens_k is None else _i32(cu_seqlens_k)
    bias = None if key_bias is None else key_bias.to(torch.float32).contiguous()
    o = torch.empty_like(q)
    scale = -1.0 if softmax_scale is None else float(softmax_scale)
    _lib.call("sa_attn_varlen_fwd", _lib.DTYPE_BF16, ATTN_MODES[mode], _lib.ptr(q), _lib.ptr(k),
              _lib.ptr(v), _lib.ptr(cu_q), _lib.ptr(cu_k), cu_q.shape[0] - 1, _lib.ptr(bias), Tq, Tk,
              H, D, scale, _lib.ptr(o), _lib.stream_of(q))
    return o


def paged_decode_attn(q, k_pages, v_pages, page_table, seq_lens, softmax_scale=None,
                      key_bias=None):
    """
    Args:
        q: (batch, num_q_heads, head_dim) bfloat16
        k_pages: (num_pages, num_kv_heads, page_size, head_dim) bfloat16
        v_pages: (num_pages, num_kv_heads, head_dim, page_size) bfloat16 -- V is
            kept transposed per page, so its MFMA operand is read straight from
            HBM (the layout vLLM also uses for its V cache)
        page_table: (batch, max_pages) int32, page ids of each row in order
            (entries past the row's last page are ignored; -1 by convention)
        seq_lens: (batch,) int32 cached tokens per row
        key_bias: (num_pages, num_kv_heads, page_size) float32 or None: added to
            every key's score except the newest (position seq_len - 1)

    Returns:
        o: (batch, num_q_heads, head_dim) bfloat16; query head h reads kv head
        h // (num_q_heads // num_kv_heads).
    """
    require_device(q, k_pages, v_pages, page_table, seq_lens, key_bias)
    b, Hq, D = q.shape
    num_pages, Hkv, ps, D2 = k_pages.shape
    if D2 != D or tuple(v_pages.shape) != (num_pages, Hkv, D, ps):
        raise ValueError("paged_decode_attn: k_pages / v_pages / q shapes disagree")
    for t in (q, k_pages, v_pages):
        if t.dtype != torch.bfloat16:
            raise TypeError("paged_decode_attn: q, k_pages, v_pages must be bfloat16")
    q = q.contiguous()
    k_pages, v_pages = k_pages.contiguous(), v_pages.contiguous()
    pt = _i32(page_table)
    sl = _i32(seq_lens)
    bias = None if key_bias is None else key_bias.to(torch.float32).contiguous()
    max_pages = pt.shape[1]
    lib = _lib.load()
    nbytes = lib.sa_paged_decode_workspace_size(b, Hq, Hkv, D, max_pages)
    ws = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=q.device)
    o = torch.empty_like(q)
    scale = -1.0 if softmax_scale is None else float(softmax_scale)
    _lib.call("sa_paged_decode_fwd", _lib.DTYPE_BF16, _lib.ptr(q), _lib.ptr(k_pages),
              _lib.ptr(v_pages), _lib.ptr(pt), _lib.ptr(sl), _lib.ptr(bias), b, Hq, Hkv, D, ps,
              max_pages, num_pages, scale, _lib.ptr(o), _lib.ptr(ws), ws.numel(),
              _lib.stream_of(q))
    return o


def score_stats(q, k, q_lengths=None, k_lengths=None, causal=True, softmax_scale=None):
    """Per-head (count, sum, sum of squares) of the valid attention scores
    scale * q.k, the statistics of the training forwards of SelectiveMHA
    (modules/selective_attention.py:234-246) and CrossSelectiveMHA
    (modules/cross_selective_attention.py:129-146), reduced in-kernel without
    forming the score matrix.

    Args:
        q: (batch, heads, q_len, head_dim), k: (batch, heads, k_len, head_dim),
            bfloat16 or float32; head_dim 32, 64, 96 or 128
        q_lengths, k_lengths: (batch,) or None; queries / keys at or past a
            row's length are left out (None: every position)
        causal: leave out keys after the query (q_len == k_len)
    Returns:
        (heads, 3) float64 on the device: count, sum, sum of squares
    """
    from .common import act_dtype_code
    require_device(q, k, q_lengths, k_lengths)
    if q.dim() != 4 or k.dim() != 4 or q.shape[:2] != k.shape[:2] or q.shape[3] != k.shape[3]:
        raise ValueError(f"score_stats: q {tuple(q.shape)} and k {tuple(k.shape)} must be "
                         "(batch, heads, len, head_dim) with matching batch, heads, head_dim")
    if q.dtype != k.dtype:
        raise ValueError("score_stats: q and k must share a dtype")
    b, H, Lq, D = q.shape
    Lk = k.shape[2]
    if causal and Lq != Lk:
        raise ValueError("score_stats: causal attention needs as many queries as keys")
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    code = act_dtype_code(q.dtype)
    q, k = q.contiguous(), k.contiguous()
    ql = None if q_lengths is None else q_lengths.to(torch.int64).contiguous()
    kl = None if k_lengths is None else k_lengths.to(torch.int64).contiguous()
    out = torch.empty((H, 3), dtype=torch.float64, device=q.device)
    lib = _lib.load()
    nbytes = lib.sa_score_stats_workspace_size(b, H, Lq)
    ws = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=q.device)
    _lib.call("sa_score_stats", code, _lib.ptr(q), _lib.ptr(k), _lib.ptr(ql), _lib.ptr(kl), b, H,
              Lq, Lk, D, 1 if causal else 0, scale, _lib.ptr(ws), nbytes, _lib.ptr(out),
              _lib.stream_of(q))
    return out
