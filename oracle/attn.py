"""CPU restatement of the attention ops (block-sparse varlen prefill, paged GQA decode).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The reference has no kernel for either op (its attention is dense torch,
modules/selective_attention.py); these follow its gated-softmax semantics
with the BASELINE's sparsity / paging:

  prefill (_build_attn_matrix :86-95, _gated_softmax mode="seq" :125-144):
      s_ij = (q_i . k_j) * scale + [j != i] * bias_j,  -inf for j > i,
      o_i  = softmax_j(s_i.) v
    restricted to keys of the query's own sequence whose 64-key block is in
    the query block's selection list.
  decode (SelectiveMHA.step :399-405, _gated_softmax mode="pos" :121-123):
      s_j = (q . k_j) * scale + [j != last] * bias_j,  o = softmax_j(s) v
    over the seq_len cached keys reached through the page table; query head
    h reads kv head h // (Hq / Hkv) (GQA).

A query with no admissible key gets a zero output.
"""
from __future__ import annotations

import math

import torch


def sparse_attn_varlen(q, k, v, cu_seqlens, block_idx, block_size=64, softmax_scale=None,
                       key_bias=None, dtype=torch.float64):
    """q, k, v (T, H, D); cu_seqlens (nseq+1,) int; block_idx (H, n_qblk, M) int,
    local key-block indices (-1 = unused); key_bias (H, T) or None.
    Returns o (T, H, D) in `dtype`."""
    T, H, D = q.shape
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(D)
    cu = [int(x) for x in cu_seqlens.tolist()]
    qf, kf, vf = q.to(dtype), k.to(dtype), v.to(dtype)
    o = torch.zeros((T, H, D), dtype=dtype)
    qblk = 0
    for s in range(len(cu) - 1):
        a, b = cu[s], cu[s + 1]
        n = b - a
        nb = math.ceil(n / block_size)
        if n == 0:
            continue
        pos = torch.arange(n)
        causal = pos[:, None] >= pos[None, :]
        blk_of_key = pos // block_size
        for h in range(H):
            sel = block_idx[h, qblk:qblk + nb].to(torch.int64)           # (nb, M)
            allowed_blocks = torch.zeros((nb, nb), dtype=torch.bool)
            for j in range(nb):
                ids = sel[j][sel[j] >= 0]
                allowed_blocks[j, ids] = True
            allow = allowed_blocks[blk_of_key[:, None], blk_of_key[None, :]] & causal
            sc = (qf[a:b, h] @ kf[a:b, h].T) * scale
            if key_bias is not None:
                bias = key_bias[h, a:b].to(dtype)[None, :].expand(n, n).clone()
                bias[pos, pos] = 0.0
                sc = sc + bias
            sc = sc.masked_fill(~allow, float("-inf"))
            m = sc.max(dim=-1, keepdim=True).values
            p = torch.where(allow, torch.exp(sc - torch.where(torch.isinf(m), 0.0, m)), 0.0)
            den = p.sum(-1, keepdim=True)
            o[a:b, h] = torch.where(den > 0, (p @ vf[a:b, h]) / torch.where(den > 0, den, 1.0), 0.0)
        qblk += nb
    return o


def paged_decode_attn(q, k_pages, v_pages, page_table, seq_lens, softmax_scale=None,
                      key_bias=None, dtype=torch.float64):
    """q (b, Hq, D); k_pages (num_pages, Hkv, page_size, D); v_pages
    (num_pages, Hkv, D, page_size) (V stored transposed per page);
    page_table (b, max_pages) int; seq_lens (b,) int; key_bias
    (num_pages, Hkv, page_size) or None.  Returns o (b, Hq, D) in `dtype`."""
    b, Hq, D = q.shape
    Hkv, ps = k_pages.shape[1], k_pages.shape[2]
    grp = Hq // Hkv
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(D)
    o = torch.zeros((b, Hq, D), dtype=dtype)
    for i in range(b):
        n = int(seq_lens[i])
        if n <= 0:
            continue
        npg = math.ceil(n / ps)
        pages = page_table[i, :npg].to(torch.int64)
        K = k_pages[pages].to(dtype)                                        # (npg, Hkv, ps, D)
        V = v_pages[pages].to(dtype).transpose(-1, -2)                      # (npg, Hkv, ps, D)
        K = K.permute(1, 0, 2, 3).reshape(Hkv, npg * ps, D)[:, :n]
        V = V.permute(1, 0, 2, 3).reshape(Hkv, npg * ps, D)[:, :n]
        K = K.repeat_interleave(grp, dim=0)
        V = V.repeat_interleave(grp, dim=0)
        sc = torch.einsum("hd,hnd->hn", q[i].to(dtype), K) * scale
        if key_bias is not None:
            kb = key_bias[pages].to(dtype).permute(1, 0, 2).reshape(Hkv, npg * ps)[:, :n]
            kb = kb.repeat_interleave(grp, dim=0).clone()
            kb[:, n - 1] = 0.0
            sc = sc + kb
        p = torch.softmax(sc, dim=-1)
        o[i] = torch.einsum("hn,hnd->hd", p, V)
    return o
