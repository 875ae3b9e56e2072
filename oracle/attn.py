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
    Returns o (T, H, D) in `dtype`.

    A row of block_idx is a set of key blocks: a repeated id counts once, and
    ids outside the sequence's blocks are ignored.  Query blocks past the
    last row of block_idx select nothing (zero outputs)."""
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
            sel = block_idx[h, qblk:qblk + nb].to(torch.int64)           # (<= nb, M)
            allowed_blocks = torch.zeros((nb, nb), dtype=torch.bool)
            for j in range(sel.shape[0]):
                ids = sel[j][(sel[j] >= 0) & (sel[j] < nb)]
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


def sparse_attn_varlen_blocks(q, k, v, cu_seqlens, block_idx, seqs, heads=None, block_size=64,
                              softmax_scale=None, key_bias=None, dtype=torch.float64):
    """sparse_attn_varlen restricted to the sequences `seqs` (indices into
    cu_seqlens) and the heads `heads` (default all), computed block by block:
    each query block gathers only its selected key blocks, so the work is
    the selected (query, key) pairs instead of a dense n x n matrix per
    sequence.  Same semantics (a repeated id counts once, ids outside the
    sequence's blocks or after the query block select nothing, the
    diagonal block is causal, key_bias skips the query's own key).
    Returns {seq: o (n, len(heads), D)} in `dtype`."""
    T, H, D = q.shape
    heads = list(range(H)) if heads is None else list(heads)
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(D)
    bs = block_size
    cu = [int(x) for x in cu_seqlens.tolist()]
    qblk0 = [0]
    for s in range(len(cu) - 1):
        qblk0.append(qblk0[-1] + math.ceil((cu[s + 1] - cu[s]) / bs))
    out = {}
    for s in seqs:
        a, b = cu[s], cu[s + 1]
        n = b - a
        nb = math.ceil(n / bs)
        res = torch.zeros((n, len(heads), D), dtype=dtype)
        if n == 0:
            out[s] = res
            continue
        pad = nb * bs - n
        qpos = torch.arange(nb * bs).view(nb, bs)                   # query position in the sequence
        for hi, h in enumerate(heads):
            rows = block_idx[h, qblk0[s]:qblk0[s] + nb].to(torch.int64)
            if rows.shape[0] < nb:                                    # missing rows select nothing
                rows = torch.cat([rows, torch.full((nb - rows.shape[0], rows.shape[1]), -1,
                                                   dtype=torch.int64)])
            M = rows.shape[1]
            ok = (rows >= 0) & (rows < nb) & (rows <= torch.arange(nb)[:, None])
            # a repeated id counts once: keep the first slot that holds it
            dup = torch.zeros_like(ok)
            for m in range(1, M):
                dup[:, m] = (rows[:, m:m + 1] == rows[:, :m]).any(-1)
            ok &= ~dup
            ids = torch.where(ok, rows, 0)
            qs = torch.nn.functional.pad(q[a:b, h].to(dtype), (0, 0, 0, pad)).view(nb, bs, D)
            ks = torch.nn.functional.pad(k[a:b, h].to(dtype), (0, 0, 0, pad)).view(nb, bs, D)
            vs = torch.nn.functional.pad(v[a:b, h].to(dtype), (0, 0, 0, pad)).view(nb, bs, D)
            kg, vg = ks[ids], vs[ids]                                 # (nb, M, bs, D)
            kpos = ids[:, :, None] * bs + torch.arange(bs)            # (nb, M, bs)
            sc = torch.einsum("jqd,jmkd->jqmk", qs, kg) * scale       # (nb, bs, M, bs)
            if key_bias is not None:
                kb = torch.nn.functional.pad(key_bias[h, a:b].to(dtype), (0, pad)).view(nb, bs)[ids]
                own = kpos[:, None, :, :] == qpos[:, :, None, None]
                sc = sc + torch.where(own, torch.zeros((), dtype=dtype), kb[:, None, :, :])
            allow = (ok[:, None, :, None] & (kpos[:, None, :, :] <= qpos[:, :, None, None])
                     & (kpos[:, None, :, :] < n) & (qpos[:, :, None, None] < n))
            sc = sc.masked_fill(~allow, float("-inf")).reshape(nb, bs, M * bs)
            m = sc.max(dim=-1, keepdim=True).values
            p = torch.where(allow.reshape(nb, bs, M * bs),
                            torch.exp(sc - torch.where(torch.isinf(m), 0.0, m)), 0.0)
            den = p.sum(-1, keepdim=True)
            o = torch.einsum("jqk,jkd->jqd", p, vg.reshape(nb, M * bs, D))
            o = torch.where(den > 0, o / torch.where(den > 0, den, 1.0), 0.0)
            res[:, hi] = o.reshape(nb * bs, D)[:n]
        out[s] = res
    return out


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
        # query heads h = kv * grp + j read kv head kv: (Hkv, grp, D) against (Hkv, n, D)
        qg = q[i].to(dtype).view(Hkv, grp, D)
        sc = torch.matmul(qg, K.transpose(-1, -2)) * scale                 # (Hkv, grp, n)
        if key_bias is not None:
            kb = key_bias[pages].to(dtype).permute(1, 0, 2).reshape(Hkv, npg * ps)[:, :n].clone()
            kb[:, n - 1] = 0.0
            sc = sc + kb[:, None, :]
        p = torch.softmax(sc, dim=-1)
        o[i] = torch.matmul(p, V).reshape(Hq, D)
    return o



def selective_mha_log_gate(select_gate, score_std, penalty, threshold=None, lengths=None):
    """log_select_gate of SelectiveMHA.forward in inference
    (modules/selective_attention.py:198-200, :259-267): gates below the
    per-head threshold become 0; log(gate) * score_std * penalty; -inf past a
    length.  select_gate (b, H, L); score_std, threshold (H,)."""
    g = select_gate.to(torch.float64).clone()
    if threshold is not None:
        g[g < threshold.to(torch.float64)[None, :, None]] = 0.0
    lg = torch.log(g) * score_std.to(torch.float64)[None, :, None] * penalty
    if lengths is not None:
        pad = torch.arange(g.shape[-1])[None, :] >= lengths.to(torch.int64)[:, None]
        lg = lg.masked_fill(pad[:, None, :], float("-inf"))
    return lg


def selective_mha_prefill_ref(q_rot, k_rot, v, log_gate, lengths=None, dtype=torch.float64):
    """SelectiveMHA.forward's inference attention (modules/selective_attention.py:
    222-290), restated in the form of its compressed branch (_build_attn_matrix
    :63-83, _gated_softmax :125-127, the output :279-281): query t attends the
    keys j < t whose gate is kept (finite log_gate), each with its log_gate,
    plus its own key without it (the self-score column).

    q_rot, k_rot, v (b, H, L, D); log_gate (b, H, L) from
    selective_mha_log_gate.  Returns (b, H, L, D); rows past a length are 0.
    """
    b, H, L, D = q_rot.shape
    scale = D ** -0.5
    q, k, vv = (t.to(dtype) for t in (q_rot, k_rot, v))
    lg = log_gate.to(dtype)
    lens = [L] * b if lengths is None else [int(x) for x in lengths.tolist()]
    out = torch.zeros(b, H, L, D, dtype=dtype)
    for i in range(b):
        n = lens[i]
        for h in range(H):
            kept = torch.nonzero(torch.isfinite(lg[i, h, :n])).flatten()
            for t in range(n):
                js = kept[kept < t]
                s = torch.cat([(k[i, h, js] @ q[i, h, t]) * scale + lg[i, h, js],
                               ((q[i, h, t] @ k[i, h, t]) * scale).reshape(1)])
                w = torch.softmax(s, 0)
                out[i, h, t] = w[:-1] @ vv[i, h, js] + w[-1] * vv[i, h, t]
    return out


def selective_mha_decode_ref(q_rot, k_cache, v_cache, log_gate_cache, dtype=torch.float64):
    """SelectiveMHA.step's attention (modules/selective_attention.py:399-405,
    _gated_softmax mode "pos" :121-123): softmax over the cached keys with
    the gate on every key but the newest.  q_rot (b, H, D); caches
    (b, H, n, D) / (b, H, n).  Keys with a -inf gate drop out, as the
    reference's compaction (_reset_cache :11-25) drops them."""
    D = q_rot.shape[-1]
    s = torch.einsum("bhd,bhnd->bhn", q_rot.to(dtype), k_cache.to(dtype)) * D ** -0.5
    s[..., :-1] = s[..., :-1] + log_gate_cache[..., :-1].to(dtype)
    return torch.einsum("bhn,bhnd->bhd", torch.softmax(s, -1), v_cache.to(dtype))


def attn_varlen(q, k, v, cu_q, mode="causal", cu_k=None, key_bias=None, softmax_scale=None,
                dtype=torch.float64):
    """Dense varlen attention in three modes (the attention of SelectiveMHA
    is_causal=True / False, modules/selective_attention.py:27-144, and of
    CrossSelectiveMHA, modules/cross_selective_attention.py:100-157):
      causal  query i sees keys j <= i of its sequence, bias not on j = i
      full    every key of its sequence, bias not on j = i
      cross   every key of cu_k[s]..cu_k[s+1], bias not on that range's key 0
    q (Tq, H, D); k, v (Tk, H, D); key_bias (H, Tk) or None.  Returns (Tq, H, D);
    a query with no key gets zeros."""
    Tq, H, D = q.shape
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(D)
    cq = [int(x) for x in cu_q.tolist()]
    ck = cq if mode != "cross" else [int(x) for x in cu_k.tolist()]
    qf, kf, vf = q.to(dtype), k.to(dtype), v.to(dtype)
    o = torch.zeros((Tq, H, D), dtype=dtype)
    for s in range(len(cq) - 1):
        a, b, ka, kb = cq[s], cq[s + 1], ck[s], ck[s + 1]
        n, nk = b - a, kb - ka
        if n <= 0 or nk <= 0:
            continue
        qi = torch.arange(n)[:, None]
        kj = torch.arange(nk)[None, :]
        allow = (kj <= qi) if mode == "causal" else torch.ones(n, nk, dtype=torch.bool)
        exempt = (kj == 0).expand(n, nk) if mode == "cross" else (kj == qi)
        for h in range(H):
            sc = (qf[a:b, h] @ kf[ka:kb, h].T) * scale
            if key_bias is not None:
                bias = key_bias[h, ka:kb].to(dtype)[None, :].expand(n, nk)
                sc = sc + torch.where(exempt, torch.zeros_like(bias), bias)
            sc = sc.masked_fill(~allow, float("-inf"))
            o[a:b, h] = torch.softmax(sc, dim=-1) @ vf[ka:kb, h]
    return o


def score_stats(q, k, scale, q_lengths=None, k_lengths=None, causal=True, dtype=torch.float64):
    """Per-head (count, sum, sum of squares) of the valid attention scores,
    the training statistics of SelectiveMHA (modules/selective_attention.py:234-246)
    and CrossSelectiveMHA (cross_selective_attention.py:129-146):
    s_ij = scale * q_i . k_j over pairs with i < q_length, j < k_length (when
    given) and j <= i (causal).  q (batch, heads, q_len, head_dim), k (batch,
    heads, k_len, head_dim).  Returns (heads, 3) in `dtype`."""
    q, k = q.to(dtype), k.to(dtype)
    b, H, Lq, _ = q.shape
    Lk = k.shape[2]
    s = torch.matmul(q, k.transpose(-2, -1)) * scale
    valid = torch.ones(b, 1, Lq, Lk, dtype=torch.bool)
    if causal:
        valid &= torch.tril(torch.ones(Lq, Lk, dtype=torch.bool))
    if q_lengths is not None:
        valid &= (torch.arange(Lq)[None, :] < q_lengths.to(torch.int64).cpu()[:, None])[:, None, :, None]
    if k_lengths is not None:
        valid &= (torch.arange(Lk)[None, :] < k_lengths.to(torch.int64).cpu()[:, None])[:, None, None, :]
    valid = valid.expand(b, H, Lq, Lk)
    sv = torch.where(valid, s, torch.zeros_like(s))
    return torch.stack([valid.sum(dim=(0, 2, 3)).to(dtype), sv.sum(dim=(0, 2, 3)),
                        (sv * sv).sum(dim=(0, 2, 3))], dim=1)


def score_std(stats):
    """The reference's per-head std from (count, sum, sum of squares)
    (:239-247): mean = sum / max(count, 1), var = sumsq / max(count, 1) -
    mean^2, std = sqrt(max(var, 0))."""
    cnt = stats[:, 0].clamp(min=1)
    mean = stats[:, 1] / cnt
    return (stats[:, 2] / cnt - mean * mean).clamp(min=0).sqrt()


def selective_mha_train_attn(q_rot, k_rot, v, select_gate, penalty, lengths=None, causal=True,
                             dtype=torch.float64):
    """The attention of SelectiveMHA's training forward (:197-277), as the
    reference composes it, in `dtype` and differentiable: scores scale * q.k
    (-inf above the diagonal when causal), the per-head std of the valid
    scores (through which gradients flow), log-gate = log(select_gate) * std
    * penalty (-inf at padded keys), added to every score but the diagonal,
    softmax over keys, times v.  q_rot, k_rot, v (batch, heads, seq_len,
    head_dim); select_gate (batch, heads, seq_len).  Returns (out (batch,
    heads, seq_len, head_dim), std (heads,))."""
    q, k, vv, sg = (x.to(dtype) for x in (q_rot, k_rot, v, select_gate))
    b, H, L, D = q.shape
    scale = D ** -0.5
    s = torch.matmul(q, k.transpose(-2, -1)) * scale
    ninf = torch.tensor(float("-inf"), dtype=dtype)
    if causal:
        s = torch.where(torch.tril(torch.ones(L, L, dtype=torch.bool)), s, ninf)
    valid = torch.isfinite(s)
    pad = None
    if lengths is not None:
        ok = torch.arange(L)[None, :] < lengths.to(torch.int64).cpu()[:, None]
        pad = ~ok
        valid = valid & ok[:, None, :, None] & ok[:, None, None, :]
    cnt = valid.sum(dim=(0, 2, 3)).to(dtype)
    sv = torch.where(valid, s, torch.zeros((), dtype=dtype))
    mean = sv.sum(dim=(0, 2, 3)) / cnt.clamp(min=1)
    var = (sv * sv).sum(dim=(0, 2, 3)) / cnt.clamp(min=1) - mean * mean
    std = var.clamp(min=0).sqrt()
    lg = torch.log(sg) * std[None, :, None] * penalty
    if pad is not None:
        lg = lg.masked_fill(pad[:, None, :], float("-inf"))
    diag = torch.eye(L, dtype=torch.bool)
    s = torch.where(diag, s, s + lg[:, :, None, :])
    return torch.softmax(s, dim=-1) @ vv, std
