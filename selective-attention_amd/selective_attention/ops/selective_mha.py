"""SelectiveMHA's attention (inference) on the gfx950 attention ops.

The reference computes SelectiveMHA's gated attention densely in torch
(modules/selective_attention.py): _build_attn_matrix (:27-97) and
_gated_softmax (:99-144) for prefill, SelectiveMHA.step (:392-405) over a
per-head compacted cache (inference/selective_attn_cache.py,
_reset_cache :11-25) for decode.  Here the same attention runs on the new
ops:

* selective_mha_prefill: each batch row is one sequence for the dense
  causal mode of attn_varlen (the block-sparse kernel over every causal
  block).  The gate
  enters as key_bias = log_gate (the diagonal is exempt, as in mode "seq").
  A key the reference drops from its compressed cache (gate zeroed or below
  the threshold, or past the length) carries key_bias = -inf, which removes
  it from the softmax exactly as compression does, while the query's own key
  stays in unbiased (the reference's self-score column).
* PagedSelectiveAttnCache: the decode cache as 64-token bf16 pages shared
  by every head of a batch row, with the gate of each cached key kept as
  key_bias pages (-inf for dropped keys; the newest key is exempt, as in
  mode "pos").  Compaction becomes a page-table rewrite: drop_evicted_pages
  removes pages whose keys every head has dropped, without moving data.

* ScoreStdFn: the per-head std of the valid scores that SelectiveMHA's
  training forward scales the log-gate by (:234-247).  Its forward is the
  in-kernel reduction score_stats (count, sum, sum of squares, no score
  matrix); its backward carries d std_h / d s_ij = (s_ij - mean_h) /
  (count_h std_h) to q and k by query chunks.
* gated_attention_train, cross_attention_train: the training attention
  itself, the reference's dense gated softmax under autograd (there is no
  attention backward kernel here), in fp32.
"""
from __future__ import annotations

import torch

from ..kernels.attention import score_stats
from ..kernels.lm_ops import paged_kv_append, paged_kv_build
from .attention import attn_varlen, paged_decode_attn


def _valid_pairs(Lk: int, q_lengths, k_lengths, causal: bool, i0: int, i1: int, device):
    """(batch or 1, 1, i1 - i0, Lk) mask of the valid (query, key) pairs for
    queries i0..i1-1: key <= query when causal, query and key inside their
    row lengths (None: every position)."""
    qi = torch.arange(i0, i1, device=device)[:, None]
    kj = torch.arange(Lk, device=device)[None, :]
    m = (kj <= qi) if causal else torch.ones(i1 - i0, Lk, dtype=torch.bool, device=device)
    m = m[None, None]
    if q_lengths is not None:
        m = m & (qi[None, None] < q_lengths.to(device=device, dtype=torch.int64)[:, None, None, None])
    if k_lengths is not None:
        m = m & (kj[None, None] < k_lengths.to(device=device, dtype=torch.int64)[:, None, None, None])
    return m


class ScoreStdFn(torch.autograd.Function):
    """std_h of the valid scores s_ij = scale q_i . k_j of head h over every
    batch row (modules/selective_attention.py:234-247,
    cross_selective_attention.py:129-146: mean = sum / count, var = sumsq /
    count - mean^2 clamped at 0, std = sqrt(var)), differentiable in q and k.

    forward(q, k, q_lengths, k_lengths, causal, chunk): q (batch, heads,
    q_len, head_dim), k (batch, heads, k_len, head_dim); returns (heads,)
    float32.  A head whose std is 0 passes no gradient back (the reference's
    sqrt would give inf * 0).
    """

    @staticmethod
    def forward(ctx, q, k, q_lengths=None, k_lengths=None, causal=True, chunk=256):
        st = score_stats(q, k, q_lengths, k_lengths, causal)
        cnt = st[:, 0].clamp(min=1)
        mean = st[:, 1] / cnt
        std = (st[:, 2] / cnt - mean * mean).clamp(min=0).sqrt()
        ctx.save_for_backward(q, k, mean, std, cnt)
        ctx.q_lengths, ctx.k_lengths, ctx.causal, ctx.chunk = q_lengths, k_lengths, causal, chunk
        return std.to(torch.float32)

    @staticmethod
    def backward(ctx, g):
        q, k, mean, std, cnt = ctx.saved_tensors
        Lq, D = q.shape[2], q.shape[3]
        Lk = k.shape[2]
        scale = D ** -0.5
        coef = torch.where(std > 0, g.double() / (cnt * std.clamp(min=1e-300)),
                           torch.zeros_like(std)).float()[None, :, None, None]
        mu = mean.float()[None, :, None, None]
        kf = k.float()
        dq = torch.zeros(q.shape, dtype=torch.float32, device=q.device)
        dk = torch.zeros(k.shape, dtype=torch.float32, device=k.device)
        for i0 in range(0, Lq, ctx.chunk):
            i1 = min(Lq, i0 + ctx.chunk)
            qc = q[:, :, i0:i1].float()
            s = torch.matmul(qc, kf.transpose(-2, -1).contiguous()) * scale
            valid = _valid_pairs(Lk, ctx.q_lengths, ctx.k_lengths, ctx.causal, i0, i1, q.device)
            gs = torch.where(valid, (s - mu) * coef, torch.zeros((), device=q.device))
            dq[:, :, i0:i1] = torch.matmul(gs, kf) * scale
            dk += torch.matmul(gs.transpose(-2, -1).contiguous(), qc) * scale
        return dq.to(q.dtype), dk.to(k.dtype), None, None, None, None


def gated_attention_train(q_rot, k_rot, v, log_gate, causal=True):
    """SelectiveMHA's training attention (modules/selective_attention.py:86-95,
    125-144): softmax_j(scale q_i . k_j + [j != i] log_gate_j) v_j with keys
    after the query at -inf when causal; dense, in fp32, under autograd.
    q_rot, k_rot, v (batch, heads, seq_len, head_dim); log_gate (batch,
    heads, seq_len).  Returns (batch, heads, seq_len, head_dim) float32."""
    L, D = q_rot.shape[-2], q_rot.shape[-1]
    s = torch.matmul(q_rot.float(), k_rot.float().transpose(-2, -1).contiguous()) * D ** -0.5
    diag = torch.eye(L, dtype=torch.bool, device=s.device)
    s = torch.where(diag, s, s + log_gate.float()[:, :, None, :])
    if causal:
        s = s.masked_fill(~torch.tril(torch.ones(L, L, dtype=torch.bool, device=s.device)),
                          float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), v.float())


def selective_mha_prefill(q_rot: torch.Tensor, k_rot: torch.Tensor, v: torch.Tensor,
                          log_gate: torch.Tensor, lengths: torch.Tensor | None = None,
                          block_size: int = 64) -> torch.Tensor:
    """
    Args (the module's tensors after RoPE, modules/selective_attention.py:250-255):
        q_rot, k_rot, v: (batch_size, num_heads, seq_len, head_dim) bf16; a
            (batch_size, seq_len, num_heads, head_dim) tensor transposed to
            this shape is read in place, any other layout is copied once
        log_gate: (batch_size, num_heads, seq_len), log(select_gate) * score_std *
            penalty; -inf for keys the reference drops (gate zeroed or below the
            threshold)
        lengths: (batch_size,) or None
    Returns:
        out: (batch_size, num_heads, seq_len, head_dim) bf16, a transposed view of
        (batch_size, seq_len, num_heads, head_dim) memory (the layout the
        module's output projection reads); rows past a length are 0.

    Each batch row is one sequence (cu_seqlens = 0, L, 2L, ...; with
    lengths, its valid rows and its padding rows are two sequences), so
    nothing is packed or copied: a query t < length only reaches keys j <= t
    of its row.  block_size is kept for the signature (the kernel's blocks
    are 64 keys).
    """
    b, H, L, D = q_rot.shape
    dev = q_rot.device
    T = b * L
    if T == 0:
        return torch.zeros(b, L, H, D, dtype=torch.bfloat16, device=dev).transpose(1, 2)

    def rows(x):   # (b, H, L, D) -> (b * L, H, D) rows, in place when possible
        return x.transpose(1, 2).to(torch.bfloat16).contiguous().view(T, H, D)

    qp, kp, vp = rows(q_rot), rows(k_rot), rows(v)
    bias = log_gate.to(torch.float32).transpose(0, 1).reshape(H, T)
    starts = torch.arange(b + 1, dtype=torch.int32, device=dev) * L
    if lengths is None:
        cu = starts
    else:
        # sequences [i L, i L + len_i) and, between them, the padding rows as
        # sequences of their own (attended among themselves, then zeroed)
        lens = lengths.to(dev, torch.int64).clamp(0, L)
        cu = torch.empty(2 * b + 1, dtype=torch.int32, device=dev)
        cu[0::2] = starts
        cu[1::2] = starts[:-1] + lens.to(torch.int32)
    o = attn_varlen(qp, kp, vp, cu, "causal", key_bias=bias).view(b, L, H, D)
    if lengths is not None:
        pad = torch.arange(L, device=dev)[None, :] >= lens[:, None]
        o.masked_fill_(pad[:, :, None, None], 0.0)
    return o.transpose(1, 2)


class PagedSelectiveAttnCache:
    """Paged decode cache of SelectiveMHA (one per layer).

    k / v pages: (num_pages, num_heads, page_size, head_dim) and
    (num_pages, num_heads, head_dim, page_size) bf16; gate pages
    (num_pages, num_heads, page_size) fp32; page_table (batch, max_pages)
    int32 and seq_lens (batch,) int32 index them.  Pages are allocated from a
    fixed pool; a batch row's tokens are in page order, its newest token last.
    """

    def __init__(self, batch_size: int, num_heads: int, head_dim: int, max_tokens: int,
                 device, page_size: int = 64, grow: bool = False):
        self.b, self.H, self.D, self.ps = batch_size, num_heads, head_dim, page_size
        self.grow = grow
        self.max_pages = max(1, (max_tokens + page_size - 1) // page_size)
        n = batch_size * self.max_pages
        self.k_pages = torch.zeros(n, num_heads, page_size, head_dim, dtype=torch.bfloat16, device=device)
        self.v_pages = torch.zeros(n, num_heads, head_dim, page_size, dtype=torch.bfloat16, device=device)
        self.gate_pages = torch.full((n, num_heads, page_size), float("-inf"), dtype=torch.float32,
                                     device=device)
        self.free = list(range(n - 1, -1, -1))
        self.rows = [[] for _ in range(batch_size)]   # page ids per batch row
        self.lens = [0] * batch_size
        self.device = device
        # device copies of the page table and lengths, refreshed when the host
        # bookkeeping changed since the last attend
        self._pt = None
        self._sl = None
        self._pt_dirty = self._sl_dirty = True
        # device mode (see enter_device_mode): lengths live on the device
        self.lens_dev = None

    # --- bookkeeping -------------------------------------------------------
    def _grow(self):
        """Double the page pool (rows keep their page ids; the page table gets
        twice the columns)."""
        n = self.k_pages.shape[0]
        dev = self.device

        def bigger(t, fill):
            out = torch.full((2 * n,) + tuple(t.shape[1:]), fill, dtype=t.dtype, device=dev)
            out[:n] = t
            return out
        self.k_pages = bigger(self.k_pages, 0)
        self.v_pages = bigger(self.v_pages, 0)
        self.gate_pages = bigger(self.gate_pages, float("-inf"))
        self.free = list(range(2 * n - 1, n - 1, -1)) + self.free
        self.max_pages *= 2
        self._pt_dirty = True

    def _alloc(self, fill: bool = True) -> int:
        """A free page; its gates are reset to -inf unless the caller writes
        every slot itself (or resets a batch of pages at once)."""
        if not self.free:
            if not self.grow:
                raise RuntimeError("PagedSelectiveAttnCache: page pool exhausted")
            self._grow()
        pid = self.free.pop()
        if fill:
            self.gate_pages[pid].fill_(float("-inf"))
        return pid

    def _slot(self, i: int, t: int):
        while len(self.rows[i]) * self.ps <= t:
            self.rows[i].append(self._alloc())
            self._pt_dirty = True
        return self.rows[i][t // self.ps], t % self.ps

    def page_table(self) -> torch.Tensor:
        """(batch, pages) int32 on the cache's device (at least max_pages columns).
        Columns past a row's pages repeat the row's last page id (0 for a row
        without pages, which the decode kernel never reads: its length is 0).
        The device-side append clamps its column to the table's width, and
        enter_device_mode gives every row at least one page, so an append past
        a row's pages lands in that row's own last page, never in another
        row's."""
        if self._pt_dirty or self._pt is None:
            width = max([self.max_pages] + [len(r) for r in self.rows])
            pt = torch.zeros(self.b, width, dtype=torch.int32)
            for i, r in enumerate(self.rows):
                if r:
                    pt[i, :len(r)] = torch.tensor(r, dtype=torch.int32)
                    pt[i, len(r):] = r[-1]
            self._pt = pt.to(self.device)
            self._pt_dirty = False
        return self._pt

    def seq_lens(self) -> torch.Tensor:
        """(batch,) int32 on the cache's device."""
        if self.lens_dev is not None:
            return self.lens_dev
        if self._sl_dirty or self._sl is None:
            self._sl = torch.tensor(self.lens, dtype=torch.int32).to(self.device)
            self._sl_dirty = False
        return self._sl

    # --- the reference's cache operations ------------------------------------
    def build(self, k_rot, v, log_gate, lengths=None):
        """SelectiveAttnCache.build_kv after prefill (selective_attn_cache.py:9-28):
        k_rot, v (batch, heads, seq_len, head_dim); log_gate (batch, heads, seq_len)."""
        L = k_rot.shape[2]
        lens = [L] * self.b if lengths is None else [min(int(x), L) for x in lengths.tolist()]
        H, D, ps = self.H, self.D, self.ps
        if k_rot.is_cuda:
            # pages of every row and head written by one kernel (every slot, no fills)
            for i in range(self.b):
                self.free.extend(self.rows[i])
                self.rows[i] = [self._alloc(fill=False) for _ in range((lens[i] + ps - 1) // ps)]
                self.lens[i] = lens[i]
            self._pt_dirty = self._sl_dirty = True
            paged_kv_build(k_rot, v, log_gate, self.page_table(), self.seq_lens(), self.k_pages,
                           self.v_pages, self.gate_pages)
            return
        for i in range(self.b):
            for pid in self.rows[i]:
                self.free.append(pid)
            n = lens[i]
            npg = (n + ps - 1) // ps
            pids = [self._alloc(fill=False) for _ in range(npg)]   # every slot written below
            self.rows[i] = pids
            self.lens[i] = n
            self._pt_dirty = self._sl_dirty = True
            if npg == 0:
                continue
            idx = torch.tensor(pids, device=self.device)
            kk = torch.zeros(H, npg * ps, D, dtype=torch.bfloat16, device=self.device)
            vv = torch.zeros_like(kk)
            gg = torch.full((H, npg * ps), float("-inf"), dtype=torch.float32, device=self.device)
            kk[:, :n] = k_rot[i, :, :n]
            vv[:, :n] = v[i, :, :n]
            gg[:, :n] = log_gate[i, :, :n].float()
            self.k_pages[idx] = kk.view(H, npg, ps, D).permute(1, 0, 2, 3)
            self.v_pages[idx] = vv.view(H, npg, ps, D).permute(1, 0, 3, 2)
            self.gate_pages[idx] = gg.view(H, npg, ps).permute(1, 0, 2)

    # --- device mode: appends without host work, for graph capture ---------
    def enter_device_mode(self, extra_tokens: int):
        """Give every row pages for `extra_tokens` more tokens, fix the page
        table, and keep the lengths on the device: append / unappend / attend
        then make no host round trip and no allocation that depends on host
        state, so a decode step can be captured in a graph and replayed.  At
        most `extra_tokens` appends may follow: the table's columns past a row's
        pages repeat its last page, so a row that runs past them overwrites
        slots of its own last page (wrong keys for that row alone, no fault)."""
        # every row gets at least one page of its own, so that a device-side
        # append (clamped to the table's width) never writes into page 0 of
        # another row, even for a row that had no tokens and no pages
        fresh = []
        for i in range(self.b):
            need = max(1, (self.lens[i] + max(extra_tokens, 0) + self.ps - 1) // self.ps)
            while len(self.rows[i]) < need:
                pid = self._alloc(fill=False)
                self.rows[i].append(pid)
                fresh.append(pid)
        if fresh:   # reset the new pages' gates in one launch
            self.gate_pages[torch.tensor(fresh, device=self.device)] = float("-inf")
            self._pt_dirty = True
        self.page_table()
        self.lens_dev = torch.tensor(self.lens, dtype=torch.int32).to(self.device)

    def exit_device_mode(self):
        self.lens = [int(x) for x in self.lens_dev.tolist()]
        self.lens_dev = None
        self._sl_dirty = True

    def _append_device(self, k_rot, v, log_gate):
        paged_kv_append(k_rot, v, log_gate, self._pt, self.lens_dev, self.k_pages, self.v_pages,
                        self.gate_pages)

    def append(self, k_rot, v, log_gate):
        """SelectiveAttnCache.update_kv (:30-47): one token per batch row;
        k_rot, v (batch, heads, head_dim); log_gate (batch, heads)."""
        if self.lens_dev is not None:
            return self._append_device(k_rot, v, log_gate)
        slots = [self._slot(i, self.lens[i]) for i in range(self.b)]
        idx = torch.tensor(slots, dtype=torch.int64).to(self.device)
        pid, s = idx[:, 0], idx[:, 1]
        self.k_pages[pid, :, s] = k_rot.to(torch.bfloat16)          # (batch, heads, head_dim)
        self.v_pages[pid, :, :, s] = v.to(torch.bfloat16)
        self.gate_pages[pid, :, s] = log_gate.to(torch.float32)     # (batch, heads)
        for i in range(self.b):
            self.lens[i] += 1
        self._sl_dirty = True

    def unappend(self, rows=None):
        """Drop the newest token again (SelectiveMHA.step :414-415 when no head
        keeps it)."""
        if self.lens_dev is not None:
            if rows is None:
                self.lens_dev -= 1
            else:
                self.lens_dev[torch.as_tensor(list(rows), device=self.device)] -= 1
            return
        for i in (range(self.b) if rows is None else rows):
            self.lens[i] -= 1
        self._sl_dirty = True

    def attend(self, q_rot) -> torch.Tensor:
        """softmax(q.k * scale + [not newest] * log_gate) v over the cached keys
        (modules/selective_attention.py:399-405); q_rot (batch, heads, head_dim)."""
        return paged_decode_attn(q_rot.to(torch.bfloat16).contiguous(), self.k_pages, self.v_pages,
                                 self.page_table(), self.seq_lens(), None, self.gate_pages)

    def drop_evicted_pages(self) -> int:
        """The reference's periodic compaction (_reset_cache :11-25) as a page
        table rewrite: every full page before the one holding the row's newest
        token whose keys all heads have dropped (-inf gate) leaves the row's
        page list (pages reserved past the newest token hold no tokens and
        stay).  Returns the number of pages freed (0 in device mode, where the
        page table is fixed)."""
        if self.lens_dev is not None:
            return 0
        # one device check for every candidate page of every row
        cand = [(i, j, pages[j]) for i, pages in enumerate(self.rows)
                for j in range(max(0, (self.lens[i] - 1) // self.ps))]
        if not cand:
            return 0
        ids = torch.tensor([pid for _, _, pid in cand], device=self.device)
        dead = torch.isinf(self.gate_pages[ids]).flatten(1).all(dim=1).tolist()
        drop = {(i, j) for (i, j, _), d in zip(cand, dead) if d}
        freed = 0
        for i in range(self.b):
            keep = []
            for j, pid in enumerate(self.rows[i]):
                if (i, j) in drop:
                    self.free.append(pid)
                    self.lens[i] -= self.ps
                    freed += 1
                else:
                    keep.append(pid)
            self.rows[i] = keep
        if freed:
            self._pt_dirty = self._sl_dirty = True
        return freed


def cross_attention_train(q, k, v, log_gate, k_lengths=None):
    """CrossSelectiveMHA's training attention (modules/cross_selective_attention.py:129-159):
    softmax_j(scale q_i . k_j + [j > 0] log_gate_j) v_j over the context keys,
    keys at or past a row's context length at -inf; dense, in fp32, under
    autograd.  q (batch, heads, q_len, head_dim); k, v (batch, heads,
    k_len, head_dim); log_gate (batch, heads, k_len).  Returns (batch, heads,
    q_len, head_dim) float32."""
    Lk, D = k.shape[2], k.shape[3]
    s = torch.matmul(q.float(), k.float().transpose(-2, -1).contiguous()) * D ** -0.5
    if k_lengths is not None:
        pad = torch.arange(Lk, device=s.device)[None, :] >= k_lengths.to(s.device)[:, None]
        s = s.masked_fill(pad[:, None, None, :], float("-inf"))
    bias = log_gate.float().clone()
    bias[..., 0] = 0.0
    s = s + bias[:, :, None, :]
    return torch.matmul(torch.softmax(s, dim=-1), v.float())
