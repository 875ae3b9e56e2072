"""Attention ops: oracle pins (CPU), workload invariants (CPU), HIP parity (GPU)."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import attn as ref
from selective_attention import workloads
from tests.helpers import assert_parity

F64 = torch.float64


# ------------------------------------------------------------------ helpers
def full_causal_selection(lens, H, bs=64, M=None):
    nbs = [math.ceil(n / bs) for n in lens]
    M = M or max(nbs)
    rows = []
    for nb in nbs:
        for j in range(nb):
            r = list(range(j + 1)) + [-1] * (M - j - 1)
            rows.append(r)
    idx = torch.tensor(rows, dtype=torch.int32)
    return idx[None].expand(H, -1, -1).contiguous()


def packed(lens, H, D, seed=0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    T = sum(lens)
    q = torch.randn(T, H, D, generator=g).to(dtype)
    k = torch.randn(T, H, D, generator=g).to(dtype)
    v = torch.randn(T, H, D, generator=g).to(dtype)
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens), 0).to(torch.int32)
    return q, k, v, cu


# ------------------------------------------------------------ oracle pins
def test_oracle_sparse_full_selection_is_causal_sdpa():
    lens, H, D = [70, 130, 5], 2, 16
    q, k, v, cu = packed(lens, H, D, dtype=F64)
    idx = full_causal_selection(lens, H)
    o = ref.sparse_attn_varlen(q, k, v, cu, idx)
    for s in range(len(lens)):
        a, b = int(cu[s]), int(cu[s + 1])
        exp = F.scaled_dot_product_attention(q[a:b].transpose(0, 1), k[a:b].transpose(0, 1),
                                             v[a:b].transpose(0, 1), is_causal=True)
        torch.testing.assert_close(o[a:b], exp.transpose(0, 1), rtol=1e-10, atol=1e-12)


def test_oracle_sparse_brute_force_with_bias():
    lens, H, D, bs = [9, 6], 1, 4, 4
    q, k, v, cu = packed(lens, H, D, seed=3, dtype=F64)
    g = torch.Generator().manual_seed(4)
    bias = torch.randn(H, sum(lens), generator=g, dtype=F64)
    # query blocks: seq0 -> 3 blocks, seq1 -> 2 blocks; drop block 0 for q-block 2 of seq0
    idx = torch.tensor([[[0, -1, -1], [0, 1, -1], [1, 2, -1], [0, -1, -1], [0, 1, -1]]],
                       dtype=torch.int32)
    o = ref.sparse_attn_varlen(q, k, v, cu, idx, block_size=bs, key_bias=bias)
    sel = {0: {0}, 1: {0, 1}, 2: {1, 2}}
    for i in range(9):  # sequence 0 by hand
        keys = [j for j in range(i + 1) if j // bs in sel[i // bs]]
        sc = torch.tensor([float(q[i, 0] @ k[j, 0]) / 2.0 + (float(bias[0, j]) if j != i else 0.0)
                           for j in keys], dtype=F64)
        p = torch.softmax(sc, 0)
        exp = sum(p[t] * v[keys[t], 0] for t in range(len(keys)))
        torch.testing.assert_close(o[i, 0], exp, rtol=1e-10, atol=1e-12)


def test_oracle_decode_identity_pages_is_sdpa():
    b, Hq, Hkv, D, ps = 3, 4, 2, 8, 4
    g = torch.Generator().manual_seed(0)
    lens = [5, 12, 1]
    npg = [math.ceil(n / ps) for n in lens]
    kp = torch.randn(sum(npg), Hkv, ps, D, generator=g, dtype=F64)
    vp = torch.randn(sum(npg), Hkv, D, ps, generator=g, dtype=F64)
    q = torch.randn(b, Hq, D, generator=g, dtype=F64)
    table = torch.full((b, max(npg)), -1, dtype=torch.int32)
    o_ = 0
    for i, n in enumerate(npg):
        table[i, :n] = torch.arange(o_, o_ + n)
        o_ += n
    out = ref.paged_decode_attn(q, kp, vp, table, torch.tensor(lens), None)
    for i, n in enumerate(lens):
        rows = table[i, :npg[i]].long()
        K = kp[rows].permute(1, 0, 2, 3).reshape(Hkv, -1, D)[:, :n].repeat_interleave(2, 0)
        V = vp[rows].permute(1, 0, 3, 2).reshape(Hkv, -1, D)[:, :n].repeat_interleave(2, 0)
        exp = F.scaled_dot_product_attention(q[i][:, None], K, V)[:, 0]
        torch.testing.assert_close(out[i], exp, rtol=1e-10, atol=1e-12)


def test_oracle_decode_bias_spares_newest_key():
    g = torch.Generator().manual_seed(1)
    kp = torch.randn(2, 1, 4, 4, generator=g, dtype=F64)
    vp = torch.randn(2, 1, 4, 4, generator=g, dtype=F64)
    q = torch.randn(1, 1, 4, generator=g, dtype=F64)
    table = torch.tensor([[1, 0]], dtype=torch.int32)
    bias = torch.full((2, 1, 4), -1e9, dtype=F64)       # every key gated off ...
    out = ref.paged_decode_attn(q, kp, vp, table, torch.tensor([6]), None, key_bias=bias)
    # ... except the newest one (position 5 = page 0, slot 1), which is exempt
    torch.testing.assert_close(out[0, 0], vp[0, 0, :, 1], rtol=1e-10, atol=1e-12)


def test_oracle_sparse_blocks_equals_dense_restatement():
    """The block-gathered sparse oracle (used at config 2's full size) equals
    the dense one, with a bias, duplicated ids, ids past the query block and
    past the sequence, -1 padding and a short block_idx."""
    lens, H, D = [200, 90, 64, 1], 3, 16
    q, k, v, cu = packed(lens, H, D, seed=12, dtype=F64)
    g = torch.Generator().manual_seed(13)
    idx, _, _ = workloads.block_selection(lens, H, 64, 3, g)
    idx = _with_duplicates(idx, g)
    idx[0, 1, -1] = 3          # after its query block
    idx[1, 2, 0] = 9           # outside the sequence
    bias = torch.randn(H, sum(lens), generator=g, dtype=F64)
    bias[:, ::5] = float("-inf")
    for sel, kb in ((idx, bias), (idx[:, :-2], None)):
        dense = ref.sparse_attn_varlen(q, k, v, cu, sel, key_bias=kb)
        blk = ref.sparse_attn_varlen_blocks(q, k, v, cu, sel, range(len(lens)), key_bias=kb)
        for s in range(len(lens)):
            a, b = int(cu[s]), int(cu[s + 1])
            torch.testing.assert_close(blk[s], dense[a:b], rtol=1e-12, atol=1e-12)
    part = ref.sparse_attn_varlen_blocks(q, k, v, cu, idx, [1], heads=[2])
    torch.testing.assert_close(part[1], ref.sparse_attn_varlen(q, k, v, cu, idx)[200:290, 2:3],
                               rtol=1e-12, atol=1e-12)


# ------------------------------------------------------- workload invariants
def test_varlen_packing_and_selection_invariants():
    g = torch.Generator().manual_seed(0)
    lens = workloads.varlen_lengths(65536, 256, 8192, g)
    assert sum(lens) == 65536 and all(1 <= n <= 8192 for n in lens)
    assert all(n >= 256 for n in lens[:-1])
    idx, seq_of, loc_of = workloads.block_selection(lens, 16, 64, 16, g)
    assert idx.shape == (16, sum(math.ceil(n / 64) for n in lens), 16)
    for h in (0, 7, 15):
        for qb in range(0, idx.shape[1], 37):
            j = int(loc_of[qb])
            row = idx[h, qb]
            used = row[row >= 0].tolist()
            assert used == sorted(used) and len(set(used)) == len(used)
            assert j in used and (j == 0 or j - 1 in used)
            assert all(0 <= x <= j for x in used)
            assert len(used) == 1 + min(1, j) + min(14, max(j - 1, 0))
            assert (row[len(used):] == -1).all()


def test_workload_generators_are_bit_stable():
    """Seeded index tensors hash to committed values (bit-exact selection/offsets)."""
    import hashlib
    import json
    import os
    fx = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "workload_hashes.json")))
    w = workloads.sparse_attn_inputs(total_tokens=65536, nheads=16, headdim=128)
    h = lambda t: hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()  # noqa: E731
    assert h(w.cu_seqlens) == fx["config2_cu_seqlens"]
    assert h(w.block_idx) == fx["config2_block_idx"]
    d = workloads.decode_inputs(batch=64, nheads_q=2, nheads_kv=1, headdim=8, device="cpu")
    assert h(d.seq_lens) == fx["config3_seq_lens"]
    assert h(d.page_table) == fx["config3_page_table"]


def test_ops_validate_shapes():
    from selective_attention.ops import paged_decode_attn, sparse_attn_varlen
    q, k, v, cu = packed([10], 2, 16)
    idx = full_causal_selection([10], 2)
    with pytest.raises(ValueError):
        sparse_attn_varlen(q, k[:5], v, cu, idx)
    with pytest.raises(ValueError):
        sparse_attn_varlen(q, k, v, cu, idx[:1])
    kp = torch.zeros(3, 1, 64, 16, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        paged_decode_attn(q[:2], kp, kp.transpose(-1, -2), torch.zeros(3, 1, dtype=torch.int32),
                          torch.ones(2, dtype=torch.int32))
    with pytest.raises(ValueError):
        paged_decode_attn(q[:2], kp, kp, torch.zeros(2, 1, dtype=torch.int32),
                          torch.ones(2, dtype=torch.int32))   # V must be (np, Hkv, D, ps)


# --------------------------------------------------------------- GPU parity
def _run_sparse(q, k, v, cu, idx, bias=None):
    from selective_attention.ops import sparse_attn_varlen
    o = sparse_attn_varlen(q.cuda(), k.cuda(), v.cuda(), cu.cuda(), idx.cuda(),
                           key_bias=None if bias is None else bias.cuda())
    torch.cuda.synchronize()
    return o


@pytest.mark.gpu
@pytest.mark.parametrize("lens,D", [([64], 128), ([200, 37, 64, 129], 128), ([300, 1, 65], 64),
                                    ([513], 128)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_sparse_attn_parity_random_selection(lens, D, with_bias):
    print(f"sparse lens={lens} D={D} bias={with_bias}", flush=True)
    H = 3
    g = torch.Generator().manual_seed(11)
    q, k, v, cu = packed(lens, H, D, seed=5)
    idx, _, _ = workloads.block_selection(lens, H, 64, 6, g)
    bias = torch.randn(H, sum(lens), generator=g) if with_bias else None
    o = _run_sparse(q, k, v, cu, idx, bias)
    exp = ref.sparse_attn_varlen(q, k, v, cu, idx, key_bias=bias)
    assert_parity(o, exp, torch.bfloat16, "o")


@pytest.mark.gpu
def test_sparse_attn_full_selection_matches_causal():
    lens, H, D = [130, 260], 2, 128
    q, k, v, cu = packed(lens, H, D, seed=2)
    o = _run_sparse(q, k, v, cu, full_causal_selection(lens, H))
    exp = ref.sparse_attn_varlen(q, k, v, cu, full_causal_selection(lens, H))
    assert_parity(o, exp, torch.bfloat16, "o")


@pytest.mark.gpu
def test_sparse_attn_more_than_64_slots():
    """A selection row longer than one wave (71 slots): the valid blocks are
    found by the scalar scan instead of the wave ballot."""
    lens, H, D = [4500], 1, 64
    q, k, v, cu = packed(lens, H, D, seed=4)
    idx = full_causal_selection(lens, H)
    assert idx.shape[2] > 64
    o = _run_sparse(q, k, v, cu, idx)
    exp = ref.sparse_attn_varlen(q, k, v, cu, idx)
    assert_parity(o, exp, torch.bfloat16, "o")


@pytest.mark.gpu
def test_sparse_attn_missing_diagonal_gives_zero_rows():
    lens, H, D = [128], 1, 64
    q, k, v, cu = packed(lens, H, D)
    idx = torch.tensor([[[-1, -1], [-1, -1]]], dtype=torch.int32)   # nothing selected
    o = _run_sparse(q, k, v, cu, idx)
    assert torch.count_nonzero(o) == 0


def _with_duplicates(idx, g):
    """Copy each row's valid ids into its -1 slots (after the valid ones, so
    the first occurrences keep their order)."""
    out = idx.clone()
    H, nq, M = idx.shape
    for h in range(H):
        for j in range(nq):
            row = out[h, j]
            valid = row[row >= 0]
            free = (row < 0).nonzero().flatten()
            if len(valid) and len(free):
                pick = valid[torch.randint(len(valid), (len(free),), generator=g)]
                row[free] = pick
    return out


def test_oracle_sparse_selection_is_a_set():
    """Repeated ids count once; rows past the end of block_idx select nothing
    (the same as a row of -1)."""
    lens, H, D = [200, 90], 2, 16
    q, k, v, cu = packed(lens, H, D, seed=8, dtype=F64)
    g = torch.Generator().manual_seed(9)
    idx, _, _ = workloads.block_selection(lens, H, 64, 3, g)
    base = ref.sparse_attn_varlen(q, k, v, cu, idx)
    dup = _with_duplicates(idx, g)
    assert not torch.equal(dup, idx)
    torch.testing.assert_close(ref.sparse_attn_varlen(q, k, v, cu, dup), base, rtol=0, atol=0)
    short = idx[:, :-2]
    padded = idx.clone()
    padded[:, -2:] = -1
    torch.testing.assert_close(ref.sparse_attn_varlen(q, k, v, cu, short),
                               ref.sparse_attn_varlen(q, k, v, cu, padded), rtol=0, atol=0)
    # and the missing rows really are zero (the last two query blocks: seq 1)
    assert torch.count_nonzero(ref.sparse_attn_varlen(q, k, v, cu, short)[200:]) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("lens,M", [([300, 130, 64], 6), ([4500], 71)])
def test_sparse_attn_duplicate_ids_attend_once(lens, M):
    """A block id repeated in a row is attended once, at its first slot: the
    output equals, bit for bit, the run on the table that keeps only each
    id's first occurrence (same walk order), and the oracle's set semantics.
    M = 71 takes the scalar slot scan instead of the wave ballot."""
    print(f"sparse duplicate ids lens={lens} M={M}", flush=True)
    H, D = 2, 64
    g = torch.Generator().manual_seed(12)
    q, k, v, cu = packed(lens, H, D, seed=6)
    if M > 64:
        idx = full_causal_selection(lens, H, M=M)
        idx[:, :, 1::3] = -1   # thin the rows out so there are free slots to fill
    else:
        idx, _, _ = workloads.block_selection(lens, H, 64, M - 2, g)
        idx = torch.cat([idx, torch.full((H, idx.shape[1], 2), -1, dtype=torch.int32)], dim=2)
    dup = _with_duplicates(idx, g)
    assert not torch.equal(dup, idx)
    first = torch.full_like(dup, -1)
    for h in range(dup.shape[0]):
        for j in range(dup.shape[1]):
            seen = []
            for kb in dup[h, j].tolist():
                if kb >= 0 and kb not in seen:
                    seen.append(kb)
            first[h, j, :len(seen)] = torch.tensor(seen, dtype=torch.int32)
    o = _run_sparse(q, k, v, cu, first)
    o_dup = _run_sparse(q, k, v, cu, dup)
    assert torch.equal(o_dup, o)
    assert_parity(o_dup, ref.sparse_attn_varlen(q, k, v, cu, dup), torch.bfloat16, "o")


@pytest.mark.gpu
def test_sparse_attn_short_block_idx_writes_every_row():
    """block_idx with fewer rows than the packing's query blocks: the rows it
    lacks select nothing and their outputs are written as zeros (the output
    buffer starts as NaN and is passed through the C ABI directly)."""
    from selective_attention import _lib
    lens, H, D = [200, 150], 2, 128
    g = torch.Generator().manual_seed(13)
    q, k, v, cu = packed(lens, H, D, seed=7)
    idx, _, _ = workloads.block_selection(lens, H, 64, 4, g)
    nq = idx.shape[1]
    short = idx[:, : nq - 3].contiguous()
    qd, kd, vd, cud, sd = q.cuda(), k.cuda(), v.cuda(), cu.cuda(), short.cuda()
    o = torch.full_like(qd, float("nan"))
    _lib.call("sa_sparse_attn_fwd", _lib.DTYPE_BF16, _lib.ptr(qd), _lib.ptr(kd), _lib.ptr(vd),
              _lib.ptr(cud), len(lens), _lib.ptr(sd), sd.shape[1], sd.shape[2], 64, None,
              q.shape[0], H, D, -1.0, _lib.ptr(o), _lib.stream_of(qd))
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all()
    exp = ref.sparse_attn_varlen(q, k, v, cu, short)
    assert_parity(o, exp, torch.bfloat16, "o")
    # the last three query blocks are the tail of sequence 1 (150 tokens = 3 blocks)
    assert torch.count_nonzero(o[200:]) == 0


@pytest.mark.gpu
def test_sparse_attn_config2_sample():
    """Config 2 (T=65536, H16, D128, the bench's own inputs) on the device:
    every head of the first three sequences and of the longest one against
    the fp64 oracle (block-gathered), every output finite."""
    w = workloads.sparse_attn_inputs()
    o = _run_sparse(w.q, w.k, w.v, w.cu_seqlens, w.block_idx).cpu()
    assert torch.isfinite(o.float()).all()
    cu = w.cu_seqlens
    longest = max(range(len(w.lens)), key=lambda s: w.lens[s])
    seqs = sorted({0, 1, 2, longest})
    print(f"config 2 sequences {seqs} (lengths {[w.lens[s] for s in seqs]}), 16 heads", flush=True)
    exp = ref.sparse_attn_varlen_blocks(w.q, w.k, w.v, cu, w.block_idx, seqs)
    for s in seqs:
        a, b = int(cu[s]), int(cu[s + 1])
        assert_parity(o[a:b], exp[s], torch.bfloat16, f"o seq {s}")


def _run_decode(d, bias=None):
    from selective_attention.ops import paged_decode_attn
    o = paged_decode_attn(d.q.cuda(), d.k_pages.cuda(), d.v_pages.cuda(), d.page_table.cuda(),
                          d.seq_lens.cuda(), key_bias=None if bias is None else bias.cuda())
    torch.cuda.synchronize()
    return o


@pytest.mark.gpu
@pytest.mark.parametrize("b,Hq,Hkv,D,minl,maxl", [(3, 8, 2, 128, 1, 200), (4, 4, 4, 64, 60, 70),
                                                   (2, 32, 8, 128, 1000, 3000),
                                                   (5, 16, 1, 128, 1, 1100),
                                                   # more than 64 rows: the separate plan kernel
                                                   (70, 4, 2, 64, 1, 300)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_paged_decode_parity(b, Hq, Hkv, D, minl, maxl, with_bias):
    print(f"decode b={b} Hq={Hq} Hkv={Hkv} D={D} len=[{minl},{maxl}] bias={with_bias}", flush=True)
    d = workloads.decode_inputs(batch=b, nheads_q=Hq, nheads_kv=Hkv, headdim=D, min_len=minl,
                                max_len=maxl, seed=3)
    g = torch.Generator().manual_seed(9)
    bias = torch.randn(d.k_pages.shape[:3], generator=g) if with_bias else None
    o = _run_decode(d, bias)
    exp = ref.paged_decode_attn(d.q, d.k_pages, d.v_pages, d.page_table, d.seq_lens,
                                key_bias=bias)
    assert_parity(o, exp, torch.bfloat16, "o")


@pytest.mark.gpu
@pytest.mark.parametrize("with_bias", [False, True])
def test_paged_decode_page128(with_bias):
    """128-token pages: two 64-key tiles per page, the second one partial or
    empty on each row's last page."""
    print(f"decode page_size=128 bias={with_bias}", flush=True)
    d = workloads.decode_inputs(batch=6, nheads_q=8, nheads_kv=2, headdim=128, min_len=1,
                                max_len=700, page_size=128, seed=5)
    g = torch.Generator().manual_seed(11)
    bias = torch.randn(d.k_pages.shape[:3], generator=g) if with_bias else None
    o = _run_decode(d, bias)
    exp = ref.paged_decode_attn(d.q, d.k_pages, d.v_pages, d.page_table, d.seq_lens,
                                key_bias=bias)
    assert_parity(o, exp, torch.bfloat16, "o")


@pytest.mark.gpu
def test_paged_decode_empty_rows_and_single_long_row():
    """Rows with no cached tokens get zeros; one long row is spread over many
    waves (more waves than tiles), each contributing a one-tile segment."""
    print("decode empty rows", flush=True)
    d = workloads.decode_inputs(batch=9, nheads_q=4, nheads_kv=1, headdim=64, min_len=1,
                                max_len=300, seed=7)
    d.seq_lens[[0, 4, 8]] = 0
    o = _run_decode(d)
    exp = ref.paged_decode_attn(d.q, d.k_pages, d.v_pages, d.page_table, d.seq_lens)
    assert_parity(o, exp, torch.bfloat16, "o")
    assert (o[[0, 4, 8]].float() == 0).all()
    print("decode single long row", flush=True)
    d = workloads.decode_inputs(batch=1, nheads_q=16, nheads_kv=2, headdim=128, min_len=5000,
                                max_len=5000, seed=8)
    o = _run_decode(d)
    exp = ref.paged_decode_attn(d.q, d.k_pages, d.v_pages, d.page_table, d.seq_lens)
    assert_parity(o, exp, torch.bfloat16, "o")


@pytest.mark.gpu
def test_paged_decode_config3_all_rows():
    """Config 3 (b64, 32q/8kv, D128, len U[1024,32768], 64-token pages) on
    the device: all 64 rows against the fp64 oracle."""
    d = workloads.decode_inputs(device="cuda")
    o = _run_decode(d).cpu()
    assert torch.isfinite(o.float()).all()
    kp, vp, table, lens, q = (t.cpu() for t in (d.k_pages, d.v_pages, d.page_table,
                                                  d.seq_lens, d.q))
    for r0 in range(0, 64, 16):
        rows = list(range(r0, r0 + 16))
        exp = ref.paged_decode_attn(q[rows], kp, vp, table[rows], lens[rows])
        assert_parity(o[rows], exp, torch.bfloat16, f"o rows {r0}..{r0 + 15}")


# ------------------------------------------------- dense varlen attention (modes)
def test_oracle_attn_varlen_causal_is_full_selection():
    lens, H, D = [70, 130, 5], 2, 16
    q, k, v, cu = packed(lens, H, D, dtype=F64)
    g = torch.Generator().manual_seed(2)
    bias = torch.randn(H, sum(lens), generator=g, dtype=F64)
    bias[:, ::7] = float("-inf")
    exp = ref.sparse_attn_varlen(q, k, v, cu, full_causal_selection(lens, H), key_bias=bias)
    torch.testing.assert_close(ref.attn_varlen(q, k, v, cu, "causal", key_bias=bias), exp,
                               rtol=1e-12, atol=1e-12)


def test_oracle_attn_varlen_full_and_cross_are_sdpa():
    lens, H, D = [33, 9], 2, 8
    q, k, v, cu = packed(lens, H, D, seed=4, dtype=F64)
    o = ref.attn_varlen(q, k, v, cu, "full")
    for s in range(2):
        a, b = int(cu[s]), int(cu[s + 1])
        e = F.scaled_dot_product_attention(q[a:b].transpose(0, 1), k[a:b].transpose(0, 1),
                                           v[a:b].transpose(0, 1))
        torch.testing.assert_close(o[a:b], e.transpose(0, 1), rtol=1e-12, atol=1e-12)
    klens = [17, 40]
    _, kk, vv, cuk = packed(klens, H, D, seed=5, dtype=F64)
    o = ref.attn_varlen(q, kk, vv, cu, "cross", cuk)
    for s in range(2):
        a, b, c, d = int(cu[s]), int(cu[s + 1]), int(cuk[s]), int(cuk[s + 1])
        e = F.scaled_dot_product_attention(q[a:b].transpose(0, 1), kk[c:d].transpose(0, 1),
                                           vv[c:d].transpose(0, 1))
        torch.testing.assert_close(o[a:b], e.transpose(0, 1), rtol=1e-12, atol=1e-12)


def test_oracle_attn_varlen_brute_force_exemptions():
    """Loop form of the biased softmax: full mode exempts the query's own key,
    cross mode the first key of the key sequence."""
    H, D = 1, 4
    q, k, v, cu = packed([6], H, D, seed=6, dtype=F64)
    _, kk, vv, cuk = packed([5], H, D, seed=7, dtype=F64)
    bias = torch.tensor([[0.3, -1.0, 2.0, -0.5, 0.1, 0.7]], dtype=F64)
    o = ref.attn_varlen(q, k, v, cu, "full", key_bias=bias)
    oc = ref.attn_varlen(q, kk, vv, cu, "cross", cuk, key_bias=bias[:, :5])
    for i in range(6):
        sc = torch.tensor([float(q[i, 0] @ k[j, 0]) / 2.0 + (0.0 if j == i else float(bias[0, j]))
                           for j in range(6)], dtype=F64)
        torch.testing.assert_close(o[i, 0], torch.softmax(sc, 0) @ v[:, 0], rtol=1e-12, atol=1e-12)
        sc = torch.tensor([float(q[i, 0] @ kk[j, 0]) / 2.0 + (0.0 if j == 0 else float(bias[0, j]))
                           for j in range(5)], dtype=F64)
        torch.testing.assert_close(oc[i, 0], torch.softmax(sc, 0) @ vv[:, 0], rtol=1e-12, atol=1e-12)


VARLEN_CASES = {
    # name: (mode, q lens, k lens (cross), D, bias)
    "causal_d128_bias": ("causal", [200, 64, 1, 130], None, 128, True),
    "full_d64_bias": ("full", [150, 0, 64, 33], None, 64, True),
    "full_d128": ("full", [257, 19], None, 128, False),
    "cross_d64_bias": ("cross", [100, 1, 70, 0], [37, 300, 0, 5], 64, True),
    "cross_d128": ("cross", [65, 128], [129, 1], 128, False),
}


@pytest.mark.gpu
@pytest.mark.parametrize("case", list(VARLEN_CASES))
def test_attn_varlen_parity(case):
    from selective_attention.ops import attn_varlen
    mode, lens, klens, D, with_bias = VARLEN_CASES[case]
    H = 3
    q, k, v, cu = packed(lens, H, D, seed=11)
    cuk = None
    if mode == "cross":
        _, k, v, cuk = packed(klens, H, D, seed=12)
    bias = None
    if with_bias:
        g = torch.Generator().manual_seed(13)
        bias = torch.randn(H, k.shape[0], generator=g)
        bias[:, ::5] = float("-inf")
    print(f"attn_varlen case={case}", flush=True)
    o = attn_varlen(q.cuda(), k.cuda(), v.cuda(), cu.cuda(), mode,
                    None if cuk is None else cuk.cuda(), None if bias is None else bias.cuda())
    torch.cuda.synchronize()
    e = ref.attn_varlen(q, k, v, cu, mode, cuk, bias)
    assert_parity(o, e, torch.bfloat16, name=case)


@pytest.mark.gpu
def test_attn_varlen_causal_dense_equals_full_selection():
    """The dense causal mode and the block-sparse op with every causal block
    selected run the same kernel body: identical bits."""
    from selective_attention.ops import attn_varlen, sparse_attn_varlen
    lens, H, D = [300, 65, 1], 2, 64
    q, k, v, cu = packed(lens, H, D, seed=14)
    g = torch.Generator().manual_seed(15)
    bias = torch.randn(H, sum(lens), generator=g).cuda()
    qd, kd, vd, cud = q.cuda(), k.cuda(), v.cuda(), cu.cuda()
    print("attn_varlen dense vs table", flush=True)
    a = attn_varlen(qd, kd, vd, cud, "causal", key_bias=bias)
    b = sparse_attn_varlen(qd, kd, vd, cud, full_causal_selection(lens, H).cuda(), key_bias=bias)
    torch.cuda.synchronize()
    assert torch.equal(a.cpu(), b.cpu())


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["full", "cross"])
def test_attn_varlen_many_sequences(mode):
    """130 sequences (the kernel finds a query block's sequence 64 sequences
    per step), lengths 0..97, cross keys of other lengths (some empty)."""
    from selective_attention.ops import attn_varlen
    g = torch.Generator().manual_seed(21)
    lens = torch.randint(0, 98, (130,), generator=g).tolist()
    H, D = 2, 64
    q, k, v, cu = packed(lens, H, D, seed=22)
    cuk = None
    if mode == "cross":
        klens = torch.randint(0, 70, (130,), generator=g).tolist()
        _, k, v, cuk = packed(klens, H, D, seed=23)
    bias = torch.randn(H, k.shape[0], generator=g)
    print(f"attn_varlen many sequences {mode}", flush=True)
    o = attn_varlen(q.cuda(), k.cuda(), v.cuda(), cu.cuda(), mode,
                    None if cuk is None else cuk.cuda(), bias.cuda())
    torch.cuda.synchronize()
    assert_parity(o, ref.attn_varlen(q, k, v, cu, mode, cuk, bias), torch.bfloat16, name=mode)
