"""SelectiveMHA's inference attention on the attention ops: oracle pins (CPU),
paged-cache bookkeeping (CPU, checked through the paged oracle), HIP parity (GPU).

The reference computes this attention densely (modules/selective_attention.py
SelectiveMHA.forward :222-290 for prefill, SelectiveMHA.step :392-415 for
decode); here it runs on sparse_attn_varlen and paged_decode_attn with the
log-gate as key_bias.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import attn as ref
from selective_attention.ops.selective_mha import PagedSelectiveAttnCache, selective_mha_prefill
from tests.helpers import assert_parity

F64 = torch.float64
BF16 = torch.bfloat16


def mha_inputs(b, H, L, D, lengths=None, thr=0.3, seed=0, dead_heads=(), zero_frac=0.05,
               dtype=BF16):
    """q_rot, k_rot, v (b, H, L, D) and log_gate (b, H, L) as SelectiveMHA.forward
    makes them in inference: sigmoid gates, a per-head threshold, some gates
    exactly zero, heads with every gate zero, padding past `lengths`."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, H, L, D, generator=g).to(dtype)
    k = torch.randn(b, H, L, D, generator=g).to(dtype)
    v = torch.randn(b, H, L, D, generator=g).to(dtype)
    gate = torch.sigmoid(2.0 * torch.randn(b, H, L, generator=g, dtype=F64))
    gate[torch.rand(b, H, L, generator=g) < zero_frac] = 0.0
    for h in dead_heads:
        gate[:, h] = 0.0
    score_std = 0.5 + torch.rand(H, generator=g, dtype=F64)
    threshold = None if thr is None else torch.full((H,), thr, dtype=F64)
    lg = ref.selective_mha_log_gate(gate, score_std, 1.5, threshold, lengths)
    return q, k, v, lg


def dense_uncompressed(q, k, v, lg):
    """The reference's other inference branch (taken when some (batch, head)
    keeps every key): the full causal score matrix (_build_attn_matrix
    :55-62), the gate added to every column and the diagonal restored
    (_gated_softmax :134-139), softmax, times v."""
    b, H, L, D = q.shape
    q, k, v, lg = (t.to(F64) for t in (q, k, v, lg))
    S = torch.matmul(q, k.transpose(-2, -1)) * D ** -0.5
    S = S.masked_fill(torch.triu(torch.ones(L, L, dtype=torch.bool), 1), float("-inf"))
    d = torch.arange(L)
    diag = S[:, :, d, d].clone()
    S = S + lg.unsqueeze(2)
    S[:, :, d, d] = diag
    return torch.softmax(S, -1) @ v


# ------------------------------------------------------------ oracle pins
def test_oracle_prefill_matches_uncompressed_branch():
    lens = torch.tensor([40, 23])
    q, k, v, lg = mha_inputs(2, 3, 40, 8, lengths=lens, dtype=F64, dead_heads=(1,))
    o = ref.selective_mha_prefill_ref(q, k, v, lg, lens)
    e = dense_uncompressed(q, k, v, lg)
    for i, n in enumerate(lens.tolist()):
        torch.testing.assert_close(o[i, :, :n], e[i, :, :n], rtol=1e-10, atol=1e-12)
        assert (o[i, :, n:] == 0).all()
    # the check discriminates: biasing the diagonal too gives another answer
    b, H, L, D = q.shape
    S = torch.matmul(q, k.transpose(-2, -1)) * D ** -0.5
    S = S.masked_fill(torch.triu(torch.ones(L, L, dtype=torch.bool), 1), float("-inf"))
    wrong = torch.softmax(S + lg.unsqueeze(2), -1) @ v
    assert not torch.allclose(wrong[0, 0, :40], o[0, 0, :40], rtol=1e-3, atol=1e-3)


def test_oracle_prefill_all_kept_is_causal_sdpa():
    q, k, v, _ = mha_inputs(2, 2, 33, 16, dtype=F64)
    lg = torch.zeros(2, 2, 33, dtype=F64)          # every gate 1: log-gate 0
    o = ref.selective_mha_prefill_ref(q, k, v, lg)
    e = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    torch.testing.assert_close(o, e, rtol=1e-10, atol=1e-12)


def test_oracle_prefill_all_dropped_is_v():
    # valid_mask.any() is False: the reference returns out_proj(v * out_gate),
    # i.e. each query's attention output is its own value
    q, k, v, _ = mha_inputs(1, 2, 20, 8, dtype=F64)
    lg = torch.full((1, 2, 20), float("-inf"), dtype=F64)
    torch.testing.assert_close(ref.selective_mha_prefill_ref(q, k, v, lg), v, rtol=0, atol=1e-14)


def test_oracle_decode_row_equals_prefill_row():
    q, k, v, lg = mha_inputs(2, 2, 30, 8, dtype=F64, seed=5)
    o = ref.selective_mha_prefill_ref(q, k, v, lg)
    for t in (0, 1, 7, 29):
        d = ref.selective_mha_decode_ref(q[:, :, t], k[:, :, :t + 1], v[:, :, :t + 1], lg[:, :, :t + 1])
        torch.testing.assert_close(d, o[:, :, t], rtol=1e-10, atol=1e-12)


def test_oracle_log_gate():
    gate = torch.tensor([[[0.9, 0.2, 0.0, 0.5]]], dtype=F64)
    lg = ref.selective_mha_log_gate(gate, torch.tensor([2.0]), 0.5, torch.tensor([0.3]),
                                    torch.tensor([3]))
    exp = torch.tensor([[[torch.log(torch.tensor(0.9, dtype=F64)).item(), float("-inf"),
                          float("-inf"), float("-inf")]]], dtype=F64)
    torch.testing.assert_close(lg, exp)


# -------------------------------------------------- paged cache bookkeeping
def _check_cache_against_dense(cache, dense, q_t):
    """The paged oracle over the cache's pages == the decode oracle over each
    row's dense key list."""
    o = ref.paged_decode_attn(q_t, cache.k_pages, cache.v_pages, cache.page_table().cpu(),
                              cache.seq_lens().cpu(), key_bias=cache.gate_pages.cpu())
    for i, (K, V, G) in enumerate(dense):
        e = ref.selective_mha_decode_ref(q_t[i:i + 1], K[None], V[None], G[None])
        torch.testing.assert_close(o[i:i + 1], e, rtol=1e-6, atol=1e-6)


def _decode_run(dev, check, b=3, H=2, D=16, L=150, lens=(150, 64, 1), steps=70, seed=0):
    """Prefill-built cache, `steps` decode appends (one dropped in every head
    and row, then unappended as SelectiveMHA.step does), a page of dropped
    keys evicted.  `check(cache, dense, q_t)` runs after every attend."""
    lens_t = torch.tensor(lens)
    q, k, v, lg = mha_inputs(b, H, L, D, lengths=lens_t, seed=seed)
    lg[0, :, 64:128] = float("-inf")             # row 0: its second page fully dropped
    cache = PagedSelectiveAttnCache(b, H, D, max_tokens=L + steps + 64, device=dev)
    cache.build(k.to(dev), v.to(dev), lg.to(dev), lens_t)
    dense = [(k[i, :, :n].to(F64), v[i, :, :n].to(F64), lg[i, :, :n].clone())
             for i, n in enumerate(lens)]
    g = torch.Generator().manual_seed(seed + 1)
    for step in range(steps):
        qt = torch.randn(b, H, D, generator=g).to(BF16)
        kt = torch.randn(b, H, D, generator=g).to(BF16)
        vt = torch.randn(b, H, D, generator=g).to(BF16)
        gt = torch.sigmoid(torch.randn(b, H, generator=g, dtype=F64))
        gt[gt < 0.3] = 0.0
        if step == 5:
            gt.zero_()
        lgt = torch.log(gt) * 1.5
        cache.append(kt.to(dev), vt.to(dev), lgt.to(dev))
        dense = [(torch.cat([K, kt[i, :, None].to(F64)], 1), torch.cat([V, vt[i, :, None].to(F64)], 1),
                  torch.cat([G, lgt[i, :, None]], 1)) for i, (K, V, G) in enumerate(dense)]
        check(cache, dense, qt)
        if not bool(torch.isfinite(lgt).any()):
            cache.unappend()
            dense = [(K[:, :-1], V[:, :-1], G[:, :-1]) for K, V, G in dense]
        if step == 10:
            freed = cache.drop_evicted_pages()
            assert freed == 1 and cache.lens[0] == 150 + 10 - 64
            check(cache, dense, qt)
    return cache


def test_paged_cache_bookkeeping_cpu():
    _decode_run("cpu", _check_cache_against_dense)


def test_paged_cache_pool_exhausted():
    cache = PagedSelectiveAttnCache(1, 1, 8, max_tokens=64, device="cpu")
    z = torch.zeros(1, 1, 64, 8)
    cache.build(z, z, torch.zeros(1, 1, 64))
    with pytest.raises(RuntimeError, match="exhausted"):
        cache.append(torch.zeros(1, 1, 8), torch.zeros(1, 1, 8), torch.zeros(1, 1))


def test_paged_cache_rebuild_returns_pages():
    cache = PagedSelectiveAttnCache(2, 1, 8, max_tokens=130, device="cpu")
    z = torch.zeros(2, 1, 130, 8)
    for _ in range(3):
        cache.build(z, z, torch.zeros(2, 1, 130))
    assert sorted(cache.free + cache.rows[0] + cache.rows[1]) == list(range(2 * 3))


def test_paged_cache_table_padding_stays_in_row():
    """Columns of the page table past a row's pages repeat that row's last
    page: the device-side append clamps an overflowing token to the last
    column, which then names the row's own page, not another row's."""
    cache = PagedSelectiveAttnCache(3, 1, 8, max_tokens=200, device="cpu")
    lens = torch.tensor([130, 10, 64])
    z = torch.zeros(3, 1, 130, 8)
    cache.build(z, z, torch.zeros(3, 1, 130), lengths=lens)
    pt = cache.page_table()
    for i, r in enumerate(cache.rows):
        assert len(r) >= 1
        assert pt[i, :len(r)].tolist() == r
        assert (pt[i, len(r):] == r[-1]).all(), f"row {i}: {pt[i].tolist()} vs pages {r}"
    # the append kernel's column for a token past the row's pages
    col = min(10 ** 6 // cache.ps, pt.shape[1] - 1)
    assert [int(pt[i, col]) for i in range(3)] == [r[-1] for r in cache.rows]


def test_device_mode_gives_empty_rows_their_own_page():
    """A row with no tokens (and no pages) entering device mode with no extra
    tokens still gets a page of its own: the device-side append of its next
    token lands there, never in page 0 of another row."""
    cache = PagedSelectiveAttnCache(3, 1, 8, max_tokens=200, device="cpu")
    z = torch.zeros(3, 1, 100, 8)
    cache.build(z, z, torch.zeros(3, 1, 100), lengths=torch.tensor([100, 0, 30]))
    assert cache.rows[1] == []
    cache.enter_device_mode(0)
    pt = cache.page_table()
    owned = [set(r) for r in cache.rows]
    assert all(len(r) >= 1 for r in cache.rows)
    assert not (owned[0] & owned[1]) and not (owned[1] & owned[2]) and not (owned[0] & owned[2])
    for i in range(3):
        assert set(pt[i].tolist()) <= owned[i], f"row {i}: {pt[i].tolist()} vs {cache.rows[i]}"
    cache.exit_device_mode()


# ------------------------------------------------------------- GPU parity
PREFILL_CASES = {
    # name: (b, H, L, D, lengths, thr, dead_heads)
    "ragged_d64": (2, 4, 200, 64, [200, 137], 0.3, (2,)),
    "full_d128": (1, 2, 130, 128, None, None, ()),
    "short_rows": (3, 2, 70, 64, [70, 1, 0], 0.5, ()),
    "long_m66": (1, 1, 4200, 64, None, 0.4, ()),
}


@pytest.mark.gpu
@pytest.mark.parametrize("case", list(PREFILL_CASES))
def test_selective_mha_prefill_parity(case):
    b, H, L, D, lens, thr, dead = PREFILL_CASES[case]
    lens_t = None if lens is None else torch.tensor(lens)
    q, k, v, lg = mha_inputs(b, H, L, D, lengths=lens_t, thr=thr, dead_heads=dead, seed=11)
    print(f"selective_mha_prefill case={case}", flush=True)
    o = selective_mha_prefill(q.cuda(), k.cuda(), v.cuda(), lg.cuda(), lens_t)
    torch.cuda.synchronize()
    e = ref.selective_mha_prefill_ref(q, k, v, lg, lens_t)
    assert_parity(o, e, BF16, name=f"prefill {case}")


@pytest.mark.gpu
@pytest.mark.parametrize("D", [64, 128])
def test_paged_cache_decode_parity(D):
    def check(cache, dense, q_t):
        o = cache.attend(q_t.cuda())
        torch.cuda.synchronize()
        for i, (K, V, G) in enumerate(dense):
            e = ref.selective_mha_decode_ref(q_t[i:i + 1], K[None], V[None], G[None])
            assert_parity(o[i:i + 1], e, BF16, name=f"decode row {i} len {cache.lens[i]}")
    print(f"paged selective cache decode D={D}", flush=True)
    _decode_run("cuda", check, H=4, D=D)


@pytest.mark.gpu
@pytest.mark.parametrize("D", [64, 128])
def test_paged_build_kernel_matches_torch_build(D):
    """The one-launch page build (transposed-view inputs, ragged lengths, a
    row of length 0, a partial last page) writes the same pages, bit for bit,
    as the torch build of the same cache on the CPU: K, V transposed, gates,
    zeros and -inf past each row's length."""
    from selective_attention.ops import PagedSelectiveAttnCache
    b, H, L = 4, 3, 200
    g = torch.Generator().manual_seed(9)
    k = torch.randn(b, L, H, D, generator=g).to(torch.bfloat16).transpose(1, 2)
    v = torch.randn(b, L, H, D, generator=g).to(torch.bfloat16).transpose(1, 2)
    lg = torch.randn(b, H, L, generator=g)
    lg[lg < -1.0] = float("-inf")
    lengths = torch.tensor([200, 131, 0, 64])
    print(f"paged build D={D}", flush=True)
    caches = []
    for dev in ("cpu", "cuda"):
        c = PagedSelectiveAttnCache(b, H, D, max_tokens=L + 64, device=dev)
        c.build(k.to(dev), v.to(dev), lg.to(dev), lengths)
        caches.append(c)
    cpu, gpu = caches
    assert cpu.rows == gpu.rows and cpu.lens == gpu.lens
    for i in range(b):
        ids = torch.tensor(cpu.rows[i], dtype=torch.long)
        if len(ids) == 0:
            continue
        assert torch.equal(gpu.k_pages[ids.cuda()].cpu(), cpu.k_pages[ids])
        assert torch.equal(gpu.v_pages[ids.cuda()].cpu(), cpu.v_pages[ids])
        assert torch.equal(gpu.gate_pages[ids.cuda()].cpu(), cpu.gate_pages[ids])


@pytest.mark.gpu
def test_decode_step_matches_prefill_row():
    """The two kernels agree where the reference's prefill and step agree:
    query t over cached keys 0..t (newest exempt) == prefill row t."""
    b, H, L, D = 2, 4, 190, 64
    q, k, v, lg = mha_inputs(b, H, L, D, seed=3)
    print("decode step vs prefill row", flush=True)
    o = selective_mha_prefill(q.cuda(), k.cuda(), v.cuda(), lg.cuda()).float().cpu()
    for t in (0, 63, 64, 129, 189):
        cache = PagedSelectiveAttnCache(b, H, D, max_tokens=L, device="cuda")
        cache.build(k[:, :, :t].cuda(), v[:, :, :t].cuda(), lg[:, :, :t].cuda())
        cache.append(k[:, :, t].cuda(), v[:, :, t].cuda(), lg[:, :, t].cuda())
        d = cache.attend(q[:, :, t].cuda()).float().cpu()
        torch.testing.assert_close(d, o[:, :, t], rtol=2e-2, atol=2e-2)


@pytest.mark.gpu
def test_selective_mha_prefill_view_input():
    """(b, L, H, D) memory passed as its (b, H, L, D) transpose (read in place)
    gives the same bits as the contiguous (b, H, L, D) input."""
    b, H, L, D = 2, 3, 150, 64
    lens = torch.tensor([150, 99])
    q, k, v, lg = mha_inputs(b, H, L, D, lengths=lens, seed=8)
    print("selective_mha_prefill view input", flush=True)
    o1 = selective_mha_prefill(q.cuda(), k.cuda(), v.cuda(), lg.cuda(), lens)
    views = [x.transpose(1, 2).contiguous().cuda().transpose(1, 2) for x in (q, k, v)]
    o2 = selective_mha_prefill(*views, lg.cuda(), lens)
    torch.cuda.synchronize()
    assert torch.equal(o1.cpu(), o2.cpu())
    assert (o1[1, :, 99:] == 0).all()


def test_drop_evicted_pages_keeps_reserved_pages():
    """Pages reserved past a row's newest token (enter_device_mode) hold no
    tokens: compaction must neither free them nor shorten the row."""
    cache = PagedSelectiveAttnCache(1, 1, 8, max_tokens=64 * 6, device="cpu")
    z = torch.zeros(1, 1, 130, 8)
    lg = torch.zeros(1, 1, 130)
    lg[0, 0, :64] = float("-inf")                     # page 0 fully dropped
    cache.build(z, z, lg)
    cache.rows[0] += [cache._alloc(), cache._alloc()]  # reserve two empty pages
    assert cache.drop_evicted_pages() == 1
    assert cache.lens == [66] and len(cache.rows[0]) == 4
    assert cache.drop_evicted_pages() == 0 and cache.lens == [66]
