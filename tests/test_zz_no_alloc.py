"""sa_paged_decode_fwd_noalloc: the decode entry point that allocates nothing
(its workspace is the library's file-scope device array), against
sa_paged_decode_fwd with a caller workspace, both through the C ABI.

Three calls in a row on the same GPU, each with a smaller input, must
each give the allocating entry point's result bit for bit (same kernels, same
wave count); a call that would need more than the array holds is refused
before any launch.
"""
import pytest
import torch

from selective_attention import _lib, workloads


def _decode_inputs(batch, seed, with_bias):
    d = workloads.decode_inputs(batch=batch, min_len=1, max_len=5000, seed=seed, device="cuda")
    bias = None
    if with_bias:
        g = torch.Generator(device="cuda").manual_seed(seed + 100)
        bias = torch.randn(d.k_pages.shape[:3], generator=g, device="cuda")
    return d, bias


def _args(d, bias):
    b, Hq, D = d.q.shape
    num_pages, Hkv, ps, _ = d.k_pages.shape
    return (_lib.DTYPE_BF16, _lib.ptr(d.q), _lib.ptr(d.k_pages), _lib.ptr(d.v_pages),
            _lib.ptr(d.page_table), _lib.ptr(d.seq_lens), _lib.ptr(bias), b, Hq, Hkv, D, ps,
            d.page_table.shape[1], num_pages, -1.0)


def _with_workspace(d, bias):
    lib = _lib.load()
    b, Hq, D = d.q.shape
    Hkv = d.k_pages.shape[1]
    nbytes = lib.sa_paged_decode_workspace_size(b, Hq, Hkv, D, d.page_table.shape[1])
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    o = torch.empty_like(d.q)
    _lib.call("sa_paged_decode_fwd", *_args(d, bias), _lib.ptr(o), _lib.ptr(ws), nbytes,
              _lib.stream_of(d.q))
    return o


def _no_alloc(d, bias):
    o = torch.full_like(d.q, float("nan"))
    _lib.call("sa_paged_decode_fwd_noalloc", *_args(d, bias), _lib.ptr(o), _lib.stream_of(d.q))
    return o


@pytest.mark.gpu
@pytest.mark.parametrize("with_bias", [False, True])
def test_no_alloc_decode_matches_workspace_entry(with_bias):
    print(f"no-alloc decode bias={with_bias}", flush=True)
    # each call smaller than the one before; the first has more than 64 rows,
    # so its row plan comes from the separate plan kernel (cum_row written
    # into the file-scope array), the others form it in the decode waves
    for batch, seed in ((66, 3), (48, 1), (5, 2)):
        d, bias = _decode_inputs(batch, seed, with_bias)
        ref = _with_workspace(d, bias)
        got = _no_alloc(d, bias)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all(), f"batch {batch}"
        assert torch.equal(got, ref), f"batch {batch}: differs from sa_paged_decode_fwd"


@pytest.mark.gpu
def test_no_alloc_decode_rejects_oversize():
    """A batch whose segment partials exceed the array is refused (return 1,
    clear message) before any launch; the output is left untouched."""
    lib = _lib.load()
    limit = lib.sa_paged_decode_noalloc_limit()
    Hq, Hkv, D = 16, 1, 128
    # per segment: 16 * 128 * 4 B of partial output, one segment per row at least
    batch = limit // (Hq * D * 4) + 1
    q = torch.zeros(1, dtype=torch.bfloat16, device="cuda")   # never read: refused first
    o = torch.full((4,), 7.0, dtype=torch.bfloat16, device="cuda")
    rc = lib.sa_paged_decode_fwd_noalloc(_lib.DTYPE_BF16, _lib.ptr(q), _lib.ptr(q), _lib.ptr(q),
                                         _lib.ptr(q), _lib.ptr(q), None, batch, Hq, Hkv, D, 64, 1,
                                         1, -1.0, _lib.ptr(o), _lib.stream_of(q))
    assert rc == 1
    assert b"scratch" in lib.sa_last_error()
    torch.cuda.synchronize()
    assert (o.float() == 7.0).all()
