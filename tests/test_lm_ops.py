"""Model-side fused kernels (csrc/lm_ops.hip) against the reference's torch
formulas: RMSNorm (modules/rms_norm.py:33-44), RoPE (modules/rope.py:9-64),
and the paged KV append against the cache's host-side append."""
import pytest
import torch

from selective_attention.modules.layers import RMSNorm, RoPE

BF16 = torch.bfloat16


def rms_ref(x, w, eps=1e-6):
    """The module's own composite (fp32 arithmetic, result in x's dtype)."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * (1.0 + w.float())).type_as(x)


def ulp_bf16_close(a, e, ulps=1):
    """|a - e| <= ulps bf16 ulps of e (elementwise)."""
    a, e = a.float(), e.float()
    ulp = torch.ldexp(torch.ones_like(e), torch.frexp(e.abs().clamp_min(1e-30)).exponent - 8)
    return bool(((a - e).abs() <= ulps * ulp).all())


@pytest.mark.gpu
@pytest.mark.parametrize("shape,groups,dtype", [((7, 1024), None, BF16), ((3, 5, 100), None, BF16),
                                                ((6, 4, 64), 4, BF16), ((9, 1024), None, torch.float32)])
def test_rms_norm_kernel(shape, groups, dtype):
    from selective_attention.kernels.lm_ops import rms_norm
    g = torch.Generator().manual_seed(0)
    x = (3 * torch.randn(*shape, generator=g)).to(dtype)
    w = 0.3 * torch.randn((shape[-1],) if groups is None else (groups, shape[-1]), generator=g)
    print(f"rms_norm {shape} groups={groups} {dtype}", flush=True)
    out = rms_norm(x.cuda(), w.cuda(), 1e-6).cpu()
    exp = rms_ref(x, w)
    if dtype == torch.float32:
        torch.testing.assert_close(out, exp, rtol=2e-6, atol=1e-6)
    else:
        assert ulp_bf16_close(out, exp, 1)


@pytest.mark.gpu
def test_rms_norm_module_dispatch():
    """The module runs the kernel under no_grad and the composite with autograd;
    both agree."""
    m = RMSNorm(256).cuda()
    with torch.no_grad():
        m.weight.copy_(0.2 * torch.randn(256))
    x = torch.randn(33, 256, device="cuda").to(BF16)
    with torch.no_grad():
        a = m(x)
    xr = x.clone().requires_grad_(True)
    b = m(xr)
    b.float().sum().backward()
    assert xr.grad is not None
    assert ulp_bf16_close(a.cpu(), b.detach().cpu(), 1)


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["seq", "pos"])
def test_rope_kernel(mode):
    rope = RoPE(64).cuda()
    g = torch.Generator().manual_seed(1)
    if mode == "seq":
        b, L, H, D = 2, 300, 4, 64
        q = torch.randn(b, L, H, D, generator=g).to(BF16).cuda()
        k = torch.randn(b, L, H, D, generator=g).to(BF16).cuda()
        eq, ek = rope(q.transpose(1, 2), k.transpose(1, 2), torch.arange(L, device="cuda"), "seq")
        eq, ek = eq.transpose(1, 2), ek.transpose(1, 2)
        yq, yk = rope.rotate_qk(q, k, None, L)
    else:
        b, H, D = 5, 4, 64
        q = torch.randn(b, H, D, generator=g).to(BF16).cuda()
        k = torch.randn(b, H, D, generator=g).to(BF16).cuda()
        pos = torch.tensor([0, 7, 4096, 31999, 123456], device="cuda")
        eq, ek = rope(q, k, pos, "pos")
        yq, yk = rope.rotate_qk(q, k, pos, b)
    print(f"rope {mode}", flush=True)
    torch.cuda.synchronize()
    assert ulp_bf16_close(yq.cpu(), eq.to(BF16).cpu(), 1)
    assert ulp_bf16_close(yk.cpu(), ek.to(BF16).cpu(), 1)


@pytest.mark.gpu
def test_paged_kv_append_kernel():
    """Device-mode appends (one kernel per step) leave the same pages and
    lengths as the host-side appends."""
    from selective_attention.ops.selective_mha import PagedSelectiveAttnCache
    b, H, D, L = 3, 2, 64, 100
    g = torch.Generator().manual_seed(2)
    k = torch.randn(b, H, L, D, generator=g).to(BF16).cuda()
    v = torch.randn(b, H, L, D, generator=g).to(BF16).cuda()
    lg = torch.randn(b, H, L, generator=g).cuda()
    lens = torch.tensor([100, 63, 1])
    caches = []
    for device_mode in (False, True):
        c = PagedSelectiveAttnCache(b, H, D, max_tokens=300, device="cuda")
        c.build(k, v, lg, lens)
        if device_mode:
            c.enter_device_mode(80)
        for t in range(70):
            gt = torch.Generator().manual_seed(100 + t)
            c.append(torch.randn(b, H, D, generator=gt).to(BF16).cuda(),
                     torch.randn(b, H, D, generator=gt).to(BF16).cuda(),
                     torch.randn(b, H, generator=gt).cuda())
        if device_mode:
            c.exit_device_mode()
        caches.append(c)
    print("paged append", flush=True)
    host, dev = caches
    assert host.lens == dev.lens == [170, 133, 71]
    for i in range(b):
        n = host.lens[i]
        for c2 in (host, dev):
            assert len(c2.rows[i]) * 64 >= n
        for t in range(n):
            ph, s = host.rows[i][t // 64], t % 64
            pd = dev.rows[i][t // 64]
            assert torch.equal(host.k_pages[ph, :, s], dev.k_pages[pd, :, s])
            assert torch.equal(host.v_pages[ph, :, :, s], dev.v_pages[pd, :, :, s])
            assert torch.equal(host.gate_pages[ph, :, s], dev.gate_pages[pd, :, s])


@pytest.mark.gpu
def test_add_rms_norm_kernel():
    from selective_attention.kernels.lm_ops import add_rms_norm
    g = torch.Generator().manual_seed(3)
    x = torch.randn(37, 1024, generator=g).to(BF16)
    y = torch.randn(37, 1024, generator=g).to(BF16)
    w = 0.3 * torch.randn(1024, generator=g)
    print("add_rms_norm", flush=True)
    s, n = add_rms_norm(x.cuda(), y.cuda(), w.cuda(), 1e-6)
    es = (x + y)                       # torch's bf16 add (fp32 arithmetic, rounded)
    assert torch.equal(s.cpu(), es)
    assert ulp_bf16_close(n.cpu(), rms_ref(es, w), 1)


@pytest.mark.gpu
@pytest.mark.parametrize("with_thr", [False, True])
def test_mha_gates_kernel(with_thr):
    """The step's gate math against the module's torch path (sigmoid, split,
    threshold, log-gate)."""
    from selective_attention.kernels.lm_ops import mha_gates
    g = torch.Generator().manual_seed(4)
    H, dim = 16, 1024
    z = (torch.randn(5, H + dim, generator=g) + 2.0).to(BF16)
    z[0, :4] = -200.0                  # sigmoid rounds to 0 in bf16: dropped
    thr = torch.full((H,), 0.9) if with_thr else None
    std = 0.5 + torch.rand(H, generator=g)
    print(f"mha_gates thr={with_thr}", flush=True)
    lg, og = mha_gates(z.cuda(), None if thr is None else thr.cuda(), std.cuda(), 2.0, H)
    sg = torch.sigmoid(z.cuda()).cpu()
    s, o = sg[:, :H], sg[:, H:]
    kept = s > 0
    if thr is not None:
        kept &= s >= thr[None, :]
    elg = torch.where(kept, torch.log(s.float()) * std * 2.0, torch.full((5, H), float("-inf")))
    assert torch.equal(og.cpu(), o)
    assert torch.equal(torch.isinf(lg.cpu()), torch.isinf(elg))
    f = torch.isfinite(elg)
    torch.testing.assert_close(lg.cpu()[f], elg[f], rtol=2e-6, atol=1e-6)


@pytest.mark.gpu
def test_silu_mul_kernel():
    import torch.nn.functional as F
    from selective_attention.kernels.lm_ops import silu_mul
    g = torch.Generator().manual_seed(5)
    a = (3 * torch.randn(9, 4096, generator=g)).to(BF16)
    c = (3 * torch.randn(9, 4096, generator=g)).to(BF16)
    print("silu_mul", flush=True)
    out = silu_mul(a.cuda(), c.cuda()).cpu()
    exp = (a.cuda() * F.silu(c.cuda())).cpu()
    assert ulp_bf16_close(out, exp, 1)


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,bias", [(1, 1040, 1024, True), (4, 4384, 1024, True),
                                        (5, 1024, 4096, True), (8, 32000, 1024, False),
                                        (4, 32000, 1024, False),
                                        (3, 100, 2048, False)])
def test_gemv_kernel(M, N, K, bias):
    """The decode linear layers: within one bf16 ulp of the exactly rounded
    product (fp32 accumulation), for every M the kernel instantiates."""
    from selective_attention.kernels.lm_ops import gemv
    g = torch.Generator().manual_seed(M * 7 + N)
    x = torch.randn(M, K, generator=g).to(BF16)
    W = (torch.randn(N, K, generator=g) / K ** 0.5).to(BF16)
    b = torch.randn(N, generator=g).to(BF16) if bias else None
    print(f"gemv M={M} N={N} K={K}", flush=True)
    y = gemv(x.cuda(), W.cuda(), None if b is None else b.cuda()).cpu()
    exact = x.double() @ W.double().T + (0 if b is None else b.double())
    # one bf16 ulp of the exact value plus the fp32 accumulation bound
    # K * 2^-24 * sum_k |x_k w_k| (matters where the sum cancels to ~0)
    mag = x.double().abs() @ W.double().abs().T
    ulp = torch.ldexp(torch.ones_like(exact), torch.frexp(exact.abs().clamp_min(1e-30)).exponent - 8)
    err = (y.double() - exact).abs()
    bound = ulp + K * 2.0 ** -24 * mag
    worst = (err / bound).max().item()
    assert worst <= 1.0, f"worst err/bound {worst:.3f} (max err {err.max().item():.3e})"


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 4, 8])
def test_gemv_multi_matches_single(M):
    """One launch over several weight matrices (sizes not multiples of the
    block's 4 columns, biases present and absent, one matrix a row block of
    another) equals the single-matrix GEMV bit for bit; with xscale it equals
    the GEMV of the bf16 product x * xscale (torch's rounding of it)."""
    from selective_attention.kernels.lm_ops import gemv, gemv_multi
    K = 1024
    g = torch.Generator().manual_seed(40 + M)
    x = torch.randn(M, K, generator=g).to(BF16).cuda()
    s = torch.randn(M, K, generator=g).to(BF16).cuda()
    big = (torch.randn(4384, K, generator=g) / K ** 0.5).to(BF16).cuda()
    Ws = list(torch.split(big, [2304, 2048, 32]))
    Ws.append((torch.randn(1041, K, generator=g) / K ** 0.5).to(BF16).cuda())
    if M == 1:   # single-column and tiny matrices: blocks with idle waves
        Ws = [(torch.randn(n, K, generator=g) / K ** 0.5).to(BF16).cuda() for n in (1, 2, 3, 5)]
    bs = [torch.randn(W.shape[0], generator=g).to(BF16).cuda() if i != 1 else None
          for i, W in enumerate(Ws)]
    print(f"gemv_multi M={M} K={K} N={[W.shape[0] for W in Ws]}", flush=True)
    for xscale in (None, s):
        ys = gemv_multi(x, Ws, bs, xscale)
        xin = x if xscale is None else x * xscale
        for W, b, y in zip(Ws, bs, ys):
            assert y.is_contiguous() and y.shape == (M, W.shape[0])
            assert torch.equal(y, gemv(xin, W, b))


def test_gemv_multi_rejects_bad_counts():
    """Argument errors come back as errors before anything is launched."""
    import ctypes
    from selective_attention import _lib
    arr = ctypes.c_void_p * 1
    with pytest.raises(RuntimeError, match="weight matrices"):
        _lib.call("sa_gemv_bf16_multi", 16, None, 1, 64, 0, arr(16), arr(None),
                  (ctypes.c_int * 1)(4), arr(16), None)
    with pytest.raises(RuntimeError, match="weight matrix 0"):
        _lib.call("sa_gemv_bf16_multi", 16, None, 1, 64, 1, arr(16), arr(None),
                  (ctypes.c_int * 1)(0), arr(16), None)


@pytest.mark.gpu
def test_linear_dispatch():
    """Linear runs the GEMV for <= 8 bf16 rows in inference and the GEMM
    otherwise; both agree with F.linear in fp32 to bf16 rounding: 1 ulp for
    the GEMV (one rounding of the fp32 sum plus bias), 2 for the GEMM
    library (which may round the product before adding the bias)."""
    import torch.nn.functional as F
    from selective_attention.modules.layers import Linear
    torch.manual_seed(0)
    lin = Linear(512, 768).cuda().to(BF16)
    g = torch.Generator(device="cuda").manual_seed(1)
    for rows, ulps in ((4, 1), (9, 2)):
        x = torch.randn(rows, 512, device="cuda", generator=g).to(BF16)
        with torch.no_grad():
            y = lin(x)
            e = F.linear(x.float(), lin.weight.float(), lin.bias.float())
        assert ulp_bf16_close(y.cpu(), e.to(BF16).cpu(), ulps), f"rows {rows}"


@pytest.mark.gpu
def test_rope_keeps_fp32_frequencies_after_bf16_cast():
    """Casting the module to bf16 must not round RoPE's frequencies: at
    position 8192 a bf16 frequency puts the angle off by radians."""
    rope = RoPE(64).cuda().to(BF16)
    assert rope.inv_freq.dtype == BF16                  # the registered buffer is cast ...
    q = torch.randn(1, 2, 64, device="cuda").to(BF16)
    pos = torch.tensor([8191], device="cuda")
    yq, _ = rope.rotate_qk(q, q, pos, 1)
    ref = RoPE(64)                                       # ... the rotation still uses fp32 ones
    eq, _ = ref(q.float().cpu(), q.float().cpu(), pos.cpu(), "pos")
    assert ulp_bf16_close(yq.cpu(), eq.to(BF16), 1)
