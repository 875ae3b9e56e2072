"""SSD chunked scan forward: HIP kernels vs the fp64 CPU oracle."""
import math

import pytest
import torch

from oracle import ssd as ref
from selective_attention import workloads
from tests.helpers import assert_parity, assert_scaled

F64 = torch.float64


def make_inputs(b=2, L=100, H=4, P=24, N=40, G=2, dtype=torch.float32, seed=0, with_h=True,
                with_bias=True, lens=None):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(b, L, H, P, generator=g).to(dtype)
    A = -torch.exp(torch.rand(H, generator=g) * math.log(16.0))
    B = (torch.randn(b, L, G, N, generator=g) / math.sqrt(N)).to(dtype)
    C = (torch.randn(b, L, G, N, generator=g) / math.sqrt(N)).to(dtype)
    dr = (torch.randn(b, L, H, generator=g) - 3.0).to(dtype)
    bias = torch.randn(H, generator=g) * 0.3 if with_bias else None
    h0 = torch.randn(b, H, P, N, generator=g) * 0.3 if with_h else None
    length = None if lens is None else torch.tensor(lens, dtype=torch.int64)
    return dict(u=u, A=A, B=B, C=C, delta_raw=dr, delta_bias=bias, h_init=h0, length=length)


def large_z(x, frac=0.05, lo=20.5, hi=150.0, seed=21):
    """Put delta_raw (+ bias) above the softplus threshold 20 on a fraction of
    the tokens: dt = z there (triton_kernels/softplus.py:5-12), up to 150, so
    an unthresholded fp32 log(exp(z) + 1) would overflow."""
    g = torch.Generator().manual_seed(seed)
    dr = x["delta_raw"].float()
    m = torch.rand(dr.shape, generator=g) < frac
    vals = lo + (hi - lo) * torch.rand(dr.shape, generator=g)
    x = dict(x)
    x["delta_raw"] = torch.where(m, vals, dr).to(x["delta_raw"].dtype)
    return x


def to_dev(x):
    return {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in x.items()}


def run_fwd(x, chunk, **kw):
    from selective_attention.ops import SSDScanFn
    xd = to_dev(x)
    y, h = SSDScanFn.apply(xd["u"], xd["A"], xd["B"], xd["C"], xd["delta_raw"], xd["delta_bias"],
                           xd["h_init"], xd["length"], chunk, kw.get("softplus", True),
                           kw.get("limit", (0.0, float("inf"))), True)
    torch.cuda.synchronize()
    return y, h


FWD_CASES = [
    ("aligned", dict(b=2, L=128, H=4, P=64, N=64, G=2), 64),
    ("ragged", dict(b=2, L=100, H=4, P=24, N=40, G=2), 32),
    ("lens", dict(b=3, L=150, H=2, P=16, N=16, G=1, lens=[150, 37, 0]), 64),
    ("noinit", dict(b=1, L=70, H=6, P=32, N=24, G=3, with_h=False, with_bias=False), 16),
    ("bigP", dict(b=1, L=96, H=2, P=130, N=120, G=1), 48),
    ("chunk1", dict(b=1, L=9, H=2, P=8, N=8, G=2), 1),
    ("chunk256", dict(b=1, L=300, H=2, P=64, N=128, G=1, lens=[281]), 256),
]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("name,shape,chunk", FWD_CASES, ids=[c[0] for c in FWD_CASES])
def test_ssd_fwd_parity(dtype, name, shape, chunk):
    print(f"ssd fwd {name} dtype={dtype} chunk={chunk}", flush=True)
    x = make_inputs(dtype=dtype, **shape)
    y_ref, h_ref = ref.ssd_scan_forward(**x, chunk_size=chunk)
    y, h = run_fwd(x, chunk)
    assert y.dtype == torch.float32 and h.dtype == torch.float32
    assert_parity(y, y_ref, dtype, "y")
    assert_parity(h, h_ref, dtype, "h_last")


@pytest.mark.gpu
@pytest.mark.parametrize("softplus,limit", [(False, (0.01, 0.2)), (True, (0.03, 0.08))])
def test_ssd_fwd_limits(softplus, limit):
    x = make_inputs(L=80, P=16, N=16, dtype=torch.float32)
    x["delta_raw"] = x["delta_raw"] + 3.0 if not softplus else x["delta_raw"]
    y_ref, h_ref = ref.ssd_scan_forward(**x, chunk_size=32, use_delta_softplus=softplus,
                                        delta_limit=limit)
    y, h = run_fwd(x, 32, softplus=softplus, limit=limit)
    assert_parity(y, y_ref, torch.float32, "y")
    assert_parity(h, h_ref, torch.float32, "h_last")


THRESHOLD_CASES = [
    (torch.float32, dict(b=2, L=200, H=4, P=24, N=40, G=2, lens=[200, 133]), 64),
    (torch.bfloat16, dict(b=2, L=320, H=8, P=64, N=128, G=2, lens=[320, 201]), 128),
]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,shape,chunk", THRESHOLD_CASES)
def test_ssd_fwd_softplus_threshold(dtype, shape, chunk):
    """delta_raw + bias in (20.5, 22) on 3 % of the tokens: dt = z there (the
    identity branch of the softplus), generic (fp32) and bf16 chunk-scan
    paths, at the stated tolerances."""
    print(f"ssd fwd large z dtype={dtype} chunk={chunk}", flush=True)
    x = large_z(make_inputs(dtype=dtype, **shape), frac=0.03, hi=22.0)
    y_ref, h_ref = ref.ssd_scan_forward(**x, chunk_size=chunk)
    y, h = run_fwd(x, chunk)
    assert_parity(y, y_ref, dtype, "y")
    assert_parity(h, h_ref, dtype, "h_last")


@pytest.mark.gpu
def test_ssd_fwd_softplus_far_above_threshold():
    """z up to 150 (bf16): an unthresholded fp32 log(exp(z) + 1) overflows
    past 88.  Outputs stay finite and within 2e-2 of their scale; single
    bf16 roundings of terms ~dt * u ~ 100 exceed the elementwise atol, so
    only the scale-aware bound is asserted here."""
    x = large_z(make_inputs(dtype=torch.bfloat16, b=2, L=320, H=8, P=64, N=128, G=2,
                            lens=[320, 201]))
    y_ref, h_ref = ref.ssd_scan_forward(**x, chunk_size=128)
    y, h = run_fwd(x, 128)
    assert_scaled(y, y_ref, "y")
    assert_scaled(h, h_ref, "h_last")


@pytest.mark.gpu
def test_ssd_fwd_intermediates():
    """dt, dc and the chunk entry states against the oracle's."""
    from selective_attention.kernels.ssd_scan import ssd_scan_forward
    x = make_inputs(b=2, L=100, H=4, P=24, N=40, G=2, lens=[100, 61])
    _, _, it = ref.ssd_scan_forward(**x, chunk_size=32, return_intermediates=True)
    xd = to_dev(x)
    _, _, (dt, dc, states) = ssd_scan_forward(
        xd["u"], xd["A"], xd["B"], xd["C"], xd["delta_raw"], xd["delta_bias"], xd["h_init"],
        xd["length"], 32, return_saved=True)
    assert_parity(dt, it["dt"], torch.float32, "dt")
    assert_parity(dc, it["dc"], torch.float32, "dc")
    assert_parity(states, it["H_in"], torch.float32, "states")


@pytest.mark.gpu
def test_ssd_fwd_config0():
    """BASELINE config 0 (fp32): y + D*x and the final state, rtol 1e-4."""
    cfg = workloads.SSD_CONFIGS[0]
    x = workloads.ssd_inputs(**cfg)
    D = x.pop("D")
    args = dict(u=x["u"], A=x["A"], B=x["B"], C=x["C"], delta_raw=x["delta_raw"],
                delta_bias=None, h_init=None, length=None)
    y_ref, h_ref = ref.ssd_scan_forward(**args, chunk_size=cfg["chunk"])
    y, h = run_fwd(args, cfg["chunk"])
    b, L, H, P = x["u"].shape
    ytot_ref = y_ref.reshape(b, L, H * P) + D.double() * x["u"].double().reshape(b, L, H * P)
    ytot = y.reshape(b, L, H * P) + D.cuda() * x["u"].cuda().reshape(b, L, H * P)
    assert_parity(ytot, ytot_ref, torch.float32, "y+D*x")
    assert_parity(h, h_ref, torch.float32, "h_last")


@pytest.mark.gpu
def test_ssd_fwd_config1_row():
    """BASELINE config 1 shapes (bf16), first batch row against the fp64 oracle."""
    cfg = dict(workloads.SSD_CONFIGS[1])
    cfg["batch"] = 1
    x = workloads.ssd_inputs(**cfg)
    x.pop("D")
    args = dict(u=x["u"], A=x["A"], B=x["B"], C=x["C"], delta_raw=x["delta_raw"],
                delta_bias=None, h_init=None, length=None)
    y_ref, h_ref = ref.ssd_scan_forward(**args, chunk_size=cfg["chunk"])
    y, h = run_fwd(args, cfg["chunk"])
    assert_parity(y, y_ref, torch.bfloat16, "y")
    assert_parity(h, h_ref, torch.bfloat16, "h_last")


@pytest.mark.gpu
def test_ssd_fwd_split_chaining_on_device():
    """scan(x[:k]) -> h; scan(x[k:], h_init=h) == scan(x) on the device."""
    x = make_inputs(b=2, L=192, H=4, P=32, N=32, G=2, dtype=torch.float32)
    y, h = run_fwd(x, 64)
    first = {k: (v[:, :64] if k in ("u", "B", "C", "delta_raw") else v) for k, v in x.items()}
    second = {k: (v[:, 64:] if k in ("u", "B", "C", "delta_raw") else v) for k, v in x.items()}
    y1, h1 = run_fwd(first, 64)
    second["h_init"] = h1.cpu()
    y2, h2 = run_fwd(second, 64)
    torch.testing.assert_close(torch.cat([y1, y2], 1), y, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(h2, h, rtol=1e-4, atol=1e-5)


def test_ssd_validation_raises_value_error():
    from selective_attention.ops import SSDScanFn
    x = make_inputs()
    with pytest.raises(ValueError):
        SSDScanFn.apply(x["u"], x["A"][:3], x["B"], x["C"], x["delta_raw"])
    with pytest.raises(ValueError):
        SSDScanFn.apply(x["u"], x["A"], x["B"][:, :5], x["C"], x["delta_raw"])
    with pytest.raises(ValueError):
        SSDScanFn.apply(x["u"][0], x["A"], x["B"], x["C"], x["delta_raw"])
    with pytest.raises(ValueError):
        SSDScanFn.apply(x["u"], x["A"], x["B"], x["C"], x["delta_raw"], None, None,
                        torch.tensor([3]))


@pytest.mark.gpu
def test_ssd_fp32_large_state_dim_is_rejected():
    """fp32 operands with state_dim > 128 do not fit the LDS tiles: a clear error."""
    x = make_inputs(b=1, L=64, H=2, P=16, N=136, G=1)
    with pytest.raises(RuntimeError, match="state_dim <= 128"):
        run_fwd(x, 32)


@pytest.mark.gpu
def test_ssd_bf16_state_dim_256():
    x = make_inputs(b=1, L=130, H=2, P=32, N=256, G=1, dtype=torch.bfloat16)
    y_ref, h_ref = ref.ssd_scan_forward(**x, chunk_size=64)
    y, h = run_fwd(x, 64)
    assert_parity(y, y_ref, torch.bfloat16, "y")
    assert_parity(h, h_ref, torch.bfloat16, "h_last")


# shapes that take the bf16 register-resident chunk-scan path (N % 32 == 0, P % 16 == 0)
FAST_CASES = [
    ("hpg3_P48", dict(b=2, L=200, H=6, P=48, N=96, G=2, lens=[200, 133]), 64),
    ("hpg8", dict(b=1, L=256, H=8, P=32, N=64, G=1), 128),
    ("chunk96", dict(b=2, L=300, H=4, P=64, N=128, G=2, lens=[300, 95]), 96),
    ("chunk32", dict(b=1, L=100, H=2, P=16, N=32, G=2, with_h=False), 32),
    ("p128_n192_c256", dict(b=2, L=600, H=2, P=128, N=192, G=1, lens=[600, 517]), 256),
    # state_dim 256: two heads per block, the second head chunk partial
    ("n256_hpg3", dict(b=1, L=160, H=3, P=64, N=256, G=1, lens=[150]), 64),
    # 75 groups of four tau tiles: the longest-first block order over several
    # full windows of one XCD's resident blocks and a partial last one
    ("windows_partial", dict(b=3, L=1100, H=10, P=64, N=128, G=5, lens=[1100, 700, 1033]), 256),
]


@pytest.mark.gpu
@pytest.mark.parametrize("name,shape,chunk", FAST_CASES, ids=[c[0] for c in FAST_CASES])
def test_ssd_fwd_bf16_fast_path(name, shape, chunk):
    print(f"ssd fwd fast {name} chunk={chunk}", flush=True)
    x = make_inputs(dtype=torch.bfloat16, **shape)
    y_ref, h_ref = ref.ssd_scan_forward(**x, chunk_size=chunk)
    y, h = run_fwd(x, chunk)
    assert_parity(y, y_ref, torch.bfloat16, "y")
    assert_parity(h, h_ref, torch.bfloat16, "h_last")


def signed_dt_inputs(softplus, dtype=torch.bfloat16, **shape):
    """Inputs for the exact-decay branch: with softplus off, dt = clamp(delta_raw)
    takes both signs (|A| kept small so exp(dc) stays moderate)."""
    x = make_inputs(dtype=dtype, with_bias=False, **shape)
    g = torch.Generator().manual_seed(17)
    x["A"] = -(torch.rand(x["A"].shape, generator=g) * 0.5 + 0.1)
    if not softplus:
        x["delta_raw"] = (torch.randn(x["delta_raw"].shape, generator=g) * 0.03 + 0.01).to(dtype)
    return x


SIGNED_LIMITS = [(False, (-0.02, 0.05)), (True, (-1.0, float("inf")))]


@pytest.mark.gpu
@pytest.mark.parametrize("softplus,limit", SIGNED_LIMITS)
def test_ssd_fwd_bf16_fast_path_signed_limits(softplus, limit):
    """A negative lower dt limit switches the bf16 chunk scan from the
    factorised off-diagonal decay to the exact per-element form (dc need not
    be monotone); with softplus off some dt are negative."""
    print(f"ssd fwd fast signed softplus={softplus} limit={limit}", flush=True)
    x = signed_dt_inputs(softplus, b=2, L=256, H=4, P=64, N=128, G=2, lens=[256, 170])
    y_ref, h_ref = ref.ssd_scan_forward(**x, chunk_size=64, use_delta_softplus=softplus,
                                        delta_limit=limit)
    y, h = run_fwd(x, 64, softplus=softplus, limit=limit)
    assert_parity(y, y_ref, torch.bfloat16, "y")
    assert_parity(h, h_ref, torch.bfloat16, "h_last")


def _nan_into_lds():
    """A GEMM of all-NaN matrices: its operand tiles fill tens of KB of LDS on
    every CU with NaN, which the next kernels there find uninitialised."""
    junk = torch.full((2048, 2048), float("nan"), device="cuda")
    (junk @ junk).sum().item()


@pytest.mark.gpu
@pytest.mark.parametrize("chunk", [16, 48, 1])
def test_ssd_short_chunk_ignores_stale_lds(chunk):
    """Regression: with chunk_size not a multiple of 32 the fp32 kernels
    stage positions past the chunk, whose scale entries were never written;
    0 * (stale NaN) turned them into NaN outputs.  Fills LDS with NaN first,
    then checks that every output and gradient is finite and matches the
    oracle."""
    print(f"ssd short chunk {chunk} after NaN in LDS", flush=True)
    from selective_attention.ops import SSDScanFn
    x = make_inputs(b=1, L=70, H=6, P=32, N=24, G=3, dtype=torch.float32, with_h=False,
                    with_bias=False)
    y_ref, h_ref = ref.ssd_scan_forward(**x, chunk_size=chunk)
    for _ in range(3):
        _nan_into_lds()
        xd = {k: (v.cuda().requires_grad_(k in ("u", "B", "C", "delta_raw"))
                  if isinstance(v, torch.Tensor) else v) for k, v in x.items()}
        y, h = SSDScanFn.apply(xd["u"], xd["A"], xd["B"], xd["C"], xd["delta_raw"], None, None,
                               None, chunk, True, (0.0, float("inf")), True)
        _nan_into_lds()
        grads = torch.autograd.grad((y,), [xd[k] for k in ("u", "B", "C", "delta_raw")],
                                    (torch.ones_like(y),))
        torch.cuda.synchronize()
        assert_parity(y, y_ref, torch.float32, "y")
        assert_parity(h, h_ref, torch.float32, "h_last")
        for gname, gv in zip(("du", "dB", "dC", "ddelta_raw"), grads):
            assert torch.isfinite(gv).all(), f"{gname}: non-finite values"


@pytest.mark.gpu
@pytest.mark.parametrize("N,chunk,lens", [(128, 96, [300, 95, 300]), (64, 256, [300, 1, 212])])
def test_ssd_fwd_chunk_state_pass_equals_two_kernels(N, chunk, lens):
    """With at least two blocks per CU (b H (P / 64) (N / 64) >= 2 CUs) the
    chunk states and state passing run as one kernel; a single batch row
    (fewer blocks) runs chunk_outer_bf16 + state_passing_fwd.  Every row's
    entry states, h_last, dt and dc are bit-equal between the two, and the
    one-kernel states match the oracle's at 1e-4 of their scale."""
    from selective_attention.kernels.ssd_scan import ssd_scan_forward
    from selective_attention.profiling import kernel_timer
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    H = 128
    b = max(3, -(-2 * cus // (H * (N // 64))))
    lens = (lens * b)[:b]
    print(f"ssd fwd one-kernel chunk states: b={b} H={H} N={N} chunk={chunk} cus={cus}", flush=True)
    x = make_inputs(dtype=torch.bfloat16, b=b, L=300, H=H, P=64, N=N, G=4, lens=lens)

    def run(xs):
        xd = to_dev(xs)
        with kernel_timer() as kt:
            _, h, (dt, dc, st) = ssd_scan_forward(xd["u"], xd["A"], xd["B"], xd["C"], xd["delta_raw"],
                                                  xd["delta_bias"], xd["h_init"], xd["length"],
                                                  chunk, return_saved=True)
            torch.cuda.synchronize()
        return (h, dt, dc, st), kt.stats

    full, kfull = run(x)
    assert "chunk_state_pass_fwd" in kfull and "state_passing_fwd" not in kfull, sorted(kfull)
    for r in (0, b - 1):
        xr = {k: (v[r:r + 1] if isinstance(v, torch.Tensor) and k not in ("A", "delta_bias") else v)
              for k, v in x.items()}
        one, kone = run(xr)
        assert "state_passing_fwd" in kone and "chunk_state_pass_fwd" not in kone, sorted(kone)
        for name, a, o in zip(("h_last", "dt", "dc", "states"), full, one):
            assert torch.equal(a[r:r + 1], o), f"row {r}: {name} differs from the two-kernel path"
    xs = {k: (v[:2] if isinstance(v, torch.Tensor) and k not in ("A", "delta_bias") else v)
          for k, v in x.items()}
    _, h_ref, it = ref.ssd_scan_forward(**xs, chunk_size=chunk, return_intermediates=True)
    assert_scaled(full[3][:2], it["H_in"], "states", frac=1e-4)
    assert_scaled(full[0][:2], h_ref, "h_last", frac=1e-4)


@pytest.mark.gpu
@pytest.mark.parametrize("shape,chunk", [
    # chunk 96: each chunk is one full and one 32-row t tile; ragged lengths
    (dict(b=2, L=300, H=4, P=64, N=128, G=2, lens=[300, 95]), 96),
    # two p tiles, three n blocks, the last chunk partial
    (dict(b=1, L=600, H=2, P=128, N=192, G=1), 256),
    # no initial state, state_dim 64
    (dict(b=2, L=256, H=4, P=64, N=64, G=1, with_h=False), 64),
])
def test_ssd_fwd_chunk_states_near_fp32(shape, chunk):
    """The chunk entry states and h_last of the bf16 path at shapes with few
    blocks (chunk_outer_bf16 + state_passing_fwd, w u as hi + lo planes)
    against the oracle's at 1e-4 of their scale, and dt, dc at the fp32
    bound."""
    from selective_attention.kernels.ssd_scan import ssd_scan_forward
    print(f"ssd fwd chunk states {shape} chunk={chunk}", flush=True)
    x = make_inputs(dtype=torch.bfloat16, **shape)
    xd = to_dev(x)
    _, h, (dt, dc, st) = ssd_scan_forward(xd["u"], xd["A"], xd["B"], xd["C"], xd["delta_raw"],
                                          xd["delta_bias"], xd["h_init"], xd["length"], chunk,
                                          return_saved=True)
    torch.cuda.synchronize()
    _, h_ref, it = ref.ssd_scan_forward(**x, chunk_size=chunk, return_intermediates=True)
    assert_parity(dt, it["dt"], torch.float32, "dt")
    assert_parity(dc, it["dc"], torch.float32, "dc")
    assert_scaled(st, it["H_in"], "states", frac=1e-4)
    assert_scaled(h, h_ref, "h_last", frac=1e-4)
