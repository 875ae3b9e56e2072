"""Selective state update (SSUFn): oracle pins (CPU) and HIP parity (GPU)."""
import math

import pytest
import torch

from oracle import ssd as ssd_ref
from oracle import ssu as ssu_ref
from selective_attention import workloads
from tests.helpers import assert_parity

F64 = torch.float64


def _small(b=3, H=4, P=8, N=12, G=2, dtype=torch.float32, seed=1, bias=True):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(b, H, P, generator=g).to(dtype)
    A = -torch.exp(torch.rand(H, generator=g) * math.log(16.0))
    B = (torch.randn(b, G, N, generator=g) / 3).to(dtype)
    C = (torch.randn(b, G, N, generator=g) / 3).to(dtype)
    dr = (torch.randn(b, H, generator=g) - 1).to(dtype)
    db = torch.randn(H, generator=g) * 0.2 if bias else None
    h = torch.randn(b, H, P, N, generator=g) * 0.1
    return dict(u=u, A=A, B=B, C=C, delta_raw=dr, delta_bias=db, h=h)


# ---------------------------------------------------------------- oracle pins
def test_oracle_ssu_equals_one_step_scan():
    x = _small(dtype=F64)
    y, h = ssu_ref.ssu_forward(**x)
    ys, hs = ssd_ref.ssd_scan_forward(x["u"][:, None], x["A"], x["B"][:, None], x["C"][:, None],
                                      x["delta_raw"][:, None], x["delta_bias"], x["h"], None, 4)
    torch.testing.assert_close(y, ys[:, 0], rtol=1e-12, atol=1e-14)
    torch.testing.assert_close(h, hs, rtol=1e-12, atol=1e-14)


def test_oracle_ssu_brute_force():
    x = _small(b=2, H=2, P=3, N=4, G=1, dtype=F64)
    y, h = ssu_ref.ssu_forward(**x, use_delta_softplus=False, delta_limit=(0.01, 0.7))
    for bb in range(2):
        for hh in range(2):
            z = float(x["delta_raw"][bb, hh] + x["delta_bias"][hh])
            dt = min(max(z, 0.01), 0.7)
            for p in range(3):
                acc = 0.0
                for n in range(4):
                    hv = (float(x["h"][bb, hh, p, n]) * math.exp(float(x["A"][hh]) * dt)
                          + dt * float(x["u"][bb, hh, p]) * float(x["B"][bb, 0, n]))
                    assert abs(hv - float(h[bb, hh, p, n])) < 1e-12
                    acc += hv * float(x["C"][bb, 0, n])
                assert abs(acc - float(y[bb, hh, p])) < 1e-12


# ---------------------------------------------------------- validation (CPU)
def test_validation_raises_value_error():
    from selective_attention.ops import SSUFn
    x = _small()
    bad = dict(x)
    bad["A"] = torch.zeros(5)
    with pytest.raises(ValueError):
        SSUFn.forward(**bad)
    bad = dict(x)
    bad["h"] = x["h"][0]
    with pytest.raises(ValueError):
        SSUFn.forward(**bad)
    bad = dict(x)
    bad["B"] = x["B"][:, :, :5]
    with pytest.raises(ValueError):
        SSUFn.forward(**bad)


def test_cpu_tensors_are_rejected():
    from selective_attention.ops import SSUFn
    with pytest.raises(ValueError):
        SSUFn.forward(**_small())


# ---------------------------------------------------------------- GPU parity
def _run_gpu(x, dtype, **kw):
    from selective_attention.ops import SSUFn
    dev = torch.device("cuda")
    xd = {k: (None if v is None else v.to(dev)) for k, v in x.items()}
    h_dev = xd["h"]
    y, h_out = SSUFn.forward(xd["u"], xd["A"], xd["B"], xd["C"], xd["delta_raw"],
                             xd["delta_bias"], h_dev, **kw)
    torch.cuda.synchronize()
    assert h_out.data_ptr() == h_dev.data_ptr(), "state must be updated in place"
    assert y.dtype == dtype
    return y, h_out


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [dict(b=3, H=4, P=8, N=12, G=2), dict(b=2, H=6, P=5, N=7, G=3),
                                   dict(b=1, H=2, P=16, N=256, G=1), dict(b=2, H=4, P=4, N=16, G=4)])
@pytest.mark.parametrize("bias", [True, False])
def test_ssu_parity_small(dtype, shape, bias):
    print(f"ssu small dtype={dtype} shape={shape} bias={bias}", flush=True)
    x = _small(dtype=dtype, bias=bias, **shape)
    y_ref, h_ref = ssu_ref.ssu_forward(**x)
    y, h = _run_gpu(x, dtype)
    assert_parity(h, h_ref, torch.float32, "h")
    assert_parity(y, y_ref, dtype, "y")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_ssu_softplus_threshold(dtype):
    """Rows with delta_raw above the softplus threshold 20 (dt = z, up to 150):
    the identity branch, no overflow; the state is all but reset there."""
    print(f"ssu large z dtype={dtype}", flush=True)
    x = _small(dtype=dtype, bias=True, b=8, H=32, P=64, N=128, G=8)
    g = torch.Generator().manual_seed(31)
    dr = x["delta_raw"].float()
    m = torch.rand(dr.shape, generator=g) < 0.25
    x["delta_raw"] = torch.where(m, 20.5 + 129.5 * torch.rand(dr.shape, generator=g),
                                 dr).to(x["delta_raw"].dtype)
    y_ref, h_ref = ssu_ref.ssu_forward(**x)
    y, h = _run_gpu(x, dtype)
    assert_parity(h, h_ref, torch.float32, "h")
    assert_parity(y, y_ref, dtype, "y")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [dict(b=3, H=4, P=8, N=12, G=2), dict(b=2, H=6, P=5, N=7, G=3),
                                   dict(b=4, H=32, P=64, N=128, G=1)])
def test_ssu_gated_matches_unfused(dtype, shape):
    """The decode step's fused kernel (state update, y + D u, SiLU gate)
    against SSUFn then the gate kernel: the same state bit for bit, and the
    same output (y rounded to the activation dtype in both)."""
    from selective_attention.kernels.ssm_io import ssm_gate_forward
    from selective_attention.kernels.ssu import ssu_gated_forward
    print(f"ssu gated dtype={dtype} shape={shape}", flush=True)
    x = _small(dtype=dtype, bias=True, **shape)
    b, H, P = x["u"].shape
    g = torch.Generator().manual_seed(3)
    D = torch.randn(H * P, generator=g).cuda()
    gate = torch.randn(b, H, P, generator=g).to(dtype).cuda()
    y, h1 = _run_gpu(x, dtype)
    e = ssm_gate_forward(y.reshape(b, H * P), x["u"].cuda().reshape(b, H * P), D,
                         gate.reshape(b, H * P)).view(b, H, P)
    xd = {k: (None if v is None else v.cuda()) for k, v in x.items()}
    out = ssu_gated_forward(xd["u"], xd["A"], xd["B"], xd["C"], xd["delta_raw"],
                            xd["delta_bias"], xd["h"], D, gate)
    torch.cuda.synchronize()
    assert torch.equal(xd["h"], h1)
    assert out.dtype == dtype and torch.equal(out, e)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [dict(b=2, H=4, P=32, N=64, G=2), dict(b=3, H=2, P=128, N=32, G=1),
                                   dict(b=1, H=6, P=96, N=128, G=3), dict(b=2, H=2, P=64, N=96, G=2)])
def test_ssu_parity_head_blocks(dtype, shape):
    """Shapes of the per-(batch row, head) kernel (P and N multiples of 32:
    1, 2 or 4 float4 strips per lane and 1, 2 or 4 rows per thread) and two
    that fall back to the row kernel (P = 96, N = 96)."""
    print(f"ssu head blocks dtype={dtype} shape={shape}", flush=True)
    x = _small(dtype=dtype, bias=True, **shape)
    y_ref, h_ref = ssu_ref.ssu_forward(**x)
    y, h = _run_gpu(x, dtype)
    assert_parity(h, h_ref, torch.float32, "h")
    assert_parity(y, y_ref, dtype, "y")


@pytest.mark.gpu
def test_ssu_gated_strided_views():
    """Gate and x as column slices of one wider projection (the layout of an
    in_proj output): the wrapper makes them contiguous, and the result equals
    the call on contiguous copies bit for bit."""
    from selective_attention.kernels.ssu import ssu_gated_forward
    dtype = torch.bfloat16
    x = _small(dtype=dtype, bias=True, b=4, H=8, P=64, N=128, G=2)
    b, H, P = x["u"].shape
    g = torch.Generator().manual_seed(5)
    proj = torch.randn(b, 3 * H * P, generator=g).to(dtype).cuda()
    gate_v = proj[:, :H * P].view(b, H, P)
    u_v = proj[:, 2 * H * P:].view(b, H, P)
    assert not gate_v.is_contiguous() and not u_v.is_contiguous()
    D = torch.randn(H * P, generator=g).cuda()
    xd = {k: (None if v is None else v.cuda()) for k, v in x.items()}
    h1, h2 = xd["h"].clone(), xd["h"].clone()
    out_v = ssu_gated_forward(u_v, xd["A"], xd["B"], xd["C"], xd["delta_raw"], xd["delta_bias"],
                              h1, D, gate_v)
    out_c = ssu_gated_forward(u_v.contiguous(), xd["A"], xd["B"], xd["C"], xd["delta_raw"],
                              xd["delta_bias"], h2, D, gate_v.contiguous())
    torch.cuda.synchronize()
    assert torch.equal(out_v, out_c) and torch.equal(h1, h2)


@pytest.mark.gpu
@pytest.mark.parametrize("softplus,limit", [(False, (0.0, 0.3)), (True, (0.02, 0.05))])
def test_ssu_parity_limits(softplus, limit):
    x = _small()
    y_ref, h_ref = ssu_ref.ssu_forward(**x, use_delta_softplus=softplus, delta_limit=limit)
    y, h = _run_gpu(x, torch.float32, use_delta_softplus=softplus, delta_limit=limit)
    assert_parity(h, h_ref, torch.float32, "h")
    assert_parity(y, y_ref, torch.float32, "y")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_ssu_parity_config3(dtype):
    print(f"ssu config3 dtype={dtype}", flush=True)
    x = workloads.ssu_inputs(dtype=dtype)
    x.pop("D")
    y_ref, h_ref = ssu_ref.ssu_forward(**x, delta_bias=None)
    y, h = _run_gpu(dict(x, delta_bias=None), dtype)
    assert_parity(h, h_ref, torch.float32, "h")
    assert_parity(y, y_ref, dtype, "y")


@pytest.mark.gpu
def test_ssu_repeated_steps_track_scan():
    """Ten decode steps == one scan over the ten tokens (state chaining)."""
    from selective_attention.ops import SSUFn
    g = torch.Generator().manual_seed(3)
    b, H, P, N, G, T = 2, 4, 8, 16, 2, 10
    u = torch.randn(b, T, H, P, generator=g)
    A = -torch.exp(torch.rand(H, generator=g) * math.log(16.0))
    B = torch.randn(b, T, G, N, generator=g) / 4
    C = torch.randn(b, T, G, N, generator=g) / 4
    dr = torch.randn(b, T, H, generator=g) - 2
    h0 = torch.randn(b, H, P, N, generator=g) * 0.1
    ys_ref, hs_ref = ssd_ref.ssd_sequential(u, A, B, C, dr, None, h0)
    dev = torch.device("cuda")
    h = h0.clone().to(dev)
    ys = []
    for t in range(T):
        y, h = SSUFn.forward(u[:, t].to(dev), A.to(dev), B[:, t].to(dev), C[:, t].to(dev),
                             dr[:, t].to(dev), None, h)
        ys.append(y)
    assert_parity(torch.stack(ys, 1), ys_ref, torch.float32, "y")
    assert_parity(h, hs_ref, torch.float32, "h")
