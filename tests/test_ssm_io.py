"""SSM block stages around the scan: oracle pins (CPU) and HIP parity (GPU).

Reference: modules/ssm.py:116-125 (SiLU + causal depthwise conv + split),
:144-150 (D skip + SiLU gate), :173-182 and inference/ssm_cache.py (decode
context).
"""
import math

import pytest
import torch

from oracle import ssm_io as ref
from tests.helpers import assert_parity

F64 = torch.float64


def conv_inputs(b=2, L=50, x_dim=48, bc_dim=16, K=4, dtype=torch.float32, seed=0, bias=True):
    g = torch.Generator().manual_seed(seed)
    ch = x_dim + 2 * bc_dim
    hbc = (torch.randn(b, L, ch, generator=g) * 1.5).to(dtype)
    w = torch.randn(ch, 1, K, generator=g) / math.sqrt(K)
    bs = torch.randn(ch, generator=g) * 0.1 if bias else None
    return hbc, w, bs


# ---------------------------------------------------------------------------
# oracle pins (CPU)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("K", [1, 2, 3, 4, 7])
@pytest.mark.parametrize("L", [1, 3, 40])
def test_oracle_conv_matches_reference_composition(K, L):
    """== F.silu -> F.conv1d(groups=ch, padding=K-1) -> [:L] (modules/ssm.py:116-118)."""
    hbc, w, bs = conv_inputs(L=L, K=K, dtype=F64)
    got = ref.conv_forward(hbc, w, bs)
    exp = ref.conv_forward_torch(hbc, w, bs)
    assert torch.allclose(got, exp, rtol=1e-12, atol=1e-12)


def test_oracle_conv_brute_force():
    hbc, w, bs = conv_inputs(b=1, L=6, x_dim=2, bc_dim=1, K=3, dtype=F64)
    got = ref.conv_forward(hbc, w, bs)
    w2 = w.reshape(w.shape[0], -1)
    for t in range(6):
        for c in range(4):
            s = bs[c].item()
            for j in range(3):
                r = t - 2 + j
                if r >= 0:
                    z = hbc[0, r, c].item()
                    s += w2[c, j].item() * z / (1 + math.exp(-z))
            assert abs(got[0, t, c].item() - s) < 1e-12


def test_oracle_conv_catches_a_shifted_window():
    """Negative control: a conv whose window is off by one row fails the
    composition pin (so the pin constrains the causal indexing)."""
    hbc, w, bs = conv_inputs(L=20, K=4, dtype=F64)
    exp = ref.conv_forward_torch(hbc, w, bs)
    shifted = ref.conv_forward(torch.cat([torch.zeros_like(hbc[:, :1]), hbc[:, :-1]], 1), w, bs)
    assert not torch.allclose(shifted, exp, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("K", [1, 4])
def test_oracle_conv_backward_matches_autograd(K):
    hbc, w, bs = conv_inputs(L=30, K=K, dtype=F64)
    g = torch.randn(hbc.shape, generator=torch.Generator().manual_seed(3), dtype=F64)
    h = hbc.clone().requires_grad_(True)
    wr = w.to(F64).clone().requires_grad_(True)
    br = bs.to(F64).clone().requires_grad_(True)
    out = ref.conv_forward_torch(h, wr, br)
    out.backward(g)
    dh, dw, db = ref.conv_backward(hbc, w, g)
    assert torch.allclose(dh, h.grad, rtol=1e-10, atol=1e-10)
    assert torch.allclose(dw, wr.grad.reshape(dw.shape), rtol=1e-10, atol=1e-10)
    assert torch.allclose(db, br.grad, rtol=1e-10, atol=1e-10)


def test_oracle_decode_steps_equal_batch_conv():
    """Streaming: steps from an all-zero context reproduce the batch conv row by row."""
    hbc, w, bs = conv_inputs(b=2, L=12, K=4, dtype=F64)
    ctx = torch.zeros(2, hbc.shape[2], 4, dtype=F64)
    batch = ref.conv_forward(hbc, w, bs)
    for t in range(12):
        out, ctx = ref.conv_step(hbc[:, t], ctx, w, bs)
        assert torch.allclose(out, batch[:, t], rtol=1e-12, atol=1e-12)


def test_oracle_build_ctx_then_step_continues_the_sequence():
    """The prefill context of rows [0, len) followed by a step on row len
    equals the batch conv at row len (per batch row, ragged lengths)."""
    hbc, w, bs = conv_inputs(b=3, L=10, K=4, dtype=F64)
    lens = torch.tensor([9, 2, 0])
    ctx = ref.build_conv_ctx(hbc, lens, 4)
    batch = ref.conv_forward(hbc, w, bs)
    for i, n in enumerate(lens.tolist()):
        out, _ = ref.conv_step(hbc[i:i + 1, n], ctx[i:i + 1], w, bs)
        assert torch.allclose(out[0], batch[i, n], rtol=1e-12, atol=1e-12)


def test_oracle_build_ctx_matches_reference_gather():
    """Restates ssm_cache.py:24-36 with torch.gather (lengths given) and the
    lengths=None branch (:18-22) on short and long rows."""
    hbc, _, _ = conv_inputs(b=3, L=5, K=4)
    lens = torch.tensor([5, 2, 7])
    x = hbc.transpose(1, 2)
    idx = torch.arange(4)[None, None, :]
    src = lens[:, None, None] - 4 + idx
    valid = (src >= 0) * (src < lens[:, None, None])
    g = torch.gather(x, 2, src.clamp(0, 4).expand(3, x.shape[1], 4)) * valid.expand(3, x.shape[1], 4)
    assert torch.equal(ref.build_conv_ctx(hbc, lens, 4), g)
    short = hbc[:, :2]
    ctx = torch.zeros(3, hbc.shape[2], 4)
    ctx[:, :, -2:] = short.transpose(1, 2)
    assert torch.equal(ref.build_conv_ctx(short, None, 4), ctx)
    assert torch.equal(ref.build_conv_ctx(hbc, None, 4), x[:, :, -4:])


def test_oracle_gate_backward_matches_autograd():
    g = torch.Generator().manual_seed(1)
    y, x, gate = (torch.randn(3, 5, 16, generator=g, dtype=F64) for _ in range(3))
    D = torch.randn(16, generator=g, dtype=F64)
    dout = torch.randn(3, 5, 16, generator=g, dtype=F64)
    leaves = [t.clone().requires_grad_(True) for t in (y, x, D, gate)]
    ref.gate_forward(*leaves).backward(dout)
    for a, b in zip(ref.gate_backward(dout, y, x, D, gate), leaves):
        assert torch.allclose(a, b.grad, rtol=1e-10, atol=1e-12)


# ---------------------------------------------------------------------------
# HIP parity (GPU)
# ---------------------------------------------------------------------------
CONV_CASES = [
    ("vec_k4", dict(b=2, L=300, x_dim=128, bc_dim=64, K=4)),
    ("scalar_odd", dict(b=2, L=37, x_dim=20, bc_dim=6, K=3)),
    ("short_seq", dict(b=3, L=2, x_dim=64, bc_dim=32, K=4)),
    ("k1_nobias", dict(b=1, L=129, x_dim=32, bc_dim=16, K=1, bias=False)),
    ("k8", dict(b=1, L=200, x_dim=256, bc_dim=8, K=8)),
]


def _dev(*ts):
    return [None if t is None else t.cuda() for t in ts]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("name,shape", CONV_CASES, ids=[c[0] for c in CONV_CASES])
def test_ssm_conv_fwd_bwd_parity(dtype, name, shape):
    from selective_attention.ops import SSMConvFn
    print(f"ssm conv {name} dtype={dtype}", flush=True)
    shape = dict(shape)
    x_dim, bc_dim = shape["x_dim"], shape["bc_dim"]
    hbc, w, bs = conv_inputs(dtype=dtype, **shape)
    gen = torch.Generator().manual_seed(7)
    gx = torch.randn(hbc.shape[0], hbc.shape[1], x_dim, generator=gen)
    gB = torch.randn(hbc.shape[0], hbc.shape[1], bc_dim, generator=gen)
    gC = torch.randn(hbc.shape[0], hbc.shape[1], bc_dim, generator=gen)
    hd, wd, bd = _dev(hbc, w, bs)
    hd.requires_grad_(True)
    wd.requires_grad_(True)
    if bd is not None:
        bd.requires_grad_(True)
    x, B, C = SSMConvFn.apply(hd, wd, bd, x_dim, bc_dim)
    assert x.is_contiguous() and B.is_contiguous() and C.is_contiguous()
    torch.autograd.backward([x, B, C], [gx.to(dtype).cuda(), gB.to(dtype).cuda(), gC.to(dtype).cuda()])
    torch.cuda.synchronize()
    exp = ref.conv_forward(hbc, w, bs)
    ex, eB, eC = ref.split(exp, x_dim, bc_dim)
    assert_parity(x, ex, dtype, "x")
    assert_parity(B, eB, dtype, "B")
    assert_parity(C, eC, dtype, "C")
    g = torch.cat([gx.to(dtype), gB.to(dtype), gC.to(dtype)], -1)
    dh, dw, db = ref.conv_backward(hbc, w, g)
    assert_parity(hd.grad, dh, dtype, "dhBC")
    # weight / bias gradients are fp32 sums over b*L rows of bf16-rounded products
    assert_parity(wd.grad.reshape(dw.shape), dw, torch.float32 if dtype == torch.float32 else torch.bfloat16, "dW")
    if bd is not None:
        assert_parity(bd.grad, db, torch.float32 if dtype == torch.float32 else torch.bfloat16, "dbias")


@pytest.mark.gpu
def test_ssm_conv_grads_deterministic():
    from selective_attention.kernels.ssm_io import ssm_conv_backward
    hbc, w, _ = conv_inputs(b=2, L=500, x_dim=128, bc_dim=64, dtype=torch.bfloat16)
    g = torch.randn(2, 500, 256, dtype=torch.bfloat16).cuda()
    hd, wd = _dev(hbc, w)
    a = ssm_conv_backward(hd, wd, g[..., :128], g[..., 128:192], g[..., 192:], 128, 64)
    b = ssm_conv_backward(hd, wd, g[..., :128], g[..., 128:192], g[..., 192:], 128, 64)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_ssm_conv_ctx_and_steps(dtype):
    """Prefill context (bit-exact gather, ragged lengths incl. 0 and < K),
    then decode steps continuing each row == the batch conv (oracle), and the
    in-place context after the steps == the oracle's."""
    from selective_attention.ops import build_conv_ctx, ssm_conv_step
    print(f"ssm conv ctx/steps dtype={dtype}", flush=True)
    x_dim, bc_dim, K = 40, 12, 4
    hbc, w, bs = conv_inputs(b=4, L=24, x_dim=x_dim, bc_dim=bc_dim, K=K, dtype=dtype)
    lens = torch.tensor([24, 3, 0, 17])
    prefix = hbc[:, :20]
    ctx = build_conv_ctx(prefix.cuda(), lens.clamp(max=20).cuda(), K)
    exp_ctx = ref.build_conv_ctx(prefix, lens.clamp(max=20), K)
    assert ctx.dtype == dtype and torch.equal(ctx.cpu(), exp_ctx)
    full_ctx = build_conv_ctx(prefix.cuda(), None, K)
    assert torch.equal(full_ctx.cpu(), ref.build_conv_ctx(prefix, None, K))
    wd, bd = _dev(w, bs)
    ectx = exp_ctx.clone()
    for t in range(4):
        row = torch.stack([hbc[i, min(int(n), 20) + t] for i, n in enumerate(lens.clamp(max=20).tolist())])
        x, B, C = ssm_conv_step(row.cuda(), ctx, wd, bd, x_dim, bc_dim)
        out, ectx = ref.conv_step(row, ectx, w, bs)
        ex, eB, eC = ref.split(out, x_dim, bc_dim)
        assert_parity(x, ex, dtype, f"x step {t}")
        assert_parity(B, eB, dtype, f"B step {t}")
        assert_parity(C, eC, dtype, f"C step {t}")
        assert torch.equal(ctx.cpu(), ectx.to(dtype)), f"context after step {t}"


GATE_CASES = [("vec", (3, 70, 256)), ("scalar", (2, 33, 20))]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("name,shape", GATE_CASES, ids=[c[0] for c in GATE_CASES])
def test_ssm_gate_fwd_bwd_parity(dtype, name, shape):
    from selective_attention.ops import SSMGateFn
    print(f"ssm gate {name} dtype={dtype}", flush=True)
    g = torch.Generator().manual_seed(2)
    y = torch.randn(*shape, generator=g)
    x = torch.randn(*shape, generator=g).to(dtype)
    gate = (torch.randn(*shape, generator=g) * 2).to(dtype)
    D = torch.randn(shape[-1], generator=g)
    dout = torch.randn(*shape, generator=g).to(dtype)
    leaves = [t.cuda().requires_grad_(True) for t in (y, x, D, gate)]
    out = SSMGateFn.apply(*leaves)
    out.backward(dout.cuda())
    torch.cuda.synchronize()
    assert out.dtype == dtype
    assert_parity(out, ref.gate_forward(y, x, D, gate), dtype, "out")
    names = ["dy", "dx", "dD", "dgate"]
    for name_, e, leaf in zip(names, ref.gate_backward(dout, y, x, D, gate), leaves):
        assert_parity(leaf.grad, e, dtype, name_)


class _RoundGradFn(torch.autograd.Function):
    """Identity whose backward rounds the incoming gradient to bf16."""

    @staticmethod
    def forward(ctx, t):
        return t.view_as(t)

    @staticmethod
    def backward(ctx, g):
        return g.to(torch.bfloat16).to(g.dtype)


def _round_grad(t):
    return _RoundGradFn.apply(t)


@pytest.mark.gpu
def test_ssm_block_core_chain():
    """The SSM block's compute between in_proj and out_proj on the new ops
    (modules/ssm.py:110-150): conv prologue -> SSDScanFn -> gate epilogue,
    forward and backward, against the oracle composition in fp64."""
    from oracle import ssd as ssd_ref
    from selective_attention.ops import SSDScanFn, SSMConvFn, SSMGateFn
    b, L, H, P, G, N, K = 2, 160, 4, 64, 2, 64, 4
    x_dim, bc_dim = H * P, G * N
    gen = torch.Generator().manual_seed(11)
    hbc, w, bs = conv_inputs(b=b, L=L, x_dim=x_dim, bc_dim=bc_dim, K=K, dtype=torch.bfloat16)
    gate = torch.randn(b, L, x_dim, generator=gen).to(torch.bfloat16)
    dr = (torch.randn(b, L, H, generator=gen) - 3.0).to(torch.bfloat16)
    A = -torch.exp(torch.rand(H, generator=gen) * math.log(16.0))
    D = torch.randn(x_dim, generator=gen)
    dout = torch.randn(b, L, x_dim, generator=gen).to(torch.bfloat16)

    hd = hbc.cuda().requires_grad_(True)
    wd, bd, gd, Dd = (t.cuda().requires_grad_(True) for t in (w, bs, gate, D))
    x, B, C = SSMConvFn.apply(hd, wd, bd, x_dim, bc_dim)
    y, _ = SSDScanFn.apply(x.view(b, L, H, P), A.cuda(), B.view(b, L, G, N), C.view(b, L, G, N),
                           dr.cuda(), None, None, None, 64, True, (0.0, float("inf")), True)
    out = SSMGateFn.apply(y.view(b, L, x_dim), x, Dd, gd)
    out.backward(dout.cuda())
    torch.cuda.synchronize()

    # fp64 oracle composition with autograd through the oracle's own pieces
    h64 = hbc.to(F64).requires_grad_(True)
    w64, b64, g64, D64 = (t.to(F64).requires_grad_(True) for t in (w, bs, gate, D))
    xbc = ref.conv_forward_torch(h64, w64, b64)
    # x, B, C and their gradients are bf16 tensors between the stages (as in
    # the reference module run in bf16): round the values straight-through,
    # and the gradients where autograd hands them over (each consumer's, and
    # their sum for x)
    ex, eB, eC = (_round_grad(t + (t.to(torch.bfloat16).to(F64) - t).detach())
                  for t in ref.split(xbc, x_dim, bc_dim))
    ey = ssd_ref.ssd_sequential(_round_grad(ex).reshape(b, L, H, P), A, eB.reshape(b, L, G, N),
                                eC.reshape(b, L, G, N), dr)[0]
    eout = ref.gate_forward(ey.reshape(b, L, x_dim), _round_grad(ex), D64, g64)
    eout.backward(dout.to(F64))
    assert_parity(out, eout.detach(), torch.bfloat16, "out")
    assert_parity(hd.grad, h64.grad, torch.bfloat16, "dhBC")
    assert_parity(wd.grad, w64.grad, torch.bfloat16, "dW")
    assert_parity(bd.grad, b64.grad, torch.bfloat16, "dbias")
    assert_parity(gd.grad, g64.grad, torch.bfloat16, "dgate")
    assert_parity(Dd.grad, D64.grad, torch.bfloat16, "dD")


GATED_CASES = [
    # bf16, head_dim 64, state_dim 64: the fused scan epilogue (y never written)
    ("fused_bf16", torch.bfloat16, dict(b=2, L=200, H=4, P=64, N=64, G=2, lens=[200, 131]), 64),
    # float32: the scan and the gate kernel in turn
    ("unfused_f32", torch.float32, dict(b=2, L=90, H=2, P=24, N=40, G=1), 32),
]


@pytest.mark.gpu
@pytest.mark.parametrize("name,dtype,shape,chunk", GATED_CASES, ids=[c[0] for c in GATED_CASES])
def test_ssd_scan_gated_parity(name, dtype, shape, chunk):
    """SSDScanGatedFn (modules/ssm.py:136-150) against the oracle: scan,
    (y + D u) silu(gate), and every gradient (du includes the D skip)."""
    from oracle import ssd as ssd_ref
    from selective_attention.kernels.ssd_scan import gated_supported
    from selective_attention.ops import SSDScanGatedFn
    from tests.test_ssd_fwd import make_inputs
    print(f"ssd scan gated {name}", flush=True)
    x = make_inputs(dtype=dtype, **shape)
    b, L, H, P = x["u"].shape
    N = x["B"].shape[-1]
    assert gated_supported(dtype, P, N) == (dtype == torch.bfloat16)
    g = torch.Generator().manual_seed(4)
    D = torch.randn(H * P, generator=g)
    gate = (torch.randn(b, L, H, P, generator=g) * 2).to(dtype)
    dout = torch.randn(b, L, H, P, generator=g).to(dtype)
    dh = torch.randn(b, H, P, N, generator=g)

    names = ["u", "A", "B", "C", "delta_raw", "delta_bias", "h_init"]
    leaves = {k: x[k].cuda().requires_grad_(True) for k in names if x[k] is not None}
    Dd, gd = D.cuda().requires_grad_(True), gate.cuda().requires_grad_(True)
    length = None if x["length"] is None else x["length"].cuda()
    out, h = SSDScanGatedFn.apply(leaves["u"], leaves["A"], leaves["B"], leaves["C"],
                                  leaves["delta_raw"], leaves.get("delta_bias"), leaves.get("h_init"),
                                  length, chunk, True, (0.0, float("inf")), Dd, gd)
    torch.autograd.backward([out, h], [dout.cuda(), dh.cuda()])
    torch.cuda.synchronize()
    assert out.dtype == dtype and h.dtype == torch.float32

    y_ref, h_ref = ssd_ref.ssd_scan_forward(**x, chunk_size=chunk)
    flat = lambda t: t.reshape(b, L, H * P)
    out_ref = ref.gate_forward(flat(y_ref), flat(x["u"]), D, flat(gate)).reshape(b, L, H, P)
    dy, dskip, dD, dgate = ref.gate_backward(flat(dout), flat(y_ref), flat(x["u"]), D, flat(gate))
    grads = ssd_ref.ssd_scan_backward(x["u"], x["A"], x["B"], x["C"], x["delta_raw"], x["delta_bias"],
                                      x["h_init"], dy.reshape(b, L, H, P), dh, x["length"], chunk)
    exp = dict(zip(names, grads))
    exp["u"] = exp["u"] + dskip.reshape(b, L, H, P)
    assert_parity(out, out_ref, dtype, "out")
    assert_parity(h, h_ref, dtype, "h_last")
    for k, leaf in leaves.items():
        tol = dtype if k in ("u", "B", "C", "delta_raw") or dtype == torch.float32 else torch.bfloat16
        assert_parity(leaf.grad, exp[k], tol, f"d{k}")
    assert_parity(Dd.grad, dD, dtype, "dD")
    assert_parity(gd.grad, dgate.reshape(b, L, H, P), dtype, "dgate")
