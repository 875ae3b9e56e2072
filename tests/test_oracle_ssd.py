"""Pins the CPU oracle of the SSD scan (oracle/ssd.py) without the reference.

The reference ships no golden vectors for this path, so the chunked
restatement is pinned by mathematics (fp64):
  * it equals the token-by-token recurrence (independent closed form);
  * it is invariant to the chunk size and chains across split sequences;
  * A = 0 reduces it to a masked matrix product;
  * its manual backward (a restatement of the reference's 9 backward
    kernels) equals finite differences (gradcheck) and torch.autograd
    through both forward formulations.
Two deliberately broken variants show the checks catch index/sign slips.
"""
import math

import pytest
import torch

from oracle import ssd as ref

F64 = torch.float64


def _inputs(b=2, L=12, H=4, P=3, N=5, G=2, seed=0, with_h=True, with_bias=True, lens=None):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(b, L, H, P, generator=g, dtype=F64)
    A = -torch.exp(torch.rand(H, generator=g, dtype=F64) * math.log(16.0))
    B = torch.randn(b, L, G, N, generator=g, dtype=F64) / 2
    C = torch.randn(b, L, G, N, generator=g, dtype=F64) / 2
    dr = torch.randn(b, L, H, generator=g, dtype=F64) - 1.0
    bias = torch.randn(H, generator=g, dtype=F64) * 0.3 if with_bias else None
    h0 = torch.randn(b, H, P, N, generator=g, dtype=F64) * 0.5 if with_h else None
    length = None if lens is None else torch.tensor(lens, dtype=torch.int64)
    return dict(u=u, A=A, B=B, C=C, delta_raw=dr, delta_bias=bias, h_init=h0, length=length)


CASES = [
    dict(),
    dict(with_h=False),
    dict(with_bias=False, lens=[12, 7]),
    dict(L=13, lens=[5, 13]),
    dict(G=1, H=3, lens=[0, 9]),
    dict(G=4, H=4, L=9),
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("chunk", [4, 5, 16])
@pytest.mark.parametrize("softplus,limit", [(True, (0.0, math.inf)), (False, (0.05, 0.4)),
                                            (True, (0.1, 0.6))])
def test_chunked_equals_sequential(case, chunk, softplus, limit):
    x = _inputs(**case)
    y, h = ref.ssd_scan_forward(**x, chunk_size=chunk, use_delta_softplus=softplus,
                                delta_limit=limit)
    ys, hs = ref.ssd_sequential(**x, use_delta_softplus=softplus, delta_limit=limit)
    torch.testing.assert_close(y, ys, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(h, hs, rtol=1e-10, atol=1e-12)


def test_chunk_size_invariance():
    x = _inputs(L=24, lens=[24, 17])
    outs = [ref.ssd_scan_forward(**x, chunk_size=c) for c in (1, 3, 8, 24, 32)]
    for y, h in outs[1:]:
        torch.testing.assert_close(y, outs[0][0], rtol=1e-10, atol=1e-12)
        torch.testing.assert_close(h, outs[0][1], rtol=1e-10, atol=1e-12)


def test_split_sequence_chaining():
    x = _inputs(L=20)
    y, h = ref.ssd_scan_forward(**x, chunk_size=8)
    cut = 11
    first = {k: (v[:, :cut] if k in ("u", "B", "C", "delta_raw") else v) for k, v in x.items()}
    second = {k: (v[:, cut:] if k in ("u", "B", "C", "delta_raw") else v) for k, v in x.items()}
    y1, h1 = ref.ssd_scan_forward(**first, chunk_size=8)
    second["h_init"] = h1
    y2, h2 = ref.ssd_scan_forward(**second, chunk_size=8)
    torch.testing.assert_close(torch.cat([y1, y2], 1), y, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(h2, h, rtol=1e-10, atol=1e-12)


def test_length_freezes_state():
    x = _inputs(L=16, lens=[9, 16])
    y, h = ref.ssd_scan_forward(**x, chunk_size=4)
    short = {k: (v[:1, :9] if k in ("u", "B", "C", "delta_raw") else v) for k, v in x.items()}
    short["h_init"] = x["h_init"][:1]
    short["length"] = None
    ys, hs = ref.ssd_scan_forward(**short, chunk_size=4)
    torch.testing.assert_close(h[:1], hs, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(y[:1, :9], ys, rtol=1e-10, atol=1e-12)
    # beyond the length y is still produced: C_t . (frozen state)
    Ch = x["C"][0, 9:].repeat_interleave(2, dim=1)                        # (7,H,N)
    torch.testing.assert_close(y[0, 9:], torch.einsum("thn,hpn->thp", Ch, hs[0]),
                               rtol=1e-10, atol=1e-12)


def test_A_zero_closed_form():
    x = _inputs(L=10, with_h=True)
    x["A"] = torch.zeros_like(x["A"])
    y, h = ref.ssd_scan_forward(**x, chunk_size=4)
    dt = ref.make_dt(x["delta_raw"], x["delta_bias"], True, (0.0, math.inf), F64)  # (b,L,H)
    Bh = x["B"].repeat_interleave(2, dim=2)
    Ch = x["C"].repeat_interleave(2, dim=2)
    CB = torch.einsum("bthn,bshn->bhts", Ch, Bh)
    mask = torch.tril(torch.ones(10, 10, dtype=torch.bool))
    yy = torch.einsum("bhts,bsh,bshp->bthp", CB * mask, dt, x["u"])
    yy = yy + torch.einsum("bthn,bhpn->bthp", Ch, x["h_init"])
    torch.testing.assert_close(y, yy, rtol=1e-10, atol=1e-12)


# ---------------------------------------------------------------------------
# backward
# ---------------------------------------------------------------------------
class _ManualSSD(torch.autograd.Function):
    """Chunked forward + the oracle's manual backward, for gradcheck."""

    @staticmethod
    def forward(ctx, u, A, B, C, dr, bias, h0, length, chunk, softplus, limit):
        ctx.save_for_backward(u, A, B, C, dr, bias, h0)
        ctx.cfg = (length, chunk, softplus, limit)
        y, h = ref.ssd_scan_forward(u, A, B, C, dr, bias, h0, length, chunk, softplus, limit)
        return y, h

    @staticmethod
    def backward(ctx, dy, dh):
        u, A, B, C, dr, bias, h0 = ctx.saved_tensors
        length, chunk, softplus, limit = ctx.cfg
        g = ref.ssd_scan_backward(u, A, B, C, dr, bias, h0, dy, dh, length, chunk, softplus, limit)
        return (*g, None, None, None, None)


def _masked_loss_grads(fwd, x, dy, dh, **kw):
    leaves = {k: v.clone().requires_grad_(True) for k, v in x.items()
              if v is not None and k != "length"}
    args = dict(x)
    args.update(leaves)
    y, h = fwd(**args, **kw)
    L = y.shape[1]
    lens = x["length"] if x["length"] is not None else torch.full((y.shape[0],), L)
    m = (torch.arange(L)[None, :] < lens[:, None]).to(y.dtype)[..., None, None]
    loss = (y * m * dy).sum() + (h * dh).sum()
    names = list(leaves)
    grads = torch.autograd.grad(loss, [leaves[k] for k in names])
    return dict(zip(names, grads))


GRAD_NAMES = ["u", "A", "B", "C", "delta_raw", "delta_bias", "h_init"]


@pytest.mark.parametrize("case", [dict(), dict(with_h=False, lens=[12, 6]), dict(L=11, lens=[3, 11]),
                                  dict(G=1, H=2, with_bias=False)])
@pytest.mark.parametrize("softplus,limit", [(True, (0.0, math.inf)), (False, (0.05, 0.5))])
def test_manual_backward_equals_autograd(case, softplus, limit):
    x = _inputs(**case)
    g = torch.Generator().manual_seed(7)
    b, L, H, P = x["u"].shape
    N = x["B"].shape[-1]
    dy = torch.randn(b, L, H, P, generator=g, dtype=F64)
    dh = torch.randn(b, H, P, N, generator=g, dtype=F64)
    man = ref.ssd_scan_backward(x["u"], x["A"], x["B"], x["C"], x["delta_raw"], x["delta_bias"],
                                x["h_init"], dy, dh, x["length"], 4, softplus, limit)
    man = dict(zip(GRAD_NAMES, man))
    auto_chunk = _masked_loss_grads(ref.ssd_scan_forward, x, dy, dh, chunk_size=4,
                                    use_delta_softplus=softplus, delta_limit=limit)
    auto_seq = _masked_loss_grads(ref.ssd_sequential, x, dy, dh, use_delta_softplus=softplus,
                                  delta_limit=limit)
    for k, v in auto_chunk.items():
        torch.testing.assert_close(man[k], v, rtol=1e-9, atol=1e-11, msg=f"chunked {k}")
        torch.testing.assert_close(man[k], auto_seq[k], rtol=1e-9, atol=1e-11, msg=f"seq {k}")
    if x["h_init"] is None:
        assert man["h_init"] is None


def test_gradcheck_manual_backward():
    x = _inputs(b=1, L=7, H=2, P=2, N=3, G=1, lens=[6])
    args = [x[k].clone().requires_grad_(True) for k in ("u", "A", "B", "C", "delta_raw",
                                                        "delta_bias", "h_init")]
    # the op ignores dy at t >= length, so differentiate the length-masked output
    m = (torch.arange(7)[None, :] < x["length"][:, None]).to(F64)[..., None, None]

    def fn(*a):
        y, h = _ManualSSD.apply(*a, x["length"], 3, True, (0.0, math.inf))
        return y * m, h

    assert torch.autograd.gradcheck(fn, args, eps=1e-6, atol=1e-7, rtol=1e-5)


def _large_z(x, frac=0.2, lo=20.5, hi=150.0, seed=23):
    """Put delta_raw above the softplus threshold (20) on a fraction of the tokens."""
    g = torch.Generator().manual_seed(seed)
    dr = x["delta_raw"]
    m = torch.rand(dr.shape, generator=g) < frac
    x = dict(x)
    x["delta_raw"] = torch.where(m, lo + (hi - lo) * torch.rand(dr.shape, generator=g, dtype=dr.dtype),
                                 dr)
    return x


def test_softplus_threshold_branch():
    """softplus20 is torch's softplus (beta 1, threshold 20): log(exp(z)+1)
    up to 20, the identity above.  In fp32 the unthresholded formula
    overflows (exp(100) = inf) where softplus20 stays finite."""
    z = torch.linspace(-30.0, 200.0, 2301, dtype=F64)
    torch.testing.assert_close(ref.softplus20(z), torch.nn.functional.softplus(z), rtol=1e-15,
                               atol=1e-15)
    assert torch.equal(ref.softplus20(z)[z > 20], z[z > 20])
    z32 = torch.tensor([19.5, 20.0, 20.5, 100.0], dtype=torch.float32)
    assert torch.isinf(torch.log(torch.exp(z32) + 1.0)[-1])
    assert torch.isfinite(ref.softplus20(z32)).all() and ref.softplus20(z32)[-1] == 100.0


@pytest.mark.parametrize("chunk", [4, 5])
def test_chunked_equals_sequential_large_z(chunk):
    """Tokens with z > 20 (dt = z, the state all but reset) in both forms."""
    x = _large_z(_inputs(L=13, lens=[13, 9]))
    y, h = ref.ssd_scan_forward(**x, chunk_size=chunk)
    ys, hs = ref.ssd_sequential(**x)
    torch.testing.assert_close(y, ys, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(h, hs, rtol=1e-10, atol=1e-12)


def test_manual_backward_equals_autograd_large_z():
    """The manual backward scales d(delta_raw) by sigmoid(z) only for z <= 20
    (backward_kernel.py:1024-1025); autograd through softplus20's branches is
    the independent check, here with ~20 % of the tokens above the threshold."""
    x = _large_z(_inputs(lens=[12, 8]), lo=20.5, hi=24.0)
    g = torch.Generator().manual_seed(8)
    b, L, H, P = x["u"].shape
    N = x["B"].shape[-1]
    dy = torch.randn(b, L, H, P, generator=g, dtype=F64)
    dh = torch.randn(b, H, P, N, generator=g, dtype=F64)
    z = x["delta_raw"] + x["delta_bias"]
    assert (z > 20).sum() > 10
    man = dict(zip(GRAD_NAMES, ref.ssd_scan_backward(
        x["u"], x["A"], x["B"], x["C"], x["delta_raw"], x["delta_bias"], x["h_init"], dy, dh,
        x["length"], 4, True, (0.0, math.inf))))
    auto = _masked_loss_grads(ref.ssd_sequential, x, dy, dh, use_delta_softplus=True,
                              delta_limit=(0.0, math.inf))
    for k, v in auto.items():
        torch.testing.assert_close(man[k], v, rtol=1e-9, atol=1e-11, msg=f"seq {k}")


# ---------------------------------------------------------------------------
# sensitivity: plausible slips in the oracle are caught by the pins above
# ---------------------------------------------------------------------------
def test_planted_mistakes_are_caught(monkeypatch):
    x = _inputs(L=12)
    ys, hs = ref.ssd_sequential(**x)

    good_scan = ref.chunk_scan_forward

    def strict_causal_scan(u, dt, dc, C, H_in, CB, dtype=F64):
        # drops the diagonal term (sigma == tau) of the intra-chunk sum
        Lc = dt.shape[-1]
        CB = CB * (1 - torch.eye(Lc, dtype=CB.dtype))
        return good_scan(u, dt, dc, C, H_in, CB, dtype)

    monkeypatch.setattr(ref, "chunk_scan_forward", strict_causal_scan)
    y, _ = ref.ssd_scan_forward(**x, chunk_size=4)
    assert not torch.allclose(y, ys, rtol=1e-6, atol=1e-8)
    monkeypatch.setattr(ref, "chunk_scan_forward", good_scan)

    good_state = ref.chunk_state_forward

    def wrong_decay_state(u, B, dt, dc, dtype=F64):
        # sign slip in the decay exponent: the min(., 0) clamp then drops the decay
        return good_state(u, B, dt, -dc, dtype)

    monkeypatch.setattr(ref, "chunk_state_forward", wrong_decay_state)
    _, h = ref.ssd_scan_forward(**x, chunk_size=4)
    assert not torch.allclose(h, hs, rtol=1e-6, atol=1e-8)
