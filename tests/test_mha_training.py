"""SelectiveMHA's training forward (modules/selective_attention.py:197-277):
the per-head score statistics reduced in-kernel (sa_score_stats), the std's
gradient (ScoreStdFn) and the whole training forward/backward of the module,
against the fp64 oracle (oracle/attn.py score_stats, selective_mha_train_attn;
oracle/lm.py selective_mha_train_forward).

CPU: oracle pins -- the statistics by brute force, the std against a direct
population std of the valid scores, the training attention at penalty 0
against causal SDPA, and the gate's effect on a single key.
GPU: kernel parity (bf16 and fp32, causal and not, ragged lengths, every
supported head_dim), determinism, the std's gradient against autograd
through the oracle, and the module's outputs, parameter gradients and
running-average update against the oracle module.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import attn as ref
from oracle import lm as lm_ref
from tests.helpers import assert_parity

F64 = torch.float64


def qk(b, H, L, D, seed=0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(b, H, L, D, generator=g).to(dtype),
            torch.randn(b, H, L, D, generator=g).to(dtype))


# ---------------------------------------------------------------- oracle pins
def test_oracle_score_stats_brute_force():
    q, k = qk(2, 3, 11, 8, dtype=F64)
    lens = torch.tensor([11, 6])
    for causal in (True, False):
        st = ref.score_stats(q, k, 0.35, lens, lens, causal)
        for h in range(3):
            c = s1 = s2 = 0.0
            for b in range(2):
                n = int(lens[b])
                for i in range(n):
                    for j in range(n if not causal else i + 1):
                        s = 0.35 * float((q[b, h, i] * k[b, h, j]).sum())
                        c, s1, s2 = c + 1, s1 + s, s2 + s * s
            assert st[h].tolist() == pytest.approx([c, s1, s2], rel=1e-12, abs=1e-12)


def test_oracle_score_std_is_population_std():
    q, k = qk(2, 2, 13, 16, seed=1, dtype=F64)
    lens = torch.tensor([13, 9])
    std = ref.score_std(ref.score_stats(q, k, 0.25, lens, lens, True))
    for h in range(2):
        vals = torch.cat([(0.25 * q[b, h, :n] @ k[b, h, :n].T)[torch.tril(torch.ones(n, n, dtype=torch.bool))]
                          for b, n in ((0, 13), (1, 9))])
        assert float(std[h]) == pytest.approx(float(vals.std(unbiased=False)), rel=1e-12)


def test_oracle_train_attn_penalty_zero_is_causal_sdpa():
    q, k = qk(2, 3, 20, 8, seed=2, dtype=F64)
    v = torch.randn(2, 3, 20, 8, dtype=F64)
    gate = torch.rand(2, 3, 20, dtype=F64) * 0.9 + 0.05
    out, _ = ref.selective_mha_train_attn(q, k, v, gate, 0.0)
    exp = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    assert torch.allclose(out, exp, atol=1e-12, rtol=1e-10)


def test_oracle_train_attn_gate_mutes_a_key_except_on_its_diagonal():
    """A key whose gate is tiny (log-gate very negative) takes no weight from
    the other queries, but its own query still sees it (diagonal exempt)."""
    q, k = qk(1, 1, 12, 8, seed=3, dtype=F64)
    v = torch.randn(1, 1, 12, 8, dtype=F64)
    gate = torch.full((1, 1, 12), 0.9, dtype=F64)
    gate[0, 0, 4] = 1e-300
    out, std = ref.selective_mha_train_attn(q, k, v, gate, 1.0)
    s = (q[0, 0] @ k[0, 0].T) / math.sqrt(8) + torch.log(gate[0, 0]) * std[0]
    s = s.masked_fill(~torch.tril(torch.ones(12, 12, dtype=torch.bool)), float("-inf"))
    s.fill_diagonal_(0.0)
    s += torch.diag((q[0, 0] * k[0, 0]).sum(-1) / math.sqrt(8))
    w = torch.softmax(s, dim=-1)
    assert float(w[7, 4]) < 1e-30 and float(w[4, 4]) > 1e-3
    assert torch.allclose(out[0, 0], w @ v[0, 0], atol=1e-12)


def test_oracle_rope_rotate_is_pairwise_rotation():
    """rope_rotate (modules/rope.py) against its definition: element i and
    i + D/2 form a pair turned by the angle pos * base^(-i / (D/2)), as the
    2x2 matrix [[cos, -sin], [sin, cos]] with the angle taken in Python
    floats.  Position 0 is the identity, pair norms are kept, and the score
    of two rotated vectors depends only on the difference of positions."""
    D, L, base = 8, 7, 10000.0
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, L, D, generator=g, dtype=F64)
    pos = torch.tensor([0, 1, 2, 5, 100, 1000, 8191])
    got = lm_ref.rope_rotate(x, pos, base)
    half = D // 2
    for t in range(L):
        for i in range(half):
            a = float(torch.tensor(float(pos[t]), dtype=torch.float32)
                      * torch.tensor(1.0 / base ** (i / half), dtype=torch.float32))
            c, s = math.cos(a), math.sin(a)
            x0, x1 = x[:, t, i], x[:, t, i + half]
            # the fp32 angle is exact in the oracle; cos/sin of it here in fp64
            torch.testing.assert_close(got[:, t, i], c * x0 - s * x1, rtol=0, atol=1e-6)
            torch.testing.assert_close(got[:, t, i + half], s * x0 + c * x1, rtol=0, atol=1e-6)
    assert torch.equal(got[:, 0], x[:, 0])
    n_in = x[..., :half] ** 2 + x[..., half:] ** 2
    n_out = got[..., :half] ** 2 + got[..., half:] ** 2
    torch.testing.assert_close(n_out, n_in, rtol=1e-12, atol=1e-12)
    q, k = torch.randn(D, generator=g, dtype=F64), torch.randn(D, generator=g, dtype=F64)
    # integer positions below 2^24 give exact fp32 angles, so shifting both
    # positions by the same amount keeps q.k up to the cos / sin rounding
    def score(m, n):
        return float((lm_ref.rope_rotate(q[None], torch.tensor([m]), base)
                      * lm_ref.rope_rotate(k[None], torch.tensor([n]), base)).sum())
    for m, n in ((5, 2), (40, 37), (300, 297)):
        assert score(m, n) == pytest.approx(score(3, 0), rel=1e-6, abs=1e-6)


def _identity_mha_params(dim, H, gate_out_bias, select_bias=None, cross=False):
    """Projection weights that are identities (zero biases) and gate
    projections with zero weight: the composition's attention then acts on
    the inputs themselves, with constant gates sigmoid(bias)."""
    eye = torch.eye(dim, dtype=F64)
    p = {"q_proj.weight": eye.clone(), "k_proj.weight": eye.clone(),
         "v_proj.weight": eye.clone(), "v_proj.bias": torch.zeros(dim, dtype=F64),
         "out_proj.weight": eye.clone(), "out_proj.bias": torch.zeros(dim, dtype=F64)}
    if cross:
        p["select_gate_proj.weight"] = torch.zeros(H, dim, dtype=F64)
        p["select_gate_proj.bias"] = select_bias.clone()
    else:
        p["gate_proj.weight"] = torch.zeros(H + dim, dim, dtype=F64)
        p["gate_proj.bias"] = torch.cat([select_bias, gate_out_bias])
    return p


def test_oracle_selective_train_forward_penalty_zero_is_rope_sdpa():
    """selective_mha_train_forward at penalty 0 with identity projections and
    constant gates: the output is causal SDPA over the RoPE-rotated heads of
    x, times sigmoid(out-gate bias) column by column."""
    b, L, H, hd = 2, 9, 2, 8
    dim = H * hd
    g = torch.Generator().manual_seed(6)
    x = torch.randn(b, L, dim, generator=g, dtype=F64)
    ob = torch.randn(dim, generator=g, dtype=F64)
    p = _identity_mha_params(dim, H, ob, torch.randn(H, generator=g, dtype=F64))
    out, _ = lm_ref.selective_mha_train_forward(p, x, None, hd, 0.0)
    xh = x.view(b, L, H, hd).transpose(1, 2)
    pos = torch.arange(L)
    e = F.scaled_dot_product_attention(lm_ref.rope_rotate(xh, pos), lm_ref.rope_rotate(xh, pos),
                                       xh, is_causal=True)
    exp = e.transpose(1, 2).reshape(b, L, dim) * torch.sigmoid(ob)
    torch.testing.assert_close(out, exp, rtol=1e-10, atol=1e-12)


def test_oracle_cross_train_penalty_zero_is_masked_sdpa():
    """cross_mha_train_forward at penalty 0 with identity projections: SDPA
    of the decoder states over the context, keys past each row's context
    length masked out; the std is the population std of exactly those
    scores (brute force)."""
    b, L, Lc, H, hd = 2, 5, 11, 2, 8
    dim = H * hd
    g = torch.Generator().manual_seed(7)
    x = torch.randn(b, L, dim, generator=g, dtype=F64)
    ctx = torch.randn(b, Lc, dim, generator=g, dtype=F64)
    lens = torch.tensor([11, 4])
    p = _identity_mha_params(dim, H, None, torch.randn(H, generator=g, dtype=F64), cross=True)
    out, std = lm_ref.cross_mha_train_forward(p, x, ctx, lens, hd, 0.0)
    qh = x.view(b, L, H, hd).transpose(1, 2)
    kh = ctx.view(b, Lc, H, hd).transpose(1, 2)
    mask = (torch.arange(Lc)[None, :] < lens[:, None])[:, None, None, :]
    e = F.scaled_dot_product_attention(qh, kh, kh, attn_mask=mask)
    torch.testing.assert_close(out, e.transpose(1, 2).reshape(b, L, dim), rtol=1e-10, atol=1e-12)
    for h in range(H):
        vals = [float(qh[i, h, t] @ kh[i, h, j]) / math.sqrt(hd)
                for i in range(b) for t in range(L) for j in range(int(lens[i]))]
        m = sum(vals) / len(vals)
        sd = math.sqrt(sum((v - m) ** 2 for v in vals) / len(vals))
        assert float(std[h]) == pytest.approx(sd, rel=1e-10)


def test_oracle_cross_train_key0_exemption_brute_force():
    """cross_mha_train_forward with a gate: a loop over (row, head, query)
    adds log(gate_j) * std_h * penalty to every valid key but key 0 and takes
    the softmax over the keys inside the context length.  A gate near 0 on
    key 0 leaves its weight untouched; the same gate on another key mutes it."""
    b, L, Lc, H, hd, pen = 2, 4, 9, 2, 8, 1.3
    dim = H * hd
    g = torch.Generator().manual_seed(8)
    x = torch.randn(b, L, dim, generator=g, dtype=F64)
    ctx = torch.randn(b, Lc, dim, generator=g, dtype=F64)
    lens = torch.tensor([9, 6])
    sb = torch.randn(H, generator=g, dtype=F64)
    p = _identity_mha_params(dim, H, None, sb, cross=True)
    # per-key gates: a non-zero gate weight on one context feature varies them
    p["select_gate_proj.weight"][:, 0] = 2.0
    ctx[:, 0, 0] = -300.0           # key 0: gate ~ e^-600 (exempt anyway)
    ctx[1, 3, 0] = -300.0           # key 3 of row 1: muted
    x[..., 0] = 0.0                 # feature 0 drives the gate only, not q.k
    out, std = lm_ref.cross_mha_train_forward(p, x, ctx, lens, hd, pen)
    gate = torch.sigmoid(ctx[..., 0:1] * 2.0 + sb)          # (b, Lc, H)
    for i in range(b):
        n = int(lens[i])
        for h in range(H):
            kh = ctx[i, :, h * hd:(h + 1) * hd]
            for t in range(L):
                q = x[i, t, h * hd:(h + 1) * hd]
                s = [float(q @ kh[j]) / math.sqrt(hd)
                     + (0.0 if j == 0 else math.log(float(gate[i, j, h])) * float(std[h]) * pen)
                     for j in range(n)]
                mx = max(s)
                w = [math.exp(v - mx) for v in s]
                z = sum(w)
                exp = sum(w[j] / z * kh[j] for j in range(n))
                torch.testing.assert_close(out[i, t, h * hd:(h + 1) * hd], exp, rtol=1e-9, atol=1e-12)
                if i == 1:
                    assert w[3] / z < 1e-100 and w[0] / z > 1e-12


# ---------------------------------------------------------------- GPU parity
STATS_CASES = [
    (torch.bfloat16, 2, 3, 200, 64, True, [200, 77]),
    (torch.bfloat16, 1, 2, 130, 128, False, None),
    (torch.bfloat16, 3, 4, 64, 32, True, [64, 1, 0]),
    (torch.float32, 2, 2, 150, 96, True, [150, 33]),
    (torch.float32, 1, 3, 97, 64, False, [60]),
    (torch.bfloat16, 1, 2, 1024, 128, True, None),
]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,b,H,L,D,causal,lens", STATS_CASES)
def test_score_stats_kernel_parity(dtype, b, H, L, D, causal, lens):
    from selective_attention.kernels.attention import score_stats
    print(f"score stats {dtype} b{b} H{H} L{L} D{D} causal={causal} lens={lens}", flush=True)
    q, k = qk(b, H, L, D, seed=L + D, dtype=dtype)
    lt = None if lens is None else torch.tensor(lens)
    scale = D ** -0.5
    exp = ref.score_stats(q, k, scale, lt, lt, causal)
    ld = None if lt is None else lt.cuda()
    got = score_stats(q.cuda(), k.cuda(), ld, ld, causal).cpu()
    again = score_stats(q.cuda(), k.cuda(), ld, ld, causal).cpu()
    assert torch.equal(got, again), "score_stats must be deterministic"
    assert torch.equal(got[:, 0], exp[:, 0]), "count"
    # fp32 products inside the kernel: relative 1e-5 of the sum of squares
    tol2 = 1e-5 * exp[:, 2].abs() + 1e-9
    assert ((got[:, 2] - exp[:, 2]).abs() <= tol2).all(), (got, exp)
    tol1 = 1e-5 * torch.sqrt(exp[:, 0] * exp[:, 2]) + 1e-9
    assert ((got[:, 1] - exp[:, 1]).abs() <= tol1).all(), (got, exp)


@pytest.mark.gpu
@pytest.mark.parametrize("causal,lens", [(True, [90, 41]), (False, None)])
def test_score_std_gradient_matches_autograd(causal, lens):
    """d std / d q, d k of ScoreStdFn (kernel forward, analytic backward by
    query chunks) against autograd through the fp64 oracle."""
    from selective_attention.ops import ScoreStdFn
    print(f"score std grad causal={causal} lens={lens}", flush=True)
    b, H, L, D = 2, 3, 90, 64
    q, k = qk(b, H, L, D, seed=7, dtype=torch.float32)
    lt = None if lens is None else torch.tensor(lens)
    g = torch.randn(H, generator=torch.Generator().manual_seed(8))
    qd, kd = q.cuda().requires_grad_(True), k.cuda().requires_grad_(True)
    ld = None if lt is None else lt.cuda()
    std = ScoreStdFn.apply(qd, kd, ld, ld, causal, 32)
    std.backward(g.cuda())
    q64, k64 = q.to(F64).requires_grad_(True), k.to(F64).requires_grad_(True)
    std64 = ref.score_std(ref.score_stats(q64, k64, D ** -0.5, lt, lt, causal))
    std64.backward(g.to(F64))
    assert_parity(std.detach().cpu(), std64.detach(), torch.float32, "std")
    assert_parity(qd.grad.cpu(), q64.grad, torch.float32, "dq")
    assert_parity(kd.grad.cpu(), k64.grad, torch.float32, "dk")


TRAIN_CASES = [
    dict(b=2, L=70, dim=96, head_dim=32, causal=True, lens=[70, 45]),
    dict(b=1, L=65, dim=128, head_dim=64, causal=True, lens=None),
    dict(b=2, L=40, dim=64, head_dim=32, causal=False, lens=[40, 23]),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", TRAIN_CASES, ids=lambda c: f"L{c['L']}_d{c['dim']}_causal{c['causal']}")
def test_selective_mha_training_forward_backward(case):
    """SelectiveMHA in training mode (fp32 parameters): outputs, gradients of
    the input and of every parameter, the score std and the running-average
    update, against the fp64 oracle module."""
    from selective_attention.modules.selective_attention import SelectiveMHA
    print(f"SelectiveMHA training {case}", flush=True)
    torch.manual_seed(11)
    b, L, dim, hd = case["b"], case["L"], case["dim"], case["head_dim"]
    m = SelectiveMHA(0, dim, hd, log_gate_penalty=1.5, is_causal=case["causal"])
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(torch.randn_like(p) * 0.2)
        m.gate_proj.bias.add_(1.0)
        m.score_std_ema.fill_(0.7)
    m = m.cuda().train()
    x = torch.randn(b, L, dim, generator=torch.Generator().manual_seed(12))
    w = torch.randn(b, L, dim, generator=torch.Generator().manual_seed(13))
    lt = None if case["lens"] is None else torch.tensor(case["lens"])
    xd = x.cuda().requires_grad_(True)
    out = m(xd, None if lt is None else lt.cuda())
    (out * w.cuda()).sum().backward()

    params = {n: p.detach().cpu().to(F64).requires_grad_(True) for n, p in m.named_parameters()}
    x64 = x.to(F64).requires_grad_(True)
    out64, std64 = lm_ref.selective_mha_train_forward(params, x64, lt, hd, 1.5, case["causal"])
    (out64 * w.to(F64)).sum().backward()

    assert_parity(out.detach().cpu(), out64.detach(), torch.float32, "out")
    assert_parity(xd.grad.cpu(), x64.grad, torch.float32, "dx")
    for n, p in m.named_parameters():
        assert_parity(p.grad.cpu(), params[n].grad, torch.float32, f"d{n}")
    ema = 0.9 * 0.7 + 0.1 * std64.detach()
    assert_parity(m.score_std_ema.cpu(), ema, torch.float32, "score_std_ema")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 64), (torch.float32, 128)])
def test_score_stats_cross_lengths(dtype, D):
    """Cross attention's statistics: every query, keys inside the context
    length (q_len != k_len)."""
    from selective_attention.kernels.attention import score_stats
    print(f"score stats cross {dtype} D{D}", flush=True)
    g = torch.Generator().manual_seed(21)
    q = torch.randn(2, 3, 50, D, generator=g).to(dtype)
    k = torch.randn(2, 3, 130, D, generator=g).to(dtype)
    kl = torch.tensor([130, 77])
    exp = ref.score_stats(q, k, D ** -0.5, None, kl, False)
    got = score_stats(q.cuda(), k.cuda(), None, kl.cuda(), False).cpu()
    assert torch.equal(got[:, 0], exp[:, 0]), "count"
    assert ((got[:, 2] - exp[:, 2]).abs() <= 1e-5 * exp[:, 2].abs() + 1e-9).all(), (got, exp)
    assert ((got[:, 1] - exp[:, 1]).abs() <= 1e-5 * torch.sqrt(exp[:, 0] * exp[:, 2]) + 1e-9).all()


@pytest.mark.gpu
@pytest.mark.parametrize("lens", [[90, 37], None])
def test_cross_mha_training_forward_backward(lens):
    """CrossSelectiveMHA in training mode (fp32 parameters): outputs, the
    gradients of the decoder input, the context and every parameter, and
    the running-average update, against the fp64 oracle module."""
    from selective_attention.modules.cross_selective_attention import CrossSelectiveMHA
    print(f"CrossSelectiveMHA training lens={lens}", flush=True)
    torch.manual_seed(31)
    b, L, Lc, dim, hd = 2, 33, 90, 96, 32
    m = CrossSelectiveMHA(0, dim, hd, log_gate_penalty=1.2)
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(torch.randn_like(p) * 0.2)
        m.select_gate_proj.bias.add_(1.0)
        m.score_std_ema.fill_(0.5)
    m = m.cuda().train()
    gen = torch.Generator().manual_seed(32)
    x, ctx = torch.randn(b, L, dim, generator=gen), torch.randn(b, Lc, dim, generator=gen)
    w = torch.randn(b, L, dim, generator=gen)
    lt = None if lens is None else torch.tensor(lens)
    xd, cd = x.cuda().requires_grad_(True), ctx.cuda().requires_grad_(True)
    out = m(xd, cd, None if lt is None else lt.cuda())
    (out * w.cuda()).sum().backward()

    params = {n: p.detach().cpu().to(F64).requires_grad_(True) for n, p in m.named_parameters()}
    x64, c64 = x.to(F64).requires_grad_(True), ctx.to(F64).requires_grad_(True)
    out64, std64 = lm_ref.cross_mha_train_forward(params, x64, c64, lt, hd, 1.2)
    (out64 * w.to(F64)).sum().backward()

    assert_parity(out.detach().cpu(), out64.detach(), torch.float32, "out")
    assert_parity(xd.grad.cpu(), x64.grad, torch.float32, "dx")
    assert_parity(cd.grad.cpu(), c64.grad, torch.float32, "dcontext")
    for n, p in m.named_parameters():
        assert_parity(p.grad.cpu(), params[n].grad, torch.float32, f"d{n}")
    assert_parity(m.score_std_ema.cpu(), 0.9 * 0.5 + 0.1 * std64.detach(), torch.float32, "ema")
