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
