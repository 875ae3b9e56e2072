"""The causal LM on the gfx950 ops (models/causal_lm.py): oracle pins on the CPU,
logits parity against the fp64 oracle model on the GPU, and the reference's
own model-level invariants (tests/test_causal_lm.py: decode steps reproduce
the full forward's logits; greedy generation agrees with teacher forcing).

Model-level tolerance (bf16 model against the oracle with the same bf16
storage points): logits within 3e-2 * max|logit| elementwise and 5e-3 *
max|logit| on average.  Argmax comparisons allow near-ties: the chosen token's
logit must be within 2e-2 * max|logit| of the row's maximum.
"""
import pytest
import torch

from oracle.lm import LMRef
from selective_attention.inference import CausalBlockCache, GenerationConfig, InferenceState
from selective_attention.models import CausalLM, CausalLMConfig

F64 = torch.float64
MAX_TOL, MEAN_TOL, TIE_TOL = 3e-2, 5e-3, 2e-2


def tiny_cfg(chunk=64, layers=2, device="cuda"):
    return CausalLMConfig(vocab_size=256, model_dim=128, head_dim=64, ssm_state_dim=64,
                          ssm_num_groups=1, ssm_chunk_size=chunk, num_layers=layers,
                          dropout_rate=0.0, device=device)


def tiny_model(cfg, seed=0):
    torch.manual_seed(seed)
    m = CausalLM(cfg)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if "norm" in name:
                p.copy_(0.2 * torch.randn_like(p))
        for blk in m.layers:
            blk.mha.score_std_ema.copy_(0.5 + torch.rand_like(blk.mha.score_std_ema))
            blk.ssm.conv.weight.mul_(2.0)
    return m.eval()


def tokens(b, L, vocab, lengths, seed=1):
    g = torch.Generator().manual_seed(seed)
    x = torch.zeros(b, L, dtype=torch.long)
    for r, n in enumerate(lengths):
        x[r, :n] = torch.randint(10, vocab, (n,), generator=g)
    return x


def assert_logits_close(a, e, name):
    a = a.detach().to("cpu", F64)
    e = e.detach().to("cpu", F64)
    scale = e.abs().max().item()
    err = (a - e).abs()
    assert torch.isfinite(a).all(), f"{name}: non-finite logits"
    assert err.max().item() <= MAX_TOL * scale, f"{name}: max err {err.max().item():.4g}, scale {scale:.4g}"
    assert err.mean().item() <= MEAN_TOL * scale, f"{name}: mean err {err.mean().item():.4g}, scale {scale:.4g}"


def assert_argmax_agrees(chosen, logits, name):
    """chosen (n,) token ids; logits (n, vocab): each chosen token is the
    row's argmax up to a near-tie."""
    lg = logits.detach().to("cpu", F64)
    top = lg.max(-1).values
    got = lg.gather(-1, chosen.to("cpu").view(-1, 1)).squeeze(-1)
    gap = (top - got) / lg.abs().max()
    assert (gap <= TIE_TOL).all(), f"{name}: tokens off the argmax by {gap.max().item():.3g} of scale"


# ------------------------------------------------------------ oracle pins (CPU)
@pytest.mark.parametrize("thr", [None, 0.88])
def test_oracle_lm_steps_reproduce_forward(thr):
    """The reference's test_forward_step invariant on the fp64 oracle: prefill
    of the first n tokens, then decode steps over the rest, give the full
    forward's logits at every position (ragged rows, chunk 16, a threshold
    that drops keys in some heads)."""
    cfg = tiny_cfg(chunk=16, device="cpu")
    m = tiny_model(cfg)
    ref = LMRef(m.state_dict(), cfg, bf16=False)
    lens = torch.tensor([40, 29])
    ids = tokens(2, 40, cfg.vocab_size, lens.tolist())
    thr_l = None if thr is None else [thr] * cfg.num_layers
    full, _ = ref.forward(ids, lens, thr_l)
    pre = torch.tensor([17, 9])
    _, states = ref.forward(ids, pre, thr_l)
    pos = pre.clone()
    for _ in range(20):
        tok = ids[torch.arange(2), pos]
        out = ref.step(tok, states, pos, thr_l)
        exp = full[torch.arange(2), pos]
        torch.testing.assert_close(out, exp, rtol=1e-9, atol=1e-9)
        pos += 1


def test_oracle_lm_all_keys_dropped():
    """A threshold above every gate drops every key: attention returns each
    query's own value (the reference's early exit), in prefill and decode."""
    cfg = tiny_cfg(chunk=16, layers=1, device="cpu")
    m = tiny_model(cfg)
    ref = LMRef(m.state_dict(), cfg, bf16=False)
    ids = tokens(1, 12, cfg.vocab_size, [12])
    full, _ = ref.forward(ids, None, [1.1])
    _, states = ref.forward(ids[:, :5], None, [1.1])
    out = ref.step(ids[:, 5], states, torch.tensor([5]), [1.1])
    torch.testing.assert_close(out, full[:, 5], rtol=1e-9, atol=1e-9)


def test_causal_lm_interfaces_cpu():
    cfg = tiny_cfg(device="cpu")
    m = CausalLM(cfg)
    assert m.lm_head.weight is m.embedding.weight
    assert len(m.layers) == cfg.num_layers
    # training runs the score statistics kernel: no CPU path, a loud error
    with pytest.raises(ValueError, match="device tensors"):
        m.layers[0].mha.train()(torch.zeros(1, 4, cfg.model_dim))
    from selective_attention.models import config4
    c4 = config4(device="cpu")
    assert (c4.model_dim, c4.head_dim, c4.ssm_state_dim, c4.vocab_size, c4.num_layers) == \
        (1024, 64, 128, 32000, 6)


# ------------------------------------------------------------------ GPU
@pytest.mark.gpu
@pytest.mark.parametrize("thr", [None, 0.88])
def test_causal_lm_prefill_parity(thr):
    cfg = tiny_cfg()
    m = tiny_model(cfg)
    ref = LMRef(m.to_bf16().state_dict(), cfg, bf16=True)
    m = m.cuda()
    lens = torch.tensor([150, 97])
    ids = tokens(2, 150, cfg.vocab_size, lens.tolist())
    thr_l = None if thr is None else [thr] * cfg.num_layers
    print(f"causal_lm prefill thr={thr}", flush=True)
    with torch.no_grad():
        out = m(ids.cuda(), lens.cuda(), thr_l).float().cpu()
    exp, _ = ref.forward(ids, lens, thr_l)
    for r, n in enumerate(lens.tolist()):
        assert_logits_close(out[r, :n], exp[r, :n], f"prefill row {r}")


@pytest.mark.gpu
def test_causal_lm_decode_parity():
    """Prefill of the first tokens, then 40 decode steps (crossing a 64-token
    page), against the oracle model's steps."""
    cfg = tiny_cfg()
    m = tiny_model(cfg, seed=2)
    ref = LMRef(m.to_bf16().state_dict(), cfg, bf16=True)
    m = m.cuda()
    thr_l = [0.88] * cfg.num_layers
    pre = torch.tensor([50, 31])
    ids = tokens(2, 100, cfg.vocab_size, [100, 100], seed=3)
    gen = GenerationConfig(bos_token_id=-1, eos_token_id=-1, pad_token_id=0,
                           attn_gate_thresholds=thr_l, cache_update_interval=16)
    cache = [CausalBlockCache() for _ in range(cfg.num_layers)]
    print("causal_lm decode", flush=True)
    with torch.no_grad():
        m(ids.cuda(), pre.cuda(), thr_l, cache)
        _, states = ref.forward(ids, pre, thr_l)
        state = InferenceState(pre.clone().cuda())
        pos = pre.clone()
        for i in range(40):
            tok = ids[torch.arange(2), pos]
            out = m.step(tok.cuda(), cache, state, gen).float().cpu()
            exp = ref.step(tok, states, pos, thr_l)
            assert_logits_close(out, exp, f"decode step {i}")
            state.update()
            pos += 1


@pytest.mark.gpu
@pytest.mark.parametrize("batch", [4, 10])
def test_causal_lm_steps_reproduce_forward(batch):
    """The reference's test_forward_step on this model: full forward logits
    against prefill + decode steps, both on the GPU.  Batch 10 runs the
    decode step's projections as GEMMs (more than 8 rows) with split views
    into the gated state update."""
    cfg = tiny_cfg()
    m = tiny_model(cfg, seed=4).to_bf16().cuda()
    thr_l = [0.88] * cfg.num_layers
    lens = torch.tensor([200, 150, 120, 90, 200, 111, 160, 95, 180, 130][:batch])
    ids = tokens(batch, 200, cfg.vocab_size, lens.tolist(), seed=5).cuda()
    gen = GenerationConfig(bos_token_id=-1, eos_token_id=-1, pad_token_id=0,
                           attn_gate_thresholds=thr_l)
    print(f"causal_lm steps vs forward batch={batch}", flush=True)
    with torch.no_grad():
        full = m(ids, lens.cuda(), thr_l).float()
        cache = [CausalBlockCache() for _ in range(cfg.num_layers)]
        pre = torch.tensor([32, 64, 70, 48, 40, 33, 90, 50, 66, 45][:batch], device="cuda")
        m(ids, pre, thr_l, cache)
        state = InferenceState(pre.clone())
        for i in range(40 if batch <= 8 else 20):
            tok = ids[torch.arange(batch, device="cuda"), state.lengths]
            out = m.step(tok, cache, state, gen).float()
            exp = full[torch.arange(batch, device="cuda"), state.lengths]
            assert_logits_close(out, exp, f"step {i}")
            assert_argmax_agrees(out.argmax(-1), exp, f"step {i}")
            state.update()


@pytest.mark.gpu
def test_causal_lm_generate_matches_teacher_forcing():
    """The reference's test_generate_forward on this model: each greedy token
    is the full forward's argmax at the previous position (up to near-ties)."""
    cfg = tiny_cfg()
    m = tiny_model(cfg, seed=6).to_bf16().cuda()
    thr_l = [0.88] * cfg.num_layers
    lens = torch.tensor([48, 96, 70, 33])
    L, new = 96, 48
    ids = tokens(4, L, cfg.vocab_size, lens.tolist(), seed=7).cuda()
    gen = GenerationConfig(bos_token_id=-1, eos_token_id=-1, pad_token_id=0, max_new_tokens=new,
                           attn_gate_thresholds=thr_l)
    print("causal_lm generate", flush=True)
    with torch.no_grad():
        seq = m.generate(ids, gen)
        clean = torch.zeros(4, L + new, dtype=torch.long, device="cuda")
        for r, n in enumerate(lens.tolist()):
            clean[r, :n] = ids[r, :n]
            clean[r, n:n + new] = seq[r, L:L + new]
        full = m(clean, lens.cuda() + new, thr_l).float()
    for i in range(new):
        p = lens + i
        chosen = clean[torch.arange(4), p.cuda()]
        assert_argmax_agrees(chosen, full[torch.arange(4), (p - 1).cuda()], f"token {i}")


@pytest.mark.gpu
def test_causal_lm_graph_replays_match_eager():
    """Decode steps replayed from one captured graph give, replay after replay,
    the logits of the same steps run eagerly (with unrelated eager work and a
    synchronisation between replays); generate with and without the graph
    returns the same tokens."""
    cfg = tiny_cfg()
    m = tiny_model(cfg, seed=8).to_bf16().cuda()
    thr_l = [0.88] * cfg.num_layers
    lens = torch.tensor([70, 41, 64], device="cuda")
    ids = tokens(3, 70, cfg.vocab_size, lens.tolist(), seed=9).cuda()
    gen = GenerationConfig(bos_token_id=-1, eos_token_id=-1, pad_token_id=0, max_new_tokens=40,
                           attn_gate_thresholds=thr_l)
    H, D = cfg.model_dim // cfg.head_dim, cfg.head_dim
    steps = 12
    print("causal_lm graph replays", flush=True)

    def prefill():
        cache = [CausalBlockCache(reserve=steps) for _ in range(cfg.num_layers)]
        h = m._hidden(ids, lens, thr_l, cache)
        lg = m.lm_head(m.norm(h[torch.arange(3, device="cuda"), lens - 1]))
        for c in cache:
            c.attn_cache.prepare_decode(steps, torch.empty(3, H, D, device="cuda"))
        return cache, InferenceState(lens.clone()), torch.argmax(lg, -1)

    with torch.no_grad():
        cache_a, st_a, tok_a = prefill()
        eager = []
        for _ in range(steps):
            lg = m.step(tok_a, cache_a, st_a, gen)
            eager.append(lg.float().cpu())
            tok_a = torch.argmax(lg, -1)
            st_a.lengths += 1

        cache_b, st_b, tok_b = prefill()
        out = torch.empty(3, cfg.vocab_size, dtype=torch.bfloat16, device="cuda")

        def body():
            lg = m.step(tok_b, cache_b, st_b, gen)
            out.copy_(lg)
            tok_b.copy_(torch.argmax(lg, -1))
            st_b.lengths.add_(1)

        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            body()
        torch.cuda.current_stream().wait_stream(side)
        torch.testing.assert_close(out.float().cpu(), eager[0], rtol=0, atol=0)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            body()
        for i in range(1, steps):
            graph.replay()
            torch.cuda.synchronize()
            torch.testing.assert_close(out.float().cpu(), eager[i], rtol=0, atol=0,
                                       msg=lambda s: f"replay {i}: {s}")
            torch.randn(1000, device="cuda").sum().item()     # unrelated eager work
        seq_g = m.generate(ids, gen, use_graph=True)
        seq_e = m.generate(ids, gen, use_graph=False)
    assert torch.equal(seq_g, seq_e)
