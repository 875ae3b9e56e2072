"""The config-4 hybrid LM at its own shapes (d_model 1024, six SSD + attention
blocks, d_state 128, 16 heads of 64, vocab 32000, bf16, random init): the
reference's model-level invariants (tests/test_causal_lm.py:55-133 decode
steps reproduce the full forward; :136-192 greedy generation agrees with
teacher forcing) on 4 rows of 4096-token prompts -- 16 chunks of 256 and
64+ pages of 64 keys per row -- and one 512-token row against the fp64
oracle model.

At these shapes every fused decode kernel runs: residual add + RMSNorm
(d_model % 512 == 0), the multi-matrix GEMV, the gated state update, the
paged KV append and the graph-captured step.
"""
import pytest
import torch

from tests.test_causal_lm import assert_argmax_agrees, assert_logits_close

PROMPT = 4096


def _model():
    from selective_attention.models import CausalLM, config4
    torch.manual_seed(0)
    cfg = config4("cuda")
    m = CausalLM(cfg)
    with torch.no_grad():
        for blk in m.layers:
            blk.mha.score_std_ema.fill_(1.0)
    return cfg, m.to_bf16().cuda().eval()


def _thresholds(cfg, value=0.5):
    return torch.full((cfg.num_layers, cfg.model_dim // cfg.head_dim), value, device="cuda")


def _ids(cfg, b, L, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randint(10, cfg.vocab_size, (b, L), device="cuda", generator=g)


def _logits_at(m, ids, lens, thr, pos):
    """Full-forward logits at positions pos (b, k) only (the head over every
    position of 4 x 4136 tokens would be a 1 GB tensor)."""
    h = m._hidden(ids, lens, thr)
    rows = torch.arange(ids.shape[0], device=ids.device)[:, None]
    return m.lm_head(m.norm(h[rows, pos])).float()


@pytest.mark.gpu
def test_config4_steps_reproduce_forward():
    from selective_attention.inference import CausalBlockCache, GenerationConfig, InferenceState
    cfg, m = _model()
    thr = _thresholds(cfg)
    steps = 40
    pre = torch.tensor([PROMPT, PROMPT - 96, PROMPT - 597, PROMPT - 5], device="cuda")
    L = PROMPT + steps
    ids = _ids(cfg, 4, L, seed=1)
    gen = GenerationConfig(bos_token_id=-1, eos_token_id=-1, pad_token_id=0,
                           attn_gate_thresholds=thr)
    print("config4 steps vs forward", flush=True)
    with torch.no_grad():
        lens = pre + steps
        pos = pre[:, None] + torch.arange(steps, device="cuda")[None, :]
        full = _logits_at(m, ids, lens, thr, pos)                      # (4, steps, vocab)
        cache = [CausalBlockCache() for _ in m.layers]
        m(ids, pre, thr, cache)
        state = InferenceState(pre.clone())
        rows = torch.arange(4, device="cuda")
        for i in range(steps):
            tok = ids[rows, state.lengths]
            out = m.step(tok, cache, state, gen).float()
            assert_logits_close(out, full[:, i], f"step {i}")
            assert_argmax_agrees(out.argmax(-1), full[:, i], f"step {i}")
            state.update()


@pytest.mark.gpu
def test_config4_generate_matches_teacher_forcing():
    from selective_attention.inference import GenerationConfig
    cfg, m = _model()
    thr = _thresholds(cfg)
    new = 32
    ids = _ids(cfg, 4, PROMPT, seed=2)
    gen = GenerationConfig(bos_token_id=-1, eos_token_id=-1, pad_token_id=0, max_new_tokens=new,
                           attn_gate_thresholds=thr)
    print("config4 generate vs teacher forcing", flush=True)
    with torch.no_grad():
        seq = m.generate(ids, gen)
        assert seq.shape == (4, PROMPT + new)
        assert torch.equal(seq[:, :PROMPT], ids)
        lens = torch.full((4,), PROMPT + new, device="cuda")
        pos = PROMPT - 1 + torch.arange(new, device="cuda")[None, :].expand(4, -1)
        full = _logits_at(m, seq, lens, thr, pos)
    for i in range(new):
        assert_argmax_agrees(seq[:, PROMPT + i], full[:, i], f"token {i}")


@pytest.mark.gpu
def test_config4_row_against_oracle():
    """One 512-token row (two chunks, eight pages) through the bf16 model on
    the GPU and the fp64 oracle model with the same bf16 storage points."""
    from oracle.lm import LMRef
    cfg, m = _model()
    thr_l = [0.5] * cfg.num_layers
    ids = _ids(cfg, 1, 512, seed=3)
    print("config4 row vs oracle", flush=True)
    ref = LMRef({k: v.cpu() for k, v in m.state_dict().items()}, cfg, bf16=True)
    with torch.no_grad():
        out = m(ids, None, _thresholds(cfg)).float().cpu()
    exp, _ = ref.forward(ids.cpu(), None, thr_l)
    assert_logits_close(out[0], exp[0], "config4 row")
