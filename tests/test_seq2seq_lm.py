"""The seq2seq LM on the gfx950 ops (models/seq2seq_lm.py): oracle pins on the
CPU, logits parity against the fp64 oracle model on the GPU, and the model
invariants (decoder steps reproduce the teacher-forced decoder; greedy
generation agrees with teacher forcing; graph replays equal eager steps).
Tolerances as in test_causal_lm.py."""
import pytest
import torch

from oracle import attn as aref
from oracle.lm import Seq2SeqRef
from selective_attention.inference import CrossBlockCache, GenerationConfig, InferenceState
from selective_attention.models import Seq2SeqLM, Seq2SeqLMConfig
from tests.test_causal_lm import assert_argmax_agrees, assert_logits_close, tokens

F64 = torch.float64


def tiny_cfg(chunk=64, layers=2, device="cuda"):
    return Seq2SeqLMConfig(vocab_size=256, model_dim=128, head_dim=64, ssm_state_dim=64,
                           ssm_num_groups=1, ssm_chunk_size=chunk, num_layers=layers,
                           dropout_rate=0.0, device=device)


def tiny_model(cfg, seed=0):
    torch.manual_seed(seed)
    m = Seq2SeqLM(cfg)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if "norm" in name:
                p.copy_(0.2 * torch.randn_like(p))
        for mod in m.modules():
            if hasattr(mod, "score_std_ema"):
                mod.score_std_ema.copy_(0.5 + torch.rand_like(mod.score_std_ema))
    return m.eval()


THR = dict(enc=[0.85, 0.9], self_=[0.88, 0.88], cross=[0.9, 0.85])


# ------------------------------------------------------------ oracle pins (CPU)
def test_oracle_seq2seq_steps_reproduce_decoder():
    """Decoder prefill of bos and steps over the rest give the teacher-forced
    decoder's logits (cache semantics: cross thresholds applied), fp64."""
    cfg = tiny_cfg(chunk=16, device="cpu")
    ref = Seq2SeqRef(tiny_model(cfg).state_dict(), cfg, bf16=False)
    lens = torch.tensor([30, 19])
    ids = tokens(2, 30, cfg.vocab_size, lens.tolist())
    dec = tokens(2, 12, cfg.vocab_size, [12, 12], seed=3)
    full, _ = ref.forward(ids, lens, dec, THR["enc"], THR["self_"], THR["cross"])
    _, states = ref.forward(ids, lens, dec[:, :1], THR["enc"], THR["self_"], THR["cross"])
    for t in range(1, 12):
        out = ref.step(dec[:, t], states, torch.full((2,), t), THR["self_"])
        torch.testing.assert_close(out, full[:, t], rtol=1e-9, atol=1e-9)


def test_oracle_cross_attention_is_multiplicative_gate():
    """Additive log-gate bias with key 0 exempt == the multiplicative form of
    the reference's _gated_softmax (cross_selective_attention.py:8-32):
    exp(s) * gate for keys >= 1, exp(s) for key 0, normalised."""
    g = torch.Generator().manual_seed(0)
    Lq, Lc, H, D = 5, 9, 2, 8
    q, k, v = (torch.randn(n, H, D, generator=g, dtype=F64) for n in (Lq, Lc, Lc))
    gate = torch.rand(H, Lc, generator=g, dtype=F64)
    gate[:, 3] = 0.0
    o = aref.attn_varlen(q, k, v, torch.tensor([0, Lq]), "cross", torch.tensor([0, Lc]),
                         key_bias=torch.log(gate))
    s = torch.einsum("qhd,khd->hqk", q, k) / D ** 0.5
    e = torch.exp(s - s.max(-1, keepdim=True).values)
    e[:, :, 1:] = e[:, :, 1:] * gate[:, None, 1:]
    w = e / e.sum(-1, keepdim=True)
    torch.testing.assert_close(o, torch.einsum("hqk,khd->qhd", w, v), rtol=1e-12, atol=1e-12)


def test_oracle_bidirectional_matches_dense_branch():
    """The encoder's attention (every key, own key unbiased) == the
    reference's uncompressed inference branch with is_causal=False: full
    score matrix, gate on every column, diagonal restored
    (selective_attention.py:55-62, :134-139)."""
    g = torch.Generator().manual_seed(1)
    L, H, D = 11, 2, 8
    q, k, v = (torch.randn(L, H, D, generator=g, dtype=F64) for _ in range(3))
    lg = torch.log(torch.rand(H, L, generator=g, dtype=F64))
    lg[:, 4] = float("-inf")
    o = aref.attn_varlen(q, k, v, torch.tensor([0, L]), "full", key_bias=lg)
    S = torch.einsum("qhd,khd->hqk", q, k) / D ** 0.5
    d = torch.arange(L)
    diag = S[:, d, d].clone()
    S = S + lg[:, None, :]
    S[:, d, d] = diag
    torch.testing.assert_close(o, torch.einsum("hqk,khd->qhd", torch.softmax(S, -1), v),
                               rtol=1e-12, atol=1e-12)


def test_seq2seq_interfaces_cpu():
    cfg = tiny_cfg(device="cpu")
    m = Seq2SeqLM(cfg)
    assert m.lm_head.weight is m.embedding.weight
    assert tuple(m.norm3.weight.shape) == (2 * cfg.model_dim // cfg.head_dim, cfg.ssm_state_dim)
    # training runs the score statistics kernel: no CPU path, a loud error
    with pytest.raises(ValueError, match="device tensors"):
        m.decoder_layers[0].cross_mha.train()(torch.zeros(1, 2, cfg.model_dim),
                                              torch.zeros(1, 3, cfg.model_dim))


# ------------------------------------------------------------------ GPU
def _gpu_pair(seed):
    cfg = tiny_cfg()
    m = tiny_model(cfg, seed)
    ref = Seq2SeqRef(m.to_bf16().state_dict(), cfg, bf16=True)
    return cfg, m.cuda(), ref


@pytest.mark.gpu
def test_seq2seq_prefill_parity():
    cfg, m, ref = _gpu_pair(0)
    lens = torch.tensor([150, 97])
    ids = tokens(2, 150, cfg.vocab_size, lens.tolist())
    dec = tokens(2, 20, cfg.vocab_size, [20, 20], seed=2)
    print("seq2seq prefill", flush=True)
    cache = [CrossBlockCache() for _ in range(cfg.num_layers)]
    with torch.no_grad():
        out = m(ids.cuda(), lens.cuda(), dec.cuda(), THR["enc"], THR["self_"], THR["cross"],
                cache).float().cpu()
    exp, _ = ref.forward(ids, lens, dec, THR["enc"], THR["self_"], THR["cross"])
    assert_logits_close(out, exp, "seq2seq prefill")


@pytest.mark.gpu
def test_seq2seq_decode_parity():
    cfg, m, ref = _gpu_pair(1)
    lens = torch.tensor([120, 64])
    ids = tokens(2, 120, cfg.vocab_size, lens.tolist(), seed=4)
    dec = tokens(2, 30, cfg.vocab_size, [30, 30], seed=5)
    gen = GenerationConfig(bos_token_id=-1, eos_token_id=-1, pad_token_id=0,
                           attn_gate_thresholds=THR["self_"])
    cache = [CrossBlockCache() for _ in range(cfg.num_layers)]
    print("seq2seq decode", flush=True)
    with torch.no_grad():
        m(ids.cuda(), lens.cuda(), dec[:, :1].cuda(), THR["enc"], THR["self_"], THR["cross"], cache)
        _, states = ref.forward(ids, lens, dec[:, :1], THR["enc"], THR["self_"], THR["cross"])
        state = InferenceState(torch.ones(2, dtype=torch.long, device="cuda"))
        for t in range(1, 30):
            out = m.step(dec[:, t].cuda(), cache, state, gen).float().cpu()
            exp = ref.step(dec[:, t], states, torch.full((2,), t), THR["self_"])
            assert_logits_close(out, exp, f"seq2seq step {t}")
            state.update()


@pytest.mark.gpu
def test_seq2seq_generate_graph_and_teacher_forcing():
    """generate with the graph == without it; each greedy token is the
    teacher-forced decoder's argmax (cache semantics) up to near-ties."""
    cfg = tiny_cfg()
    m = tiny_model(cfg, seed=6).to_bf16().cuda()
    lens = torch.tensor([90, 40, 64])
    ids = tokens(3, 90, cfg.vocab_size, lens.tolist(), seed=7).cuda()
    new = 40
    gen = GenerationConfig(bos_token_id=1, eos_token_id=-1, pad_token_id=0, max_new_tokens=new,
                           enc_attn_gate_thresholds=THR["enc"], attn_gate_thresholds=THR["self_"],
                           cross_attn_gate_thresholds=THR["cross"])
    print("seq2seq generate", flush=True)
    with torch.no_grad():
        seq_g = m.generate(ids, gen, use_graph=True)
        seq_e = m.generate(ids, gen, use_graph=False)
        assert torch.equal(seq_g, seq_e)
        cache = [CrossBlockCache() for _ in range(cfg.num_layers)]
        full = m(ids, lens.cuda(), seq_g, THR["enc"], THR["self_"], THR["cross"], cache).float()
    for t in range(1, new):
        assert_argmax_agrees(seq_g[:, t], full[:, t - 1], f"token {t}")
