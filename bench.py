#!/usr/bin/env python3
"""Benchmark of the selective-attention kernel layer on one MI355X.

Headline (BASELINE.json metric, configs[1]): SSD chunked scan forward +
backward, b8 L4096 H32 P64 N128 G8 chunk 256, bf16 activations, fp32 state.
One step = SSDScanFn forward + backward (torch.autograd.grad for u, A, B, C,
delta_raw) over one batch of synthetic inputs already resident in HBM.
value = tokens/s over the whole job (one GPU).

Extra fields on the same JSON line:
  roofline      op-level HBM roofline of the fwd+bwd step (algorithmic bytes
                at the dtypes passed / step time), plus live per-kernel
                durations (HIP events on the launch stream) and the dominant
                kernel; `traffic` comes from the committed rocprofv3 PMC
                summary when present.
  cpu_baseline  the fp32 CPU restatement (oracle/) on this host's cores:
                `value` is the config 1 fwd+bwd on one batch row (tokens/s);
                `legs` adds the whole config 0 forward and the config 3
                decode step (8 of 64 attention rows, scaled, + the state
                update); `host` records the CPU count, threads and model.
  decode        config 3 decode step (paged GQA attention + state update),
                us/step, against the HBM roofline.
  sparse_attn   config 2 block-sparse varlen attention, against bf16 MFMA.
  ssm_io        the SSM block's conv prologue and gate epilogue at config 1's
                model shapes, and the scan with the epilogue fused.
  selective_mha SelectiveMHA's prefill and paged decode at config 4's
                attention shapes.
  causal_lm     config 4: the hybrid LM's batch-4 prefill of 8192 tokens and
                256 greedy decode steps (decode step replayed from a graph).
  seq2seq       the seq2seq LM at config 4's dimensions (synthetic workload).

Timings are medians over the timed calls (each call between its own pair of
HIP events on the launch stream); ms_per_step_mean is the bracketed total / K.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu-baseline]
                       [--ssd-only] [--legs decode,sparse,...] [--copy-probe-mib M]
       python bench.py --pmc-summary run_counter_collection.csv [more.csv ...]
                       [--pmc-kernels name,name]
The second form reads rocprofv3 --pmc CSV files (no GPU) and prints, per
kernel, each counter's mean per dispatch as a markdown table.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.join(ROOT, "selective-attention_amd")
for _p in (ROOT, PKG_ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_DENSE_TFLOPS = 2500.0     # MI355X dense bf16 MFMA


def ssd_alg_bytes(b, L, H, P, G, N, act_bytes=2, y_bytes=4, dy_bytes=4):
    """Each input read once and each output written once, forward + backward."""
    u = b * L * H * P * act_bytes
    bc = b * L * G * N * act_bytes
    dr = b * L * H * act_bytes
    y = b * L * H * P * y_bytes
    h_last = b * H * P * N * 4
    dy = b * L * H * P * dy_bytes
    fwd = u + 2 * bc + dr + y + h_last
    bwd = (u + 2 * bc + dr + dy) + (u + 2 * bc + dr)
    return fwd + bwd


def ssd_alg_flops(b, L, H, P, G, N, Lc):
    """MFMA contractions counted causally: fwd per (b,c,h) 2LcPN + 2LcPN + Lc^2 P,
    per (b,c,g) Lc^2 N; backward = 2x forward."""
    nc = math.ceil(L / Lc)
    fwd = b * nc * (H * (4 * Lc * P * N + Lc * Lc * P) + G * Lc * Lc * N)
    return 3 * fwd


def _ssd_step_leg(args, torch, cfg, workload, traffic_file=None):
    """SSDScanFn forward + backward (autograd.grad for u, A, B, C, delta_raw)
    at the shapes of cfg, bf16 activations, fp32 state, fp32 y and dy; times
    the step and every kernel (HIP events on the launch stream)."""
    from selective_attention import workloads
    from selective_attention.ops import SSDScanFn
    from selective_attention.profiling import kernel_timer

    dev = torch.device("cuda:0")
    x = workloads.ssd_inputs(**cfg, device=dev, with_dy=True)
    b, L, H, P = x["u"].shape
    G, N = x["B"].shape[2], x["B"].shape[3]
    Lc = cfg["chunk"]
    leaves = [x[k].requires_grad_(True) for k in ("u", "A", "B", "C", "delta_raw")]
    dy = x["dy"]
    inf = float("inf")

    def step():
        y, h = SSDScanFn.apply(x["u"], x["A"], x["B"], x["C"], x["delta_raw"], None, None, None,
                               Lc, True, (0.0, inf), True)
        return torch.autograd.grad((y,), leaves, (dy,))

    ms, ms_mean = _time_steps(torch, step, args.steps, args.warmup)

    # profiled pass: same steps, per-kernel HIP events on the launch stream
    with kernel_timer() as kt:
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
    kernels = {}
    for name, st in sorted(kt.stats.items(), key=lambda kv: -kv[1]["total_ms"]):
        kernels[name] = {"avg_us": round(st["avg_us"], 2),
                         "per_step_us": round(1000.0 * st["total_ms"] / args.steps, 2),
                         "launches_per_step": st["count"] // args.steps}
    dominant = next(iter(kernels)) if kernels else None
    kernel_sum_us = sum(v["per_step_us"] for v in kernels.values())

    alg = ssd_alg_bytes(b, L, H, P, G, N)
    flops = ssd_alg_flops(b, L, H, P, G, N, Lc)
    achieved = alg / (ms / 1e3) / 1e9
    traffic = None
    if traffic_file:
        tpath = os.path.join(ROOT, "profiles", traffic_file)
        if os.path.exists(tpath):
            with open(tpath) as f:
                traffic = json.load(f).get("hbm_bytes_per_step")
    roofline = {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "scope": "SSD scan fwd+bwd step (all kernels of one op call)",
        "algorithmic_bytes": alg,
        "mfma_tflops": round(flops / (ms / 1e3) / 1e12, 1),
        "mfma_frac": round(flops / (ms / 1e3) / 1e12 / BF16_DENSE_TFLOPS, 4),
        "dominant_kernel": dominant,
        "kernel_sum_us": round(kernel_sum_us, 1),
        "kernels": kernels,
    }
    return dict(ms=ms, ms_mean=ms_mean, tokens=b * L, roofline=roofline,
                config={"workload": workload, "batch": b, "seq_len": L,
                        "nheads": H, "headdim": P, "dstate": N, "ngroups": G, "chunk": Lc,
                        "activations": "bf16", "state": "fp32", "y_dtype": "fp32"})


def run_ssd(args, torch):
    from selective_attention import workloads
    return _ssd_step_leg(args, torch, dict(workloads.SSD_CONFIGS[1]), "ssd_scan_fwd_bwd_config1",
                         "ssd_fwd_bwd_config1_traffic.json")


# SSD fwd+bwd at the SSM shapes of the models: config 4's hybrid LM (d_model
# 1024, expand 2, head_dim 64, state 128, one group) and the reference's
# default CausalLMConfig (models/causal_lm.py:11-22: d_model 512, state 64,
# one group; SSM expand 2, head_dim 64)
SSD_MODEL_SHAPES = {
    "config4_ssm": dict(batch=4, seqlen=8192, nheads=32, headdim=64, dstate=128, ngroups=1,
                        chunk=256, dtype=None),
    "reference_default_ssm": dict(batch=8, seqlen=4096, nheads=16, headdim=64, dstate=64,
                                  ngroups=1, chunk=256, dtype=None),
}


def run_ssd_shapes(args, torch):
    """The headline step at the models' own SSM shapes (see SSD_MODEL_SHAPES)."""
    out = {}
    for name, cfg in SSD_MODEL_SHAPES.items():
        cfg = dict(cfg, dtype=torch.bfloat16)
        r = _ssd_step_leg(args, torch, cfg, f"ssd_scan_fwd_bwd_{name}")
        rf = r["roofline"]
        out[name] = {"ms_per_step": round(r["ms"], 3),
                     "tokens_per_s": round(r["tokens"] / (r["ms"] / 1e3), 1),
                     "hbm_frac": rf["frac"], "achieved_gbs": rf["achieved"],
                     "algorithmic_bytes": rf["algorithmic_bytes"], "mfma_frac": rf["mfma_frac"],
                     "kernels_per_step_us": {k: v["per_step_us"] for k, v in rf["kernels"].items()},
                     "config": r["config"]}
    return out


def _time_steps(torch, fn, steps, warmup):
    """`warmup` untimed calls, then exactly `steps` timed calls bracketed by
    synchronisations, each between its own pair of events on the launch
    stream.  Returns (median ms per call, mean ms per call)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record(stream)
    for i in range(steps):
        fn()
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    per = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(steps))
    mid = len(per) // 2
    median = per[mid] if len(per) % 2 else 0.5 * (per[mid - 1] + per[mid])
    return median, ev[0].elapsed_time(ev[steps]) / steps


def _time_events(torch, fn, steps, warmup):
    """Median ms per call (see _time_steps)."""
    return _time_steps(torch, fn, steps, warmup)[0]


def run_decode(args, torch):
    """Config 3 decode step: paged GQA attention (b64, 32q/8kv, D128, 64-token
    pages, len U[1024,32768]) + selective state update (H32 P64 N128 G8)."""
    from selective_attention import workloads
    from selective_attention.ops import SSUFn, paged_decode_attn
    from selective_attention.profiling import kernel_timer

    dev = torch.device("cuda:0")
    d = workloads.decode_inputs(device=dev)
    x = workloads.ssu_inputs(device=dev)
    h = x["h"]

    def attn():
        return paged_decode_attn(d.q, d.k_pages, d.v_pages, d.page_table, d.seq_lens)

    def ssu():
        return SSUFn.forward(x["u"], x["A"], x["B"], x["C"], x["delta_raw"], None, h)

    def step():
        attn()
        ssu()

    steps = max(args.steps, 10)
    ms_step = _time_events(torch, step, steps, args.warmup)
    ms_attn = _time_events(torch, attn, steps, 2)
    ms_ssu = _time_events(torch, ssu, steps, 2)
    with kernel_timer() as kt:
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
    kernels = {k: round(v["avg_us"], 2) for k, v in kt.stats.items()}

    lens = d.seq_lens.to("cpu", torch.int64)
    b, Hq, D = d.q.shape
    Hkv, ps = d.k_pages.shape[1], d.k_pages.shape[2]
    npg = (lens + ps - 1) // ps
    kv_bytes = int(lens.sum()) * Hkv * D * 2 * 2
    attn_bytes = kv_bytes + 2 * b * Hq * D * 2 + int(npg.sum()) * 4
    Hs, P, N = x["h"].shape[1], x["h"].shape[2], x["h"].shape[3]
    G = x["B"].shape[1]
    ssu_bytes = 2 * b * Hs * P * N * 4 + b * Hs * P * 2 * 2 + 2 * b * G * N * 2 + b * Hs * 2
    total = attn_bytes + ssu_bytes
    gbs = total / (ms_step / 1e3) / 1e9
    return {
        "us_per_step": round(ms_step * 1e3, 1),
        "attn_us": round(ms_attn * 1e3, 1),
        "ssu_us": round(ms_ssu * 1e3, 1),
        "config": {"workload": "decode_config3", "batch": b, "q_heads": Hq, "kv_heads": Hkv,
                   "headdim": D, "page_size": ps, "kv_tokens": int(lens.sum()),
                   "ssu": f"H{Hs} P{P} N{N} G{G} fp32 state"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": total,
                     "attn_frac": round(attn_bytes / (ms_attn / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
                     "ssu_frac": round(ssu_bytes / (ms_ssu / 1e3) / 1e9 / HBM_PEAK_GBS, 4)},
        "kernels_avg_us": kernels,
    }


def sparse_pairs(lens, block_idx, bs=64):
    """Admissible (query, key) pairs of the block-sparse causal pattern."""
    import math
    idx = block_idx.to("cpu")
    H = idx.shape[0]
    total = 0
    qb = 0
    for n in lens:
        nb = math.ceil(n / bs)
        for j in range(nb):
            nq = min(bs, n - j * bs)
            sel = idx[:, qb, :]
            for h in range(H):
                for kb in sel[h].tolist():
                    if kb < 0 or kb > j:
                        continue
                    if kb < j:
                        total += nq * bs
                    else:
                        total += nq * (nq + 1) // 2
            qb += 1
    return total


def run_sparse(args, torch):
    """Config 2: varlen block-sparse causal attention, T=65536, H16, D128."""
    from selective_attention import workloads
    from selective_attention.ops import sparse_attn_varlen

    dev = torch.device("cuda:0")
    w = workloads.sparse_attn_inputs(device=dev)

    def fn():
        return sparse_attn_varlen(w.q, w.k, w.v, w.cu_seqlens, w.block_idx)

    ms = _time_events(torch, fn, max(args.steps, 10), args.warmup)
    T, H, D = w.q.shape
    pairs = sparse_pairs(w.lens, w.block_idx)
    flops = 4 * D * pairs
    tf = flops / (ms / 1e3) / 1e12
    return {"us": round(ms * 1e3, 1), "tokens_per_s": round(T / (ms / 1e3), 1),
            "config": {"workload": "sparse_attn_config2", "tokens": T, "heads": H, "headdim": D,
                       "sequences": len(w.lens), "block": 64, "max_blocks": w.block_idx.shape[2]},
            "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": BF16_DENSE_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tf / BF16_DENSE_TFLOPS, 4),
                         "algorithmic_flops": flops, "qk_pairs": pairs}}


def run_selective_mha(args, torch):
    """SelectiveMHA's attention at config 4's shapes (16 heads x 64, batch 4,
    8192-token prefill): the gated causal prefill on the block-sparse kernel
    (every causal block selected, log-gate as key bias, ~20 % of keys
    dropped), then one decode step over the prefill's paged cache (append the
    new token, attend, and take it out again so every step sees the same
    length).  Kernel times come from HIP events on the launch stream."""
    from selective_attention.ops.selective_mha import PagedSelectiveAttnCache, selective_mha_prefill
    from selective_attention.profiling import kernel_timer

    dev = torch.device("cuda:0")
    b, H, L, D = 4, 16, 8192, 64
    g = torch.Generator(device=dev).manual_seed(4)
    rnd = lambda *shape: torch.randn(*shape, device=dev, generator=g)
    q, k, v = (rnd(b, H, L, D).to(torch.bfloat16) for _ in range(3))
    gate = torch.sigmoid(rnd(b, H, L) + 1.0)
    lg = torch.log(torch.where(gate < 0.6, torch.zeros_like(gate), gate))

    def prefill():
        return selective_mha_prefill(q, k, v, lg)

    steps = max(args.steps // 2, 5)
    ms_pre = _time_events(torch, prefill, steps, max(args.warmup, 1))
    with kernel_timer() as kt:
        for _ in range(steps):
            prefill()
        torch.cuda.synchronize()
    pre_kernels = {n: round(x["avg_us"], 2) for n, x in kt.stats.items()}
    pairs = b * H * L * (L + 1) // 2
    flops = 4 * D * pairs
    sp_us = pre_kernels.get("sparse_attn_fwd", ms_pre * 1e3)
    tf = flops / (sp_us / 1e6) / 1e12

    cache = PagedSelectiveAttnCache(b, H, D, max_tokens=L + 64, device=dev)
    cache.build(k, v, lg)
    qt, kt_, vt = (rnd(b, H, D).to(torch.bfloat16) for _ in range(3))
    lgt = torch.log(torch.sigmoid(rnd(b, H) + 1.0))

    def step():
        cache.append(kt_, vt, lgt)
        o = cache.attend(qt)
        cache.unappend()
        return o

    cache.append(kt_, vt, lgt)

    def attend():
        return cache.attend(qt)

    dsteps = max(args.steps, 20)
    ms_att = _time_events(torch, attend, dsteps, args.warmup)
    with kernel_timer() as kt:
        for _ in range(dsteps):
            attend()
        torch.cuda.synchronize()
    dec_kernels = {n: round(x["avg_us"], 2) for n, x in kt.stats.items()}
    cache.unappend()
    ms_step = _time_events(torch, step, dsteps, args.warmup)
    n = L + 1
    dec_bytes = b * H * n * (2 * D * 2 + 4) + 2 * b * H * D * 2 + b * ((n + 63) // 64) * 4
    gbs = dec_bytes / (ms_att / 1e3) / 1e9
    return {
        "prefill_us": round(ms_pre * 1e3, 1),
        "prefill_tokens_per_s": round(b * L / (ms_pre / 1e3), 1),
        "prefill_kernels_avg_us": pre_kernels,
        "decode_attend_us": round(ms_att * 1e3, 1),
        "decode_step_us": round(ms_step * 1e3, 1),
        "decode_kernels_avg_us": dec_kernels,
        "config": {"workload": "selective_mha_config4", "batch": b, "heads": H, "headdim": D,
                   "prefill_len": L, "gate_threshold": 0.6, "page_size": 64},
        "roofline": {
            "prefill": {"bound": "mfma", "achieved": round(tf, 1), "peak": BF16_DENSE_TFLOPS,
                        "unit": "TFLOP/s", "frac": round(tf / BF16_DENSE_TFLOPS, 4),
                        "algorithmic_flops": flops, "qk_pairs": pairs},
            "decode_attend": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                              "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                              "algorithmic_bytes": dec_bytes}},
    }


def run_causal_lm(args, torch, new_tokens=256):
    """Config 4: the random-init hybrid causal LM (config4(): d_model 1024, six
    blocks of SSD (expand 2, d_state 128, headdim 64) then selective attention
    (16 heads x 64), vocab 32000, bf16), batch 4 prefill of 8192 uniform-random
    tokens, then `new_tokens` greedy decode steps; attention gate threshold 0.5
    per head (the reference's warm-up value), score statistics set to 1.
    Prefill and decode are timed with the host clock around synchronised runs
    (decode is host-launch bound)."""
    from selective_attention.inference import CausalBlockCache, GenerationConfig, InferenceState
    from selective_attention.models import CausalLM, config4
    from selective_attention.profiling import kernel_timer

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    cfg = config4("cuda")
    m = CausalLM(cfg)
    with torch.no_grad():
        for blk in m.layers:
            blk.mha.score_std_ema.fill_(1.0)
    m = m.to_bf16().to(dev).eval()
    b, L = 4, 8192
    g = torch.Generator(device=dev).manual_seed(1)
    ids = torch.randint(10, cfg.vocab_size, (b, L), device=dev, generator=g)
    thr = torch.full((cfg.num_layers, cfg.model_dim // cfg.head_dim), 0.5, device=dev)
    gen = GenerationConfig(bos_token_id=-1, eos_token_id=-1, pad_token_id=0,
                           max_new_tokens=new_tokens, attn_gate_thresholds=thr)
    lengths = torch.full((b,), L, device=dev)

    def prefill():
        cache = [CausalBlockCache(reserve=new_tokens) for _ in m.layers]
        h = m._hidden(ids, lengths, thr, cache)
        return cache, m.lm_head(m.norm(h[:, -1]))

    with torch.no_grad():
        m.generate(ids[:, :512], GenerationConfig(bos_token_id=-1, eos_token_id=-1, pad_token_id=0,
                                                  max_new_tokens=4, attn_gate_thresholds=thr))
        prefill()
        torch.cuda.synchronize()
        reps = 3
        t0 = time.perf_counter()
        for _ in range(reps):
            cache, logits = prefill()
        torch.cuda.synchronize()
        t_pre = (time.perf_counter() - t0) / reps
        with kernel_timer() as kt:
            prefill()
            torch.cuda.synchronize()
        pre_kernels = {n: round(x["total_ms"] * 1e3, 1) for n, x in kt.stats.items()}
        # eager decode steps (one host launch per op), for comparison
        state = InferenceState(lengths.clone())
        nxt = logits.argmax(-1)
        for _ in range(4):
            logits = m.step(nxt, cache, state, gen)
            state.update()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(32):
            nxt = torch.argmax(torch.softmax(logits, -1), -1)
            logits = m.step(nxt, cache, state, gen)
            state.update()
        torch.cuda.synchronize()
        t_eager = (time.perf_counter() - t0) / 32
        del cache
        # generate(): prefill + new_tokens greedy steps, the decode step replayed from a graph
        t0 = time.perf_counter()
        seq = m.generate(ids, gen)
        torch.cuda.synchronize()
        t_gen = time.perf_counter() - t0
        t_dec = (t_gen - t_pre) / (new_tokens - 1)
        assert seq.shape == (b, L + new_tokens)
    return {"generate_s": round(t_gen, 4),
            "tokens_per_s": round(b * (L + new_tokens) / t_gen, 1),
            "prefill_ms": round(t_pre * 1e3, 2),
            "prefill_tokens_per_s": round(b * L / t_pre, 1),
            "decode_ms_per_step": round(t_dec * 1e3, 3),
            "decode_tokens_per_s": round(b / t_dec, 1),
            "decode_eager_ms_per_step": round(t_eager * 1e3, 3),
            "prefill_kernel_us_total": pre_kernels,
            "config": {"workload": "hybrid_lm_config4", "batch": b, "prompt": L,
                       "new_tokens": new_tokens, "model_dim": cfg.model_dim,
                       "blocks": cfg.num_layers, "mixers": "SSD, attention alternating",
                       "vocab": cfg.vocab_size, "dtype": "bf16", "attn_gate_threshold": 0.5}}


def run_seq2seq(args, torch, enc_len=4096, new_tokens=128):
    """The seq2seq LM (no BASELINE config: a synthetic workload at config 4's
    dimensions): d_model 1024, six encoder BiBlocks and six decoder
    CrossBlocks (SSD d_state 128, 16 attention heads x 64), vocab 32000,
    bf16; batch 4 encoder inputs of `enc_len` random tokens, greedy decoding
    of `new_tokens` tokens; gate thresholds 0.5, score statistics 1.  Host
    clock around synchronised runs; decode per step = (generate - prefill) /
    (new_tokens - 1)."""
    from selective_attention.inference import CrossBlockCache, GenerationConfig
    from selective_attention.models import Seq2SeqLM, Seq2SeqLMConfig
    from selective_attention.profiling import kernel_timer

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    cfg = Seq2SeqLMConfig(vocab_size=32000, model_dim=1024, head_dim=64, ssm_state_dim=128,
                          ssm_num_groups=1, ssm_chunk_size=256, num_layers=6, dropout_rate=0.0,
                          device="cuda")
    m = Seq2SeqLM(cfg)
    with torch.no_grad():
        for mod in m.modules():
            if hasattr(mod, "score_std_ema"):
                mod.score_std_ema.fill_(1.0)
    m = m.to_bf16().to(dev).eval()
    b = 4
    g = torch.Generator(device=dev).manual_seed(1)
    ids = torch.randint(10, cfg.vocab_size, (b, enc_len), device=dev, generator=g)
    H = cfg.model_dim // cfg.head_dim
    thr = torch.full((cfg.num_layers, H), 0.5, device=dev)
    gen = GenerationConfig(bos_token_id=1, eos_token_id=-1, pad_token_id=0,
                           max_new_tokens=new_tokens, enc_attn_gate_thresholds=thr,
                           attn_gate_thresholds=thr, cross_attn_gate_thresholds=thr)
    lengths = torch.full((b,), enc_len, device=dev)
    bos = torch.ones(b, 1, dtype=torch.long, device=dev)

    def prefill():
        cache = [CrossBlockCache(reserve=new_tokens) for _ in m.decoder_layers]
        return m(ids, lengths, bos, thr, thr, thr, cache)

    with torch.no_grad():
        m.generate(ids[:, :256], GenerationConfig(bos_token_id=1, eos_token_id=-1, pad_token_id=0,
                                                  max_new_tokens=4))
        prefill()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(3):
            prefill()
        torch.cuda.synchronize()
        t_pre = (time.perf_counter() - t0) / 3
        with kernel_timer() as kt:
            prefill()
            torch.cuda.synchronize()
        kernels = {n: round(x["total_ms"] * 1e3, 1) for n, x in kt.stats.items()}
        t0 = time.perf_counter()
        seq = m.generate(ids, gen)
        torch.cuda.synchronize()
        t_gen = time.perf_counter() - t0
    assert seq.shape == (b, new_tokens)
    t_dec = (t_gen - t_pre) / (new_tokens - 1)
    return {"generate_s": round(t_gen, 4),
            "encode_prefill_ms": round(t_pre * 1e3, 2),
            "encoder_tokens_per_s": round(b * enc_len / t_pre, 1),
            "decode_ms_per_step": round(t_dec * 1e3, 3),
            "decode_tokens_per_s": round(b / t_dec, 1),
            "prefill_kernel_us_total": kernels,
            "config": {"workload": "seq2seq_synthetic", "batch": b, "encoder_len": enc_len,
                       "new_tokens": new_tokens, "model_dim": cfg.model_dim,
                       "encoder_blocks": cfg.num_layers, "decoder_blocks": cfg.num_layers,
                       "vocab": cfg.vocab_size, "dtype": "bf16", "attn_gate_threshold": 0.5}}


def _scan_gate_fusion(args, torch):
    """SSD forward + SSM epilogue at config 1: the scan then the gate kernel
    (fp32 y written and re-read) against the epilogue fused into the chunk
    scan (bf16 out and yd written, no y)."""
    from selective_attention import workloads
    from selective_attention.kernels.ssd_scan import ssd_scan_forward, ssd_scan_forward_gated
    from selective_attention.kernels.ssm_io import ssm_gate_forward

    dev = torch.device("cuda:0")
    cfg = dict(workloads.SSD_CONFIGS[1])
    x = workloads.ssd_inputs(**cfg, device=dev)
    b, L, H, P = x["u"].shape
    g = torch.Generator(device=dev).manual_seed(1)
    D = torch.randn(H * P, device=dev, generator=g)
    gate = torch.randn(b, L, H, P, device=dev, generator=g).to(x["u"].dtype)
    lim = (0.0, float("inf"))

    def unfused():
        y, _ = ssd_scan_forward(x["u"], x["A"], x["B"], x["C"], x["delta_raw"], None, None, None,
                                cfg["chunk"], True, lim)
        return ssm_gate_forward(y.view(b, L, H * P), x["u"].view(b, L, H * P), D,
                                gate.view(b, L, H * P))

    def fused():
        return ssd_scan_forward_gated(x["u"], x["A"], x["B"], x["C"], x["delta_raw"], None, None,
                                      None, cfg["chunk"], True, lim, D, gate)

    steps = max(args.steps, 10)
    ms_u = _time_events(torch, unfused, steps, args.warmup)
    ms_f = _time_events(torch, fused, steps, args.warmup)
    return {"unfused_us": round(ms_u * 1e3, 1), "fused_us": round(ms_f * 1e3, 1),
            "config": "ssd_scan_fwd_config1 + (y + D u) silu(gate), bf16 out"}


def run_ssm_io(args, torch):
    """The SSM block's stages around the scan at config 1's model shapes
    (b8, L4096, x_dim 2048 = 32 heads x 64, B/C 8 groups x 128, conv K=4,
    bf16 activations, fp32 y): the SiLU + causal-conv prologue (forward and
    backward) and the D-skip / SiLU-gate epilogue (forward and backward).
    Each kernel's time comes from HIP events on its launch stream; bytes are
    the algorithmic ones (each input read once, each output written once)."""
    from selective_attention.kernels.ssm_io import (ssm_conv_backward, ssm_conv_forward,
                                                    ssm_gate_backward, ssm_gate_forward)
    from selective_attention.profiling import kernel_timer

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    b, L, x_dim, bc_dim, K = 8, 4096, 2048, 1024, 4
    ch = x_dim + 2 * bc_dim
    bf = torch.bfloat16
    hbc = torch.randn(b, L, ch, device=dev, generator=g).to(bf)
    w = torch.randn(ch, K, device=dev, generator=g) * 0.5
    bias = torch.randn(ch, device=dev, generator=g) * 0.1
    dxbc = torch.randn(b, L, ch, device=dev, generator=g).to(bf)
    dx, dB, dC = dxbc[..., :x_dim].contiguous(), dxbc[..., x_dim:x_dim + bc_dim].contiguous(), \
        dxbc[..., x_dim + bc_dim:].contiguous()
    y = torch.randn(b, L, x_dim, device=dev, generator=g)
    x = torch.randn(b, L, x_dim, device=dev, generator=g).to(bf)
    gate = torch.randn(b, L, x_dim, device=dev, generator=g).to(bf)
    D = torch.randn(x_dim, device=dev, generator=g)
    dout = torch.randn(b, L, x_dim, device=dev, generator=g).to(bf)

    def step():
        ssm_conv_forward(hbc, w, bias, x_dim, bc_dim)
        ssm_conv_backward(hbc, w, dx, dB, dC, x_dim, bc_dim)
        ssm_gate_forward(y, x, D, gate)
        ssm_gate_backward(dout, y, x, D, gate)

    steps = max(args.steps, 10)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    with kernel_timer() as kt:
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
    act = b * L * ch * 2            # one bf16 pass over hBC-shaped data
    row = b * L * x_dim             # elements of y / x / gate
    nbytes = {"ssm_conv_fwd": 2 * act, "ssm_conv_bwd": 3 * act,
              "ssm_gate_fwd": row * (4 + 2 + 2 + 2), "ssm_gate_bwd": row * (2 + 4 + 2 + 2 + 4 + 2 + 2)}
    # each backward's fixed-order reduction of its weight / D partials counts with it
    extra = {"ssm_conv_bwd": "ssm_conv_grad_reduce", "ssm_gate_bwd": "ssm_gate_dD_reduce"}
    kernels = {}
    for k, nb in nbytes.items():
        us = kt.stats[k]["avg_us"]
        if k in extra and extra[k] in kt.stats:
            us += kt.stats[extra[k]]["avg_us"]
        gbs = nb / (us / 1e6) / 1e9
        kernels[k] = {"avg_us": round(us, 2), "algorithmic_bytes": nb, "achieved_gbs": round(gbs, 1),
                      "frac": round(gbs / HBM_PEAK_GBS, 4)}
    tot_b = sum(nbytes.values())
    tot_us = sum(v["avg_us"] for v in kernels.values())
    gbs = tot_b / (tot_us / 1e6) / 1e9
    fused = _scan_gate_fusion(args, torch)
    return {"us": round(tot_us, 1),
            "scan_gate_forward": fused,
            "config": {"workload": "ssm_io_config1", "batch": b, "seq_len": L, "x_dim": x_dim,
                       "bc_dim": bc_dim, "conv_kernel": K, "activations": "bf16", "y": "fp32"},
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "algorithmic_bytes": tot_b},
            "kernels": kernels,
            "aux_kernels_us": {k: round(v["avg_us"], 2) for k, v in kt.stats.items() if k not in nbytes},
            "note": "ssm_conv_bwd / ssm_gate_bwd include their partial-sum reductions"}


def _cpu_host(torch, threads):
    """Who ran the CPU baseline: logical CPUs the OS reports, the CPUs this
    process may run on, the torch threads used, and the CPU model."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    return {"cpu_count": os.cpu_count(), "affinity_cpus": affinity,
            "torch_threads": torch.get_num_threads(), "threads_requested": threads,
            "cpu_model": model}


def _median_time(fn, budget_s, max_reps=5):
    """1 warm-up call, then the median of up to max_reps timed calls that fit
    in budget_s (at least one)."""
    t0 = time.perf_counter()
    fn()
    first = time.perf_counter() - t0
    reps = max(1, min(max_reps, int(budget_s / max(first, 1e-3))))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], reps


def cpu_baseline(torch, budget_s):
    """The fp32 CPU restatement of the reference's algorithms (oracle/: the
    reference has no CPU path of its own) on this host, on bounded samples:

      value   config 1 fwd+bwd (oracle/ssd.py through its manual backward) on
              one of the 8 batch rows: tokens/s of that row
      legs    config 0 forward (the BASELINE-named CPU configuration, whole),
              config 3 decode (page gather + GQA softmax for 8 of the 64 rows,
              plus the whole state update), us per step scaled to 64 rows

    Threads: OMP_NUM_THREADS when set (the GPU box's CPU share), else every
    logical CPU.  Each figure is the median of up to 5 runs after 1 warm-up."""
    from oracle import attn as attn_ref
    from oracle import ssd as ref
    from oracle import ssu as ssu_ref
    from selective_attention import workloads

    threads = int(os.environ.get("OMP_NUM_THREADS") or 0) or (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    f32 = torch.float32
    inf = float("inf")
    share = budget_s / 3.0

    # config 1: one batch row, forward + backward
    cfg = dict(workloads.SSD_CONFIGS[1])
    cfg["batch"] = 1
    x = workloads.ssd_inputs(**cfg, with_dy=True)

    def c1():
        ref.ssd_scan_forward(x["u"], x["A"], x["B"], x["C"], x["delta_raw"], None, None, None,
                             cfg["chunk"], True, (0.0, inf), f32)
        ref.ssd_scan_backward(x["u"], x["A"], x["B"], x["C"], x["delta_raw"], None, None,
                              x["dy"], None, None, cfg["chunk"], True, (0.0, inf), f32)

    t1, r1 = _median_time(c1, share)
    tok1 = cfg["seqlen"]

    # config 0: the whole forward
    cfg0 = workloads.SSD_CONFIGS[0]
    x0 = workloads.ssd_inputs(**cfg0)

    def c0():
        y, _ = ref.ssd_scan_forward(x0["u"], x0["A"], x0["B"], x0["C"], x0["delta_raw"], None,
                                    None, None, cfg0["chunk"], True, (0.0, inf), f32)
        b, L, H, P = x0["u"].shape
        return y.reshape(b, L, H * P) + x0["D"] * x0["u"].reshape(b, L, H * P)

    t0, r0 = _median_time(c0, share)
    tok0 = cfg0["batch"] * cfg0["seqlen"]

    # config 3: 8 of the 64 decode rows (their pages copied to the host) + the state update
    rows = 8
    d = workloads.decode_inputs(device="cuda:0")
    total_tokens = int(d.seq_lens.to("cpu", torch.int64).sum())
    lens = d.seq_lens[:rows].to("cpu", torch.int64)
    ps = d.k_pages.shape[2]
    npg = [int((n + ps - 1) // ps) for n in lens.tolist()]
    pt = d.page_table[:rows].to("cpu", torch.int64)
    used = torch.cat([pt[i, :npg[i]] for i in range(rows)])
    kp = d.k_pages[used.to(d.k_pages.device)].cpu()
    vp = d.v_pages[used.to(d.v_pages.device)].cpu()
    local = torch.full_like(pt, -1)
    o = 0
    for i in range(rows):
        local[i, :npg[i]] = torch.arange(o, o + npg[i])
        o += npg[i]
    q = d.q[:rows].cpu()
    del d
    s3 = workloads.ssu_inputs()

    def attn():
        attn_ref.paged_decode_attn(q, kp, vp, local, lens, dtype=f32)

    def ssu():
        ssu_ref.ssu_forward(s3["u"], s3["A"], s3["B"], s3["C"], s3["delta_raw"], None, s3["h"],
                            dtype=f32)

    ta, ra = _median_time(attn, share / 2)
    ts, rs = _median_time(ssu, share / 2)
    # the attention's work is proportional to the cached tokens it reads:
    # scale the sample by the tokens of all 64 rows over those of the sample
    scale = total_tokens / int(lens.sum())
    return {"value": round(tok1 / t1, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"config 1 fwd+bwd on 1 of 8 batch rows (L={tok1}), fp32 torch restatement "
                      f"(oracle/ssd.py), median of {r1} after 1 warm-up: {t1:.2f} s per row",
            "host": _cpu_host(torch, threads),
            "legs": {
                "config0_fwd": {"tokens_per_s": round(tok0 / t0, 1), "ms": round(t0 * 1e3, 2),
                                "sample": f"whole config 0 forward (b2 L512 H8 P64 N64, y + D x "
                                          f"and h_last), median of {r0}"},
                "config3_decode": {"us_per_step": round((ta * scale + ts) * 1e6, 1),
                                   "attn_us": round(ta * scale * 1e6, 1),
                                   "ssu_us": round(ts * 1e6, 1),
                                   "sample": f"paged GQA attention on rows 0-{rows - 1} "
                                             f"({int(lens.sum())} cached tokens) scaled by "
                                             f"{scale:.3f} to the {total_tokens} cached tokens of "
                                             f"all 64 rows, plus the whole state update "
                                             f"(b64 H32 P64 N128), medians of {ra} / {rs}"},
            }}


# shader engines of an MI355X (8 XCDs x 4): SQ_BUSY_CYCLES sums over them, and
# each has 32 SIMDs, so SIMD-cycles of a dispatch = 32 x SQ_BUSY_CYCLES
MI355X_SIMDS_PER_SE = 32


def pmc_summary(paths, kernels=None):
    """Markdown table of rocprofv3 --pmc counters: per kernel (template
    arguments kept, namespace dropped), the mean of each counter over its
    dispatches; with the SQ counters present also per-wave instruction counts,
    the share of wave-cycles spent waiting and the MFMA pipe's busy share of
    all SIMD-cycles."""
    import collections
    import csv
    import re
    agg = collections.defaultdict(lambda: collections.defaultdict(list))
    order = []
    for path in paths:
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                name = r["Kernel_Name"]
                m = re.search(r"(\w+_kernel)(<[^(]*>)?", name)
                k = (m.group(1) + (m.group(2) or "")) if m else name[:60]
                k = k.replace("sa::", "")
                if "copyBuffer" in k or "elementwise" in k:   # one row per launch shape
                    k += f" [grid {r.get('Grid_Size', '?')}]"
                if kernels and not any(x in k for x in kernels):
                    continue
                if k not in agg:
                    order.append(k)
                agg[k][r["Counter_Name"]].append(float(r["Counter_Value"]))
    counters = sorted({c for k in order for c in agg[k]})
    lines = ["| kernel | dispatches | " + " | ".join(counters) + " | derived |",
             "|---|---:|" + "---:|" * len(counters) + "---|"]
    for k in order:
        mean = {c: sum(v) / len(v) for c, v in agg[k].items()}
        n = max(len(v) for v in agg[k].values())
        der = []
        waves = mean.get("SQ_WAVES")
        if waves:
            for c, lab in (("SQ_INSTS_MFMA", "mfma/wave"), ("SQ_INSTS_VALU", "valu/wave"),
                           ("SQ_INSTS_LDS", "lds/wave")):
                if c in mean:
                    der.append(f"{lab} {mean[c] / waves:.0f}")
        if mean.get("SQ_WAVE_CYCLES") and "SQ_WAIT_ANY" in mean:
            der.append(f"wait {mean['SQ_WAIT_ANY'] / mean['SQ_WAVE_CYCLES']:.0%} of wave-cycles")
        if mean.get("SQ_BUSY_CYCLES") and "SQ_VALU_MFMA_BUSY_CYCLES" in mean:
            der.append(f"MFMA busy {mean['SQ_VALU_MFMA_BUSY_CYCLES'] / (MI355X_SIMDS_PER_SE * mean['SQ_BUSY_CYCLES']):.1%} of SIMD-cycles")
        vals = " | ".join(f"{mean[c]:,.0f}" if c in mean else "" for c in counters)
        lines.append(f"| `{k}` | {n} | {vals} | {'; '.join(der)} |")
    return "\n".join(lines)


def main():
    if "--pmc-summary" in sys.argv:
        ap = argparse.ArgumentParser()
        ap.add_argument("--pmc-summary", nargs="+", required=True)
        ap.add_argument("--pmc-kernels", default=None,
                        help="comma-separated substrings; only kernels whose name holds one")
        a = ap.parse_args()
        print(pmc_summary(a.pmc_summary, a.pmc_kernels.split(",") if a.pmc_kernels else None))
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--ssd-only", action="store_true", help="skip every leg after the headline")
    ap.add_argument("--legs", default=None,
                    help="comma-separated subset of the legs after the headline "
                         "(decode, sparse, ssm_io, selective_mha, causal_lm, seq2seq)")
    ap.add_argument("--cpu-budget-s", type=float, default=20.0)
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="after the timed work, run 3 plain device copies of this many MiB "
                         "(the reference kernel for scaling HBM counters read under rocprofv3)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)

    import torch

    res = run_ssd(args, torch)
    ms = res["ms"]
    out = {
        "metric": "SSD scan fwd+bwd tokens/s & % roofline; decode attn+state us/step @ batch 64",
        "value": round(res["tokens"] / (ms / 1e3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "ms_per_step_mean": round(res["ms_mean"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded BASELINE config 1 recipe, resident in HBM)",
        "config": res["config"],
        "roofline": res["roofline"],
    }
    legs = [("ssd_shapes", "ssd_model_shapes", run_ssd_shapes),
            ("decode", "decode", run_decode), ("sparse", "sparse_attn", run_sparse),
            ("ssm_io", "ssm_io", run_ssm_io), ("selective_mha", "selective_mha", run_selective_mha),
            ("causal_lm", "causal_lm", run_causal_lm), ("seq2seq", "seq2seq", run_seq2seq)]
    want = set() if args.ssd_only else (
        {n for n, _, _ in legs} if args.legs is None else set(args.legs.split(",")))
    unknown = want - {n for n, _, _ in legs}
    if unknown:
        print(f"bench.py: unknown legs {sorted(unknown)}", file=sys.stderr)
        sys.exit(2)
    for name, key, fn in legs:
        if name in want:
            out[key] = fn(args, torch)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(torch, args.cpu_budget_s)
    if args.copy_probe_mib > 0:
        n = args.copy_probe_mib << 18   # float32 elements
        src = torch.ones(n, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        out["copy_probe_bytes"] = 4 * n
    print(json.dumps(out))


if __name__ == "__main__":
    main()
