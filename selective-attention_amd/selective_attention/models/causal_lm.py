"""CausalLM (models/causal_lm.py:10-244) on the gfx950 ops: embedding, a
stack of CausalBlocks (SSM -> SelectiveMHA -> SwiGLU, pre-norm residual),
final RMSNorm, LM head tied to the embedding; forward, step and greedy
generate with the reference's interfaces.

Precision: to_bf16() puts the matmul weights and activations in bfloat16
and keeps the SSM's A_log / delta_bias / D and conv weights, the RMSNorm
weights and the attention score statistics in float32 (all are per-channel
vectors); RoPE's frequencies and angles are fp32 whatever the module dtype.
Not built: training through SelectiveMHA (no attention backward kernel),
the gate-analysis statistics and compute_attn_gate_threshold (calibration
runs on analysis histograms, outside the kernel path).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List

import torch
import torch.nn as nn

from ..inference import CausalBlockCache, GenerationConfig, InferenceState
from ..modules.layers import Linear
from ..modules import CausalBlock, RMSNorm
from ._graph import graph_decode


@dataclass
class CausalLMConfig:
    vocab_size: int = 32000
    model_dim: int = 512
    head_dim: int = 64
    attn_log_gate_penalty: float = 2.0
    ssm_state_dim: int = 64
    ssm_conv_kernel_size: int = 4
    ssm_num_groups: int = 1
    ssm_chunk_size: int = 256
    num_layers: int = 4
    dropout_rate: float = 0.15
    device: str | None = "cuda"


def config4(device="cuda") -> CausalLMConfig:
    """The hybrid LM of the benchmark's config 4: d_model 1024, SSD blocks
    with expand 2, d_state 128, headdim 64; selective attention with 16 heads
    of 64; vocab 32000.  Its 12 layers alternating SSD and attention are six
    CausalBlocks (each runs an SSM and then a SelectiveMHA)."""
    return CausalLMConfig(vocab_size=32000, model_dim=1024, head_dim=64, ssm_state_dim=128,
                          ssm_num_groups=1, ssm_chunk_size=256, num_layers=6, dropout_rate=0.0,
                          device=device)


class CausalLM(nn.Module):
    def __init__(self, cfg: CausalLMConfig | None = None):
        super().__init__()
        cfg = cfg or CausalLMConfig()
        self.cfg = cfg
        self.embedding = nn.Embedding(cfg.vocab_size, cfg.model_dim)
        self.layers = nn.ModuleList([
            CausalBlock(layer_idx=i, model_dim=cfg.model_dim, head_dim=cfg.head_dim,
                        attn_log_gate_penalty=cfg.attn_log_gate_penalty,
                        ssm_state_dim=cfg.ssm_state_dim,
                        ssm_conv_kernel_size=cfg.ssm_conv_kernel_size,
                        ssm_num_groups=cfg.ssm_num_groups, ssm_chunk_size=cfg.ssm_chunk_size,
                        dropout_rate=cfg.dropout_rate, device=cfg.device)
            for i in range(cfg.num_layers)])
        self.norm = RMSNorm(cfg.model_dim)
        self.lm_head = Linear(cfg.model_dim, cfg.vocab_size, bias=False)
        self.lm_head.weight = self.embedding.weight

    def to_bf16(self) -> "CausalLM":
        self.to(torch.bfloat16)
        for blk in self.layers:
            for p in (blk.ssm.A_log, blk.ssm.delta_bias, blk.ssm.D, blk.ssm.conv.weight,
                      blk.ssm.conv.bias, blk.norm1.weight, blk.norm2.weight, blk.norm3.weight):
                p.data = p.data.float()
            blk.mha.score_std_ema.data = blk.mha.score_std_ema.data.float()
        self.norm.weight.data = self.norm.weight.data.float()
        return self

    def _hidden(self, input_ids, lengths=None, attn_gate_thresholds=None, cache=None):
        h = self.embedding(input_ids)
        for i, layer in enumerate(self.layers):
            thr = attn_gate_thresholds[i] if attn_gate_thresholds is not None else None
            h, _ = layer(h, lengths=lengths, attn_gate_threshold=thr,
                         cache=cache[i] if cache is not None else None)
        return h

    def forward(self, input_ids: torch.Tensor, lengths: torch.Tensor | None = None,
                attn_gate_thresholds: torch.Tensor | List | None = None,
                cache: list | None = None, analysis_cfg=None, stats=None):
        """input_ids (batch_size, seq_len) -> logits (batch_size, seq_len, vocab_size)."""
        return self.lm_head(self.norm(self._hidden(input_ids, lengths, attn_gate_thresholds, cache)))

    def step(self, input_ids: torch.Tensor, cache: list, state: InferenceState,
             gen_cfg: GenerationConfig, analysis_cfg=None, stats=None):
        """input_ids (batch_size,) -> logits (batch_size, vocab_size).  Each
        block's last residual add runs with the next block's first norm (and
        the last one with the final norm): one kernel each."""
        h = self.embedding(input_ids)
        pend = None
        for i, layer in enumerate(self.layers):
            h, pend = layer.step(h, cache[i], state, gen_cfg, pending=pend, defer_add=True)
        return self.lm_head(self.norm.add_forward(h, pend)[1])

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, gen_cfg: GenerationConfig, analysis_cfg=None,
                 use_graph: bool = True, check_every: int = 16):
        """Greedy decoding (models/causal_lm.py:143-221): prefill, then up to
        max_new_tokens steps; tokens after the first eos become eos.
        Returns seq_ids (batch_size, seq_len + max_new_tokens).

        With use_graph, one decode step (the six blocks, the head, the argmax
        and the length update) is captured once in a HIP graph and replayed
        per token; the attention caches first fix their pages for the whole
        generation (enter_device_mode), so a replay needs no host work.  The
        stop test (every row has produced eos) is read every `check_every`
        tokens: tokens past a row's first eos are overwritten with eos at the
        end either way, so the output is the same as testing every token.
        Cache compaction is skipped in this mode (it frees memory only)."""
        b, L = input_ids.shape
        dev = input_ids.device
        new = gen_cfg.max_new_tokens
        cache = [CausalBlockCache(reserve=new) for _ in self.layers]
        lengths = (input_ids != gen_cfg.pad_token_id).sum(dim=1)
        state = InferenceState(lengths.clone())
        h = self._hidden(input_ids, lengths, gen_cfg.attn_gate_thresholds, cache)
        # logits of each row's last token only (the rows the reference keeps)
        logits = self.lm_head(self.norm(h[torch.arange(b, device=dev), lengths - 1]))
        seq_ids = torch.full((b, L + new), gen_cfg.pad_token_id, dtype=input_ids.dtype, device=dev)
        seq_ids[:, :L] = input_ids
        if new <= 0:
            return seq_ids
        if use_graph and dev.type == "cuda":
            self._generate_graph(logits, cache, state, gen_cfg, seq_ids, L, check_every)
        else:
            finished = torch.zeros(b, dtype=torch.bool, device=dev)
            for _ in range(new):
                nxt = torch.argmax(torch.softmax(logits, dim=-1), dim=-1)
                seq_ids[:, L + state.step] = nxt
                finished |= nxt == gen_cfg.eos_token_id
                if bool(finished.all()):
                    break
                logits = self.step(nxt, cache, state, gen_cfg)
                state.update()
        first_eos = (seq_ids == gen_cfg.eos_token_id).float().cumsum(dim=1) >= 1
        return torch.where(first_eos, gen_cfg.eos_token_id, seq_ids)

    def _generate_graph(self, logits, cache, state, gen_cfg, seq_ids, L, check_every):
        new = gen_cfg.max_new_tokens
        H, D = self.cfg.model_dim // self.cfg.head_dim, self.cfg.head_dim
        like = torch.empty(logits.shape[0], H, D, device=logits.device)
        for c in cache:
            c.attn_cache.prepare_decode(new, like)
        try:
            tok = torch.argmax(torch.softmax(logits, dim=-1), dim=-1)
            seq_ids[:, L] = tok
            state.step = 0

            def body():
                lg = self.step(tok, cache, state, gen_cfg)
                tok.copy_(torch.argmax(torch.softmax(lg, dim=-1), dim=-1))
                state.lengths.add_(1)

            def on_token(i):
                seq_ids[:, L + i] = tok
                state.step = i

            eos = gen_cfg.eos_token_id
            done = lambda: bool((seq_ids[:, L:L + state.step + 1] == eos).any(dim=1).all())
            graph_decode(body, new - 1, on_token, done, check_every)
        finally:
            for c in cache:
                c.attn_cache.pages.exit_device_mode()
