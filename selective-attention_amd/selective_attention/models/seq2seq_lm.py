"""Seq2SeqLM (models/seq2seq_lm.py:10-304) on the gfx950 ops: an encoder of
BiBlocks and a final SSM whose last state (normalised per head by norm3)
seeds every decoder SSM, a decoder of CrossBlocks attending the encoder
output, and a LM head tied to the embedding; forward, step and greedy
generate with the reference's interfaces.  Inference only where attention
is involved (no attention backward kernel); to_bf16() as for CausalLM.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn

from ..inference import CrossBlockCache, GenerationConfig, InferenceState
from ..modules.layers import Linear
from ..modules import SSM, BiBlock, CrossBlock, RMSNorm
from ._graph import graph_decode


@dataclass
class Seq2SeqLMConfig:
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


def _thr(t, i):
    return t[i] if t is not None else None


class Seq2SeqLM(nn.Module):
    def __init__(self, cfg: Seq2SeqLMConfig | None = None):
        super().__init__()
        cfg = cfg or Seq2SeqLMConfig()
        self.cfg = cfg
        blk = dict(model_dim=cfg.model_dim, head_dim=cfg.head_dim,
                   attn_log_gate_penalty=cfg.attn_log_gate_penalty, ssm_state_dim=cfg.ssm_state_dim,
                   ssm_conv_kernel_size=cfg.ssm_conv_kernel_size, ssm_num_groups=cfg.ssm_num_groups,
                   ssm_chunk_size=cfg.ssm_chunk_size, dropout_rate=cfg.dropout_rate,
                   device=cfg.device)
        self.embedding = nn.Embedding(cfg.vocab_size, cfg.model_dim)
        self.norm1 = RMSNorm(cfg.model_dim)
        self.norm2 = RMSNorm(cfg.model_dim)
        self.norm3 = RMSNorm(dim=cfg.ssm_state_dim, num_groups=cfg.model_dim * 2 // cfg.head_dim)
        self.norm4 = RMSNorm(cfg.model_dim)
        self.encoder_layers = nn.ModuleList([BiBlock(layer_idx=i, **blk)
                                             for i in range(cfg.num_layers)])
        self.ssm = SSM(layer_idx=cfg.num_layers, model_dim=cfg.model_dim,
                       state_dim=cfg.ssm_state_dim, conv_kernel_size=cfg.ssm_conv_kernel_size,
                       head_dim=cfg.head_dim, num_groups=cfg.ssm_num_groups,
                       chunk_size=cfg.ssm_chunk_size, dropout_rate=cfg.dropout_rate,
                       device=cfg.device)
        self.decoder_layers = nn.ModuleList([CrossBlock(layer_idx=i, **blk)
                                             for i in range(cfg.num_layers)])
        self.lm_head = Linear(cfg.model_dim, cfg.vocab_size, bias=False)
        self.lm_head.weight = self.embedding.weight
        self.dropout = nn.Dropout(cfg.dropout_rate)

    def to_bf16(self) -> "Seq2SeqLM":
        fp32 = [p for n, p in self.named_parameters()
                if n.endswith(("A_log", "delta_bias", ".D", "ssm.conv.weight", "ssm.conv.bias"))
                or "norm" in n]
        keep = {id(p): p.data.clone() for p in fp32}
        self.to(torch.bfloat16)
        for p in fp32:
            p.data = keep[id(p)].float()
        for m in self.modules():
            if hasattr(m, "score_std_ema"):
                m.score_std_ema.data = m.score_std_ema.data.float()
        return self

    def encode(self, input_ids, lengths, enc_attn_gate_thresholds=None):
        """Encoder output (batch, enc_len, model_dim) and the decoders' initial
        SSM state (batch, heads, head_dim, state_dim) float32 (:151-169)."""
        h = self.embedding(input_ids)
        for i, layer in enumerate(self.encoder_layers):
            h, _ = layer(h, lengths=lengths, attn_gate_threshold=_thr(enc_attn_gate_thresholds, i))
        s, ssm_hiddens = self.ssm(self.norm1(h), lengths=lengths)
        h = self.norm2(h + self.dropout(s))
        ssm_hiddens = self.norm3(ssm_hiddens.transpose(1, 2)).transpose(1, 2).contiguous()
        return h, ssm_hiddens

    def decode(self, decoder_input_ids, context, context_lengths, ssm_hiddens,
               attn_gate_thresholds=None, cross_attn_gate_thresholds=None, cache=None):
        h = self.embedding(decoder_input_ids)
        for i, layer in enumerate(self.decoder_layers):
            h = layer(h, context=context, context_lengths=context_lengths, ssm_hiddens=ssm_hiddens,
                      self_attn_gate_threshold=_thr(attn_gate_thresholds, i),
                      cross_attn_gate_threshold=_thr(cross_attn_gate_thresholds, i),
                      cache=cache[i] if cache is not None else None)
        return self.lm_head(self.norm4(h))

    def forward(self, input_ids: torch.Tensor, lengths: torch.Tensor,
                decoder_input_ids: torch.Tensor, enc_attn_gate_thresholds=None,
                attn_gate_thresholds=None, cross_attn_gate_thresholds=None, cache=None,
                analysis_cfg=None, stats=None):
        """input_ids (batch, enc_len), lengths (batch,), decoder_input_ids
        (batch, dec_len) -> logits (batch, dec_len, vocab_size)."""
        context, ssm_hiddens = self.encode(input_ids, lengths, enc_attn_gate_thresholds)
        return self.decode(decoder_input_ids, context, lengths, ssm_hiddens, attn_gate_thresholds,
                           cross_attn_gate_thresholds, cache)

    def step(self, input_ids: torch.Tensor, cache, state: InferenceState,
             gen_cfg: GenerationConfig, analysis_cfg=None, stats=None):
        """input_ids (batch,) -> logits (batch, vocab_size); residual adds
        as in CausalLM.step."""
        h = self.embedding(input_ids)
        pend = None
        for i, layer in enumerate(self.decoder_layers):
            h, pend = layer.step(h, cache[i], state, gen_cfg, pending=pend, defer_add=True)
        return self.lm_head(self.norm4.add_forward(h, pend)[1])

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, gen_cfg: GenerationConfig, analysis_cfg=None,
                 use_graph: bool = True, check_every: int = 16):
        """Greedy decoding (:213-300): the decoder starts from bos, then up to
        max_new_tokens - 1 steps; tokens after the first eos become eos.
        Returns seq_ids (batch, max_new_tokens).  use_graph / check_every as
        in CausalLM.generate."""
        b = input_ids.shape[0]
        dev = input_ids.device
        new = gen_cfg.max_new_tokens
        cache = [CrossBlockCache(reserve=new) for _ in self.decoder_layers]
        state = InferenceState(torch.ones(b, dtype=torch.long, device=dev))
        lengths = (input_ids != gen_cfg.pad_token_id).sum(dim=1)
        seq_ids = torch.full((b, new), gen_cfg.pad_token_id, dtype=input_ids.dtype, device=dev)
        seq_ids[:, 0] = gen_cfg.bos_token_id
        logits = self.forward(input_ids, lengths, seq_ids[:, :1], gen_cfg.enc_attn_gate_thresholds,
                              gen_cfg.attn_gate_thresholds, gen_cfg.cross_attn_gate_thresholds,
                              cache).squeeze(1)
        eos = gen_cfg.eos_token_id
        if new > 1 and use_graph and dev.type == "cuda":
            H, D = self.cfg.model_dim // self.cfg.head_dim, self.cfg.head_dim
            like = torch.empty(b, H, D, device=dev)
            for c in cache:
                c.attn_cache.prepare_decode(new, like)
            try:
                tok = torch.argmax(logits, dim=-1)
                seq_ids[:, 1] = tok
                state.step = 0

                def body():
                    lg = self.step(tok, cache, state, gen_cfg)
                    tok.copy_(torch.argmax(lg, dim=-1))
                    state.lengths.add_(1)

                def on_token(i):
                    seq_ids[:, 1 + i] = tok
                    state.step = i

                done = lambda: bool((seq_ids[:, 1:2 + state.step] == eos).any(dim=1).all())
                graph_decode(body, new - 2, on_token, done, check_every)
            finally:
                for c in cache:
                    c.attn_cache.pages.exit_device_mode()
        else:
            finished = torch.zeros(b, dtype=torch.bool, device=dev)
            for _ in range(new - 1):
                nxt = torch.argmax(logits, dim=-1)
                seq_ids[:, state.step + 1] = nxt
                finished |= nxt == eos
                if bool(finished.all()):
                    break
                logits = self.step(nxt, cache, state, gen_cfg)
                state.update()
        first_eos = (seq_ids == eos).float().cumsum(dim=1) >= 1
        return torch.where(first_eos, eos, seq_ids)
