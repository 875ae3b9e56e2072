"""The language models on the gfx950 ops (reference: selective_attention/models)."""
from .causal_lm import CausalLM, CausalLMConfig, config4
from .seq2seq_lm import Seq2SeqLM, Seq2SeqLMConfig

__all__ = ["CausalLM", "CausalLMConfig", "config4", "Seq2SeqLM", "Seq2SeqLMConfig"]
