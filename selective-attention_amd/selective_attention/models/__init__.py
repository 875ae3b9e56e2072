"""The causal LM on the gfx950 ops (reference: selective_attention/models)."""
from .causal_lm import CausalLM, CausalLMConfig, config4

__all__ = ["CausalLM", "CausalLMConfig", "config4"]
