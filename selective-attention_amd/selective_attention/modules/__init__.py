"""The causal LM's modules on the gfx950 ops (reference: selective_attention/modules)."""
from .causal_block import CausalBlock
from .layers import RMSNorm, RoPE, SwiGLU
from .selective_attention import SelectiveMHA
from .ssm import SSM

__all__ = ["CausalBlock", "RMSNorm", "RoPE", "SwiGLU", "SelectiveMHA", "SSM"]
