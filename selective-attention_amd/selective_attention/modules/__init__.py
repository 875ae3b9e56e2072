"""The causal LM's modules on the gfx950 ops (reference: selective_attention/modules)."""
from .causal_block import CausalBlock
from .cross_selective_attention import CrossSelectiveMHA
from .layers import RMSNorm, RoPE, SwiGLU
from .selective_attention import SelectiveMHA
from .seq2seq_blocks import BiBlock, CrossBlock
from .ssm import SSM

__all__ = ["CausalBlock", "BiBlock", "CrossBlock", "RMSNorm", "RoPE", "SwiGLU", "SelectiveMHA",
           "CrossSelectiveMHA", "SSM"]
