"""MI355X-native kernel layer of selective-attention.

`selective_attention.ops` keeps the reference's op signatures
(SSDScanFn, SSUFn) and adds sparse_attn_varlen / paged_decode_attn.  All
compute runs in libsa_hip.so (hand-written gfx950 HIP kernels behind a C
ABI); there is no CPU or PyTorch fallback.
"""
__version__ = "0.1.0"
