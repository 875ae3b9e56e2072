from .attention import attn_varlen, paged_decode_attn, sparse_attn_varlen
from .selective_mha import (PagedSelectiveAttnCache, ScoreStdFn, cross_attention_train,
                           gated_attention_train, selective_mha_prefill)
from .ssd_scan import SSDScanFn
from .ssm_io import SSDScanGatedFn, SSMConvFn, SSMGateFn, build_conv_ctx, ssm_conv_step
from .ssu import SSUFn

__all__ = ["SSDScanFn", "SSUFn", "sparse_attn_varlen", "paged_decode_attn", "SSMConvFn",
           "SSMGateFn", "SSDScanGatedFn", "build_conv_ctx", "ssm_conv_step",
           "selective_mha_prefill", "PagedSelectiveAttnCache", "attn_varlen", "ScoreStdFn",
           "gated_attention_train", "cross_attention_train"]
