"""ctypes binding of libsa_hip.so, the C-ABI library of gfx950 kernels.

The library is loaded from this package directory.  There is no fallback:
if the library is missing or a symbol is absent, the import of the ops fails
with an error that says how to build it.  Every entry point returns 0 on
success; any other value is turned into a RuntimeError carrying
sa_last_error().
"""
from __future__ import annotations

import ctypes
import os

LIB_NAME = "libsa_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float
_sz = ctypes.c_size_t

# name -> argtypes; kept in the same order as include/sa_hip.h
SIGNATURES: dict[str, list] = {
    "sa_version": [],
    "sa_last_error": [],
    "sa_profile_enable": [_i],
    "sa_profile_collect": [ctypes.c_char_p, _i, ctypes.POINTER(_f), ctypes.POINTER(_i), _i],
    "sa_ssu_fwd": [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _f, _f, _vp],
    "sa_ssu_fwd_gated": [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                         _i, _f, _f, _vp],
    "sa_ssd_fwd": [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                   _i, _i, _i, _i, _i, _i, _i, _i, _f, _f,
                   _vp, _vp, _vp, _vp, _vp, _vp],
    "sa_ssd_bwd_workspace_size": [_i, _i, _i, _i, _i, _i, _i, _i],
    "sa_paged_decode_workspace_size": [_i, _i, _i, _i, _i],
    "sa_paged_decode_fwd": [_i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _f,
                            _vp, _vp, _sz, _vp],
    "sa_paged_decode_noalloc_limit": [],
    "sa_paged_decode_fwd_noalloc": [_i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i,
                                    _f, _vp, _vp],
    "sa_sparse_attn_fwd": [_i, _vp, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _vp, _i, _i, _i, _f,
                           _vp, _vp],
    "sa_attn_varlen_fwd": [_i, _i, _vp, _vp, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _i, _f, _vp, _vp],
    "sa_rms_norm_fwd": [_i, _vp, _vp, _i64, _i, _i, _f, _vp, _vp],
    "sa_rope_bf16": [_i, _vp, _vp, _vp, _vp, _i64, _i, _i, _vp, _vp, _i, _vp],
    "sa_paged_kv_build": [_vp, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _vp, _i, _i, _i,
                          _i, _i, _vp, _vp, _vp, _vp],
    "sa_paged_kv_append": [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp],
    "sa_add_rms_norm_bf16": [_vp, _vp, _vp, _i64, _i, _f, _vp, _vp, _vp],
    "sa_mha_gates_bf16": [_vp, _vp, _vp, _f, _i64, _i, _i, _vp, _vp, _vp],
    "sa_silu_mul_bf16": [_vp, _vp, _i64, _vp, _vp],
    "sa_score_stats_workspace_size": [_i, _i, _i],
    "sa_score_stats": [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _f, _vp, _sz, _vp, _vp],
    "sa_gemv_bf16": [_vp, _vp, _vp, _i, _i, _i, _vp, _vp],
    "sa_gemv_bf16_multi": [_vp, _vp, _i, _i, _i, ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                           ctypes.POINTER(_i), ctypes.POINTER(_vp), _vp],
    "sa_ssd_bwd": [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                   _i, _i, _i, _i, _i, _i, _i, _i, _f, _f, _i,
                   _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    "sa_ssm_conv_fwd": [_i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp],
    "sa_ssm_conv_bwd_workspace_size": [_i, _i, _i, _i],
    "sa_ssm_conv_bwd": [_i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp,
                        _vp, _sz, _vp],
    "sa_ssm_conv_step": [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp],
    "sa_ssm_gate_fwd": [_i, _vp, _vp, _vp, _vp, _i64, _i, _vp, _vp],
    "sa_ssm_gate_bwd_workspace_size": [_i64, _i],
    "sa_ssm_gate_bwd": [_i, _vp, _vp, _i, _vp, _vp, _vp, _i64, _i, _vp, _vp, _vp, _vp, _vp, _sz,
                        _vp],
    "sa_ssd_fwd_gated_supported": [_i, _i, _i],
    "sa_ssd_fwd_gated": [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                         _i, _i, _i, _i, _i, _i, _i, _i, _f, _f,
                         _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
}

RESTYPES = {"sa_last_error": ctypes.c_char_p, "sa_profile_enable": None, "sa_ssd_bwd_workspace_size": ctypes.c_size_t,
            "sa_paged_decode_workspace_size": ctypes.c_size_t,
            "sa_paged_decode_noalloc_limit": ctypes.c_size_t,
            "sa_ssm_conv_bwd_workspace_size": ctypes.c_size_t,
            "sa_ssm_gate_bwd_workspace_size": ctypes.c_size_t,
            "sa_score_stats_workspace_size": ctypes.c_size_t}

DTYPE_F32 = 0
DTYPE_BF16 = 1

_lib = None


class LibraryNotBuilt(ImportError):
    pass


def load(path: str | None = None):
    """Load (once) and return the ctypes library handle."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise LibraryNotBuilt(
            f"{p} not found: build it with `python selective-attention_amd/build.py` "
            "(hipcc --offload-arch=gfx950); there is no CPU fallback")
    lib = ctypes.CDLL(p)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError here means a stale build
        fn.argtypes = argtypes
        fn.restype = RESTYPES.get(name, ctypes.c_int)
    if path is None:
        _lib = lib
    return lib


def call(name: str, *args) -> None:
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.sa_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (code {rc}): {msg}")


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for an absent optional tensor)."""
    return None if t is None else t.data_ptr()


def stream_of(t) -> int:
    import torch
    return torch.cuda.current_stream(t.device).cuda_stream
