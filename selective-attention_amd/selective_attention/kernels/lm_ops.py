"""Host wrappers of the model-side ops (csrc/lm_ops.hip): fused RMSNorm (alone
and with the residual add before it), fused rotary embedding of q and k,
SelectiveMHA's decode-step gates, SwiGLU's gated product, and the paged
KV-cache append of a decode step."""
from __future__ import annotations

import torch

from .. import _lib
from .common import act_dtype_code, require_device


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """x (..., dim) contiguous f32 / bf16; weight (dim,) or (groups, dim) with
    x (..., groups, dim).  Returns x * rsqrt(mean(x^2) + eps) * (1 + weight)
    in x's dtype."""
    require_device(x, weight)
    dim = x.shape[-1]
    groups = 1 if weight.dim() == 1 else weight.shape[0]
    w = weight.to(torch.float32).contiguous()
    x = x.contiguous()
    out = torch.empty_like(x)
    _lib.call("sa_rms_norm_fwd", act_dtype_code(x.dtype), _lib.ptr(x), _lib.ptr(w),
              x.numel() // max(dim, 1), dim, groups, float(eps), _lib.ptr(out), _lib.stream_of(x))
    return out


def rope_qk(q: torch.Tensor, k: torch.Tensor, inv_freq: torch.Tensor,
            positions: torch.Tensor | None, period: int):
    """q, k (..., heads, head_dim) with the same shape; row r of the flattened
    leading dimensions is at positions[r % period] (int64), or at r % period
    when positions is None.  Returns the rotated q, k in bfloat16."""
    require_device(q, k, inv_freq, positions)
    H, D = q.shape[-2], q.shape[-1]
    q, k = q.contiguous(), k.to(q.dtype).contiguous()
    rows = q.numel() // (H * D)
    yq = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
    yk = torch.empty_like(yq)
    pos = None if positions is None else positions.to(torch.int64).contiguous()
    f = inv_freq.to(torch.float32).contiguous()
    _lib.call("sa_rope_bf16", act_dtype_code(q.dtype), _lib.ptr(q), _lib.ptr(k), _lib.ptr(yq),
              _lib.ptr(yk), rows, H, D, _lib.ptr(f), _lib.ptr(pos), int(period), _lib.stream_of(q))
    return yq, yk


def paged_kv_append(k, v, log_gate, page_table, seq_lens, k_pages, v_pages, gate_pages):
    """k, v (batch, heads, head_dim) bf16; log_gate (batch, heads) f32;
    page_table (batch, max_pages) int32; seq_lens (batch,) int32, advanced
    in place; the pages as in PagedSelectiveAttnCache."""
    require_device(k, v, log_gate, page_table, seq_lens, k_pages, v_pages, gate_pages)
    b, H, D = k.shape
    ps = k_pages.shape[2]
    k = k.to(torch.bfloat16).contiguous()
    v = v.to(torch.bfloat16).contiguous()
    lg = log_gate.to(torch.float32).contiguous()
    for t, name in ((page_table, "page_table"), (seq_lens, "seq_lens")):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"paged_kv_append: {name} must be a contiguous int32 tensor")
    _lib.call("sa_paged_kv_append", _lib.ptr(k), _lib.ptr(v), _lib.ptr(lg), _lib.ptr(page_table),
              _lib.ptr(seq_lens), b, H, D, ps, page_table.shape[1], _lib.ptr(k_pages),
              _lib.ptr(v_pages), _lib.ptr(gate_pages), _lib.stream_of(k))


def paged_kv_build(k, v, log_gate, page_table, seq_lens, k_pages, v_pages, gate_pages):
    """k, v (batch, heads, seq_len, head_dim) bf16 (any strides with head_dim
    contiguous, e.g. transposed views of (batch, seq_len, heads, head_dim));
    log_gate (batch, heads, seq_len); page_table (batch, max_pages) int32;
    seq_lens (batch,) int32: tokens t < seq_lens[r] of row r go to its pages
    (PagedSelectiveAttnCache layouts), the rest of its last page is zeroed
    with -inf gates.  One launch."""
    require_device(k, v, log_gate, page_table, seq_lens, k_pages, v_pages, gate_pages)
    b, H, L, D = k.shape
    if b == 0 or L == 0:
        return   # no tokens: no row has a page to write
    ps = k_pages.shape[2]
    k = k.to(torch.bfloat16)
    v = v.to(torch.bfloat16)
    if k.stride(3) != 1 or v.stride() != k.stride() or any(x % 8 for x in k.stride()[:3]):
        k, v = k.contiguous(), v.contiguous()
    lg = log_gate.to(torch.float32)
    for t, name in ((page_table, "page_table"), (seq_lens, "seq_lens")):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"paged_kv_build: {name} must be a contiguous int32 tensor")
    sb, sh, st = k.stride(0), k.stride(1), k.stride(2)
    _lib.call("sa_paged_kv_build", _lib.ptr(k), _lib.ptr(v), sb, st, sh, _lib.ptr(lg),
              lg.stride(0), lg.stride(1), lg.stride(2), _lib.ptr(page_table), _lib.ptr(seq_lens),
              b, H, D, ps, page_table.shape[1], _lib.ptr(k_pages), _lib.ptr(v_pages),
              _lib.ptr(gate_pages), _lib.stream_of(k))


def add_rms_norm_supported(x: torch.Tensor, weight: torch.Tensor) -> bool:
    d = x.shape[-1]
    return (x.is_cuda and x.dtype == torch.bfloat16 and x.is_contiguous() and weight.dim() == 1
            and d % 512 == 0 and d <= 4096)


def add_rms_norm(x: torch.Tensor, y: torch.Tensor, weight: torch.Tensor, eps: float):
    """(x + y, RMSNorm(x + y)) for bf16 rows; see add_rms_norm_supported."""
    require_device(x, y, weight)
    y = y.to(x.dtype).contiguous()
    w = weight.to(torch.float32).contiguous()
    out = torch.empty_like(x)
    nrm = torch.empty_like(x)
    dim = x.shape[-1]
    _lib.call("sa_add_rms_norm_bf16", _lib.ptr(x), _lib.ptr(y), _lib.ptr(w), x.numel() // dim, dim,
              float(eps), _lib.ptr(out), _lib.ptr(nrm), _lib.stream_of(x))
    return out, nrm


def mha_gates(g: torch.Tensor, threshold: torch.Tensor | None, score_std: torch.Tensor,
              penalty: float, heads: int):
    """g (rows, heads + dim) bf16 -> (log_gate (rows, heads) f32, out_gate (rows, dim) bf16)."""
    require_device(g, threshold, score_std)
    g = g.contiguous()
    rows, W = g.shape
    dim = W - heads
    lg = torch.empty(rows, heads, dtype=torch.float32, device=g.device)
    og = torch.empty(rows, dim, dtype=torch.bfloat16, device=g.device)
    thr = None if threshold is None else threshold.to(torch.float32).contiguous()
    std = score_std.to(torch.float32).contiguous()
    _lib.call("sa_mha_gates_bf16", _lib.ptr(g), _lib.ptr(thr), _lib.ptr(std), float(penalty), rows,
              heads, dim, _lib.ptr(lg), _lib.ptr(og), _lib.stream_of(g))
    return lg, og


def silu_mul(a: torch.Tensor, c: torch.Tensor) -> torch.Tensor:
    """bf16(a * bf16(silu(c))) for bf16 tensors of one shape (numel % 8 == 0)."""
    require_device(a, c)
    a, c = a.contiguous(), c.contiguous()
    out = torch.empty_like(a)
    _lib.call("sa_silu_mul_bf16", _lib.ptr(a), _lib.ptr(c), a.numel(), _lib.ptr(out),
              _lib.stream_of(a))
    return out


def gemv_supported(x: torch.Tensor, weight: torch.Tensor) -> bool:
    K = x.shape[-1]
    return (x.is_cuda and x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
            and weight.is_contiguous() and K % 8 == 0 and K <= 4096
            and 0 < x.numel() // max(K, 1) <= 8
            and weight.data_ptr() % 16 == 0)


def gemv(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    """x (..., K) with at most 8 rows, weight (N, K), bias (N,) or None, all
    bf16 -> (..., N): the decode steps' linear layers."""
    require_device(x, weight, bias)
    K = x.shape[-1]
    N = weight.shape[0]
    xc = x.contiguous()
    if xc.data_ptr() % 16:
        xc = xc.clone()
    M = xc.numel() // K
    y = torch.empty(*x.shape[:-1], N, dtype=torch.bfloat16, device=x.device)
    b = None if bias is None else bias.to(torch.bfloat16).contiguous()
    _lib.call("sa_gemv_bf16", _lib.ptr(xc), _lib.ptr(weight), _lib.ptr(b), M, N, K, _lib.ptr(y),
              _lib.stream_of(x))
    return y


def gemv_multi(x: torch.Tensor, weights, biases, xscale: torch.Tensor | None = None):
    """x (..., K) with at most 8 rows; weights: 1..4 bf16 (N_i, K) matrices
    (contiguous, 16-byte aligned: row blocks of one weight qualify); biases:
    matching (N_i,) bf16 tensors or None -> [(..., N_i)], one launch.  With
    xscale (same shape as x) the product bf16(x * xscale) is the input."""
    import ctypes
    require_device(x, *weights)
    K = x.shape[-1]
    n = len(weights)
    if not 1 <= n <= 4:
        raise ValueError(f"gemv_multi: 1..4 weight matrices, got {n}")
    for w in weights:
        if w.shape[-1] != K or not gemv_supported(x, w):
            raise ValueError(f"gemv_multi: weight {tuple(w.shape)} does not fit x {tuple(x.shape)}")
    xc = x.contiguous()
    if xc.data_ptr() % 16:
        xc = xc.clone()
    gc = None
    if xscale is not None:
        if xscale.shape != x.shape or xscale.dtype != torch.bfloat16:
            raise ValueError("gemv_multi: xscale must be bf16 of x's shape")
        gc = xscale.contiguous()
        if gc.data_ptr() % 16:
            gc = gc.clone()
    M = xc.numel() // K
    ys = [torch.empty(*x.shape[:-1], w.shape[0], dtype=torch.bfloat16, device=x.device)
          for w in weights]
    bs = [None if b is None else b.to(torch.bfloat16).contiguous() for b in biases]
    arr = ctypes.c_void_p * n
    _lib.call("sa_gemv_bf16_multi", _lib.ptr(xc), _lib.ptr(gc), M, K, n,
              arr(*[w.data_ptr() for w in weights]), arr(*[_lib.ptr(b) for b in bs]),
              (ctypes.c_int * n)(*[w.shape[0] for w in weights]),
              arr(*[y.data_ptr() for y in ys]), _lib.stream_of(x))
    return ys
