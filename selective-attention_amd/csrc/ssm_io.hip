// SSM block input / output stages around the SSD scan (gfx950).
//
// Prologue (modules/ssm.py:116-125, step: :173-182; cache: inference/ssm_cache.py:8-43):
//   xBC[b, t, c] = bias[c] + sum_{j<K} w[c, j] silu(hBC[b, t - K + 1 + j, c])
// (SiLU first, then a depthwise causal conv with zero history), split into
// x = xBC[..., :x_dim], B, C (each written to its own contiguous buffer, so
// the scan reads them without a copy).  Decode keeps the last K raw hBC
// rows per channel (conv_ctx, (b, channels, K)) and applies the same conv
// to that window after shifting the new row in.
//
// Epilogue (modules/ssm.py:144-150, step: :200-202):
//   out = (y + D x) silu(gate)
//
// All of these are HBM streams.  Threads own 8 consecutive channels (one
// 16-byte bf16 vector; a scalar variant covers channel counts that are not
// multiples of 8).  The conv kernels and the gate backward give a thread a
// run of consecutive rows: 32 for the conv kernels, which slide the K-row
// window in registers so every input row is read once (plus K - 1 halo rows
// per run), and 32 for the gate backward (fewer partial sums); a 256-thread
// block is 32 channel groups x 8 runs, and the weight / bias / D gradients
// are summed over the block's runs in LDS and written as one partial per
// block, then reduced in a fixed order (deterministic, no atomics).  The
// gate forward, which sums nothing, gives a thread one row (see there).
#include "common.h"
#include "prof.h"

namespace sa {
namespace {

constexpr int kCG = 32;      // channel groups per block
constexpr int kRuns = 8;     // row runs per block
constexpr int kConvRun = 32; // rows per run, conv kernels (K - 1 halo rows per run)
constexpr int kGbwdRun = 32; // rows per run, gate backward (fewer dD partials)
constexpr int kConvRows = kRuns * kConvRun;   // rows per block
constexpr int kGbwdRows = kRuns * kGbwdRun;

__device__ __forceinline__ float sigmoid_f(float z) { return fast_sigmoid(z); }
__device__ __forceinline__ float silu_f(float z) { return z * sigmoid_f(z); }
// d silu / dz = s (1 + z (1 - s)), s = sigmoid(z)
__device__ __forceinline__ float dsilu_f(float z) {
  const float s = sigmoid_f(z);
  return s * (1.0f + z * (1.0f - s));
}

// V consecutive elements <-> fp32
template <typename T, int V>
__device__ __forceinline__ void load_v(const T* p, float (&v)[V]) {
  if constexpr (V == 8 && sizeof(T) == 2) {
    const uint4 q = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bf16lo_to_f32(w[i]);
      v[2 * i + 1] = bf16hi_to_f32(w[i]);
    }
  } else if constexpr (V == 8) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else if constexpr (V == 4 && sizeof(T) == 2) {
    const uint2 q = *reinterpret_cast<const uint2*>(p);
    v[0] = bf16lo_to_f32(q.x); v[1] = bf16hi_to_f32(q.x);
    v[2] = bf16lo_to_f32(q.y); v[3] = bf16hi_to_f32(q.y);
  } else if constexpr (V == 4) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = load_f32(p + i);
  }
}
template <typename T, int V>
__device__ __forceinline__ void store_v(T* p, const float (&v)[V]) {
  if constexpr (V == 8 && sizeof(T) == 2) {
    *reinterpret_cast<uint4*>(p) = uint4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                         pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
  } else if constexpr (V == 8) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
  } else if constexpr (V == 4 && sizeof(T) == 2) {
    *reinterpret_cast<uint2*>(p) = uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  } else if constexpr (V == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) st(p + i, v[i]);
  }
}
template <int V>
__device__ __forceinline__ void zero_v(float (&v)[V]) {
#pragma unroll
  for (int i = 0; i < V; ++i) v[i] = 0.f;
}

// The split of a channel group: destination base (row 0 of batch row b) and row stride.
template <typename T>
__device__ __forceinline__ T* split_dst(T* x, T* Bo, T* Co, int c0, int x_dim, int bc_dim,
                                        long row0, int& rs) {
  if (c0 < x_dim) {
    rs = x_dim;
    return x + row0 * x_dim + c0;
  }
  if (c0 < x_dim + bc_dim) {
    rs = bc_dim;
    return Bo + row0 * bc_dim + (c0 - x_dim);
  }
  rs = bc_dim;
  return Co + row0 * bc_dim + (c0 - x_dim - bc_dim);
}

// ---------------------------------------------------------------------------
// prologue forward.  grid.x = batch * row blocks, grid.y = channel blocks.
// ---------------------------------------------------------------------------
template <typename T, int V, int K>
__global__ __launch_bounds__(256) void ssm_conv_fwd_kernel(
    const T* __restrict__ hbc, const float* __restrict__ w, const float* __restrict__ bias,
    T* __restrict__ x, T* __restrict__ Bo, T* __restrict__ Co, int L, int Dc, int x_dim,
    int bc_dim, int rblocks) {
  const int cg = threadIdx.x % kCG, run = threadIdx.x / kCG;
  const int b = blockIdx.x / rblocks;
  const int t0 = (blockIdx.x % rblocks) * kConvRows + run * kConvRun;
  const int c0 = (blockIdx.y * kCG + cg) * V;
  if (c0 >= Dc || t0 >= L) return;
  float wk[K][V], bs[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
#pragma unroll
    for (int j = 0; j < K; ++j) wk[j][v] = w[(c0 + v) * K + j];
    bs[v] = bias ? bias[c0 + v] : 0.f;
  }
  const long row0 = static_cast<long>(b) * L;
  const T* src = hbc + row0 * Dc + c0;
  int rs;
  T* dst = split_dst(x, Bo, Co, c0, x_dim, bc_dim, row0, rs);
  // silu of the K - 1 rows before t0 (zero history before row 0)
  float win[K > 1 ? K - 1 : 1][V];
#pragma unroll
  for (int i = 0; i < K - 1; ++i) {
    const int r = t0 - (K - 1) + i;
    if (r >= 0) {
      load_v<T, V>(src + static_cast<long>(r) * Dc, win[i]);
#pragma unroll
      for (int v = 0; v < V; ++v) win[i][v] = silu_f(win[i][v]);
    } else {
      zero_v(win[i]);
    }
  }
  const int tn = min(kConvRun, L - t0);
#pragma unroll 4
  for (int i = 0; i < tn; ++i) {
    const int t = t0 + i;
    float cur[V], o[V];
    load_v<T, V>(src + static_cast<long>(t) * Dc, cur);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      cur[v] = silu_f(cur[v]);
      float a = bs[v];
#pragma unroll
      for (int j = 0; j < K - 1; ++j) a += wk[j][v] * win[j][v];
      o[v] = a + wk[K - 1][v] * cur[v];
    }
#pragma unroll
    for (int j = 0; j + 1 < K - 1; ++j)
#pragma unroll
      for (int v = 0; v < V; ++v) win[j][v] = win[j + 1][v];
    if constexpr (K > 1) {
#pragma unroll
      for (int v = 0; v < V; ++v) win[K - 2][v] = cur[v];
    }
    store_v<T, V>(dst + static_cast<long>(t) * rs, o);
  }
}

// conv_ctx[b, c, j] = hBC[b, len_b - K + j, c] inside [0, len_b), else 0
// (inference/ssm_cache.py:8-36).  One thread per (b, c).
template <typename T>
__global__ __launch_bounds__(256) void ssm_conv_ctx_kernel(const T* __restrict__ hbc,
                                                           const int64_t* __restrict__ lengths,
                                                           T* __restrict__ ctx, int batch, int L,
                                                           int Dc, int K) {
  const long e = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= static_cast<long>(batch) * Dc) return;
  const int b = static_cast<int>(e / Dc), c = static_cast<int>(e % Dc);
  const long len = lengths ? lengths[b] : L;
  for (int j = 0; j < K; ++j) {
    const long s = len - K + j;
    float v = 0.f;
    if (s >= 0 && s < len && L > 0) {
      const long sc = s < L - 1 ? s : L - 1;
      v = load_f32(hbc + (static_cast<long>(b) * L + sc) * Dc + c);
    }
    st(ctx + e * K + j, v);
  }
}

// ---------------------------------------------------------------------------
// prologue backward.  g = (dx | dB | dC) by channel:
//   dhBC[s] = silu'(hBC[s]) sum_j w[j] g[s + K - 1 - j]
//   dW[j]   = sum_t g[t] silu(hBC[t - K + 1 + j]),  dbias = sum_t g[t]
// Per-block partials of (dW, dbias): part[row block][c][K + 1].
// ---------------------------------------------------------------------------
template <typename T, int V, int K>
__global__ __launch_bounds__(256) void ssm_conv_bwd_kernel(
    const T* __restrict__ hbc, const float* __restrict__ w, const T* __restrict__ dx,
    const T* __restrict__ dB, const T* __restrict__ dC, T* __restrict__ dhbc,
    float* __restrict__ part, int L, int Dc, int x_dim, int bc_dim, int rblocks) {
  __shared__ float red[kRuns][kCG * V];
  const int cg = threadIdx.x % kCG, run = threadIdx.x / kCG;
  const int b = blockIdx.x / rblocks;
  const int t0 = (blockIdx.x % rblocks) * kConvRows + run * kConvRun;
  const int c0 = (blockIdx.y * kCG + cg) * V;
  float dw[K][V], db[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    db[v] = 0.f;
#pragma unroll
    for (int j = 0; j < K; ++j) dw[j][v] = 0.f;
  }
  if (c0 < Dc && t0 < L) {
    float wk[K][V];
#pragma unroll
    for (int v = 0; v < V; ++v)
#pragma unroll
      for (int j = 0; j < K; ++j) wk[j][v] = w[(c0 + v) * K + j];
    const long row0 = static_cast<long>(b) * L;
    const T* src = hbc + row0 * Dc + c0;
    int gs;
    const T* gsrc = split_dst(const_cast<T*>(dx), const_cast<T*>(dB), const_cast<T*>(dC), c0,
                              x_dim, bc_dim, row0, gs);
    // look-behind: silu(hBC) of rows t0 - K + 1 .. t0 - 1; look-ahead: g rows t0 .. t0 + K - 2
    float sw[K > 1 ? K - 1 : 1][V], gw[K > 1 ? K - 1 : 1][V];
#pragma unroll
    for (int i = 0; i < K - 1; ++i) {
      const int r = t0 - (K - 1) + i;
      if (r >= 0) {
        load_v<T, V>(src + static_cast<long>(r) * Dc, sw[i]);
#pragma unroll
        for (int v = 0; v < V; ++v) sw[i][v] = silu_f(sw[i][v]);
      } else {
        zero_v(sw[i]);
      }
      const int q = t0 + i;
      if (q < L) load_v<T, V>(gsrc + static_cast<long>(q) * gs, gw[i]);
      else zero_v(gw[i]);
    }
    const int tn = min(kConvRun, L - t0);
    for (int i = 0; i < tn; ++i) {
      const int s = t0 + i;
      float h[V], gn[V], out[V];
      load_v<T, V>(src + static_cast<long>(s) * Dc, h);
      if (s + K - 1 < L) load_v<T, V>(gsrc + static_cast<long>(s + K - 1) * gs, gn);
      else zero_v(gn);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float sl = silu_f(h[v]);
        // g[s + k] for k = 0 .. K - 1: gw[0 .. K - 2] then gn
        const float g0 = K > 1 ? gw[0][v] : gn[v];   // g[s]
        float a = wk[0][v] * gn[v];                   // j = 0 pairs with g[s + K - 1]
#pragma unroll
        for (int j = 1; j < K; ++j) a += wk[j][v] * gw[K - 1 - j][v];
        out[v] = dsilu_f(h[v]) * a;
        // dW[j] += g[s] silu(hBC[s - K + 1 + j]): sw[0 .. K - 2] then sl
#pragma unroll
        for (int j = 0; j < K - 1; ++j) dw[j][v] += g0 * sw[j][v];
        dw[K - 1][v] += g0 * sl;
        db[v] += g0;
        h[v] = sl;
      }
      store_v<T, V>(dhbc + (row0 + s) * Dc + c0, out);
#pragma unroll
      for (int j = 0; j + 1 < K - 1; ++j)
#pragma unroll
        for (int v = 0; v < V; ++v) {
          sw[j][v] = sw[j + 1][v];
          gw[j][v] = gw[j + 1][v];
        }
      if constexpr (K > 1) {
#pragma unroll
        for (int v = 0; v < V; ++v) {
          sw[K - 2][v] = h[v];
          gw[K - 2][v] = gn[v];
        }
      }
    }
  }
  // sum the block's runs (same channels), one partial per row block and
  // entry j (taps 0 .. K - 1, then the bias): part[row block][c][K + 1]
  const int cbase = blockIdx.y * kCG * V;
  float* pb = part + static_cast<long>(blockIdx.x) * Dc * (K + 1);
#pragma unroll
  for (int j = 0; j <= K; ++j) {
#pragma unroll
    for (int v = 0; v < V; ++v) red[run][cg * V + v] = j < K ? dw[j < K ? j : 0][v] : db[v];
    __syncthreads();
    for (int e = threadIdx.x; e < kCG * V; e += 256) {
      const int c = cbase + e;
      if (c < Dc) {
        float s = 0.f;
#pragma unroll
        for (int r = 0; r < kRuns; ++r) s += red[r][e];
        pb[static_cast<long>(c) * (K + 1) + j] = s;
      }
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void fill_zero_kernel(float* __restrict__ p, long n) {
  const long e = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  if (e < n) p[e] = 0.f;
}

// out[e] = sum_p part[p][e] over np partials, e < n.  A block takes 32
// entries; its 8 waves-slices sum the partials p = slice (mod 8) four at a
// time, then the slices are added in order: a fixed summation order.
constexpr int kRedE = 32, kRedS = 8;
__global__ __launch_bounds__(256) void reduce_partials_kernel(const float* __restrict__ part,
                                                              int np, long n,
                                                              float* __restrict__ out) {
  __shared__ float red[kRedS][kRedE];
  const int el = threadIdx.x % kRedE, sl = threadIdx.x / kRedE;
  const long e = static_cast<long>(blockIdx.x) * kRedE + el;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  if (e < n) {
    int p = sl;
    for (; p + 3 * kRedS < np; p += 4 * kRedS) {
      a0 += part[static_cast<long>(p) * n + e];
      a1 += part[static_cast<long>(p + kRedS) * n + e];
      a2 += part[static_cast<long>(p + 2 * kRedS) * n + e];
      a3 += part[static_cast<long>(p + 3 * kRedS) * n + e];
    }
    for (; p < np; p += kRedS) a0 += part[static_cast<long>(p) * n + e];
  }
  red[sl][el] = (a0 + a1) + (a2 + a3);
  __syncthreads();
  if (sl == 0 && e < n) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < kRedS; ++k) s += red[k][el];
    out[e] = s;
  }
}
inline unsigned reduce_blocks(long n) { return static_cast<unsigned>((n + kRedE - 1) / kRedE); }

// (dW, dbias) from the interleaved [c][K + 1] sums
__global__ __launch_bounds__(256) void conv_grad_scatter_kernel(const float* __restrict__ sums,
                                                                int Dc, int K,
                                                                float* __restrict__ dw,
                                                                float* __restrict__ db) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= Dc) return;
  for (int j = 0; j < K; ++j) dw[c * K + j] = sums[c * (K + 1) + j];
  if (db) db[c] = sums[c * (K + 1) + K];
}

// ---------------------------------------------------------------------------
// decode step: ctx <- (ctx[1:], hbc_t); xBC = bias + sum_j w[j] silu(ctx[j]).
// One thread per (b, c).
// ---------------------------------------------------------------------------
template <typename T, int K>
__global__ __launch_bounds__(256) void ssm_conv_step_kernel(
    const T* __restrict__ hbc_t, T* __restrict__ ctx, const float* __restrict__ w,
    const float* __restrict__ bias, T* __restrict__ x, T* __restrict__ Bo, T* __restrict__ Co,
    int batch, int Dc, int x_dim, int bc_dim) {
  const long e = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= static_cast<long>(batch) * Dc) return;
  const int b = static_cast<int>(e / Dc), c = static_cast<int>(e % Dc);
  T* cx = ctx + e * K;
  float win[K];
#pragma unroll
  for (int j = 0; j + 1 < K; ++j) win[j] = load_f32(cx + j + 1);
  win[K - 1] = load_f32(hbc_t + e);
  float a = bias ? bias[c] : 0.f;
#pragma unroll
  for (int j = 0; j < K; ++j) {
    st(cx + j, win[j]);
    a += w[c * K + j] * silu_f(win[j]);
  }
  int rs;
  T* dst = split_dst(x, Bo, Co, c, x_dim, bc_dim, b, rs);
  st(dst, a);
}

// ---------------------------------------------------------------------------
// epilogue: out = (y + D x) silu(g); backward dy = dout silu(g), dx = D dy,
// dg = dout (y + D x) silu'(g), dD = sum_rows dy x (per-block partials).
// grid.x = row blocks, grid.y = channel blocks.
// ---------------------------------------------------------------------------
// One block per (row, 256 V channels): every wave reads and writes
// consecutive bytes of one row (1 KB of bf16, 2 KB of y), and a thread
// handles one vector of one row.  Runs of rows per thread (8 or 16, the
// block then walking a 64-row x 256-channel or 16 x 2048 tile) measured
// 145-153 us at config 1's shapes against 130 us for this form.
template <typename T, int V>
__global__ __launch_bounds__(256) void ssm_gate_fwd_kernel(const float* __restrict__ y,
                                                           const T* __restrict__ x,
                                                           const float* __restrict__ D,
                                                           const T* __restrict__ g,
                                                           T* __restrict__ out, long rows,
                                                           int dim) {
  const long r = blockIdx.x;
  const int c0 = (blockIdx.y * 256 + threadIdx.x) * V;
  if (c0 >= dim || r >= rows) return;
  const long off = r * dim + c0;
  float yv[V], xv[V], gv[V], o[V];
  load_v<float, V>(y + off, yv);
  load_v<T, V>(x + off, xv);
  load_v<T, V>(g + off, gv);
#pragma unroll
  for (int v = 0; v < V; ++v) o[v] = (yv[v] + D[c0 + v] * xv[v]) * silu_f(gv[v]);
  store_v<T, V>(out + off, o);
}

// YD: y holds yd = y + D x in T (saved by the fused scan epilogue) instead of the fp32 y
template <typename T, int V, bool YD>
__global__ __launch_bounds__(256) void ssm_gate_bwd_kernel(
    const T* __restrict__ dout, const void* __restrict__ y, const T* __restrict__ x,
    const float* __restrict__ D, const T* __restrict__ g, float* __restrict__ dy,
    T* __restrict__ dx, T* __restrict__ dg, float* __restrict__ part, long rows, int dim) {
  __shared__ float red[kRuns][kCG * V];
  const int cg = threadIdx.x % kCG, run = threadIdx.x / kCG;
  const long r0 = static_cast<long>(blockIdx.x) * kGbwdRows + run * kGbwdRun;
  const int c0 = (blockIdx.y * kCG + cg) * V;
  float dd[V];
  zero_v(dd);
  if (c0 < dim && r0 < rows) {
    float dv[V];
#pragma unroll
    for (int v = 0; v < V; ++v) dv[v] = D[c0 + v];
    const int tn = static_cast<int>(min(static_cast<long>(kGbwdRun), rows - r0));
#pragma unroll 4
    for (int i = 0; i < tn; ++i) {
      const long off = (r0 + i) * dim + c0;
      float ov[V], yv[V], xv[V], gv[V], a[V], b2[V], c2[V];
      load_v<T, V>(dout + off, ov);
      if constexpr (YD) load_v<T, V>(static_cast<const T*>(y) + off, yv);
      else load_v<float, V>(static_cast<const float*>(y) + off, yv);
      load_v<T, V>(x + off, xv);
      load_v<T, V>(g + off, gv);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float s = sigmoid_f(gv[v]);
        const float d = ov[v] * gv[v] * s;                       // dout silu(g)
        a[v] = d;
        b2[v] = dv[v] * d;
        const float yd = YD ? yv[v] : yv[v] + dv[v] * xv[v];
        c2[v] = ov[v] * yd * s * (1.0f + gv[v] * (1.0f - s));
        dd[v] += d * xv[v];
      }
      store_v<float, V>(dy + off, a);
      store_v<T, V>(dx + off, b2);
      store_v<T, V>(dg + off, c2);
    }
  }
#pragma unroll
  for (int v = 0; v < V; ++v) red[run][cg * V + v] = dd[v];
  __syncthreads();
  const int cbase = blockIdx.y * kCG * V;
  for (int e = threadIdx.x; e < kCG * V; e += 256) {
    const int c = cbase + e;
    if (c >= dim) continue;
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < kRuns; ++r) s += red[r][e];
    part[static_cast<long>(blockIdx.x) * dim + c] = s;
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
inline bool al16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int conv_rblocks(int L) { return (L + kConvRows - 1) / kConvRows; }

template <typename T, int V, int K>
int launch_conv_fwd(const void* hbc, const float* w, const float* bias, void* x, void* Bo, void* Co,
                    int batch, int L, int Dc, int x_dim, int bc_dim, hipStream_t s) {
  const int rb = conv_rblocks(L);
  const dim3 grid(batch * rb, (Dc + kCG * V - 1) / (kCG * V));
  ProfScope prof_("ssm_conv_fwd", s);
  hipLaunchKernelGGL((ssm_conv_fwd_kernel<T, V, K>), grid, dim3(256), 0, s,
                     static_cast<const T*>(hbc), w, bias, static_cast<T*>(x), static_cast<T*>(Bo),
                     static_cast<T*>(Co), L, Dc, x_dim, bc_dim, rb);
  SA_CHECK_LAUNCH("ssm_conv_fwd");
  return 0;
}

template <typename T, int V, int K>
int launch_conv_bwd(const void* hbc, const float* w, const void* dx, const void* dB, const void* dC,
                    void* dhbc, float* part, int batch, int L, int Dc, int x_dim, int bc_dim,
                    hipStream_t s) {
  const int rb = conv_rblocks(L);
  const dim3 grid(batch * rb, (Dc + kCG * V - 1) / (kCG * V));
  ProfScope prof_("ssm_conv_bwd", s);
  hipLaunchKernelGGL((ssm_conv_bwd_kernel<T, V, K>), grid, dim3(256), 0, s,
                     static_cast<const T*>(hbc), w, static_cast<const T*>(dx),
                     static_cast<const T*>(dB), static_cast<const T*>(dC), static_cast<T*>(dhbc),
                     part, L, Dc, x_dim, bc_dim, rb);
  SA_CHECK_LAUNCH("ssm_conv_bwd");
  return 0;
}

template <typename T, int V>
int dispatch_conv_k(int K, bool bwd, const void* hbc, const float* w, const float* bias,
                    const void* a0, const void* a1, const void* a2, void* o0, void* o1, void* o2,
                    float* part, int batch, int L, int Dc, int x_dim, int bc_dim, hipStream_t s) {
#define SA_CONV_CASE(KK)                                                                         \
  case KK:                                                                                       \
    return bwd ? launch_conv_bwd<T, V, KK>(hbc, w, a0, a1, a2, o0, part, batch, L, Dc, x_dim,    \
                                           bc_dim, s)                                            \
               : launch_conv_fwd<T, V, KK>(hbc, w, bias, o0, o1, o2, batch, L, Dc, x_dim, bc_dim, \
                                           s);
  switch (K) {
    SA_CONV_CASE(1)
    SA_CONV_CASE(2)
    SA_CONV_CASE(3)
    SA_CONV_CASE(4)
    SA_CONV_CASE(5)
    SA_CONV_CASE(6)
    SA_CONV_CASE(7)
    SA_CONV_CASE(8)
  }
#undef SA_CONV_CASE
  SA_CHECK_ARG(false, "ssm conv: kernel size %d outside [1, 8]", K);
  return 1;
}

template <typename T>
int dispatch_conv(int K, bool bwd, bool vec, const void* hbc, const float* w, const float* bias,
                  const void* a0, const void* a1, const void* a2, void* o0, void* o1, void* o2,
                  float* part, int batch, int L, int Dc, int x_dim, int bc_dim, hipStream_t s) {
  if (vec)
    return dispatch_conv_k<T, 8>(K, bwd, hbc, w, bias, a0, a1, a2, o0, o1, o2, part, batch, L, Dc,
                                 x_dim, bc_dim, s);
  return dispatch_conv_k<T, 1>(K, bwd, hbc, w, bias, a0, a1, a2, o0, o1, o2, part, batch, L, Dc,
                               x_dim, bc_dim, s);
}

int check_conv_dims(const char* who, int batch, int L, int Dc, int K, int x_dim, int bc_dim) {
  SA_CHECK_ARG(batch >= 0 && L >= 0 && Dc > 0 && x_dim >= 0 && bc_dim >= 0,
               "%s: bad sizes b=%d L=%d channels=%d x_dim=%d bc_dim=%d", who, batch, L, Dc, x_dim,
               bc_dim);
  SA_CHECK_ARG(x_dim + 2 * bc_dim == Dc, "%s: x_dim (%d) + 2 bc_dim (%d) != channels (%d)", who,
               x_dim, bc_dim, Dc);
  SA_CHECK_ARG(K >= 1 && K <= 8, "%s: kernel size %d outside [1, 8]", who, K);
  return 0;
}

size_t conv_part_elems(int batch, int L, int Dc, int K) {
  return static_cast<size_t>(batch) * conv_rblocks(L) * Dc * (K + 1);
}

}  // namespace
}  // namespace sa

using sa::bf16;

extern "C" int sa_ssm_conv_fwd(int dtype, const void* hbc, const float* weight, const float* bias,
                               int batch, int seqlen, int channels, int kernel, int x_dim,
                               int bc_dim, void* x, void* B, void* C, const int64_t* lengths,
                               void* conv_ctx, void* stream) {
  if (int rc = sa::check_conv_dims("sa_ssm_conv_fwd", batch, seqlen, channels, kernel, x_dim, bc_dim))
    return rc;
  SA_CHECK_ARG(dtype == sa::kF32 || dtype == sa::kBF16, "sa_ssm_conv_fwd: unsupported dtype %d", dtype);
  const bool conv = x || B || C;   // all three NULL: only conv_ctx is written
  SA_CHECK_ARG(hbc && weight && (conv || conv_ctx), "sa_ssm_conv_fwd: null tensor pointer");
  SA_CHECK_ARG(!conv || ((x || x_dim == 0) && (B || bc_dim == 0) && (C || bc_dim == 0)),
               "sa_ssm_conv_fwd: null output pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = channels % 8 == 0 && x_dim % 8 == 0 && bc_dim % 8 == 0 && sa::al16(hbc) &&
                   sa::al16(x) && sa::al16(B) && sa::al16(C);
  if (conv && batch > 0 && seqlen > 0) {
    const int rc = dtype == sa::kF32
        ? sa::dispatch_conv<float>(kernel, false, vec, hbc, weight, bias, nullptr, nullptr, nullptr,
                                   x, B, C, nullptr, batch, seqlen, channels, x_dim, bc_dim, s)
        : sa::dispatch_conv<bf16>(kernel, false, vec, hbc, weight, bias, nullptr, nullptr, nullptr,
                                  x, B, C, nullptr, batch, seqlen, channels, x_dim, bc_dim, s);
    if (rc) return rc;
  }
  if (conv_ctx && batch > 0) {
    const long n = static_cast<long>(batch) * channels;
    const dim3 grid(static_cast<unsigned>((n + 255) / 256));
    sa::ProfScope prof_("ssm_conv_ctx", s);
    if (dtype == sa::kF32)
      hipLaunchKernelGGL(sa::ssm_conv_ctx_kernel<float>, grid, dim3(256), 0, s,
                         static_cast<const float*>(hbc), lengths, static_cast<float*>(conv_ctx),
                         batch, seqlen, channels, kernel);
    else
      hipLaunchKernelGGL(sa::ssm_conv_ctx_kernel<bf16>, grid, dim3(256), 0, s,
                         static_cast<const bf16*>(hbc), lengths, static_cast<bf16*>(conv_ctx),
                         batch, seqlen, channels, kernel);
    SA_CHECK_LAUNCH("ssm_conv_ctx");
  }
  return 0;
}

extern "C" size_t sa_ssm_conv_bwd_workspace_size(int batch, int seqlen, int channels, int kernel) {
  if (batch <= 0 || seqlen <= 0 || channels <= 0 || kernel < 1 || kernel > 8) return 0;
  const size_t part = sa::conv_part_elems(batch, seqlen, channels, kernel);
  const size_t sums = static_cast<size_t>(channels) * (kernel + 1);
  return (part + sums) * sizeof(float);
}

extern "C" int sa_ssm_conv_bwd(int dtype, const void* hbc, const float* weight, const void* dx,
                               const void* dB, const void* dC, int batch, int seqlen,
                               int channels, int kernel, int x_dim, int bc_dim, void* dhbc,
                               float* dweight, float* dbias, void* workspace,
                               size_t workspace_bytes, void* stream) {
  if (int rc = sa::check_conv_dims("sa_ssm_conv_bwd", batch, seqlen, channels, kernel, x_dim, bc_dim))
    return rc;
  SA_CHECK_ARG(dtype == sa::kF32 || dtype == sa::kBF16, "sa_ssm_conv_bwd: unsupported dtype %d", dtype);
  SA_CHECK_ARG(hbc && weight && dhbc && dweight && (dx || x_dim == 0) && (dB || bc_dim == 0) &&
                   (dC || bc_dim == 0),
               "sa_ssm_conv_bwd: null tensor pointer");
  const size_t need = sa_ssm_conv_bwd_workspace_size(batch, seqlen, channels, kernel);
  SA_CHECK_ARG(workspace_bytes >= need && (need == 0 || workspace),
               "sa_ssm_conv_bwd: workspace %zu B < required %zu B", workspace_bytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (need == 0) {   // no rows: zero weight / bias gradients (a fill kernel, capturable)
    const long nw = static_cast<long>(channels) * kernel;
    hipLaunchKernelGGL(sa::fill_zero_kernel, dim3(static_cast<unsigned>((nw + 255) / 256)), dim3(256),
                       0, s, dweight, nw);
    if (dbias)
      hipLaunchKernelGGL(sa::fill_zero_kernel, dim3((channels + 255) / 256), dim3(256), 0, s, dbias,
                         static_cast<long>(channels));
    SA_CHECK_LAUNCH("sa_ssm_conv_bwd zero fill");
    return 0;
  }
  const bool vec = channels % 8 == 0 && x_dim % 8 == 0 && bc_dim % 8 == 0 && sa::al16(hbc) &&
                   sa::al16(dx) && sa::al16(dB) && sa::al16(dC) && sa::al16(dhbc);
  float* part = static_cast<float*>(workspace);
  const size_t np_elems = sa::conv_part_elems(batch, seqlen, channels, kernel);
  float* sums = part + np_elems;
  const int rc = dtype == sa::kF32
      ? sa::dispatch_conv<float>(kernel, true, vec, hbc, weight, nullptr, dx, dB, dC, dhbc, nullptr,
                                 nullptr, part, batch, seqlen, channels, x_dim, bc_dim, s)
      : sa::dispatch_conv<bf16>(kernel, true, vec, hbc, weight, nullptr, dx, dB, dC, dhbc, nullptr,
                                nullptr, part, batch, seqlen, channels, x_dim, bc_dim, s);
  if (rc) return rc;
  const long n = static_cast<long>(channels) * (kernel + 1);
  const int np = batch * sa::conv_rblocks(seqlen);
  {
    sa::ProfScope prof_("ssm_conv_grad_reduce", s);
    hipLaunchKernelGGL(sa::reduce_partials_kernel, dim3(sa::reduce_blocks(n)), dim3(256), 0, s,
                       part, np, n, sums);
    SA_CHECK_LAUNCH("ssm_conv_grad_reduce");
  }
  hipLaunchKernelGGL(sa::conv_grad_scatter_kernel, dim3((channels + 255) / 256), dim3(256), 0, s,
                     sums, channels, kernel, dweight, dbias);
  SA_CHECK_LAUNCH("ssm_conv_grad_scatter");
  return 0;
}

extern "C" int sa_ssm_conv_step(int dtype, const void* hbc_t, void* conv_ctx, const float* weight,
                                const float* bias, int batch, int channels, int kernel, int x_dim,
                                int bc_dim, void* x, void* B, void* C, void* stream) {
  if (int rc = sa::check_conv_dims("sa_ssm_conv_step", batch, 1, channels, kernel, x_dim, bc_dim))
    return rc;
  SA_CHECK_ARG(dtype == sa::kF32 || dtype == sa::kBF16, "sa_ssm_conv_step: unsupported dtype %d", dtype);
  SA_CHECK_ARG(hbc_t && conv_ctx && weight && (x || x_dim == 0) && (B || bc_dim == 0) &&
                   (C || bc_dim == 0),
               "sa_ssm_conv_step: null tensor pointer");
  if (batch == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const long n = static_cast<long>(batch) * channels;
  const dim3 grid(static_cast<unsigned>((n + 255) / 256));
  sa::ProfScope prof_("ssm_conv_step", s);
#define SA_STEP_CASE(KK)                                                                         \
  case KK:                                                                                       \
    if (dtype == sa::kF32)                                                                       \
      hipLaunchKernelGGL((sa::ssm_conv_step_kernel<float, KK>), grid, dim3(256), 0, s,           \
                         static_cast<const float*>(hbc_t), static_cast<float*>(conv_ctx), weight, \
                         bias, static_cast<float*>(x), static_cast<float*>(B),                   \
                         static_cast<float*>(C), batch, channels, x_dim, bc_dim);                \
    else                                                                                         \
      hipLaunchKernelGGL((sa::ssm_conv_step_kernel<bf16, KK>), grid, dim3(256), 0, s,            \
                         static_cast<const bf16*>(hbc_t), static_cast<bf16*>(conv_ctx), weight,  \
                         bias, static_cast<bf16*>(x), static_cast<bf16*>(B),                     \
                         static_cast<bf16*>(C), batch, channels, x_dim, bc_dim);                 \
    break;
  switch (kernel) {
    SA_STEP_CASE(1)
    SA_STEP_CASE(2)
    SA_STEP_CASE(3)
    SA_STEP_CASE(4)
    SA_STEP_CASE(5)
    SA_STEP_CASE(6)
    SA_STEP_CASE(7)
    SA_STEP_CASE(8)
  }
#undef SA_STEP_CASE
  SA_CHECK_LAUNCH("ssm_conv_step");
  return 0;
}

extern "C" int sa_ssm_gate_fwd(int dtype, const float* y, const void* x, const float* D,
                               const void* gate, int64_t rows, int dim, void* out, void* stream) {
  SA_CHECK_ARG(rows >= 0 && dim > 0, "sa_ssm_gate_fwd: bad sizes rows=%lld dim=%d",
               static_cast<long long>(rows), dim);
  SA_CHECK_ARG(dtype == sa::kF32 || dtype == sa::kBF16, "sa_ssm_gate_fwd: unsupported dtype %d", dtype);
  SA_CHECK_ARG(y && x && D && gate && out, "sa_ssm_gate_fwd: null tensor pointer");
  if (rows == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = dim % 8 == 0 && sa::al16(y) && sa::al16(x) && sa::al16(gate) && sa::al16(out);
  const int V = vec ? 8 : 1;
  SA_CHECK_ARG(rows <= 0x7fffffff, "sa_ssm_gate_fwd: %lld rows exceed the grid",
               static_cast<long long>(rows));
  const dim3 grid(static_cast<unsigned>(rows), (dim + 256 * V - 1) / (256 * V));
  sa::ProfScope prof_("ssm_gate_fwd", s);
  if (dtype == sa::kF32) {
    if (vec)
      hipLaunchKernelGGL((sa::ssm_gate_fwd_kernel<float, 8>), grid, dim3(256), 0, s, y,
                         static_cast<const float*>(x), D, static_cast<const float*>(gate),
                         static_cast<float*>(out), static_cast<long>(rows), dim);
    else
      hipLaunchKernelGGL((sa::ssm_gate_fwd_kernel<float, 1>), grid, dim3(256), 0, s, y,
                         static_cast<const float*>(x), D, static_cast<const float*>(gate),
                         static_cast<float*>(out), static_cast<long>(rows), dim);
  } else {
    if (vec)
      hipLaunchKernelGGL((sa::ssm_gate_fwd_kernel<bf16, 8>), grid, dim3(256), 0, s, y,
                         static_cast<const bf16*>(x), D, static_cast<const bf16*>(gate),
                         static_cast<bf16*>(out), static_cast<long>(rows), dim);
    else
      hipLaunchKernelGGL((sa::ssm_gate_fwd_kernel<bf16, 1>), grid, dim3(256), 0, s, y,
                         static_cast<const bf16*>(x), D, static_cast<const bf16*>(gate),
                         static_cast<bf16*>(out), static_cast<long>(rows), dim);
  }
  SA_CHECK_LAUNCH("ssm_gate_fwd");
  return 0;
}

extern "C" size_t sa_ssm_gate_bwd_workspace_size(int64_t rows, int dim) {
  if (rows <= 0 || dim <= 0) return 0;
  const size_t rb = static_cast<size_t>((rows + sa::kGbwdRows - 1) / sa::kGbwdRows);
  return rb * dim * sizeof(float);
}

extern "C" int sa_ssm_gate_bwd(int dtype, const void* dout, const void* y, int y_is_yd,
                               const void* x, const float* D, const void* gate, int64_t rows,
                               int dim, float* dy, void* dx, void* dgate, float* dD,
                               void* workspace, size_t workspace_bytes, void* stream) {
  SA_CHECK_ARG(rows >= 0 && dim > 0, "sa_ssm_gate_bwd: bad sizes rows=%lld dim=%d",
               static_cast<long long>(rows), dim);
  SA_CHECK_ARG(dtype == sa::kF32 || dtype == sa::kBF16, "sa_ssm_gate_bwd: unsupported dtype %d", dtype);
  SA_CHECK_ARG(dout && y && x && D && gate && dy && dx && dgate && dD,
               "sa_ssm_gate_bwd: null tensor pointer");
  const size_t need = sa_ssm_gate_bwd_workspace_size(rows, dim);
  SA_CHECK_ARG(workspace_bytes >= need && (need == 0 || workspace),
               "sa_ssm_gate_bwd: workspace %zu B < required %zu B", workspace_bytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (rows == 0) {
    hipLaunchKernelGGL(sa::fill_zero_kernel, dim3((dim + 255) / 256), dim3(256), 0, s, dD,
                       static_cast<long>(dim));
    SA_CHECK_LAUNCH("sa_ssm_gate_bwd zero fill");
    return 0;
  }
  const bool vec = dim % 8 == 0 && sa::al16(dout) && sa::al16(y) && sa::al16(x) && sa::al16(gate) &&
                   sa::al16(dy) && sa::al16(dx) && sa::al16(dgate);
  const int V = vec ? 8 : 1;
  const int rb = static_cast<int>((rows + sa::kGbwdRows - 1) / sa::kGbwdRows);
  const dim3 grid(rb, (dim + sa::kCG * V - 1) / (sa::kCG * V));
  float* part = static_cast<float*>(workspace);
  {
    sa::ProfScope prof_("ssm_gate_bwd", s);
#define SA_GATE_BWD(TT, VV, YDD)                                                                 \
  hipLaunchKernelGGL((sa::ssm_gate_bwd_kernel<TT, VV, YDD>), grid, dim3(256), 0, s,              \
                     static_cast<const TT*>(dout), y, static_cast<const TT*>(x), D,              \
                     static_cast<const TT*>(gate), dy, static_cast<TT*>(dx),                     \
                     static_cast<TT*>(dgate), part, static_cast<long>(rows), dim)
    if (dtype == sa::kF32) {
      if (vec) { if (y_is_yd) SA_GATE_BWD(float, 8, true); else SA_GATE_BWD(float, 8, false); }
      else { if (y_is_yd) SA_GATE_BWD(float, 1, true); else SA_GATE_BWD(float, 1, false); }
    } else {
      if (vec) { if (y_is_yd) SA_GATE_BWD(bf16, 8, true); else SA_GATE_BWD(bf16, 8, false); }
      else { if (y_is_yd) SA_GATE_BWD(bf16, 1, true); else SA_GATE_BWD(bf16, 1, false); }
    }
#undef SA_GATE_BWD
    SA_CHECK_LAUNCH("ssm_gate_bwd");
  }
  sa::ProfScope prof_("ssm_gate_dD_reduce", s);
  hipLaunchKernelGGL(sa::reduce_partials_kernel, dim3(sa::reduce_blocks(dim)), dim3(256), 0, s,
                     part, rb, static_cast<long>(dim), dD);
  SA_CHECK_LAUNCH("ssm_gate_dD_reduce");
  return 0;
}
