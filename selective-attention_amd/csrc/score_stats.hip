// Per-head statistics of the valid attention scores, for SelectiveMHA's
// training forward: the count, sum and sum of squares of
//   s_ij = scale * q_i . k_j
// over the valid (query i, key j) pairs of every batch row -- i inside the
// row's query length, j inside its key length and, for causal attention,
// j <= i.  The score matrix is never written: each tile of scores is reduced
// where the MFMA leaves it.
//
// Replaces the dense reductions of modules/selective_attention.py:234-246
// (self attention: query and key lengths both the row's length) and
// modules/cross_selective_attention.py:129-146 (cross attention: every
// query, keys inside the context length): valid mask, masked_fill,
// sum / square().sum() over batch, queries and keys.  The std and the
// running average stay with the caller.
//
// score_stats_kernel: one block per (batch row, head, 64-query block); wave
// w owns queries 16 w .. 16 w + 15 of the block.  Per 16-key tile, the K rows
// are the MFMA A operand and the wave's queries (kept in registers) the B
// operand, so a lane holds 4 keys of its own query.  fp32 inputs are split
// into bf16 hi + lo (products hi*hi + lo*hi + hi*lo).  Per-lane tile sums
// are fp32, running sums fp64; each block writes (count, sum, sum^2) and
// score_stats_reduce sums those in a fixed order (deterministic).
#include "common.h"
#include "prof.h"

namespace sa {

// 8 consecutive elements of a row as bf16 (hi) and the rounding remainder (lo)
__device__ __forceinline__ void load8_split(const bf16* p, bool ok, v8bf& hi, v8bf& lo) {
  hi = ok ? load_v8bf(p) : zero_v8bf();
  lo = zero_v8bf();
}
__device__ __forceinline__ void load8_split(const float* p, bool ok, v8bf& hi, v8bf& lo) {
  if (!ok) {
    hi = lo = zero_v8bf();
    return;
  }
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  split_p(v4f{a.x, a.y, a.z, a.w}, v4f{b.x, b.y, b.z, b.w}, hi, lo);
}

template <typename T, int D>
__global__ __launch_bounds__(256) void score_stats_kernel(const T* __restrict__ q,
                                                          const T* __restrict__ k,
                                                          const int64_t* __restrict__ q_length,
                                                          const int64_t* __restrict__ k_length,
                                                          int H, int Lq, int Lk, int causal,
                                                          float scale, double* __restrict__ part) {
  constexpr int KS = D / 32;
  constexpr bool SPLIT = sizeof(T) == 4;
  constexpr int TU = 4;   // 16-key tiles per step (loads issued together)
  __shared__ double red[4][3];
  const int nqb = (Lq + 63) / 64;
  const int qb = blockIdx.x % nqb;
  const int bh = blockIdx.x / nqb;
  const int b = bh / H;
  const int qlen = q_length ? static_cast<int>(min(max(q_length[b], int64_t{0}), int64_t{Lq})) : Lq;
  const int klen = k_length ? static_cast<int>(min(max(k_length[b], int64_t{0}), int64_t{Lk})) : Lk;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, li = lane & 15, lg = lane >> 4;
  const T* qh = q + static_cast<long>(bh) * Lq * D;
  const T* kh = k + static_cast<long>(bh) * Lk * D;
  const int qi = 64 * qb + 16 * w + li;   // this lane's query
  const bool qv = qi < qlen;

  v8bf qf[KS], ql[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    load8_split(qh + static_cast<long>(min(qi, Lq - 1)) * D + 32 * ks + 8 * lg, qv, qf[ks], ql[ks]);

  double s1 = 0.0, s2 = 0.0;
  int cnt = 0;
  // keys [0, kend): the row's key length, and for causal attention up to this block's last query
  const int kend = causal ? min(klen, 64 * qb + 64) : klen;
  for (int k0 = 0; k0 < kend; k0 += 16 * TU) {
    v8bf kf[TU][KS], kl[TU][KS];
#pragma unroll
    for (int u = 0; u < TU; ++u) {
      const int kr = k0 + 16 * u + li;   // the key row this lane supplies
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        load8_split(kh + static_cast<long>(min(kr, Lk - 1)) * D + 32 * ks + 8 * lg, kr < kend,
                    kf[u][ks], kl[u][ks]);
    }
#pragma unroll
    for (int u = 0; u < TU; ++u) {
      v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        acc = mfma_bf16(kf[u][ks], qf[ks], acc);
        if constexpr (SPLIT) {
          acc = mfma_bf16(kl[u][ks], qf[ks], acc);
          acc = mfma_bf16(kf[u][ks], ql[ks], acc);
        }
      }
      // acc[r]: key k0 + 16 u + 4 lg + r, query qi
      float t1 = 0.f, t2 = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = k0 + 16 * u + 4 * lg + r;
        const bool ok = qv && key < klen && (!causal || key <= qi);
        const float s = acc[r] * scale;
        t1 += ok ? s : 0.f;
        t2 += ok ? s * s : 0.f;
        cnt += ok ? 1 : 0;
      }
      s1 += t1;
      s2 += t2;
    }
  }
  double c = static_cast<double>(cnt);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    s1 += __shfl_xor(s1, o, 64);
    s2 += __shfl_xor(s2, o, 64);
    c += __shfl_xor(c, o, 64);
  }
  if (lane == 0) {
    red[w][0] = c;
    red[w][1] = s1;
    red[w][2] = s2;
  }
  __syncthreads();
  if (tid < 3) {
    double* out = part + (static_cast<long>(bh) * nqb + qb) * 3;
    out[tid] = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
  }
}

// out[h] = (count, sum, sum^2) over batch rows and query blocks of head h
__global__ __launch_bounds__(256) void score_stats_reduce_kernel(const double* __restrict__ part,
                                                                 int batch, int H, int nqb,
                                                                 double* __restrict__ out) {
  __shared__ double red[256][3];
  const int h = blockIdx.x, tid = threadIdx.x;
  double a[3] = {0.0, 0.0, 0.0};
  const int items = batch * nqb;
  for (int it = tid; it < items; it += 256) {
    const int b = it / nqb, qb = it % nqb;
    const double* p = part + ((static_cast<long>(b) * H + h) * nqb + qb) * 3;
    a[0] += p[0];
    a[1] += p[1];
    a[2] += p[2];
  }
#pragma unroll
  for (int i = 0; i < 3; ++i) red[tid][i] = a[i];
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s)
#pragma unroll
      for (int i = 0; i < 3; ++i) red[tid][i] += red[tid + s][i];
    __syncthreads();
  }
  if (tid < 3) out[h * 3 + tid] = red[0][tid];
}

template <typename T, int D>
int launch_score_stats(const void* q, const void* k, const int64_t* q_length, const int64_t* k_length,
                       int batch, int H, int Lq, int Lk, int causal, float scale, double* part,
                       double* out, hipStream_t s) {
  const int nqb = (Lq + 63) / 64;
  const long blocks = static_cast<long>(batch) * H * nqb;
  {
    ProfScope prof_("score_stats", s);
    hipLaunchKernelGGL((score_stats_kernel<T, D>), dim3(static_cast<unsigned>(blocks)), dim3(256),
                       0, s, static_cast<const T*>(q), static_cast<const T*>(k), q_length,
                       k_length, H, Lq, Lk, causal, scale, part);
    SA_CHECK_LAUNCH("score_stats");
  }
  ProfScope prof_("score_stats_reduce", s);
  hipLaunchKernelGGL(score_stats_reduce_kernel, dim3(H), dim3(256), 0, s, part, batch, H, nqb, out);
  SA_CHECK_LAUNCH("score_stats_reduce");
  return 0;
}

template <typename T>
int dispatch_score_stats(int D, const void* q, const void* k, const int64_t* q_length,
                         const int64_t* k_length, int batch, int H, int Lq, int Lk, int causal,
                         float scale, double* part, double* out, hipStream_t s) {
#define SA_SS(DD) \
  launch_score_stats<T, DD>(q, k, q_length, k_length, batch, H, Lq, Lk, causal, scale, part, out, s)
  switch (D) {
    case 32: return SA_SS(32);
    case 64: return SA_SS(64);
    case 96: return SA_SS(96);
    case 128: return SA_SS(128);
    default: break;
  }
#undef SA_SS
  sa_set_error("sa_score_stats: head_dim %d not supported (32, 64, 96, 128)", D);
  return 1;
}

}  // namespace sa

extern "C" size_t sa_score_stats_workspace_size(int batch, int heads, int q_len) {
  if (batch <= 0 || heads <= 0 || q_len <= 0) return 0;
  return static_cast<size_t>(batch) * heads * ((q_len + 63) / 64) * 3 * sizeof(double);
}

extern "C" int sa_score_stats(int dtype, const void* q, const void* k, const int64_t* q_length,
                              const int64_t* k_length, int batch, int heads, int q_len, int k_len,
                              int head_dim, int causal, float scale, void* workspace,
                              size_t workspace_bytes, double* out, void* stream) {
  SA_CHECK_ARG(batch >= 0 && heads > 0 && q_len >= 0 && k_len >= 0 && head_dim > 0,
               "sa_score_stats: bad sizes b=%d H=%d Lq=%d Lk=%d D=%d", batch, heads, q_len, k_len,
               head_dim);
  SA_CHECK_ARG(!causal || q_len == k_len, "sa_score_stats: causal needs q_len == k_len");
  SA_CHECK_ARG(q && k && out, "sa_score_stats: null tensor pointer");
  // the same checks for empty and non-empty calls: dtype and head_dim first
  SA_CHECK_ARG(dtype == sa::kBF16 || dtype == sa::kF32, "sa_score_stats: unsupported dtype %d",
               dtype);
  SA_CHECK_ARG(head_dim == 32 || head_dim == 64 || head_dim == 96 || head_dim == 128,
               "sa_score_stats: head_dim %d not supported (32, 64, 96, 128)", head_dim);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (batch == 0 || q_len == 0 || k_len == 0) {   // no pairs: the reduction writes zeros
    hipLaunchKernelGGL(sa::score_stats_reduce_kernel, dim3(heads), dim3(256), 0, s, nullptr, 0,
                       heads, 0, out);
    SA_CHECK_LAUNCH("score_stats_reduce");
    return 0;
  }
  const size_t need = sa_score_stats_workspace_size(batch, heads, q_len);
  SA_CHECK_ARG(workspace && workspace_bytes >= need,
               "sa_score_stats: workspace of %zu B, %zu B needed", workspace_bytes, need);
  SA_CHECK_ARG(((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k)) & 15) == 0,
               "sa_score_stats: q and k must be 16-byte aligned");
  double* part = static_cast<double*>(workspace);
  if (dtype == sa::kBF16)
    return sa::dispatch_score_stats<sa::bf16>(head_dim, q, k, q_length, k_length, batch, heads,
                                              q_len, k_len, causal, scale, part, out, s);
  if (dtype == sa::kF32)
    return sa::dispatch_score_stats<float>(head_dim, q, k, q_length, k_length, batch, heads, q_len,
                                           k_len, causal, scale, part, out, s);
  sa_set_error("sa_score_stats: unsupported dtype %d", dtype);
  return 1;
}
