// Model-side ops of the LMs around the mixers (gfx950): fused RMSNorm (alone
// and with the residual add before it), fused rotary embedding of q and k,
// SelectiveMHA's gate math, SwiGLU's gated product, and the paged KV-cache
// append of a decode step.
//
// Each replaces a chain of small torch kernels (RMSNorm: cast, square, mean,
// add, rsqrt, two multiplies, cast back; RoPE: slices, concatenation, cos,
// sin, multiplies, sum, cast; append: index arithmetic and three scatters),
// which at decode batch sizes are launch-bound.  All three are HBM streams
// (or tiny): one read and one write per element.
//
//   rms_norm   out = x * rsqrt(mean(x^2) + eps) * (1 + w[row % groups])
//              (modules/rms_norm.py:33-44), fp32 arithmetic, out in x's dtype.
//              One wave per row; the row is read twice, the second time from
//              cache.
//   rope       y = x cos(p f) + rotate_half(x) sin(p f), f the module's
//              inv_freq buffer (modules/rope.py:9-64), angles and products
//              in fp32 as the module computes them, y in bf16 (the attention
//              kernels' input).  Position of row r: positions[r % period],
//              or r % period when positions is null (prefill: r = b L + t).
//   paged_append  one token per batch row into its page (SelectiveAttnCache
//              update_kv, inference/selective_attn_cache.py:30-42): slot =
//              seq_lens[row], page = page_table[row][slot / page_size]; K
//              row-major per page, V transposed per page, the log-gate beside
//              them; then seq_lens[row] += 1.  One block per row.
#include "common.h"
#include "prof.h"

namespace sa {
namespace {

template <typename T>
__global__ __launch_bounds__(256) void rms_norm_kernel(const T* __restrict__ x,
                                                       const float* __restrict__ w,
                                                       T* __restrict__ out, long rows, int dim,
                                                       int groups, float eps) {
  const int lane = threadIdx.x & 63;
  const long row = static_cast<long>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * dim;
  T* orow = out + row * dim;
  float ss = 0.0f;
  for (int i = lane; i < dim; i += 64) {
    const float v = to_f32(xr[i]);
    ss += v * v;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  const float scale = 1.0f / sqrtf(ss / static_cast<float>(dim) + eps);
  const float* wr = w + static_cast<long>(row % groups) * dim;
  for (int i = lane; i < dim; i += 64) orow[i] = from_f32<T>(to_f32(xr[i]) * scale * (1.0f + wr[i]));
}

// 8-wide bf16 variant for dim % 512 == 0 (16-byte loads, 8 elements a lane a step)
__global__ __launch_bounds__(256) void rms_norm_bf16x8_kernel(const uint4* __restrict__ x,
                                                              const float* __restrict__ w,
                                                              uint4* __restrict__ out, long rows,
                                                              int dim, int groups, float eps) {
  const int lane = threadIdx.x & 63;
  const long row = static_cast<long>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nv = dim / 8;
  const uint4* xr = x + row * nv;
  uint4* orow = out + row * nv;
  float ss = 0.0f;
  for (int i = lane; i < nv; i += 64) {
    const uint4 q = xr[i];
    const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = bf16lo_to_f32(u[j]), b = bf16hi_to_f32(u[j]);
      ss += a * a + b * b;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  const float scale = 1.0f / sqrtf(ss / static_cast<float>(dim) + eps);
  const float* wr = w + static_cast<long>(row % groups) * dim;
  for (int i = lane; i < nv; i += 64) {
    const uint4 q = xr[i];
    const uint32_t u[4] = {q.x, q.y, q.z, q.w};
    uint32_t r[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float w0 = 1.0f + wr[8 * i + 2 * j], w1 = 1.0f + wr[8 * i + 2 * j + 1];
      r[j] = pack_bf16x2(bf16lo_to_f32(u[j]) * scale * w0, bf16hi_to_f32(u[j]) * scale * w1);
    }
    orow[i] = uint4{r[0], r[1], r[2], r[3]};
  }
}

// thread = (row, head, 4 consecutive pairs i .. i+3 of the half dimension)
template <typename T>
__global__ __launch_bounds__(256) void rope_kernel(const T* __restrict__ x0, const T* __restrict__ x1,
                                                   bf16* __restrict__ y0, bf16* __restrict__ y1,
                                                   long rows, int heads, int D,
                                                   const float* __restrict__ inv_freq,
                                                   const int64_t* __restrict__ positions, int period) {
  const int half = D / 2, quads = half / 4;
  const long per_tensor = rows * heads * quads;
  long id = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (id >= 2 * per_tensor) return;
  const bool second = id >= per_tensor;
  if (second) id -= per_tensor;
  const T* x = second ? x1 : x0;
  bf16* y = second ? y1 : y0;
  const int qd = static_cast<int>(id % quads);
  const long rh = id / quads;                 // row * heads + head
  const long row = rh / heads;
  const long pi = row % period;
  const float pos = positions ? static_cast<float>(positions[pi]) : static_cast<float>(pi);
  const T* xr = x + rh * D;
  bf16* yr = y + rh * D;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = 4 * qd + j;
    const float ang = pos * inv_freq[i];
    const float c = cosf(ang), s = sinf(ang);
    const float a = to_f32(xr[i]), b = to_f32(xr[i + half]);
    // x cos + rotate_half(x) sin with each product and the sum rounded to
    // fp32 on its own (no contraction to fma), as the module's torch ops do
    yr[i] = from_f32<bf16>(__fadd_rn(__fmul_rn(a, c), -__fmul_rn(b, s)));
    yr[i + half] = from_f32<bf16>(__fadd_rn(__fmul_rn(b, c), __fmul_rn(a, s)));
  }
}

__global__ __launch_bounds__(256) void paged_append_kernel(
    const bf16* __restrict__ k, const bf16* __restrict__ v, const float* __restrict__ log_gate,
    const int32_t* __restrict__ page_table, int32_t* __restrict__ seq_lens, int heads, int D,
    int ps, int max_pages, bf16* __restrict__ k_pages, bf16* __restrict__ v_pages,
    float* __restrict__ gate_pages) {
  const int row = blockIdx.x;
  const int t = seq_lens[row];
  const int col = min(t / ps, max_pages - 1);
  const long pid = page_table[static_cast<long>(row) * max_pages + col];
  const int s = t % ps;
  const int n = heads * D;
  for (int e = threadIdx.x; e < n; e += blockDim.x) {
    const int h = e / D, d = e - h * D;
    const long src = (static_cast<long>(row) * heads + h) * D + d;
    const long ph = pid * heads + h;
    k_pages[(ph * ps + s) * D + d] = k[src];
    v_pages[(ph * D + d) * ps + s] = v[src];
    if (d == 0) gate_pages[ph * ps + s] = log_gate[static_cast<long>(row) * heads + h];
  }
  __syncthreads();   // every thread has read seq_lens[row]
  if (threadIdx.x == 0) seq_lens[row] = t + 1;
}

// out = x + y (rounded to x's dtype), nrm = rms_norm(out): the residual add
// of a pre-norm block fused with the next norm.  bf16, dim % 512 == 0,
// dim <= 512 VPL; the row stays in registers between the two passes.
template <int VPL>
__global__ __launch_bounds__(256) void add_rms_norm_kernel(const uint4* __restrict__ x,
                                                           const uint4* __restrict__ y,
                                                           const float* __restrict__ w,
                                                           uint4* __restrict__ out,
                                                           uint4* __restrict__ nrm, long rows,
                                                           int dim, float eps) {
  const int lane = threadIdx.x & 63;
  const long row = static_cast<long>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nv = dim / 8;
  const long base = row * nv;
  uint32_t sv[VPL][4];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int i = lane + 64 * j;
    if (i < nv) {
      const uint4 a = x[base + i], c = y[base + i];
      const uint32_t ua[4] = {a.x, a.y, a.z, a.w}, uc[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        sv[j][q] = pack_bf16x2(bf16lo_to_f32(ua[q]) + bf16lo_to_f32(uc[q]),
                               bf16hi_to_f32(ua[q]) + bf16hi_to_f32(uc[q]));
        const float lo = bf16lo_to_f32(sv[j][q]), hi = bf16hi_to_f32(sv[j][q]);
        ss += lo * lo + hi * hi;
      }
      out[base + i] = uint4{sv[j][0], sv[j][1], sv[j][2], sv[j][3]};
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  const float scale = 1.0f / sqrtf(ss / static_cast<float>(dim) + eps);
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int i = lane + 64 * j;
    if (i < nv) {
      uint32_t r[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float w0 = 1.0f + w[8 * i + 2 * q], w1 = 1.0f + w[8 * i + 2 * q + 1];
        r[q] = pack_bf16x2(bf16lo_to_f32(sv[j][q]) * scale * w0, bf16hi_to_f32(sv[j][q]) * scale * w1);
      }
      nrm[base + i] = uint4{r[0], r[1], r[2], r[3]};
    }
  }
}

// SelectiveMHA's gates at a decode step: g = gate_proj output (rows, H + dim)
// bf16.  Columns < H: select gate s = bf16(sigmoid(g)); kept = s > 0 and
// s >= thr[h]; lg = kept ? log(s) * std[h] * penalty : -inf (fp32, (rows, H)).
// Columns >= H: the out gate bf16(sigmoid(g)) ((rows, dim)).
__global__ __launch_bounds__(256) void mha_gates_kernel(const bf16* __restrict__ g,
                                                        const float* __restrict__ thr,
                                                        const float* __restrict__ std_h,
                                                        float penalty, float* __restrict__ lg,
                                                        bf16* __restrict__ og, long rows, int H,
                                                        int dim) {
  const int W = H + dim;
  const long id = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (id >= rows * W) return;
  const long r = id / W;
  const int col = static_cast<int>(id - r * W);
  const float z = to_f32(g[id]);
  const float sg = to_f32(from_f32<bf16>(1.0f / (1.0f + expf(-z))));
  if (col < H) {
    const bool kept = sg > 0.0f && (thr == nullptr || sg >= thr[col]);
    lg[r * H + col] = kept ? __fmul_rn(__fmul_rn(logf(sg), std_h[col]), penalty) : -__builtin_huge_valf();
  } else {
    og[r * dim + (col - H)] = from_f32<bf16>(sg);
  }
}

// SwiGLU's gated product: out = bf16(a * bf16(silu(c))), all bf16
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint4* __restrict__ a,
                                                       const uint4* __restrict__ c,
                                                       uint4* __restrict__ out, long n8) {
  const long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n8) return;
  const uint4 qa = a[i], qc = c[i];
  const uint32_t ua[4] = {qa.x, qa.y, qa.z, qa.w}, uc[4] = {qc.x, qc.y, qc.z, qc.w};
  uint32_t r[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float c0 = bf16lo_to_f32(uc[q]), c1 = bf16hi_to_f32(uc[q]);
    const uint32_t s = pack_bf16x2(c0 / (1.0f + expf(-c0)), c1 / (1.0f + expf(-c1)));
    r[q] = pack_bf16x2(bf16lo_to_f32(ua[q]) * bf16lo_to_f32(s), bf16hi_to_f32(ua[q]) * bf16hi_to_f32(s));
  }
  out[i] = uint4{r[0], r[1], r[2], r[3]};
}

// y[m, n] = bf16(sum_k x[m, k] W[n, k] + bias[n]) for M <= 8 rows (decode),
// for up to kGemvSegs weight matrices of the same x in one launch (segment i:
// W_i (N_i, K), bias_i, its own contiguous output y_i (M, N_i); blocks
// blk0[i] .. blk0[i+1]-1 compute its columns).  A 256-thread block computes 4
// output columns, one per wave; x (M x K bf16) is staged in LDS once per
// block, optionally times xscale (M x K bf16) and rounded to bf16, i.e. the
// bf16 product x * xscale.  Lane l of a wave streams the 16-byte pieces
// k = 8 l + 512 j of W's row n (all of them issued before the first FMA,
// KP <= 8 pieces: K <= 4096), takes the matching x pieces from LDS, and the
// wave sums the M partials with xor shuffles.  fp32 accumulation.
constexpr int kGemvSegs = 4;
struct GemvSegs {
  const uint4* W[kGemvSegs];
  const bf16* bias[kGemvSegs];
  bf16* y[kGemvSegs];
  int N[kGemvSegs];
  int blk0[kGemvSegs + 1];
  int nseg;
};

__device__ __forceinline__ uint32_t mul_bf16x2(uint32_t a, uint32_t b) {
  return pack_bf16x2(bf16lo_to_f32(a) * bf16lo_to_f32(b), bf16hi_to_f32(a) * bf16hi_to_f32(b));
}

template <int M, int KP>
__global__ __launch_bounds__(256) void gemv_bf16_kernel(const uint4* __restrict__ x,
                                                        const uint4* __restrict__ xscale,
                                                        const GemvSegs sg, int K) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  uint4* xs = reinterpret_cast<uint4*>(smem_raw);   // [M][K / 8]
  const int kv = K / 8;
  for (int e = threadIdx.x; e < M * kv; e += 256) {
    uint4 v = x[e];
    if (xscale) {
      const uint4 g = xscale[e];
      v = uint4{mul_bf16x2(v.x, g.x), mul_bf16x2(v.y, g.y), mul_bf16x2(v.z, g.z), mul_bf16x2(v.w, g.w)};
    }
    xs[e] = v;
  }
  // this block's segment (block-uniform)
  const int bid = blockIdx.x;
  int seg = 0;
#pragma unroll
  for (int i = 1; i < kGemvSegs; ++i) seg += (i < sg.nseg && bid >= sg.blk0[i]) ? 1 : 0;
  const int N = sg.N[seg];
  const int lane = threadIdx.x & 63;
  const int n = (bid - sg.blk0[seg]) * 4 + (threadIdx.x >> 6);
  const int nr = min(n, N - 1);
  const uint4* wr = sg.W[seg] + static_cast<long>(nr) * kv;
  uint4 wq[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    const int p = lane + 64 * j;
    wq[j] = p < kv ? wr[p] : uint4{0u, 0u, 0u, 0u};
  }
  __syncthreads();
  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.0f;
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    const int p = lane + 64 * j;
    if (p >= kv) break;
    const uint32_t wu[4] = {wq[j].x, wq[j].y, wq[j].z, wq[j].w};
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint4 xq = xs[m * kv + p];
      const uint32_t xu[4] = {xq.x, xq.y, xq.z, xq.w};
#pragma unroll
      for (int q = 0; q < 4; ++q)
        acc[m] += bf16lo_to_f32(xu[q]) * bf16lo_to_f32(wu[q]) + bf16hi_to_f32(xu[q]) * bf16hi_to_f32(wu[q]);
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc[m] += __shfl_xor(acc[m], o, 64);
  }
  if (lane < M && n < N) {
    float v = acc[0];
#pragma unroll
    for (int m = 1; m < M; ++m) v = lane == m ? acc[m] : v;
    const bf16* bias = sg.bias[seg];
    const float bv = bias ? to_f32(bias[n]) : 0.0f;
    sg.y[seg][static_cast<long>(lane) * N + n] = from_f32<bf16>(v + bv);
  }
}

}  // namespace
}  // namespace sa

namespace sa {
namespace {
template <int M>
void launch_gemv(const uint4* x, const uint4* xscale, const GemvSegs& sg, int K, hipStream_t s) {
  const dim3 grid(sg.blk0[sg.nseg]);
  const size_t smem = static_cast<size_t>(M) * K * 2;   // <= 64 KB (M <= 8, K <= 4096)
  const int kp = (K / 8 + 63) / 64;                      // 16-byte pieces per lane
  if (kp <= 2)
    hipLaunchKernelGGL((gemv_bf16_kernel<M, 2>), grid, dim3(256), smem, s, x, xscale, sg, K);
  else if (kp <= 4)
    hipLaunchKernelGGL((gemv_bf16_kernel<M, 4>), grid, dim3(256), smem, s, x, xscale, sg, K);
  else
    hipLaunchKernelGGL((gemv_bf16_kernel<M, 8>), grid, dim3(256), smem, s, x, xscale, sg, K);
}

int gemv_run(const char* who, const void* x, const void* xscale, int M, int K, int nseg,
             const void* const* W, const void* const* bias, const int* N, void* const* y,
             void* stream) {
  SA_CHECK_ARG(M >= 1 && M <= 8 && K > 0 && K % 8 == 0 && K <= 4096,
               "%s: M %d must be 1..8 and K %d a multiple of 8, at most 4096", who, M, K);
  SA_CHECK_ARG(nseg >= 1 && nseg <= kGemvSegs, "%s: %d weight matrices, 1..%d allowed", who, nseg,
               kGemvSegs);
  SA_CHECK_ARG(x && W && N && y, "%s: null pointer", who);
  SA_CHECK_ARG(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(xscale)) & 15) == 0,
               "%s: x and xscale must be 16-byte aligned", who);
  GemvSegs sg{};
  sg.nseg = nseg;
  sg.blk0[0] = 0;
  for (int i = 0; i < nseg; ++i) {
    SA_CHECK_ARG(W[i] && y[i] && N[i] > 0, "%s: weight matrix %d: null pointer or N %d", who, i,
                 N[i]);
    SA_CHECK_ARG((reinterpret_cast<uintptr_t>(W[i]) & 15) == 0, "%s: W %d must be 16-byte aligned",
                 who, i);
    SA_CHECK_ARG(sg.blk0[i] + (N[i] + 3) / 4 < (1 << 30), "%s: too many columns", who);
    sg.W[i] = static_cast<const uint4*>(W[i]);
    sg.bias[i] = bias ? static_cast<const bf16*>(bias[i]) : nullptr;
    sg.y[i] = static_cast<bf16*>(y[i]);
    sg.N[i] = N[i];
    sg.blk0[i + 1] = sg.blk0[i] + (N[i] + 3) / 4;
  }
  for (int i = nseg; i < kGemvSegs; ++i) sg.blk0[i + 1] = sg.blk0[nseg];
  hipStream_t s = static_cast<hipStream_t>(stream);
  ProfScope prof_("gemv", s);
  const uint4* xv = static_cast<const uint4*>(x);
  const uint4* gv = static_cast<const uint4*>(xscale);
  switch (M) {
    case 1: launch_gemv<1>(xv, gv, sg, K, s); break;
    case 2: launch_gemv<2>(xv, gv, sg, K, s); break;
    case 3: launch_gemv<3>(xv, gv, sg, K, s); break;
    case 4: launch_gemv<4>(xv, gv, sg, K, s); break;
    case 5: launch_gemv<5>(xv, gv, sg, K, s); break;
    case 6: launch_gemv<6>(xv, gv, sg, K, s); break;
    case 7: launch_gemv<7>(xv, gv, sg, K, s); break;
    default: launch_gemv<8>(xv, gv, sg, K, s); break;
  }
  SA_CHECK_LAUNCH(who);
  return 0;
}
}  // namespace
}  // namespace sa

extern "C" int sa_gemv_bf16(const void* x, const void* W, const void* bias, int M, int N, int K,
                            void* y, void* stream) {
  return sa::gemv_run("sa_gemv_bf16", x, nullptr, M, K, 1, &W, &bias, &N, &y, stream);
}

extern "C" int sa_gemv_bf16_multi(const void* x, const void* xscale, int M, int K, int nseg,
                                  const void* const* W, const void* const* bias, const int* N,
                                  void* const* y, void* stream) {
  return sa::gemv_run("sa_gemv_bf16_multi", x, xscale, M, K, nseg, W, bias, N, y, stream);
}

extern "C" int sa_add_rms_norm_bf16(const void* x, const void* y, const float* weight, long rows,
                                    int dim, float eps, void* out, void* nrm, void* stream) {
  SA_CHECK_ARG(rows >= 0 && dim > 0 && dim % 512 == 0 && dim <= 4096,
               "sa_add_rms_norm_bf16: dim %d must be a multiple of 512, at most 4096", dim);
  SA_CHECK_ARG(x && y && weight && out && nrm, "sa_add_rms_norm_bf16: null pointer");
  SA_CHECK_ARG(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y) |
                 reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(nrm)) & 15) == 0,
               "sa_add_rms_norm_bf16: tensors must be 16-byte aligned");
  if (rows == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const long blocks = (rows + 3) / 4;
  sa::ProfScope prof_("add_rms_norm", s);
  const int vpl = dim / 512;
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), 0, s, static_cast<const uint4*>(x),
                       static_cast<const uint4*>(y), weight, static_cast<uint4*>(out),
                       static_cast<uint4*>(nrm), rows, dim, eps);
  };
  if (vpl <= 2) go(sa::add_rms_norm_kernel<2>);
  else if (vpl <= 4) go(sa::add_rms_norm_kernel<4>);
  else go(sa::add_rms_norm_kernel<8>);
  SA_CHECK_LAUNCH("add_rms_norm");
  return 0;
}

extern "C" int sa_mha_gates_bf16(const void* g, const float* thr, const float* score_std,
                                 float penalty, long rows, int heads, int dim, float* log_gate,
                                 void* out_gate, void* stream) {
  SA_CHECK_ARG(rows >= 0 && heads > 0 && dim > 0, "sa_mha_gates_bf16: bad sizes");
  SA_CHECK_ARG(g && score_std && log_gate && out_gate, "sa_mha_gates_bf16: null pointer");
  if (rows == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const long n = rows * (heads + dim);
  sa::ProfScope prof_("mha_gates", s);
  hipLaunchKernelGGL(sa::mha_gates_kernel, dim3((n + 255) / 256), dim3(256), 0, s,
                     static_cast<const sa::bf16*>(g), thr, score_std, penalty, log_gate,
                     static_cast<sa::bf16*>(out_gate), rows, heads, dim);
  SA_CHECK_LAUNCH("mha_gates");
  return 0;
}

extern "C" int sa_silu_mul_bf16(const void* a, const void* c, long n, void* out, void* stream) {
  SA_CHECK_ARG(n >= 0 && n % 8 == 0, "sa_silu_mul_bf16: n %ld must be a multiple of 8", n);
  SA_CHECK_ARG(a && c && out, "sa_silu_mul_bf16: null pointer");
  SA_CHECK_ARG(((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(c) |
                 reinterpret_cast<uintptr_t>(out)) & 15) == 0,
               "sa_silu_mul_bf16: tensors must be 16-byte aligned");
  if (n == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const long n8 = n / 8;
  sa::ProfScope prof_("silu_mul", s);
  hipLaunchKernelGGL(sa::silu_mul_kernel, dim3((n8 + 255) / 256), dim3(256), 0, s,
                     static_cast<const uint4*>(a), static_cast<const uint4*>(c),
                     static_cast<uint4*>(out), n8);
  SA_CHECK_LAUNCH("silu_mul");
  return 0;
}

extern "C" int sa_rms_norm_fwd(int dtype, const void* x, const float* weight, long rows, int dim,
                               int groups, float eps, void* out, void* stream) {
  SA_CHECK_ARG(dtype == sa::kF32 || dtype == sa::kBF16, "sa_rms_norm_fwd: dtype %d", dtype);
  SA_CHECK_ARG(rows >= 0 && dim > 0 && groups > 0, "sa_rms_norm_fwd: bad sizes");
  SA_CHECK_ARG(x && weight && out, "sa_rms_norm_fwd: null pointer");
  if (rows == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const long blocks = (rows + 3) / 4;
  sa::ProfScope prof_("rms_norm", s);
  if (dtype == sa::kBF16 && dim % 512 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(out) & 15) == 0) {
    hipLaunchKernelGGL(sa::rms_norm_bf16x8_kernel, dim3(blocks), dim3(256), 0, s,
                       static_cast<const uint4*>(x), weight, static_cast<uint4*>(out), rows, dim,
                       groups, eps);
  } else if (dtype == sa::kBF16) {
    hipLaunchKernelGGL(sa::rms_norm_kernel<sa::bf16>, dim3(blocks), dim3(256), 0, s,
                       static_cast<const sa::bf16*>(x), weight, static_cast<sa::bf16*>(out), rows,
                       dim, groups, eps);
  } else {
    hipLaunchKernelGGL(sa::rms_norm_kernel<float>, dim3(blocks), dim3(256), 0, s,
                       static_cast<const float*>(x), weight, static_cast<float*>(out), rows, dim,
                       groups, eps);
  }
  SA_CHECK_LAUNCH("rms_norm");
  return 0;
}

extern "C" int sa_rope_bf16(int dtype, const void* x0, const void* x1, void* y0, void* y1,
                            long rows, int heads, int head_dim, const float* inv_freq,
                            const int64_t* positions, int period, void* stream) {
  SA_CHECK_ARG(dtype == sa::kF32 || dtype == sa::kBF16, "sa_rope_bf16: dtype %d", dtype);
  SA_CHECK_ARG(rows >= 0 && heads > 0 && head_dim > 0 && head_dim % 8 == 0 && period > 0,
               "sa_rope_bf16: bad sizes (head_dim must be a multiple of 8)");
  SA_CHECK_ARG(x0 && x1 && y0 && y1 && inv_freq, "sa_rope_bf16: null pointer");
  if (rows == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const long threads = 2 * rows * heads * (head_dim / 8);
  const long blocks = (threads + 255) / 256;
  sa::ProfScope prof_("rope", s);
  if (dtype == sa::kBF16) {
    hipLaunchKernelGGL(sa::rope_kernel<sa::bf16>, dim3(blocks), dim3(256), 0, s,
                       static_cast<const sa::bf16*>(x0), static_cast<const sa::bf16*>(x1),
                       static_cast<sa::bf16*>(y0), static_cast<sa::bf16*>(y1), rows, heads, head_dim,
                       inv_freq, positions, period);
  } else {
    hipLaunchKernelGGL(sa::rope_kernel<float>, dim3(blocks), dim3(256), 0, s,
                       static_cast<const float*>(x0), static_cast<const float*>(x1),
                       static_cast<sa::bf16*>(y0), static_cast<sa::bf16*>(y1), rows, heads, head_dim,
                       inv_freq, positions, period);
  }
  SA_CHECK_LAUNCH("rope");
  return 0;
}

namespace sa {
namespace {
// Paged cache build after prefill.  Block (page slot j of row r, head h)
// writes the K page [ps][D], the V page transposed [D][ps] (through an LDS
// tile) and the gate page [ps] of tokens j ps .. j ps + ps - 1 of row r:
// zero K / V and a -inf gate past the row's length.  k / v element strides
// (batch, token, head; D contiguous) and log_gate strides (batch, head, token).
__global__ __launch_bounds__(256) void paged_build_kernel(
    const bf16* __restrict__ k, const bf16* __restrict__ v, long sb, long st, long sh,
    const float* __restrict__ lg, long gb, long gh, long gt, const int32_t* __restrict__ page_table,
    const int32_t* __restrict__ seq_lens, int H, int D, int ps, int max_pages,
    bf16* __restrict__ k_pages, bf16* __restrict__ v_pages, float* __restrict__ gate_pages) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  bf16* tile = reinterpret_cast<bf16*>(smem_raw);   // [ps][D + 8] V rows of the page
  const int LDT = D + 8;
  const int r = blockIdx.x / max_pages, j = blockIdx.x % max_pages, h = blockIdx.y;
  const int n = seq_lens[r];
  const int t0 = j * ps;
  if (t0 >= n) return;   // block-uniform: this page slot holds no token of the row
  const long pg = (static_cast<long>(page_table[r * max_pages + j]) * H + h) * ps * D;
  const bf16* kr = k + r * sb + h * sh;
  const bf16* vr = v + r * sb + h * sh;
  const int dv = D / 8;
  for (int e = threadIdx.x; e < ps * dv; e += 256) {
    const int sl = e / dv, c8 = e % dv, t = t0 + sl;
    uint4 kq = uint4{0u, 0u, 0u, 0u}, vq = uint4{0u, 0u, 0u, 0u};
    if (t < n) {
      kq = *reinterpret_cast<const uint4*>(kr + t * st + 8 * c8);
      vq = *reinterpret_cast<const uint4*>(vr + t * st + 8 * c8);
    }
    *reinterpret_cast<uint4*>(k_pages + pg + static_cast<long>(sl) * D + 8 * c8) = kq;
    *reinterpret_cast<uint4*>(tile + sl * LDT + 8 * c8) = vq;
  }
  const float* gr = lg + r * gb + h * gh;
  float* gp = gate_pages + (pg / D);
  for (int sl = threadIdx.x; sl < ps; sl += 256) gp[sl] = t0 + sl < n ? gr[(t0 + sl) * gt] : -__builtin_inff();
  __syncthreads();
  // V^T: eight consecutive slots of one d row per thread
  const int s8n = ps / 8;
  for (int e = threadIdx.x; e < D * s8n; e += 256) {
    const int d = e / s8n, s8 = e % s8n;
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = tile[(8 * s8 + 2 * i) * LDT + d].x, hi = tile[(8 * s8 + 2 * i + 1) * LDT + d].x;
      w[i] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(v_pages + pg + static_cast<long>(d) * ps + 8 * s8) = uint4{w[0], w[1], w[2], w[3]};
  }
}
}  // namespace
}  // namespace sa

extern "C" int sa_paged_kv_build(const void* k, const void* v, long sb, long st, long sh,
                                 const float* log_gate, long gb, long gh, long gt,
                                 const int32_t* page_table, const int32_t* seq_lens, int batch,
                                 int heads, int head_dim, int page_size, int max_pages,
                                 void* k_pages, void* v_pages, float* gate_pages, void* stream) {
  SA_CHECK_ARG(batch >= 0 && heads > 0 && head_dim > 0 && head_dim % 8 == 0 && head_dim <= 256 &&
                   page_size > 0 && page_size % 8 == 0 && max_pages > 0 &&
                   static_cast<long>(page_size) * (head_dim + 8) * 2 <= 64 * 1024,
               "sa_paged_kv_build: bad sizes batch=%d heads=%d head_dim=%d page_size=%d max_pages=%d",
               batch, heads, head_dim, page_size, max_pages);
  SA_CHECK_ARG(k && v && log_gate && page_table && seq_lens && k_pages && v_pages && gate_pages,
               "sa_paged_kv_build: null pointer");
  SA_CHECK_ARG(((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15) == 0 &&
                   sb % 8 == 0 && st % 8 == 0 && sh % 8 == 0,
               "sa_paged_kv_build: k / v and their strides must keep 16-byte alignment");
  if (batch == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  sa::ProfScope prof_("paged_build", s);
  const size_t smem = static_cast<size_t>(page_size) * (head_dim + 8) * 2;
  hipLaunchKernelGGL(sa::paged_build_kernel, dim3(batch * max_pages, heads), dim3(256), smem, s,
                     static_cast<const sa::bf16*>(k), static_cast<const sa::bf16*>(v), sb, st, sh,
                     log_gate, gb, gh, gt, page_table, seq_lens, heads, head_dim, page_size,
                     max_pages, static_cast<sa::bf16*>(k_pages), static_cast<sa::bf16*>(v_pages),
                     gate_pages);
  SA_CHECK_LAUNCH("paged_build");
  return 0;
}

extern "C" int sa_paged_kv_append(const void* k, const void* v, const float* log_gate,
                                  const int32_t* page_table, int32_t* seq_lens, int batch,
                                  int heads, int head_dim, int page_size, int max_pages,
                                  void* k_pages, void* v_pages, float* gate_pages, void* stream) {
  SA_CHECK_ARG(batch >= 0 && heads > 0 && head_dim > 0 && page_size > 0 && max_pages > 0,
               "sa_paged_kv_append: bad sizes");
  SA_CHECK_ARG(k && v && log_gate && page_table && seq_lens && k_pages && v_pages && gate_pages,
               "sa_paged_kv_append: null pointer");
  if (batch == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  sa::ProfScope prof_("paged_append", s);
  hipLaunchKernelGGL(sa::paged_append_kernel, dim3(batch), dim3(256), 0, s,
                     static_cast<const sa::bf16*>(k), static_cast<const sa::bf16*>(v), log_gate,
                     page_table, seq_lens, heads, head_dim, page_size, max_pages,
                     static_cast<sa::bf16*>(k_pages), static_cast<sa::bf16*>(v_pages), gate_pages);
  SA_CHECK_LAUNCH("paged_append");
  return 0;
}
