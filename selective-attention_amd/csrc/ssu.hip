// Single-step selective state update (decode), gfx950.
//
//   dt = clamp(softplus20(delta_raw + bias))
//   h  <- h * exp(A * dt) + dt * u (x) B          (in place, fp32 state)
//   y  = h . C                                     (dtype of u)
//
// Replaces ssu_forward / ssu_forward_kernel
// (triton_kernels/ssu/forward.py:7-63, ssu/forward_kernel.py:6-79).
//
// Pure HBM stream: the state (b, H, P, N) fp32 is read and written once.
// Shapes with P and N multiples of 32 run ssu_head_kernel (one block per
// batch row, head and range of state rows, sharing dt, the decay and B / C);
// others run ssu_fwd_kernel, where a row (b, h, p) of N states is owned by
// ROW_LANES lanes holding float4 strips and ROWS rows per thread are issued
// back to back.  y is a segmented lane reduction (xor shuffles inside the row
// group).
#include "common.h"
#include "prof.h"

constexpr int kSsuStrips = 8;   // float4 of state per thread in the per-head kernel

namespace sa {

template <typename T, int ROW_LANES, int ROWS, bool GATED>
__global__ __launch_bounds__(256) void ssu_fwd_kernel(
    const T* __restrict__ u, const float* __restrict__ A, const T* __restrict__ Bm,
    const T* __restrict__ Cm, const T* __restrict__ delta_raw, const float* __restrict__ delta_bias,
    float* __restrict__ h, T* __restrict__ y, const float* __restrict__ Dskip,
    const T* __restrict__ gate, int batch, int H, int P, int G, int N, int softplus, float dmin,
    float dmax, int vec4) {
  constexpr int kRowsPerBlock = (256 / ROW_LANES) * ROWS;
  const int lane_in_row = threadIdx.x % ROW_LANES;
  const int row_slot = threadIdx.x / ROW_LANES;  // 0 .. 256/ROW_LANES-1
  const long total_rows = static_cast<long>(batch) * H * P;
  const int hpg = H / G;

#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const long row = static_cast<long>(blockIdx.x) * kRowsPerBlock + r * (256 / ROW_LANES) + row_slot;
    // rows beyond the end still take part in the shuffles below (with zeros)
    const bool valid = row < total_rows;
    const long rr = valid ? row : 0;
    const int p = static_cast<int>(rr % P);
    const long bh = rr / P;
    const int hh = static_cast<int>(bh % H);
    const int bb = static_cast<int>(bh / H);
    const int g = hh / hpg;

    float z = load_f32(delta_raw + static_cast<long>(bb) * H + hh);
    if (delta_bias) z += delta_bias[hh];
    const float dt = make_dt(z, softplus != 0, dmin, dmax);
    const float decay = expf(A[hh] * dt);
    const float du = dt * load_f32(u + (static_cast<long>(bb) * H + hh) * P + p);

    const T* Brow = Bm + (static_cast<long>(bb) * G + g) * N;
    const T* Crow = Cm + (static_cast<long>(bb) * G + g) * N;
    float* hrow = h + rr * N;

    float part = 0.f;
    if (vec4) {
      for (int n = 4 * lane_in_row; n < N; n += 4 * ROW_LANES) {
        if (!valid) break;
        float4 hv = ld_nt(reinterpret_cast<const float4*>(hrow + n));
        float b0 = load_f32(Brow + n), b1 = load_f32(Brow + n + 1), b2 = load_f32(Brow + n + 2), b3 = load_f32(Brow + n + 3);
        float c0 = load_f32(Crow + n), c1 = load_f32(Crow + n + 1), c2 = load_f32(Crow + n + 2), c3 = load_f32(Crow + n + 3);
        hv.x = hv.x * decay + du * b0;
        hv.y = hv.y * decay + du * b1;
        hv.z = hv.z * decay + du * b2;
        hv.w = hv.w * decay + du * b3;
        st_nt(reinterpret_cast<float4*>(hrow + n), hv);
        part += hv.x * c0 + hv.y * c1 + hv.z * c2 + hv.w * c3;
      }
    } else {
      for (int n = lane_in_row; n < N; n += ROW_LANES) {
        if (!valid) break;
        const float hv = __builtin_nontemporal_load(hrow + n) * decay + du * load_f32(Brow + n);
        __builtin_nontemporal_store(hv, hrow + n);
        part += hv * load_f32(Crow + n);
      }
    }
#pragma unroll
    for (int o = ROW_LANES / 2; o > 0; o >>= 1) part += __shfl_xor(part, o, 64);
    if (valid && lane_in_row == 0) {
      if constexpr (GATED) {
        // SSM block epilogue on y rounded to T: (y + D u) silu(gate), as the gate kernel
        const float yv = to_f32(from_f32<T>(part));
        const float xv = load_f32(u + rr);
        const float gv = load_f32(gate + rr);
        st(y + rr, (yv + Dskip[hh * P + p] * xv) * (gv * fast_sigmoid(gv)));
      } else {
        st(y + rr, part);
      }
    }
  }
}

// Four values of B or C at n (n a multiple of 4, the row 8-byte aligned for
// bf16 and 16-byte aligned for fp32), kept in their storage type until used.
template <typename T> struct Quad;
template <> struct Quad<bf16> {
  uint2 q;
  __device__ __forceinline__ void load(const bf16* p) { q = *reinterpret_cast<const uint2*>(p); }
  __device__ __forceinline__ float operator[](int i) const {
    const uint32_t w = i < 2 ? q.x : q.y;
    return (i & 1) ? bf16hi_to_f32(w) : bf16lo_to_f32(w);
  }
};
template <> struct Quad<float> {
  float4 q;
  __device__ __forceinline__ void load(const float* p) { q = *reinterpret_cast<const float4*>(p); }
  __device__ __forceinline__ float operator[](int i) const {
    return i == 0 ? q.x : i == 1 ? q.y : i == 2 ? q.z : q.w;
  }
};

// One block per (batch row, head, range of 32 PASSES state rows): the rows
// share dt, the decay and the B / C rows, loaded once per thread.  A row of N
// states is owned by 8 lanes, each holding VPL float4 strips (n = 4 lane +
// 32 i), and a thread owns PASSES rows (p = p0 + 32 pass + thread / 8): all of
// its state loads are issued before any arithmetic.  Plain (cached) loads and
// stores: on this in-place read-modify-write they measured faster than the
// non-temporal forms.
template <typename T, int VPL, int PASSES, bool GATED>
__global__ __launch_bounds__(256) void ssu_head_kernel(
    const T* __restrict__ u, const float* __restrict__ A, const T* __restrict__ Bm,
    const T* __restrict__ Cm, const T* __restrict__ delta_raw, const float* __restrict__ delta_bias,
    float* __restrict__ h, T* __restrict__ y, const float* __restrict__ Dskip,
    const T* __restrict__ gate, int H, int P, int G, int softplus, float dmin, float dmax) {
  constexpr int N = 32 * VPL;
  const int nrb = P / (32 * PASSES);              // row ranges per (batch row, head)
  const int bh = blockIdx.x / nrb, p0 = (blockIdx.x % nrb) * (32 * PASSES);
  const int hh = bh % H, bb = bh / H, g = hh / (H / G);
  const int li = threadIdx.x & 7, slot = threadIdx.x >> 3;
  float* hb = h + (static_cast<long>(bh) * P + p0) * N + 4 * li;

  float4 hv[PASSES][VPL];
#pragma unroll
  for (int r = 0; r < PASSES; ++r)
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      hv[r][i] = *reinterpret_cast<const float4*>(hb + (32 * r + slot) * N + 32 * i);

  float z = load_f32(delta_raw + bh);
  if (delta_bias) z += delta_bias[hh];
  const float dt = make_dt(z, softplus != 0, dmin, dmax);
  const float decay = expf(A[hh] * dt);
  const T* Brow = Bm + (static_cast<long>(bb) * G + g) * N + 4 * li;
  const T* Crow = Cm + (static_cast<long>(bb) * G + g) * N + 4 * li;
  Quad<T> bv[VPL], cv[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    bv[i].load(Brow + 32 * i);
    cv[i].load(Crow + 32 * i);
  }
  float part[PASSES];
#pragma unroll
  for (int r = 0; r < PASSES; ++r) {
    const int p = 32 * r + slot;   // relative to p0
    const float du = dt * load_f32(u + static_cast<long>(bh) * P + p0 + p);
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      float4 v = hv[r][i];
      v.x = v.x * decay + du * bv[i][0];
      v.y = v.y * decay + du * bv[i][1];
      v.z = v.z * decay + du * bv[i][2];
      v.w = v.w * decay + du * bv[i][3];
      *reinterpret_cast<float4*>(hb + p * N + 32 * i) = v;
      acc += v.x * cv[i][0] + v.y * cv[i][1] + v.z * cv[i][2] + v.w * cv[i][3];
    }
    part[r] = acc;
  }
#pragma unroll
  for (int r = 0; r < PASSES; ++r) {
    float v = part[r];
    v += __shfl_xor(v, 4, 64);
    v += __shfl_xor(v, 2, 64);
    v += __shfl_xor(v, 1, 64);
    if (li == 0) {
      const long row = static_cast<long>(bh) * P + p0 + 32 * r + slot;
      if constexpr (GATED) {
        // SSM block epilogue on y rounded to T: (y + D u) silu(gate), as the gate kernel
        const float yv = to_f32(from_f32<T>(v));
        const float xv = load_f32(u + row);
        const float gv = load_f32(gate + row);
        st(y + row, (yv + Dskip[hh * P + p0 + 32 * r + slot] * xv) * (gv * fast_sigmoid(gv)));
      } else {
        st(y + row, v);
      }
    }
  }
}

template <typename T, int VPL, int PASSES>
static int launch_ssu_head(const void* u, const float* A, const void* B, const void* C,
                           const void* delta_raw, const float* delta_bias, float* h, void* y,
                           const float* Dskip, const void* gate, int batch, int H, int P, int G,
                           int softplus, float dmin, float dmax, hipStream_t stream) {
  const long blocks = static_cast<long>(batch) * H * (P / (32 * PASSES));
  if (blocks == 0) return 0;
  ProfScope prof_(gate ? "ssu_fwd_gated" : "ssu_fwd", stream);
  if (gate)
    hipLaunchKernelGGL((ssu_head_kernel<T, VPL, PASSES, true>), dim3(static_cast<unsigned>(blocks)),
                       dim3(256), 0, stream, static_cast<const T*>(u), A, static_cast<const T*>(B),
                       static_cast<const T*>(C), static_cast<const T*>(delta_raw), delta_bias, h,
                       static_cast<T*>(y), Dskip, static_cast<const T*>(gate), H, P, G, softplus,
                       dmin, dmax);
  else
    hipLaunchKernelGGL((ssu_head_kernel<T, VPL, PASSES, false>), dim3(static_cast<unsigned>(blocks)),
                       dim3(256), 0, stream, static_cast<const T*>(u), A, static_cast<const T*>(B),
                       static_cast<const T*>(C), static_cast<const T*>(delta_raw), delta_bias, h,
                       static_cast<T*>(y), nullptr, nullptr, H, P, G, softplus, dmin, dmax);
  SA_CHECK_LAUNCH(gate ? "ssu_fwd_gated" : "ssu_fwd");
  return 0;
}

template <typename T, int ROW_LANES>
static int launch_ssu(const void* u, const float* A, const void* B, const void* C,
                      const void* delta_raw, const float* delta_bias, float* h, void* y,
                      const float* Dskip, const void* gate, int batch, int H, int P, int G, int N,
                      int softplus, float dmin, float dmax, hipStream_t stream) {
  constexpr int ROWS = 2;
  constexpr int kRowsPerBlock = (256 / ROW_LANES) * ROWS;
  const long total_rows = static_cast<long>(batch) * H * P;
  const long blocks = (total_rows + kRowsPerBlock - 1) / kRowsPerBlock;
  if (blocks == 0) return 0;
  ProfScope prof_(gate ? "ssu_fwd_gated" : "ssu_fwd", stream);
  const int vec4 = (N % 4 == 0 && (reinterpret_cast<uintptr_t>(h) & 15) == 0) ? 1 : 0;
  if (gate)
    hipLaunchKernelGGL((ssu_fwd_kernel<T, ROW_LANES, ROWS, true>), dim3(static_cast<unsigned>(blocks)),
                       dim3(256), 0, stream, static_cast<const T*>(u), A, static_cast<const T*>(B),
                       static_cast<const T*>(C), static_cast<const T*>(delta_raw), delta_bias, h,
                       static_cast<T*>(y), Dskip, static_cast<const T*>(gate), batch, H, P, G, N,
                       softplus, dmin, dmax, vec4);
  else
    hipLaunchKernelGGL((ssu_fwd_kernel<T, ROW_LANES, ROWS, false>), dim3(static_cast<unsigned>(blocks)),
                       dim3(256), 0, stream, static_cast<const T*>(u), A, static_cast<const T*>(B),
                       static_cast<const T*>(C), static_cast<const T*>(delta_raw), delta_bias, h,
                       static_cast<T*>(y), nullptr, nullptr, batch, H, P, G, N, softplus, dmin,
                       dmax, vec4);
  SA_CHECK_LAUNCH(gate ? "ssu_fwd_gated" : "ssu_fwd");
  return 0;
}

template <typename T>
static int dispatch_ssu(const void* u, const float* A, const void* B, const void* C,
                        const void* delta_raw, const float* delta_bias, float* h, void* y,
                        const float* Dskip, const void* gate, int batch, int H, int P, int G,
                        int N, int softplus, float dmin, float dmax, hipStream_t stream) {
  // per-head blocks: N = 32 VPL (VPL 1, 2, 4), P a multiple of 32, aligned rows;
  // PASSES rows per thread so that a thread holds kSsuStrips float4 of state
  const uintptr_t ba = reinterpret_cast<uintptr_t>(B) | reinterpret_cast<uintptr_t>(C);
  const bool head_ok = (reinterpret_cast<uintptr_t>(h) & 15) == 0 &&
                       (ba & (sizeof(T) == 2 ? 7 : 15)) == 0 && P % 32 == 0 && N % 32 == 0;
  if (head_ok) {
    const int vpl = N / 32;
    int passes = 1;
    while (passes * 2 * vpl <= kSsuStrips && P % (64 * passes) == 0) passes *= 2;
#define SA_SSU_HEAD(V, R)                                                                   \
  if (vpl == V && passes == R)                                                              \
    return launch_ssu_head<T, V, R>(u, A, B, C, delta_raw, delta_bias, h, y, Dskip, gate, \
                                    batch, H, P, G, softplus, dmin, dmax, stream);
    SA_SSU_HEAD(1, 1) SA_SSU_HEAD(1, 2) SA_SSU_HEAD(1, 4) SA_SSU_HEAD(1, 8)
    SA_SSU_HEAD(2, 1) SA_SSU_HEAD(2, 2) SA_SSU_HEAD(2, 4)
    SA_SSU_HEAD(4, 1) SA_SSU_HEAD(4, 2)
#undef SA_SSU_HEAD
  }
  // lanes per state row: enough float4 strips to cover N once, at most 64
  const bool vec4 = N % 4 == 0 && (reinterpret_cast<uintptr_t>(h) & 15) == 0;
  const int strips = vec4 ? N / 4 : N;
  if (strips <= 8)
    return launch_ssu<T, 8>(u, A, B, C, delta_raw, delta_bias, h, y, Dskip, gate, batch, H,
                            P, G, N, softplus, dmin, dmax, stream);
  if (strips <= 16)
    return launch_ssu<T, 16>(u, A, B, C, delta_raw, delta_bias, h, y, Dskip, gate, batch, H,
                             P, G, N, softplus, dmin, dmax, stream);
  if (strips <= 32)
    return launch_ssu<T, 32>(u, A, B, C, delta_raw, delta_bias, h, y, Dskip, gate, batch, H,
                             P, G, N, softplus, dmin, dmax, stream);
  return launch_ssu<T, 64>(u, A, B, C, delta_raw, delta_bias, h, y, Dskip, gate, batch, H,
                           P, G, N, softplus, dmin, dmax, stream);
}

}  // namespace sa

namespace sa {
static int ssu_entry(const char* who, int dtype, const void* u, const float* A, const void* B,
                     const void* C, const void* delta_raw, const float* delta_bias, float* h,
                     void* y, const float* Dskip, const void* gate, int batch, int num_heads,
                     int head_dim, int num_groups, int state_dim, int use_softplus,
                     float delta_min, float delta_max, void* stream) {
  SA_CHECK_ARG(batch >= 0 && num_heads > 0 && head_dim > 0 && num_groups > 0 && state_dim > 0,
               "%s: bad sizes b=%d H=%d P=%d G=%d N=%d", who, batch, num_heads, head_dim,
               num_groups, state_dim);
  SA_CHECK_ARG(num_heads % num_groups == 0, "%s: num_heads %% num_groups != 0", who);
  SA_CHECK_ARG(u && A && B && C && delta_raw && h && y, "%s: null tensor pointer", who);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == kF32)
    return dispatch_ssu<float>(u, A, B, C, delta_raw, delta_bias, h, y, Dskip, gate, batch,
                               num_heads, head_dim, num_groups, state_dim, use_softplus, delta_min,
                               delta_max, s);
  if (dtype == kBF16)
    return dispatch_ssu<bf16>(u, A, B, C, delta_raw, delta_bias, h, y, Dskip, gate, batch,
                              num_heads, head_dim, num_groups, state_dim, use_softplus, delta_min,
                              delta_max, s);
  sa_set_error("%s: unsupported dtype %d", who, dtype);
  return 1;
}
}  // namespace sa

extern "C" int sa_ssu_fwd(int dtype, const void* u, const float* A, const void* B, const void* C,
                          const void* delta_raw, const float* delta_bias, float* h, void* y,
                          int batch, int num_heads, int head_dim, int num_groups, int state_dim,
                          int use_softplus, float delta_min, float delta_max, void* stream) {
  return sa::ssu_entry("sa_ssu_fwd", dtype, u, A, B, C, delta_raw, delta_bias, h, y, nullptr,
                       nullptr, batch, num_heads, head_dim, num_groups, state_dim, use_softplus,
                       delta_min, delta_max, stream);
}

extern "C" int sa_ssu_fwd_gated(int dtype, const void* u, const float* A, const void* B,
                                const void* C, const void* delta_raw, const float* delta_bias,
                                float* h, const float* D, const void* gate, void* out, int batch,
                                int num_heads, int head_dim, int num_groups, int state_dim,
                                int use_softplus, float delta_min, float delta_max, void* stream) {
  SA_CHECK_ARG(D && gate, "sa_ssu_fwd_gated: null D or gate");
  return sa::ssu_entry("sa_ssu_fwd_gated", dtype, u, A, B, C, delta_raw, delta_bias, h, out, D,
                       gate, batch, num_heads, head_dim, num_groups, state_dim, use_softplus,
                       delta_min, delta_max, stream);
}
