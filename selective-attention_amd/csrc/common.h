// Shared device helpers for the gfx950 kernels of the selective-attention
// kernel layer: dtype handling, MFMA wave tiles, wave/block reductions and
// the reference's softplus.  Written for CDNA4 (wave64, 16x16 MFMA tiles).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sa {

// ---------------------------------------------------------------------------
// dtypes
// ---------------------------------------------------------------------------
enum DType : int { kF32 = 0, kBF16 = 1 };

struct bf16 {  // raw bfloat16 bits; arithmetic always happens in fp32
  uint16_t x;
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) {
  return __uint_as_float(static_cast<uint32_t>(v.x) << 16);
}

// round-to-nearest-even fp32 -> bf16; lowers to gfx950's v_cvt_pk_bf16_f32
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
// two floats -> packed bf16x2 (a in the low half)
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const v2bf v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float bf16lo_to_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi_to_f32(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// 2^x on the transcendental unit (v_exp_f32); decay factors exp(d) are
// evaluated as exp2(d * log2(e)) on pre-scaled cumulative sums
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
constexpr float kLog2e = 1.4426950408889634f;
// sigmoid on the transcendental unit (v_exp_f32, v_rcp_f32; ~1 ulp each):
// the SiLU of the SSM block's conv prologue and gate epilogue
__device__ __forceinline__ float fast_sigmoid(float z) {
  return __builtin_amdgcn_rcpf(1.0f + fast_exp2(-z * kLog2e));
}

template <typename T> struct Conv;
template <> struct Conv<float> {
  __device__ __forceinline__ static float from(float v) { return v; }
};
template <> struct Conv<bf16> {
  __device__ __forceinline__ static bf16 from(float v) { return bf16{f32_to_bf16_bits(v)}; }
};
template <typename T> __device__ __forceinline__ T from_f32(float v) { return Conv<T>::from(v); }

template <typename T> __device__ __forceinline__ float load_f32(const T* p) { return to_f32(*p); }
template <typename T> __device__ __forceinline__ void st(T* p, float v) { *p = from_f32<T>(v); }

// ---------------------------------------------------------------------------
// reference softplus: log(exp(z) + 1) for z <= 20, identity above
// (triton_kernels/softplus.py:8, forward_kernel.py:77).  Accurate libm calls:
// the +1 rounding dominates and must match the fp32 reference bit-for-bit in
// spirit, so no fast-math intrinsics here.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float softplus20(float z) {
  return z <= 20.0f ? logf(expf(z) + 1.0f) : z;
}

__device__ __forceinline__ float sigmoidf_acc(float z) { return 1.0f / (1.0f + expf(-z)); }

// dt = clamp(softplus(z)) -- shared by the chunk cumsum and the state update
__device__ __forceinline__ float make_dt(float z, bool softplus, float dmin, float dmax) {
  float d = softplus ? softplus20(z) : z;
  return fminf(fmaxf(d, dmin), dmax);
}

// ---------------------------------------------------------------------------
// MFMA traits.  MT is the matrix-core operand type: float (IEEE fp32 products,
// v_mfma_f32_16x16x4_f32) or bf16 (v_mfma_f32_16x16x32_bf16, gfx950).
//
// Operands live in LDS "k-contiguous": A as [m][k] rows, B as [n][k] rows.
// Lane l supplies row (l & 15) of A / column (l & 15) of B and KPL
// consecutive k values starting at KPL * (l >> 4).  A and B use the same
// (lane, slot) -> k assignment, so the product is exact whatever order the
// hardware sums k in.  The 16x16 fp32 result: lane l holds rows
// 4 * (l >> 4) + i (i = 0..3) of column (l & 15).
// ---------------------------------------------------------------------------
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef uint16_t v8u16 __attribute__((ext_vector_type(8)));

template <typename MT> struct Mfma;

template <> struct Mfma<float> {
  static constexpr int KSTEP = 16;  // k per call (4 MFMA issues of k=4)
  __device__ __forceinline__ static v4f mma(const float* A, int lda, const float* B, int ldb,
                                            v4f c, int lane) {
    const float* a = A + (lane & 15) * lda + (lane >> 4);
    const float* b = B + (lane & 15) * ldb + (lane >> 4);
#pragma unroll
    for (int s = 0; s < 4; ++s)
      c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[4 * s], b[4 * s], c, 0, 0, 0);
    return c;
  }
};

template <> struct Mfma<bf16> {
  static constexpr int KSTEP = 32;
  __device__ __forceinline__ static v4f mma(const bf16* A, int lda, const bf16* B, int ldb, v4f c,
                                            int lane) {
    const v8bf a = *reinterpret_cast<const v8bf*>(A + (lane & 15) * lda + 8 * (lane >> 4));
    const v8bf b = *reinterpret_cast<const v8bf*>(B + (lane & 15) * ldb + 8 * (lane >> 4));
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

// A wave computes a (16*TM) x (16*TN) fp32 tile:
//   acc[i][j] += A[16i.., 0:K] * B[16j.., 0:K]^T
// A: LDS [rows][lda], B: LDS [cols][ldb], both k-contiguous; K % KSTEP == 0.
template <typename MT, int TM, int TN>
__device__ __forceinline__ void wave_mma(v4f (&acc)[TM][TN], const MT* A, int lda, const MT* B,
                                         int ldb, int K, int lane) {
  for (int k = 0; k < K; k += Mfma<MT>::KSTEP) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = Mfma<MT>::mma(A + 16 * i * lda + k, lda, B + 16 * j * ldb + k, ldb, acc[i][j],
                                  lane);
  }
}

// Split-precision variant for operands that originate in fp32 (gradients,
// states, scaled tiles): such an operand is staged as two bf16 planes,
// x = hi + lo with hi = bf16(x), lo = bf16(x - hi), the lo plane `plane`
// elements after the hi plane.  Products keep hi*hi + lo*hi + hi*lo, dropping
// lo*lo (~2^-16 relative), so the result is close to an fp32 GEMM.
// SA / SB say which operands carry a lo plane.  For MT = float the split is
// never used (the fp32 MFMA is exact) and SA = SB = false.
template <typename MT, int TM, int TN, bool SA, bool SB>
__device__ __forceinline__ void wave_mma_split(v4f (&acc)[TM][TN], const MT* A, int lda, int aplane,
                                               const MT* B, int ldb, int bplane, int K, int lane) {
  for (int k = 0; k < K; k += Mfma<MT>::KSTEP) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const MT* a = A + 16 * i * lda + k;
        const MT* b = B + 16 * j * ldb + k;
        acc[i][j] = Mfma<MT>::mma(a, lda, b, ldb, acc[i][j], lane);
        if (SA) acc[i][j] = Mfma<MT>::mma(a + aplane, lda, b, ldb, acc[i][j], lane);
        if (SB) acc[i][j] = Mfma<MT>::mma(a, lda, b + bplane, ldb, acc[i][j], lane);
      }
  }
}

// ---------------------------------------------------------------------------
// register-resident bf16 MFMA helpers (16x16x32): operand fragments held in
// registers, and the "transposed score" layout shared by the attention and
// SSD tile kernels.  A 16x16 result tile computed with A-operand rows mapped
// through key_of_row leaves every lane holding, for its column, 8 consecutive
// keys across two tiles (2s, 2s+1) -- exactly the B-operand fragment of the
// next MFMA that contracts over those keys.
// ---------------------------------------------------------------------------
__device__ __forceinline__ v8bf load_v8bf(const bf16* p) {
  return *reinterpret_cast<const v8bf*>(p);
}
// Non-temporal (streaming) accesses for data touched once per step: such
// lines are kept out of the caches and leave no write-back traffic behind.
typedef float v4f_nt __attribute__((ext_vector_type(4)));
typedef unsigned v2u_nt __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float4 ld_nt(const float4* p) {
  const v4f_nt v = __builtin_nontemporal_load(reinterpret_cast<const v4f_nt*>(p));
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void st_nt(float4* p, const float4& v) {
  __builtin_nontemporal_store(v4f_nt{v.x, v.y, v.z, v.w}, reinterpret_cast<v4f_nt*>(p));
}
__device__ __forceinline__ void st_nt(uint2* p, const uint2& v) {
  __builtin_nontemporal_store(v2u_nt{v.x, v.y}, reinterpret_cast<v2u_nt*>(p));
}

// Raw buffer reads (stride 0, gfx9 config dword 0x00020000): the base lives
// in a wave-uniform resource, the lane offset in one VGPR and the per-load
// step in an SGPR, so a run of loads from one base needs no per-load VALU
// address arithmetic.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           0x7fffffff, 0x00020000);
}
__device__ __forceinline__ v8bf buf_load_v8bf(__amdgpu_buffer_rsrc_t r, unsigned voff_bytes,
                                              unsigned soff_bytes) {
  return __builtin_bit_cast(v8bf, __builtin_amdgcn_raw_buffer_load_b128(r, voff_bytes, soff_bytes, 0));
}
__device__ __forceinline__ v8bf zero_v8bf() {
  const uint4 z = {0u, 0u, 0u, 0u};
  return __builtin_bit_cast(v8bf, z);
}
__device__ __forceinline__ v8bf pack_p(const v4f& lo, const v4f& hi) {
  const uint4 r = {pack_bf16x2(lo[0], lo[1]), pack_bf16x2(lo[2], lo[3]), pack_bf16x2(hi[0], hi[1]),
                   pack_bf16x2(hi[2], hi[3])};
  return __builtin_bit_cast(v8bf, r);
}
__device__ __forceinline__ v4f mfma_bf16(const v8bf& a, const v8bf& b, const v4f& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 16-byte global load, zero when !ok
__device__ __forceinline__ uint4 ld16(const void* p, bool ok) {
  return ok ? *reinterpret_cast<const uint4*>(p) : uint4{0u, 0u, 0u, 0u};
}
// From four rows of 8 bf16 (r0..r3, one uint4 each) take column j (0..7) as
// 4 consecutive bf16: the transposed 4-element run written to LDS.
__device__ __forceinline__ uint2 col4_bf16(const uint4& r0, const uint4& r1, const uint4& r2,
                                           const uint4& r3, int j) {
  const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
  const int w = j >> 1;
  const uint32_t a0 = w == 0 ? r0.x : w == 1 ? r0.y : w == 2 ? r0.z : r0.w;
  const uint32_t a1 = w == 0 ? r1.x : w == 1 ? r1.y : w == 2 ? r1.z : r1.w;
  const uint32_t a2 = w == 0 ? r2.x : w == 1 ? r2.y : w == 2 ? r2.z : r2.w;
  const uint32_t a3 = w == 0 ? r3.x : w == 1 ? r3.y : w == 2 ? r3.z : r3.w;
  return uint2{__builtin_amdgcn_perm(a1, a0, sel), __builtin_amdgcn_perm(a3, a2, sel)};
}

// fp32 pair (a, b) of 4+4 values as two bf16 fragments: hi = bf16(x) and
// lo = bf16(x - hi), so that hi + lo carries ~16 mantissa bits into an MFMA
__device__ __forceinline__ void split_p(const v4f& a, const v4f& b, v8bf& hi, v8bf& lo) {
  const uint4 h = {pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(b[0], b[1]),
                   pack_bf16x2(b[2], b[3])};
  const uint4 l = {pack_bf16x2(a[0] - bf16lo_to_f32(h.x), a[1] - bf16hi_to_f32(h.x)),
                   pack_bf16x2(a[2] - bf16lo_to_f32(h.y), a[3] - bf16hi_to_f32(h.y)),
                   pack_bf16x2(b[0] - bf16lo_to_f32(h.z), b[1] - bf16hi_to_f32(h.z)),
                   pack_bf16x2(b[2] - bf16lo_to_f32(h.w), b[3] - bf16hi_to_f32(h.w))};
  hi = __builtin_bit_cast(v8bf, h);
  lo = __builtin_bit_cast(v8bf, l);
}
// 8 consecutive fp32 (two float4) as hi / lo bf16 fragments
__device__ __forceinline__ void split8(const float4& a, const float4& b, v8bf& hi, v8bf& lo) {
  split_p(v4f{a.x, a.y, a.z, a.w}, v4f{b.x, b.y, b.z, b.w}, hi, lo);
}

// LDS transpose read (ds_read_b64_tr_b16).  `x` points at element [k0][c0]
// of a row-major bf16 LDS tile with row length ld (elements, ld*2 a multiple
// of 8 bytes); every lane of a 16-lane group receives the column
// x[k0 .. k0+7][c0 + (lane & 15)] -- the MFMA operand fragment for a
// contraction over the tile's rows.  Within a 16-lane group, lane i loads the
// 4 elements at [k0 + i/4][c0 + 4(i%4)] and the hardware hands lane j the
// elements [k0 + m][c0 + j], m = 0..3.
typedef short v4i16 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ v8bf lds_tr8(const bf16* x, int ld, int lane) {
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  const int i = lane & 15;
  const bf16* p = x + (i >> 2) * ld + 4 * (i & 3);
  const v4i16 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p));
  const v4i16 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p + 4 * ld));
  return __builtin_bit_cast(v8bf, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}

// LDS DMA written as instructions the compiler does not interpret: it then
// inserts no waits of its own for them (it cannot tell which LDS bytes a DMA
// writes, and would otherwise hold every LDS read until all DMA in flight had
// landed); the kernel waits with explicit vmcnt and barriers.  Each lane's
// data goes to LDS byte address lds + 16 lane (4 lane for the dword form),
// from base + off (off in bytes).  m0 carries the LDS address; nothing else
// in the kernels that use these relies on m0.
//
// lds_addr: the LDS byte address of a generic pointer into LDS, as a
// wave-uniform value (the DMA helpers take it through readfirstlane, which
// costs nothing where it already sits in a scalar register).  A generic LDS address is the shared aperture in the
// high half and the LDS offset in the low half, so the low 32 bits are the
// address (no address-space cast, whose null check costs a 64-bit compare
// and select per use).  Kernels take it once per stage, outside their loops.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p)));
}
__device__ __forceinline__ void dma_lds16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base),
               "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
}
__device__ __forceinline__ void dma_lds4(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base),
               "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt immediate: vmcnt(N), expcnt and lgkmcnt not waited for
template <int N>
constexpr int vm_wait() {
  return (N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14);
}
constexpr int kLgkmWait0 = 0xF | (7 << 4) | (3 << 14);   // lgkmcnt(0) only
// vmcnt(N) and lgkmcnt(0): the wave's LDS accesses are complete as well
template <int N>
constexpr int vm_lgkm_wait() {
  return (N & 15) | (7 << 4) | ((N >> 4) << 14);
}

// key (within a 64-key tile) held by MFMA row c of score tile kt
__device__ __forceinline__ int key_of_row(int kt, int c) {
  return 32 * (kt >> 1) + 8 * (c >> 2) + 4 * (kt & 1) + (c & 3);
}

template <int TM, int TN>
__device__ __forceinline__ void zero_acc(v4f (&acc)[TM][TN]) {
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
}

// row / column of element r (0..3) of a 16x16 result fragment held by `lane`
__device__ __forceinline__ int frag_row(int lane, int r) { return 4 * (lane >> 4) + r; }
__device__ __forceinline__ int frag_col(int lane) { return lane & 15; }

// padded LDS row length (elements) for a k extent: keeps 16-byte alignment and
// shifts consecutive rows across banks
template <typename MT> __host__ __device__ constexpr int lds_ld(int k) {
  return k + (sizeof(MT) == 2 ? 8 : 4);
}

// ---------------------------------------------------------------------------
// wave / block reductions and scans (wave64)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
// inclusive prefix sum across the 64 lanes of a wave
__device__ __forceinline__ float wave_incl_scan(float v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    float t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  return v;
}

// ---------------------------------------------------------------------------
// XCD-aware block order.  Workgroups are dealt round-robin over the 8 XCDs;
// remapping gives each XCD a contiguous range of logical tiles so that tiles
// sharing operands (e.g. heads of one group) share an L2.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int xcd_swizzle(int bid, int nblocks) {
  constexpr int kXcd = 8;
  int per = nblocks / kXcd;
  int rem = nblocks - per * kXcd;
  int xcd = bid % kXcd;
  int slot = bid / kXcd;
  if (slot >= per) return bid;  // tail blocks keep their id (only when nblocks % 8 != 0)
  (void)rem;
  return xcd * per + slot;
}

// Block order for launches whose blocks come in groups of nk with unequal
// work (member k of a group walks nk - k tiles, say).  Blocks that share an
// XCD (consecutive ids after xcd_swizzle) are taken in windows of one XCD's
// resident blocks (32 CUs x 2 blocks = 64 on MI355X): a window holds
// max(1, 64 / nk) whole groups and issues member 0 of each of its groups
// first, then member 1, and so on (the second half of the members in
// reverse, below).  Each resident round then ends on the shorter half of
// the members, and a group's members still run within one window of each
// other (what they share stays in L2).  bid in [0, nblocks), nblocks a
// multiple of nk; returns the member k and the group index.  Kernels that
// run three blocks per CU pass their own resident count.
template <int kResidentPerXcd = 64>
__device__ __forceinline__ void xcd_window_order(int bid, int nblocks, int nk, int& k, int& grp) {
  const int wg = max(1, kResidentPerXcd / nk);        // groups per window
  const int ngrp = nblocks / nk;
  const int win = bid / (wg * nk), inw = bid - win * (wg * nk);
  const int wsz = min(wg, ngrp - win * wg);           // the last window may be short
  k = inw / wsz;
  grp = win * wg + (inw - k * wsz);
  // members 0 .. nk/2 - 1 first, then the others shortest first, so that
  // where the blocks of a window land in CU order the second block of a CU
  // tends to be member nk - 1 - j beside member j (measured: 0.3-1 % on the
  // SSD step at config 1, config 4's SSM shape and the reference default)
  if (k >= nk / 2) k = nk - 1 - (k - nk / 2);
}

}  // namespace sa

// host-side error plumbing shared by every entry point (defined in abi.cpp)
extern "C" void sa_set_error(const char* fmt, ...);

#define SA_CHECK_ARG(cond, ...)        \
  do {                                 \
    if (!(cond)) {                     \
      sa_set_error(__VA_ARGS__);       \
      return 1;                        \
    }                                  \
  } while (0)

// a HIP runtime call that must succeed (its code becomes return value 2)
#define SA_CHECK_LAUNCH_RC(call, what)                                               \
  do {                                                                               \
    hipError_t e_ = (call);                                                          \
    if (e_ != hipSuccess) {                                                          \
      sa_set_error("%s failed: %s", what, hipGetErrorString(e_));                    \
      return 2;                                                                      \
    }                                                                                \
  } while (0)

#define SA_CHECK_LAUNCH(what)                                                        \
  do {                                                                               \
    hipError_t e_ = hipGetLastError();                                               \
    if (e_ != hipSuccess) {                                                          \
      sa_set_error("%s: launch failed: %s", what, hipGetErrorString(e_));            \
      return 2;                                                                      \
    }                                                                                \
  } while (0)
