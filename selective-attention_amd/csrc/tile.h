// Global -> LDS tile staging for the MFMA kernels (256-thread blocks).
//
// MFMA operands sit in LDS k-contiguous (see common.h).  Two staging shapes:
//   stage_rows       LDS[r][k] = scale(r,k) * src[r*rs + k]   (k contiguous in HBM)
//   stage_transposed LDS[c][r] = scale(r,c) * src[r*rs + c]   (c contiguous in HBM,
//                                                             r becomes the k index)
// Out-of-range elements are written as zeros so every MFMA k-step is exact.
// Global reads are 8-element vectors (16 B for bf16) when the caller says
// the rows are 16-byte aligned.
#pragma once

#include "common.h"

namespace sa {

template <typename TS> struct Vec8;
template <> struct Vec8<bf16> {
  __device__ __forceinline__ static void load(const bf16* p, float (&v)[8]) {
    const uint4 raw = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = __uint_as_float(w[j] << 16);
      v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  }
};
template <> struct Vec8<float> {
  __device__ __forceinline__ static void load(const float* p, float (&v)[8]) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
};

// Store 8 values; with plane != 0 (bf16 only) also the rounding residuals
// lo = bf16(x - hi) into the lo plane `plane` elements further.
template <typename MT> struct Store8;
template <> struct Store8<bf16> {
  __device__ __forceinline__ static void store(bf16* p, const float (&v)[8], int plane = 0) {
    uint16_t hb[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) hb[j] = f32_to_bf16_bits(v[j]);
    uint4 raw;
    raw.x = hb[0] | (static_cast<uint32_t>(hb[1]) << 16);
    raw.y = hb[2] | (static_cast<uint32_t>(hb[3]) << 16);
    raw.z = hb[4] | (static_cast<uint32_t>(hb[5]) << 16);
    raw.w = hb[6] | (static_cast<uint32_t>(hb[7]) << 16);
    *reinterpret_cast<uint4*>(p) = raw;
    if (plane) {
      uint16_t lb[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        lb[j] = f32_to_bf16_bits(v[j] - __uint_as_float(static_cast<uint32_t>(hb[j]) << 16));
      raw.x = lb[0] | (static_cast<uint32_t>(lb[1]) << 16);
      raw.y = lb[2] | (static_cast<uint32_t>(lb[3]) << 16);
      raw.z = lb[4] | (static_cast<uint32_t>(lb[5]) << 16);
      raw.w = lb[6] | (static_cast<uint32_t>(lb[7]) << 16);
      *reinterpret_cast<uint4*>(p + plane) = raw;
    }
  }
};
template <> struct Store8<float> {
  __device__ __forceinline__ static void store(float* p, const float (&v)[8], int = 0) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
};

// one element, optionally split into hi/lo planes (bf16 only)
__device__ __forceinline__ void store_split(float* p, float v, int) { *p = v; }
__device__ __forceinline__ void store_split(bf16* p, float v, int plane) {
  const uint16_t hb = f32_to_bf16_bits(v);
  p->x = hb;
  if (plane) p[plane].x = f32_to_bf16_bits(v - __uint_as_float(static_cast<uint32_t>(hb) << 16));
}

struct NoScale {
  __device__ __forceinline__ float operator()(int, int) const { return 1.0f; }
};

// LDS[r][k] (r < R, k < K; K % 8 == 0) from src rows of stride rs (elements).
// Valid region: r < rvalid, k < kvalid.  vec: rows are 16-byte aligned and
// kvalid % 8 == 0 so whole 8-vectors can be read.
template <typename MT, typename TS, typename Scale>
__device__ __forceinline__ void stage_rows(MT* lds, int ld, const TS* src, long rs, int R, int K,
                                           int rvalid, int kvalid, bool vec, Scale scale,
                                           int plane = 0) {
  const int kv = K / 8;
  for (int v = threadIdx.x; v < R * kv; v += blockDim.x) {
    const int r = v / kv;
    const int k0 = (v - r * kv) * 8;
    float x[8];
    if (r < rvalid && vec && k0 + 8 <= kvalid) {
      Vec8<TS>::load(src + r * rs + k0, x);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        x[j] = (r < rvalid && k0 + j < kvalid) ? load_f32(src + r * rs + k0 + j) : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] *= scale(r, k0 + j);
    Store8<MT>::store(lds + r * ld + k0, x, plane);
  }
}

// LDS[c][r] (c < Cn, r < R) from src[r*rs + c]; valid r < rvalid, c < cvalid.
// vec: rows 16-byte aligned and cvalid % 8 == 0.  Cn % 8 == 0.
template <typename MT, typename TS, typename Scale>
__device__ __forceinline__ void stage_transposed(MT* lds, int ld, const TS* src, long rs, int R,
                                                 int Cn, int rvalid, int cvalid, bool vec,
                                                 Scale scale, int plane = 0) {
  const int cv = Cn / 8;
  for (int v = threadIdx.x; v < R * cv; v += blockDim.x) {
    const int r = v / cv;
    const int c0 = (v - r * cv) * 8;
    float x[8];
    if (r < rvalid && vec && c0 + 8 <= cvalid) {
      Vec8<TS>::load(src + r * rs + c0, x);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        x[j] = (r < rvalid && c0 + j < cvalid) ? load_f32(src + r * rs + c0 + j) : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) store_split(lds + (c0 + j) * ld + r, x[j] * scale(r, c0 + j), plane);
  }
}

__host__ __device__ constexpr int round_up(int x, int m) { return (x + m - 1) / m * m; }

}  // namespace sa
