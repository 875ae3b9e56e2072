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
// Store 8 values; with plane != 0 (bf16 only) also the rounding residuals
// lo = bf16(x - hi) into the lo plane `plane` elements further.
template <typename MT> struct Store8;
template <> struct Store8<bf16> {
  __device__ __forceinline__ static void store(bf16* p, const float (&v)[8], int plane = 0) {
    uint4 raw;
    raw.x = pack_bf16x2(v[0], v[1]);
    raw.y = pack_bf16x2(v[2], v[3]);
    raw.z = pack_bf16x2(v[4], v[5]);
    raw.w = pack_bf16x2(v[6], v[7]);
    *reinterpret_cast<uint4*>(p) = raw;
    if (plane) {
      uint4 lo;
      lo.x = pack_bf16x2(v[0] - bf16lo_to_f32(raw.x), v[1] - bf16hi_to_f32(raw.x));
      lo.y = pack_bf16x2(v[2] - bf16lo_to_f32(raw.y), v[3] - bf16hi_to_f32(raw.y));
      lo.z = pack_bf16x2(v[4] - bf16lo_to_f32(raw.z), v[5] - bf16hi_to_f32(raw.z));
      lo.w = pack_bf16x2(v[6] - bf16lo_to_f32(raw.w), v[7] - bf16hi_to_f32(raw.w));
      *reinterpret_cast<uint4*>(p + plane) = lo;
    }
  }
};
template <> struct Store8<float> {
  __device__ __forceinline__ static void store(float* p, const float (&v)[8], int = 0) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
};

// 4 consecutive k values of one LDS row (8 B for bf16, 16 B for fp32)
template <typename MT> struct Store4;
template <> struct Store4<bf16> {
  __device__ __forceinline__ static void store(bf16* p, float a, float b, float c, float d,
                                               int plane) {
    uint2 raw;
    raw.x = pack_bf16x2(a, b);
    raw.y = pack_bf16x2(c, d);
    *reinterpret_cast<uint2*>(p) = raw;
    if (plane) {
      uint2 lo;
      lo.x = pack_bf16x2(a - bf16lo_to_f32(raw.x), b - bf16hi_to_f32(raw.x));
      lo.y = pack_bf16x2(c - bf16lo_to_f32(raw.y), d - bf16hi_to_f32(raw.y));
      *reinterpret_cast<uint2*>(p + plane) = lo;
    }
  }
};
template <> struct Store4<float> {
  __device__ __forceinline__ static void store(float* p, float a, float b, float c, float d, int) {
    *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
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

template <typename A, typename B> struct SameT { static constexpr bool value = false; };
template <typename A> struct SameT<A, A> { static constexpr bool value = true; };

// LDS[r][k] (r < R, k < K; K % 8 == 0) from src rows of stride rs (elements).
// Valid region: r < rvalid, k < kvalid.  vec: rows are 16-byte aligned and
// kvalid % 8 == 0 so whole 8-vectors can be read.  A bf16 -> bf16 copy
// without scaling or split moves raw 16-byte vectors.
template <typename MT, typename TS, typename Scale>
__device__ __forceinline__ void stage_rows(MT* lds, int ld, const TS* src, long rs, int R, int K,
                                           int rvalid, int kvalid, bool vec, Scale scale,
                                           int plane = 0) {
  constexpr bool kRaw = SameT<MT, TS>::value && SameT<Scale, NoScale>::value;
  const int kv = K / 8;
  for (int v = threadIdx.x; v < R * kv; v += blockDim.x) {
    const int r = v / kv;
    const int k0 = (v - r * kv) * 8;
    const bool full = r < rvalid && vec && k0 + 8 <= kvalid;
    if constexpr (kRaw) {
      if (full && plane == 0) {
        if constexpr (sizeof(MT) == 2) {
          *reinterpret_cast<uint4*>(lds + r * ld + k0) =
              *reinterpret_cast<const uint4*>(src + r * rs + k0);
        } else {
          *reinterpret_cast<float4*>(lds + r * ld + k0) =
              *reinterpret_cast<const float4*>(src + r * rs + k0);
          *reinterpret_cast<float4*>(lds + r * ld + k0 + 4) =
              *reinterpret_cast<const float4*>(src + r * rs + k0 + 4);
        }
        continue;
      }
    }
    float x[8];
    if (full) {
      Vec8<TS>::load(src + r * rs + k0, x);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        x[j] = (r < rvalid && k0 + j < kvalid) ? load_f32(src + r * rs + k0 + j) : 0.0f;
    }
    if constexpr (!SameT<Scale, NoScale>::value) {
      // only in-range elements are scaled: past the valid rows or columns the
      // scale may read a table entry nobody wrote, and 0 * NaN is NaN
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (r < rvalid && k0 + j < kvalid) x[j] *= scale(r, k0 + j);
    }
    Store8<MT>::store(lds + r * ld + k0, x, plane);
  }
}

// LDS[c][r] (c < Cn, r < R) from src[r*rs + c]; valid r < rvalid, c < cvalid.
// vec: rows 16-byte aligned and cvalid % 8 == 0.  R % 4 == 0, Cn % 8 == 0.
// Each thread reads a 4 (r) x 8 (c) block with 8-wide vector loads and
// writes it transposed as 8 runs of 4 consecutive k; the 16 lanes of a row
// group cover 64 consecutive k of one LDS row, so the writes are
// bank-conflict free.
template <typename MT, typename TS, typename Scale>
__device__ __forceinline__ void stage_transposed(MT* lds, int ld, const TS* src, long rs, int R,
                                                 int Cn, int rvalid, int cvalid, bool vec,
                                                 Scale scale, int plane = 0) {
  const int rq = R / 4, cv = Cn / 8;
  for (int v = threadIdx.x; v < rq * cv; v += blockDim.x) {
    const int a = v % rq;
    const int r0 = a * 4;
    const int c0 = (v / rq) * 8;
    float x[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = r0 + i;
      if (r < rvalid && vec && c0 + 8 <= cvalid) {
        Vec8<TS>::load(src + r * rs + c0, x[i]);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          x[i][j] = (r < rvalid && c0 + j < cvalid) ? load_f32(src + r * rs + c0 + j) : 0.0f;
      }
      if constexpr (!SameT<Scale, NoScale>::value) {
        // only in-range elements are scaled (see stage_rows)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (r < rvalid && c0 + j < cvalid) x[i][j] *= scale(r, c0 + j);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      Store4<MT>::store(lds + (c0 + j) * ld + r0, x[0][j], x[1][j], x[2][j], x[3][j], plane);
  }
}

__host__ __device__ constexpr int round_up(int x, int m) { return (x + m - 1) / m * m; }

// 64 x (32 NK) bf16 tile in registers, raw 16-byte copies shared by NTHR threads.
// Rows past rows_valid read row rows_valid - 1 and are zeroed (unconditional loads).
template <int NK, int NTHR>
struct BfTile {
  static constexpr int PER = 64 * 4 * NK / NTHR;   // uint4 per thread
  uint4 v[PER];
  __device__ __forceinline__ void load(const bf16* src, int rs, int rows_valid, int tid) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = tid + NTHR * i;
      const int row = e / (4 * NK), c8 = e % (4 * NK);
      v[i] = *reinterpret_cast<const uint4*>(src + static_cast<unsigned>(min(row, rows_valid - 1) * rs + 8 * c8));
      if (row >= rows_valid) v[i] = uint4{0u, 0u, 0u, 0u};
    }
  }
  __device__ __forceinline__ void commit(bf16* dst, int ld, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = tid + NTHR * i;
      const int row = e / (4 * NK), c8 = e % (4 * NK);
      *reinterpret_cast<uint4*>(dst + row * ld + 8 * c8) = v[i];
    }
  }
};

}  // namespace sa
