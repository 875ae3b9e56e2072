// Shapes and shared launch helpers of the SSD chunked scan kernels.
#pragma once

#include "common.h"
#include "tile.h"

namespace sa {

struct SsdDims {
  int b, L, H, P, G, N, Lc, nc;
};

// effective sequence length of batch row b: clamp(length[b], 0, L), or L
// when no lengths are given
__device__ __forceinline__ int seq_limit(const int64_t* length, int b, int L) {
  if (!length) return L;   // no lengths: every row is full
  long v = length[b];
  return static_cast<int>(v < 0 ? 0 : (v > L ? L : v));
}
// positions of chunk c inside the length (may be <= 0)
__device__ __forceinline__ int chunk_limit(int len, int c, int Lc) {
  return min(Lc, len - c * Lc);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// ---------------------------------------------------------------------------
// LDS row layouts of the bf16 SSD tile kernels.  Rows of 64 bf16 (128 bytes)
// and 128 bf16 (256 bytes) are stored unpadded, 16-byte chunk c of row r at
// chunk c ^ f(r).  The gfx950 LDS does not map banks by the low address bits
// alone (16 lanes reading distinct chunks of one 256-byte span can still
// conflict, depending on their rows and on the chunks the other lane groups
// of the instruction read), so f was chosen by measurement: every XOR of row
// bits into chunk bits was run on these kernels' read sets -- 16-byte
// fragments of the key_of_row row sets and of 16 consecutive rows, and
// ds_read_b64_tr_b16 transposed reads -- and these give
// SQ_LDS_BANK_CONFLICT = 0 on all of them.  Neither uses row bits 2 or 5,
// so rows r, r + 4 and r + 32 share the permutation.  Other row widths keep
// 16 bytes of padding per row.
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ int swz_r128(int r) {
  return (((r >> 1) & 1) << 1) | (((r >> 3) & 1) << 2);
}
__host__ __device__ __forceinline__ int swz_r256(int r) {
  return ((r & 1) << 1) | (((r >> 1) & 1) << 2) | (((r >> 3) & 1) << 3);
}
template <int W>
struct LdsTile {
  static constexpr bool kSwz = W == 64 || W == 128;
  static constexpr int kLd = kSwz ? W : W + 8;   // row stride (elements)
  // element offset of (row, col), col a multiple of 4
  __host__ __device__ __forceinline__ static int off(int r, int col) {
    if constexpr (W == 64) return r * 64 + 8 * ((col >> 3) ^ swz_r128(r)) + (col & 7);
    else if constexpr (W == 128) return r * 128 + 8 * ((col >> 3) ^ swz_r256(r)) + (col & 7);
    else return r * kLd + col;
  }
};
// transposed read at precomputed element offsets: off0 addresses this lane's
// row k0 + (lane & 15) / 4, off1 the row 4 further on (see tile_tr8)
__device__ __forceinline__ v8bf tile_tr8_at(const bf16* t, int off0, int off1) {
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  const v4i16 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(t + off0));
  const v4i16 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(t + off1));
  return __builtin_bit_cast(v8bf, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}
// a BfTile's registers (64 rows of 32 NK bf16) into an LdsTile<32 NK>
template <int NK, int NTHR>
__device__ __forceinline__ void commit_lds(const BfTile<NK, NTHR>& t, bf16* dst, int tid) {
#pragma unroll
  for (int i = 0; i < BfTile<NK, NTHR>::PER; ++i) {
    const int e = tid + NTHR * i;
    const int row = e / (4 * NK), c8 = e % (4 * NK);
    *reinterpret_cast<uint4*>(dst + LdsTile<32 * NK>::off(row, 8 * c8)) = t.v[i];
  }
}
// transposed read (ds_read_b64_tr_b16): every lane of a 16-lane group
// receives rows k0 .. k0 + 7 of column c0 + (lane & 15) of an LdsTile<W>
template <int W>
__device__ __forceinline__ v8bf tile_tr8(const bf16* t, int k0, int c0, int lane) {
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  const int i = lane & 15, r = k0 + (i >> 2), col = c0 + 4 * (i & 3);
  const v4i16 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(t + LdsTile<W>::off(r, col)));
  const v4i16 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(t + LdsTile<W>::off(r + 4, col)));
  return __builtin_bit_cast(v8bf, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}

inline int make_dims(int b, int L, int H, int P, int G, int N, int Lc, SsdDims* d,
                     const char* who) {
  SA_CHECK_ARG(b >= 0 && L >= 0 && H > 0 && P > 0 && G > 0 && N > 0,
               "%s: bad sizes b=%d L=%d H=%d P=%d G=%d N=%d", who, b, L, H, P, G, N);
  SA_CHECK_ARG(H % G == 0, "%s: num_heads (%d) %% num_groups (%d) != 0", who, H, G);
  SA_CHECK_ARG(Lc >= 1 && Lc <= 1024, "%s: chunk_size %d outside [1, 1024]", who, Lc);
  SA_CHECK_ARG(N <= 256, "%s: state_dim %d > 256 is not supported", who, N);
  d->b = b; d->L = L; d->H = H; d->P = P; d->G = G; d->N = N; d->Lc = Lc;
  d->nc = (L + Lc - 1) / Lc;
  return 0;
}

// launchers shared between the forward and backward translation units
template <typename T>
int launch_chunk_cumsum(const void* delta_raw, const float* A, const float* bias,
                        const int64_t* length, float* dt, float* dc, const SsdDims& d, int sp,
                        float lo, float hi, hipStream_t s);

// MODE 0: chunk states from (u, B); MODE 1: dH_intra from (dy, C)
template <typename MT, typename TA, typename TB, int MODE>
int launch_chunk_outer(const void* a, const void* b, const float* dt, const float* dc,
                       const int64_t* length, float* out, const SsdDims& d, hipStream_t s);

// fused bf16 backward (headdim 64, state_dim 128): source-strip kernel (du,
// dB, decay sums, dCB planes) and target-strip kernel (dC, x_C); defined in
// ssd_bwd_fused.hip.  dyp: dy as bf16 hi + lo planes [b][nc][G][Lc/64][H/G]
// [2][64][64]; dSp: dS as hi + lo planes [b][nc][H][2][64][N]; dcbp: dCB^T
// planes [b][nc][G][Lc/64][Lc/64][2][64][64].  dt_nonneg: every dt is >= 0
// (delta_min >= 0), so each head's dc is monotone within a chunk
bool ssd_bwd_fused_shape_ok(const SsdDims& d);
bool ssd_bwd_fused_ok(const SsdDims& d, const void* u, const void* B, const void* C,
                      const void* dy);
int launch_ssd_bwd_fused(const void* u, const void* B, const void* C, const bf16* dyp,
                         const float* dt, const float* dc, const float* states, const bf16* dSp,
                         const int64_t* length, void* du, void* dB, void* dC, bf16* dcbp,
                         float* ddt_part, float* xB_part, float* xC_part, float* qpart,
                         float* rpart, const SsdDims& d, bool dt_nonneg,
                         hipStream_t s);

// dH_intra (chunk_outer MODE 1, bf16 dy) that also writes dy as the hi + lo
// planes of the fused backward
int launch_dstate_planes(const float* dy, const void* C, const float* dt, const float* dc,
                         const int64_t* length, float* out, bf16* dyp, const SsdDims& d,
                         hipStream_t s);

}  // namespace sa
