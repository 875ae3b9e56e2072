// SSD chunked scan backward: the intra-chunk kernels of the bf16 path for
// headdim 64, state_dim 128, chunk_size a multiple of 64, at most 4 heads per
// group (gfx950).
//
// Replaces the reference's intra-chunk backward kernels
// (triton_kernels/ssd_scan/backward_kernel.py: _chunk_scan_bwd_dx :187-317,
// _chunk_scan_bwd_dcb :569-668, the dC / dB kernels :337-551 and the
// decay-gradient sums :689-765, :783-911) with two kernels over one chunk of
// one group (its HPG heads), each tile a 64-token strip:
//
//   ssd_bwd_src (one block per (b, c, group, source strip S), 4 waves; wave
//     w owns the 16 source columns sigma = 64 S + 16 w + lane % 16; the
//     group's heads run two at a time, one launch per pair, the last launch
//     adding the earlier pairs' dCB shares and writing dB and the planes):
//       du     = dt * (e^{dc_last - dc} B.dS^T  +  L^T dy),  L = C.B^T o decay
//       dB     = sum_h w_h u_h.dS_h  +  dCB^T C,            dCB = sum_h (dy_h u_h^T) dt decay
//       x_B, ddt_direct, the column sums q and (per source strip) row sums r
//       of M = W o CB for the decay gradient, and dCB of every target strip
//       T >= S (bf16 hi + lo planes, [sigma][tau], read by ssd_bwd_tgt)
//   ssd_bwd_tgt (one block per (b, c, group, target strip T, half of N), 4
//     waves; wave w owns the 16 target rows tau = 64 T + 16 w + lane % 16):
//       dC     = sum_h e^{dc} dy_h.H_in_h  +  sum_{S <= T} dCB B,  and x_C
//     (x_C as one partial per half)
//
// Operands reach LDS by DMA (global_load_lds, 16 bytes per lane) from bf16
// planes written by the kernels before them: dy as hi + lo planes (by the
// dH_intra kernel), dS as hi + lo planes (by the state-passing backward), B,
// C and u as given.  fp32-origin operands (dy, dS, H_in, the decayed C.B^T
// and dCB) are carried as hi + lo bf16 planes, their products as
// hi*hi + lo*hi + hi*lo (or hi*x + lo*x against an exact bf16 operand), so
// every product is close to an fp32 one.
//
// A product's result fragment (rows in registers, column on the lane) feeds
// the next product that contracts over those rows straight from registers:
// the rows are visited through key_of_row, so each lane holds 8 consecutive
// rows per 32-row k step.  LDS tiles are unpadded (DMA writes 1 KB runs) and
// their 16-byte chunks are XOR-swizzled per row so that the row reads (row
// sets of key_of_row or 16 consecutive rows) and the ds_read_b64_tr_b16
// transposed reads hit distinct banks.
#include "ssd_common.h"
#include "prof.h"

namespace sa {

// ---------------------------------------------------------------------------
// LDS layouts.  Chunk c (16 bytes) of row r is stored at chunk c ^ f(r):
// swz_r128 / swz_r256 (ssd_common.h) for the source kernel's tiles,
// swz_k128 for the target kernel's.
// ---------------------------------------------------------------------------
// 128-byte rows (64 bf16) of the target kernel's tiles, read transposed
__host__ __device__ __forceinline__ int swz_k128(int r) {
  return ((r >> 4) & 1) | (((r >> 1) & 1) << 1) | (((r >> 3) & 1) << 2);
}

// C tiles of the source kernel: 256-byte rows at state_dim 128, 128-byte
// rows at state_dim 64
template <int NK>
__host__ __device__ __forceinline__ int swz_c(int r) { return NK == 4 ? swz_r256(r) : swz_r128(r); }

// element offset of (row, col) in a swizzled tile with RC 16-byte chunks per row
template <int RC, int (*F)(int)>
__device__ __forceinline__ int toff(int row, int col) {
  return row * (RC * 8) + 8 * ((col >> 3) ^ (F(row) & (RC - 1))) + (col & 7);
}

// lane offset (elements, row stride grs) of DMA instruction i of wave w for a
// 64-row swizzled tile with RC chunks per row
template <int RC, int (*F)(int)>
__device__ __forceinline__ int dma_off(int i, int w, int lane, int grs) {
  const int inst = w * (RC / 4) + i;
  const int pos = inst * 64 + lane;
  const int row = pos / RC, pc = pos % RC;
  return row * grs + 8 * (pc ^ (F(row) & (RC - 1)));
}
// Tile copies into LDS through dma_lds16 (common.h), which the compiler does
// not see as LDS writes, so it holds no LDS access or load use for them; the
// kernels order them with their own waits.  lds: the tile's LDS byte
// address; the 4 waves of a block share a copy, one 1 KB DMA instruction per
// 64 chunks.  dma_pre_op: a full 64-row tile from per-lane element offsets
// (dma_off); dma_tile_op: rows past rows_valid repeat row rows_valid - 1.
template <int RC>
__device__ __forceinline__ void dma_pre_op(uint32_t lds, const bf16* g, const int (&off)[RC / 4], int w) {
#pragma unroll
  for (int i = 0; i < RC / 4; ++i)
    dma_lds16(g, 2u * static_cast<uint32_t>(off[i]), lds + (static_cast<uint32_t>(w * (RC / 4) + i) << 10));
}
template <int RC, int (*F)(int)>
__device__ __forceinline__ void dma_tile_op(uint32_t lds, const bf16* g, int grs, int rows_valid,
                                            int w, int lane) {
#pragma unroll
  for (int i = 0; i < RC / 4; ++i) {
    const int inst = w * (RC / 4) + i;
    const int pos = inst * 64 + lane;
    const int row = pos / RC, pc = pos % RC;
    const int gr = row < rows_valid ? row : rows_valid - 1;
    dma_lds16(g, 2u * static_cast<uint32_t>(gr * grs + 8 * (pc ^ (F(row) & (RC - 1)))),
              lds + (static_cast<uint32_t>(inst) << 10));
  }
}

// Lane offset (elements) for DMA instruction i of wave w into a swz_k128
// [sigma][tau] plane of a dCB tile.  The source kernel stores a tile in lane
// order: dCB[tau = 8 c .. 8 c + 7][sigma] of plane p (hi, lo), c = 4 ks + lg,
// is chunk q = 2 ks + p of lane (lg, li = sigma % 16) of wave sigma / 16, at
// element 2048 q + 8 (64 wave + 4 li + lg).  This returns the hi plane's
// chunk for the LDS position; the lo plane's is 2048 elements further on.
__device__ __forceinline__ int dcb_lane_off(int i, int w, int lane) {
  const int pos = (w * 2 + i) * 64 + lane;   // LDS chunk, 8 per 128-byte row
  const int sigma = pos >> 3;
  const int c = (pos & 7) ^ (swz_k128(sigma) & 7);
  return 2 * (c >> 2) * 2048 + ((sigma >> 4) * 64 + (sigma & 15) * 4 + (c & 3)) * 8;
}

// Output tiles leave through LDS.  A lane's 8-byte pieces of a row-major
// [64 rows][RC 16-byte chunks] bf16 tile go in at chunk c ^ (row % RC), and
// the tile goes out as whole rows, 16 bytes per lane: each store instruction
// of a wave then writes whole cache lines (stored from the MFMA fragments,
// one instruction wrote 32 bytes of each of 16 rows).
template <int RC>
__device__ __forceinline__ void stage_out8(bf16* t, int row, int col, uint2 v) {
  const int c = col >> 3;
  *reinterpret_cast<uint2*>(t + row * (RC * 8) + 8 * (c ^ (row & (RC - 1))) + (col & 7)) = v;
}
// rows r < rows_valid of a staged tile to g + r grs
template <int RC>
__device__ __forceinline__ void write_rows(const bf16* t, bf16* g, int grs, int rows_valid, int tid) {
#pragma unroll
  for (int i = 0; i < RC / 4; ++i) {
    const int e = tid + 256 * i, r = e / RC, c = e % RC;
    if (r < rows_valid)
      *reinterpret_cast<uint4*>(g + static_cast<unsigned>(r * grs + 8 * c)) =
          *reinterpret_cast<const uint4*>(t + r * (RC * 8) + 8 * (c ^ (r & (RC - 1))));
  }
}

// fragment of 8 consecutive bf16 of one swizzled row
template <int RC, int (*F)(int)>
__device__ __forceinline__ v8bf row_frag(const bf16* t, int row, int col) {
  return load_v8bf(t + toff<RC, F>(row, col));
}

// transposed read: every lane of a 16-lane group receives rows k0..k0+7 of
// column c0 + (lane & 15) (k0 a multiple of 8, c0 a multiple of 16)
template <int RC, int (*F)(int)>
__device__ __forceinline__ v8bf tr_frag(const bf16* t, int k0, int c0, int lane) {
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  const int i = lane & 15;
  const int r0 = k0 + (i >> 2), col = c0 + 4 * (i & 3);
  const v4i16 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(t + toff<RC, F>(r0, col)));
  const v4i16 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(t + toff<RC, F>(r0 + 4, col)));
  return __builtin_bit_cast(v8bf, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}

// transposed read at a precomputed lane offset: `off` addresses rows
// k0 + i/4 (i = lane & 15), the second half rows k0 + 4 + i/4 at `off2`
__device__ __forceinline__ v8bf tr_at(const bf16* t, int off, int off2) {
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  const v4i16 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(t + off));
  const v4i16 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(t + off2));
  return __builtin_bit_cast(v8bf, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}
// tile row offset of key_of_row(kt, .) relative to key_of_row(0, .)
__host__ __device__ constexpr int kro(int kt) { return 32 * (kt >> 1) + 4 * (kt & 1); }

// lane offset of the first transposed read of rows k0.. (k0 = 8 (lane >> 4) +
// k_extra), columns c0 + 4 (i & 3)
template <int RC, int (*F)(int)>
__device__ __forceinline__ int tr_first(int k0, int c0, int lane) {
  const int i = lane & 15;
  return toff<RC, F>(k0 + (i >> 2), c0 + 4 * (i & 3));
}

__device__ __forceinline__ float dot4_bf16(const v4f& a, const uint2& q) {
  return a[0] * bf16lo_to_f32(q.x) + a[1] * bf16hi_to_f32(q.x) + a[2] * bf16lo_to_f32(q.y) +
         a[3] * bf16hi_to_f32(q.y);
}
__device__ __forceinline__ uint2 pack4_bf16(const v4f& v) {
  return uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
}
// sum over the 4 lane groups (lanes l, l^16, l^32, l^48)
__device__ __forceinline__ float group_sum(float v) {
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Row sums across the 16 lanes of each lane group: lane li of the group
// returns the sum over the group's lanes of v[li].  Each step pairs lanes that
// differ in one bit of li (row_mirror: bit 3, row_half_mirror: bit 2,
// quad_perm 3210: bit 1, quad_perm 1032: bit 0) and keeps the half of the
// values selected by that bit.
__device__ __forceinline__ float transpose_reduce16(float (&m)[16], int li) {
  {
    const bool up = li & 8;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float a = m[j] + dpp_f<0x140>(m[j]), b = m[j + 8] + dpp_f<0x140>(m[j + 8]);
      m[j] = up ? b : a;
    }
  }
  {
    const bool up = li & 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = m[j] + dpp_f<0x141>(m[j]), b = m[j + 4] + dpp_f<0x141>(m[j + 4]);
      m[j] = up ? b : a;
    }
  }
  {
    const bool up = li & 2;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float a = m[j] + dpp_f<0x1B>(m[j]), b = m[j + 2] + dpp_f<0x1B>(m[j + 2]);
      m[j] = up ? b : a;
    }
  }
  const bool up = li & 1;
  const float a = m[0] + dpp_f<0xB1>(m[0]), b = m[1] + dpp_f<0xB1>(m[1]);
  return up ? b : a;
}

constexpr int kPlaneT = 64 * 64;   // bf16 elements of one 64 x 64 plane tile

// index of this thread's wave in the block, as a wave-uniform (scalar) value
__device__ __forceinline__ int wave_index() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// every outstanding memory operation of the wave has completed (DMA included)
__device__ __forceinline__ void wait_all_mem() { __builtin_amdgcn_s_waitcnt(0); }

// an opaque copy of v: values derived from it are recomputed where they are
// used instead of being hoisted out of loops into long-lived registers
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// ---------------------------------------------------------------------------
// source-strip kernel.  One 256-thread block per (b, c, group, source strip S),
// two blocks per CU.  Wave w owns the source columns sigma = 64 S + 16 w +
// lane % 16.  The block walks the group's heads in passes of HS heads (two,
// or one for a one-head group): du, x_B, ddt, q, r of those heads.  dB and
// the dCB planes need every head of the group.  dB^T stays in registers from
// the first pass to the last (state part of every head, then the intra part
// in the last pass).  dCB of a target strip is summed over the passes in the
// 64 bytes per lane that the last pass overwrites with the hi / lo planes: a
// pass other than the last stores its running fp32 sum there and the next
// pass adds its share to it (each lane reads back only what it wrote).
// Passes other than the last hold their heads' u rows in registers; every
// pass holds the source row's B.
// ---------------------------------------------------------------------------
template <int NK>
struct SrcSmem {
  static constexpr int N = 32 * NK;
  static constexpr int kStage = 2 * kPlaneT;       // bf16: one head's dy tile or dS n half (hi, lo)
  static constexpr int kC = 64 * N;                // bf16: one C tile
};

enum SrcMode { kSrcOnly = 0, kSrcFirst = 1, kSrcMiddle = 2, kSrcLast = 3 };
// pass plans: one pass (at most HS heads), two passes, more than two
enum SrcPlan { kPlanOne = 0, kPlanTwo = 1, kPlanMany = 2 };

template <int NK, int HS, int PLAN>
__global__ __launch_bounds__(256, 2) void ssd_bwd_src_kernel(
    const bf16* __restrict__ u, const bf16* __restrict__ Bm, const bf16* __restrict__ Cm,
    const bf16* __restrict__ dyp, const float* __restrict__ dt, const float* __restrict__ dc,
    const bf16* __restrict__ dSp, const int64_t* __restrict__ length, bf16* __restrict__ du,
    bf16* __restrict__ dB, bf16* __restrict__ dcbp, float* __restrict__ ddt_part,
    float* __restrict__ xB_part, float* __restrict__ qpart, float* __restrict__ rpart,
    SsdDims d, int mono) {
  using SM = SrcSmem<NK>;
  constexpr int N = SM::N;
  constexpr int NH = N / 64;     // 64-wide n halves of a dS tile
  constexpr int NT = N / 16;     // 16-row n tiles of dB^T
  static_assert(NH == 1 || NH == 2, "ssd_bwd_src: state_dim 64 or 128");
  static_assert(HS == 1 || HS == 2, "ssd_bwd_src: one or two heads per pass");
  // One LDS object per stage buffer.  The DMA into them goes through
  // dma_lds16, which the compiler does not see as an LDS write (with the
  // builtin it held LDS accesses and load uses inside a stage until the next
  // stage's DMA had landed); end_stage's wait and barrier order it.
  __shared__ __align__(16) bf16 stg0[SM::kStage];   // [hi, lo][64][64]
  __shared__ __align__(16) bf16 stg1[SM::kStage];
  __shared__ __align__(16) bf16 Cs0[SM::kC];        // [64][N]
  __shared__ __align__(16) bf16 Cs1[SM::kC];
  __shared__ __align__(16) float dcs[2 * HS * 64];   // [T parity][head of the pass][64] dc (log2)
  __shared__ __align__(16) float ats[2 * HS * 64];   // [T parity][head of the pass][64] e^{dc - dc_T0}
  __shared__ __align__(16) float rx[2 * 4 * 64];     // [stage parity][4 waves][64] row sums
  auto stg = [&](int par) -> bf16* { return par ? stg1 : stg0; };
  auto Cs = [&](int par) -> bf16* { return par ? Cs1 : Cs0; };
  const uint32_t l_stg0 = lds_addr(stg0), l_stg1 = lds_addr(stg1);
  const uint32_t l_cs0 = lds_addr(Cs0), l_cs1 = lds_addr(Cs1);

  const int hpg = d.H / d.G;
  const int npass = (hpg + HS - 1) / HS;
  const int stiles = d.Lc / 64;
  const int bid = xcd_swizzle(blockIdx.x, gridDim.x);
  // strip S walks stiles - S target strips: longest first in each window of
  // one XCD's resident blocks, so that launch rounds end on short blocks
  // while a tile's strips still run close together in time (its dy and C
  // tiles are read by every strip from L2)
  int S, rest;
  xcd_window_order(bid, gridDim.x, stiles, S, rest);
  const int g = rest % d.G;
  rest /= d.G;
  const int c = rest % d.nc;
  const int b = rest / d.nc;
  const int s0 = 64 * S;
  const int qlim = min(d.Lc, d.L - c * d.Lc);
  const int len = seq_limit(length, b, d.L);
  const int lim = max(0, chunk_limit(len, c, d.Lc));
  const long tok0 = static_cast<long>(b) * d.L + static_cast<long>(c) * d.Lc;
  const int u_rs = d.H * 64, act_rs = d.G * N;
  const int tid = threadIdx.x, lane = tid & 63, lg = lane >> 4, li = lane & 15;
  const int w = wave_index();
  const int sl = 16 * w + li;        // this lane's source column within the strip
  const int sig = s0 + sl;           // its chunk position
  const int h0 = g * hpg;
  const long bhc0 = (static_cast<long>(b) * d.H + h0) * d.nc + c;   // head k: + k nc
  const int hstride = d.nc * d.Lc;
  const long bcg = (static_cast<long>(b) * d.nc + c) * d.G + g;
  const bf16* uc = u + tok0 * u_rs + h0 * 64;
  const bf16* Bc = Bm + tok0 * act_rs + static_cast<long>(g) * N;
  const bf16* Cc = Cm + tok0 * act_rs + static_cast<long>(g) * N;
  const float* dcc = dc + bhc0 * d.Lc;
  const float* dtc = dt + bhc0 * d.Lc;
  bf16* duc = du + tok0 * u_rs + h0 * 64;
  bf16* dBc = dB + tok0 * act_rs + static_cast<long>(g) * N;
  float* ddtc = ddt_part + bhc0 * d.Lc;
  float* xBc = xB_part + bhc0 * d.Lc;
  float* qc = qpart + bhc0 * d.Lc;
  float* rc = rpart + (bhc0 * stiles + S) * d.Lc;   // head k: + k nc stiles Lc
  const int rstride = d.nc * stiles * d.Lc;

  if (s0 >= lim) {   // the strip is past the length: zero outputs and partials
    for (int e = tid; e < 64 * hpg * 8; e += 256) {
      const int row = e / (hpg * 8), col8 = e % (hpg * 8);
      if (s0 + row < qlim)
        *reinterpret_cast<uint4*>(duc + static_cast<unsigned>((s0 + row) * u_rs + 8 * col8)) = uint4{0u, 0u, 0u, 0u};
    }
    for (int e = tid; e < 64 * (N / 8); e += 256) {
      const int row = e / (N / 8), col8 = e % (N / 8);
      if (s0 + row < qlim)
        *reinterpret_cast<uint4*>(dBc + static_cast<unsigned>((s0 + row) * act_rs + 8 * col8)) = uint4{0u, 0u, 0u, 0u};
    }
    for (int k = 0; k < hpg; ++k) {
      if (tid < 64) {
        ddtc[k * hstride + s0 + tid] = 0.f;
        xBc[k * hstride + s0 + tid] = 0.f;
        qc[k * hstride + s0 + tid] = 0.f;
      }
      for (int t = s0 + tid; t < d.Lc; t += 256) rc[k * rstride + t] = 0.f;
    }
    return;
  }

  const bool sv = sig < lim;
  const int scl = min(sig, lim - 1);       // clamped source row (a valid address)
  const int ntile = (lim + 63) / 64 - S;   // target strips T = S .. S + ntile - 1

  // Stages of a pass: first one state stage per head of the pass, its dS n
  // half 0 in the stage buffer and n half 1 in a C buffer (no C tile is in
  // use before the pair stages); then per target strip T = S + Ti the dy
  // tile of head h = 0..HS-1 of the pass (C_T and the dc tables come with
  // h == 0).  C buffers: strip T's tile goes into buffer (T - S) & 1, and
  // state stage j takes buffer (HS - j) & 1, a compile-time choice (the last
  // state stage takes buffer 1, which the first pair stage's tile does not
  // go into).
  constexpr int nst = HS;
  auto state_cpar = [&](int j) { return (HS - j) & 1; };
  const int n_stage = nst + HS * ntile;
  const bf16* dyg = dyp + (bcg * stiles) * (static_cast<long>(hpg) * 2 * kPlaneT);   // + (T hpg + k) 2 kPlaneT
  const bf16* dSg = dSp + ((static_cast<long>(b) * d.nc + c) * d.H + h0) * (2L * 64 * N);
  constexpr int RCB = N / 8;   // 16-byte chunks of a dB row

  // this lane's 64 bytes of the dCB tile (S, Tp): chunk q = 2 ks + (hi, lo)
  // holds dCB[tau = 64 Tp + 32 ks + 8 lg .. + 7][sigma = sig] of that plane.
  // The tile is stored in lane order, chunk q of lane (lg, li) of wave w at
  // byte 4096 q + 16 (64 w + 4 li + lg): each store instruction of a wave
  // writes 1 KB of whole cache lines, and the four chunks of one sigma row
  // (lg = 0..3) are 64 contiguous bytes for the target kernel's DMA, which
  // puts the chunks back into [sigma][tau] order (dcb_lane_off).
  auto dcb_at = [&](int Tp, int q) -> bf16* {
    return dcbp + ((bcg * stiles + S) * stiles + Tp) * (2L * kPlaneT) + q * 2048 +
           (w * 64 + li * 4 + lg) * 8;
  };

  // dB^T rows n = 16 nt + 4 lg + r, column sig: the state part of every head
  // (every pass), then the intra part (last pass)
  v4f dBT[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) dBT[nt] = v4f{0.f, 0.f, 0.f, 0.f};

  // one pass over heads KB .. KB + HS - 1 (those < hpg)
  auto run_pass = [&](auto mode_c, const int pass) {
    constexpr int MODE = decltype(mode_c)::value;
    constexpr bool last = MODE == kSrcOnly || MODE == kSrcLast;
    constexpr bool first = MODE == kSrcOnly || MODE == kSrcFirst;
    const int KB = pass * HS;
    float pdc = 0.f, pdc0 = 0.f;   // dc prefetch of the next target strip (head tid / 64, row tid % 64)
    // Values derived from the lane id are recomputed in each pass (and the
    // DMA lane offsets where a stage is issued, a few integer operations
    // each) from an opaque copy of it, so that none of them is held in a
    // register from one pass to the next.
    const int lnp = opaque(lane);
    const int lgp = lnp >> 4, lip = lnp & 15;
    auto lane_offsets = [&](int (&gs)[2], int (&gy)[2], int (&gc)[NK]) {
      const int ln = opaque(lane);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        gs[i] = dma_off<8, swz_r128>(i, w, ln, N);
        gy[i] = dma_off<8, swz_r128>(i, w, ln, 64);
      }
#pragma unroll
      for (int i = 0; i < NK; ++i) gc[i] = dma_off<NK * 4, swz_c<NK>>(i, w, ln, act_rs);
    };
    // per-lane element offsets of the fragment reads inside a tile (the
    // swizzle of every row this lane reads depends on lane bits only, so
    // each read is a precomputed offset plus a compile-time constant)
    const int rl = 8 * (lip >> 2) + (lip & 3);   // key_of_row(kt, li) = rl + kro(kt)
    int o_w[2], o_tr[4], o_c[NK];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) o_w[ks] = toff<8, swz_r128>(rl, 32 * ks + 8 * lgp);
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) o_tr[pt] = tr_first<8, swz_r128>(8 * lgp, 16 * pt, lnp);
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) o_c[ks] = toff<NK * 4, swz_c<NK>>(rl, 32 * ks + 8 * lgp);
    // B of this lane's source row (all N): the same in every stage of the pass
    const bf16* brow = Bc + static_cast<unsigned>(scl * act_rs + 8 * lgp);
    v8bf Bh[NK];
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) Bh[ks] = sv ? load_v8bf(brow + 32 * ks) : zero_v8bf();
    auto issue = [&](int j, int par) {   // par: the stage's buffer
      const uint32_t dst = par ? l_stg1 : l_stg0;
      int gs[2], gy[2], gc[NK];
      lane_offsets(gs, gy, gc);
      if (j < nst) {
        const int k = KB + j;
        if (k < hpg) {
          const bf16* src = dSg + k * (2L * 64 * N);
          const uint32_t cdst = state_cpar(j) ? l_cs1 : l_cs0;
          dma_pre_op<8>(dst, src, gs, w);
          dma_pre_op<8>(dst + 2 * kPlaneT, src + 64L * N, gs, w);
          if constexpr (NH == 2) {
            dma_pre_op<8>(cdst, src + 64, gs, w);
            dma_pre_op<8>(cdst + 2 * kPlaneT, src + 64 + 64L * N, gs, w);
          }
        }
      } else {
        const int qq = j - nst, Ti = qq / HS, h = qq % HS, T = S + Ti, k = KB + h;
        if (k < hpg) {
          const bf16* src = dyg + (static_cast<long>(T) * hpg + k) * (2L * kPlaneT);
          dma_pre_op<8>(dst, src, gy, w);
          dma_pre_op<8>(dst + 2 * kPlaneT, src + kPlaneT, gy, w);
        }
        if (h == 0) {
          const int t0 = 64 * T;
          const uint32_t cdst = ((T - S) & 1) ? l_cs1 : l_cs0;
          const bf16* csrc = Cc + static_cast<long>(t0) * act_rs;
          if (qlim - t0 >= 64) dma_pre_op<NK * 4>(cdst, csrc, gc, w);
          else dma_tile_op<NK * 4, swz_c<NK>>(cdst, csrc, act_rs, qlim - t0, w, lane);
          if (tid < HS * 64) {   // raw: nothing waits for these before the stage's end
            const int k2 = min(KB + (tid >> 6), hpg - 1);
            const float* dch = dcc + k2 * hstride + t0;
            pdc = dch[tid & 63];
            pdc0 = dch[0];
          }
        }
      }
    };
    // the next stage after stage j (buffer par) of this pass
    auto issue_next = [&](int j, int par) {
      if (j + 1 < n_stage) issue(j + 1, par ^ 1);
    };
    // end of the stage before stage j: the dc tables of a new target strip,
    // then every DMA of the next stage complete and visible
    auto end_stage = [&](int j) {
      if (j < n_stage && j >= nst && (j - nst) % HS == 0 && tid < HS * 64) {
        const int T = S + (j - nst) / HS;
        dcs[(T & 1) * HS * 64 + tid] = pdc * kLog2e;
        ats[(T & 1) * HS * 64 + tid] = fast_exp2(fminf(pdc * kLog2e - pdc0 * kLog2e, 0.f));
      }
      wait_all_mem();
      __syncthreads();
    };
    auto flush_r = [&](int j, int par) {   // the row sums pair stage j left in LDS -> rpart
      const int qq = j - nst, Ti = qq / HS, k = KB + qq % HS;
      if (tid < 64 && k < hpg) {
        const float* rr = rx + par * 256;
        rc[k * rstride + 64 * (S + Ti) + tid] = rr[tid] + rr[64 + tid] + rr[128 + tid] + rr[192 + tid];
      }
    };

    // u rows of this pass' heads: held for the whole pass by the first pass.
    // The others (which hold the running dCB sum or finish dB) have no
    // registers to spare: they hold the u row of one head (un), the one the
    // next stage needs (stages walk the pass' heads in turn, starting with
    // KB), reloaded in each stage once that stage's last use of it is done,
    // so that no stage waits on a load (which would also wait for the DMA
    // issued before it).  Rows past the length are zeroed where used.  A
    // stage of an absent head (KB + h >= hpg, only h = 1 with KB = hpg - 1)
    // loads nothing: un then holds head hpg - 1 = KB, what the next stage
    // (head KB) needs.
    constexpr bool kHold = first && !last;
    v8bf Uh[HS][2];
    v8bf un[2];
    auto load_un = [&](int h) {   // u row of head KB + h (clamped to a valid head)
      const bf16* urow = uc + min(KB + h, hpg - 1) * 64 + static_cast<unsigned>(scl * u_rs + 8 * lg);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) un[ks] = load_v8bf(urow + 32 * ks);
    };
    auto use_un = [&](v8bf (&f)[2]) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) f[ks] = sv ? un[ks] : zero_v8bf();
    };
    if constexpr (kHold) {
#pragma unroll
      for (int h = 0; h < HS; ++h) {
        const int k = KB + h;
        const bf16* urow = uc + min(k, hpg - 1) * 64 + static_cast<unsigned>(scl * u_rs + 8 * lg);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          Uh[h][ks] = sv && k < hpg ? load_v8bf(urow + 32 * ks) : zero_v8bf();
      }
    } else {
      load_un(0);
    }
    // this pass' dc and dt at the source row and dc at the chunk end: loaded
    // ahead of the first stage's DMA and landed by its wait (a load used in
    // a stage waits for the DMA issued before it as well)
    float dcr[HS], dtr[HS], dcl[HS];
    uint2 uxh[HS][4];   // u of head KB + h at this lane's column, for x_B
#pragma unroll
    for (int h = 0; h < HS; ++h) {
      const int k = min(KB + h, hpg - 1);
      dcr[h] = dcc[k * hstride + scl];
      dtr[h] = dtc[k * hstride + scl];
      dcl[h] = dcc[k * hstride + d.Lc - 1];
      const bf16* urow4 = uc + k * 64 + static_cast<unsigned>(scl * u_rs + 4 * lg);
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) uxh[h][pt] = *reinterpret_cast<const uint2*>(urow4 + 16 * pt);
    }
    asm volatile("" ::: "memory");   // the loads stay ahead of the wait
    issue(0, nst & 1);   // stage j has buffer parity (j + nst) & 1
    wait_all_mem();
    __syncthreads();

    v4f duT[HS][4];   // du^T of this pass' heads: rows p = 16 pt + 4 lg + r, column sig
    float qacc[HS], dtk[HS], dck[HS], ekh[HS];
#pragma unroll
    for (int h = 0; h < HS; ++h) {
      dck[h] = dcr[h] * kLog2e;
      dtk[h] = sv ? dtr[h] : 0.f;
      // e^{min(dc_last - dc_sig, 0)}: the state weight is ekh dt
      ekh[h] = fast_exp2(fminf(dcl[h] * kLog2e - dck[h], 0.f));
      qacc[h] = 0.f;
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) duT[h][pt] = v4f{0.f, 0.f, 0.f, 0.f};
    }

    // ---- state stages: dB^T += w dS^T.u^T, du^T += dS.B^T ----
    {
      int o_sd[2], o_st[4][2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) o_sd[ks] = toff<8, swz_r128>(li, 32 * ks + 8 * lg);
#pragma unroll
      for (int nt4 = 0; nt4 < 4; ++nt4) {
        o_st[nt4][0] = tr_first<8, swz_r128>(8 * lg, 16 * nt4, lane);
        o_st[nt4][1] = tr_first<8, swz_r128>(8 * lg + 4, 16 * nt4, lane);
      }
      // dB^T rows of the n half in stage buffer Y from a head's dS, its u row
      // uf at this lane's column and its state weight wk
      auto state_dB = [&](const bf16* Yh, const v8bf (&uf)[2], float wk, int half) {
        const bf16* Yl = Yh + kPlaneT;
#pragma unroll
        for (int nt4 = 0; nt4 < 4; ++nt4) {
          v4f tmp = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const int a0 = o_st[nt4][0] + 32 * ks * 64, a1 = o_st[nt4][1] + 32 * ks * 64;
            tmp = mfma_bf16(tr_at(Yh, a0, a1), uf[ks], tmp);
            tmp = mfma_bf16(tr_at(Yl, a0, a1), uf[ks], tmp);
          }
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2)   // constant register index of dBT
            if (h2 == half) dBT[4 * h2 + nt4] += tmp * wk;
        }
      };
#pragma unroll
      for (int h = 0; h < HS; ++h) {
        const int k = KB + h;
        const bool kv = k < hpg;
        const int j = h, par = (h + HS) & 1;
        v8bf ul[2] = {Uh[h][0], Uh[h][1]};
        if constexpr (!kHold) use_un(ul);
        issue_next(j, par);
        if (kv) {
#pragma unroll
          for (int half = 0; half < NH; ++half) {
            const bf16* Yh = half ? Cs(state_cpar(j)) : stg(par);
            const bf16* Yl = Yh + kPlaneT;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
              for (int pt = 0; pt < 4; ++pt) {
                const int off = o_sd[ks] + 16 * pt * 64;
                duT[h][pt] = mfma_bf16(load_v8bf(Yh + off), Bh[2 * half + ks], duT[h][pt]);
                duT[h][pt] = mfma_bf16(load_v8bf(Yl + off), Bh[2 * half + ks], duT[h][pt]);
              }
            state_dB(Yh, ul, ekh[h] * dtk[h], half);
            // the next stage's u row (the next head of the pass)
            if (!kHold && half == NH - 1) load_un((h + 1) % HS);
            __builtin_amdgcn_sched_barrier(0);   // the halves' operand reads stay apart
          }
          // head k's state part is complete: scale by e^{dc_last - dc_sig}; x_B
          const float ek = ekh[h];
          float sx = 0.f;
#pragma unroll
          for (int pt = 0; pt < 4; ++pt) {
            duT[h][pt] *= ek;
            sx += dot4_bf16(duT[h][pt], uxh[h][pt]);
          }
          sx = group_sum(sv ? sx : 0.f) * dtk[h];
          if (lg == 0) xBc[k * hstride + sig] = sx;
        }
        end_stage(j + 1);
      }
    }

    // the dCB of target strip Tp: store this pass' running sum (fp32, in the
    // bytes of the planes), or (last pass) finish it: dB^T[n, sig] += sum_t
    // C[t, n] dCB[t, sig] and store the hi / lo planes
    // (prev: the running sum of the passes before, loaded at the end of the
    // stage before)
    auto load_prev = [&](int Tp, float4 (&prev)[4]) {
      if constexpr (!first) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) prev[kt] = *reinterpret_cast<const float4*>(dcb_at(Tp, kt));
      }
    };
    auto finish_pair = [&](int Tp, v4f (&dCBa)[4], const float4 (&prev)[4]) {
      if constexpr (!first) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) dCBa[kt] += v4f{prev[kt].x, prev[kt].y, prev[kt].z, prev[kt].w};
      }
      if constexpr (!last) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
          *reinterpret_cast<float4*>(dcb_at(Tp, kt)) = make_float4(dCBa[kt][0], dCBa[kt][1], dCBa[kt][2], dCBa[kt][3]);
        return;
      }
      const bf16* Cb = Cs((Tp - S) & 1);
      const int ctb = tr_first<NK * 4, swz_c<NK>>(8 * lg, 0, lane);   // column tile 0
      const int cfx = 16 * (swz_r256(8 * lg + ((lane & 15) >> 2)) >> 1);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        v8bf dh, dl;
        split_p(dCBa[2 * ks], dCBa[2 * ks + 1], dh, dl);
        *reinterpret_cast<v8bf*>(dcb_at(Tp, 2 * ks)) = dh;
        *reinterpret_cast<v8bf*>(dcb_at(Tp, 2 * ks + 1)) = dl;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          v8bf a;
          if constexpr (NK == 4) {
            // column tile nt: chunk pair nt of the row, XOR-swizzled
            const int a0 = ctb - (cfx & 0x70) + (((16 * nt) ^ cfx) & 0x70) + 32 * ks * N;
            a = tr_at(Cb, a0, a0 + 4 * N);
          } else {
            a = tr_frag<8, swz_r128>(Cb, 32 * ks + 8 * lg, 16 * nt, lane);
          }
          dBT[nt] = mfma_bf16(a, dh, dBT[nt]);
          dBT[nt] = mfma_bf16(a, dl, dBT[nt]);
          if (nt & 1) __builtin_amdgcn_sched_barrier(0);
        }
      }
    };

    // ---- pair stages: target strip T = S + Ti, head k = KB + h ----
    v4f dCBa[4];
    float4 prev[4];
    for (int Ti = 0; Ti < ntile; ++Ti) {
      const int T = S + Ti, t0 = 64 * T;
      const bf16* Cb = Cs((T - S) & 1);
      const bool diag = Ti == 0;
      const bool fact = !diag && mono;
      v4f CB[4];
#pragma unroll
      for (int h = 0; h < HS; ++h) {
        const int j = nst + Ti * HS + h;
        const int k = KB + h;
        const bool kv = k < hpg;
        const int par = HS == 1 ? (Ti & 1) : h;
        v8bf uf[2] = {Uh[h][0], Uh[h][1]};
        if constexpr (!kHold) use_un(uf);
        // with one head per pass, the next stage brings the C tile of strip
        // T + 1 into the buffer finish_pair(T - 1) reads: finish it first
        if (HS == 1 && Ti > 0) {
          finish_pair(T - 1, dCBa, prev);
          __syncthreads();
        }
        issue_next(j, par);
        if (j > nst) flush_r(j - 1, par ^ 1);
        if (HS > 1 && h == 0 && Ti > 0) finish_pair(T - 1, dCBa, prev);
        const bf16* Yh = stg(par);
        const bf16* Yl = Yh + kPlaneT;
        if (h == 0) {
#pragma unroll
          for (int kt = 0; kt < 4; ++kt) {
            CB[kt] = v4f{0.f, 0.f, 0.f, 0.f};
            dCBa[kt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < NK; ++ks)
              CB[kt] = mfma_bf16(load_v8bf(Cb + o_c[ks] + kro(kt) * N), Bh[ks], CB[kt]);
          }
        }
        if (kv) {
          const float* dcT = dcs + (T & 1) * HS * 64 + 64 * h;
          const float* atT = ats + (T & 1) * HS * 64 + 64 * h;
          const float dk = dck[h], dtv = dtk[h];
          // W[t, sig] = dy[t] . u[sig]
          // the four row tiles' accumulators in turn, one (k step, plane)
          // slice at a time: no MFMA waits on the one before it
          v4f W[4];
#pragma unroll
          for (int kt = 0; kt < 4; ++kt) W[kt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int q2 = 0; q2 < 4; ++q2) {
            const int ks = q2 >> 1;
            const bf16* Yp = (q2 & 1) ? Yl : Yh;
            v8bf f[4];
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) f[kt] = load_v8bf(Yp + o_w[ks] + kro(kt) * 64);
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) W[kt] = mfma_bf16(f[kt], uf[ks], W[kt]);
            __builtin_amdgcn_sched_barrier(0);   // bound the operand reads in flight
          }
          if constexpr (!kHold) load_un((h + 1) % HS);   // the next stage's u row
          // decay and masks: dCB += W', M = W' o CB (q: column sums, r: row sums); W <- L
          float m[16];
          float qs = 0.f;
          if (fact) {
            // off the diagonal with a monotone dc, e^{min(dc_t - dc_sig, 0)} =
            // e^{min(dc_t - dc_t0, 0)} e^{min(dc_t0 - dc_sig, 0)}
            const float bk = fast_exp2(fminf(dcT[0] - dk, 0.f));
            const float bdt = bk * dtv;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
              const int tb = 32 * (kt >> 1) + 8 * lg + 4 * (kt & 1);
              const float4 aq = *reinterpret_cast<const float4*>(atT + tb);
              const float av[4] = {aq.x, aq.y, aq.z, aq.w};
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const float wv = W[kt][r] * (av[r] * bdt);
                dCBa[kt][r] += wv;
                const float mv = wv * CB[kt][r];
                m[4 * kt + r] = mv;
                qs += mv;
                W[kt][r] = CB[kt][r] * (av[r] * bk);
              }
            }
          } else {
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
              const int tb = 32 * (kt >> 1) + 8 * lg + 4 * (kt & 1);
              const float4 dq = *reinterpret_cast<const float4*>(dcT + tb);
              const float dv[4] = {dq.x, dq.y, dq.z, dq.w};
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int t = t0 + tb + r;
                float dec = fast_exp2(fminf(dv[r] - dk, 0.f));
                dec = (t >= sig && t < lim) ? dec : 0.f;
                const float wv = W[kt][r] * dtv * dec;
                dCBa[kt][r] += wv;
                const float mv = t > sig ? wv * CB[kt][r] : 0.f;
                m[4 * kt + r] = mv;
                qs += mv;
                W[kt][r] = CB[kt][r] * dec;
              }
            }
          }
          qacc[h] += qs;
          rx[par * 256 + w * 64 + key_of_row(li >> 2, 4 * lg + (li & 3))] =
              transpose_reduce16(m, li);
          // du^T[p, sig] += sum_t dy[t, p] L[t, sig]  (L and dy as hi + lo)
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            v8bf lh, ll;
            split_p(W[2 * ks], W[2 * ks + 1], lh, ll);
#pragma unroll
            for (int pt = 0; pt < 4; ++pt) {
              const int a0 = o_tr[pt] + 32 * ks * 64;
              const v8bf yh = tr_at(Yh, a0, a0 + 4 * 64);
              const v8bf yl = tr_at(Yl, a0, a0 + 4 * 64);
              duT[h][pt] = mfma_bf16(yh, lh, duT[h][pt]);
              duT[h][pt] = mfma_bf16(yl, lh, duT[h][pt]);
              duT[h][pt] = mfma_bf16(yh, ll, duT[h][pt]);
              if (pt & 1) __builtin_amdgcn_sched_barrier(0);
            }
          }
        }
        // the running dCB sum of the passes before, for finish_pair in the
        // next stage
        if (h == HS - 1) load_prev(T, prev);
        end_stage(j + 1);
      }
    }
    flush_r(n_stage - 1, HS == 1 ? ((ntile - 1) & 1) : HS - 1);
    finish_pair(S + ntile - 1, dCBa, prev);
    // every wave is done with the stage buffers: they stage du (stg0) and,
    // after the last pass, dB (stg1)
    __syncthreads();

    // ---- du, ddt_direct, q of this pass' heads ----
#pragma unroll
    for (int h = 0; h < HS; ++h) {
      const int k = KB + h;
      if (k >= hpg) continue;
      const bf16* urow = uc + k * 64 + static_cast<unsigned>(scl * u_rs + 4 * lg);
      float sx = 0.f;
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) sx += dot4_bf16(duT[h][pt], *reinterpret_cast<const uint2*>(urow + 16 * pt));
      sx = group_sum(sv ? sx : 0.f);
      const float qv = group_sum(qacc[h]);
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) stage_out8<8>(stg0 + h * 4096, sl, 16 * pt + 4 * lg, pack4_bf16(duT[h][pt] * dtk[h]));
      if (lg == 0) {
        ddtc[k * hstride + sig] = sx;
        qc[k * hstride + sig] = qv;
      }
    }
    // row-sum partials of target strips past the length are zero
    for (int k = KB; k < min(KB + HS, hpg); ++k)
      for (int t = 64 * (S + ntile) + tid; t < d.Lc; t += 256) rc[k * rstride + t] = 0.f;
    if constexpr (last) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) stage_out8<RCB>(stg1, sl, 16 * nt + 4 * lg, pack4_bf16(dBT[nt]));
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < HS; ++h)
      if (KB + h < hpg) write_rows<8>(stg0 + h * 4096, duc + (KB + h) * 64 + s0 * u_rs, u_rs, qlim - s0, tid);
    if constexpr (last) write_rows<RCB>(stg1, dBc + s0 * act_rs, act_rs, qlim - s0, tid);
    // the next pass' first DMA goes into these buffers
    if constexpr (!last) __syncthreads();
  };

  // one instantiation per pass plan, so that a launch carries only the pass
  // bodies it runs (each body is 20-25 KB of code)
  if constexpr (PLAN == kPlanOne) {
    run_pass(std::integral_constant<int, kSrcOnly>{}, 0);
  } else if constexpr (PLAN == kPlanTwo) {
    run_pass(std::integral_constant<int, kSrcFirst>{}, 0);
    run_pass(std::integral_constant<int, kSrcLast>{}, 1);
  } else {
    run_pass(std::integral_constant<int, kSrcFirst>{}, 0);
    for (int pass = 1; pass + 1 < npass; ++pass)
      run_pass(std::integral_constant<int, kSrcMiddle>{}, pass);
    run_pass(std::integral_constant<int, kSrcLast>{}, npass - 1);
  }
}

// ---------------------------------------------------------------------------
// target-strip kernel: dC and x_C.  One block per (b, c, group, target strip
// T, half of N): the two halves of a strip split every product over n (no
// MFMA is done twice), run side by side (half is the fastest block index)
// and share dy and the dCB tiles through L2.  A stage is 24 KB of LDS and a
// block holds two, so three blocks share a CU.  x_C is a sum over n: each
// half writes its own partial (slot 2 bhc + half).
// ---------------------------------------------------------------------------
template <int NK>
struct TgtSmem {
  static constexpr int NHALF = NK / 2;   // blocks per target strip (64 n each)
  static constexpr int NH = 32 * NK / NHALF;   // n of one block
  // a stage: this half of H_in of one head (hi, lo: 2 x 64 x NH) or this
  // half of B_S (64 x NH) + dCB^T (hi, lo: 2 x 64 x 64)
  static constexpr int kStage = 2 * 64 * NH > 64 * NH + 2 * kPlaneT ? 2 * 64 * NH : 64 * NH + 2 * kPlaneT;
  static constexpr size_t bytes = 2 * kStage * 2;
};

template <int NK>
__global__ __launch_bounds__(256, 3) void ssd_bwd_tgt_kernel(
    const bf16* __restrict__ Bm, const bf16* __restrict__ Cm, const bf16* __restrict__ dyp,
    const float* __restrict__ dc, const float* __restrict__ states,
    const bf16* __restrict__ dcbp, const int64_t* __restrict__ length, bf16* __restrict__ dC,
    float* __restrict__ xC_part, SsdDims d) {
  using SM = TgtSmem<NK>;
  constexpr int N = 32 * NK;
  constexpr int NH = SM::NH;
  static_assert(NH == 64, "ssd_bwd_tgt: state_dim 128");
  constexpr int NTH = NH / 16;   // n tiles of this half
  extern __shared__ __align__(16) unsigned char smem_raw[];
  bf16* stg = reinterpret_cast<bf16*>(smem_raw);   // [2][kStage]

  const int HPG = d.H / d.G;
  const int ttiles = d.Lc / 64;
  constexpr int NHALF = SM::NHALF;
  const int bid = xcd_swizzle(blockIdx.x, gridDim.x);
  const int half = NHALF == 2 ? (bid & 1) : 0;
  int rest = NHALF == 2 ? (bid >> 1) : bid;
  // target strip T walks T + 1 source strips: longest first in windows of one
  // XCD's resident blocks (three per CU, the two halves of a tile adjacent:
  // 48 tile pairs)
  int T;
  xcd_window_order<48>(rest, gridDim.x / NHALF, ttiles, T, rest);
  T = ttiles - 1 - T;
  const int g = rest % d.G;
  rest /= d.G;
  const int c = rest % d.nc;
  const int b = rest / d.nc;
  const int t0 = 64 * T, n0 = NH * half;
  const int qlim = min(d.Lc, d.L - c * d.Lc);
  const int len = seq_limit(length, b, d.L);
  const int lim = max(0, chunk_limit(len, c, d.Lc));
  const long tok0 = static_cast<long>(b) * d.L + static_cast<long>(c) * d.Lc;
  const int act_rs = d.G * N;
  const int tid = threadIdx.x, lane = tid & 63, lg = lane >> 4, li = lane & 15;
  const int w = wave_index();
  const int tl = 16 * w + li;   // this lane's target row within the strip
  const int tau = t0 + tl;
  const int h0 = g * HPG;
  const long bhc0 = (static_cast<long>(b) * d.H + h0) * d.nc + c;
  const int hstride = d.nc * d.Lc;
  const long bcg = (static_cast<long>(b) * d.nc + c) * d.G + g;
  const bf16* Bc = Bm + tok0 * act_rs + static_cast<long>(g) * N + n0;
  const bf16* Cc = Cm + tok0 * act_rs + static_cast<long>(g) * N + n0;
  const float* Hc = states + ((static_cast<long>(b) * d.nc + c) * d.H + h0) * (64L * N) + n0;
  const float* dcc = dc + bhc0 * d.Lc;
  bf16* dCc = dC + tok0 * act_rs + static_cast<long>(g) * N + n0;
  float* xCc = xC_part + (bhc0 * NHALF + half) * d.Lc;   // head k: + NHALF k hstride

  if (t0 >= lim) {
    for (int e = tid; e < 64 * (NH / 8); e += 256) {
      const int row = e / (NH / 8), col8 = e % (NH / 8);
      if (t0 + row < qlim)
        *reinterpret_cast<uint4*>(dCc + static_cast<unsigned>((t0 + row) * act_rs + 8 * col8)) = uint4{0u, 0u, 0u, 0u};
    }
    for (int k = 0; k < HPG; ++k)
      if (tid < 64) xCc[NHALF * k * hstride + t0 + tid] = 0.f;
    return;
  }

  const int tcl = min(tau, qlim - 1);   // clamped target row (a valid address)
  // C of this lane's row at the dC^T fragment positions n = n0 + 16 nt + 4 lg + r
  uint2 cv[NTH];
  {
    const bf16* crow = Cc + static_cast<unsigned>(tcl * act_rs + 4 * lg);
#pragma unroll
    for (int nt = 0; nt < NTH; ++nt) cv[nt] = *reinterpret_cast<const uint2*>(crow + 16 * nt);
  }
  // dy planes of this lane's row: [head][k step][hi, lo]
  const bf16* dyg = dyp + ((bcg * ttiles + T) * HPG) * (2L * kPlaneT) + tl * 64 + 8 * lg;
  auto load_dy = [&](int k, v8bf (&f)[2][2]) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      f[ks][0] = load_v8bf(dyg + k * (2L * kPlaneT) + 32 * ks);
      f[ks][1] = load_v8bf(dyg + k * (2L * kPlaneT) + kPlaneT + 32 * ks);
    }
  };

  // stage j: j < HPG: this half of H_in of head j (fp32 -> hi, lo through
  // registers); then S = j - HPG = 0..T: this half of B_S and dCB^T of (S, T) by DMA
  const int nstage = HPG + T + 1;
  float4 ph[4];   // H prefetch: row tid / 4, columns n0 + 16 (tid % 4) .. +15
  float dce_n;    // dc of this lane's row for the prefetched head
  auto load_h = [&](int k) {
    dce_n = dcc[k * hstride + tcl];
    const float* src = Hc + k * (64L * N) + (tid >> 2) * N + 16 * (tid & 3);
#pragma unroll
    for (int i = 0; i < 4; ++i) ph[i] = *reinterpret_cast<const float4*>(src + 4 * i);
  };
  auto commit_h = [&](int jj) {
    bf16* dst = stg + (jj & 1) * SM::kStage;
    const int row = tid >> 2;
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {   // 16-byte chunks 2 (tid % 4) + cc
      const float v[8] = {ph[2 * cc].x, ph[2 * cc].y, ph[2 * cc].z, ph[2 * cc].w,
                          ph[2 * cc + 1].x, ph[2 * cc + 1].y, ph[2 * cc + 1].z, ph[2 * cc + 1].w};
      uint32_t hi[4], lo[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        hi[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
        lo[e] = pack_bf16x2(v[2 * e] - bf16lo_to_f32(hi[e]), v[2 * e + 1] - bf16hi_to_f32(hi[e]));
      }
      const int off = toff<8, swz_k128>(row, 8 * (2 * (tid & 3) + cc));
      *reinterpret_cast<uint4*>(dst + off) = uint4{hi[0], hi[1], hi[2], hi[3]};
      *reinterpret_cast<uint4*>(dst + 64 * NH + off) = uint4{lo[0], lo[1], lo[2], lo[3]};
    }
  };
  // The intra stages' DMA goes through dma_lds16, which the compiler does not
  // see as an LDS write: with the builtin it held every stage's first LDS
  // read until the next stage's DMA (issued just before) had landed, so no
  // load overlapped any compute.  The end-of-stage wait and barrier order
  // the DMA before the next stage's reads.  Lane offsets in bytes: B tile
  // row brow[i], swizzled column bcol[i]; the dCB planes in lane order.
  int brow[2], bcol[2];
  uint32_t o_bt[2], o_dcb[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int pos = (w * 2 + i) * 64 + lane;
    brow[i] = pos >> 3;
    bcol[i] = 8 * ((pos & 7) ^ (swz_k128(brow[i]) & 7));
    o_bt[i] = 2u * static_cast<uint32_t>(brow[i] * act_rs + bcol[i]);
    o_dcb[i] = 2u * static_cast<uint32_t>(dcb_lane_off(i, w, lane));
  }
  const uint32_t lds_st = lds_addr(stg), lds_wave = static_cast<uint32_t>(2 * w) << 10;
  auto issue_intra = [&](int jj) {
    const int S = jj - HPG;
    const uint32_t base = lds_st + static_cast<uint32_t>((jj & 1) * SM::kStage * 2);
    const int qv = min(64, qlim - 64 * S);   // rows past it repeat row qv - 1
    const bf16* bsrc = Bc + static_cast<long>(64 * S) * act_rs;
    const bf16* src = dcbp + ((bcg * ttiles + S) * ttiles + T) * (2L * kPlaneT);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t ob = qv < 64 ? 2u * static_cast<uint32_t>(min(brow[i], qv - 1) * act_rs + bcol[i]) : o_bt[i];
      dma_lds16(bsrc, ob, base + lds_wave + (i << 10));
      dma_lds16(src, o_dcb[i], base + 2 * 64 * NH + lds_wave + (i << 10));
      dma_lds16(src, o_dcb[i] + 4096u, base + 2 * (64 * NH + kPlaneT) + lds_wave + (i << 10));
    }
  };

  v4f dCT[NTH];   // dC^T rows n = n0 + 16 nt + 4 lg + r, column tau
#pragma unroll
  for (int nt = 0; nt < NTH; ++nt) dCT[nt] = v4f{0.f, 0.f, 0.f, 0.f};
  v8bf dyf[2][2], dyn[2][2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) dyn[ks][0] = dyn[ks][1] = zero_v8bf();
  load_h(0);
  load_dy(0, dyf);
  float dce = dce_n;
  commit_h(0);
  // The loads before the loop land here (the empty asm statements take their
  // values).  Left to itself the compiler sinks them into the first stage,
  // and its waits for them inside the loop also hold every stage's prefetch.
  asm volatile("" : "+v"(dce));
#pragma unroll
  for (int nt = 0; nt < NTH; ++nt) asm volatile("" : "+v"(cv[nt]));
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) asm volatile("" : "+v"(dyf[ks][0]), "+v"(dyf[ks][1]));
  __syncthreads();

  // x_C of head j is stored at the start of stage j + 1, before that stage's
  // loads, so that the end-of-stage wait does not wait for the store
  float xs = 0.f;
  for (int j = 0; j < nstage; ++j) {
    if (j >= 1 && j - 1 < HPG && lg == 0) xCc[NHALF * (j - 1) * hstride + tau] = tau < lim ? xs : 0.f;
    if (j + 1 < HPG) {
      load_h(j + 1);
      load_dy(j + 1, dyn);
    } else if (j + 1 < nstage) {
      issue_intra(j + 1);
    }
    const bf16* Sg = stg + (j & 1) * SM::kStage;
    if (j < HPG) {
      // X^T[n, tau] = sum_p H[p, n] dy[tau, p]; dC^T += e^{dc_tau} X^T; x_C
      v4f X[NTH];
#pragma unroll
      for (int nt = 0; nt < NTH; ++nt) X[nt] = v4f{0.f, 0.f, 0.f, 0.f};
      // the H fragments of column tile nt + 1 are read while tile nt's MFMAs run
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        v8bf hh_n = tr_frag<8, swz_k128>(Sg, 32 * ks + 8 * lg, 0, lane);
        v8bf hl_n = tr_frag<8, swz_k128>(Sg + 64 * NH, 32 * ks + 8 * lg, 0, lane);
#pragma unroll
        for (int nt = 0; nt < NTH; ++nt) {
          const v8bf hh = hh_n, hl = hl_n;
          if (nt + 1 < NTH) {
            hh_n = tr_frag<8, swz_k128>(Sg, 32 * ks + 8 * lg, 16 * (nt + 1), lane);
            hl_n = tr_frag<8, swz_k128>(Sg + 64 * NH, 32 * ks + 8 * lg, 16 * (nt + 1), lane);
          }
          __builtin_amdgcn_sched_barrier(0);
          X[nt] = mfma_bf16(hh, dyf[ks][0], X[nt]);
          X[nt] = mfma_bf16(hl, dyf[ks][0], X[nt]);
          X[nt] = mfma_bf16(hh, dyf[ks][1], X[nt]);
        }
      }
      const float e = fast_exp2(dce * kLog2e);
      float s = 0.f;
#pragma unroll
      for (int nt = 0; nt < NTH; ++nt) {
        X[nt] *= e;
        s += dot4_bf16(X[nt], cv[nt]);
        dCT[nt] += X[nt];
      }
      xs = group_sum(s);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        dyf[ks][0] = dyn[ks][0];
        dyf[ks][1] = dyn[ks][1];
      }
      dce = dce_n;
    } else {
      // dC^T[n, tau] += sum_sig B[sig, n] dCB[tau, sig]
      const bf16* Bt = Sg;
      const bf16* Dh = Sg + 64 * NH;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const v8bf bh = tr_frag<8, swz_k128>(Dh, 32 * ks + 8 * lg, 16 * w, lane);
        const v8bf bl = tr_frag<8, swz_k128>(Dh + kPlaneT, 32 * ks + 8 * lg, 16 * w, lane);
        v8bf a_n = tr_frag<8, swz_k128>(Bt, 32 * ks + 8 * lg, 0, lane);
#pragma unroll
        for (int nt = 0; nt < NTH; ++nt) {
          const v8bf a = a_n;
          if (nt + 1 < NTH) a_n = tr_frag<8, swz_k128>(Bt, 32 * ks + 8 * lg, 16 * (nt + 1), lane);
          __builtin_amdgcn_sched_barrier(0);
          dCT[nt] = mfma_bf16(a, bh, dCT[nt]);
          dCT[nt] = mfma_bf16(a, bl, dCT[nt]);
        }
      }
    }
    if (j + 1 < HPG) commit_h(j + 1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  // (the loop ended with a barrier: the stage buffers are free)
#pragma unroll
  for (int nt = 0; nt < NTH; ++nt) stage_out8<8>(stg, tl, 16 * nt + 4 * lg, pack4_bf16(dCT[nt]));
  __syncthreads();
  write_rows<8>(stg, dCc + t0 * act_rs, act_rs, qlim - t0, tid);
}

// The host pass leaves the stubs of ssd_bwd_src_kernel undefined when it only
// meets them through a launch (its device lambdas are not substituted there);
// explicit instantiation makes it emit them.
#define SA_SRC_INST(NK, HS, PLAN)                                                                \
  template __global__ void ssd_bwd_src_kernel<NK, HS, PLAN>(                                     \
      const bf16*, const bf16*, const bf16*, const bf16*, const float*, const float*,            \
      const bf16*, const int64_t*, bf16*, bf16*, bf16*, float*, float*, float*, float*,          \
      SsdDims, int);
SA_SRC_INST(4, 1, kPlanOne)
SA_SRC_INST(4, 2, kPlanOne)
SA_SRC_INST(4, 2, kPlanTwo)
SA_SRC_INST(4, 2, kPlanMany)
SA_SRC_INST(2, 1, kPlanOne)
SA_SRC_INST(2, 2, kPlanOne)
SA_SRC_INST(2, 2, kPlanTwo)
SA_SRC_INST(2, 2, kPlanMany)
#undef SA_SRC_INST

template <typename K>
int raise_smem(K kernel, size_t bytes, const char* who) {
  if (bytes <= 64 * 1024) return 0;
  const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           static_cast<int>(bytes));
  SA_CHECK_ARG(e == hipSuccess, "%s: %zu B of LDS refused: %s", who, bytes, hipGetErrorString(e));
  return 0;
}

template <int NK>
int launch_fused_nk(const void* u, const void* B, const void* C, const bf16* dyp,
                    const float* dt, const float* dc, const float* states, const bf16* dSp,
                    const int64_t* length, void* du, void* dB, void* dC, bf16* dcbp,
                    float* ddt_part, float* xB_part, float* xC_part, float* qpart, float* rpart,
                    const SsdDims& d, bool dt_nonneg, hipStream_t s) {
  const long blocks = static_cast<long>(d.b) * d.nc * d.G * (d.Lc / 64);
  {
    // one launch walks every head of the group (in passes of two heads
    // inside each block)
    ProfScope prof_("ssd_bwd_src", s);
    const int hpg = d.H / d.G;
    auto kernel = hpg == 1   ? ssd_bwd_src_kernel<NK, 1, kPlanOne>
                  : hpg <= 2 ? ssd_bwd_src_kernel<NK, 2, kPlanOne>
                  : hpg <= 4 ? ssd_bwd_src_kernel<NK, 2, kPlanTwo>
                             : ssd_bwd_src_kernel<NK, 2, kPlanMany>;
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(256), 0, s,
                       static_cast<const bf16*>(u), static_cast<const bf16*>(B),
                       static_cast<const bf16*>(C), dyp, dt, dc, dSp, length,
                       static_cast<bf16*>(du), static_cast<bf16*>(dB), dcbp, ddt_part, xB_part,
                       qpart, rpart, d, dt_nonneg ? 1 : 0);
    SA_CHECK_LAUNCH("ssd_bwd_src");
  }
  {
    const size_t smem = TgtSmem<NK>::bytes;
    if (const int rc = raise_smem(ssd_bwd_tgt_kernel<NK>, smem, "ssd_bwd_tgt")) return rc;
    ProfScope prof_("ssd_bwd_tgt", s);
    hipLaunchKernelGGL((ssd_bwd_tgt_kernel<NK>), dim3(TgtSmem<NK>::NHALF * blocks), dim3(256), smem,
                       s, static_cast<const bf16*>(B), static_cast<const bf16*>(C), dyp, dc, states,
                       dcbp, length, static_cast<bf16*>(dC), xC_part, d);
    SA_CHECK_LAUNCH("ssd_bwd_tgt");
  }
  return 0;
}

int launch_ssd_bwd_fused(const void* u, const void* B, const void* C, const bf16* dyp,
                         const float* dt, const float* dc, const float* states, const bf16* dSp,
                         const int64_t* length, void* du, void* dB, void* dC, bf16* dcbp,
                         float* ddt_part, float* xB_part, float* xC_part, float* qpart,
                         float* rpart, const SsdDims& d, bool dt_nonneg, hipStream_t s) {
  if (d.N == 64)
    return launch_fused_nk<2>(u, B, C, dyp, dt, dc, states, dSp, length, du, dB, dC, dcbp,
                              ddt_part, xB_part, xC_part, qpart, rpart, d, dt_nonneg, s);
  return launch_fused_nk<4>(u, B, C, dyp, dt, dc, states, dSp, length, du, dB, dC, dcbp,
                            ddt_part, xB_part, xC_part, qpart, rpart, d, dt_nonneg, s);
}

bool ssd_bwd_fused_shape_ok(const SsdDims& d) {
  return d.P == 64 && (d.N == 64 || d.N == 128) && d.Lc % 64 == 0 && d.H / d.G >= 1;
}

bool ssd_bwd_fused_ok(const SsdDims& d, const void* u, const void* B, const void* C,
                      const void* dy) {
  return ssd_bwd_fused_shape_ok(d) && aligned16(u) && aligned16(B) && aligned16(C) &&
         aligned16(dy);
}

}  // namespace sa
