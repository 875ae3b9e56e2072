// SSD chunked scan, backward pass (gfx950).
//
// Replaces ssd_scan_backward (reference triton_kernels/ssd_scan/backward.py:467-555)
// and its nine Triton kernels + host glue.  The forward's dt, dc and chunk
// entry states (H_in) are reused instead of recomputed.  Every reduction is
// deterministic (per-tile partials, fixed-order sums); the reference's
// atomics (backward_kernel.py:317, :427, :542, :1033, :1039) are gone.
//
//   dH_intra   = chunk_outer<MODE 1>                        (backward_kernel.py:23-92)
//   state_passing_bwd: dS_c, ddc_last, dh_init              (:110-167)
//   chunk_du_bwd:  acc = e^{min(dc_last-dc,0)} B.dS^T + (CB^T o decay) dy'
//                  du = acc dt, ddt_direct = sum_p acc u     (:187-317)
//   chunk_dcb_bwd: dCB = sum_h W_h, W_h = (dy' u^T) dt_s e^{min(dc_t-dc_s,0)} (t>=s)
//                  + row/column sums of W_h o CB for the intra-chunk decay
//                  gradient                                 (:569-668, :783-911)
//   chunk_dbdc_bwd: dB = sum_h w_h u.dS + dCB^T C ;  dC = sum_h e^{dc} dy'.H_in + dCB B
//                  + x_B / x_C decay-gradient terms          (:337-551, :689-765)
//   chunk_cumsum_bwd: da = dA_intra + dA_B + dA_C, ddt, d delta_raw, dA/dbias
//                  partials                                 (backward.py:544-548, :930-1039)
//   param_grad_reduce: dA, d delta_bias                     (replaces the atomics)
//
// dA_intra[k] = sum_{t >= k > s} M[t,s] for the strictly lower M = W o CB is
// computed as the exclusive prefix over k of (colsum(M)[k] - rowsum(M)[k]):
// T(k+1) - T(k) = sum_{t>k} M[t,k] - sum_{s<k} M[k,s].
#include "ssd_common.h"
#include "prof.h"

namespace sa {

// per-row sums of a wave's 32x32 fragment pair (over the wave's 32 columns);
// every lane of a 16-lane group ends up holding the sums of its rows
__device__ __forceinline__ void frag_row_sums(const float (&v)[2][2][4], float (&rs)[2][4]) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float s = v[i][0][r] + v[i][1][r];
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) s += __shfl_xor(s, o, 64);
      rs[i][r] = s;
    }
}
// per-column sums over the wave's 32 rows; lanes 0..15 (and their copies)
// hold column (lane & 15) + 16 j
__device__ __forceinline__ void frag_col_sums(const float (&v)[2][2][4], float (&cs)[2]) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) s += v[i][j][r];
    s += __shfl_xor(s, 16, 64);
    s += __shfl_xor(s, 32, 64);
    cs[j] = s;
  }
}

// ---------------------------------------------------------------------------
// workspace layout of the backward (shared by the size query and the launch)
// ---------------------------------------------------------------------------
struct BwdWs {
  size_t dS, dCB, ddt_part, xB_part, xC_part, rsum, qpart, ddc_part, dA_part, db_part;
  size_t dyp, dSp, dcbp, total;   // bf16 planes of the fused path
  int ptiles, ntiles, ttiles, per_bh;
  bool fused;
};

inline size_t al256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

inline BwdWs bwd_layout(const SsdDims& d, size_t mt_bytes) {
  BwdWs w;
  w.ptiles = (d.P + 63) / 64;
  w.ntiles = (d.N + 63) / 64;
  w.ttiles = (d.Lc + 63) / 64;
  const long PN = static_cast<long>(d.P) * d.N;
  w.per_bh = static_cast<int>((PN + 1023) / 1024);
  const size_t bhc = static_cast<size_t>(d.b) * d.H * d.nc;
  size_t o = 0;
  // A bf16 shape the fused kernels take may still run the generic ones (the
  // pointer alignment decides at launch), so for such shapes the region
  // after dS holds either layout: the generic path's fp32 dCB, or the fused
  // path's bf16 planes and parked dB part, and is sized for the larger.
  w.fused = mt_bytes == 2 && ssd_bwd_fused_shape_ok(d);
  w.dS = o;        o = al256(o + bhc * PN * 4);
  const size_t bncg = static_cast<size_t>(d.b) * d.nc * d.G;
  const size_t region = o;
  // the generic path's fp32 dCB
  w.dCB = region;
  const size_t generic_end = al256(region + bncg * d.Lc * d.Lc * 4);
  // the fused path: dy and dS as hi + lo planes, dCB^T as planes
  w.dyp = o;       o = al256(o + (w.fused ? bhc * d.Lc * 64 * 2 * 2 : 0));
  w.dSp = o;       o = al256(o + (w.fused ? bhc * PN * 2 * 2 : 0));
  w.dcbp = o;      o = al256(o + (w.fused ? bncg * w.ttiles * w.ttiles * 2 * 64 * 64 * 2 : 0));
  if (o < generic_end) o = generic_end;
  w.ddt_part = o;  o = al256(o + bhc * w.ptiles * d.Lc * 4);
  w.xB_part = o;   o = al256(o + bhc * w.ntiles * d.Lc * 4);
  w.xC_part = o;   o = al256(o + bhc * w.ntiles * d.Lc * 4);
  w.rsum = o;      o = al256(o + bhc * w.ttiles * d.Lc * 4);
  w.qpart = o;     o = al256(o + bhc * w.ttiles * d.Lc * 4);
  w.ddc_part = o;  o = al256(o + bhc * w.per_bh * 4);
  w.dA_part = o;   o = al256(o + bhc * 4);
  w.db_part = o;   o = al256(o + bhc * 4);
  w.total = o;
  return w;
}

// ---------------------------------------------------------------------------
// state passing (backward), reverse over chunks:
//   ddc_last[c] = exp(dc_last[c]) <H_in[c], G>;  dS_c = G;
//   G <- exp(dc_last[c]) G + dH_intra[c];        dh_init = G
// dS enters holding dH_intra and leaves holding dS (in place).
// ---------------------------------------------------------------------------
// With dSp set, dS is written as bf16 hi + lo planes ([b][nc][H][2][P*N], the
// fused backward's operand) instead of in place.
__global__ __launch_bounds__(256) void state_passing_bwd_kernel(
    const float* __restrict__ states, float* __restrict__ dS, const float* __restrict__ dh_last,
    float* __restrict__ dh_init, const float* __restrict__ dc, float* __restrict__ ddc_part,
    bf16* __restrict__ dSp, SsdDims d) {
  constexpr int GRP = 8;   // chunks whose two loads are in flight together
  __shared__ float red[GRP][4];
  const long PN = static_cast<long>(d.P) * d.N;
  const int per_bh = static_cast<int>((PN + 1023) / 1024);
  const int bh = blockIdx.x / per_bh;
  const int blk = blockIdx.x % per_bh;
  const long e0 = (static_cast<long>(blk) * 256 + threadIdx.x) * 4;
  const int h = bh % d.H, b = bh / d.H;
  const bool valid = e0 < PN;
  const bool full = valid && e0 + 4 <= PN && (PN % 4 == 0);
  auto load4 = [&](const float* p, float (&v)[4]) {
    if (full) {
      float4 t = *reinterpret_cast<const float4*>(p);
      v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    } else {
      for (int j = 0; j < 4; ++j) v[j] = (e0 + j < PN) ? p[j] : 0.0f;
    }
  };
  auto store4 = [&](float* p, const float (&v)[4]) {
    if (full) {
      *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      for (int j = 0; j < 4; ++j)
        if (e0 + j < PN) p[j] = v[j];
    }
  };
  float G[4] = {0.f, 0.f, 0.f, 0.f};
  if (dh_last && valid) load4(dh_last + static_cast<long>(bh) * PN + e0, G);
  const float* dcl = dc + static_cast<long>(bh) * d.nc * d.Lc + (d.Lc - 1);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  for (int chi = d.nc - 1; chi >= 0; chi -= GRP) {
    const int cn = min(GRP, chi + 1);
    float hin[GRP][4], dh[GRP][4];
#pragma unroll
    for (int j = 0; j < GRP; ++j) {
      if (j < cn && valid) {
        const long off = ((static_cast<long>(b) * d.nc + (chi - j)) * d.H + h) * PN + e0;
        load4(states + off, hin[j]);
        load4(dS + off, dh[j]);
      } else {
        for (int q = 0; q < 4; ++q) hin[j][q] = dh[j][q] = 0.f;
      }
    }
    float part[GRP];
#pragma unroll
    for (int j = 0; j < GRP; ++j) {
      part[j] = 0.f;
      if (j < cn) {
        const int c = chi - j;
        const float sc = expf(dcl[static_cast<long>(c) * d.Lc]);
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) s += hin[j][q] * G[q];
        part[j] = s * sc;
        if (valid) {
          const long bhc = (static_cast<long>(b) * d.nc + c) * d.H + h;
          if (dSp) {   // full float4 groups only (PN % 4 == 0 on this path)
            uint32_t hi[2], lo[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              hi[q] = pack_bf16x2(G[2 * q], G[2 * q + 1]);
              lo[q] = pack_bf16x2(G[2 * q] - bf16lo_to_f32(hi[q]), G[2 * q + 1] - bf16hi_to_f32(hi[q]));
            }
            *reinterpret_cast<uint2*>(dSp + bhc * 2 * PN + e0) = uint2{hi[0], hi[1]};
            *reinterpret_cast<uint2*>(dSp + bhc * 2 * PN + PN + e0) = uint2{lo[0], lo[1]};
          } else {
            store4(dS + bhc * PN + e0, G);
          }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) G[q] = sc * G[q] + dh[j][q];
      }
    }
#pragma unroll
    for (int j = 0; j < GRP; ++j) {
      const float s = wave_sum(part[j]);
      if (lane == 0) red[j][wid] = s;
    }
    __syncthreads();
    if (threadIdx.x < cn) {
      const int j = threadIdx.x;
      const float s = red[j][0] + red[j][1] + red[j][2] + red[j][3];
      ddc_part[(static_cast<long>(bh) * d.nc + (chi - j)) * per_bh + blk] = s;
    }
    __syncthreads();
  }
  if (dh_init && valid) store4(dh_init + static_cast<long>(bh) * PN + e0, G);
}

// ---------------------------------------------------------------------------
// du / ddt_direct: one 64 (tau) x 64 (p) tile per block.
// ---------------------------------------------------------------------------
template <typename MT, typename T>
__global__ __launch_bounds__(256) void chunk_du_bwd_kernel(
    const T* __restrict__ u, const T* __restrict__ Bm, const T* __restrict__ Cm,
    const float* __restrict__ dy, const float* __restrict__ dt, const float* __restrict__ dc,
    const float* __restrict__ dS, const int64_t* __restrict__ length, T* __restrict__ du,
    float* __restrict__ ddt_part, SsdDims d, int vec_act, int vec_dy, int vec_f32) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int NP = round_up(d.N, 32);
  const int LDN = lds_ld<MT>(NP);
  constexpr int LD64 = lds_ld<MT>(64);
  constexpr bool SPLIT = sizeof(MT) == 2;  // fp32-origin operands carry a lo plane
  constexpr int NPL = SPLIT ? 2 : 1;
  const int XPL = SPLIT ? 64 * LDN : 0;
  constexpr int LPL = SPLIT ? 64 * LD64 : 0;
  MT* Bt = reinterpret_cast<MT*>(smem_raw);  // [64][LDN] B rows of the tau tile
  MT* Xs = Bt + 64 * LDN;                    // [NPL][64][LDN] dS p-rows, then C sigma rows
  MT* Ls = Xs + NPL * 64 * LDN;              // [NPL][64][LD64]
  MT* Ys = Ls + NPL * 64 * LD64;             // [NPL][64][LD64] dy^T [p][sigma]
  float* dcs = reinterpret_cast<float*>(Ys + NPL * 64 * LD64);  // [Lc]
  float* red = dcs + d.Lc;                                  // [2][64]

  const int ttiles = (d.Lc + 63) / 64, ptiles = (d.P + 63) / 64;
  const int bid = xcd_swizzle(blockIdx.x, gridDim.x);
  const int tile = bid % (ttiles * ptiles);
  int rest = bid / (ttiles * ptiles);
  const int h = rest % d.H;
  rest /= d.H;
  const int c = rest % d.nc;
  const int b = rest / d.nc;
  const int ti = tile / ptiles, pti = tile % ptiles;
  const int t0 = ti * 64, p0 = pti * 64;
  const int g = h / (d.H / d.G);
  const int qlim = min(d.Lc, d.L - c * d.Lc);
  const int len = seq_limit(length, b, d.L);
  const int lim = max(0, chunk_limit(len, c, d.Lc));
  const long crow = ((static_cast<long>(b) * d.H + h) * d.nc + c) * d.Lc;
  float* dpart = ddt_part + (crow / d.Lc * ptiles + pti) * d.Lc;  // (b,H,nc,ptiles,Lc)
  const long tok0 = static_cast<long>(b) * d.L + static_cast<long>(c) * d.Lc;
  const long u_rs = static_cast<long>(d.H) * d.P, act_rs = static_cast<long>(d.G) * d.N;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = (wid >> 1) * 32, wn = (wid & 1) * 32;

  if (t0 >= lim) {  // whole tile at/after the length: zero gradients
    for (int e = threadIdx.x; e < 64 * 64; e += 256) {
      const int tl = e / 64, pl = e % 64;
      const int t = t0 + tl, p = p0 + pl;
      if (t < qlim && p < d.P) du[(tok0 + t) * u_rs + static_cast<long>(h) * d.P + p] = from_f32<T>(0.f);
    }
    for (int t = t0 + threadIdx.x; t < min(t0 + 64, d.Lc); t += 256) dpart[t] = 0.f;
    return;
  }
  for (int t = threadIdx.x; t < d.Lc; t += 256) dcs[t] = dc[crow + t] * kLog2e;
  const int rv = min(64, lim - t0);
  stage_rows<MT>(Bt, LDN, Bm + (tok0 + t0) * act_rs + static_cast<long>(g) * d.N, act_rs, 64, NP,
                 rv, d.N, vec_act != 0, NoScale{});
  stage_rows<MT>(Xs, LDN, dS + (((static_cast<long>(b) * d.nc + c) * d.H + h) * d.P + p0) * d.N,
                 d.N, 64, NP, d.P - p0, d.N, vec_f32 != 0, NoScale{}, XPL);
  __syncthreads();
  v4f acc[2][2];
  zero_acc(acc);
  wave_mma_split<MT, 2, 2, false, SPLIT>(acc, Bt + wm * LDN, LDN, 0, Xs + wn * LDN, LDN, XPL, NP,
                                         lane);
  const float dc_last = dcs[d.Lc - 1];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + wm + 16 * i + frag_row(lane, r);
      const float e = t < lim ? fast_exp2(fminf(dc_last - dcs[t], 0.0f)) : 0.0f;
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j][r] *= e;
    }
  __syncthreads();

  const float* dybase = dy + (tok0 * d.H + h) * static_cast<long>(d.P) + p0;
  for (int s0 = t0; s0 < lim; s0 += 64) {
    const int sv = min(64, lim - s0);
    stage_rows<MT>(Xs, LDN, Cm + (tok0 + s0) * act_rs + static_cast<long>(g) * d.N, act_rs, 64,
                   NP, sv, d.N, vec_act != 0, NoScale{});
    stage_transposed<MT>(Ys, LD64, dybase + static_cast<long>(s0) * u_rs, u_rs, 64, 64, sv,
                         d.P - p0, vec_dy != 0, NoScale{}, LPL);
    __syncthreads();
    v4f cbt[2][2];
    zero_acc(cbt);
    wave_mma<MT, 2, 2>(cbt, Bt + wm * LDN, LDN, Xs + wn * LDN, LDN, NP, lane);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tl = wm + 16 * i + frag_row(lane, r);
          const int sl = wn + 16 * j + frag_col(lane);
          const int t = t0 + tl, s = s0 + sl;
          float v = 0.0f;
          if (s >= t && s < lim) v = cbt[i][j][r] * fast_exp2(fminf(dcs[s] - dcs[t], 0.0f));
          store_split(Ls + tl * LD64 + sl, v, LPL);
        }
    __syncthreads();
    wave_mma_split<MT, 2, 2, SPLIT, SPLIT>(acc, Ls + wm * LD64, LD64, LPL, Ys + wn * LD64, LD64,
                                           LPL, 64, lane);
    __syncthreads();
  }

  // du = acc * dt ; ddt_direct partial = sum_p acc * u
  const float* dtrow = dt + crow;
  float prod[2][2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = t0 + wm + 16 * i + frag_row(lane, r);
        const int p = p0 + wn + 16 * j + frag_col(lane);
        float pv = 0.f;
        if (t < qlim && p < d.P) {
          const long off = (tok0 + t) * u_rs + static_cast<long>(h) * d.P + p;
          float g_u = 0.f;
          if (t < lim) {
            g_u = acc[i][j][r] * dtrow[t];
            pv = acc[i][j][r] * load_f32(u + off);
          }
          du[off] = from_f32<T>(g_u);
        }
        prod[i][j][r] = pv;
      }
  float rs[2][4];
  frag_row_sums(prod, rs);
  if ((lane & 15) == 0) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[(wn / 32) * 64 + wm + 16 * i + frag_row(lane, r)] = rs[i][r];
  }
  __syncthreads();
  for (int tl = threadIdx.x; tl < 64; tl += 256) {
    const int t = t0 + tl;
    if (t < d.Lc) dpart[t] = red[tl] + red[64 + tl];
  }
}

// ---------------------------------------------------------------------------
// dCB and the intra-chunk decay-gradient sums: one 64-row tau tile (I) of
// one (b, c, group) per block; loops over sigma tiles J <= I and the heads
// of the group.
// ---------------------------------------------------------------------------
template <typename MT, typename T>
__global__ __launch_bounds__(256) void chunk_dcb_bwd_kernel(
    const T* __restrict__ u, const T* __restrict__ Bm, const T* __restrict__ Cm,
    const float* __restrict__ dy, const float* __restrict__ dt, const float* __restrict__ dc,
    const int64_t* __restrict__ length, float* __restrict__ dCB, float* __restrict__ rsum,
    float* __restrict__ qpart, SsdDims d, int vec_act, int vec_dy) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int NP = round_up(d.N, 32);
  const int LDN = lds_ld<MT>(NP);
  constexpr int LD64 = lds_ld<MT>(64);
  const int hpg = d.H / d.G;
  constexpr bool SPLIT = sizeof(MT) == 2;
  constexpr int NPL = SPLIT ? 2 : 1;
  constexpr int YPL = SPLIT ? 64 * LD64 : 0;
  MT* Cs = reinterpret_cast<MT*>(smem_raw);  // [64][LDN] C rows of I
  MT* Xs = Cs + 64 * LDN;                    // [64][LDN] B rows of J
  MT* Ys = Xs + 64 * LDN;                    // [NPL][64][LD64] dy rows of I (p chunk)
  MT* Us = Ys + NPL * 64 * LD64;             // [64][LD64] u rows of J (p chunk)
  float* f = reinterpret_cast<float*>(Us + 64 * LD64);
  float* dcI = f;          // [64]
  float* dcJ = f + 64;     // [64]
  float* dtJ = f + 128;    // [64]
  float* rpart = f + 192;  // [2][64]
  float* cpart = f + 320;  // [2][64]
  float* racc = f + 448;   // [hpg][64]

  const int ttiles = (d.Lc + 63) / 64;
  const int bid = xcd_swizzle(blockIdx.x, gridDim.x);
  const int I = bid % ttiles;
  int rest = bid / ttiles;
  const int g = rest % d.G;
  rest /= d.G;
  const int c = rest % d.nc;
  const int b = rest / d.nc;
  const int t0 = I * 64;
  const int len = seq_limit(length, b, d.L);
  const int lim = max(0, chunk_limit(len, c, d.Lc));
  const long tok0 = static_cast<long>(b) * d.L + static_cast<long>(c) * d.Lc;
  const long u_rs = static_cast<long>(d.H) * d.P, act_rs = static_cast<long>(d.G) * d.N;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = (wid >> 1) * 32, wn = (wid & 1) * 32;
  const long dcb_base = ((static_cast<long>(b) * d.nc + c) * d.G + g) * d.Lc * d.Lc;

  const int nJ = lim > t0 ? min(I + 1, (lim + 63) / 64) : 0;  // sigma tiles computed
  // columns no tile of this block covers: zero partial column sums
  for (int k = 0; k < hpg; ++k) {
    const int hh = g * hpg + k;
    float* qp = qpart + ((((static_cast<long>(b) * d.H + hh) * d.nc + c) * ttiles + I) * d.Lc);
    for (int s = nJ * 64 + threadIdx.x; s < d.Lc; s += 256) qp[s] = 0.f;
  }
  for (int e = threadIdx.x; e < hpg * 64; e += 256) racc[e] = 0.f;
  if (nJ == 0) {
    __syncthreads();
    for (int k = 0; k < hpg; ++k) {
      const int hh = g * hpg + k;
      float* rr = rsum + (((static_cast<long>(b) * d.H + hh) * d.nc + c) * d.Lc);
      for (int t = t0 + threadIdx.x; t < min(t0 + 64, d.Lc); t += 256) rr[t] = 0.f;
    }
    return;
  }
  const int rvI = min(64, lim - t0);
  stage_rows<MT>(Cs, LDN, Cm + (tok0 + t0) * act_rs + static_cast<long>(g) * d.N, act_rs, 64, NP,
                 rvI, d.N, vec_act != 0, NoScale{});

  for (int J = 0; J < nJ; ++J) {
    const int s0 = J * 64;
    const int rvJ = min(64, lim - s0);
    stage_rows<MT>(Xs, LDN, Bm + (tok0 + s0) * act_rs + static_cast<long>(g) * d.N, act_rs, 64,
                   NP, rvJ, d.N, vec_act != 0, NoScale{});
    __syncthreads();
    v4f cb[2][2];
    zero_acc(cb);
    wave_mma<MT, 2, 2>(cb, Cs + wm * LDN, LDN, Xs + wn * LDN, LDN, NP, lane);
    float dcb[2][2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) dcb[i][j][r] = 0.f;

    for (int k = 0; k < hpg; ++k) {
      const int hh = g * hpg + k;
      const long crow = ((static_cast<long>(b) * d.H + hh) * d.nc + c) * d.Lc;
      __syncthreads();  // previous head's Ys/Us reads and dc/dt uses are done
      if (threadIdx.x < 64) {
        const int t = t0 + threadIdx.x, s = s0 + threadIdx.x;
        dcI[threadIdx.x] = t < d.Lc ? dc[crow + t] * kLog2e : 0.f;
        dcJ[threadIdx.x] = s < d.Lc ? dc[crow + s] * kLog2e : 0.f;
        dtJ[threadIdx.x] = s < d.Lc ? dt[crow + s] : 0.f;
      }
      v4f w[2][2];
      zero_acc(w);
      for (int pc = 0; pc < d.P; pc += 64) {
        stage_rows<MT>(Ys, LD64, dy + ((tok0 + t0) * d.H + hh) * static_cast<long>(d.P) + pc,
                       u_rs, 64, 64, rvI, d.P - pc, vec_dy != 0, NoScale{}, YPL);
        stage_rows<MT>(Us, LD64, u + ((tok0 + s0) * d.H + hh) * static_cast<long>(d.P) + pc,
                       u_rs, 64, 64, rvJ, d.P - pc, vec_act != 0, NoScale{});
        __syncthreads();
        wave_mma_split<MT, 2, 2, SPLIT, false>(w, Ys + wm * LD64, LD64, YPL, Us + wn * LD64, LD64,
                                               0, 64, lane);
        __syncthreads();
      }
      float m[2][2][4];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int tl = wm + 16 * i + frag_row(lane, r);
            const int sl = wn + 16 * j + frag_col(lane);
            const int t = t0 + tl, s = s0 + sl;
            float W = 0.f;
            if (t >= s && t < lim && s < lim)
              W = w[i][j][r] * dtJ[sl] * fast_exp2(fminf(dcI[tl] - dcJ[sl], 0.0f));
            dcb[i][j][r] += W;
            m[i][j][r] = t > s ? W * cb[i][j][r] : 0.f;
          }
      float rs[2][4], cs[2];
      frag_row_sums(m, rs);
      frag_col_sums(m, cs);
      if ((lane & 15) == 0) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) rpart[(wn / 32) * 64 + wm + 16 * i + frag_row(lane, r)] = rs[i][r];
      }
      if (lane < 16) {
#pragma unroll
        for (int j = 0; j < 2; ++j) cpart[(wm / 32) * 64 + wn + 16 * j + lane] = cs[j];
      }
      __syncthreads();
      if (threadIdx.x < 64) {
        racc[k * 64 + threadIdx.x] += rpart[threadIdx.x] + rpart[64 + threadIdx.x];
        const int s = s0 + threadIdx.x;
        if (s < d.Lc) {
          float* qp = qpart + ((((static_cast<long>(b) * d.H + hh) * d.nc + c) * ttiles + I) * d.Lc);
          qp[s] = cpart[threadIdx.x] + cpart[64 + threadIdx.x];
        }
      }
    }
    // store this dCB tile (t rows of I, s cols of J)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = t0 + wm + 16 * i + frag_row(lane, r);
          const int s = s0 + wn + 16 * j + frag_col(lane);
          if (t < d.Lc && s < d.Lc) dCB[dcb_base + static_cast<long>(t) * d.Lc + s] = dcb[i][j][r];
        }
  }
  __syncthreads();
  for (int k = 0; k < hpg; ++k) {
    const int hh = g * hpg + k;
    float* rr = rsum + (((static_cast<long>(b) * d.H + hh) * d.nc + c) * d.Lc);
    for (int tl = threadIdx.x; tl < 64; tl += 256)
      if (t0 + tl < d.Lc) rr[t0 + tl] = racc[k * 64 + tl];
  }
}

// ---------------------------------------------------------------------------
// dB (WHICH 0) / dC (WHICH 1): one 64-row x 64-col (n) tile of one
// (b, c, group) per block, summed over the heads of the group.
// ---------------------------------------------------------------------------
template <typename MT, typename T>
__global__ __launch_bounds__(256) void chunk_dbdc_bwd_kernel(
    const T* __restrict__ u, const T* __restrict__ Bm, const T* __restrict__ Cm,
    const float* __restrict__ dy, const float* __restrict__ dt, const float* __restrict__ dc,
    const float* __restrict__ states, const float* __restrict__ dS, const float* __restrict__ dCB,
    const int64_t* __restrict__ length, T* __restrict__ dB, T* __restrict__ dC,
    float* __restrict__ xB_part, float* __restrict__ xC_part, SsdDims d, int vec_act, int vec_dy,
    int vec_f32, int vec_dcb) {
  constexpr int LD64 = lds_ld<MT>(64);
  constexpr bool SPLIT = sizeof(MT) == 2;
  constexpr int NPL = SPLIT ? 2 : 1;
  constexpr int PL = SPLIT ? 64 * LD64 : 0;
  __shared__ __align__(16) MT As[NPL * 64 * LD64];
  __shared__ __align__(16) MT Xs[NPL * 64 * LD64];
  __shared__ float scl[64];
  __shared__ float red[2 * 64];

  const int ttiles = (d.Lc + 63) / 64, ntiles = (d.N + 63) / 64;
  const int hpg = d.H / d.G;
  const int bid = xcd_swizzle(blockIdx.x, gridDim.x);
  const int which = bid % 2;
  int rest = bid / 2;
  const int nti = rest % ntiles;
  rest /= ntiles;
  const int ti = rest % ttiles;
  rest /= ttiles;
  const int g = rest % d.G;
  rest /= d.G;
  const int c = rest % d.nc;
  const int b = rest / d.nc;
  const int r0 = ti * 64, n0 = nti * 64;
  const int qlim = min(d.Lc, d.L - c * d.Lc);
  if (r0 >= qlim) return;
  const int len = seq_limit(length, b, d.L);
  const int lim = max(0, chunk_limit(len, c, d.Lc));
  const long tok0 = static_cast<long>(b) * d.L + static_cast<long>(c) * d.Lc;
  const long u_rs = static_cast<long>(d.H) * d.P, act_rs = static_cast<long>(d.G) * d.N;
  const long PN = static_cast<long>(d.P) * d.N;
  const T* act = which ? Cm : Bm;  // the operand whose gradient this is
  T* out = which ? dC : dB;
  float* xpart = which ? xC_part : xB_part;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = (wid >> 1) * 32, wn = (wid & 1) * 32;
  const int rv = max(0, min(64, lim - r0));

  v4f acc[2][2];
  zero_acc(acc);
  for (int k = 0; k < hpg; ++k) {
    const int hh = g * hpg + k;
    const long crow = ((static_cast<long>(b) * d.H + hh) * d.nc + c) * d.Lc;
    float* xp = xpart + ((crow / d.Lc) * ntiles + nti) * d.Lc;
    __syncthreads();
    if (threadIdx.x < 64) {
      const int t = r0 + threadIdx.x;
      float s = 0.f;
      if (t < lim) {
        if (which) s = expf(dc[crow + t]);
        else s = expf(fminf(dc[crow + d.Lc - 1] - dc[crow + t], 0.0f)) * dt[crow + t];
      }
      scl[threadIdx.x] = s;
    }
    v4f tmp[2][2];
    zero_acc(tmp);
    const float* st = (which ? states : dS) +
                      (((static_cast<long>(b) * d.nc + c) * d.H + hh) * d.P) * d.N + n0;
    for (int pc = 0; pc < d.P; pc += 64) {
      if (which)
        stage_rows<MT>(As, LD64, dy + ((tok0 + r0) * d.H + hh) * static_cast<long>(d.P) + pc, u_rs,
                       64, 64, rv, d.P - pc, vec_dy != 0, NoScale{}, PL);
      else
        stage_rows<MT>(As, LD64, u + ((tok0 + r0) * d.H + hh) * static_cast<long>(d.P) + pc, u_rs,
                       64, 64, rv, d.P - pc, vec_act != 0, NoScale{});
      // Xs[n][p] = state[p][n]
      stage_transposed<MT>(Xs, LD64, st + static_cast<long>(pc) * d.N, d.N, 64, 64, d.P - pc,
                           d.N - n0, vec_f32 != 0, NoScale{}, PL);
      __syncthreads();
      if (which)
        wave_mma_split<MT, 2, 2, SPLIT, SPLIT>(tmp, As + wm * LD64, LD64, PL, Xs + wn * LD64, LD64,
                                               PL, 64, lane);
      else
        wave_mma_split<MT, 2, 2, false, SPLIT>(tmp, As + wm * LD64, LD64, 0, Xs + wn * LD64, LD64,
                                               PL, 64, lane);
      __syncthreads();
    }
    float prod[2][2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int rl = wm + 16 * i + frag_row(lane, r);
          const int n = n0 + wn + 16 * j + frag_col(lane);
          const float v = tmp[i][j][r] * scl[rl];
          acc[i][j][r] += v;
          float pv = 0.f;
          if (r0 + rl < lim && n < d.N)
            pv = v * load_f32(act + (tok0 + r0 + rl) * act_rs + static_cast<long>(g) * d.N + n);
          prod[i][j][r] = pv;
        }
    float rs[2][4];
    frag_row_sums(prod, rs);
    if ((lane & 15) == 0) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[(wn / 32) * 64 + wm + 16 * i + frag_row(lane, r)] = rs[i][r];
    }
    __syncthreads();
    if (threadIdx.x < 64) {
      const int t = r0 + threadIdx.x;
      if (t < d.Lc) xp[t] = red[threadIdx.x] + red[64 + threadIdx.x];
    }
  }

  // intra-chunk part through dCB
  const float* dcb = dCB + ((static_cast<long>(b) * d.nc + c) * d.G + g) * d.Lc * d.Lc;
  if (which) {
    // dC[t] += sum_{s <= t} dCB[t,s] B[s]
    for (int s0 = 0; s0 <= r0 && s0 < lim; s0 += 64) {
      const int sv = min(64, lim - s0);
      __syncthreads();
      stage_rows<MT>(As, LD64, dcb + static_cast<long>(r0) * d.Lc + s0, d.Lc, 64, 64, rv,
                     min(64, d.Lc - s0), vec_dcb != 0, NoScale{}, PL);
      stage_transposed<MT>(Xs, LD64, Bm + (tok0 + s0) * act_rs + static_cast<long>(g) * d.N + n0,
                           act_rs, 64, 64, sv, d.N - n0, vec_act != 0, NoScale{});
      __syncthreads();
      wave_mma_split<MT, 2, 2, SPLIT, false>(acc, As + wm * LD64, LD64, PL, Xs + wn * LD64, LD64,
                                             0, 64, lane);
    }
  } else {
    // dB[s] += sum_{t >= s} dCB[t,s] C[t]
    for (int tt = r0; tt < lim; tt += 64) {
      const int tv = min(64, lim - tt);
      __syncthreads();
      // As[s][t] = dCB[tt+t][r0+s]
      stage_transposed<MT>(As, LD64, dcb + static_cast<long>(tt) * d.Lc + r0, d.Lc, 64, 64, tv,
                           min(64, d.Lc - r0), vec_dcb != 0, NoScale{}, PL);
      stage_transposed<MT>(Xs, LD64, Cm + (tok0 + tt) * act_rs + static_cast<long>(g) * d.N + n0,
                           act_rs, 64, 64, tv, d.N - n0, vec_act != 0, NoScale{});
      __syncthreads();
      wave_mma_split<MT, 2, 2, SPLIT, false>(acc, As + wm * LD64, LD64, PL, Xs + wn * LD64, LD64,
                                             0, 64, lane);
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = r0 + wm + 16 * i + frag_row(lane, r);
        const int n = n0 + wn + 16 * j + frag_col(lane);
        if (t < qlim && n < d.N)
          out[(tok0 + t) * act_rs + static_cast<long>(g) * d.N + n] =
              from_f32<T>(t < lim ? acc[i][j][r] : 0.f);
      }
}

// ---------------------------------------------------------------------------
// decay-gradient assembly and the delta_raw gradient: one block per (b,c,h).
// ---------------------------------------------------------------------------
// exclusive block scan of one value per thread (256 threads); returns the
// exclusive prefix and writes the block total to *total
// exclusive prefix sums of three values at once (one pair of barriers);
// wt3 holds 4 waves x 3 floats
__device__ __forceinline__ void block_excl_scan3(const float (&v)[3], float* wt3, float (&base)[3],
                                                 float (&tot)[3]) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  float incl[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    incl[i] = wave_incl_scan(v[i], lane);
    if (lane == 63) wt3[wid * 3 + i] = incl[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    base[i] = incl[i] - v[i];
    tot[i] = 0.f;
    for (int w = 0; w < 4; ++w) {
      if (w < wid) base[i] += wt3[w * 3 + i];
      tot[i] += wt3[w * 3 + i];
    }
  }
  __syncthreads();
}

// block sums of two values at once
__device__ __forceinline__ void block_sum2(float& a, float& b, float* wt3) {
  a = wave_sum(a);
  b = wave_sum(b);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) {
    wt3[wid * 3] = a;
    wt3[wid * 3 + 1] = b;
  }
  __syncthreads();
  a = wt3[0] + wt3[3] + wt3[6] + wt3[9];
  b = wt3[1] + wt3[4] + wt3[7] + wt3[10];
  __syncthreads();
}

__device__ __forceinline__ float block_sum(float v, float* wtot) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) wtot[wid] = v;
  __syncthreads();
  const float s = wtot[0] + wtot[1] + wtot[2] + wtot[3];
  __syncthreads();
  return s;
}

// sum over k < n of base[k * stride], added in order k = 0, 1, ...: the
// first M loads are issued together (clamped to a valid k) before any is
// used; a loop that adds each load before the next is issued waits a memory
// round trip per term
template <int M>
__device__ __forceinline__ float sum_parts(const float* base, long stride, int n) {   // n >= 1
  float v[M];
#pragma unroll
  for (int k = 0; k < M; ++k) v[k] = base[static_cast<long>(min(k, n - 1)) * stride];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < M; ++k) s += k < n ? v[k] : 0.f;
  for (int k = M; k < n; ++k) s += base[static_cast<long>(k) * stride];
  return s;
}

// PER: positions per thread, (Lc + 255) / 256
template <typename T, int PER>
__global__ __launch_bounds__(256) void chunk_cumsum_bwd_kernel(
    const T* __restrict__ delta_raw, const float* __restrict__ A,
    const float* __restrict__ delta_bias, const int64_t* __restrict__ length,
    const float* __restrict__ dt, const float* __restrict__ ddt_part,
    const float* __restrict__ xB_part, const float* __restrict__ xC_part,
    const float* __restrict__ rsum, const float* __restrict__ qpart,
    const float* __restrict__ ddc_part, T* __restrict__ ddelta_raw, float* __restrict__ dA_part,
    float* __restrict__ db_part, SsdDims d, int ptiles, int ntiles, int xctiles, int ttiles,
    int rtiles, int per_bh, int has_init, int softplus, float lo, float hi) {
  __shared__ float wtot[4 * 3];
  const int h = blockIdx.x % d.H;
  const int c = (blockIdx.x / d.H) % d.nc;
  const int b = blockIdx.x / (d.H * d.nc);
  const long bhc = (static_cast<long>(b) * d.H + h) * d.nc + c;
  const long crow = bhc * d.Lc;
  const int len = seq_limit(length, b, d.L);
  const int lim = chunk_limit(len, c, d.Lc);
  const int qlim = min(d.Lc, d.L - c * d.Lc);
  const int tb = threadIdx.x * PER;

  // every global load is issued here, ahead of the block reductions (a
  // barrier orders memory, so loads placed after one wait for it)
  float ddc = 0.f;
  for (int k = threadIdx.x; k < per_bh; k += 256) ddc += ddc_part[bhc * per_bh + k];
  // loads from clamped (valid) positions, unconditionally, so that they are
  // all in flight together; positions past Lc, qlim or lim are masked after
  float qr[PER], xb[PER], xc[PER], zv[PER], dtv[PER], ddtd[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int t = tb + j;
    const int tl = min(t, d.Lc - 1), tq = min(t, qlim - 1);
    const float q = sum_parts<4>(qpart + bhc * ttiles * d.Lc + tl, d.Lc, ttiles);
    const float x1 = sum_parts<2>(xB_part + bhc * ntiles * d.Lc + tl, d.Lc, ntiles);
    const float x2 = sum_parts<2>(xC_part + bhc * xctiles * d.Lc + tl, d.Lc, xctiles);
    // row sums: partials of the source tiles k <= t / 64 (rtiles == 1: complete)
    const float r = sum_parts<4>(rsum + bhc * rtiles * d.Lc + tl, d.Lc, min(rtiles, tl / 64 + 1));
    const long off = (static_cast<long>(b) * d.L + static_cast<long>(c) * d.Lc + tq) * d.H + h;
    const float z = load_f32(delta_raw + off);
    const float dtt = dt[crow + tl];
    const float dd = sum_parts<2>(ddt_part + bhc * ptiles * d.Lc + tl, d.Lc, ptiles);
    const bool tv = t < d.Lc, tin = tv && t < lim;
    qr[j] = tv ? q - r : 0.f;
    xb[j] = tv && t < lim - 1 ? x1 : 0.f;
    xc[j] = tin ? x2 : 0.f;
    zv[j] = tin ? z : 0.f;
    dtv[j] = tin ? dtt : 0.f;
    ddtd[j] = tin ? dd : 0.f;
  }
  // ddc_last of this chunk (sum of the state-passing partials)
  ddc = block_sum(ddc, wtot);
  if (!has_init && c == 0) ddc = 0.f;
  float sqr = 0.f, sxb = 0.f, sxc = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if (tb + j == d.Lc - 1) xc[j] += ddc;
    sqr += qr[j];
    sxb += xb[j];
    sxc += xc[j];
  }
  float ex[3], tt[3];
  block_excl_scan3({sqr, sxb, sxc}, wtot, ex, tt);
  const float eq = ex[0], eb = ex[1], ec = ex[2], tc = tt[2];
  const float a = A[h];
  const float bias = delta_bias ? delta_bias[h] : 0.0f;
  float rq = eq, rb = eb, rc = ec;
  float dA_loc = 0.f, db_loc = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int t = tb + j;
    if (t < d.Lc) {
      const float dA_intra = rq, dA_B = rb, dA_C = tc - rc;  // exclusive, exclusive, suffix
      rq += qr[j];
      rb += xb[j];
      rc += xc[j];
      if (t < qlim) {
        const long off = (static_cast<long>(b) * d.L + static_cast<long>(c) * d.Lc + t) * d.H + h;
        float g = 0.f;
        if (t < lim) {
          const float da = dA_intra + dA_B + dA_C;
          const float z = zv[j] + bias;
          const float sp = softplus ? softplus20(z) : z;
          g = da * a + ddtd[j];
          if (sp < lo || sp > hi) g = 0.f;
          if (softplus && z <= 20.0f) g *= sigmoidf_acc(z);
          dA_loc += da * dtv[j];
          db_loc += g;
        }
        ddelta_raw[off] = from_f32<T>(g);
      }
    }
  }
  block_sum2(dA_loc, db_loc, wtot);
  if (threadIdx.x == 0) {
    dA_part[(static_cast<long>(b) * d.nc + c) * d.H + h] = dA_loc;
    db_part[(static_cast<long>(b) * d.nc + c) * d.H + h] = db_loc;
  }
}

__global__ __launch_bounds__(256) void param_grad_reduce_kernel(const float* __restrict__ dA_part,
                                                                const float* __restrict__ db_part,
                                                                float* __restrict__ dA,
                                                                float* __restrict__ dbias,
                                                                int rows, int H) {
  __shared__ float wtot[4];
  const int h = blockIdx.x;
  float s1 = 0.f, s2 = 0.f;
  for (int r = threadIdx.x; r < rows; r += 256) {
    s1 += dA_part[static_cast<long>(r) * H + h];
    s2 += db_part[static_cast<long>(r) * H + h];
  }
  s1 = block_sum(s1, wtot);
  s2 = block_sum(s2, wtot);
  if (threadIdx.x == 0) {
    dA[h] = s1;
    if (dbias) dbias[h] = s2;
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
template <typename MT>
size_t du_smem(const SsdDims& d) {
  const int NP = round_up(d.N, 32);
  const int npl = sizeof(MT) == 2 ? 2 : 1;
  return sizeof(MT) * ((1 + npl) * 64 * lds_ld<MT>(NP) + 2 * npl * 64 * lds_ld<MT>(64)) +
         sizeof(float) * (d.Lc + 128);
}
template <typename MT>
size_t dcb_smem(const SsdDims& d) {
  const int NP = round_up(d.N, 32);
  const int npl = sizeof(MT) == 2 ? 2 : 1;
  return sizeof(MT) * (2 * 64 * lds_ld<MT>(NP) + (npl + 1) * 64 * lds_ld<MT>(64)) +
         sizeof(float) * (448 + 64 * (d.H / d.G));
}

template <typename K>
int set_smem(K kernel, size_t bytes, const char* who) {
  if (bytes <= 64 * 1024) return 0;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(bytes));
  SA_CHECK_ARG(e == hipSuccess, "%s: %zu B of LDS refused: %s", who, bytes, hipGetErrorString(e));
  return 0;
}

template <typename T, typename MT>
int ssd_bwd_impl(const void* u_, const float* A, const void* B_, const void* C_,
                 const void* delta_raw_, const float* bias, const int64_t* length,
                 const float* dy, const float* dh_last, const float* dt, const float* dc,
                 const float* states, const SsdDims& d, int sp, float lo, float hi, int has_init,
                 void* du_, float* dA, void* dB_, void* dC_, void* ddelta_, float* dbias,
                 float* dh_init, unsigned char* ws, hipStream_t s) {
  const T* u = static_cast<const T*>(u_);
  const T* Bm = static_cast<const T*>(B_);
  const T* Cm = static_cast<const T*>(C_);
  const BwdWs w = bwd_layout(d, sizeof(MT));
  float* dS = reinterpret_cast<float*>(ws + w.dS);
  float* dCB = reinterpret_cast<float*>(ws + w.dCB);
  float* ddt_part = reinterpret_cast<float*>(ws + w.ddt_part);
  float* xB_part = reinterpret_cast<float*>(ws + w.xB_part);
  float* xC_part = reinterpret_cast<float*>(ws + w.xC_part);
  float* rsum = reinterpret_cast<float*>(ws + w.rsum);
  float* qpart = reinterpret_cast<float*>(ws + w.qpart);
  float* ddc_part = reinterpret_cast<float*>(ws + w.ddc_part);
  float* dA_part = reinterpret_cast<float*>(ws + w.dA_part);
  float* db_part = reinterpret_cast<float*>(ws + w.db_part);

  const int vec_act = aligned16(u) && aligned16(Bm) && aligned16(Cm) && d.P % 8 == 0 &&
                      d.N % 8 == 0;
  const int vec_dy = aligned16(dy) && d.P % 8 == 0;
  const int vec_f32 = aligned16(ws) && d.N % 8 == 0;
  const int vec_dcb = d.Lc % 8 == 0;
  const long bnc = static_cast<long>(d.b) * d.nc;
  int rc;

  const bool fused = sizeof(T) == 2 && w.fused && ssd_bwd_fused_ok(d, u, Bm, Cm, dy);
  bf16* dyp = reinterpret_cast<bf16*>(ws + w.dyp);
  bf16* dSp = reinterpret_cast<bf16*>(ws + w.dSp);
  bf16* dcbp = reinterpret_cast<bf16*>(ws + w.dcbp);
  // 1. dH_intra -> dS buffer (the fused path also writes dy as hi + lo planes)
  if (fused) {
    if ((rc = launch_dstate_planes(dy, C_, dt, dc, length, dS, dyp, d, s))) return rc;
  } else {
    if ((rc = launch_chunk_outer<MT, float, T, 1>(dy, C_, dt, dc, length, dS, d, s))) return rc;
  }
  // 2. reverse state passing (the fused path writes dS as hi + lo planes)
  {
    const long blocks = static_cast<long>(d.b) * d.H * w.per_bh;
    ProfScope prof_("state_passing_bwd", s);
    hipLaunchKernelGGL(state_passing_bwd_kernel, dim3(blocks), dim3(256), 0, s, states, dS,
                       dh_last, dh_init, dc, ddc_part, fused ? dSp : nullptr, d);
    SA_CHECK_LAUNCH("state_passing_bwd");
  }
  int ptiles = w.ptiles, ntiles = w.ntiles, xctiles = w.ntiles, qtiles = w.ttiles, rtiles = 1;
  if (fused) {
    // 3-5 fused: du, dB, dC, decay sums
    if ((rc = launch_ssd_bwd_fused(u, Bm, Cm, dyp, dt, dc, states, dSp, length, du_, dB_, dC_,
                                   dcbp, ddt_part, xB_part, xC_part, qpart, rsum, d,
                                   lo >= 0.f, s)))
      return rc;
    ptiles = ntiles = qtiles = 1;
    xctiles = d.N / 64;   // x_C: one partial per 64 n (ssd_bwd_tgt block)
    rtiles = d.Lc / 64;
  } else {
  // 3. du, ddt_direct
  {
    const size_t smem = du_smem<MT>(d);
    if ((rc = set_smem(chunk_du_bwd_kernel<MT, T>, smem, "chunk_du_bwd"))) return rc;
    const long blocks = static_cast<long>(w.ttiles) * w.ptiles * bnc * d.H;
    ProfScope prof_("chunk_du_bwd", s);
    hipLaunchKernelGGL((chunk_du_bwd_kernel<MT, T>), dim3(blocks), dim3(256), smem, s, u, Bm, Cm,
                       dy, dt, dc, dS, length, static_cast<T*>(du_), ddt_part, d, vec_act, vec_dy,
                       vec_f32);
    SA_CHECK_LAUNCH("chunk_du_bwd");
  }
  // 4. dCB and intra-chunk decay sums
  {
    const size_t smem = dcb_smem<MT>(d);
    if ((rc = set_smem(chunk_dcb_bwd_kernel<MT, T>, smem, "chunk_dcb_bwd"))) return rc;
    const long blocks = static_cast<long>(w.ttiles) * bnc * d.G;
    ProfScope prof_("chunk_dcb_bwd", s);
    hipLaunchKernelGGL((chunk_dcb_bwd_kernel<MT, T>), dim3(blocks), dim3(256), smem, s, u, Bm, Cm,
                       dy, dt, dc, length, dCB, rsum, qpart, d, vec_act, vec_dy);
    SA_CHECK_LAUNCH("chunk_dcb_bwd");
  }
  // 5. dB, dC
  {
    const long blocks = 2L * w.ntiles * w.ttiles * bnc * d.G;
    ProfScope prof_("chunk_dbdc_bwd", s);
    hipLaunchKernelGGL((chunk_dbdc_bwd_kernel<MT, T>), dim3(blocks), dim3(256), 0, s, u, Bm, Cm, dy,
                       dt, dc, states, dS, dCB, length, static_cast<T*>(dB_), static_cast<T*>(dC_),
                       xB_part, xC_part, d, vec_act, vec_dy, vec_f32, vec_dcb);
    SA_CHECK_LAUNCH("chunk_dbdc_bwd");
  }
  }
  // 6. decay-gradient assembly, d delta_raw, dA/dbias partials
  {
    const long blocks = bnc * d.H;
    ProfScope prof_("chunk_cumsum_bwd", s);
    const int per = (d.Lc + 255) / 256;   // 1..4: chunk sizes are validated to [1, 1024]
    auto kernel = per <= 1 ? chunk_cumsum_bwd_kernel<T, 1>
                  : per == 2 ? chunk_cumsum_bwd_kernel<T, 2>
                  : per == 3 ? chunk_cumsum_bwd_kernel<T, 3>
                             : chunk_cumsum_bwd_kernel<T, 4>;
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(256), 0, s,
                       static_cast<const T*>(delta_raw_), A, bias, length, dt, ddt_part, xB_part,
                       xC_part, rsum, qpart, ddc_part, static_cast<T*>(ddelta_), dA_part, db_part,
                       d, ptiles, ntiles, xctiles, qtiles, rtiles, w.per_bh, has_init, sp, lo, hi);
    SA_CHECK_LAUNCH("chunk_cumsum_bwd");
  }
  // 7. dA, dbias
  {
    ProfScope prof_("param_grad_reduce", s);
    hipLaunchKernelGGL(param_grad_reduce_kernel, dim3(d.H), dim3(256), 0, s, dA_part, db_part, dA,
                       dbias, static_cast<int>(bnc), d.H);
    SA_CHECK_LAUNCH("param_grad_reduce");
  }
  return 0;
}

}  // namespace sa

extern "C" size_t sa_ssd_bwd_workspace_size(int dtype, int batch, int seqlen, int num_heads,
                                            int head_dim, int num_groups, int state_dim,
                                            int chunk_size) {
  sa::SsdDims d;
  if (sa::make_dims(batch, seqlen, num_heads, head_dim, num_groups, state_dim, chunk_size, &d,
                    "sa_ssd_bwd_workspace_size"))
    return 0;
  return sa::bwd_layout(d, dtype == sa::kBF16 ? 2 : 4).total;
}

extern "C" int sa_ssd_bwd(int dtype, const void* u, const float* A, const void* B, const void* C,
                          const void* delta_raw, const float* delta_bias, const int64_t* length,
                          const float* dy, const float* dh_last, const float* dt, const float* dc,
                          const float* states, int batch, int seqlen, int num_heads, int head_dim,
                          int num_groups, int state_dim, int chunk_size, int use_softplus,
                          float delta_min, float delta_max, int has_h_init, void* du, float* dA,
                          void* dB, void* dC, void* ddelta_raw, float* ddelta_bias,
                          float* dh_init, void* workspace, size_t workspace_bytes, void* stream) {
  sa::SsdDims d;
  int rc = sa::make_dims(batch, seqlen, num_heads, head_dim, num_groups, state_dim, chunk_size, &d,
                         "sa_ssd_bwd");
  if (rc) return rc;
  SA_CHECK_ARG(dtype == sa::kF32 || dtype == sa::kBF16, "sa_ssd_bwd: unsupported dtype %d", dtype);
  SA_CHECK_ARG(dtype == sa::kBF16 || state_dim <= 128,
               "sa_ssd_bwd: float32 path supports state_dim <= 128 (got %d)", state_dim);
  SA_CHECK_ARG(u && A && B && C && delta_raw && dy && dt && dc && states && du && dA &&
                   dB && dC && ddelta_raw && workspace,
               "sa_ssd_bwd: null tensor pointer");
  const size_t need = sa::bwd_layout(d, dtype == sa::kBF16 ? 2 : 4).total;
  SA_CHECK_ARG(workspace_bytes >= need, "sa_ssd_bwd: workspace %zu B < required %zu B",
               workspace_bytes, need);
  if (d.b == 0 || d.L == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  if (dtype == sa::kF32)
    return sa::ssd_bwd_impl<float, float>(u, A, B, C, delta_raw, delta_bias, length, dy, dh_last,
                                          dt, dc, states, d, use_softplus, delta_min, delta_max,
                                          has_h_init, du, dA, dB, dC, ddelta_raw, ddelta_bias,
                                          dh_init, ws, s);
  return sa::ssd_bwd_impl<sa::bf16, sa::bf16>(u, A, B, C, delta_raw, delta_bias, length, dy,
                                              dh_last, dt, dc, states, d, use_softplus, delta_min,
                                              delta_max, has_h_init, du, dA, dB, dC, ddelta_raw,
                                              ddelta_bias, dh_init, ws, s);
}
