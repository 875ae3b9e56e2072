// SSD chunked scan, forward pass (gfx950).
//
// Replaces ssd_scan_forward (reference triton_kernels/ssd_scan/forward.py:223-276)
// and its five Triton kernels with four HIP kernels:
//
//   chunk_cumsum    dt = clamp(softplus20(delta_raw+bias)), 0 at t >= length;
//                   dc = inclusive cumsum over the chunk of dt*A
//                   (forward_kernel.py:20-87)
//   chunk_outer     S_c[p,n] = sum_tau u[tau,p] w_tau B[tau,n],
//                   w_tau = exp(min(dc_last-dc_tau,0)) dt_tau   (forward_kernel.py:108-185)
//                   -- the same kernel computes the backward's dH_intra with
//                   (dy, exp(dc) [tau<lim], C) in place of (u, w, B)
//   state_passing   H_in[0] = h_init | 0, H_in[c+1] = exp(dc_last[c]) H_in[c] + S_c,
//                   in place over the chunk-state buffer (forward_kernel.py:203-250)
//   chunk_scan      y = exp(dc) C.H_in^T + (tril(C.B^T) o decay o dt) . u
//                   (forward_kernel.py:351-455); the C.B^T tile is recomputed
//                   per (tau-tile, sigma-tile) on the matrix cores instead of
//                   materialising CB (bmm_chunk_forward, :271-328) in HBM.
//
// Layouts (all row-major, contiguous):
//   u (b,L,H,P)  B,C (b,L,G,N)  delta_raw (b,L,H)  [activations: fp32 | bf16]
//   dt, dc (b,H,nc,Lc) fp32   states (b,nc,H,P,N) fp32   y (b,L,H,P) fp32
#include "ssd_common.h"
#include "prof.h"

namespace sa {

// ---------------------------------------------------------------------------
// chunk cumsum: one block per (b, c, h); each thread owns up to Lc/256
// consecutive positions, the block adds the per-thread totals in a scan.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void chunk_cumsum_kernel(
    const T* __restrict__ delta_raw, const float* __restrict__ A,
    const float* __restrict__ delta_bias, const int64_t* __restrict__ length,
    float* __restrict__ dt_out, float* __restrict__ dc_out, SsdDims d, int softplus, float dmin,
    float dmax) {
  __shared__ float wave_tot[4];
  const int h = blockIdx.x % d.H;
  const int c = (blockIdx.x / d.H) % d.nc;
  const int b = blockIdx.x / (d.H * d.nc);
  const int len = seq_limit(length, b, d.L);
  const int lim = chunk_limit(len, c, d.Lc);
  const float a = A[h];
  const float bias = delta_bias ? delta_bias[h] : 0.0f;
  const int per = (d.Lc + 255) / 256;  // positions per thread (<= 4)
  const int t0 = threadIdx.x * per;
  float v[4];
  float run = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[j] = 0.0f;
    const int tau = t0 + j;
    if (j < per && tau < lim) {
      const long t = static_cast<long>(c) * d.Lc + tau;
      const float z = load_f32(delta_raw + (static_cast<long>(b) * d.L + t) * d.H + h) + bias;
      v[j] = make_dt(z, softplus != 0, dmin, dmax);
    }
  }
  float part[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    run += v[j] * a;
    part[j] = run;
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  float incl = wave_incl_scan(run, lane);
  if (lane == 63) wave_tot[wid] = incl;
  __syncthreads();
  float base = incl - run;
  for (int w = 0; w < wid; ++w) base += wave_tot[w];
  const long row = ((static_cast<long>(b) * d.H + h) * d.nc + c) * d.Lc;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int tau = t0 + j;
    if (j < per && tau < d.Lc) {
      dt_out[row + tau] = v[j];
      dc_out[row + tau] = base + part[j];
    }
  }
}

// ---------------------------------------------------------------------------
// chunk outer product: out[(b,c,h)][p][n] = sum_tau a(tau,p) b(tau,n)
//   MODE 0 (chunk state):  a = u * exp(min(dc_last-dc,0)) * dt,  b = B,  tau < seq end
//   MODE 1 (dH_intra):     a = dy * exp(dc) [tau < lim],          b = C,  tau < lim
// One 64x64 (p, n) tile per block, k = tau in steps of 32 through LDS.
// ---------------------------------------------------------------------------
template <typename MT, typename TA, typename TB, int MODE>
__global__ __launch_bounds__(256) void chunk_outer_kernel(
    const TA* __restrict__ a_src, const TB* __restrict__ b_src, const float* __restrict__ dt,
    const float* __restrict__ dc, const int64_t* __restrict__ length, float* __restrict__ out,
    SsdDims d, int vec_a, int vec_b) {
  constexpr int KC = 32;
  constexpr int LD = lds_ld<MT>(KC);
  // the gradient operand of MODE 1 is fp32 in origin: split it on the bf16 path
  constexpr bool SA = MODE == 1 && sizeof(MT) == 2;
  constexpr int APLANE = SA ? 64 * LD : 0;
  __shared__ __align__(16) MT As[(SA ? 2 : 1) * 64 * LD];
  __shared__ __align__(16) MT Bs[64 * LD];
  __shared__ float scl[1024];

  const int ptiles = (d.P + 63) / 64, ntiles = (d.N + 63) / 64;
  const int bid = xcd_swizzle(blockIdx.x, gridDim.x);
  const int tile = bid % (ptiles * ntiles);
  int rest = bid / (ptiles * ntiles);
  const int h = rest % d.H;
  rest /= d.H;
  const int c = rest % d.nc;
  const int b = rest / d.nc;
  const int p0 = (tile / ntiles) * 64, n0 = (tile % ntiles) * 64;
  const int g = h / (d.H / d.G);

  const long crow = ((static_cast<long>(b) * d.H + h) * d.nc + c) * d.Lc;
  const int len = seq_limit(length, b, d.L);
  const int klim = MODE == 0 ? min(d.Lc, d.L - c * d.Lc) : max(0, chunk_limit(len, c, d.Lc));
  // per-tau scale for the a operand
  const float dc_last = dc[crow + d.Lc - 1];
  for (int t = threadIdx.x; t < d.Lc; t += 256) {
    float s;
    if (MODE == 0) s = expf(fminf(dc_last - dc[crow + t], 0.0f)) * dt[crow + t];
    else s = t < klim ? expf(dc[crow + t]) : 0.0f;
    scl[t] = s;
  }
  __syncthreads();

  const long tok0 = static_cast<long>(b) * d.L + static_cast<long>(c) * d.Lc;
  const TA* a_base = a_src + (tok0 * d.H + h) * d.P + p0;
  const TB* b_base = b_src + (tok0 * d.G + g) * d.N + n0;
  const long a_rs = static_cast<long>(d.H) * d.P, b_rs = static_cast<long>(d.G) * d.N;

  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = (wid >> 1) * 32, wn = (wid & 1) * 32;
  v4f acc[2][2];
  zero_acc(acc);
  for (int k0 = 0; k0 < klim; k0 += KC) {
    const int kv = min(KC, klim - k0);
    const float* sk = scl + k0;
    stage_transposed<MT>(As, LD, a_base + k0 * a_rs, a_rs, KC, 64, kv, d.P - p0, vec_a != 0,
                         [sk](int r, int) { return sk[r]; }, APLANE);
    stage_transposed<MT>(Bs, LD, b_base + k0 * b_rs, b_rs, KC, 64, kv, d.N - n0, vec_b != 0,
                         NoScale{});
    __syncthreads();
    wave_mma_split<MT, 2, 2, SA, false>(acc, As + wm * LD, LD, APLANE, Bs + wn * LD, LD, 0, KC,
                                        lane);
    __syncthreads();
  }
  float* o = out + (((static_cast<long>(b) * d.nc + c) * d.H + h) * d.P) * d.N;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int p = p0 + wm + 16 * i + frag_row(lane, r);
        const int n = n0 + wn + 16 * j + frag_col(lane);
        if (p < d.P && n < d.N) o[static_cast<long>(p) * d.N + n] = acc[i][j][r];
      }
}

// Two bf16 values (one 32-bit word) times sc, as hi + lo bf16 pairs: hi =
// bf16(x sc), lo = bf16(x sc - hi) with the residual from one fused
// multiply-add.  Written out, so that the chunk-state kernels that must agree
// bit for bit (chunk_outer_bf16_kernel<., 0>, chunk_state_pass_kernel) do
// not depend on where the compiler contracts a multiply and a subtract.
__device__ __forceinline__ void split_scaled(uint32_t v, float sc, uint32_t& hi, uint32_t& lo) {
  const float x0 = bf16lo_to_f32(v), x1 = bf16hi_to_f32(v);
  hi = pack_bf16x2(x0 * sc, x1 * sc);
  lo = pack_bf16x2(__builtin_fmaf(x0, sc, -bf16lo_to_f32(hi)), __builtin_fmaf(x1, sc, -bf16hi_to_f32(hi)));
}

// ---------------------------------------------------------------------------
// chunk outer products, bf16 fast path (P and N multiples of 64):
//   MODE 0: states[p][n] = sum_t u[t,p] w_t B[t,n],  w_t = e^{min(dc_last - dc_t, 0)} dt_t
//   MODE 1: dH[p][n]     = sum_t dy[t,p] e^{dc_t} C[t,n]   (t < length); with
//           dyp set (P = 64) it also writes dy (zero at t >= length) as the
//           hi + lo bf16 planes the fused backward reads, [b][nc][G][Lc/64]
//           [H/G][2][64][64]
// One block per (b, chunk, head, 64-wide p tile), 4 waves; wave w computes
// D^T[n][p] for its N/4 columns n and the 64 p.  Both operands come from
// row-major t tiles in LDS through transpose reads: A = X^T (X = B or C) and
// the B operand = the scaled U (MODE 0, one bf16 plane) or the scaled dy
// (MODE 1, hi + lo planes).  Each lane ends with 4 consecutive n of one p
// (16-byte stores).  t tiles are prefetched into registers during the
// previous tile's MFMAs and committed to a single LDS stage (35 KB at
// N = 128), so three or four blocks share a CU: more resident blocks hide
// the loads better than a second stage did (chunk states 88 -> 72-78 us).
// ---------------------------------------------------------------------------
template <int NK, int MODE>
__global__ __launch_bounds__(256, 3) void chunk_outer_bf16_kernel(
    const void* __restrict__ a_src, const bf16* __restrict__ x_src, const float* __restrict__ dt,
    const float* __restrict__ dc, const int64_t* __restrict__ length, float* __restrict__ out,
    bf16* __restrict__ dyp, SsdDims d) {
  constexpr int N = 32 * NK;
  using TA = LdsTile<64>;                  // the scaled operand's planes
  using TX = LdsTile<N>;                   // the B or C tile
  constexpr int PLA = 64 * TA::kLd;        // elements per plane
  constexpr int NPL = 2;                   // hi + lo planes of the scaled operand
  constexpr int NTW = N / 64;              // 16-wide n tiles per wave
  extern __shared__ __align__(16) unsigned char smem_raw[];
  bf16* sm = reinterpret_cast<bf16*>(smem_raw);   // As [NPL][64 rows], Xs [64 rows]

  const int ptiles = d.P / 64;
  const int bid = xcd_swizzle(blockIdx.x, gridDim.x);
  const int pti = bid % ptiles;
  int rest = bid / ptiles;
  const int h = rest % d.H;
  rest /= d.H;
  const int c = rest % d.nc;
  const int b = rest / d.nc;
  const int p0 = 64 * pti;
  const int g = h / (d.H / d.G);
  const long crow = ((static_cast<long>(b) * d.H + h) * d.nc + c) * d.Lc;
  const int qlim = min(d.Lc, d.L - c * d.Lc);
  const int klim = MODE == 0 ? qlim : max(0, chunk_limit(seq_limit(length, b, d.L), c, d.Lc));
  const int tid = threadIdx.x, lane = tid & 63, li = lane & 15, lg = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  float* o = out + (((static_cast<long>(b) * d.nc + c) * d.H + h) * d.P + p0) * N;
  v4f acc[NTW][4];
#pragma unroll
  for (int i = 0; i < NTW; ++i)
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) acc[i][pt] = v4f{0.f, 0.f, 0.f, 0.f};

  if (klim > 0) {
    const long tok0 = static_cast<long>(b) * d.L + static_cast<long>(c) * d.Lc;
    const int a_rs = d.H * d.P, x_rs = d.G * N;
    const bf16* xc = x_src + tok0 * x_rs + static_cast<long>(g) * N;
    const float dcl = dc[crow + d.Lc - 1] * kLog2e;
    // Prefetch registers.  A row's dc (and dt) are loaded with the tile and
    // turned into its scale only at the commit: a use at load time would
    // make the compiler wait there for the whole prefetch (loads complete in
    // order), before the current tile's MFMAs.
    int slot_tile = 0;   // tile index held by the prefetch registers
    uint4 pa0[MODE == 0 ? 2 : 1];
    float4 pa1[MODE == 1 ? 4 : 1];
    float pdc[2], pdt[2];   // dc, dt of the rows (clamped to klim - 1)
    // scale of row t of the held tile from its dc, dt (0 past klim)
    auto row_scale = [&](int t, float dcv, float dtv) __attribute__((always_inline)) {
      float sc;
      // (the fused multiply-add written out: chunk_state_pass_kernel forms the
      // same argument, and the two must agree bit for bit)
      if constexpr (MODE == 0) sc = fast_exp2(fminf(__builtin_fmaf(dcv, -kLog2e, dcl), 0.f)) * dtv;
      else sc = fast_exp2(dcv * kLog2e);
      return t < klim ? sc : 0.f;
    };
    BfTile<NK, 256> px;
    auto load_tile = [&](int tt) __attribute__((always_inline)) {
      const int t0 = 64 * tt, kv = min(64, klim - t0);
      slot_tile = tt;
      if constexpr (MODE == 0) {
        const bf16* ac = static_cast<const bf16*>(a_src) + tok0 * a_rs + h * d.P + p0;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int e = tid + 256 * i, row = e >> 3;
          pa0[i] = *reinterpret_cast<const uint4*>(ac + static_cast<unsigned>((t0 + min(row, kv - 1)) * a_rs + 8 * (e & 7)));
          const int tc = min(t0 + row, klim - 1);
          pdc[i] = dc[crow + tc];
          pdt[i] = dt[crow + tc];
        }
      } else {
        const float* ac = static_cast<const float*>(a_src) + tok0 * a_rs + h * d.P + p0;
        const int row = tid >> 2;
        const float* pp = ac + static_cast<unsigned>((t0 + min(row, kv - 1)) * a_rs + 16 * (tid & 3));
#pragma unroll
        for (int i = 0; i < 4; ++i) pa1[i] = *reinterpret_cast<const float4*>(pp + 4 * i);
        pdc[0] = dc[crow + min(t0 + row, klim - 1)];
      }
      px.load(xc + static_cast<long>(t0) * x_rs, x_rs, kv, tid);
    };
    auto commit_tile = [&]() __attribute__((always_inline)) {
      bf16* As = sm;
      bf16* Xs = As + NPL * PLA;
      if constexpr (MODE == 0) {
        // w * u is fp32 (dt up to z > 20 makes it large): hi + lo planes keep
        // the chunk states near fp32, which the backward's dC, dA and
        // d(delta_raw) inherit
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int e = tid + 256 * i, row = e >> 3;
          const float sc = row_scale(64 * slot_tile + row, pdc[i], pdt[i]);
          const uint32_t q[4] = {pa0[i].x, pa0[i].y, pa0[i].z, pa0[i].w};
          uint32_t r[4], rl[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) split_scaled(q[j], sc, r[j], rl[j]);
          const int ao = TA::off(row, 8 * (e & 7));
          *reinterpret_cast<uint4*>(As + ao) = uint4{r[0], r[1], r[2], r[3]};
          *reinterpret_cast<uint4*>(As + PLA + ao) = uint4{rl[0], rl[1], rl[2], rl[3]};
        }
      } else {
        const int row = tid >> 2, c0 = 16 * (tid & 3);
        const float sc = row_scale(64 * slot_tile + row, pdc[0], 0.f);
        uint32_t hi[8], lo[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v[4] = {pa1[i].x * sc, pa1[i].y * sc, pa1[i].z * sc, pa1[i].w * sc};
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const uint32_t hh = pack_bf16x2(v[2 * j], v[2 * j + 1]);
            hi[2 * i + j] = hh;
            lo[2 * i + j] = pack_bf16x2(v[2 * j] - bf16lo_to_f32(hh), v[2 * j + 1] - bf16hi_to_f32(hh));
          }
        }
        const int ao0 = TA::off(row, c0), ao1 = TA::off(row, c0 + 8);
        *reinterpret_cast<uint4*>(As + ao0) = uint4{hi[0], hi[1], hi[2], hi[3]};
        *reinterpret_cast<uint4*>(As + ao1) = uint4{hi[4], hi[5], hi[6], hi[7]};
        *reinterpret_cast<uint4*>(As + PLA + ao0) = uint4{lo[0], lo[1], lo[2], lo[3]};
        *reinterpret_cast<uint4*>(As + PLA + ao1) = uint4{lo[4], lo[5], lo[6], lo[7]};
      }
      commit_lds(px, Xs, tid);
      if constexpr (MODE == 1) {
        if (dyp) {
          // the unscaled tile rows as planes (zero rows past the length),
          // stored after the tile's loads are used: the compiler would
          // otherwise wait for these stores before those uses
          const int row = tid >> 2, c0 = 16 * (tid & 3);
          const int tt = slot_tile;
          const bool in = 64 * tt + row < klim;
          uint32_t uh[8], ul[8];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float v[4] = {in ? pa1[i].x : 0.f, in ? pa1[i].y : 0.f, in ? pa1[i].z : 0.f,
                                in ? pa1[i].w : 0.f};
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
              const uint32_t hh = pack_bf16x2(v[2 * jj], v[2 * jj + 1]);
              uh[2 * i + jj] = hh;
              ul[2 * i + jj] = pack_bf16x2(v[2 * jj] - bf16lo_to_f32(hh), v[2 * jj + 1] - bf16hi_to_f32(hh));
            }
          }
          const int hpg = d.H / d.G;
          const long tileo = ((((static_cast<long>(b) * d.nc + c) * d.G + g) * (d.Lc / 64) + tt) * hpg +
                              (h - g * hpg)) * (2L * 64 * 64);
          uint4* ph = reinterpret_cast<uint4*>(dyp + tileo + row * 64 + c0);
          uint4* pl = reinterpret_cast<uint4*>(dyp + tileo + 64 * 64 + row * 64 + c0);
          ph[0] = uint4{uh[0], uh[1], uh[2], uh[3]};
          ph[1] = uint4{uh[4], uh[5], uh[6], uh[7]};
          pl[0] = uint4{ul[0], ul[1], ul[2], ul[3]};
          pl[1] = uint4{ul[4], ul[5], ul[6], ul[7]};
        }
      }
    };

    const int ntt = (klim + 63) / 64;
    load_tile(0);
    commit_tile();
    __syncthreads();
    for (int tt = 0; tt < ntt; ++tt) {
      const bool has_next = tt + 1 < ntt;
      if (has_next) load_tile(tt + 1);
      const bf16* As = sm;
      const bf16* Xs = As + NPL * PLA;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        v8bf bop[4][NPL];
#pragma unroll
        for (int pt = 0; pt < 4; ++pt)
#pragma unroll
          for (int pl = 0; pl < NPL; ++pl)
            bop[pt][pl] = tile_tr8<64>(As + pl * PLA, 32 * ks + 8 * lg, 16 * pt, lane);
#pragma unroll
        for (int i = 0; i < NTW; ++i) {
          const v8bf a = tile_tr8<N>(Xs, 32 * ks + 8 * lg, 16 * (NTW * w + i), lane);
#pragma unroll
          for (int pt = 0; pt < 4; ++pt)
#pragma unroll
            for (int pl = 0; pl < NPL; ++pl) acc[i][pt] = mfma_bf16(a, bop[pt][pl], acc[i][pt]);
        }
      }
      __syncthreads();   // every wave is done with the stage
      if (has_next) commit_tile();
      __syncthreads();
    }
  }
  // D^T[n][p]: lane holds n = 16 nt + 4 lg + r of p = 16 pt + li
#pragma unroll
  for (int i = 0; i < NTW; ++i)
#pragma unroll
    for (int pt = 0; pt < 4; ++pt)
      *reinterpret_cast<float4*>(o + static_cast<unsigned>((16 * pt + li) * N + 16 * (NTW * w + i) + 4 * lg)) =
          make_float4(acc[i][pt][0], acc[i][pt][1], acc[i][pt][2], acc[i][pt][3]);
}

// ---------------------------------------------------------------------------
// chunk states and state passing in one kernel (forward, bf16, P and N
// multiples of 64):
//   S_c[p][n] = sum_t u[t,p] w_t B[t,n],  w_t = e^{min(dc_last - dc_t, 0)} dt_t
//   states[c] = H_c,  H_{c+1} = e^{dc_last(c)} H_c + S_c,  H_0 = h_init or 0,
//   h_last = H_nc
// One block per (b, head, 64-wide p tile, 64 NB-wide n block), 4 NB waves:
// wave w accumulates S_c^T[n][p] for the block's n columns 16 w .. 16 w + 15
// and its 64 p, and holds H_c in the same fragment layout (lane: n = n0 +
// 16 w + 4 lg + r, p = p0 + 16 pt + li).  The block walks every 64-token t
// tile of every chunk in order, so the chunk states never leave the chip.
// With NB = 2 (state_dim a multiple of 128) one 512-thread block covers 128
// n: each u tile is brought in and split once for both halves, half the
// split work per thread (one block per CU instead of two of 64 n).
// A tile's raw u and B rows and its dc, dt go from HBM straight into one of
// NS LDS stages (global_load_lds, issued NS - 1 tiles ahead and waited for
// with explicit counts; three stages at NB = 1, four at NB = 2).  Step g
// refills, after its MFMAs, the stage step g - 1 consumed (every wave is past
// it at step g's barrier), so a step has one barrier.  Step g runs tile g's MFMAs (w u as hi + lo planes,
// B from the stage) while the waves scale tile g + 1's u by w_t and split it
// into its planes in place (w u is fp32), so that the split's latency does
// not sit between a tile's arrival and its MFMAs.  The products and their
// order are chunk_outer_bf16_kernel<., 0>'s and the update is
// state_passing_fwd_kernel's.
// ---------------------------------------------------------------------------
template <int NB>
__global__ __launch_bounds__(256 * NB, 2 / NB) void chunk_state_pass_kernel(
    const bf16* __restrict__ u, const bf16* __restrict__ Bm, const float* __restrict__ dt,
    const float* __restrict__ dc, const float* __restrict__ h_init, float* __restrict__ states,
    float* __restrict__ h_last, SsdDims d) {
  using TL = LdsTile<64>;                      // u tile and its planes
  using TB = LdsTile<64 * NB>;                 // B tile: 64 rows of the block's 64 NB n
  constexpr int NT = 256 * NB;                 // threads
  constexpr int NW = 4 * NB;                   // waves
  constexpr int PL = 64 * TL::kLd;             // bf16 per 64 x 64 plane
  constexpr int XL = 64 * TB::kLd;             // bf16 of the B tile
  constexpr int NS = NB == 2 ? 4 : 3;          // DMA stages (four fit beside one 512-thread block)
  constexpr int UI = 2 / NB;                   // u DMA instructions per wave per tile
  constexpr int BI = 2;                        // B DMA instructions per wave per tile
  constexpr int kDma = UI + BI + 1;            // DMA instructions per wave per tile
  // stage (bf16): u tile, then its hi plane in place; lo plane (+PL); B tile
  // (+2 PL); NW x 64 fp32 row values (+2 PL + XL): dc, dt, 64 copies of the
  // chunk's last dc, spare copies of dt
  constexpr int kStage = 2 * PL + XL + NW * 128;
  __shared__ __align__(16) bf16 stg[NS * kStage];

  const int ptiles = d.P / 64, nblk = d.N / (64 * NB);
  const int bid = xcd_swizzle(blockIdx.x, gridDim.x);
  int rest = bid;
  const int nb = rest % nblk;
  rest /= nblk;
  const int pti = rest % ptiles;
  rest /= ptiles;
  const int h = rest % d.H;
  const int b = rest / d.H;
  const int p0 = 64 * pti, n0 = 64 * NB * nb;
  const int g = h / (d.H / d.G);
  const int tid = threadIdx.x, lane = tid & 63, li = lane & 15, lg = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int a_rs = d.H * d.P, x_rs = d.G * d.N;
  const long PN = static_cast<long>(d.P) * d.N;
  const long bh = static_cast<long>(b) * d.H + h;
  // this lane's element offset inside a [P][N] state: + 16 pt N
  const int eo = (p0 + li) * d.N + n0 + 16 * w + 4 * lg;

  v4f H[4], S[4];
#pragma unroll
  for (int pt = 0; pt < 4; ++pt) {
    S[pt] = v4f{0.f, 0.f, 0.f, 0.f};
    H[pt] = v4f{0.f, 0.f, 0.f, 0.f};
    if (h_init) {
      const float4 v = *reinterpret_cast<const float4*>(h_init + bh * PN + eo + 16 * pt * d.N);
      H[pt] = v4f{v.x, v.y, v.z, v.w};
    }
  }
  // the initial state has arrived before the loop, whose waits count DMA
  // and the state stores only
  __builtin_amdgcn_s_waitcnt(vm_wait<0>());

  // t tiles: every chunk but the last has tpc, the last ntt_last; walkers
  // hold (chunk, t tile in it, tiles in the chunk) and advance without division
  const int tpc = (d.Lc + 63) / 64;
  const int qlast = d.L - (d.nc - 1) * d.Lc;
  const int ntt_last = (qlast + 63) / 64;
  const int ntiles = (d.nc - 1) * tpc + ntt_last;
  struct Walk {
    int c, tt, ntt;
  };
  auto adv = [&](Walk& x) __attribute__((always_inline)) {
    if (++x.tt == x.ntt) {
      x.tt = 0;
      ++x.c;
      x.ntt = x.c == d.nc - 1 ? ntt_last : tpc;
    }
  };
  auto rows_of = [&](const Walk& x) { return min(64, min(d.Lc, d.L - x.c * d.Lc) - 64 * x.tt); };

  // per-lane LDS element offsets, the same in every stage: transposed reads
  // of the planes (rows 8 lg + (li / 4) and + 4 of k step 0, columns 16 pt +
  // 4 (li % 4); k step 1 is 32 rows on) and of B (columns 16 w + 4 (li %
  // 4)), and the u chunks this thread splits
  int o_b[4][2], o_x[2], ao[UI];
#pragma unroll
  for (int pt = 0; pt < 4; ++pt)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) o_b[pt][hh] = TL::off(8 * lg + 4 * hh + (li >> 2), 16 * pt + 4 * (li & 3));
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) o_x[hh] = TB::off(8 * lg + 4 * hh + (li >> 2), 16 * w + 4 * (li & 3));
#pragma unroll
  for (int i = 0; i < UI; ++i) ao[i] = TL::off((tid + NT * i) >> 3, 8 * ((tid + NT * i) & 7));

  // u DMA instruction i of this wave fills plane bytes 1024 (UI w + i) + 16
  // lane: row pos / 8 with pos = 64 (UI w + i) + lane, stored chunk pos % 8,
  // which holds logical chunk (pos % 8) ^ swz_r128(row) (the LdsTile<64>
  // layout); B instruction i fills tile bytes 1024 (BI w + i) + 16 lane, 8 NB
  // chunks per row (the LdsTile<64 NB> layout).  Lane byte offsets of a full
  // tile's u and B rows:
  int urow[UI], ucol[UI], xrow[BI], xcol[BI];
  uint32_t du[UI], dx[BI];
#pragma unroll
  for (int i = 0; i < UI; ++i) {
    const int pos = 64 * (UI * w + i) + lane;
    urow[i] = pos >> 3;
    ucol[i] = 8 * ((pos & 7) ^ swz_r128(pos >> 3));
    du[i] = 2u * static_cast<uint32_t>(urow[i] * a_rs + ucol[i]);
  }
#pragma unroll
  for (int i = 0; i < BI; ++i) {
    const int pos = 64 * (BI * w + i) + lane;
    constexpr int RC = 8 * NB;   // 16-byte chunks per B row
    xrow[i] = pos / RC;
    xcol[i] = 8 * ((pos % RC) ^ (NB == 1 ? swz_r128(pos / RC) : swz_r256(pos / RC)));
    dx[i] = 2u * static_cast<uint32_t>(xrow[i] * x_rs + xcol[i]);
  }
  const uint32_t lds_st = lds_addr(stg);
  // tile x into stage st: UI + BI sixteen-byte and 1 four-byte DMA per wave
  // (wave 0 brings the tile's dc, wave 1 its dt, wave 2 64 copies of the
  // chunk's last dc, the others spare copies of dt, so that every wave counts
  // the same number per tile).  Rows past the chunk repeat its last (their
  // scale is 0).
  auto issue = [&](const Walk& x, int st) __attribute__((always_inline)) {
    const int t0 = 64 * x.tt, qv = rows_of(x);
    const long tok = static_cast<long>(b) * d.L + static_cast<long>(x.c) * d.Lc + t0;
    const bf16* ub = u + tok * a_rs + h * d.P + p0;
    const bf16* xb = Bm + tok * x_rs + static_cast<long>(g) * d.N + n0;
    const uint32_t base = lds_st + static_cast<uint32_t>(st * kStage * 2);   // bytes
#pragma unroll
    for (int i = 0; i < UI; ++i) {
      uint32_t ou = du[i];
      if (qv < 64) ou = 2u * static_cast<uint32_t>(min(urow[i], qv - 1) * a_rs + ucol[i]);
      dma_lds16(ub, ou, base + (static_cast<uint32_t>(UI * w + i) << 10));
    }
#pragma unroll
    for (int i = 0; i < BI; ++i) {
      uint32_t ox = dx[i];
      if (qv < 64) ox = 2u * static_cast<uint32_t>(min(xrow[i], qv - 1) * x_rs + xcol[i]);
      dma_lds16(xb, ox, base + 4 * PL + (static_cast<uint32_t>(BI * w + i) << 10));
    }
    const long crow = (bh * d.nc + x.c) * d.Lc;
    const float* rv = w == 2 ? dc + crow + d.Lc - 1 : ((w == 0) ? dc : dt) + crow + t0;
    const uint32_t ro = w == 2 ? 0u : 4u * static_cast<uint32_t>(min(lane, qv - 1));
    dma_lds4(rv, ro, base + 4 * PL + 2 * XL + 256 * w);
  };
  // tile x's u in stage ST -> (w u) hi plane in place, lo plane at +PL
  auto split = [&](const Walk& x, auto stc) __attribute__((always_inline)) {
    bf16* sb = stg + decltype(stc)::value * kStage;
    const int qv = rows_of(x);
    const float* rdc = reinterpret_cast<const float*>(sb + 2 * PL + XL);
    const float* rdt = rdc + 64;
    const float dcl = rdc[128] * kLog2e;
#pragma unroll
    for (int i = 0; i < UI; ++i) {
      const int row = (tid + NT * i) >> 3;
      const uint4 q = *reinterpret_cast<const uint4*>(sb + ao[i]);
      // rows past the chunk hold copies of its last row (finite): the scale is
      // computed in every lane and masked by a select, not a branch
      // (the argument's fused multiply-add written out, as chunk_outer_bf16_kernel
      // forms it: where the compiler contracts would otherwise differ)
      float sc = fast_exp2(fminf(__builtin_fmaf(rdc[row], -kLog2e, dcl), 0.f)) * rdt[row];
      asm volatile("" : "+v"(sc));
      sc = row < qv ? sc : 0.f;
      const uint32_t v[4] = {q.x, q.y, q.z, q.w};
      uint32_t r[4], rl[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) split_scaled(v[j], sc, r[j], rl[j]);
      *reinterpret_cast<uint4*>(sb + ao[i]) = uint4{r[0], r[1], r[2], r[3]};
      *reinterpret_cast<uint4*>(sb + PL + ao[i]) = uint4{rl[0], rl[1], rl[2], rl[3]};
    }
  };

  // prologue: tiles 0 .. NS - 2 (the last again past the end) into stages 0 .. NS - 2
  Walk wi{0, 0, d.nc == 1 ? ntt_last : tpc};
  int gi = 0;   // tile index of wi
  auto adv_issue = [&]() __attribute__((always_inline)) {
    if (gi + 1 < ntiles) {
      adv(wi);
      ++gi;
    }
  };
#pragma unroll
  for (int st = 0; st < NS - 1; ++st) {
    issue(wi, st);
    adv_issue();
  }
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(vm_wait<(NS - 2) * kDma>());
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  Walk wc{0, 0, d.nc == 1 ? ntt_last : tpc};   // the tile computed
  Walk wsp = wc;                               // the tile split (one ahead)
  split(wsp, std::integral_constant<int, 0>{});
  adv(wsp);
  bool stored = false;   // the step before stored a state (4 stores per wave)
  int gt = 0;
  // step gt (its stage ST = gt % NS, a compile-time value in the unrolled loop)
  auto step = [&](auto stc) __attribute__((always_inline)) {
    constexpr int ST = decltype(stc)::value;
    const bf16* sb = stg + ST * kStage;
    // tile gt + 1 has landed (tiles gt + 2 .. gt + NS - 2 may still be in
    // flight, and with NS >= 4 the state stores of step gt - 1, which follow
    // tile gt + 1's DMA; with NS = 3 they precede it); tile gt's planes are
    // visible: the waits take lgkmcnt(0) too, since this barrier is the
    // step's only one and follows the split's LDS writes of step gt - 1
    asm volatile("" ::: "memory");
    if (NS >= 4 && stored) __builtin_amdgcn_s_waitcnt(vm_lgkm_wait<(NS - 3) * kDma + (NS >= 4 ? 4 : 0)>());
    else __builtin_amdgcn_s_waitcnt(vm_lgkm_wait<(NS - 3) * kDma>());
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    stored = wc.tt == 0;
    if (stored) {   // the chunk's entry state
      float* o = states + (static_cast<long>(b) * d.nc + wc.c) * d.H * PN + static_cast<long>(h) * PN + eo;
#pragma unroll
      for (int pt = 0; pt < 4; ++pt)
        *reinterpret_cast<float4*>(o + 16 * pt * d.N) = make_float4(H[pt][0], H[pt][1], H[pt][2], H[pt][3]);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      v8bf bop[4][2];
#pragma unroll
      for (int pt = 0; pt < 4; ++pt)
#pragma unroll
        for (int pl = 0; pl < 2; ++pl)
          bop[pt][pl] = tile_tr8_at(sb + pl * PL + 32 * TL::kLd * ks, o_b[pt][0], o_b[pt][1]);
      const v8bf a = tile_tr8_at(sb + 2 * PL + 32 * TB::kLd * ks, o_x[0], o_x[1]);
#pragma unroll
      for (int pt = 0; pt < 4; ++pt)
#pragma unroll
        for (int pl = 0; pl < 2; ++pl) S[pt] = mfma_bf16(a, bop[pt][pl], S[pt]);
    }
    if (gt + 1 < ntiles) split(wsp, std::integral_constant<int, (ST + 1) % NS>{});
    if (wc.tt == wc.ntt - 1) {   // the chunk's last tile: pass the state on
      const float sc = expf(reinterpret_cast<const float*>(sb + 2 * PL + XL)[128]);
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) H[pt][r] = sc * H[pt][r] + S[pt][r];
        S[pt] = v4f{0.f, 0.f, 0.f, 0.f};
      }
    }
    // refill the stage step gt - 1 consumed with tile gt + NS - 1 (the last
    // tile again past the end, so that every step waits the same): every wave
    // passed this step's barrier after its last use of that stage
    issue(wi, (ST + NS - 1) % NS);
    adv_issue();
    adv(wc);
    adv(wsp);
    ++gt;
  };
  while (gt < ntiles) {
    step(std::integral_constant<int, 0>{});
    if (gt >= ntiles) break;
    step(std::integral_constant<int, 1>{});
    if (gt >= ntiles) break;
    step(std::integral_constant<int, 2>{});
    if constexpr (NS == 4) {
      if (gt >= ntiles) break;
      step(std::integral_constant<int, 3 % NS>{});
    }
  }
  // drain the surplus DMA before the block ends
  __builtin_amdgcn_s_waitcnt(vm_wait<0>());
  float* o = h_last + bh * PN + eo;
#pragma unroll
  for (int pt = 0; pt < 4; ++pt)
    *reinterpret_cast<float4*>(o + 16 * pt * d.N) = make_float4(H[pt][0], H[pt][1], H[pt][2], H[pt][3]);
}

// ---------------------------------------------------------------------------
// state passing (forward): sequential over chunks, parallel over (b, h, P*N).
// Loads of a group of chunks are issued together before the dependent math.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void state_passing_fwd_kernel(
    float* __restrict__ states, const float* __restrict__ h_init, float* __restrict__ h_last,
    const float* __restrict__ dc, SsdDims d) {
  const long PN = static_cast<long>(d.P) * d.N;
  const int per_bh = static_cast<int>((PN + 1023) / 1024);
  const int bh = blockIdx.x / per_bh;
  const long e0 = (static_cast<long>(blockIdx.x % per_bh) * 256 + threadIdx.x) * 4;
  const int h = bh % d.H, b = bh / d.H;
  if (e0 >= PN) return;
  const bool full = e0 + 4 <= PN && (PN % 4 == 0);
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
  float hv[4] = {0.f, 0.f, 0.f, 0.f};
  if (h_init) load4(h_init + static_cast<long>(bh) * PN + e0, hv);
  const float* dcl = dc + static_cast<long>(bh) * d.nc * d.Lc + (d.Lc - 1);
  constexpr int GRP = 16;   // chunks whose loads are in flight together (16: all of config 1's)
  for (int c0 = 0; c0 < d.nc; c0 += GRP) {
    float s[GRP][4];
    const int cn = min(GRP, d.nc - c0);
#pragma unroll
    for (int j = 0; j < GRP; ++j)
      if (j < cn) load4(states + ((static_cast<long>(b) * d.nc + c0 + j) * d.H + h) * PN + e0, s[j]);
#pragma unroll
    for (int j = 0; j < GRP; ++j) {
      if (j < cn) {
        float* dst = states + ((static_cast<long>(b) * d.nc + c0 + j) * d.H + h) * PN + e0;
        store4(dst, hv);
        const float sc = expf(dcl[static_cast<long>(c0 + j) * d.Lc]);
#pragma unroll
        for (int q = 0; q < 4; ++q) hv[q] = sc * hv[q] + s[j][q];
      }
    }
  }
  store4(h_last + static_cast<long>(bh) * PN + e0, hv);
}

// ---------------------------------------------------------------------------
// chunk scan: one 64 (tau) x 64 (p) tile of y per block.
//   y  = exp(dc_tau) * sum_n C[tau,n] H_in[p,n]
//      + sum_{sigma <= tau} CB[tau,sigma] exp(min(dc_tau - dc_sigma, 0)) dt_sigma u[sigma,p]
// CB tiles come from C (kept in LDS for the whole tau tile) and a staged
// B sigma-tile.  NP = N rounded up to 32 (<= 256).
// ---------------------------------------------------------------------------
template <typename MT, typename T>
__global__ __launch_bounds__(256) void chunk_scan_fwd_kernel(
    const T* __restrict__ u, const T* __restrict__ Bm, const T* __restrict__ Cm,
    const float* __restrict__ dt, const float* __restrict__ dc, const float* __restrict__ states,
    float* __restrict__ y, SsdDims d, int vec_act, int vec_state) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int NP = round_up(d.N, 32);
  const int LDN = lds_ld<MT>(NP);
  constexpr int LD64 = lds_ld<MT>(64);
  MT* Cs = reinterpret_cast<MT*>(smem_raw);          // [64][LDN]   C tau-tile
  MT* Xs = Cs + 64 * LDN;                            // [64][LDN]   H_in p-tile, then B sigma-tile
  MT* Ls = Xs + 64 * LDN;                            // [64][LD64]  masked, scaled CB tile
  MT* Us = Ls + 64 * LD64;                           // [64][LD64]  u^T sigma-tile
  float* dts = reinterpret_cast<float*>(Us + 64 * LD64);  // [Lc]
  float* dcs = dts + d.Lc;                                // [Lc]

  const int ttiles = (d.Lc + 63) / 64, ptiles = (d.P + 63) / 64;
  const int bid = xcd_swizzle(blockIdx.x, gridDim.x);
  const int tile = bid % (ttiles * ptiles);
  int rest = bid / (ttiles * ptiles);
  const int h = rest % d.H;
  rest /= d.H;
  const int c = rest % d.nc;
  const int b = rest / d.nc;
  const int t0 = (tile / ptiles) * 64, p0 = (tile % ptiles) * 64;
  const int g = h / (d.H / d.G);
  const int qlim = min(d.Lc, d.L - c * d.Lc);  // rows of this chunk inside the sequence
  if (t0 >= qlim) return;

  const long crow = ((static_cast<long>(b) * d.H + h) * d.nc + c) * d.Lc;
  for (int t = threadIdx.x; t < d.Lc; t += 256) {
    dts[t] = dt[crow + t];
    dcs[t] = dc[crow + t] * kLog2e;  // exp(x) = exp2(x log2 e) below
  }
  const long tok0 = static_cast<long>(b) * d.L + static_cast<long>(c) * d.Lc;
  const long act_rs = static_cast<long>(d.G) * d.N;
  const T* Cbase = Cm + (tok0 * d.G + g) * d.N;
  const T* Bbase = Bm + (tok0 * d.G + g) * d.N;
  const float* Hbase = states + (((static_cast<long>(b) * d.nc + c) * d.H + h) * d.P + p0) * d.N;
  stage_rows<MT>(Cs, LDN, Cbase + static_cast<long>(t0) * act_rs, act_rs, 64, NP, qlim - t0, d.N,
                 vec_act != 0, NoScale{});
  stage_rows<MT>(Xs, LDN, Hbase, d.N, 64, NP, d.P - p0, d.N, vec_state != 0, NoScale{});
  __syncthreads();

  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = (wid >> 1) * 32, wn = (wid & 1) * 32;
  v4f acc[2][2];
  zero_acc(acc);
  wave_mma<MT, 2, 2>(acc, Cs + wm * LDN, LDN, Xs + wn * LDN, LDN, NP, lane);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + wm + 16 * i + frag_row(lane, r);
      const float e = t < d.Lc ? fast_exp2(dcs[t]) : 0.0f;
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j][r] *= e;
    }
  __syncthreads();

  const long u_rs = static_cast<long>(d.H) * d.P;
  const T* ubase = u + (tok0 * d.H + h) * d.P + p0;
  const int s_end = min(t0 + 64, qlim);
  for (int s0 = 0; s0 < s_end; s0 += 64) {
    const int sv = min(64, qlim - s0);
    stage_rows<MT>(Xs, LDN, Bbase + static_cast<long>(s0) * act_rs, act_rs, 64, NP, sv, d.N,
                   vec_act != 0, NoScale{});
    stage_transposed<MT>(Us, LD64, ubase + static_cast<long>(s0) * u_rs, u_rs, 64, 64, sv,
                         d.P - p0, vec_act != 0, NoScale{});
    __syncthreads();
    v4f cb[2][2];
    zero_acc(cb);
    wave_mma<MT, 2, 2>(cb, Cs + wm * LDN, LDN, Xs + wn * LDN, LDN, NP, lane);
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
          if (s <= t && s < qlim && t < d.Lc)
            v = cb[i][j][r] * fast_exp2(fminf(dcs[t] - dcs[s], 0.0f)) * dts[s];
          Ls[tl * LD64 + sl] = from_f32<MT>(v);
        }
    __syncthreads();
    wave_mma<MT, 2, 2>(acc, Ls + wm * LD64, LD64, Us + wn * LD64, LD64, 64, lane);
    __syncthreads();
  }

  float* ybase = y + (tok0 * d.H + h) * d.P;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = t0 + wm + 16 * i + frag_row(lane, r);
        const int p = p0 + wn + 16 * j + frag_col(lane);
        if (t < qlim && p < d.P) ybase[static_cast<long>(t) * u_rs + p] = acc[i][j][r];
      }
}

// The SSM epilogue fused into the bf16 chunk scan (modules/ssm.py:144-150):
// out = (y + D u) silu(gate) and yd = y + D u, both bf16 (b, L, H, P), in place
// of the fp32 y.  D: (H * P,) float32; gate: (b, L, H, P) bf16.
struct GateOut {
  const float* D;
  const bf16* gate;
  bf16* out;
  bf16* yd;
};

// bf16 elements of the chunk-scan region that holds the HC heads' U tiles
// (HC LdsTile<64> tiles) and, after the sigma loop, one H_in tile
// (LdsTile<N>, 64 rows)
template <int NK, int HC>
constexpr int chunk_scan_ureg() {
  constexpr int u = HC * 64 * LdsTile<64>::kLd, hn = 64 * LdsTile<32 * NK>::kLd;
  return u > hn ? u : hn;
}

// ---------------------------------------------------------------------------
// chunk scan, bf16 fast path.  One block per (b, chunk, group, 64-row tau
// tile, 64-wide p tile, chunk of HC heads); wave w owns tau columns
// 16w..16w+15.  The raw C.B^T tile of each 64-row sigma tile is computed once
// (transposed, rows = sigma in key_of_row order, columns = tau) and shared by
// the HC heads: per head it is decayed in registers and fed as the B operand
// of Y^T[p][tau] += U^T[p][sigma] S^T[sigma][tau] (U read through LDS
// transpose reads).  C rows stay in registers for the whole block.
//   Y^T = U^T . S^T + exp(dc_tau) * H_in . C^T
// With dt >= 0 (mono) the decay of a sigma tile below the diagonal factors as
//   e^{dc_tau - dc_sig} = e^{dc_tau - dc_t0} * e^{dc_t0 - dc_sig}  (both <= 1):
// the sigma factor (times dt) is a per-tile table, the tau factor scales the
// accumulator once before the diagonal tile, which is decayed exactly.
// Tiles are prefetched into registers during the previous tile's MFMAs.
// ---------------------------------------------------------------------------
template <int NK, int HC, bool GATED>
__global__ __launch_bounds__(256, 2) void chunk_scan_fwd_bf16_kernel(
    const bf16* __restrict__ u, const bf16* __restrict__ Bm, const bf16* __restrict__ Cm,
    const float* __restrict__ dt, const float* __restrict__ dc, const float* __restrict__ states,
    float* __restrict__ y, GateOut go, SsdDims d, int mono) {
  constexpr int N = 32 * NK;
  using TB = LdsTile<N>;    // B sigma tile and H_in tile: 64 rows of N
  using TU = LdsTile<64>;   // U tiles: 64 sigma rows of 64 p
  constexpr int PLU = 64 * TU::kLd;
  constexpr int HQ = N / 16;   // float4 of an H tile per thread (64 x N fp32 / 256 threads)
  constexpr int UREG = chunk_scan_ureg<NK, HC>();   // bf16 of the U tiles / H_in tile region
  extern __shared__ __align__(16) unsigned char smem_raw[];
  bf16* Bs = reinterpret_cast<bf16*>(smem_raw);  // B rows of the sigma tile (TB)
  bf16* Us = Bs + 64 * TB::kLd;                  // [HC] U rows per head (TU); later the H_in tile (TB)
  float* tab = reinterpret_cast<float*>(Us + UREG);   // [HC][64] e^{dc_t0 - dc_sig} dt_sig
  float* dcd = tab + HC * 64;                                 // [HC][64] dc_sig (log2)
  float* dtd = dcd + HC * 64;                                 // [HC][64] dt_sig (0 past qlim)

  const int hpg = d.H / d.G;
  const int nhc = (hpg + HC - 1) / HC;
  const int ttiles = (d.Lc + 63) / 64, ptiles = (d.P + 63) / 64;
  const int bid = xcd_swizzle(blockIdx.x, gridDim.x);
  int rest = bid;
  // tau tile ti walks ti + 1 sigma tiles: longest first in each window of one
  // XCD's resident blocks (the launch rounds end on short blocks)
  int ti;
  xcd_window_order(bid, gridDim.x, ttiles, ti, rest);
  ti = ttiles - 1 - ti;
  const int pti = rest % ptiles;
  rest /= ptiles;
  const int hc = rest % nhc;
  rest /= nhc;
  const int g = rest % d.G;
  rest /= d.G;
  const int c = rest % d.nc;
  const int b = rest / d.nc;
  const int t0 = ti * 64, p0 = pti * 64;
  const int qlim = min(d.Lc, d.L - c * d.Lc);
  if (t0 >= qlim) return;
  const int h0 = g * hpg + hc * HC;
  const int nh = min(HC, hpg - hc * HC);

  const int tid = threadIdx.x, lane = tid & 63, cl = lane & 15, lg = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tau = t0 + 16 * w + cl;  // this lane's output column
  const long tok0 = static_cast<long>(b) * d.L + static_cast<long>(c) * d.Lc;
  const int act_rs = d.G * N, u_rs = d.H * d.P;
  const bf16* Bc = Bm + tok0 * act_rs + static_cast<long>(g) * N;
  const bf16* uc = u + tok0 * u_rs + h0 * d.P;
  const long crow0 = ((static_cast<long>(b) * d.H + h0) * d.nc + c) * d.Lc;   // dc / dt rows
  const long hrow = static_cast<long>(d.nc) * d.Lc;                          // per head

  v8bf Cw[NK];
  {
    const bf16* crow = Cm + (tok0 + min(tau, qlim - 1)) * act_rs + static_cast<long>(g) * N + 8 * lg;
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) Cw[ks] = tau < qlim ? load_v8bf(crow + 32 * ks) : zero_v8bf();
  }
  float dct[HC], lf[HC];
#pragma unroll
  for (int k = 0; k < HC; ++k) {
    const float* dch = dc + crow0 + min(k, nh - 1) * hrow;
    dct[k] = dch[min(tau, d.Lc - 1)] * kLog2e;
    lf[k] = fast_exp2(fminf(dct[k] - dch[t0] * kLog2e, 0.f));
  }
  v4f acc[HC][4];
#pragma unroll
  for (int k = 0; k < HC; ++k)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[k][t] = v4f{0.f, 0.f, 0.f, 0.f};

  // ---- sigma-tile staging (registers -> LDS) ----
  uint4 pb[NK];
  uint4 pu[HC][2];
  // raw dc / dt of the tile: the scaling and masking wait for commit_tile,
  // since arithmetic on a value right after its load waits for every load
  // issued before it (the tile's whole prefetch)
  float pdc = 0.f, pdt = 0.f, pdc0 = 0.f;
  bool pdt_ok = false;
  auto load_tile = [&](int s) {
    const int s0 = 64 * s, sv = min(64, qlim - s0);
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const int e = tid + 256 * i;
      const int row = e / (4 * NK), c8 = e % (4 * NK);
      pb[i] = *reinterpret_cast<const uint4*>(Bc + static_cast<unsigned>((s0 + min(row, sv - 1)) * act_rs + 8 * c8));
      if (row >= sv) pb[i] = uint4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int k = 0; k < HC; ++k)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = tid + 256 * i;
        const int row = e >> 3, col = p0 + 8 * (e & 7);
        const bf16* src = uc + min(k, nh - 1) * d.P +
                          static_cast<unsigned>((s0 + min(row, sv - 1)) * u_rs + min(col, d.P - 8));
        pu[k][i] = *reinterpret_cast<const uint4*>(src);
        if (row >= sv || col >= d.P || k >= nh) pu[k][i] = uint4{0u, 0u, 0u, 0u};
      }
    {
      const int k = tid >> 6, sig = s0 + (tid & 63);
      const float* dch = dc + crow0 + min(k, nh - 1) * hrow;
      pdc = dch[min(sig, d.Lc - 1)];
      pdc0 = dch[t0];
      pdt = dt[crow0 + min(k, nh - 1) * hrow + min(sig, d.Lc - 1)];
      pdt_ok = sig < qlim && k < nh;
    }
  };
  auto commit_tile = [&]() {
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const int e = tid + 256 * i;
      const int row = e / (4 * NK), c8 = e % (4 * NK);
      *reinterpret_cast<uint4*>(Bs + TB::off(row, 8 * c8)) = pb[i];
    }
#pragma unroll
    for (int k = 0; k < HC; ++k)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = tid + 256 * i;
        *reinterpret_cast<uint4*>(Us + k * PLU + TU::off(e >> 3, 8 * (e & 7))) = pu[k][i];
      }
    // with four heads every thread writes (a compile-time true condition:
    // under a runtime one the compiler moved the dc / dt loads of load_tile
    // into this branch, after the tile's MFMAs)
    if (HC * 64 >= 256 || tid < HC * 64) {
      const float c = pdc * kLog2e, t = pdt_ok ? pdt : 0.f;
      dcd[tid] = c;
      dtd[tid] = t;
      tab[tid] = t * fast_exp2(fminf(pdc0 * kLog2e - c, 0.f));
    }
  };

  // H_in staging for the state contribution (one head per stage, bf16 in the U tiles' space)
  bf16* Hs = Us;   // 64 rows of N bf16 (TB), in the U tiles' region
  float4 ph[HQ];
  auto load_h = [&](int k) {
    const float* Hb = states + (((static_cast<long>(b) * d.nc + c) * d.H + h0 + k) * d.P + p0) * N;
#pragma unroll
    for (int i = 0; i < HQ; ++i) {
      const int e = tid + 256 * i;
      const int row = e / (N / 4), c4 = e % (N / 4);
      ph[i] = *reinterpret_cast<const float4*>(Hb + static_cast<unsigned>(min(row, d.P - p0 - 1) * N + 4 * c4));
    }
  };
  // rows past P are zeroed here, not in load_h: a select right after the load
  // would wait for it there, before the MFMAs it is meant to overlap
  auto commit_h = [&]() {
#pragma unroll
    for (int i = 0; i < HQ; ++i) {
      const int e = tid + 256 * i;
      const int row = e / (N / 4), c4 = e % (N / 4);
      const uint2 v = uint2{pack_bf16x2(ph[i].x, ph[i].y), pack_bf16x2(ph[i].z, ph[i].w)};
      *reinterpret_cast<uint2*>(Hs + TB::off(row, 4 * c4)) = p0 + row < d.P ? v : uint2{0u, 0u};
    }
  };
  load_tile(0);
  commit_tile();
  __syncthreads();
  // one sigma tile: C.B^T, decay, Y^T += U^T S^T for every head
  // DIAG and FACT are compile-time, so that the decay of a tile is straight-line
  // code (a runtime choice per element row put a branch and an LDS wait
  // around every four products)
  auto sigma_tile = [&](int s, auto diag_c, auto fact_c) __attribute__((always_inline)) {
    constexpr bool DIAG = decltype(diag_c)::value, FACT = decltype(fact_c)::value;
    const int s0 = 64 * s;
    if (DIAG && mono) {
#pragma unroll
      for (int k = 0; k < HC; ++k)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[k][t] *= lf[k];
    }
    v4f cbt[4];
    // step i = (ks, kt): the B fragment of step i + 1 is read while step i's
    // MFMA runs, and consecutive MFMAs go to different accumulators
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) cbt[kt] = v4f{0.f, 0.f, 0.f, 0.f};
    v8bf bnx = load_v8bf(Bs + TB::off(key_of_row(0, cl), 8 * lg));
#pragma unroll
    for (int i = 0; i < 4 * NK; ++i) {
      const int ks = i / 4, kt = i % 4;
      const v8bf bf = bnx;
      if (i + 1 < 4 * NK)
        bnx = load_v8bf(Bs + TB::off(key_of_row((i + 1) % 4, cl), 8 * lg + 32 * ((i + 1) / 4)));
      __builtin_amdgcn_sched_barrier(0);
      cbt[kt] = mfma_bf16(bf, Cw[ks], cbt[kt]);
    }
    // every head slot runs, also past nh: its U tile and dt are zero
#pragma unroll
    for (int k = 0; k < HC; ++k) {
      v4f sk[4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const int tb = 32 * (kt >> 1) + 8 * lg + 4 * (kt & 1);   // 4 consecutive sigma rows
        if constexpr (FACT) {
          const float4 tq = *reinterpret_cast<const float4*>(tab + k * 64 + tb);
          sk[kt] = cbt[kt] * v4f{tq.x, tq.y, tq.z, tq.w};
        } else {
          const float4 dq = *reinterpret_cast<const float4*>(dcd + k * 64 + tb);
          const float4 tq = *reinterpret_cast<const float4*>(dtd + k * 64 + tb);
          const float dv[4] = {dq.x, dq.y, dq.z, dq.w}, tv[4] = {tq.x, tq.y, tq.z, tq.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float e = fast_exp2(fminf(dct[k] - dv[i], 0.f)) * tv[i];
            if constexpr (DIAG) {
              // e computed in every lane (the compiler would otherwise branch
              // around it per element) and the mask taken as a select
              asm volatile("" : "+v"(e));
              sk[kt][i] = s0 + tb + i <= tau ? cbt[kt][i] * e : 0.f;
            } else {
              sk[kt][i] = cbt[kt][i] * e;   // sigma < t0 <= tau
            }
          }
        }
      }
      const bf16* ut = Us + k * PLU;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const v8bf pbk = pack_p(sk[2 * ks], sk[2 * ks + 1]);
#pragma unroll
        for (int t = 0; t < 4; ++t)
          acc[k][t] = mfma_bf16(tile_tr8<64>(ut, 32 * ks + 8 * lg, 16 * t, lane), pbk, acc[k][t]);
      }
    }
  };
  auto below_diag = [&](auto fact_c) __attribute__((always_inline)) {
    for (int s = 0; s < ti; ++s) {
      load_tile(s + 1);
      sigma_tile(s, std::false_type{}, fact_c);
      __syncthreads();  // every wave is done with this tile
      commit_tile();
      __syncthreads();
    }
  };
  if (mono) below_diag(std::true_type{});
  else below_diag(std::false_type{});
  // the diagonal tile prefetches the first head's H_in instead (when its
  // registers fit beside the tile's: state_dim <= 192)
  constexpr bool kEarlyH = NK <= 6;
  if constexpr (kEarlyH) load_h(0);
  sigma_tile(ti, std::true_type{}, std::false_type{});
  __syncthreads();
  if constexpr (!kEarlyH) load_h(0);

  // ---- state contribution exp(dc_tau) * H_in . C^T, one head per stage ----
  // Without the gate epilogue, the y rows of head k leave through LDS as soon
  // as its state part is added, so that their stores overlap the next head's
  // stage: lane pieces in at 16-byte chunk c ^ (row % 16) of [64 rows][64 p]
  // fp32, then whole 256-byte rows out, 16 bytes per lane (stored from the
  // fragments, one instruction wrote 64 bytes of each of 16 rows).  The
  // staging is the B tile's space when that holds 16 KB, else the U region
  // past the H_in tile; either is disjoint from H_in.
  constexpr int kHsBytes = static_cast<int>(sizeof(bf16)) * 64 * TB::kLd;
  constexpr int kYsOff = kHsBytes >= 64 * 64 * 4 ? 0 : 2 * kHsBytes;
  static_assert(kYsOff + 64 * 64 * 4 <= static_cast<int>(sizeof(bf16)) * (64 * TB::kLd + UREG),
                "chunk_scan_fwd: the y staging fits in the tile region");
  float* ys = reinterpret_cast<float*>(smem_raw + kYsOff);
  const int rl = 16 * w + cl;
  commit_h();
  __syncthreads();
#pragma unroll
  for (int k = 0; k < HC; ++k) {
    if (k >= nh) break;
    const bool more = k + 1 < nh;
    if (more) load_h(k + 1);
    const float e = fast_exp2(dct[k]);
    {
      v4f st[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) st[t] = v4f{0.f, 0.f, 0.f, 0.f};
      v8bf hnx = load_v8bf(Hs + TB::off(cl, 8 * lg));
#pragma unroll
      for (int i = 0; i < 4 * NK; ++i) {
        const int ks = i / 4, t = i % 4;
        const v8bf hf = hnx;
        if (i + 1 < 4 * NK)
          hnx = load_v8bf(Hs + TB::off(16 * ((i + 1) % 4) + cl, 8 * lg + 32 * ((i + 1) / 4)));
        __builtin_amdgcn_sched_barrier(0);
        st[t] = mfma_bf16(hf, Cw[ks], st[t]);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[k][t] += st[t] * e;
    }
    if constexpr (!GATED) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        *reinterpret_cast<float4*>(ys + rl * 64 + 4 * ((4 * t + lg) ^ (rl & 15))) =
            make_float4(acc[k][t][0], acc[k][t][1], acc[k][t][2], acc[k][t][3]);
      __syncthreads();   // head k's rows staged; every wave is done with its H_in tile
      if (more) commit_h();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e2 = tid + 256 * i, r = e2 >> 4, ch = e2 & 15;
        if (t0 + r < qlim && p0 + 4 * ch < d.P)
          *reinterpret_cast<float4*>(y + (tok0 + t0 + r) * u_rs + static_cast<long>(h0 + k) * d.P + p0 + 4 * ch) =
              *reinterpret_cast<const float4*>(ys + r * 64 + 4 * (ch ^ (r & 15)));
      }
      if (more) __syncthreads();   // the next H_in tile is in; the staging is free
    } else if (more) {
      __syncthreads();
      commit_h();
      __syncthreads();
    }
  }
  if constexpr (GATED) {
    if (tau < qlim) {
      // SSM epilogue: yd = y + D u, out = yd silu(gate) (bf16; y itself is not stored)
#pragma unroll
      for (int k = 0; k < HC; ++k) {
        if (k >= nh) break;
        const long row = (tok0 + tau) * u_rs + static_cast<long>(h0 + k) * d.P;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int p = p0 + 16 * t + 4 * lg;
          if (p >= d.P) continue;
          const uint2 uq = *reinterpret_cast<const uint2*>(u + row + p);
          const uint2 gq = *reinterpret_cast<const uint2*>(go.gate + row + p);
          const float4 dq = *reinterpret_cast<const float4*>(go.D + (h0 + k) * d.P + p);
          const float uv[4] = {bf16lo_to_f32(uq.x), bf16hi_to_f32(uq.x), bf16lo_to_f32(uq.y), bf16hi_to_f32(uq.y)};
          const float gv[4] = {bf16lo_to_f32(gq.x), bf16hi_to_f32(gq.x), bf16lo_to_f32(gq.y), bf16hi_to_f32(gq.y)};
          const float Dv[4] = {dq.x, dq.y, dq.z, dq.w};
          float yd[4], o[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            yd[i] = acc[k][t][i] + Dv[i] * uv[i];
            o[i] = yd[i] * gv[i] * fast_sigmoid(gv[i]);
          }
          *reinterpret_cast<uint2*>(go.out + row + p) = uint2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
          *reinterpret_cast<uint2*>(go.yd + row + p) = uint2{pack_bf16x2(yd[0], yd[1]), pack_bf16x2(yd[2], yd[3])};
        }
      }
    }
  }
}

size_t chunk_scan_smem(int N, int Lc, bool bf) {
  const int NP = round_up(N, 32);
  const size_t e = bf ? 2 : 4;
  const int LDN = NP + (bf ? 8 : 4), LD64 = 64 + (bf ? 8 : 4);
  return e * (2 * 64 * LDN + 2 * 64 * LD64) + 2 * sizeof(float) * Lc;
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
template <typename T>
int launch_chunk_cumsum(const void* delta_raw, const float* A, const float* bias,
                        const int64_t* length, float* dt, float* dc, const SsdDims& d, int sp,
                        float lo, float hi, hipStream_t s) {
  const long blocks = static_cast<long>(d.b) * d.nc * d.H;
  ProfScope prof_("chunk_cumsum_fwd", s);
  hipLaunchKernelGGL(chunk_cumsum_kernel<T>, dim3(blocks), dim3(256), 0, s,
                     static_cast<const T*>(delta_raw), A, bias, length, dt, dc, d, sp, lo, hi);
  SA_CHECK_LAUNCH("chunk_cumsum");
  return 0;
}

template <int NK, int MODE>
int launch_chunk_outer_bf16_nk(const void* a, const void* x, const float* dt, const float* dc,
                               const int64_t* length, float* out, const SsdDims& d, hipStream_t s,
                               bf16* dyp = nullptr) {
  const long blocks = static_cast<long>(d.P / 64) * d.H * d.nc * d.b;
  const size_t smem = sizeof(bf16) * 64 * (2 * LdsTile<64>::kLd + LdsTile<32 * NK>::kLd);
  if (smem > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(chunk_outer_bf16_kernel<NK, MODE>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem));
    SA_CHECK_ARG(e == hipSuccess, "chunk_outer_bf16: %zu B of LDS refused", smem);
  }
  ProfScope prof_(MODE == 0 ? "chunk_state_fwd" : "chunk_dstate_bwd", s);
  hipLaunchKernelGGL((chunk_outer_bf16_kernel<NK, MODE>), dim3(blocks), dim3(256), smem, s, a,
                     static_cast<const bf16*>(x), dt, dc, length, out, dyp, d);
  SA_CHECK_LAUNCH("chunk_outer_bf16");
  return 0;
}

template <typename MT, typename TA, typename TB, int MODE>
int launch_chunk_outer(const void* a, const void* bsrc, const float* dt, const float* dc,
                       const int64_t* length, float* out, const SsdDims& d, hipStream_t s) {
  if (sizeof(MT) == 2 && sizeof(TB) == 2 && d.P % 64 == 0 && d.N % 64 == 0 && aligned16(a) &&
      aligned16(bsrc)) {
    switch (d.N / 64) {
      case 1: return launch_chunk_outer_bf16_nk<2, MODE>(a, bsrc, dt, dc, length, out, d, s);
      case 2: return launch_chunk_outer_bf16_nk<4, MODE>(a, bsrc, dt, dc, length, out, d, s);
      case 3: return launch_chunk_outer_bf16_nk<6, MODE>(a, bsrc, dt, dc, length, out, d, s);
      default: return launch_chunk_outer_bf16_nk<8, MODE>(a, bsrc, dt, dc, length, out, d, s);
    }
  }
  const long blocks = static_cast<long>((d.P + 63) / 64) * ((d.N + 63) / 64) * d.b * d.nc * d.H;
  const int vec_a = aligned16(a) && (static_cast<long>(d.H) * d.P) % 8 == 0 && d.P % 8 == 0;
  const int vec_b = aligned16(bsrc) && (static_cast<long>(d.G) * d.N) % 8 == 0 && d.N % 8 == 0;
  ProfScope prof_(MODE == 0 ? "chunk_state_fwd" : "chunk_dstate_bwd", s);
  hipLaunchKernelGGL((chunk_outer_kernel<MT, TA, TB, MODE>), dim3(blocks), dim3(256), 0, s,
                     static_cast<const TA*>(a), static_cast<const TB*>(bsrc), dt, dc, length, out,
                     d, vec_a, vec_b);
  SA_CHECK_LAUNCH("chunk_outer");
  return 0;
}

int launch_dstate_planes(const float* dy, const void* C, const float* dt, const float* dc,
                         const int64_t* length, float* out, bf16* dyp, const SsdDims& d,
                         hipStream_t s) {
  SA_CHECK_ARG(d.P == 64 && (d.N == 64 || d.N == 128) && d.Lc % 64 == 0 && aligned16(dy) &&
                   aligned16(C),
               "launch_dstate_planes: P 64, N 64 or 128, chunk %% 64 and aligned operands required");
  if (d.N == 64) return launch_chunk_outer_bf16_nk<2, 1>(dy, C, dt, dc, length, out, d, s, dyp);
  return launch_chunk_outer_bf16_nk<4, 1>(dy, C, dt, dc, length, out, d, s, dyp);
}

// compute units of the current device (cached per device; 256 if unknown)
int device_cus() {
  static int cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      return 256;
    cache[dev] = cus;
  }
  return cache[dev];
}

// chunk states and state passing in one kernel: bf16 u and B, head_dim and
// state_dim multiples of 64, 16-byte aligned operands, and at least two
// blocks per CU.  Its blocks walk every chunk in order, so it wins only
// while every CU holds two of them (config 1: 512 blocks of 64 t tiles,
// 108 us against 127 for the two kernels); with fewer, longer walks it
// loses (config 4's SSM shape, 256 blocks of 128 tiles: 154 against ~127 us;
// the reference default, 128 blocks: 80 us).
// n blocks of 128 (one 512-thread block per CU) where state_dim allows,
// else of 64 (two 256-thread blocks per CU); 0: the fused kernel does not fit
static int chunk_state_pass_nb(const SsdDims& d) {
  if (d.P % 64 != 0 || d.N % 64 != 0) return 0;
  const long bhp = static_cast<long>(d.b) * d.H * (d.P / 64);
  if (d.N % 128 == 0 && bhp * (d.N / 128) >= device_cus()) return 2;
  if (bhp * (d.N / 64) >= 2L * device_cus()) return 1;
  return 0;
}
bool chunk_state_pass_ok(const SsdDims& d, const void* u, const void* B, const float* h_init,
                         const float* states, const float* h_last) {
  return chunk_state_pass_nb(d) > 0 && aligned16(u) && aligned16(B) &&
         (!h_init || aligned16(h_init)) && aligned16(states) && aligned16(h_last);
}
int launch_chunk_state_pass(const void* u, const void* B, const float* dt, const float* dc,
                            const float* h_init, float* states, float* h_last, const SsdDims& d,
                            hipStream_t s) {
  const int nb = chunk_state_pass_nb(d);
  SA_CHECK_ARG(nb > 0, "chunk_state_pass: shape not covered");
  const long blocks = static_cast<long>(d.b) * d.H * (d.P / 64) * (d.N / (64 * nb));
  ProfScope prof_("chunk_state_pass_fwd", s);
  if (nb == 2)
    hipLaunchKernelGGL(chunk_state_pass_kernel<2>, dim3(blocks), dim3(512), 0, s,
                       static_cast<const bf16*>(u), static_cast<const bf16*>(B), dt, dc, h_init,
                       states, h_last, d);
  else
    hipLaunchKernelGGL(chunk_state_pass_kernel<1>, dim3(blocks), dim3(256), 0, s,
                       static_cast<const bf16*>(u), static_cast<const bf16*>(B), dt, dc, h_init,
                       states, h_last, d);
  SA_CHECK_LAUNCH("chunk_state_pass");
  return 0;
}

int launch_state_passing_fwd(float* states, const float* h_init, float* h_last, const float* dc,
                             const SsdDims& d, hipStream_t s) {
  const long PN = static_cast<long>(d.P) * d.N;
  const long blocks = static_cast<long>(d.b) * d.H * ((PN + 1023) / 1024);
  ProfScope prof_("state_passing_fwd", s);
  hipLaunchKernelGGL(state_passing_fwd_kernel, dim3(blocks), dim3(256), 0, s, states, h_init,
                     h_last, dc, d);
  SA_CHECK_LAUNCH("state_passing_fwd");
  return 0;
}

template <typename MT, typename T>
int launch_chunk_scan(const void* u, const void* B, const void* C, const float* dt,
                      const float* dc, const float* states, float* y, const SsdDims& d,
                      hipStream_t s) {
  const long blocks = static_cast<long>((d.Lc + 63) / 64) * ((d.P + 63) / 64) * d.b * d.nc * d.H;
  const size_t smem = chunk_scan_smem(d.N, d.Lc, sizeof(MT) == 2);
  const int vec_act = aligned16(u) && aligned16(B) && aligned16(C) && d.P % 8 == 0 &&
                      d.N % 8 == 0 && (static_cast<long>(d.H) * d.P) % 8 == 0;
  const int vec_state = aligned16(states) && d.N % 8 == 0;
  if (smem > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(chunk_scan_fwd_kernel<MT, T>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(smem));
    SA_CHECK_ARG(e == hipSuccess, "chunk_scan_fwd: %zu B of LDS refused: %s", smem,
                 hipGetErrorString(e));
  }
  ProfScope prof_("chunk_scan_fwd", s);
  hipLaunchKernelGGL((chunk_scan_fwd_kernel<MT, T>), dim3(blocks), dim3(256), smem, s,
                     static_cast<const T*>(u), static_cast<const T*>(B), static_cast<const T*>(C),
                     dt, dc, states, y, d, vec_act, vec_state);
  SA_CHECK_LAUNCH("chunk_scan_fwd");
  return 0;
}

// bf16 fast path: N a multiple of 32 (<= 256), P a multiple of 16
template <int NK>
int launch_chunk_scan_bf16_nk(const void* u, const void* B, const void* C, const float* dt,
                              const float* dc, const float* states, float* y, const SsdDims& d,
                              int mono, const GateOut* go, hipStream_t s) {
  constexpr int HC = NK <= 6 ? 4 : 2;   // heads per block (state_dim > 192: registers)
  const int hpg = d.H / d.G;
  const int nhc = (hpg + HC - 1) / HC;
  const long blocks = static_cast<long>((d.Lc + 63) / 64) * ((d.P + 63) / 64) * nhc * d.G *
                      d.nc * d.b;
  const size_t smem = sizeof(bf16) * (64 * LdsTile<32 * NK>::kLd + chunk_scan_ureg<NK, HC>()) +
                      sizeof(float) * HC * 192;
  auto run = [&](auto kernel, const char* name) -> int {
    if (smem > 64 * 1024) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         static_cast<int>(smem));
      SA_CHECK_ARG(e == hipSuccess, "chunk_scan_fwd_bf16: %zu B of LDS refused", smem);
    }
    ProfScope prof_(name, s);
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(256), smem, s, static_cast<const bf16*>(u),
                       static_cast<const bf16*>(B), static_cast<const bf16*>(C), dt, dc, states,
                       y, go ? *go : GateOut{}, d, mono);
    SA_CHECK_LAUNCH("chunk_scan_fwd_bf16");
    return 0;
  };
  if (go) return run(chunk_scan_fwd_bf16_kernel<NK, HC, true>, "chunk_scan_fwd_gated");
  return run(chunk_scan_fwd_bf16_kernel<NK, HC, false>, "chunk_scan_fwd");
}

inline bool chunk_scan_bf16_ok(const SsdDims& d, const void* u, const void* B, const void* C,
                               const float* states) {
  return d.N % 32 == 0 && d.N <= 256 && d.P % 8 == 0 && aligned16(u) && aligned16(B) &&
         aligned16(C) && aligned16(states);
}

int launch_chunk_scan_bf16(const void* u, const void* B, const void* C, const float* dt,
                           const float* dc, const float* states, float* y, const SsdDims& d,
                           int mono, const GateOut* go, hipStream_t s) {
  switch (d.N / 32) {
    case 1: return launch_chunk_scan_bf16_nk<1>(u, B, C, dt, dc, states, y, d, mono, go, s);
    case 2: return launch_chunk_scan_bf16_nk<2>(u, B, C, dt, dc, states, y, d, mono, go, s);
    case 3: return launch_chunk_scan_bf16_nk<3>(u, B, C, dt, dc, states, y, d, mono, go, s);
    case 4: return launch_chunk_scan_bf16_nk<4>(u, B, C, dt, dc, states, y, d, mono, go, s);
    case 5: return launch_chunk_scan_bf16_nk<5>(u, B, C, dt, dc, states, y, d, mono, go, s);
    case 6: return launch_chunk_scan_bf16_nk<6>(u, B, C, dt, dc, states, y, d, mono, go, s);
    case 7: return launch_chunk_scan_bf16_nk<7>(u, B, C, dt, dc, states, y, d, mono, go, s);
    default: return launch_chunk_scan_bf16_nk<8>(u, B, C, dt, dc, states, y, d, mono, go, s);
  }
}

template <typename T, typename MT>
int ssd_fwd_impl(const void* u, const float* A, const void* B, const void* C,
                 const void* delta_raw, const float* bias, const float* h_init,
                 const int64_t* length, const SsdDims& d, int sp, float lo, float hi, float* y,
                 float* h_last, float* dt, float* dc, float* states, hipStream_t s,
                 const GateOut* go = nullptr) {
  int rc;
  const bool fast = sizeof(T) == 2 && chunk_scan_bf16_ok(d, u, B, C, states);
  SA_CHECK_ARG(!go || fast, "sa_ssd_fwd_gated: the fused epilogue needs the bf16 fast path "
               "(state_dim a multiple of 32, <= 256; head_dim a multiple of 8; 16-byte aligned)");
  if ((rc = launch_chunk_cumsum<T>(delta_raw, A, bias, length, dt, dc, d, sp, lo, hi, s))) return rc;
  if (sizeof(T) == 2 && chunk_state_pass_ok(d, u, B, h_init, states, h_last)) {
    if ((rc = launch_chunk_state_pass(u, B, dt, dc, h_init, states, h_last, d, s))) return rc;
  } else {
    if ((rc = launch_chunk_outer<MT, T, T, 0>(u, B, dt, dc, length, states, d, s))) return rc;
    if ((rc = launch_state_passing_fwd(states, h_init, h_last, dc, d, s))) return rc;
  }
  if (fast) return launch_chunk_scan_bf16(u, B, C, dt, dc, states, y, d, lo >= 0.f ? 1 : 0, go, s);
  return launch_chunk_scan<MT, T>(u, B, C, dt, dc, states, y, d, s);
}

template int launch_chunk_outer<float, float, float, 1>(const void*, const void*, const float*,
                                                        const float*, const int64_t*, float*,
                                                        const SsdDims&, hipStream_t);
template int launch_chunk_outer<bf16, float, bf16, 1>(const void*, const void*, const float*,
                                                      const float*, const int64_t*, float*,
                                                      const SsdDims&, hipStream_t);
template int launch_chunk_outer<bf16, bf16, bf16, 1>(const void*, const void*, const float*,
                                                     const float*, const int64_t*, float*,
                                                     const SsdDims&, hipStream_t);

}  // namespace sa

extern "C" int sa_ssd_fwd(int dtype, const void* u, const float* A, const void* B, const void* C,
                          const void* delta_raw, const float* delta_bias, const float* h_init,
                          const int64_t* length, int batch, int seqlen, int num_heads,
                          int head_dim, int num_groups, int state_dim, int chunk_size,
                          int use_softplus, float delta_min, float delta_max, float* y,
                          float* h_last, float* dt, float* dc, float* states, void* stream) {
  sa::SsdDims d;
  int rc = sa::make_dims(batch, seqlen, num_heads, head_dim, num_groups, state_dim, chunk_size, &d,
                         "sa_ssd_fwd");
  if (rc) return rc;
  SA_CHECK_ARG(u && A && B && C && delta_raw && y && h_last && dt && dc && states,
               "sa_ssd_fwd: null tensor pointer");
  SA_CHECK_ARG(dtype != sa::kF32 || state_dim <= 128,
               "sa_ssd_fwd: float32 path supports state_dim <= 128 (got %d)", state_dim);
  if (d.b == 0 || d.L == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == sa::kF32)
    return sa::ssd_fwd_impl<float, float>(u, A, B, C, delta_raw, delta_bias, h_init, length, d,
                                          use_softplus, delta_min, delta_max, y, h_last, dt, dc,
                                          states, s);
  if (dtype == sa::kBF16)
    return sa::ssd_fwd_impl<sa::bf16, sa::bf16>(u, A, B, C, delta_raw, delta_bias, h_init, length,
                                                d, use_softplus, delta_min, delta_max, y, h_last,
                                                dt, dc, states, s);
  sa_set_error("sa_ssd_fwd: unsupported dtype %d", dtype);
  return 1;
}

extern "C" int sa_ssd_fwd_gated_supported(int dtype, int head_dim, int state_dim) {
  return dtype == sa::kBF16 && head_dim % 8 == 0 && state_dim % 32 == 0 && state_dim <= 256 ? 1 : 0;
}

extern "C" int sa_ssd_fwd_gated(int dtype, const void* u, const float* A, const void* B,
                                const void* C, const void* delta_raw, const float* delta_bias,
                                const float* h_init, const int64_t* length, int batch, int seqlen,
                                int num_heads, int head_dim, int num_groups, int state_dim,
                                int chunk_size, int use_softplus, float delta_min, float delta_max,
                                const float* D, const void* gate, void* out, void* yd,
                                float* h_last, float* dt, float* dc, float* states, void* stream) {
  sa::SsdDims d;
  int rc = sa::make_dims(batch, seqlen, num_heads, head_dim, num_groups, state_dim, chunk_size, &d,
                         "sa_ssd_fwd_gated");
  if (rc) return rc;
  SA_CHECK_ARG(sa_ssd_fwd_gated_supported(dtype, head_dim, state_dim),
               "sa_ssd_fwd_gated: needs bfloat16 activations, head_dim %% 8 == 0 and state_dim a "
               "multiple of 32 up to 256 (got dtype %d, P=%d, N=%d)", dtype, head_dim, state_dim);
  SA_CHECK_ARG(u && A && B && C && delta_raw && D && gate && out && yd && h_last && dt &&
                   dc && states,
               "sa_ssd_fwd_gated: null tensor pointer");
  SA_CHECK_ARG(sa::aligned16(D) && sa::aligned16(gate) && sa::aligned16(out) && sa::aligned16(yd),
               "sa_ssd_fwd_gated: D, gate, out and yd must be 16-byte aligned");
  if (d.b == 0 || d.L == 0) return 0;
  const sa::GateOut go{D, static_cast<const sa::bf16*>(gate), static_cast<sa::bf16*>(out),
                       static_cast<sa::bf16*>(yd)};
  return sa::ssd_fwd_impl<sa::bf16, sa::bf16>(u, A, B, C, delta_raw, delta_bias, h_init, length, d,
                                              use_softplus, delta_min, delta_max, nullptr, h_last,
                                              dt, dc, states, static_cast<hipStream_t>(stream), &go);
}
