// Attention ops of the kernel layer (gfx950, bf16):
//   sparse_attn_fwd   varlen block-sparse causal self-attention (prefill)
//   paged_decode      split-KV paged GQA decode attention + LSE merge
//
// The reference has no kernel for either (its attention is dense torch in
// modules/selective_attention.py); semantics follow its gated softmax:
// scores q.k*scale (+ optional per-key log-gate bias, exempt on the diagonal
// for prefill, mode "seq" :125-144, and on the newest key for decode,
// mode "pos" :121-123), softmax, times V.
//
// MFMA layout (16x16x32 bf16): scores are computed transposed,
// S^T[key][q] = K . Q^T, so a lane holds 4 keys of one query column.  That is
// already the B-operand fragment of O^T = V^T . P^T: P never goes through
// LDS, and the running max / sum of query q stay in the lanes holding
// O^T[:, q].  Within a 64-key tile, MFMA row c of score tile kt is mapped to
// key  32(kt/2) + 8(c/4) + 4(kt%2) + c%4  (key_of_row), so the 8 keys a lane
// contributes to one 32-key step of V^T . P^T are consecutive and its V^T
// operand is a single 16-byte read: from LDS for prefill (V transposed on
// staging) and straight from HBM for decode, whose V pages are stored
// transposed, (num_pages, Hkv, D, page_size).
#include "common.h"
#include "prof.h"
#include "tile.h"

namespace sa {

constexpr float kNegInf = -__builtin_huge_valf();

// Online-softmax update for one block of keys.  s[kt][i]: log2-domain scores
// of keys 16kt + 4g + i for query column (lane & 15); masked entries are
// -inf.  Converts s to probabilities in place, rescales o, updates m and l.
template <int KT, int DT>
__device__ __forceinline__ void softmax_block(v4f (&s)[KT], v4f (&o)[DT], float& m, float& l) {
  float mx = kNegInf;
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[kt][i]);
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  const float m_new = fmaxf(m, mx);
  const float alpha = (m == kNegInf) ? 0.0f : fast_exp2(m - m_new);
  float sum = 0.0f;
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = (s[kt][i] == kNegInf) ? 0.0f : fast_exp2(s[kt][i] - m_new);
      s[kt][i] = p;
      sum += p;
    }
  sum += __shfl_xor(sum, 16, 64);
  sum += __shfl_xor(sum, 32, 64);
  l = l * alpha + sum;
  m = m_new;
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] *= alpha;
}

// O^T[d][q] += sum_key V^T[d][key] P^T[key][q] over 64 keys; Vt points at
// V^T[0][tile start] with row stride ldv; s: probabilities from softmax_block
template <int DT>
__device__ __forceinline__ void pv_block(v4f (&o)[DT], const v4f (&s)[4], const bf16* Vt, int ldv,
                                         int lane) {
  const int c = lane & 15, g = lane >> 4;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const v8bf pb = pack_p(s[2 * ks], s[2 * ks + 1]);
#pragma unroll
    for (int t = 0; t < DT; ++t)
      o[t] = mfma_bf16(load_v8bf(Vt + (16 * t + c) * ldv + 32 * ks + 8 * g), pb, o[t]);
  }
}

// ---------------------------------------------------------------------------
// block-sparse varlen prefill.  One workgroup per (head, 64-query block);
// wave w owns query rows 16w..16w+15 of the block.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void sparse_attn_fwd_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const int32_t* __restrict__ cu, int nseq, const int32_t* __restrict__ block_idx, int n_qblk,
    int max_blocks, const float* __restrict__ key_bias, bf16* __restrict__ o, int T, int H,
    float scale_log2) {
  constexpr int BS = 64;
  constexpr int LDK = D + 8, LDV = BS + 8;
  constexpr int DT = D / 16, KS = D / 32;
  __shared__ __align__(16) bf16 Ks[BS * LDK];
  __shared__ __align__(16) bf16 Vt[D * LDV];

  const int lid = xcd_swizzle(blockIdx.x, gridDim.x);
  const int h = lid / n_qblk;
  const int gq = lid - h * n_qblk;
  // locate the query block's sequence: q blocks are numbered sequence by sequence
  int s = 0, first = 0, start = 0, n = 0;
  for (; s < nseq; ++s) {
    const int a = min(max(cu[s], 0), T), b = min(max(cu[s + 1], a), T);
    const int nb = (b - a + BS - 1) / BS;
    if (gq < first + nb) {
      start = a;
      n = b - a;
      break;
    }
    first += nb;
  }
  if (s == nseq) return;  // more query blocks than the packing holds
  const int jq = gq - first;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int qloc = jq * BS + 16 * wid + c;  // this lane's query (local position)
  const long rs = static_cast<long>(H) * D;
  const bf16* qrow = q + (start + static_cast<long>(min(qloc, n - 1))) * rs + static_cast<long>(h) * D;
  v8bf qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    qf[ks] = qloc < n ? load_v8bf(qrow + 32 * ks + 8 * g) : zero_v8bf();
  const float* bias = key_bias ? key_bias + static_cast<long>(h) * T + start : nullptr;

  float m = kNegInf, l = 0.0f;
  v4f acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};

  const int32_t* sel = block_idx + (static_cast<long>(h) * n_qblk + gq) * max_blocks;
  const int nkb = (n + BS - 1) / BS;
  for (int e = 0; e < max_blocks; ++e) {
    const int kb = sel[e];
    if (kb < 0 || kb >= nkb || kb > jq) continue;  // unused slot / outside the causal range
    const int k0 = kb * BS;
    const int nk = min(BS, n - k0);
    __syncthreads();
    stage_rows<bf16>(Ks, LDK, k + (start + static_cast<long>(k0)) * rs + static_cast<long>(h) * D, rs,
                     BS, D, nk, D, true, NoScale{});
    stage_transposed<bf16>(Vt, LDV, v + (start + static_cast<long>(k0)) * rs + static_cast<long>(h) * D,
                           rs, BS, D, nk, D, true, NoScale{});
    __syncthreads();
    v4f sc[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      sc[kt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        sc[kt] = mfma_bf16(load_v8bf(Ks + key_of_row(kt, c) * LDK + 32 * ks + 8 * g), qf[ks],
                           sc[kt]);
    }
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kl = key_of_row(kt, 4 * g + i);
        const int key = k0 + kl;
        float val = kNegInf;
        if (kl < nk && key <= qloc && qloc < n) {
          val = sc[kt][i] * scale_log2;
          if (bias && key != qloc) val += bias[key] * kLog2e;
        }
        sc[kt][i] = val;
      }
    softmax_block<4, DT>(sc, acc, m, l);
    pv_block<DT>(acc, sc, Vt, LDV, lane);
  }
  if (qloc < n) {
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    bf16* orow = o + (start + static_cast<long>(qloc)) * rs + static_cast<long>(h) * D;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      uint2 w;
      w.x = pack_bf16x2(acc[t][0] * inv, acc[t][1] * inv);
      w.y = pack_bf16x2(acc[t][2] * inv, acc[t][3] * inv);
      *reinterpret_cast<uint2*>(orow + 16 * t + 4 * g) = w;
    }
  }
}

// ---------------------------------------------------------------------------
// paged GQA decode, split over pages.  One wave per (batch row, kv head,
// split of PPS pages); the query heads of the group sit in the first lanes
// of each 16-lane column group (columns >= group size are padding).  No LDS:
// K rows and V^T rows go from HBM straight into MFMA operands; all loads of
// a 64-key tile are issued before its first MFMA.
// ---------------------------------------------------------------------------
template <int D>
struct DecodeTile {
  v8bf kf[4][D / 32];
  v8bf vf[2][D / 16];
  long kbase;  // key index of the tile's first key in the K pool (per kv head)
  int nk;      // valid keys (0: skip)
  int pos0;    // sequence position of the tile's first key
};

template <int D>
__device__ __forceinline__ void decode_load(DecodeTile<D>& T, const bf16* __restrict__ kp,
                                            const bf16* __restrict__ vp, int page, int Hkv,
                                            int kvh, int ps, int num_pages, int k0, int nk_page,
                                            int pos0, int c, int g) {
  constexpr int KS = D / 32, DT = D / 16;
  T.nk = (page < 0 || page >= num_pages) ? 0 : min(64, nk_page - k0);
  T.pos0 = pos0;
  const long pbase = (static_cast<long>(max(page, 0)) * Hkv + kvh) * ps;
  T.kbase = pbase + k0;
  const bf16* kbase = kp + (pbase + k0) * D;
  const bf16* vbase = vp + pbase * D + k0;  // V^T page: [D][ps]
  const int nk = T.nk;
  // Every address below stays inside the (clamped) page: keys past nk are
  // read but never used -- their scores are replaced by -inf and their V
  // entries are zeroed by a bit mask, so stale pool contents cannot leak in.
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    const int key = key_of_row(kt, c);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) T.kf[kt][ks] = load_v8bf(kbase + key * D + 32 * ks + 8 * g);
  }
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int kk = 32 * ks + 8 * g;
    uint32_t mk[4];
#pragma unroll
    for (int w = 0; w < 4; ++w)
      mk[w] = (kk + 2 * w < nk ? 0x0000ffffu : 0u) | (kk + 2 * w + 1 < nk ? 0xffff0000u : 0u);
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      uint4 r = *reinterpret_cast<const uint4*>(vbase + static_cast<long>(16 * t + c) * ps + kk);
      r.x &= mk[0];
      r.y &= mk[1];
      r.z &= mk[2];
      r.w &= mk[3];
      T.vf[ks][t] = __builtin_bit_cast(v8bf, r);
    }
  }
}

template <int D>
__device__ __forceinline__ void decode_compute(const DecodeTile<D>& T, const v8bf (&qf)[D / 32],
                                               v4f (&acc)[D / 16], float& m, float& l,
                                               const float* __restrict__ key_bias, int n,
                                               int grp, float scale_log2, int c, int g) {
  constexpr int KS = D / 32, DT = D / 16;
  if (T.nk <= 0) return;
  v4f sc[4];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    sc[kt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) sc[kt] = mfma_bf16(T.kf[kt][ks], qf[ks], sc[kt]);
  }
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kl = key_of_row(kt, 4 * g + i);
      float val = kNegInf;
      if (kl < T.nk && c < grp) {
        val = sc[kt][i] * scale_log2;
        if (key_bias && T.pos0 + kl != n - 1) val += key_bias[T.kbase + kl] * kLog2e;
      }
      sc[kt][i] = val;
    }
  softmax_block<4, DT>(sc, acc, m, l);
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const v8bf pb = pack_p(sc[2 * ks], sc[2 * ks + 1]);
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] = mfma_bf16(T.vf[ks][t], pb, acc[t]);
  }
}

template <int D>
__global__ __launch_bounds__(64) void paged_decode_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ kp, const bf16* __restrict__ vp,
    const int32_t* __restrict__ page_table, const int32_t* __restrict__ seq_lens,
    const float* __restrict__ key_bias, float* __restrict__ part_o, float* __restrict__ part_ml,
    int Hq, int Hkv, int ps, int max_pages, int num_pages, int pps, int max_splits,
    float scale_log2) {
  constexpr int DT = D / 16, KS = D / 32;
  const int item = blockIdx.x;
  const int split = item % max_splits;
  const int rest = item / max_splits;
  const int kvh = rest % Hkv;
  const int bi = rest / Hkv;
  const int grp = Hq / Hkv;
  const int n = min(max(seq_lens[bi], 0), max_pages * ps);
  const int npg = (n + ps - 1) / ps;
  const int p_begin = split * pps, p_end = min(npg, p_begin + pps);
  if (p_begin >= p_end) return;
  const int lane = threadIdx.x, c = lane & 15, g = lane >> 4;

  const bf16* qrow = q + (static_cast<long>(bi) * Hq + kvh * grp + min(c, grp - 1)) * D;
  v8bf qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) qf[ks] = c < grp ? load_v8bf(qrow + 32 * ks + 8 * g) : zero_v8bf();

  float m = kNegInf, l = 0.0f;
  v4f acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};

  // 64-key tiles of this split, in order
  const int tiles_per_page = ps / 64;
  const int ntiles = (p_end - p_begin) * tiles_per_page;
  const int32_t* prow = page_table + static_cast<long>(bi) * max_pages;
  auto load = [&](DecodeTile<D>& T, int t) {
    const int pg = p_begin + t / tiles_per_page;
    const int k0 = (t % tiles_per_page) * 64;
    decode_load<D>(T, kp, vp, prow[pg], Hkv, kvh, ps, num_pages, k0, min(ps, n - pg * ps),
                   pg * ps + k0, c, g);
  };
  DecodeTile<D> A;
  for (int t = 0; t < ntiles; ++t) {
    load(A, t);
    decode_compute<D>(A, qf, acc, m, l, key_bias, n, grp, scale_log2, c, g);
  }
  // partial results: O^T[d][q] unnormalised, with m (log2 domain) and l
  const long slot = (static_cast<long>(bi) * Hkv + kvh) * max_splits + split;
  if (c < grp) {
    float* po = part_o + (slot * grp + c) * D;
#pragma unroll
    for (int t = 0; t < DT; ++t)
      *reinterpret_cast<float4*>(po + 16 * t + 4 * g) = make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
    if (g == 0) {
      part_ml[(slot * grp + c) * 2] = m;
      part_ml[(slot * grp + c) * 2 + 1] = l;
    }
  }
}

// merge the splits of one (batch row, query head); one wave, the split
// weights exp2(m_s - M) computed lane-parallel into LDS
__global__ __launch_bounds__(64) void paged_decode_merge_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_ml,
    const int32_t* __restrict__ seq_lens, bf16* __restrict__ o, int Hq, int Hkv, int D, int ps,
    int max_pages, int pps, int max_splits) {
  __shared__ float wsh[1024];
  const int qh = blockIdx.x % Hq;
  const int bi = blockIdx.x / Hq;
  const int grp = Hq / Hkv;
  const int kvh = qh / grp, qi = qh % grp;
  const int n = min(max(seq_lens[bi], 0), max_pages * ps);
  const int npg = (n + ps - 1) / ps;
  const int nsplit = min((npg + pps - 1) / pps, 1024);
  const long slot0 = (static_cast<long>(bi) * Hkv + kvh) * max_splits;
  const int lane = threadIdx.x;
  float M = kNegInf;
  for (int s = lane; s < nsplit; s += 64) M = fmaxf(M, part_ml[((slot0 + s) * grp + qi) * 2]);
  M = wave_max(M);
  float L = 0.0f;
  for (int s = lane; s < nsplit; s += 64) {
    const float ms = part_ml[((slot0 + s) * grp + qi) * 2];
    const float w = (ms == kNegInf) ? 0.0f : fast_exp2(ms - M);
    wsh[s] = w;
    L += w * part_ml[((slot0 + s) * grp + qi) * 2 + 1];
  }
  L = wave_sum(L);
  __syncthreads();
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  for (int d0 = 2 * lane; d0 < D; d0 += 128) {
    float a0 = 0.f, a1 = 0.f;
    int s = 0;
    for (; s + 4 <= nsplit; s += 4) {
      float2 v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        v[j] = *reinterpret_cast<const float2*>(part_o + ((slot0 + s + j) * grp + qi) * D + d0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        a0 += wsh[s + j] * v[j].x;
        a1 += wsh[s + j] * v[j].y;
      }
    }
    for (; s < nsplit; ++s) {
      const float2 v = *reinterpret_cast<const float2*>(part_o + ((slot0 + s) * grp + qi) * D + d0);
      a0 += wsh[s] * v.x;
      a1 += wsh[s] * v.y;
    }
    *reinterpret_cast<uint32_t*>(o + (static_cast<long>(bi) * Hq + qh) * D + d0) =
        pack_bf16x2(a0 * inv, a1 * inv);
  }
}

constexpr int kDecodePPS = 8;  // pages per split

inline size_t decode_ws_bytes(int b, int Hq, int Hkv, int D, int max_pages) {
  const int max_splits = (max_pages + kDecodePPS - 1) / kDecodePPS;
  const size_t slots = static_cast<size_t>(b) * Hkv * max_splits * (Hq / Hkv);
  return slots * (D + 2) * sizeof(float) + 256;
}

}  // namespace sa

extern "C" size_t sa_paged_decode_workspace_size(int batch, int num_q_heads, int num_kv_heads,
                                                 int head_dim, int max_pages) {
  if (batch < 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads || max_pages < 0) return 0;
  return sa::decode_ws_bytes(batch, num_q_heads, num_kv_heads, head_dim, max_pages);
}

extern "C" int sa_paged_decode_fwd(int dtype, const void* q, const void* k_pages,
                                   const void* v_pages, const int32_t* page_table,
                                   const int32_t* seq_lens, const float* key_bias, int batch,
                                   int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                                   int max_pages, int num_pages, float softmax_scale, void* o,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  SA_CHECK_ARG(dtype == sa::kBF16, "sa_paged_decode_fwd: only bfloat16 is supported");
  SA_CHECK_ARG(batch >= 0 && num_kv_heads > 0 && num_q_heads > 0 &&
                   num_q_heads % num_kv_heads == 0 && num_q_heads / num_kv_heads <= 16,
               "sa_paged_decode_fwd: need Hq %% Hkv == 0 and Hq/Hkv <= 16 (Hq=%d Hkv=%d)",
               num_q_heads, num_kv_heads);
  SA_CHECK_ARG(head_dim == 64 || head_dim == 128, "sa_paged_decode_fwd: head_dim %d not in {64,128}",
               head_dim);
  SA_CHECK_ARG(page_size == 64 || page_size == 128,
               "sa_paged_decode_fwd: page_size %d not in {64, 128}", page_size);
  SA_CHECK_ARG(q && k_pages && v_pages && page_table && seq_lens && o && workspace,
               "sa_paged_decode_fwd: null pointer");
  const size_t need = sa::decode_ws_bytes(batch, num_q_heads, num_kv_heads, head_dim, max_pages);
  SA_CHECK_ARG(workspace_bytes >= need, "sa_paged_decode_fwd: workspace %zu B < %zu B",
               workspace_bytes, need);
  if (batch == 0 || max_pages == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int max_splits = (max_pages + sa::kDecodePPS - 1) / sa::kDecodePPS;
  const int grp = num_q_heads / num_kv_heads;
  float* part_o = static_cast<float*>(workspace);
  float* part_ml = part_o + static_cast<size_t>(batch) * num_kv_heads * max_splits * grp * head_dim;
  const float scale = softmax_scale > 0.f ? softmax_scale : 1.0f / sqrtf(static_cast<float>(head_dim));
  const float sl2 = scale * sa::kLog2e;
  const long items = static_cast<long>(batch) * num_kv_heads * max_splits;
  {
    sa::ProfScope prof_("paged_decode", s);
    if (head_dim == 128)
      hipLaunchKernelGGL(sa::paged_decode_kernel<128>, dim3(items), dim3(64), 0, s,
                         static_cast<const sa::bf16*>(q), static_cast<const sa::bf16*>(k_pages),
                         static_cast<const sa::bf16*>(v_pages), page_table, seq_lens, key_bias,
                         part_o, part_ml, num_q_heads, num_kv_heads, page_size, max_pages,
                         num_pages, sa::kDecodePPS, max_splits, sl2);
    else
      hipLaunchKernelGGL(sa::paged_decode_kernel<64>, dim3(items), dim3(64), 0, s,
                         static_cast<const sa::bf16*>(q), static_cast<const sa::bf16*>(k_pages),
                         static_cast<const sa::bf16*>(v_pages), page_table, seq_lens, key_bias,
                         part_o, part_ml, num_q_heads, num_kv_heads, page_size, max_pages,
                         num_pages, sa::kDecodePPS, max_splits, sl2);
    SA_CHECK_LAUNCH("paged_decode");
  }
  {
    sa::ProfScope prof_("paged_decode_merge", s);
    hipLaunchKernelGGL(sa::paged_decode_merge_kernel, dim3(batch * num_q_heads), dim3(64), 0, s,
                       part_o, part_ml, seq_lens, static_cast<sa::bf16*>(o), num_q_heads,
                       num_kv_heads, head_dim, page_size, max_pages, sa::kDecodePPS, max_splits);
    SA_CHECK_LAUNCH("paged_decode_merge");
  }
  return 0;
}

extern "C" int sa_sparse_attn_fwd(int dtype, const void* q, const void* k, const void* v,
                                  const int32_t* cu_seqlens, int num_seqs,
                                  const int32_t* block_idx, int n_qblk, int max_blocks,
                                  int block_size, const float* key_bias, int total_tokens,
                                  int num_heads, int head_dim, float softmax_scale, void* o,
                                  void* stream) {
  SA_CHECK_ARG(dtype == sa::kBF16, "sa_sparse_attn_fwd: only bfloat16 is supported");
  SA_CHECK_ARG(block_size == 64, "sa_sparse_attn_fwd: block_size must be 64 (got %d)", block_size);
  SA_CHECK_ARG(head_dim == 64 || head_dim == 128, "sa_sparse_attn_fwd: head_dim %d not in {64,128}",
               head_dim);
  SA_CHECK_ARG(num_seqs >= 0 && n_qblk >= 0 && max_blocks >= 0 && num_heads > 0 &&
                   total_tokens >= 0,
               "sa_sparse_attn_fwd: bad sizes");
  SA_CHECK_ARG(q && k && v && cu_seqlens && o && (block_idx || n_qblk == 0),
               "sa_sparse_attn_fwd: null pointer");
  if (n_qblk == 0 || num_seqs == 0 || total_tokens == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const float scale = softmax_scale > 0.f ? softmax_scale : 1.0f / sqrtf(static_cast<float>(head_dim));
  const long blocks = static_cast<long>(num_heads) * n_qblk;
  sa::ProfScope prof_("sparse_attn_fwd", s);
  if (head_dim == 128)
    hipLaunchKernelGGL(sa::sparse_attn_fwd_kernel<128>, dim3(blocks), dim3(256), 0, s,
                       static_cast<const sa::bf16*>(q), static_cast<const sa::bf16*>(k),
                       static_cast<const sa::bf16*>(v), cu_seqlens, num_seqs, block_idx, n_qblk,
                       max_blocks, key_bias, static_cast<sa::bf16*>(o), total_tokens, num_heads,
                       scale * sa::kLog2e);
  else
    hipLaunchKernelGGL(sa::sparse_attn_fwd_kernel<64>, dim3(blocks), dim3(256), 0, s,
                       static_cast<const sa::bf16*>(q), static_cast<const sa::bf16*>(k),
                       static_cast<const sa::bf16*>(v), cu_seqlens, num_seqs, block_idx, n_qblk,
                       max_blocks, key_bias, static_cast<sa::bf16*>(o), total_tokens, num_heads,
                       scale * sa::kLog2e);
  SA_CHECK_LAUNCH("sparse_attn_fwd");
  return 0;
}
