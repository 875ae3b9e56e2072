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
#include "decode.h"

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

// ---------------------------------------------------------------------------
// block-sparse varlen prefill.  One workgroup per (head, 64-query block),
// four waves: wave w owns query rows 32 (w & 1) .. +31 and, of every selected
// 64-key block, keys 32 (w >> 1) .. +31.  Each K or V^T fragment read from
// LDS feeds two MFMAs (two 16-query tiles).  The two key halves run
// independent online softmaxes and are merged through LDS at the end.
//
// K and V tiles (and the block's key biases) go from HBM straight into LDS
// (global_load_lds, 16 bytes per lane) in two stages: the next selected block
// streams in while the current one is computed, with no staging registers
// and one barrier per block.  The tiles are unpadded
// ([key][D] bf16) with the 16-byte chunks of row r permuted (k_swz, v_swz),
// so the K fragment reads (16 rows, one chunk) and the V^T transpose reads
// (ds_read_b64_tr_b16: 8 rows, a chunk pair) hit distinct LDS banks.
// ---------------------------------------------------------------------------
template <int D>
struct SparseSmem {
  static constexpr int tile = 64 * D;               // bf16 per K or V tile
  static constexpr int stage = 2 * tile + 128;      // bf16: K, V, the 64 fp32 key biases
};

// chunk permutations of row r (16-byte chunks; D = 128: 16 per row, D = 64:
// 8).  The K tile is read as MFMA A fragments (16 rows key_of_row(kt, 0..15),
// one chunk per 16-lane group), the V tile by ds_read_b64_tr_b16 (rows
// 8g + 0..3 and + 4, one chunk pair per group), so each gets its own
// permutation; both were chosen with the LDS bank-conflict counter
// (SQ_LDS_BANK_CONFLICT = 0 for these read sets on gfx950).  The V
// permutation never uses bit 2 of r, so rows r and r + 4 (the two halves of
// one transpose read) share it.
template <int D>
__device__ __forceinline__ int k_swz(int r) {
  if constexpr (D == 128) return (r & 3) | (((r >> 3) & 3) << 2);
  else return (((r >> 1) & 1) << 2) | (((r >> 3) & 1) << 1) | ((r >> 4) & 1);
}
template <int D>
__device__ __forceinline__ int v_swz(int r) {
  if constexpr (D == 128) return ((r & 3) << 2) | (((r >> 3) & 1) << 1) | ((r >> 4) & 1);
  else return (((r >> 1) & 1) << 2) | (((r >> 3) & 1) << 1) | ((r >> 4) & 1);
}

// p[i] for a wave-uniform i through the constant address space: a scalar
// load, counted by lgkmcnt rather than the vector memory counter
__device__ __forceinline__ int32_t load_uniform(const int32_t* p, int i) {
  typedef const __attribute__((address_space(4))) int32_t cint;
  return ((cint*)p)[__builtin_amdgcn_readfirstlane(i)];
}

// Online softmax with a lazy reference.  s[kt][i] holds log2-domain scores of
// this lane's keys for query column lane & 15 (-inf where masked).  The
// running reference m of a column (log2 domain, shared by its
// four lane groups) is raised, and O and the partial sums rescaled, only when
// some score exceeds it by more than 2^8: the common block needs no cross-lane
// reduction at all, and probabilities stay <= 256.  l is this lane's partial
// row sum (its own keys); the four lane groups' parts are added at the end.
// The scores may come unscaled: the log2-domain score is s * sc (sc > 0), and
// the scale is folded into the exponent's argument.
template <int KT, int DT>
__device__ __forceinline__ void softmax_lazy(v4f (&s)[KT], v4f (&o)[DT], float& m, float& l,
                                             float sc = 1.0f) {
  float mx = kNegInf;
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[kt][i]);
  mx *= sc;
  if (__ballot(mx > m + 8.0f)) {
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    if (mx > m + 8.0f) {   // the column's new reference
      if (m != kNegInf) {   // (while m = -inf, every p so far was 0: l and o are 0)
        const float alpha = fast_exp2(m - mx);
        l *= alpha;
#pragma unroll
        for (int t = 0; t < DT; ++t) o[t] *= alpha;
      }
      m = mx;
    }
  }
  // masked scores are -inf; a column without any admissible key yet keeps
  // m = -inf and only -inf scores, so a zero reference gives p = 0 there
  const float mref = m == kNegInf ? 0.0f : m;
  float sum = 0.0f;
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = fast_exp2(fmaf(s[kt][i], sc, -mref));
      s[kt][i] = p;
      sum += p;
    }
  l += sum;
}

// MODE (which keys a query sees, and which key is exempt from the bias):
//   kCausalSelf  keys j <= i of the query's own sequence; j = i exempt
//   kFullSelf    every key of the query's own sequence;  j = i exempt
//   kCross       every key of the sequence's key range cu_k[s]..cu_k[s+1]
//                (k, v, key_bias indexed by key token); key 0 exempt
// SEL (how the key blocks are chosen, fixed per launch):
//   kSelDense    every key block the mode admits (no table)
//   kSelShort    a block_idx row of at most 64 slots, held one slot per lane
//   kSelLong     a longer row, read slot by slot with scalar loads
constexpr int kCausalSelf = 0, kFullSelf = 1, kCross = 2;
constexpr int kSelDense = 0, kSelShort = 1, kSelLong = 2;

// Workgroups per CU the register budget is set for: at D = 64 a workgroup
// holds 33 KB of LDS, so four fit (dense self-attention fits 128 VGPRs; the
// table walks and the cross mode would spill there and take three); at
// D = 128 (66 KB) two.
template <int D, int MODE, int SEL>
constexpr int attn_blocks_per_cu() {
  return D == 64 ? (SEL == kSelDense && MODE != kCross ? 4 : 3) : 2;
}

template <int D, bool BIAS, int MODE, int SEL>
__global__ __launch_bounds__(256, (attn_blocks_per_cu<D, MODE, SEL>())) void sparse_attn_fwd_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const int32_t* __restrict__ cu, const int32_t* __restrict__ cu_k, int nseq,
    const int32_t* __restrict__ block_idx, int n_qblk, int max_blocks, int grid_qblk,
    const float* __restrict__ key_bias, bf16* __restrict__ o, int T, int Tk, int H,
    float scale_log2) {
  constexpr int BS = 64;
  using SM = SparseSmem<D>;
  constexpr int DT = D / 16, KS = D / 32;
  constexpr int IPW = D / 32;   // 1 KB DMA instructions per wave per tile (tile = 128 D bytes)
  // two stages as separate LDS objects; they also hold the final merge
  __shared__ __align__(16) bf16 stage0[SM::stage];
  __shared__ __align__(16) bf16 stage1[SM::stage];

  const int lid = xcd_swizzle(blockIdx.x, gridDim.x);
  // grid_qblk >= the query blocks of the packing: surplus ids find no sequence
  // and exit; a query block past the rows of block_idx has no selection
  const int h = lid / grid_qblk;
  // a head's query blocks from the last to the first: in causal modes a
  // block's work grows with its position in the sequence, so the longest
  // go first and each launch round ends on short ones
  const int gq = grid_qblk - 1 - (lid - h * grid_qblk);
  const int tid = threadIdx.x, lane = tid & 63;
  // locate the query block's sequence (q blocks are numbered sequence by
  // sequence): 64 sequences per step, one per lane, a prefix sum of their
  // block counts and a ballot for the one holding block gq
  int start = 0, n = 0, jq = -1, seq = 0;
  for (int s0 = 0, first = 0; s0 < nseq && jq < 0; s0 += 64) {
    const int si = s0 + lane;
    int a = 0, nb = 0, len = 0;
    if (si < nseq) {
      a = min(max(cu[si], 0), T);
      len = min(max(cu[si + 1], a), T) - a;
      nb = (len + BS - 1) / BS;
    }
    int incl = nb;
#pragma unroll
    for (int o2 = 1; o2 < 64; o2 <<= 1) {
      const int t = __shfl_up(incl, o2, 64);
      if (lane >= o2) incl += t;
    }
    const int excl = first + incl - nb;
    const uint64_t hit = __ballot(si < nseq && gq >= excl && gq < excl + nb);
    if (hit) {
      const int L = __builtin_ctzll(hit);
      start = __builtin_amdgcn_readlane(a, L);
      n = __builtin_amdgcn_readlane(len, L);
      jq = gq - __builtin_amdgcn_readlane(excl, L);
      seq = s0 + L;
    }
    first += __builtin_amdgcn_readlane(incl, 63);
  }
  if (jq < 0) return;  // more query blocks than the packing holds
  // the key range: the query's own sequence, or its key sequence for kCross
  int kstart = start, nks = n;
  if constexpr (MODE == kCross) {
    kstart = min(max(cu_k[seq], 0), Tk);
    nks = min(max(cu_k[seq + 1], kstart), Tk) - kstart;
  }
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qh = w & 1, kh = w >> 1;
  const int c = lane & 15, g = lane >> 4;
  const long rs = static_cast<long>(H) * D;
  const bf16* kbase = k + static_cast<long>(kstart) * rs + static_cast<long>(h) * D;
  const bf16* vbase = v + static_cast<long>(kstart) * rs + static_cast<long>(h) * D;

  // this lane's two query columns (16-query tiles jt = 0, 1 of the wave's 32 rows)
  int qloc[2];
  v8bf qf[2][KS];
#pragma unroll
  for (int jt = 0; jt < 2; ++jt) {
    qloc[jt] = jq * BS + 32 * qh + 16 * jt + c;
    const bf16* qrow = q + (start + static_cast<long>(min(qloc[jt], n - 1))) * rs + static_cast<long>(h) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[jt][ks] = qloc[jt] < n ? load_v8bf(qrow + 32 * ks + 8 * g) : zero_v8bf();
  }
  const float* bias = BIAS ? key_bias + static_cast<long>(h) * Tk + kstart : nullptr;
  // the whole query block is inside the sequence: only the diagonal block needs masks
  const bool qfull = (jq + 1) * BS <= n;

  // the selected blocks that are inside the key range (and causally visible
  // for kCausalSelf), in order; dense: slots are the blocks themselves
  // A block id repeated within a row is attended once, at its first slot:
  // the selection is a set of key blocks.
  constexpr bool dense = SEL == kSelDense;
  const bool has_row = dense || (gq < n_qblk && max_blocks > 0);
  const int nkb = (nks + BS - 1) / BS;
  const int nslot = dense ? (MODE == kCausalSelf ? min(jq + 1, nkb) : nkb) : (has_row ? max_blocks : 0);
  const int32_t* sel = has_row && !dense ? block_idx + (static_cast<long>(h) * n_qblk + gq) * max_blocks : nullptr;
  constexpr bool simple = SEL == kSelShort;
  int my_kb = -1;
  uint64_t vmask = 0;
  if (simple && has_row) {
    my_kb = lane < max_blocks ? sel[lane] : -1;
    bool ok = my_kb >= 0 && my_kb < nkb && (MODE != kCausalSelf || my_kb <= jq);
    for (int j = 0; j + 1 < max_blocks; ++j) {
      const int kj = __builtin_amdgcn_readlane(my_kb, j);
      ok = ok && !(lane > j && my_kb == kj);
    }
    vmask = __ballot(ok);
  }
  // (wave-uniform slot indices: the general path's table reads are scalar
  // loads, which do not count against the vector memory counter the DMA
  // pipeline waits on)
  auto next_valid = [&](int e) -> int {   // first valid slot >= e, or nslot
    if (dense) return min(e, nslot);
    if (simple) {
      const uint64_t mm = e >= 64 ? 0ull : (vmask >> e);
      return mm ? e + __builtin_ctzll(mm) : nslot;
    }
    for (e = __builtin_amdgcn_readfirstlane(e); e < nslot; ++e) {
      const int kb = load_uniform(sel, e);
      if (kb >= 0 && kb < nkb && (MODE != kCausalSelf || kb <= jq)) {
        bool dup = false;
        for (int j = 0; j < e && !dup; ++j) dup = load_uniform(sel, j) == kb;
        if (!dup) return e;
      }
    }
    return nslot;
  };
  auto block_of = [&](int e) -> int {
    return dense ? e : simple ? __builtin_amdgcn_readlane(my_kb, e) : load_uniform(sel, e);
  };

  // DMA of block kb into a stage: lane l of this wave's instruction i fills
  // tile bytes 1024 (IPW w + i) + 16 l, i.e. row `row`, stored chunk `ch`,
  // which holds logical chunk ch ^ k_swz(row) (K) or ch ^ v_swz(row) (V).  Rows past the sequence
  // repeat its last key (their scores are masked to -inf, so p = 0).
  // full blocks use per-lane element offsets computed once (32-bit, added to
  // the block's wave-uniform base); the last, partial block of a sequence
  // clamps its rows
  int dma_k[IPW], dma_v[IPW];
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    const int pos = ((w * IPW + i) << 10) + (lane << 4);
    const int row = pos / (2 * D), ch = (pos % (2 * D)) >> 4;
    dma_k[i] = row * static_cast<int>(rs) + 8 * (ch ^ k_swz<D>(row));
    dma_v[i] = row * static_cast<int>(rs) + 8 * (ch ^ v_swz<D>(row));
  }
  // LDS byte addresses of this wave's DMA destinations in stage 0 (stage 1
  // is SM::stage * 2 bytes further on): K and V chunks 1 KB apart, the biases
  const uint32_t lds_st0 = lds_addr(stage0), lds_st1 = lds_addr(stage1);
  const uint32_t lds_wave = static_cast<uint32_t>(w * IPW) << 10;
  auto issue_kv = [&](int kb, uint32_t st) __attribute__((always_inline)) {
    const int k0 = kb * BS, nk = min(BS, nks - k0);
    const uint32_t kt = st + lds_wave, vt = kt + 2 * SM::tile;
    const bf16* kb0 = kbase + static_cast<long>(k0) * rs;
    const bf16* vb0 = vbase + static_cast<long>(k0) * rs;
    if constexpr (BIAS) {   // the block's key biases (rows past the sequence repeat the last)
      if (w == 0) dma_lds4(bias, 4u * min(k0 + lane, nks - 1), st + 4 * SM::tile);
    }
    if (nk == BS) {
#pragma unroll
      for (int i = 0; i < IPW; ++i) {
        dma_lds16(kb0, 2u * dma_k[i], kt + (i << 10));
        dma_lds16(vb0, 2u * dma_v[i], vt + (i << 10));
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      const int pos = ((w * IPW + i) << 10) + (lane << 4);
      const int row = pos / (2 * D);
      const int rr = min(row, nk - 1);
      const int ch = (pos % (2 * D)) >> 4;
      const int koff = rr * static_cast<int>(rs) + 8 * (ch ^ k_swz<D>(row));
      const int voff = rr * static_cast<int>(rs) + 8 * (ch ^ v_swz<D>(row));
      dma_lds16(kb0, 2u * koff, kt + (i << 10));
      dma_lds16(vb0, 2u * voff, vt + (i << 10));
    }
  };

  float m[2] = {kNegInf, kNegInf}, l[2] = {0.f, 0.f};
  v4f acc[2][DT];
#pragma unroll
  for (int jt = 0; jt < 2; ++jt)
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[jt][t] = v4f{0.f, 0.f, 0.f, 0.f};

  // per-lane pieces of the swizzled LDS addresses
  int krow_off[2], kswz[2];
#pragma unroll
  for (int u2 = 0; u2 < 2; ++u2) {
    const int r = key_of_row(2 * kh + u2, c);
    krow_off[u2] = r * D;
    kswz[u2] = k_swz<D>(r);
  }
  const int vr = 32 * kh + 8 * g + ((lane & 15) >> 2);   // V^T read rows vr and vr + 4
  const int vswz = v_swz<D>(vr);
  const int vhalf = 4 * ((lane & 15) & 1);               // element offset inside the chunk
  const int vchunk = ((lane & 15) & 3) >> 1;              // chunk of the pair

  // Pipeline: the tiles of block e + 1 land in one stage while block e is
  // computed from the other.  The loop is unrolled by two so that each stage
  // is a fixed LDS object.
  int e = 0, en = 0;
  // one key block: computed from stage cur while the next block's tiles land in nxt
  auto step = [&](bf16* cur, uint32_t nxt_lds) __attribute__((always_inline)) {
    const int kb = block_of(e);
    const int enn = en < nslot ? next_valid(en + 1) : nslot;   // the block after next
    const int k0 = kb * BS;
    const int nk = min(BS, nks - k0);
    // one barrier per block: this block's tiles have landed and are visible,
    // and every wave is done with the previous block, whose stage the next
    // block's DMA refills
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(vm_wait<0>());
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (en < nslot) issue_kv(block_of(en), nxt_lds);
    const bf16* Ks = cur;
    const bf16* Vs = Ks + SM::tile;
    // bias of the wave's keys 32 kh + 8g + 0..7
    float bk[8];
    if constexpr (BIAS) {
      const float* bs = reinterpret_cast<const float*>(Vs + SM::tile) + 32 * kh + 8 * g;
      const float4 b0 = *reinterpret_cast<const float4*>(bs);
      const float4 b1 = *reinterpret_cast<const float4*>(bs + 4);
      bk[0] = b0.x; bk[1] = b0.y; bk[2] = b0.z; bk[3] = b0.w;
      bk[4] = b1.x; bk[5] = b1.y; bk[6] = b1.z; bk[7] = b1.w;
    }

    // S^T = K . Q^T for the wave's 32 keys (score tiles kt = 2 kh, 2 kh + 1)
    v4f sc[2][2];
#pragma unroll
    for (int jt = 0; jt < 2; ++jt)
#pragma unroll
      for (int u2 = 0; u2 < 2; ++u2) sc[jt][u2] = v4f{0.f, 0.f, 0.f, 0.f};
    v8bf kfr[2][KS];   // every K fragment read before the first MFMA
#pragma unroll
    for (int u2 = 0; u2 < 2; ++u2)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kfr[u2][ks] = load_v8bf(Ks + krow_off[u2] + 8 * ((4 * ks + g) ^ kswz[u2]));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int u2 = 0; u2 < 2; ++u2)
#pragma unroll
        for (int jt = 0; jt < 2; ++jt) sc[jt][u2] = mfma_bf16(kfr[u2][ks], qf[jt][ks], sc[jt][u2]);
    // scale; bias (not on the exempt key) and causal / length masks where needed.
    // Interior blocks (no mask, no exempt key): for kCausalSelf the blocks
    // before the diagonal; otherwise full key blocks other than the one
    // holding the exempt key (the diagonal block, or block 0 for kCross)
    const bool interior = MODE == kCausalSelf
                              ? (kb < jq && qfull)
                              : (qfull && k0 + BS <= nks && kb != (MODE == kCross ? 0 : jq));
    // interior blocks without a bias keep raw scores (the scale goes into the
    // exponent); otherwise scale, bias and masks are applied in place.  The
    // block-uniform test is made once: tested per element inside the unrolled
    // loops it became a branch per score.
    float scl = scale_log2;
    if (!interior) {
      scl = 1.0f;
#pragma unroll
      for (int jt = 0; jt < 2; ++jt)
#pragma unroll
        for (int u2 = 0; u2 < 2; ++u2)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int kl = key_of_row(2 * kh + u2, 4 * g + i);   // = 32 kh + 8g + 4 u2 + i
            const int key = k0 + kl;
            float val = sc[jt][u2][i] * scale_log2;
            const bool exempt = MODE == kCross ? key == 0 : key == qloc[jt];
            if constexpr (BIAS) val += exempt ? 0.f : bk[4 * u2 + i] * kLog2e;
            val = (kl < nk && (MODE != kCausalSelf || key <= qloc[jt]) && qloc[jt] < n) ? val : kNegInf;
            sc[jt][u2][i] = val;
          }
    } else if constexpr (BIAS) {   // no mask and no exempt key: scale and bias only
      scl = 1.0f;
      float bl[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) bl[j] = bk[j] * kLog2e;
#pragma unroll
      for (int jt = 0; jt < 2; ++jt)
#pragma unroll
        for (int u2 = 0; u2 < 2; ++u2)
#pragma unroll
          for (int i = 0; i < 4; ++i) sc[jt][u2][i] = fmaf(sc[jt][u2][i], scale_log2, bl[4 * u2 + i]);
    }
    // the V^T fragments of the wave's 32 keys, read before the softmax so
    // that their LDS latency passes under its VALU work
    v8bf vfr[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
      const bf16* p = Vs + vr * D + 8 * ((2 * t + vchunk) ^ vswz) + vhalf;
      const v4i16 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p));
      const v4i16 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p + 4 * D));
      vfr[t] = __builtin_bit_cast(v8bf, __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int jt = 0; jt < 2; ++jt) softmax_lazy<2, DT>(sc[jt], acc[jt], m[jt], l[jt], scl);
    // O^T += V^T . P^T over the wave's 32 keys
    {
      const v8bf pb0 = pack_p(sc[0][0], sc[0][1]);
      const v8bf pb1 = pack_p(sc[1][0], sc[1][1]);
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        acc[0][t] = mfma_bf16(vfr[t], pb0, acc[0][t]);
        acc[1][t] = mfma_bf16(vfr[t], pb1, acc[1][t]);
      }
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(kLgkmWait0);
    e = en;
    en = enn;
  };
  e = next_valid(0);
  en = e < nslot ? next_valid(e + 1) : nslot;
  // the query fragments (and the selection row) have arrived before the loop:
  // nothing the compiler tracks is in flight inside it
  __builtin_amdgcn_s_waitcnt(vm_wait<0>());
  if (e < nslot) issue_kv(block_of(e), lds_st0);
  while (e < nslot) {
    step(stage0, lds_st1);
    if (e >= nslot) break;
    step(stage1, lds_st0);
  }
  // every wave is done with the tiles before the merge reuses the LDS
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // the row sums so far are per lane (its own keys): add the four lane groups
#pragma unroll
  for (int jt = 0; jt < 2; ++jt) {
    l[jt] += __shfl_xor(l[jt], 16, 64);
    l[jt] += __shfl_xor(l[jt], 32, 64);
  }
  // merge the two key halves: waves kh = 1 hand (m, l, O^T) to waves kh = 0
  // [qh][2 jt][DT][64 lanes] float4 in stage 0, [qh][2 jt][m, l][64 lanes] in stage 1
  float4* xo = reinterpret_cast<float4*>(stage0) + qh * 2 * DT * 64;
  float* xm = reinterpret_cast<float*>(stage1) + qh * 2 * 2 * 64;
  static_assert(2 * 2 * DT * 64 * 16 <= SM::stage * 2, "merge fits stage 0");
  if (kh == 1) {
#pragma unroll
    for (int jt = 0; jt < 2; ++jt) {
#pragma unroll
      for (int t = 0; t < DT; ++t)
        xo[(jt * DT + t) * 64 + lane] = make_float4(acc[jt][t][0], acc[jt][t][1], acc[jt][t][2], acc[jt][t][3]);
      xm[(jt * 2) * 64 + lane] = m[jt];
      xm[(jt * 2 + 1) * 64 + lane] = l[jt];
    }
  }
  __syncthreads();
  if (kh == 1) return;
  // the wave's 32 merged rows, normalised, go out through LDS as whole rows
  // (16 bytes per lane): [32 rows][D] bf16 in stage 1 past the m / l
  // exchange, 16-byte chunk c of row r at c ^ (r % RCH)
  constexpr int RCH = D / 8;
  static_assert(1024 + 2 * 32 * D <= SM::stage, "output rows fit stage 1");
  bf16* ot = stage1 + 1024 + qh * 32 * D;
#pragma unroll
  for (int jt = 0; jt < 2; ++jt) {
    const float m1 = xm[(jt * 2) * 64 + lane], l1 = xm[(jt * 2 + 1) * 64 + lane];
    const float mm = fmaxf(m[jt], m1);
    const float a0 = m[jt] == kNegInf ? 0.f : fast_exp2(m[jt] - mm);
    const float a1 = m1 == kNegInf ? 0.f : fast_exp2(m1 - mm);
    const float lt = l[jt] * a0 + l1 * a1;
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    const float b0 = a0 * inv, b1 = a1 * inv;
    const int r = 16 * jt + c;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      const float4 o1 = xo[(jt * DT + t) * 64 + lane];
      const float r0 = fmaf(acc[jt][t][0], b0, o1.x * b1), r1 = fmaf(acc[jt][t][1], b0, o1.y * b1);
      const float r2 = fmaf(acc[jt][t][2], b0, o1.z * b1), r3 = fmaf(acc[jt][t][3], b0, o1.w * b1);
      const int ch = 2 * t + (g >> 1);
      *reinterpret_cast<uint2*>(ot + r * D + 8 * (ch ^ (r & (RCH - 1))) + 4 * (g & 1)) =
          uint2{pack_bf16x2(r0, r1), pack_bf16x2(r2, r3)};
    }
  }
  const int q0 = jq * BS + 32 * qh;
  bf16* obase = o + (start + static_cast<long>(q0)) * rs + static_cast<long>(h) * D;
#pragma unroll
  for (int i = 0; i < RCH / 2; ++i) {
    const int e = lane + 64 * i, r = e / RCH, ch = e % RCH;
    if (q0 + r < n)
      *reinterpret_cast<uint4*>(obase + r * rs + 8 * ch) =
          *reinterpret_cast<const uint4*>(ot + r * D + 8 * (ch ^ (r & (RCH - 1))));
  }
}

template <int D, bool BIAS, int MODE>
int launch_sparse(const void* q, const void* k, const void* v, const int32_t* cu,
                  const int32_t* cu_k, int nseq, const int32_t* block_idx, int n_qblk,
                  int max_blocks, int grid_qblk, int dense_all, const float* key_bias, void* o, int T,
                  int Tk, int H, float scale_log2, hipStream_t s) {
  const long blocks = static_cast<long>(H) * grid_qblk;
  ProfScope prof_(MODE == kCausalSelf ? "sparse_attn_fwd" : MODE == kFullSelf ? "attn_full_fwd" : "attn_cross_fwd", s);
#define SA_SPARSE_LAUNCH(SEL)                                                                     \
  hipLaunchKernelGGL((sparse_attn_fwd_kernel<D, BIAS, MODE, SEL>), dim3(blocks), dim3(256), 0, s, \
                     static_cast<const bf16*>(q), static_cast<const bf16*>(k),                    \
                     static_cast<const bf16*>(v), cu, cu_k, nseq, block_idx, n_qblk, max_blocks,  \
                     grid_qblk, key_bias, static_cast<bf16*>(o), T, Tk, H, scale_log2)
  if (dense_all) SA_SPARSE_LAUNCH(kSelDense);
  else if (max_blocks <= 64) SA_SPARSE_LAUNCH(kSelShort);
  else SA_SPARSE_LAUNCH(kSelLong);
#undef SA_SPARSE_LAUNCH
  return 0;
}

template <int D, int MODE>
int launch_attn_d(const void* q, const void* k, const void* v, const int32_t* cu,
                  const int32_t* cu_k, int nseq, const int32_t* block_idx, int n_qblk,
                  int max_blocks, int grid_qblk, int dense_all, const float* key_bias, void* o,
                  int T, int Tk, int H, float scale_log2, hipStream_t s) {
  return key_bias ? launch_sparse<D, true, MODE>(q, k, v, cu, cu_k, nseq, block_idx, n_qblk, max_blocks,
                                                 grid_qblk, dense_all, key_bias, o, T, Tk, H, scale_log2, s)
                  : launch_sparse<D, false, MODE>(q, k, v, cu, cu_k, nseq, block_idx, n_qblk,
                                                  max_blocks, grid_qblk, dense_all, key_bias, o, T, Tk,
                                                  H, scale_log2, s);
}

// grid_qblk: query blocks per head in the grid, at least the packing's
// sum over sequences of ceil(len / 64) (total_q / 64 + nseq bounds it);
// dense_all: every admissible key block, no table
int launch_attn(int mode, int D, const void* q, const void* k, const void* v, const int32_t* cu,
                const int32_t* cu_k, int nseq, const int32_t* block_idx, int n_qblk, int max_blocks,
                int grid_qblk, int dense_all, const float* key_bias, void* o, int T, int Tk, int H,
                float scale_log2, hipStream_t s) {
#define SA_ATTN_ARGS q, k, v, cu, cu_k, nseq, block_idx, n_qblk, max_blocks, grid_qblk, dense_all, key_bias, o, T, Tk, H, scale_log2, s
  if (D == 128) {
    if (mode == kCausalSelf) return launch_attn_d<128, kCausalSelf>(SA_ATTN_ARGS);
    if (mode == kFullSelf) return launch_attn_d<128, kFullSelf>(SA_ATTN_ARGS);
    return launch_attn_d<128, kCross>(SA_ATTN_ARGS);
  }
  if (mode == kCausalSelf) return launch_attn_d<64, kCausalSelf>(SA_ATTN_ARGS);
  if (mode == kFullSelf) return launch_attn_d<64, kFullSelf>(SA_ATTN_ARGS);
  return launch_attn_d<64, kCross>(SA_ATTN_ARGS);
#undef SA_ATTN_ARGS
}

// ---------------------------------------------------------------------------
// paged GQA decode, stream-K over 64-key tiles.  The work is the global list
// of tiles in (batch row, kv head, tile) order; a plan kernel prefix-sums the
// tiles per row, and the decode kernel runs one resident round of W waves,
// wave w taking tiles [floor(wT/W), floor((w+1)T/W)).  Every wave streams the
// same number of tiles whatever the spread of sequence lengths, so no wave
// slot idles while a long split finishes.  A wave writes one partial
// (unnormalised O^T, running max and sum) for each (row, kv head) it touches,
// under segment id  row * Hkv + kv head + w:  ids grow along the tile order,
// so the segments of one (row, kv head) are consecutive and the merge kernel
// reads them as one contiguous run.
//
// Inside a wave the query heads of the group sit in the first lanes of each
// 16-lane column group (columns >= group size are padding).  No LDS: K rows
// and V^T rows go from HBM straight into MFMA operands.  The K and V halves
// of consecutive tiles are software-pipelined through one register buffer
// each: K of tile t+1 is in flight while tile t's softmax and V^T.P^T run, V
// of tile t+1 while tile t+1's K.Q^T runs, so the wave always has HBM reads
// outstanding.  Page ids are fetched 64 at a time, one per lane, and
// broadcast with readlane.
// ---------------------------------------------------------------------------
template <bool B>
struct BoolC {
  static constexpr bool value = B;
};

struct DecodeSlot {
  long kidx;  // index of the tile's first key in the (page, kv head, key) pool
  int nk;     // valid keys of the tile (0: invalid page id)
  int pos0;   // sequence position of the tile's first key
  int k0;     // offset of the tile inside its page
};

// K rows of a 64-key tile as A operands of S^T = K.Q^T: lane (c, g) reads key
// key_of_row(kt, c), dims 32ks + 8g .. +7
template <int D>
__device__ __forceinline__ void decode_load_k(v8bf (&kf)[4][D / 32], const bf16* __restrict__ kt0,
                                              int c, int g) {
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks)
      kf[kt][ks] = load_v8bf(kt0 + static_cast<unsigned>(key_of_row(kt, c) * D + 32 * ks + 8 * g));
}

// V^T rows of a 64-key tile as A operands of O^T += V^T.P^T: lane (c, g)
// reads dim 16t + c, keys 32ks + 8g .. +7 (a 16-byte run of the page's V^T row)
// (voff = 2 (c * ps + 8g) bytes, per lane; the row step 32 * ps bytes is
// wave-uniform and goes into the scalar offset)
template <int D>
__device__ __forceinline__ void decode_load_v(v8bf (&vf)[2][D / 16], const bf16* __restrict__ vt0,
                                              int ps, unsigned voff) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(vt0);
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int t = 0; t < D / 16; ++t)
      vf[ks][t] = buf_load_v8bf(r, voff, static_cast<unsigned>(32 * t * ps + 64 * ks));
}

// tiles of row r: ceil(clamp(seq_lens[r], 0, max_pages * ps) / 64)
__device__ __forceinline__ int decode_row_len(const int32_t* seq_lens, int r, int max_pages, int ps) {
  return min(max(seq_lens[r], 0), max_pages * ps);
}

// cum_row[r] = 64-key tiles of rows < r (per kv head), r = 0..b.  One block.
__global__ __launch_bounds__(1024) void paged_decode_plan_kernel(
    const int32_t* __restrict__ seq_lens, int b, int ps, int max_pages,
    int32_t* __restrict__ cum_row) {
  __shared__ int wtot[16];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  int carry = 0;
  if (tid == 0) cum_row[0] = 0;
  for (int base = 0; base < b; base += 1024) {
    const int r = base + tid;
    int v = r < b ? (decode_row_len(seq_lens, r, max_pages, ps) + 63) >> 6 : 0;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(v, o, 64);
      if (lane >= o) v += t;
    }
    if (lane == 63) wtot[wid] = v;
    __syncthreads();
    int pre = carry, tot = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      pre += j < wid ? wtot[j] : 0;
      tot += wtot[j];
    }
    if (r < b) cum_row[r + 1] = pre + v;
    carry += tot;
    __syncthreads();  // wtot is rewritten by the next chunk
  }
}

// first tile of wave w and the wave that holds tile g (W waves, T tiles)
__device__ __forceinline__ long decode_wave_begin(int w, long T, int W) {
  return static_cast<long>(w) * T / W;
}
__device__ __forceinline__ int decode_wave_of(long g, long T, int W) {
  return static_cast<int>(((g + 1) * W + T - 1) / T - 1);
}

template <int D, bool BIAS>
__global__ __launch_bounds__(64, 2) void paged_decode_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ kp, const bf16* __restrict__ vp,
    const int32_t* __restrict__ page_table, const int32_t* __restrict__ seq_lens,
    const float* __restrict__ key_bias, int32_t* __restrict__ cum_row,
    float* __restrict__ part_o, float* __restrict__ part_ml, int b, int Hq, int Hkv, int ps,
    int max_pages, int num_pages, int W, float scale_log2) {
  constexpr int DT = D / 16, KS = D / 32;
  const int w = blockIdx.x;
  const int lane = threadIdx.x, c = lane & 15, g = lane >> 4;
  // b <= 64: every wave forms the row plan itself, lane r holding row r's
  // 64-key tiles and the tiles of the rows before it (cum_row[r]); wave 0
  // stores cum_row for the merge.  Larger batches read the plan kernel's.
  const bool lane_plan = b <= 64;
  int ex_l = 0, tot = 0;
  if (lane_plan) {
    const int nb = lane < b ? (decode_row_len(seq_lens, lane, max_pages, ps) + 63) >> 6 : 0;
    int incl = nb;
#pragma unroll
    for (int o2 = 1; o2 < 64; o2 <<= 1) {
      const int t = __shfl_up(incl, o2, 64);
      if (lane >= o2) incl += t;
    }
    ex_l = incl - nb;
    tot = __builtin_amdgcn_readlane(incl, 63);
    if (w == 0 && lane < b) {
      cum_row[lane + 1] = incl;
      if (lane == 0) cum_row[0] = 0;
    }
  }
  // cum_row[r] for a wave-uniform r in [0, b]
  auto crow = [&](int r) -> int {
    return lane_plan ? (r < 64 ? __builtin_amdgcn_readlane(ex_l, r) : tot) : cum_row[r];
  };
  const long T = static_cast<long>(Hkv) * crow(b);
  // with at most T waves every wave gets at least one tile, which keeps the
  // segment ids of one (row, kv head) consecutive
  W = static_cast<int>(min(static_cast<long>(W), T));
  if (w >= W) return;
  long gt = decode_wave_begin(w, T, W);
  const long gt_end = decode_wave_begin(w + 1, T, W);
  const int grp = Hq / Hkv;
  const int pshift = ps == 128 ? 7 : 6;  // page size 64 or 128
  const int tshift = pshift - 6;         // log2(64-key tiles per page)
  const unsigned voff = static_cast<unsigned>(2 * (c * ps + 8 * g));

  // row of the first tile: the largest r with Hkv * cum_row[r] <= gt, by a
  // 64-ary search (cum_row is non-decreasing; invariant: answer in [lo, lo + span))
  int bi = 0;
  if (lane_plan) {   // cum_row is non-decreasing in the lane: a prefix of lanes qualifies
    bi = __popcll(__ballot(lane < b && static_cast<long>(Hkv) * ex_l <= gt)) - 1;
  } else {
    int lo = 0, span = b;
    while (span > 1) {
      const int step = (span + 63) >> 6;
      const int r = lo + lane * step;
      const bool le = r < lo + span && static_cast<long>(Hkv) * cum_row[r] <= gt;
      const int k = __popcll(__ballot(le));  // >= 1: lane 0 reads cum_row[lo]
      const int nlo = lo + (k - 1) * step;
      span = min(step, lo + span - nlo);
      lo = nlo;
    }
    bi = lo;
  }

  while (gt < gt_end) {
    long rb = static_cast<long>(Hkv) * crow(bi);
    int tb = crow(bi + 1) - crow(bi);
    while (gt >= rb + static_cast<long>(Hkv) * tb) {  // rows with no tiles
      ++bi;
      rb = static_cast<long>(Hkv) * crow(bi);
      tb = crow(bi + 1) - crow(bi);
    }
    const int off = static_cast<int>(gt - rb);
    const int kvh = off / tb;
    const int t_begin = off - kvh * tb;
    const int t_end = t_begin + static_cast<int>(min(gt_end - gt, static_cast<long>(tb - t_begin)));
    const int n = decode_row_len(seq_lens, bi, max_pages, ps);
    const int32_t* prow = page_table + static_cast<long>(bi) * max_pages;

    const bf16* qrow = q + (static_cast<long>(bi) * Hq + kvh * grp + min(c, grp - 1)) * D;
    v8bf qf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = c < grp ? load_v8bf(qrow + 32 * ks + 8 * g) : zero_v8bf();
    float m = kNegInf, l = 0.0f;
    v4f acc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};

    // runs of at most 64 pages: lane j holds the id of the run's page p0 + j
    for (int r0 = t_begin; r0 < t_end;) {
      const int p0 = r0 >> tshift;
      const int r1 = min(t_end, (p0 + 64) << tshift);
      const int my_page = lane <= ((r1 - 1) >> tshift) - p0 ? prow[p0 + lane] : -1;
      // Invalid page ids (< 0 or >= num_pages) read page 0, which exists
      // (num_pages >= 1), and contribute no keys.  Tile t < ceil(n / 64)
      // holds min(64, n - 64t) >= 1 keys.
      auto slot_of = [&](int t) {
        const int page = __builtin_amdgcn_readlane(my_page, (t >> tshift) - p0);
        const int k0 = (t & tshift) * 64;
        const bool ok = page >= 0 && page < num_pages;
        DecodeSlot sl;
        sl.nk = ok ? min(64, n - 64 * t) : 0;
        sl.kidx = (static_cast<long>(ok ? page : 0) * Hkv + kvh) * ps + k0;
        sl.pos0 = 64 * t;
        sl.k0 = k0;
        return sl;
      };
      auto k_ptr = [&](const DecodeSlot& sl) { return kp + sl.kidx * D; };
      // V^T page (D, ps) of (page, kv head) starts at key index kidx - k0
      auto v_ptr = [&](const DecodeSlot& sl) { return vp + (sl.kidx - sl.k0) * D + sl.k0; };

      v8bf kf[4][KS];
      v8bf vf[2][DT];
      DecodeSlot cur = slot_of(r0);
      decode_load_k<D>(kf, k_ptr(cur), c, g);
      decode_load_v<D>(vf, v_ptr(cur), ps, voff);
      // Wait for the run's first tile here, so that at the loop head the only
      // loads in flight are the previous iteration's K then V.  With the last
      // tile peeled off, the loads inside the loop are unconditional and every
      // wait in the body stays partial: K.Q^T waits for K only, V^T.P^T for V
      // of this tile only (the next tile's K still in flight).
      __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0)
      auto tile = [&](auto more_c, const DecodeSlot& nxt) __attribute__((always_inline)) {
        constexpr bool kMore = decltype(more_c)::value;
        const int g8 = 8 * g;
        // log-gate bias of the lane's keys 8g..8g+7 and 32+8g..32+8g+7 (a page
        // holds ps >= 64 keys, so all 64 reads stay inside the page)
        float4 bv[4];
        if constexpr (BIAS) {
          const float* brow = key_bias + cur.kidx + g8;
#pragma unroll
          for (int j = 0; j < 4; ++j)
            bv[j] = *reinterpret_cast<const float4*>(brow + 32 * (j >> 1) + 4 * (j & 1));
        }
        // S^T = K.Q^T for the 64 keys of the tile
        v4f sc[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          sc[kt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) sc[kt] = mfma_bf16(kf[kt][ks], qf[ks], sc[kt]);
        }
        if constexpr (kMore) decode_load_k<D>(kf, k_ptr(nxt), c, g);
        // scale, bias (not on the newest key), mask keys past the tile / padding
        // columns.  Entry (kt, i) of lane (c, g) is key 8g + r of the tile with
        // r = key_of_row(kt, i) (key_of_row(kt, 4g + i) = 8g + key_of_row(kt, i)),
        // so every bound below is a scalar compared with 8g.
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = key_of_row(kt, i);
            float val = kNegInf;
            if (g8 < cur.nk - r && c < grp) {
              val = sc[kt][i] * scale_log2;
              if constexpr (BIAS) {
                const float4 b4 = bv[kt];  // keys 32(kt/2) + 4(kt%2) + 8g + i
                const float bi4 = i == 0 ? b4.x : i == 1 ? b4.y : i == 2 ? b4.z : b4.w;
                if (g8 != n - 1 - cur.pos0 - r) val += bi4 * kLog2e;
              }
            }
            sc[kt][i] = val;
          }
        softmax_block<4, DT>(sc, acc, m, l);
        if (cur.nk > 0) {
          // keys past nk hold stale pool contents (possibly inf/nan): zero their V
          if (cur.nk < 64) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
              const int kk = 32 * ks + 8 * g;
              uint32_t mk[4];
#pragma unroll
              for (int q2 = 0; q2 < 4; ++q2)
                mk[q2] = (kk + 2 * q2 < cur.nk ? 0x0000ffffu : 0u) |
                         (kk + 2 * q2 + 1 < cur.nk ? 0xffff0000u : 0u);
#pragma unroll
              for (int tt = 0; tt < DT; ++tt) {
                uint4 x = __builtin_bit_cast(uint4, vf[ks][tt]);
                x.x &= mk[0];
                x.y &= mk[1];
                x.z &= mk[2];
                x.w &= mk[3];
                vf[ks][tt] = __builtin_bit_cast(v8bf, x);
              }
            }
          }
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const v8bf pb = pack_p(sc[2 * ks], sc[2 * ks + 1]);
#pragma unroll
            for (int tt = 0; tt < DT; ++tt) acc[tt] = mfma_bf16(vf[ks][tt], pb, acc[tt]);
          }
        }
        if constexpr (kMore) decode_load_v<D>(vf, v_ptr(nxt), ps, voff);
      };
      for (int t = r0; t + 1 < r1; ++t) {
        const DecodeSlot nxt = slot_of(t + 1);
        tile(BoolC<true>{}, nxt);
        cur = nxt;
      }
      tile(BoolC<false>{}, cur);
      r0 = r1;
    }

    // partial of this segment: O^T[d][q] unnormalised, with m (log2 domain) and l
    const long seg = static_cast<long>(bi) * Hkv + kvh + w;
    if (c < grp) {
      float* po = part_o + (seg * grp + c) * D;
#pragma unroll
      for (int t = 0; t < DT; ++t)
        *reinterpret_cast<float4*>(po + 16 * t + 4 * g) = make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
      if (g == 0) {
        part_ml[(seg * grp + c) * 2] = m;
        part_ml[(seg * grp + c) * 2 + 1] = l;
      }
    }
    gt += t_end - t_begin;
  }
}

// merge the segments of one (batch row, query head); one wave, the segment
// weights exp2(m_s - M) computed lane-parallel into LDS.  A row with no keys
// gets zeros.

__global__ __launch_bounds__(64) void paged_decode_merge_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_ml,
    const int32_t* __restrict__ cum_row, bf16* __restrict__ o, int b, int Hq, int Hkv, int D,
    int W) {
  __shared__ float wsh[kDecodeMaxWaves];
  const int qh = blockIdx.x % Hq;
  const int bi = blockIdx.x / Hq;
  const int grp = Hq / Hkv;
  const int kvh = qh / grp, qi = qh % grp;
  const int lane = threadIdx.x;
  bf16* orow = o + (static_cast<long>(bi) * Hq + qh) * D;
  const int tb = cum_row[bi + 1] - cum_row[bi];
  if (tb <= 0) {
    for (int d0 = 2 * lane; d0 < D; d0 += 128) *reinterpret_cast<uint32_t*>(orow + d0) = 0u;
    return;
  }
  const long T = static_cast<long>(Hkv) * cum_row[b];
  W = static_cast<int>(min(static_cast<long>(W), T));  // as in the decode kernel
  const long g0 = static_cast<long>(Hkv) * cum_row[bi] + static_cast<long>(kvh) * tb;
  const int w0 = decode_wave_of(g0, T, W), w1 = decode_wave_of(g0 + tb - 1, T, W);
  const int nseg = w1 - w0 + 1;  // <= W
  const long slot0 = static_cast<long>(bi) * Hkv + kvh + w0;
  float M = kNegInf;
  for (int s = lane; s < nseg; s += 64) M = fmaxf(M, part_ml[((slot0 + s) * grp + qi) * 2]);
  M = wave_max(M);
  float L = 0.0f;
  for (int s = lane; s < nseg; s += 64) {
    const float ms = part_ml[((slot0 + s) * grp + qi) * 2];
    const float wgt = (ms == kNegInf) ? 0.0f : fast_exp2(ms - M);
    wsh[s] = wgt;
    L += wgt * part_ml[((slot0 + s) * grp + qi) * 2 + 1];
  }
  L = wave_sum(L);
  __syncthreads();
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  for (int d0 = 2 * lane; d0 < D; d0 += 128) {
    float a0 = 0.f, a1 = 0.f;
    int s = 0;
    for (; s + 4 <= nseg; s += 4) {
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
    for (; s < nseg; ++s) {
      const float2 v = *reinterpret_cast<const float2*>(part_o + ((slot0 + s) * grp + qi) * D + d0);
      a0 += wsh[s] * v.x;
      a1 += wsh[s] * v.y;
    }
    *reinterpret_cast<uint32_t*>(orow + d0) = pack_bf16x2(a0 * inv, a1 * inv);
  }
}

// waves of one resident round: CUs x resident 64-thread blocks per CU
template <typename K>
int decode_waves(K kern, int variant) {
  static int cache[64][4] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 1024;
  if (cache[dev][variant] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 64, 0) != hipSuccess ||
        cus <= 0 || per_cu <= 0)
      return 1024;
    cache[dev][variant] = min(cus * per_cu, kDecodeMaxWaves);
  }
  return cache[dev][variant];
}

}  // namespace sa

extern "C" size_t sa_paged_decode_workspace_size(int batch, int num_q_heads, int num_kv_heads,
                                                 int head_dim, int max_pages) {
  if (batch < 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads || max_pages < 0) return 0;
  return sa::decode_ws_layout(batch, num_q_heads, num_kv_heads, head_dim, sa::kDecodeMaxWaves,
                              nullptr, nullptr);
}

namespace sa {

// Argument checks shared by the decode entry points (0 = ok).
int decode_check(int dtype, const void* q, const void* k_pages, const void* v_pages,
                 const int32_t* page_table, const int32_t* seq_lens, const float* key_bias,
                 int batch, int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                 int max_pages, int num_pages, const void* o, const char* who) {
  SA_CHECK_ARG(dtype == sa::kBF16, "%s: only bfloat16 is supported", who);
  SA_CHECK_ARG(batch >= 0 && num_kv_heads > 0 && num_q_heads > 0 &&
                   num_q_heads % num_kv_heads == 0 && num_q_heads / num_kv_heads <= 16,
               "%s: need Hq %% Hkv == 0 and Hq/Hkv <= 16 (Hq=%d Hkv=%d)", who, num_q_heads,
               num_kv_heads);
  SA_CHECK_ARG(head_dim == 64 || head_dim == 128, "%s: head_dim %d not in {64,128}", who,
               head_dim);
  SA_CHECK_ARG(page_size == 64 || page_size == 128, "%s: page_size %d not in {64, 128}", who,
               page_size);
  SA_CHECK_ARG(max_pages >= 0 && static_cast<long>(max_pages) * page_size <= (1L << 30),
               "%s: max_pages %d too large", who, max_pages);
  SA_CHECK_ARG(static_cast<long>(batch) * num_kv_heads * ((static_cast<long>(max_pages) * page_size + 63) / 64) < (1L << 31),
               "%s: more than 2^31 key tiles", who);
  SA_CHECK_ARG(q && k_pages && v_pages && page_table && seq_lens && o, "%s: null pointer", who);
  SA_CHECK_ARG(num_pages >= 1 || batch == 0, "%s: empty page pool", who);
  SA_CHECK_ARG(!key_bias || (reinterpret_cast<uintptr_t>(key_bias) & 15) == 0,
               "%s: key_bias must be 16-byte aligned", who);
  return 0;
}

// waves of the stream-K launch for this head_dim / bias variant
int decode_wave_count(int head_dim, bool bias) {
  if (head_dim == 128)
    return bias ? decode_waves(paged_decode_kernel<128, true>, 0)
                : decode_waves(paged_decode_kernel<128, false>, 1);
  return bias ? decode_waves(paged_decode_kernel<64, true>, 2)
              : decode_waves(paged_decode_kernel<64, false>, 3);
}

// plan (more than 64 rows), stream-K decode and merge on workspace `ws` with W waves
int decode_launch(const void* q, const void* k_pages, const void* v_pages,
                  const int32_t* page_table, const int32_t* seq_lens, const float* key_bias,
                  int batch, int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                  int max_pages, int num_pages, float softmax_scale, void* o, const DecodeWs& ws,
                  int W, hipStream_t s) {
  const float scale = softmax_scale > 0.f ? softmax_scale : 1.0f / sqrtf(static_cast<float>(head_dim));
  const float sl2 = scale * sa::kLog2e;
  if (batch > 64) {   // up to 64 rows the decode waves form the plan themselves
    sa::ProfScope prof_("paged_decode_plan", s);
    hipLaunchKernelGGL(sa::paged_decode_plan_kernel, dim3(1), dim3(1024), 0, s, seq_lens, batch,
                       page_size, max_pages, ws.cum_row);
    SA_CHECK_LAUNCH("paged_decode_plan");
  }
  {
    sa::ProfScope prof_("paged_decode", s);
    auto launch = [&](auto kern) {
      hipLaunchKernelGGL(kern, dim3(W), dim3(64), 0, s, static_cast<const sa::bf16*>(q),
                         static_cast<const sa::bf16*>(k_pages),
                         static_cast<const sa::bf16*>(v_pages), page_table, seq_lens, key_bias,
                         ws.cum_row, ws.part_o, ws.part_ml, batch, num_q_heads, num_kv_heads,
                         page_size, max_pages, num_pages, W, sl2);
    };
    if (head_dim == 128)
      key_bias ? launch(sa::paged_decode_kernel<128, true>) : launch(sa::paged_decode_kernel<128, false>);
    else
      key_bias ? launch(sa::paged_decode_kernel<64, true>) : launch(sa::paged_decode_kernel<64, false>);
    SA_CHECK_LAUNCH("paged_decode");
  }
  {
    sa::ProfScope prof_("paged_decode_merge", s);
    hipLaunchKernelGGL(sa::paged_decode_merge_kernel, dim3(batch * num_q_heads), dim3(64), 0, s,
                       ws.part_o, ws.part_ml, ws.cum_row, static_cast<sa::bf16*>(o), batch,
                       num_q_heads, num_kv_heads, head_dim, W);
    SA_CHECK_LAUNCH("paged_decode_merge");
  }
  return 0;
}

}  // namespace sa

extern "C" int sa_paged_decode_fwd(int dtype, const void* q, const void* k_pages,
                                   const void* v_pages, const int32_t* page_table,
                                   const int32_t* seq_lens, const float* key_bias, int batch,
                                   int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                                   int max_pages, int num_pages, float softmax_scale, void* o,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  if (const int rc = sa::decode_check(dtype, q, k_pages, v_pages, page_table, seq_lens, key_bias,
                                      batch, num_q_heads, num_kv_heads, head_dim, page_size,
                                      max_pages, num_pages, o, "sa_paged_decode_fwd"))
    return rc;
  SA_CHECK_ARG(workspace, "sa_paged_decode_fwd: null workspace");
  sa::DecodeWs ws;
  const size_t need = sa::decode_ws_layout(batch, num_q_heads, num_kv_heads, head_dim,
                                           sa::kDecodeMaxWaves, workspace, &ws);
  SA_CHECK_ARG(workspace_bytes >= need, "sa_paged_decode_fwd: workspace %zu B < %zu B",
               workspace_bytes, need);
  if (batch == 0) return 0;
  const int W = sa::decode_wave_count(head_dim, key_bias != nullptr);
  return sa::decode_launch(q, k_pages, v_pages, page_table, seq_lens, key_bias, batch,
                           num_q_heads, num_kv_heads, head_dim, page_size, max_pages, num_pages,
                           softmax_scale, o, ws, W, static_cast<hipStream_t>(stream));
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
  if (num_seqs == 0 || total_tokens == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const float scale = softmax_scale > 0.f ? softmax_scale : 1.0f / sqrtf(static_cast<float>(head_dim));
  // every query block of the packing gets a workgroup, whatever n_qblk says:
  // rows block_idx lacks select nothing (their outputs are zeros), rows past
  // the packing are never read
  const int grid_qblk = n_qblk > total_tokens / 64 + num_seqs ? n_qblk : total_tokens / 64 + num_seqs;
  const float sl2 = scale * sa::kLog2e;
  const int rc = sa::launch_attn(sa::kCausalSelf, head_dim, q, k, v, cu_seqlens, cu_seqlens, num_seqs,
                                 block_idx, n_qblk, max_blocks, grid_qblk, 0, key_bias, o, total_tokens,
                                 total_tokens, num_heads, sl2, s);
  if (rc) return rc;
  SA_CHECK_LAUNCH("sparse_attn_fwd");
  return 0;
}

extern "C" int sa_attn_varlen_fwd(int dtype, int mode, const void* q, const void* k, const void* v,
                                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                  int num_seqs, const float* key_bias, int total_q, int total_k,
                                  int num_heads, int head_dim, float softmax_scale, void* o,
                                  void* stream) {
  SA_CHECK_ARG(dtype == sa::kBF16, "sa_attn_varlen_fwd: only bfloat16 is supported");
  SA_CHECK_ARG(mode == sa::kCausalSelf || mode == sa::kFullSelf || mode == sa::kCross,
               "sa_attn_varlen_fwd: mode %d not in {0 causal, 1 full, 2 cross}", mode);
  SA_CHECK_ARG(head_dim == 64 || head_dim == 128, "sa_attn_varlen_fwd: head_dim %d not in {64,128}",
               head_dim);
  SA_CHECK_ARG(num_seqs >= 0 && num_heads > 0 && total_q >= 0 && total_k >= 0,
               "sa_attn_varlen_fwd: bad sizes");
  SA_CHECK_ARG(mode == sa::kCross || total_k == total_q,
               "sa_attn_varlen_fwd: self-attention needs total_k == total_q");
  SA_CHECK_ARG(q && k && v && cu_seqlens_q && o && (mode != sa::kCross || cu_seqlens_k),
               "sa_attn_varlen_fwd: null pointer");
  if (num_seqs == 0 || total_q == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const float scale = softmax_scale > 0.f ? softmax_scale : 1.0f / sqrtf(static_cast<float>(head_dim));
  // upper bound on the query blocks (sum over sequences of ceil(len / 64));
  // blocks past the real count find no sequence and exit
  const int n_qblk = total_q / 64 + num_seqs;
  const int32_t* cu_k = mode == sa::kCross ? cu_seqlens_k : cu_seqlens_q;
  const int Tk = mode == sa::kCross ? total_k : total_q;
  const int rc = sa::launch_attn(mode, head_dim, q, k, v, cu_seqlens_q, cu_k, num_seqs, nullptr,
                                 n_qblk, 0, n_qblk, 1, key_bias, o, total_q, Tk, num_heads,
                                 scale * sa::kLog2e, s);
  if (rc) return rc;
  SA_CHECK_LAUNCH("attn_varlen_fwd");
  return 0;
}
