/*
 * sa_hip.h - C ABI of libsa_hip.so, the MI355X (gfx950) kernel layer of
 * selective-attention.
 *
 * Conventions (all entry points):
 *   - plain device pointers, int sizes, no torch types; tensors are dense
 *     row-major (contiguous) in the shapes documented per function;
 *   - dtype codes: 0 = float32, 1 = bfloat16 (activations); states, A and
 *     delta_bias are always float32;
 *   - `stream` is a hipStream_t (passed as void*); every launch is
 *     asynchronous on it, nothing synchronises the host;
 *   - return 0 on success, 1 for an argument error, 2 for a HIP launch
 *     error; the message is in sa_last_error() (thread-local).  No C++
 *     exception crosses the ABI;
 *   - the library allocates no device memory: outputs and workspaces are
 *     passed in by the caller (the Python layer takes them from torch's
 *     caching allocator).
 */
#ifndef SA_HIP_H_
#define SA_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Library version (incremented on ABI changes). */
int sa_version(void);

/* Message of the last failing call on this thread. */
const char* sa_last_error(void);

/*
 * Per-kernel timing (no counterpart in the reference; a measurement aid).
 * When enabled, every kernel launch is bracketed by HIP events recorded on
 * its stream.  sa_profile_collect synchronises them, aggregates by kernel
 * name (NUL-separated into names_buf), writes total milliseconds and launch
 * counts, clears the records and returns the number of distinct kernels
 * (-1 on a HIP error).  Safe to call from several host threads: the
 * records are guarded by one mutex, taken by a launch only while timing is
 * on, and a launch's record is published only once both of its events are
 * recorded, so a collect never sees a launch in progress; the records of
 * all threads are aggregated together.
 */
void sa_profile_enable(int on);
int sa_profile_collect(char* names_buf, int names_len, float* total_ms, int* counts,
                       int max_kernels);

/*
 * Single-step selective state update, in place on the fp32 state.
 * Replaces ssu_forward (reference triton_kernels/ssu/forward.py:7-63,
 * kernel ssu/forward_kernel.py:6-79), called by SSUFn.forward
 * (ops/ssu.py:8-63).
 *   u (b,H,P), B,C (b,G,N), delta_raw (b,H): dtype `dtype`
 *   A (H,), delta_bias (H,) or NULL: float32
 *   h (b,H,P,N) float32, read and overwritten
 *   y (b,H,P): dtype `dtype`
 *   dt = clamp(softplus20(delta_raw + bias), delta_min, delta_max)
 *   h = h*exp(A*dt) + dt*u (x) B ;  y = h . C
 */
int sa_ssu_fwd(int dtype, const void* u, const float* A, const void* B, const void* C,
               const void* delta_raw, const float* delta_bias, float* h, void* y, int batch,
               int num_heads, int head_dim, int num_groups, int state_dim, int use_softplus,
               float delta_min, float delta_max, void* stream);

/*
 * sa_ssu_fwd with the SSM block's epilogue of the decode step (SSM.step,
 * reference modules/ssm.py:195-204: y + D x, times silu(gate)) applied in
 * the same kernel: out (b,H,P) = (bf(y) + D[h*P + p] u) * silu(gate), with y
 * first rounded to `dtype` as the unfused path stores it; u is the x of that
 * epilogue.  D (H*P,) float32; gate (b,H,P) dtype; out (b,H,P) dtype.  The
 * state update is sa_ssu_fwd's.
 */
int sa_ssu_fwd_gated(int dtype, const void* u, const float* A, const void* B, const void* C,
                     const void* delta_raw, const float* delta_bias, float* h, const float* D,
                     const void* gate, void* out, int batch, int num_heads, int head_dim,
                     int num_groups, int state_dim, int use_softplus, float delta_min,
                     float delta_max, void* stream);

/*
 * SSD chunked scan, forward.  Replaces ssd_scan_forward (reference
 * triton_kernels/ssd_scan/forward.py:223-276: chunk_cumsum_forward :14,
 * chunk_state_forward :62, state_passing_forward :102, bmm_chunk_forward
 * :139, chunk_scan_forward :175), called by SSDScanFn.forward
 * (ops/ssd_scan.py:70-73).
 *   u (b,L,H,P), B,C (b,L,G,N), delta_raw (b,L,H): dtype `dtype`
 *   A (H,), delta_bias (H,) or NULL, h_init (b,H,P,N) or NULL: float32
 *   length (b,) int64 (clamped to [0, L]), or NULL for full rows (what the
 *   reference builds with torch.full when the caller passes none);
 *   chunk_size in [1, 1024]; N <= 256
 * Outputs (float32): y (b,L,H,P), h_last (b,H,P,N), and the intermediates the
 * backward consumes: dt, dc (b,H,nc,Lc) and states (b,nc,H,P,N), which holds
 * the state entering each chunk on return (nc = ceil(L/Lc)).
 */
int sa_ssd_fwd(int dtype, const void* u, const float* A, const void* B, const void* C,
               const void* delta_raw, const float* delta_bias, const float* h_init,
               const int64_t* length, int batch, int seqlen, int num_heads, int head_dim,
               int num_groups, int state_dim, int chunk_size, int use_softplus, float delta_min,
               float delta_max, float* y, float* h_last, float* dt, float* dc, float* states,
               void* stream);

/*
 * Workspace bytes sa_ssd_bwd needs for these sizes (0 on bad arguments).
 */
size_t sa_ssd_bwd_workspace_size(int dtype, int batch, int seqlen, int num_heads, int head_dim,
                                 int num_groups, int state_dim, int chunk_size);

/*
 * SSD chunked scan, backward.  Replaces ssd_scan_backward (reference
 * triton_kernels/ssd_scan/backward.py:467-555 and its kernels
 * backward_kernel.py:23-1039), called by SSDScanFn.backward
 * (ops/ssd_scan.py:84-96).  Consumes the forward's dt, dc, states.
 *   dy (b,L,H,P) float32; dh_last (b,H,P,N) float32 or NULL
 *   outputs: du (dtype, like u), dB, dC (dtype), ddelta_raw (dtype),
 *            dA (H,) f32, ddelta_bias (H,) f32 or NULL, dh_init (b,H,P,N) f32
 *            or NULL (written when has_h_init)
 *   workspace: caller-allocated device memory of at least
 *              sa_ssd_bwd_workspace_size(...) bytes, 256-byte aligned
 * Gradients at t >= length are zero and dy there is ignored.  All
 * reductions are deterministic (no atomics).
 */
int sa_ssd_bwd(int dtype, const void* u, const float* A, const void* B, const void* C,
               const void* delta_raw, const float* delta_bias, const int64_t* length,
               const float* dy, const float* dh_last, const float* dt, const float* dc,
               const float* states, int batch, int seqlen, int num_heads, int head_dim,
               int num_groups, int state_dim, int chunk_size, int use_softplus, float delta_min,
               float delta_max, int has_h_init, void* du, float* dA, void* dB, void* dC,
               void* ddelta_raw, float* ddelta_bias, float* dh_init, void* workspace,
               size_t workspace_bytes, void* stream);

/*
 * Varlen block-sparse causal self-attention (prefill), bfloat16.  No
 * counterpart kernel in the reference: semantics of SelectiveMHA's gated
 * softmax (modules/selective_attention.py:27-144, mode "seq") restricted to
 * selected 64-key blocks of the query's own sequence.
 *   q, k, v, o: (total_tokens, num_heads, head_dim) bf16, head_dim in {64,128}
 *   cu_seqlens: (num_seqs+1,) int32; block_idx: (num_heads, n_qblk, max_blocks)
 *   int32, local key-block ids per 64-query block (-1 unused); key_bias:
 *   (num_heads, total_tokens) f32 or NULL (not applied on the diagonal);
 *   softmax_scale <= 0 selects 1/sqrt(head_dim).
 */
int sa_sparse_attn_fwd(int dtype, const void* q, const void* k, const void* v,
                       const int32_t* cu_seqlens, int num_seqs, const int32_t* block_idx,
                       int n_qblk, int max_blocks, int block_size, const float* key_bias,
                       int total_tokens, int num_heads, int head_dim, float softmax_scale, void* o,
                       void* stream);

/*
 * Dense varlen attention (prefill), bfloat16, in three modes:
 *   mode 0  causal self-attention: query i of a sequence sees keys j <= i;
 *           the key bias is not applied on j = i (SelectiveMHA, is_causal,
 *           modules/selective_attention.py:27-144, mode "seq")
 *   mode 1  bidirectional self-attention: every key of the sequence, bias not
 *           applied on j = i (SelectiveMHA with is_causal=False, the encoder
 *           blocks of modules/bi_block.py:51-94; self mask :84-86)
 *   mode 2  cross-attention: query i of sequence s sees every key of the key
 *           sequence cu_seqlens_k[s]..cu_seqlens_k[s+1]; the bias is not
 *           applied on its key 0 (CrossSelectiveMHA,
 *           modules/cross_selective_attention.py:63-157)
 * No counterpart kernel in the reference (its attention is dense torch).
 *   q, o: (total_q, num_heads, head_dim); k, v: (total_k, num_heads, head_dim)
 *   bf16, head_dim in {64,128}; cu_seqlens_q / _k: (num_seqs+1,) int32
 *   (cu_seqlens_k only read in mode 2; modes 0 and 1 need total_k == total_q);
 *   key_bias: (num_heads, total_k) f32 or NULL; softmax_scale <= 0 selects
 *   1/sqrt(head_dim).  A query with no key gets zeros.
 */
int sa_attn_varlen_fwd(int dtype, int mode, const void* q, const void* k, const void* v,
                       const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int num_seqs,
                       const float* key_bias, int total_q, int total_k, int num_heads, int head_dim,
                       float softmax_scale, void* o, void* stream);

/*
 * RMSNorm of `rows` rows of `dim` elements (modules/rms_norm.py:33-44):
 * out = x * rsqrt(mean(x^2) + eps) * (1 + weight[row % groups]), fp32
 * arithmetic, out in x's dtype (f32 or bf16); weight (groups, dim) f32.
 */
int sa_rms_norm_fwd(int dtype, const void* x, const float* weight, long rows, int dim, int groups,
                    float eps, void* out, void* stream);

/*
 * Residual add fused with the next RMSNorm (the pre-norm blocks,
 * modules/causal_block.py:84-98): out = bf16(x + y), nrm = RMSNorm(out) with
 * weight (dim,) f32; bf16 rows of dim elements, dim % 512 == 0, dim <= 4096,
 * 16-byte aligned.
 */
int sa_add_rms_norm_bf16(const void* x, const void* y, const float* weight, long rows, int dim,
                         float eps, void* out, void* nrm, void* stream);

/*
 * SelectiveMHA.step's gates (modules/selective_attention.py:378-387): g =
 * gate_proj output (rows, heads + dim) bf16; s = bf16(sigmoid(g)); for the
 * first `heads` columns log_gate (rows, heads) f32 = log(s) * score_std[h] *
 * penalty where s > 0 and s >= thr[h] (thr may be NULL), -inf elsewhere;
 * the rest -> out_gate (rows, dim) bf16 = s.
 */
int sa_mha_gates_bf16(const void* g, const float* thr, const float* score_std, float penalty,
                      long rows, int heads, int dim, float* log_gate, void* out_gate, void* stream);

/*
 * Per-head statistics of the valid attention scores s_ij = scale * q_i . k_j,
 * for the training forwards of SelectiveMHA and CrossSelectiveMHA:
 * out[h] = (count, sum, sum of squares) in fp64 over every batch row's valid
 * pairs (query i < q_length[b], key j < k_length[b], and j <= i when
 * causal != 0), the score matrix never written.  Replaces the dense
 * reductions of the reference's modules/selective_attention.py:234-246
 * (q_length = k_length = the row lengths) and
 * modules/cross_selective_attention.py:129-146 (q_length NULL, k_length the
 * context lengths); the std and running average stay with the caller.
 * q (batch, heads, q_len, head_dim), k (batch, heads, k_len, head_dim)
 * contiguous, bf16 (dtype 1) or fp32 (dtype 0), 16-byte aligned; head_dim
 * 32, 64, 96 or 128; a NULL length means every position; causal needs
 * q_len == k_len; workspace of sa_score_stats_workspace_size(batch, heads,
 * q_len) bytes.  Deterministic.
 */
size_t sa_score_stats_workspace_size(int batch, int heads, int q_len);
int sa_score_stats(int dtype, const void* q, const void* k, const int64_t* q_length,
                   const int64_t* k_length, int batch, int heads, int q_len, int k_len,
                   int head_dim, int causal, float scale, void* workspace, size_t workspace_bytes,
                   double* out, void* stream);

/*
 * Small-batch linear layer of the decode steps (nn.Linear with x of at most 8
 * rows): y (M, N) = bf16(x (M, K) . W (N, K)^T + bias (N,)), bf16, fp32
 * accumulation; M in 1..8, K % 8 == 0, K <= 4096, x and W 16-byte aligned; bias may
 * be NULL.
 */
int sa_gemv_bf16(const void* x, const void* W, const void* bias, int M, int N, int K, void* y,
                 void* stream);

/*
 * Several small-batch linear layers of the same x in one launch (the decode
 * step's gate/q/k/v projections of SelectiveMHA.step,
 * modules/selective_attention.py:370,380-382; SwiGLU's two input
 * projections, modules/feed_forward.py:11-12; the three row blocks of
 * SSM.in_proj that SSM.step splits, modules/ssm.py:163-165): for i < nseg
 * (1..4),
 * y[i] (M, N[i]) = bf16(xs (M, K) . W[i] (N[i], K)^T + bias[i]), each y[i]
 * contiguous.  xs = x, or bf16(x * xscale) elementwise when xscale (M, K)
 * bf16 is not NULL (the out_gate product before out_proj,
 * modules/selective_attention.py:446).  bias
 * may be NULL (no biases) or hold NULL entries.  Limits as sa_gemv_bf16;
 * the pointer arrays are read on the host during the call.
 */
int sa_gemv_bf16_multi(const void* x, const void* xscale, int M, int K, int nseg,
                       const void* const* W, const void* const* bias, const int* N, void* const* y,
                       void* stream);

/*
 * SwiGLU's gated product (modules/feed_forward.py:10-11): out = bf16(a *
 * bf16(silu(c))), n bf16 elements (n % 8 == 0, 16-byte aligned).
 */
int sa_silu_mul_bf16(const void* a, const void* c, long n, void* out, void* stream);

/*
 * Rotary embedding of two tensors at once (q and k; modules/rope.py:9-64):
 * y = x cos(p f) + rotate_half(x) sin(p f) for x0 -> y0 and x1 -> y1, each
 * (rows, heads, head_dim) in `dtype` (f32 or bf16), y in bf16; f = inv_freq
 * (head_dim / 2,) f32; position of row r = positions[r % period] (int64), or
 * r % period when positions is NULL.  head_dim % 8 == 0.
 */
int sa_rope_bf16(int dtype, const void* x0, const void* x1, void* y0, void* y1, long rows,
                 int heads, int head_dim, const float* inv_freq, const int64_t* positions,
                 int period, void* stream);

/*
 * Paged cache build after a prefill (PagedSelectiveAttnCache.build; the
 * reference's SelectiveAttnCache.build_kv, inference/selective_attn_cache.py:9-28):
 * for row r and page slot j < ceil(seq_lens[r] / page_size), page
 * page_table[r, j] receives tokens j*page_size .. of row r for every head:
 * k_pages (n, heads, page_size, head_dim) and v_pages transposed
 * (n, heads, head_dim, page_size) bf16, gate_pages (n, heads, page_size) f32
 * = log_gate; zero K / V and -inf gates past seq_lens[r].  k, v bf16 with
 * element strides sb (batch), st (token), sh (head), head_dim contiguous;
 * log_gate f32 with strides gb, gh, gt.  page_table (batch, max_pages) int32;
 * head_dim % 8 == 0, page_size % 8 == 0.
 */
int sa_paged_kv_build(const void* k, const void* v, long sb, long st, long sh,
                      const float* log_gate, long gb, long gh, long gt, const int32_t* page_table,
                      const int32_t* seq_lens, int batch, int heads, int head_dim, int page_size,
                      int max_pages, void* k_pages, void* v_pages, float* gate_pages,
                      void* stream);

/*
 * One decode token per batch row into a paged KV cache
 * (SelectiveAttnCache.update_kv, inference/selective_attn_cache.py:30-42):
 * slot seq_lens[r], page page_table[r][slot / page_size] (column clamped to
 * max_pages - 1); k, v (batch, heads, head_dim) bf16 into k_pages
 * (num_pages, heads, page_size, head_dim) and v_pages (num_pages, heads,
 * head_dim, page_size), log_gate (batch, heads) f32 into gate_pages
 * (num_pages, heads, page_size); then seq_lens[r] += 1 on the device.
 */
int sa_paged_kv_append(const void* k, const void* v, const float* log_gate,
                       const int32_t* page_table, int32_t* seq_lens, int batch, int heads,
                       int head_dim, int page_size, int max_pages, void* k_pages, void* v_pages,
                       float* gate_pages, void* stream);

/* Workspace bytes of sa_paged_decode_fwd: segment partials for
 * batch * num_kv_heads + 8192 segments, plus a per-row tile prefix sum. */
size_t sa_paged_decode_workspace_size(int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                      int max_pages);

/*
 * Paged GQA decode attention, bfloat16.  No counterpart kernel in the
 * reference: semantics of SelectiveMHA.step (modules/selective_attention.py:
 * 392-405, mode "pos") over a paged cache.
 *   q, o: (batch, Hq, D) bf16; k_pages: (num_pages, Hkv, page_size, D) bf16;
 *   v_pages: (num_pages, Hkv, D, page_size) bf16 (V transposed per page);
 *   page_size in {64,128}, D in {64,128}, Hq/Hkv <= 16; page_table:
 *   (batch, max_pages) int32; seq_lens: (batch,) int32; key_bias:
 *   (num_pages, Hkv, page_size) f32 or NULL (not applied to the newest key).
 *   Page ids outside [0, num_pages) contribute no keys; num_pages >= 1;
 *   key_bias 16-byte aligned.  Three launches: a per-row tile prefix sum,
 *   the stream-K decode (one resident round of waves, equal tile ranges,
 *   one partial per (row, kv head) a wave touches), then a log-sum-exp merge.
 */
int sa_paged_decode_fwd(int dtype, const void* q, const void* k_pages, const void* v_pages,
                        const int32_t* page_table, const int32_t* seq_lens, const float* key_bias,
                        int batch, int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                        int max_pages, int num_pages, float softmax_scale, void* o,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * Allocation-free paged GQA decode attention.  No counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops or harnesses that forbid hipMalloc).  Same
 * arguments, semantics, kernels and result bits as sa_paged_decode_fwd,
 * without the workspace: the segment partials live in a file-scope device
 * array of sa_paged_decode_noalloc_limit() bytes (32 MiB), one per GPU, held
 * until the process ends.  A call that would need more scratch than that
 * (batch * Hkv + the launch's waves segments of (Hq/Hkv) * D + 2 floats,
 * plus the row prefix sum) fails with return value 1 before any launch.
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (other streams, other threads) race and must be serialised by the
 * caller.  Nothing in the array needs clearing between calls.
 */
size_t sa_paged_decode_noalloc_limit(void);
int sa_paged_decode_fwd_noalloc(int dtype, const void* q, const void* k_pages,
                                const void* v_pages, const int32_t* page_table,
                                const int32_t* seq_lens, const float* key_bias, int batch,
                                int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                                int max_pages, int num_pages, float softmax_scale, void* o,
                                void* stream);

/*
 * SSM prologue: SiLU, then the depthwise causal conv (zero history), then the
 * split into x / B / C.  Replaces the torch ops of SSM.forward
 * (reference modules/ssm.py:116-125: F.silu, nn.Conv1d(padding=K-1) sliced
 * to seq_len, torch.split) and, with conv_ctx set, SSMCache.build_conv_ctx
 * (inference/ssm_cache.py:8-36).
 *   hbc (b,L,channels): dtype `dtype`; weight (channels,K) float32 (the
 *   Conv1d weight (channels,1,K)); bias (channels,) float32 or NULL
 *   x (b,L,x_dim), B and C (b,L,bc_dim), x_dim + 2*bc_dim = channels:
 *   dtype `dtype`, each contiguous
 *   xBC[b,t,c] = bias[c] + sum_{j<K} weight[c,j] * silu(hbc[b,t-K+1+j,c])
 *   conv_ctx (b,channels,K) or NULL: hbc[b, len_b-K+j, c] for
 *   0 <= len_b-K+j < len_b, else 0; len_b = lengths[b] (int64) or L.
 *   x, B and C all NULL: only conv_ctx is written.  1 <= K <= 8.
 */
int sa_ssm_conv_fwd(int dtype, const void* hbc, const float* weight, const float* bias, int batch,
                    int seqlen, int channels, int kernel, int x_dim, int bc_dim, void* x, void* B,
                    void* C, const int64_t* lengths, void* conv_ctx, void* stream);

size_t sa_ssm_conv_bwd_workspace_size(int batch, int seqlen, int channels, int kernel);

/*
 * Backward of sa_ssm_conv_fwd (the reference gets it from torch autograd
 * through F.silu and nn.Conv1d, modules/ssm.py:116-118).
 *   dx, dB, dC: gradients of x, B, C (dtype `dtype`); dhbc (b,L,channels);
 *   dweight (channels,K), dbias (channels,) or NULL: float32, overwritten.
 *   The weight and bias gradients are summed per 256-row block and then in a
 *   fixed order (bit-reproducible).
 */
int sa_ssm_conv_bwd(int dtype, const void* hbc, const float* weight, const void* dx,
                    const void* dB, const void* dC, int batch, int seqlen, int channels,
                    int kernel, int x_dim, int bc_dim, void* dhbc, float* dweight, float* dbias,
                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * SSM decode-step prologue.  Replaces SSMCache.update
 * (inference/ssm_cache.py:38-43: roll the context left, put the new row
 * last) and the conv of SSM.step (modules/ssm.py:173-182).
 *   hbc_t (b,channels), conv_ctx (b,channels,K) updated in place: dtype
 *   `dtype`; weight, bias as in sa_ssm_conv_fwd; x (b,x_dim), B, C (b,bc_dim).
 */
int sa_ssm_conv_step(int dtype, const void* hbc_t, void* conv_ctx, const float* weight,
                     const float* bias, int batch, int channels, int kernel, int x_dim,
                     int bc_dim, void* x, void* B, void* C, void* stream);

/*
 * SSM epilogue: out = (y + D*x) * silu(gate).  Replaces
 * modules/ssm.py:144-150 (and the step's :200-202).
 *   y (rows,dim) float32 (the scan output); x, gate, out (rows,dim): dtype
 *   `dtype`; D (dim,) float32.
 */
int sa_ssm_gate_fwd(int dtype, const float* y, const void* x, const float* D, const void* gate,
                    int64_t rows, int dim, void* out, void* stream);

size_t sa_ssm_gate_bwd_workspace_size(int64_t rows, int dim);

/*
 * Backward of sa_ssm_gate_fwd (torch autograd in the reference):
 *   dy = dout*silu(gate) (float32); dx = D*dy; dgate = dout*(y+D*x)*silu'(gate)
 *   (dtype `dtype`); dD (dim,) float32 = sum over rows of dy*x, summed per
 *   256-row block and then in a fixed order.
 *   y: the float32 scan output, or with y_is_yd the `dtype` tensor yd = y+D*x
 *   that sa_ssd_fwd_gated saves.
 */
int sa_ssm_gate_bwd(int dtype, const void* dout, const void* y, int y_is_yd, const void* x,
                    const float* D, const void* gate, int64_t rows, int dim, float* dy, void* dx,
                    void* dgate, float* dD, void* workspace, size_t workspace_bytes, void* stream);

/*
 * 1 when sa_ssd_fwd_gated handles these sizes (bfloat16, head_dim % 8 == 0,
 * state_dim a multiple of 32 up to 256), else 0.
 */
int sa_ssd_fwd_gated_supported(int dtype, int head_dim, int state_dim);

/*
 * SSD chunked scan forward with the SSM epilogue fused into its output
 * stage: SSDScanFn (ops/ssd_scan.py:7-80) followed by modules/ssm.py:144-150
 * ((y + D*u) * silu(gate)) in one pass, so the float32 y is never written.
 * Arguments as sa_ssd_fwd, plus D (H*P,) float32 and gate (b,L,H,P) bf16;
 * outputs out = (y + D*u)*silu(gate) and yd = y + D*u, (b,L,H,P) bf16 (yd is
 * what sa_ssm_gate_bwd needs), with h_last, dt, dc, states as in sa_ssd_fwd.
 * D, gate, out, yd 16-byte aligned.
 */
int sa_ssd_fwd_gated(int dtype, const void* u, const float* A, const void* B, const void* C,
                     const void* delta_raw, const float* delta_bias, const float* h_init,
                     const int64_t* length, int batch, int seqlen, int num_heads, int head_dim,
                     int num_groups, int state_dim, int chunk_size, int use_softplus,
                     float delta_min, float delta_max, const float* D, const void* gate, void* out,
                     void* yd, float* h_last, float* dt, float* dc, float* states, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SA_HIP_H_ */
