// Allocation-free paged decode attention (sa_paged_decode_fwd_noalloc): the
// entry point for callers that cannot allocate device memory (code under
// graph capture, serving loops that forbid hipMalloc).  It runs the kernels
// of sa_paged_decode_fwd on a workspace held in a file-scope device array.
#include "decode.h"

#include <mutex>

// ---------------------------------------------------------------------------
// Allocation-free variant: the workspace is a file-scope device array of
// kScratchBytes, one copy per GPU, held until the process ends.  Host code
// reaches it only through the address hipGetSymbolAddress returns for the
// current device (the array's name on the host is not a device address).
// ---------------------------------------------------------------------------
namespace sa {
constexpr size_t kScratchBytes = size_t(32) << 20;
constexpr int kMaxDevices = 64;
}  // namespace sa

__device__ __align__(256) unsigned char scratch[sa::kScratchBytes];

namespace sa {
namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// this device's copy of `scratch` (resolved once per device, with the device current)
int scratch_of_current_device(void** out) {
  int dev = -1;
  SA_CHECK_LAUNCH_RC(hipGetDevice(&dev), "sa_paged_decode_fwd_noalloc: hipGetDevice");
  SA_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "sa_paged_decode_fwd_noalloc: device %d >= %d", dev,
               kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    SA_CHECK_LAUNCH_RC(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                       "sa_paged_decode_fwd_noalloc: hipGetSymbolAddress(scratch)");
    SA_CHECK_ARG(p != nullptr, "sa_paged_decode_fwd_noalloc: no address for scratch on device %d",
                 dev);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}
}  // namespace
}  // namespace sa

extern "C" size_t sa_paged_decode_noalloc_limit(void) { return sa::kScratchBytes; }

extern "C" int sa_paged_decode_fwd_noalloc(int dtype, const void* q, const void* k_pages,
                                           const void* v_pages, const int32_t* page_table,
                                           const int32_t* seq_lens, const float* key_bias,
                                           int batch, int num_q_heads, int num_kv_heads,
                                           int head_dim, int page_size, int max_pages,
                                           int num_pages, float softmax_scale, void* o,
                                           void* stream) {
  if (const int rc = sa::decode_check(dtype, q, k_pages, v_pages, page_table, seq_lens, key_bias,
                                      batch, num_q_heads, num_kv_heads, head_dim, page_size,
                                      max_pages, num_pages, o, "sa_paged_decode_fwd_noalloc"))
    return rc;
  if (batch == 0) return 0;
  const int W = sa::decode_wave_count(head_dim, key_bias != nullptr);
  // size the partials for the waves this launch uses (the allocating entry
  // sizes them for the most waves any device could use)
  const size_t need = sa::decode_ws_layout(batch, num_q_heads, num_kv_heads, head_dim, W,
                                           nullptr, nullptr);
  SA_CHECK_ARG(need <= sa::kScratchBytes,
               "sa_paged_decode_fwd_noalloc: needs %zu B of scratch, more than its %zu B "
               "(batch %d, %d q heads, %d kv heads, head_dim %d); use sa_paged_decode_fwd",
               need, sa::kScratchBytes, batch, num_q_heads, num_kv_heads, head_dim);
  void* base = nullptr;
  if (const int rc = sa::scratch_of_current_device(&base)) return rc;
  sa::DecodeWs ws;
  sa::decode_ws_layout(batch, num_q_heads, num_kv_heads, head_dim, W, base, &ws);
  // every byte the merge reads is written earlier in the same call (cum_row
  // by the plan kernel or, up to 64 rows, by decode wave 0; each segment
  // partial by its wave): nothing is cleared
  return sa::decode_launch(q, k_pages, v_pages, page_table, seq_lens, key_bias, batch,
                           num_q_heads, num_kv_heads, head_dim, page_size, max_pages, num_pages,
                           softmax_scale, o, ws, W, static_cast<hipStream_t>(stream));
}

