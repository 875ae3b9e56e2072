// Paged decode attention: workspace layout and the launch shared by the
// decode entry points (attention.hip, decode_noalloc.hip).
#pragma once

#include "common.h"

namespace sa {

// most waves a stream-K decode launch uses on any device
constexpr int kDecodeMaxWaves = 8192;

// workspace: segment partials for b * Hkv + W segment ids (segment id =
// row * Hkv + kv head + wave, wave < W), then cum_row (b + 1 ints)
struct DecodeWs {
  float* part_o;
  float* part_ml;
  int32_t* cum_row;
};
inline size_t decode_ws_layout(int b, int Hq, int Hkv, int D, int W, void* base, DecodeWs* out) {
  const size_t segs = static_cast<size_t>(b) * Hkv + W;
  const size_t grp = static_cast<size_t>(Hq / Hkv);
  const size_t o_bytes = (segs * grp * D * sizeof(float) + 255) & ~size_t(255);
  const size_t ml_bytes = (segs * grp * 2 * sizeof(float) + 255) & ~size_t(255);
  const size_t cum_bytes = ((static_cast<size_t>(b) + 1) * sizeof(int32_t) + 255) & ~size_t(255);
  if (out) {
    char* p = static_cast<char*>(base);
    out->part_o = reinterpret_cast<float*>(p);
    out->part_ml = reinterpret_cast<float*>(p + o_bytes);
    out->cum_row = reinterpret_cast<int32_t*>(p + o_bytes + ml_bytes);
  }
  return o_bytes + ml_bytes + cum_bytes + 256;
}

int decode_check(int dtype, const void* q, const void* k_pages, const void* v_pages,
                 const int32_t* page_table, const int32_t* seq_lens, const float* key_bias,
                 int batch, int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                 int max_pages, int num_pages, const void* o, const char* who);
int decode_wave_count(int head_dim, bool bias);
int decode_launch(const void* q, const void* k_pages, const void* v_pages,
                  const int32_t* page_table, const int32_t* seq_lens, const float* key_bias,
                  int batch, int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                  int max_pages, int num_pages, float softmax_scale, void* o, const DecodeWs& ws,
                  int W, hipStream_t s);

}  // namespace sa
