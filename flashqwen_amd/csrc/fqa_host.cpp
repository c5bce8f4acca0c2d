// fqa_host.cpp — host-side helpers of the C ABI (no device work).
#include <cmath>

#include "../../include/fqa.h"

extern "C" {

// RopeTables::Build (engine/src/model_runtime.cu:111-126): float pow/cos/sin,
// angle = p * theta^(-2i/head_dim), tables [max_pos][head_dim/2].  Same float calls as
// the reference so the tables are bit-identical to its.
int fqa_rope_tables(int32_t max_pos, int32_t head_dim, float theta, float* cos_tab,
                    float* sin_tab) {
  if (max_pos < 0 || head_dim < 2 || head_dim % 2 || !cos_tab || !sin_tab) return FQA_EINVAL;
  const int half = head_dim / 2;
  for (int p = 0; p < max_pos; ++p)
    for (int i = 0; i < half; ++i) {
      float inv = std::pow(theta, -2.0f * i / head_dim);
      float ang = p * inv;
      cos_tab[(int64_t)p * half + i] = std::cos(ang);
      sin_tab[(int64_t)p * half + i] = std::sin(ang);
    }
  return FQA_OK;
}

// Bytes of one layer's pool: pages x kv heads x (K + V) x 16 tokens x head_dim bf16
// (the per-block term of KvStore's sizing, kv_store.cu:24-26, for one layer).
int64_t fqa_pool_bytes(const fqa_dims* dims, int64_t pages) {
  if (!dims || pages < 0) return FQA_EINVAL;
  return pages * dims->n_kv_heads * 2 * (int64_t)dims->page_size * dims->head_dim * 2;
}

const char* fqa_version(void) { return "fqa 0.1 gfx950"; }

}  // extern "C"
