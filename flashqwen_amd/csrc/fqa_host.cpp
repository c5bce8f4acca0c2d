// fqa_host.cpp — host-side helpers of the C ABI (no device work).
#include <hip/hip_runtime_api.h>

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

// KvStore's pool sizing (kv_store.cu:10-33): the pool gets what is left of
// total * fraction after `used` bytes, in whole blocks of layers x 2 x 16 x kv_dim bf16.
// The product total * fraction is taken in float, as the reference's expression
// `totalb * gpu_mem_fraction` (size_t times float) is, so the page count is the same.
// Fewer pages than one max_ctx sequence needs is FQA_ENOSPACE (the reference throws).
int fqa_pool_pages(const fqa_dims* dims, uint64_t total_bytes, uint64_t used_bytes,
                   float fraction, int32_t layers, int32_t max_ctx, int64_t* pages) {
  // any positive finite fraction, as the reference's constructor takes it (above 1 the
  // budget exceeds the device; the allocation is what then fails)
  if (!dims || !pages || layers < 1 || max_ctx < 1 || !(fraction > 0.f) ||
      !std::isfinite(fraction) || static_cast<float>(total_bytes) * fraction >= 1.8e19f ||
      dims->page_size < 1 || dims->n_kv_heads < 1 || dims->head_dim < 1)
    return FQA_EINVAL;
  *pages = 0;
  const uint64_t budget = static_cast<uint64_t>(static_cast<float>(total_bytes) * fraction);
  const uint64_t avail = budget > used_bytes ? budget - used_bytes : 0;
  const uint64_t per_block = static_cast<uint64_t>(layers) * 2 * dims->page_size *
                             dims->n_kv_heads * dims->head_dim * 2;
  const uint64_t n = avail / per_block;
  const int64_t need = (max_ctx + dims->page_size - 1) / dims->page_size;
  // the reference stores the count in an int; block ids here are int32 as well
  *pages = n > 0x7fffffffULL ? 0x7fffffff : static_cast<int64_t>(n);
  return *pages < need ? FQA_ENOSPACE : FQA_OK;
}

// The same sizing from the current device's hipMemGetInfo (what the reference's
// constructor does with cudaMemGetInfo): used = total - free.
int fqa_pool_pages_device(const fqa_dims* dims, float fraction, int32_t layers,
                          int32_t max_ctx, int64_t* pages) {
  if (!pages) return FQA_EINVAL;
  size_t freeb = 0, totalb = 0;
  if (hipMemGetInfo(&freeb, &totalb) != hipSuccess) return FQA_ELAUNCH;
  return fqa_pool_pages(dims, totalb, totalb - freeb, fraction, layers, max_ctx, pages);
}

const char* fqa_version(void) { return "fqa 0.1 gfx950"; }

}  // extern "C"
