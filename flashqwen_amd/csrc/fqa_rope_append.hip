// fqa_rope_append.hip — fused per-head QK-RMSNorm + rotate-half RoPE + paged KV append.
//
// Replaces HeadNormRopeKernel (engine/src/kernels.cu:97-131, launched :133-139) and
// StoreKvKernel (engine/src/kv_store.cu:48-75), which the reference runs as two
// launches with one 128-thread block per (row, head) and one bf16 element per thread.
//
// Here one 16-lane group owns one head of one row: lane j holds dims [4j, 4j+4) and
// [64+4j, 64+4j+4), so both halves of every rotate-half pair sit in the same lane and
// RoPE needs no data exchange; the sum of squares is a 16-lane butterfly.  A 256-thread
// workgroup covers 16 heads, three workgroups cover one row's 32 q + 8 k + 8 v heads.
// Memory-bound: per row 12 KiB read, 8 KiB (q) + 4 KiB (k, v) written.
//
// Semantics (kernels.cu:113-129): y = x * rsqrt(mean(x^2) + eps) * w in fp32, then
// y1' = y1*cos - y2*sin, y2' = y2*cos + y1*sin with no intermediate bf16 rounding,
// one RNE rounding to bf16 at the end.  V is copied unchanged.
#include "fqa_common.h"

namespace fqa {
namespace {

constexpr int kHeadsPerRow = kHq + 2 * kHkv;  // 48
constexpr int kHeadsPerBlock = 16;
constexpr int kBlocksPerRow = kHeadsPerRow / kHeadsPerBlock;  // 3

struct AppendArgs {
  uint16_t* qkv;
  const float* wq;
  const float* wk;
  const float* cos_tab;
  const float* sin_tab;
  int rope_max_pos;
  const int32_t* positions;
  const int32_t* slots;
  const int32_t* meta;
  uint16_t* pool;
  long long pool_pages;
  int stride;
  float eps;
  int write_k;
};

__device__ __forceinline__ void unpack4(uint2 v, float* f) {
  f[0] = __uint_as_float(v.x << 16);
  f[1] = __uint_as_float(v.x & 0xffff0000u);
  f[2] = __uint_as_float(v.y << 16);
  f[3] = __uint_as_float(v.y & 0xffff0000u);
}

__global__ void __launch_bounds__(256) qknorm_rope_append_kernel(AppendArgs a) {
  const int row = blockIdx.x / kBlocksPerRow;
  if (row >= a.meta[FQA_META_ROWS]) return;
  const int head = (blockIdx.x % kBlocksPerRow) * kHeadsPerBlock + (threadIdx.x >> 4);
  const int j = threadIdx.x & 15;

  const int pos = a.positions[row];
  if (pos < 0 || pos >= a.rope_max_pos) return;
  uint16_t* src = a.qkv + (long long)row * a.stride + head * kD;
  uint2 lo = *reinterpret_cast<const uint2*>(src + 4 * j);
  uint2 hi = *reinterpret_cast<const uint2*>(src + 64 + 4 * j);

  const int slot = a.slots[row];
  const long long page = slot / kPage;
  const int tok = slot % kPage;
  const bool page_ok = slot >= 0 && page < a.pool_pages;

  if (head >= kHq + kHkv) {  // v head: copy into V^T [d][16 tokens]
    if (!page_ok) return;
    const int kvh = head - kHq - kHkv;
    uint16_t* vt = a.pool + run_offset(page, kvh) + kVOff + tok;
    const uint16_t l4[4] = {(uint16_t)lo.x, (uint16_t)(lo.x >> 16), (uint16_t)lo.y,
                            (uint16_t)(lo.y >> 16)};
    const uint16_t h4[4] = {(uint16_t)hi.x, (uint16_t)(hi.x >> 16), (uint16_t)hi.y,
                            (uint16_t)(hi.y >> 16)};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      vt[(4 * j + i) * kPage] = l4[i];
      vt[(64 + 4 * j + i) * kPage] = h4[i];
    }
    return;
  }

  float x1[4], x2[4];
  unpack4(lo, x1);
  unpack4(hi, x2);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) ss += x1[i] * x1[i] + x2[i] * x2[i];
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) ss += __shfl_xor(ss, m, kWave);
  const float inv = 1.0f / sqrtf(ss / (float)kD + a.eps);

  const float* w = head < kHq ? a.wq : a.wk;
  const float4 w1 = *reinterpret_cast<const float4*>(w + 4 * j);
  const float4 w2 = *reinterpret_cast<const float4*>(w + 64 + 4 * j);
  const float4 c4 = *reinterpret_cast<const float4*>(a.cos_tab + (long long)pos * 64 + 4 * j);
  const float4 s4 = *reinterpret_cast<const float4*>(a.sin_tab + (long long)pos * 64 + 4 * j);
  const float wa[4] = {w1.x, w1.y, w1.z, w1.w}, wb[4] = {w2.x, w2.y, w2.z, w2.w};
  const float cs[4] = {c4.x, c4.y, c4.z, c4.w}, sn[4] = {s4.x, s4.y, s4.z, s4.w};
  float o1[4], o2[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float y1 = x1[i] * inv * wa[i];
    float y2 = x2[i] * inv * wb[i];
    o1[i] = y1 * cs[i] - y2 * sn[i];
    o2[i] = y2 * cs[i] + y1 * sn[i];
  }
  uint2 olo = make_uint2(pack_bf16x2(o1[0], o1[1]), pack_bf16x2(o1[2], o1[3]));
  uint2 ohi = make_uint2(pack_bf16x2(o2[0], o2[1]), pack_bf16x2(o2[2], o2[3]));
  if (head < kHq || a.write_k) {
    *reinterpret_cast<uint2*>(src + 4 * j) = olo;
    *reinterpret_cast<uint2*>(src + 64 + 4 * j) = ohi;
  }
  if (head >= kHq && page_ok) {  // k head: K [16 tokens][128]
    uint16_t* kd = a.pool + run_offset(page, head - kHq) + tok * kD;
    *reinterpret_cast<uint2*>(kd + 4 * j) = olo;
    *reinterpret_cast<uint2*>(kd + 64 + 4 * j) = ohi;
  }
}

bool dims_ok(const fqa_dims* d) {
  return d && d->n_q_heads == kHq && d->n_kv_heads == kHkv && d->head_dim == kD &&
         d->page_size == kPage && d->qkv_stride >= kQkvStride && d->qkv_stride % 4 == 0;
}

}  // namespace
}  // namespace fqa

using namespace fqa;

extern "C" int fqa_qknorm_rope_append(const fqa_dims* dims, uint16_t* qkv, const float* q_norm_w,
                                      const float* k_norm_w, const float* cos_tab,
                                      const float* sin_tab, int32_t rope_max_pos,
                                      const int32_t* positions,
                                      const int32_t* slot_mapping, const int32_t* meta,
                                      int32_t rows_bound, uint16_t* pool, int64_t pool_pages,
                                      int32_t write_k_inplace, void* stream) {
  if (!dims) return FQA_EINVAL;
  if (!dims_ok(dims)) return FQA_EUNSUPPORTED;
  if (rows_bound < 0 || pool_pages < 1 || rope_max_pos < 1 || !meta) return FQA_EINVAL;
  if (rows_bound == 0) return FQA_OK;
  if (!qkv || !q_norm_w || !k_norm_w || !cos_tab || !sin_tab || !positions || !slot_mapping ||
      !pool)
    return FQA_EINVAL;
  AppendArgs a{qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, rope_max_pos, positions, slot_mapping, meta, pool,
               pool_pages, dims->qkv_stride, dims->eps, write_k_inplace};
  hipLaunchKernelGGL(qknorm_rope_append_kernel, dim3(rows_bound * kBlocksPerRow), dim3(256), 0,
                     (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? FQA_OK : FQA_ELAUNCH;
}
