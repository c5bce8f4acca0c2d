// fqa_append_math.h — the per-head QK-RMSNorm + rotate-half RoPE of one (row, head), as
// fqa_qknorm_rope_append and the QKV projection's fused epilogue both compute it.  One
// definition keeps the two bit-identical (same operations in the same order).
#pragma once

#include "fqa_common.h"

namespace fqa {

__device__ __forceinline__ void unpack4(uint2 v, float* f) {
  f[0] = __uint_as_float(v.x << 16);
  f[1] = __uint_as_float(v.x & 0xffff0000u);
  f[2] = __uint_as_float(v.y << 16);
  f[3] = __uint_as_float(v.y & 0xffff0000u);
}

// HeadNormRopeKernel's math (engine/src/kernels.cu:97-131) for one head of one row, held
// by a 16-lane group: lane j of the group holds dims 4j..4j+3 (lo) and 64+4j..64+4j+3 (hi)
// as packed bf16, so both halves of every rotate-half pair sit in one lane.
// y = x * rsqrt(mean(x^2) + eps) * w, then (y1, y2) -> (y1 c - y2 s, y2 c + y1 s), fp32
// throughout, one bf16 rounding at the end (the sum of squares and the rotation use fused
// multiply-adds as written).  The sum of squares is a 16-lane butterfly:
// all 64 lanes of the wave must call this together.
__device__ __forceinline__ void norm_rope_head(uint2 lo, uint2 hi, const float (&wa)[4],
                                               const float (&wb)[4], const float (&cs)[4],
                                               const float (&sn)[4], float eps, uint2& olo,
                                               uint2& ohi) {
  // Every fused multiply-add is written out and no other is allowed: with the compiler
  // free to contract, the two callers' inlined copies were contracted differently.
#pragma clang fp contract(off)
  float x1[4], x2[4];
  unpack4(lo, x1);
  unpack4(hi, x2);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    ss = fmaf(x1[e], x1[e], ss);
    ss = fmaf(x2[e], x2[e], ss);
  }
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) ss += __shfl_xor(ss, m, kWave);
  const float inv = 1.0f / sqrtf(ss / (float)kD + eps);
  float o1[4], o2[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float y1 = x1[e] * inv * wa[e];
    const float y2 = x2[e] * inv * wb[e];
    o1[e] = fmaf(y1, cs[e], -(y2 * sn[e]));
    o2[e] = fmaf(y2, cs[e], y1 * sn[e]);
  }
  olo = make_uint2(pack_bf16x2(o1[0], o1[1]), pack_bf16x2(o1[2], o1[3]));
  ohi = make_uint2(pack_bf16x2(o2[0], o2[1]), pack_bf16x2(o2[2], o2[3]));
}

}  // namespace fqa
