// fqa_common.h — shared device helpers for the gfx950 attention-path kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fqa.h"

namespace fqa {

constexpr int kD = 128;        // head_dim
constexpr int kHq = 32;        // query heads
constexpr int kHkv = 8;        // kv heads
constexpr int kG = kHq / kHkv; // GQA group (query heads per kv head)
constexpr int kPage = FQA_PAGE_TOKENS;
constexpr int kQkvStride = (kHq + 2 * kHkv) * kD;  // 6144
// One (page, kv head) run in the pool: K [16][128] then V^T [128][16], bf16.
constexpr int kRunElems = 2 * kPage * kD;  // 4096 elements = 8 KiB
constexpr int kVOff = kPage * kD;          // V^T starts 2048 elements into the run
constexpr int kWave = 64;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ int64_t run_offset(int64_t page, int kvh) {
  return (page * kHkv + kvh) * (int64_t)kRunElems;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float((uint32_t)b << 16);
}

// Round-to-nearest-even float -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// Two floats -> packed bf16x2 in one dword (RNE), one conversion instruction.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float wave_max_xor(float v, int mask) {
  return fmaxf(v, __shfl_xor(v, mask, kWave));
}

// max(v[l], v[l ^ 32]) with v_permlane32_swap (a VALU op; __shfl_xor goes through the
// LDS crossbar at ~100 cycles).  With both operands = v, the swap leaves the low half of
// v in both halves of one result and the high half in both halves of the other.
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// max(v[l], v[l ^ 16]) with v_permlane16_swap (odd and even 16-lane rows exchanged).
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Sum over l, l^16, l^32, l^48 (the four 16-lane rows) with permlane swaps.
__device__ __forceinline__ float sum_rows4(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ---- wave-level integer scans and reductions on DPP ----------------------------------
// Each step is a VALU op with a lane-shifted operand (row_shr within 16-lane rows, then
// row_bcast across rows), a few cycles each; __shfl_* goes through ds_bpermute (~100
// cycles per step).  Bound-control makes shifted-in lanes read 0.
enum : int {
  kDppRowShr1 = 0x111,
  kDppRowShr2 = 0x112,
  kDppRowShr4 = 0x114,
  kDppRowShr8 = 0x118,
  kDppRowBcast15 = 0x142,
  kDppRowBcast31 = 0x143,
  kDppWaveShr1 = 0x138,
};

// Inclusive prefix sum over the 64 lanes of the wave.
__device__ __forceinline__ int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, kDppRowShr1, 0xf, 0xf, true);
  x += __builtin_amdgcn_update_dpp(0, x, kDppRowShr2, 0xf, 0xf, true);
  x += __builtin_amdgcn_update_dpp(0, x, kDppRowShr4, 0xf, 0xf, true);
  x += __builtin_amdgcn_update_dpp(0, x, kDppRowShr8, 0xf, 0xf, true);
  x += __builtin_amdgcn_update_dpp(0, x, kDppRowBcast15, 0xa, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, kDppRowBcast31, 0xc, 0xf, false);
  return x;
}

// Max / min over the wave (result in every lane): the scan pattern with max/min, then
// lane 63 holds the answer.  `id` is the identity (shifted-in lanes read it).
template <bool kMax>
__device__ __forceinline__ int wave_extreme(int x, int id) {
  auto op = [](int a, int b) { return kMax ? (a > b ? a : b) : (a < b ? a : b); };
  x = op(x, __builtin_amdgcn_update_dpp(id, x, kDppRowShr1, 0xf, 0xf, false));
  x = op(x, __builtin_amdgcn_update_dpp(id, x, kDppRowShr2, 0xf, 0xf, false));
  x = op(x, __builtin_amdgcn_update_dpp(id, x, kDppRowShr4, 0xf, 0xf, false));
  x = op(x, __builtin_amdgcn_update_dpp(id, x, kDppRowShr8, 0xf, 0xf, false));
  x = op(x, __builtin_amdgcn_update_dpp(id, x, kDppRowBcast15, 0xa, 0xf, false));
  x = op(x, __builtin_amdgcn_update_dpp(id, x, kDppRowBcast31, 0xc, 0xf, false));
  return __builtin_amdgcn_readlane(x, 63);
}

// Greedy tie order of the reference's ArgmaxKernel (engine/src/kernels.cu:184-214): 256
// threads scan columns i = tid (mod 256) keeping the first strict maximum, then a tree
// reduction keeps the lower slot unless the upper one is strictly larger.  Among equal
// maxima that tree prefers the thread whose bit-reversed id is smallest (slot pairs that
// differ in bit 0 are merged last), and within a thread the smallest column.  So column
// i wins a tie against column j iff greedy_key(i) < greedy_key(j) (columns below 2^24).
__device__ __forceinline__ uint32_t greedy_key(int i) {
  return ((__builtin_bitreverse32((uint32_t)i & 255u) >> 24) << 24) | ((uint32_t)i >> 8);
}
// ... and a row whose largest logit is not above -1e30 (the reference's starting value)
// gives column 0.
constexpr float kGreedyFloor = -1e30f;

}  // namespace fqa
