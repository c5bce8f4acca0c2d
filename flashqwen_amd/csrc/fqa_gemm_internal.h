// fqa_gemm_internal.h — the projection GEMM as a building block of fused entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fqa {

// The norm / RoPE / append a QKV projection's epilogue applies when it runs unsplit
// (the arguments of fqa_qknorm_rope_append).
struct GemmAppend {
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
  float eps;
  int write_k;
};

// y = x . W^T with fqa_gemm's argument rules.  When the plan splits K, only the split
// kernel runs: the fp32 partials land in `workspace` as [splits][M][N] and the caller
// consumes them (in split order, as fqa_gemm's reduction does); otherwise bf16 y is
// written.  Returns the number of splits (>= 1), 0 for M = 0, or an FQA_E code.
// With `app` (N = 6144, y = the qkv buffer), an unsplit plan on the 256-row tiles applies
// the per-head norm + RoPE + paged append in its epilogue instead of writing bf16 y, with
// the results fqa_qknorm_rope_append would give on that y; *appended says so.
int gemm_launch_partials(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y,
                         int64_t ldy, int32_t M, int32_t N, int32_t K, void* workspace,
                         int64_t workspace_bytes, hipStream_t st,
                         const GemmAppend* app = nullptr, bool* appended = nullptr);

}  // namespace fqa
