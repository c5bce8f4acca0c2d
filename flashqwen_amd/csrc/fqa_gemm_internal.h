// fqa_gemm_internal.h — the projection GEMM as a building block of fused entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fqa {

// y = x . W^T with fqa_gemm's argument rules.  When the plan splits K, only the split
// kernel runs: the fp32 partials land in `workspace` as [splits][M][N] and the caller
// consumes them (in split order, as fqa_gemm's reduction does); otherwise bf16 y is
// written.  Returns the number of splits (>= 1), 0 for M = 0, or an FQA_E code.
int gemm_launch_partials(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y,
                         int64_t ldy, int32_t M, int32_t N, int32_t K, void* workspace,
                         int64_t workspace_bytes, hipStream_t st);

}  // namespace fqa
