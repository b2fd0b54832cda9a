// The wide GEMM over packed weights (M > 128: prefill chunks), behind plm_gemm_packed and
// plm_gemm_packed_f32out. Arguments are checked by the caller (csrc/packed_api.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace plm {

// K splits the wide kernel uses for this shape (1: none), and the workspace bytes it needs (0
// without splits: the counter area, then one fp32 tile per (tile, split)).
int wide_split(int64_t M, int64_t N, int64_t K);
int64_t wide_workspace(int64_t M, int64_t N, int64_t K);

// Y = X W^T (Y fp32 when out_f32) for 128 < M; returns a PLM_* status.
int wide_gemm(int32_t dtype, const void* x, int64_t ldx, const void* wp, void* y, int64_t ldy, int64_t M, int64_t N,
              int64_t K, void* workspace, size_t workspace_bytes, hipStream_t stream, int out_f32);

}  // namespace plm
