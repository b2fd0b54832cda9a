// The wide GEMM over packed weights (M > 128: prefill chunks), behind plm_gemm_packed and
// plm_gemm_packed_f32out. Arguments are checked by the caller (csrc/packed_api.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace plm {

// K splits the wide kernel uses for this shape (1: none), and the workspace bytes it needs (0
// without splits: the counter area, then one fp32 tile per (tile, split)). The split only sets the
// speed, so a caller whose scratch is fixed gives its size as `cap`: the split is then the largest
// the scratch holds (down to 1, which needs none).
constexpr int64_t kNoCap = INT64_MAX;
int wide_split(int64_t M, int64_t N, int64_t K, int64_t cap = kNoCap);
int64_t wide_workspace(int64_t M, int64_t N, int64_t K, int64_t cap = kNoCap);

// Y = X W^T (Y fp32 when out_f32) for 128 < M; returns a PLM_* status.
int wide_gemm(int32_t dtype, const void* x, int64_t ldx, const void* wp, void* y, int64_t ldy, int64_t M, int64_t N,
              int64_t K, void* workspace, size_t workspace_bytes, hipStream_t stream, int out_f32, int64_t cap = kNoCap);

}  // namespace plm
