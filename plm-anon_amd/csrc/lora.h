// Gated low-rank correction of a linear's output (plm/gated_lora.py:45-57): rows m >= gated_from of
// Y (already the base product in the model dtype) become
//   round(Y[m, n] + sum_j h[m - gated_from, s*rank + j] * B[n, j])
// with s the shard holding column n, h = X[gated_from:] A^T in the model dtype and B the shards'
// up-projections stacked by output column — the reference's one addmm_ per shard, in place.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace plm {

struct LoraArgs {
  uint16_t* y;        // [M][ldy]
  int64_t ldy;
  const uint16_t* h;  // [M - gated_from][ldh]
  const uint16_t* b;  // [N][rank], 16-byte aligned
  int ldh, rank, gated_from, M, N;
  int shard_end[3];   // exclusive column ends of the first three shards, ascending (N past the last)
};

// Launches the correction (rank a multiple of 8) on `stream`; dtype is PLM_BF16 or PLM_F16.
hipError_t lora_apply(int32_t dtype, const LoraArgs& z, hipStream_t stream);

}  // namespace plm
