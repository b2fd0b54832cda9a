// Gated low-rank correction on gfx950 (the arithmetic is described in lora.h): one thread per four
// consecutive output columns of one gated row; h and B rows are read 16 bytes at a time (rank is a
// multiple of 8), a row's h slice is shared by the workgroup's threads through the caches.
#include "lora.h"

#include "plm_amd.h"
#include "tile.h"

namespace plm {
namespace {

constexpr int kLoraThreads = 256;

template <int DT>
__device__ __forceinline__ float dot8(u32x4 a, u32x4 b, float acc) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    acc += from_bits16<DT>(static_cast<uint16_t>(a[w] & 0xffffu)) * from_bits16<DT>(static_cast<uint16_t>(b[w] & 0xffffu));
    acc += from_bits16<DT>(static_cast<uint16_t>(a[w] >> 16)) * from_bits16<DT>(static_cast<uint16_t>(b[w] >> 16));
  }
  return acc;
}

template <int DT>
__global__ __launch_bounds__(kLoraThreads) void lora_apply_kernel(LoraArgs z) {
  const int m = z.gated_from + static_cast<int>(blockIdx.y);
  const int c0 = (static_cast<int>(blockIdx.x) * kLoraThreads + static_cast<int>(threadIdx.x)) * 4;
  if (m >= z.M || c0 >= z.N) return;
  const uint16_t* hrow = z.h + static_cast<int64_t>(m - z.gated_from) * z.ldh;
  uint16_t* yrow = z.y + static_cast<int64_t>(m) * z.ldy;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = c0 + i;
    if (c >= z.N) continue;
    const int s = (c >= z.shard_end[0]) + (c >= z.shard_end[1]) + (c >= z.shard_end[2]);  // shard of column c
    const u32x4* hs = reinterpret_cast<const u32x4*>(hrow + s * z.rank);
    const u32x4* br = reinterpret_cast<const u32x4*>(z.b + static_cast<int64_t>(c) * z.rank);
    float acc = 0.f;
#pragma unroll 4
    for (int j = 0; j < z.rank / 8; ++j) acc = dot8<DT>(hs[j], br[j], acc);
    yrow[c] = to_bits16<DT>(from_bits16<DT>(yrow[c]) + acc);
  }
}

}  // namespace

hipError_t lora_apply(int32_t dtype, const LoraArgs& z, hipStream_t stream) {
  if (z.M <= z.gated_from) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((z.N + 4 * kLoraThreads - 1) / (4 * kLoraThreads)),
                  static_cast<unsigned>(z.M - z.gated_from));
  if (dtype == PLM_BF16)
    hipLaunchKernelGGL(lora_apply_kernel<DT_BF16>, grid, dim3(kLoraThreads), 0, stream, z);
  else
    hipLaunchKernelGGL(lora_apply_kernel<DT_F16>, grid, dim3(kLoraThreads), 0, stream, z);
  return hipGetLastError();
}

}  // namespace plm
