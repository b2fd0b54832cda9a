// plm_gemm_packed_noalloc: plm_gemm_packed for callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The same kernel
// and argument checks; its split-K scratch (the counter area's arrival counters and the fp32
// partials) lives in this file's device array `scratch` instead of a caller's workspace. Nothing
// here calls hipMalloc, hipFree or an allocating library routine.
//
// Each device the library runs on holds its own copy of `scratch` (PLM_NOALLOC_SCRATCH_BYTES) until
// the process ends. Every call on a device shares that copy: calls that overlap on one device (two
// streams, two threads) race and give wrong results. The counter area must be zero when a launch
// starts; every launch leaves it zero, and the first call on a device clears it once (a fill
// kernel on the caller's stream, so it is ordered before that call's launch and can be captured).
#include <hip/hip_runtime.h>

#include <mutex>

#include "packed_gemm.h"
#include "plm_amd.h"

namespace plm {
namespace {

constexpr size_t kScratchBytes = PLM_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes > kCounterBytes, "the scratch holds the counter area and the split partials");

// Host code must not pass `scratch` itself to a kernel: in host code the name is a stand-in, not a
// device address. scratch_on_device() resolves the address once per device.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_lock;
void* g_scratch[kMaxDevices] = {};

__global__ __launch_bounds__(256) void clear_counters_kernel(uint32_t* p, uint32_t words) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < words; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// The device address of `scratch` on the current device (looked up, and its counter area cleared
// on `stream`, on the first call with that device current).
int scratch_on_device(void** out, hipStream_t stream) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return PLM_ERR_LAUNCH;
  std::lock_guard<std::mutex> guard(g_lock);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return PLM_ERR_LAUNCH;
    hipLaunchKernelGGL(clear_counters_kernel, dim3(64), dim3(256), 0, stream, static_cast<uint32_t*>(p),
                       static_cast<uint32_t>(kCounterBytes / 4));
    if (hipGetLastError() != hipSuccess) return PLM_ERR_LAUNCH;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return PLM_OK;
}

}  // namespace
}  // namespace plm

extern "C" {

int plm_gemm_packed_noalloc(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, void* y, int64_t ldy,
                            int64_t M, int64_t N, int64_t K, const plm_tile* tile, void* stream) {
  // Wide calls (M > 128) split K only as far as the scratch holds.
  const int64_t cap = static_cast<int64_t>(plm::kScratchBytes);
  const int64_t need = plm::packed_gemm_workspace(M, N, K, tile, cap);
  if (need < 0)  // an invalid tile or size: the regular checks name it
    return plm::packed_gemm_call(dtype, x, ldx, packed_w, y, ldy, M, N, K, tile, nullptr, 0, stream, 0);
  if (static_cast<uint64_t>(need) > plm::kScratchBytes) return PLM_ERR_WORKSPACE;
  void* ws = nullptr;
  if (need > 0) {
    const int status = plm::scratch_on_device(&ws, static_cast<hipStream_t>(stream));
    if (status != PLM_OK) return status;
  }
  return plm::packed_gemm_call(dtype, x, ldx, packed_w, y, ldy, M, N, K, tile, ws, need > 0 ? plm::kScratchBytes : 0,
                               stream, 0, cap);
}

}  // extern "C"
