// C ABI of the skinny GEMM (declared in include/plm_amd.h).
#include <hip/hip_runtime.h>

#include "gemm_kernel.h"
#include "plm_amd.h"

namespace plm {

hipError_t dispatch(int dtype, const GemmArgs& a, const plm_tile& t, hipStream_t s, bool dry) {
  if (dtype == PLM_BF16) return gemm_dispatch_bf16(a, t, s, dry);
  if (dtype == PLM_F16) return gemm_dispatch_f16(a, t, s, dry);
  return hipErrorInvalidConfiguration;
}


}  // namespace plm

extern "C" {

size_t plm_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, const plm_tile* tile) {
  (void)K;
  if (tile == nullptr || tile->split_k <= 1 || tile->wave_frags <= 0 || M <= 0 || N <= 0) return 0;
  return plm::kCounterBytes + static_cast<size_t>(tile->split_k) * M * N * sizeof(float);
}

int plm_gemm_tile_supported(int32_t dtype, int64_t M, int64_t K, const plm_tile* tile) {
  if (tile == nullptr || M < 1 || M > 128 || K < 1 || K > (int64_t(1) << 30)) return 0;
  if (tile->split_k < 1 || tile->k_waves < 1) return 0;
  plm::GemmArgs a{};
  a.M = static_cast<int>(M);
  a.K = static_cast<int>(K);
  return plm::dispatch(dtype, a, *tile, nullptr, true) == hipSuccess ? 1 : 0;
}

namespace {

int gemm_entry(int32_t dtype, const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy, int64_t M,
               int64_t N, int64_t K, const plm_tile* tile, void* workspace, size_t workspace_bytes, void* stream,
               int out_f32) {
  if (x == nullptr || w == nullptr || y == nullptr || tile == nullptr) return PLM_ERR_ARGUMENT;
  if (dtype != PLM_BF16 && dtype != PLM_F16) return PLM_ERR_ARGUMENT;
  if (M < 1 || M > 128 || N < 1 || K < 8 || K % 8 != 0 || N > (int64_t(1) << 30) || K > (int64_t(1) << 30))
    return PLM_ERR_ARGUMENT;
  if (ldx < K || ldw < K || ldy < N) return PLM_ERR_ARGUMENT;
  if (tile->split_k < 1 || tile->split_k > 64 || tile->wave_frags < 1 || tile->wave_frags > 4) return PLM_ERR_ARGUMENT;
  // Buffer offsets are 31-bit: X and one weight tile must each span less than 2 GiB.
  if (M * ldx * 2 >= (int64_t(1) << 31) || 16 * tile->wave_frags * ldw * 2 >= (int64_t(1) << 31)) return PLM_ERR_ARGUMENT;
  if (ldx % 8 != 0 || ldw % 8 != 0 || !plm::aligned16_ptr(x) || !plm::aligned16_ptr(w)) return PLM_ERR_ALIGNMENT;
  if (!plm_gemm_tile_supported(dtype, M, K, tile)) return PLM_ERR_TILE;
  const size_t need = plm_gemm_workspace_bytes(M, N, K, tile);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || !plm::aligned16_ptr(workspace))) return PLM_ERR_WORKSPACE;
  // One arrival counter per weight tile when K is split across workgroups.
  if (need > 0 && (N + 16 * tile->wave_frags - 1) / (16 * tile->wave_frags) > plm::kMaxCounters) return PLM_ERR_ARGUMENT;

  plm::GemmArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(w);
  a.y = static_cast<uint16_t*>(y);
  a.ldx = ldx;
  a.ldw = ldw;
  a.ldy = ldy;
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.K = static_cast<int>(K);
  a.split = tile->split_k;
  a.out_f32 = out_f32;
  if (need > 0) {
    a.counter = static_cast<int*>(workspace);
    a.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + plm::kCounterBytes);
  }
  const hipError_t err = plm::dispatch(dtype, a, *tile, static_cast<hipStream_t>(stream), false);
  return err == hipSuccess ? PLM_OK : PLM_ERR_LAUNCH;
}

}  // namespace

int plm_gemm(int32_t dtype, const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy, int64_t M,
             int64_t N, int64_t K, const plm_tile* tile, void* workspace, size_t workspace_bytes, void* stream) {
  return gemm_entry(dtype, x, ldx, w, ldw, y, ldy, M, N, K, tile, workspace, workspace_bytes, stream, 0);
}

int plm_gemm_f32out(int32_t dtype, const void* x, int64_t ldx, const void* w, int64_t ldw, float* y, int64_t ldy,
                    int64_t M, int64_t N, int64_t K, const plm_tile* tile, void* workspace, size_t workspace_bytes,
                    void* stream) {
  return gemm_entry(dtype, x, ldx, w, ldw, y, ldy, M, N, K, tile, workspace, workspace_bytes, stream, 1);
}

const char* plm_status_string(int32_t status) {
  switch (status) {
    case PLM_OK: return "ok";
    case PLM_ERR_ARGUMENT: return "invalid argument (size, stride, dtype or null pointer)";
    case PLM_ERR_ALIGNMENT: return "pointer or leading dimension not 16-byte aligned";
    case PLM_ERR_TILE: return "no compiled kernel for this tile configuration and M";
    case PLM_ERR_WORKSPACE: return "workspace missing or too small";
    case PLM_ERR_LAUNCH: return "HIP kernel launch failed";
  }
  return "unknown status";
}

}  // extern "C"
