// Wide GEMM over packed weights: Y[M,N] = X[M,K] · W[N,K]^T for M > 128 (the prefill chunks the
// reference hands to F.linear, plm/rounds.py:16, plm/fast_gemm.py:108-111), so that a caller that
// keeps only the packed copy of a weight has a compute-bound kernel for them.
//
// A workgroup tile is 128 weight rows x 128 X rows; its four wavefronts each compute 64 x 64
// (4 x 4 MFMA fragments of 16 x 16, v_mfma_f32_16x16x32_{bf16,f16}). Per 32-wide K step the
// workgroup stages the tile's 8 weight fragments (packed: each a contiguous KiB already in operand
// order) and 8 X fragments (16 rows x 64 bytes, loaded coalesced, a quad of lanes per row, and
// written to LDS in operand order) through registers into one of two LDS slots; every wavefront
// then reads its 4 + 4
// operands lane-linearly (no bank conflicts) and issues 16 MFMAs. Global loads run kStages K steps
// ahead in registers. Each X fragment is read from LDS by two wavefronts and each weight fragment
// by two, so a K step moves 16 KiB from L2 per workgroup for 512 MFMA passes of 16 cycles.
//
// Thin shapes (few tiles for 256 CUs) split K: each split writes its fp32 tile to the workspace
// (device-coherent), and the last split of the tile to arrive adds the splits in order 0..S-1 and
// writes Y, so results are bitwise reproducible run to run. Rows past N or M and K past K are
// loaded as zeros (buffer range checks and per-lane masks) and never stored.
#include <hip/hip_runtime.h>

#include "plm_amd.h"
#include "tile.h"
#include "wide_gemm.h"

namespace plm {
namespace {

constexpr int kWideRows = 128;                // weight rows and X rows per tile
constexpr int kWideFrags = kWideRows / 16;    // fragments per side
constexpr int kWideWaves = 4;
constexpr int kWideStages = 6;                // K steps of global loads in flight
constexpr int kWideThreads = 64 * kWideWaves;
constexpr uint32_t kWideNoLoad = 0x80000000u;

struct WideArgs {
  const void* x;
  const void* w;
  void* y;
  int64_t ldx, ldy;
  int M, N, Ks, k_last, mtiles, split, out_f32;
  float* partial;  // split > 1: [tile][split][wave][16 fragments][64 lanes] f32x4
  int* arrive;     // split > 1: one arrival counter per tile
};

template <int DT>
__device__ __forceinline__ void wide_store4(const WideArgs& a, int m, int n, f32x4 v) {
  const int left = a.N - n;
  if (a.out_f32) {
    float* y = static_cast<float*>(a.y) + static_cast<int64_t>(m) * a.ldy + n;
    if (left >= 4 && (reinterpret_cast<uintptr_t>(y) & 15) == 0) {
      *reinterpret_cast<f32x4*>(y) = v;
    } else {
      for (int j = 0; j < 4 && j < left; ++j) y[j] = v[j];
    }
    return;
  }
  uint16_t* y = static_cast<uint16_t*>(a.y) + static_cast<int64_t>(m) * a.ldy + n;
  const uint16_t h[4] = {to_bits16<DT>(v[0]), to_bits16<DT>(v[1]), to_bits16<DT>(v[2]), to_bits16<DT>(v[3])};
  if (left >= 4 && (reinterpret_cast<uintptr_t>(y) & 7) == 0) {
    *reinterpret_cast<uint64_t*>(y) = (static_cast<uint64_t>(h[0]) | (static_cast<uint64_t>(h[1]) << 16)) |
                                      ((static_cast<uint64_t>(h[2]) | (static_cast<uint64_t>(h[3]) << 16)) << 32);
  } else {
    for (int j = 0; j < 4 && j < left; ++j) y[j] = h[j];
  }
}

__device__ __forceinline__ void wide_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int DT>
__global__ __launch_bounds__(kWideThreads, 2) void wide_gemm_kernel(WideArgs a) {
  // [slot][fragment: 8 weight, then 8 X][lane]: 2 x 16 KiB
  __shared__ __attribute__((aligned(16))) u32x4 lds[2][2 * kWideFrags][64];
  __shared__ int last_flag;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wn = wave & 1, wm = wave >> 1;  // this wavefront's 64 weight rows and 64 X rows
  // item = (tile, split), split fastest; tile = (nt, mt), mt fastest, so the X tiles that share a
  // weight tile run side by side.
  const int item = blockIdx.x;
  const int tile = item / a.split, sp = item - tile * a.split;
  const int nt = tile / a.mtiles, mt = tile - nt * a.mtiles;
  const int s_lo = static_cast<int>(static_cast<int64_t>(sp) * a.Ks / a.split);
  const int s_hi = static_cast<int>(static_cast<int64_t>(sp + 1) * a.Ks / a.split);
  const int steps = (s_hi - s_lo + kWideStages - 1) / kWideStages * kWideStages;  // padded: zero steps

  const auto wr = make_rsrc(a.w, static_cast<uint32_t>(pack_bytes(a.N, a.Ks)));
  const uint32_t wgroup = pack_group_bytes(a.N);
  const auto xr = make_rsrc(a.x, static_cast<uint32_t>(static_cast<int64_t>(a.M) * a.ldx * 2));
  // This wavefront stages weight fragments 2w, 2w+1 and X fragments 2w, 2w+1 of every K step.
  uint32_t wo[2], xo[2], xl[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int f = nt * kWideFrags + 2 * wave + q;
    wo[q] = pack_row_offset(f) + static_cast<uint32_t>(lane) * 16u;
    // Coalesced: a quad of lanes reads one row's 64 bytes (row lane/4, bytes 16*(lane%4)); the
    // LDS write puts each 16 bytes where the operand layout wants them (x_slot).
    const int row = mt * kWideRows + 16 * (2 * wave + q) + (lane >> 2);
    xo[q] = row < a.M ? static_cast<uint32_t>(static_cast<int64_t>(row) * a.ldx * 2) + 16u * static_cast<uint32_t>(lane & 3)
                      : kOutOfRange;
    xl[q] = 8 * (lane & 3) < a.k_last ? xo[q] : kOutOfRange;  // the last K step: lanes past K
  }
  const int x_slot = 16 * (lane & 3) + (lane >> 2);  // operand lane of row lane/4, K chunk lane%4
  u32x4 rw[kWideStages][2], rx[kWideStages][2];
  // Step index t (relative to s_lo) into register slot t % kWideStages; steps past s_hi load zeros.
  auto load = [&](int t, u32x4 (&w)[2], u32x4 (&x)[2]) {
    const int s = s_lo + t;
    const bool live = s < s_hi;
    const uint32_t sw = live ? pack_step_offset(s, wgroup) : kWideNoLoad;
    const uint32_t sx = live ? static_cast<uint32_t>(s) * 64u : kWideNoLoad;
    const bool last = s == a.Ks - 1;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      w[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, wo[q], static_cast<int>(sw), 0));
      x[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, last ? xl[q] : xo[q], static_cast<int>(sx), 0));
    }
  };
  auto stage = [&](int slot, const u32x4 (&w)[2], const u32x4 (&x)[2]) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      lds[slot][2 * wave + q][lane] = w[q];
      lds[slot][kWideFrags + 2 * wave + q][x_slot] = x[q];
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < kWideStages; ++j) load(j, rw[j], rx[j]);
  stage(0, rw[0], rx[0]);
  load(kWideStages, rw[0], rx[0]);
  for (int t0 = 0; t0 < steps; t0 += kWideStages) {
#pragma unroll
    for (int j = 0; j < kWideStages; ++j) {
      const int t = t0 + j;
      wide_sync();  // slot t&1 holds step t; slot (t+1)&1 is no longer read
      const int jn = j + 1 == kWideStages ? 0 : j + 1;  // a constant once the loop is unrolled
      stage((t + 1) & 1, rw[jn], rx[jn]);
      load(t + 1 + kWideStages, rw[jn], rx[jn]);
      u32x4 A[4], B[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) A[i] = lds[t & 1][4 * wn + i][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) B[i] = lds[t & 1][kWideFrags + 4 * wm + i][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[i][k] = mfma_16x16x32<DT>(A[i], B[k], acc[i][k]);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);

  // Fragment (i, k) of this wavefront: weight rows n0 + 16i + 4*(lane/16) + r, X row m0 + 16k + lane%16.
  const int n0 = nt * kWideRows + 64 * wn + 4 * (lane >> 4);
  const int m0 = mt * kWideRows + 64 * wm + (lane & 15);
  if (a.split == 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int m = m0 + 16 * k, n = n0 + 16 * i;
        if (m < a.M && n < a.N) wide_store4<DT>(a, m, n, acc[i][k]);
      }
    return;
  }
  // Split partial: this wavefront's 16 fp32 fragments (16 KiB), written through.
  const auto prs = make_rsrc(reinterpret_cast<f32x4*>(a.partial) + static_cast<int64_t>(tile) * a.split * kWideWaves * 16 * 64,
                             static_cast<uint32_t>(a.split) * kWideWaves * 16 * 1024u);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int k = 0; k < 4; ++k)
      __builtin_amdgcn_raw_buffer_store_b128(
          __builtin_bit_cast(u32x4, acc[i][k]), prs,
          static_cast<uint32_t>(((sp * kWideWaves + wave) * 16 + 4 * i + k) * 1024 + lane * 16), 0, kCoherent);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int before = __hip_atomic_fetch_add(a.arrive + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_flag = before == a.split - 1;
    if (last_flag) __hip_atomic_store(a.arrive + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last_flag) return;
#pragma unroll 1
  for (int q = 0; q < 16; ++q) {
    const int i = q >> 2, k = q & 3;
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < a.split; ++s0)
      v += __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     prs, static_cast<uint32_t>(((s0 * kWideWaves + wave) * 16 + q) * 1024 + lane * 16), 0, kCoherent));
    const int m = m0 + 16 * k, n = n0 + 16 * i;
    if (m < a.M && n < a.N) wide_store4<DT>(a, m, n, v);
  }
}

int64_t wide_tiles(int64_t M, int64_t N) { return ((N + kWideRows - 1) / kWideRows) * ((M + kWideRows - 1) / kWideRows); }

}  // namespace

int wide_split(int64_t M, int64_t N, int64_t K, int64_t cap) {
  const int64_t tiles = wide_tiles(M, N), ks = (K + 31) / 32;
  const auto bytes = [&](int64_t s) { return static_cast<int64_t>(kCounterBytes) + tiles * s * kWideWaves * 16 * 1024; };
  int64_t split = 1;
  while (tiles * split * 2 <= 320 && ks / (split * 2) >= 16 && split < 8 && bytes(split * 2) <= cap) split *= 2;
  return static_cast<int>(split);
}

int64_t wide_workspace(int64_t M, int64_t N, int64_t K, int64_t cap) {
  const int split = wide_split(M, N, K, cap);
  if (split == 1) return 0;
  return static_cast<int64_t>(kCounterBytes) + wide_tiles(M, N) * split * kWideWaves * 16 * 1024;
}

int wide_gemm(int32_t dtype, const void* x, int64_t ldx, const void* wp, void* y, int64_t ldy, int64_t M, int64_t N,
              int64_t K, void* workspace, size_t workspace_bytes, hipStream_t stream, int out_f32, int64_t cap) {
  WideArgs a{};
  a.x = x;
  a.w = wp;
  a.y = y;
  a.ldx = ldx;
  a.ldy = ldy;
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.Ks = static_cast<int>((K + 31) / 32);
  a.k_last = static_cast<int>(K - 32 * (a.Ks - 1));
  a.mtiles = static_cast<int>((M + kWideRows - 1) / kWideRows);
  a.split = wide_split(M, N, K, cap);
  a.out_f32 = out_f32;
  const int64_t items = wide_tiles(M, N) * a.split;
  if (a.split > 1) {
    const int64_t need = wide_workspace(M, N, K, cap);
    if (workspace == nullptr || static_cast<int64_t>(workspace_bytes) < need ||
        (reinterpret_cast<uintptr_t>(workspace) & 15) != 0)
      return PLM_ERR_WORKSPACE;
    if (wide_tiles(M, N) > kPackedBarrierBase - kPackedArriveBase || need - static_cast<int64_t>(kCounterBytes) >= (int64_t(1) << 31))
      return PLM_ERR_ARGUMENT;
    a.arrive = static_cast<int*>(workspace) + kPackedArriveBase;
    a.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
  }
  if (items > (int64_t(1) << 24) || M * ldx * 2 >= (int64_t(1) << 31)) return PLM_ERR_ARGUMENT;
  if (dtype == PLM_BF16)
    hipLaunchKernelGGL(wide_gemm_kernel<DT_BF16>, dim3(static_cast<unsigned>(items)), dim3(kWideThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(wide_gemm_kernel<DT_F16>, dim3(static_cast<unsigned>(items)), dim3(kWideThreads), 0, stream, a);
  return hipGetLastError() == hipSuccess ? PLM_OK : PLM_ERR_LAUNCH;
}

}  // namespace plm
