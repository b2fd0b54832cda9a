// Device building blocks shared by the GEMM and the fused LM-head verify kernels.
//
// Orientation: a wavefront computes a slab of Y^T = W · X^T with v_mfma_f32_16x16x32_{bf16,f16}.
// The MFMA's A operand is a 16-row weight fragment (16 rows of W[N,K], the long dimension), its
// B operand a 16-row fragment of X[M,K] (the skinny round dimension). Lane l supplies row l%16
// and the eight K elements [8*(l/16), 8*(l/16)+8) of a 32-wide K step to both operands, so every
// operand is one 16-byte global load per lane, straight from HBM into VGPRs (weights are read
// exactly once and need no LDS staging). Accumulator register r of lane l holds
// D[row = 4*(l/16) + r][col = l%16], i.e. weight row n0 + 16f + 4*(l/16) + r and X row 16t + l%16.
//
// Bit-identity contract: wave_mma() visits K steps in ascending order and wg_sum() adds the
// wavefronts' partials in a fixed order, so any kernel that calls them with the same tile
// geometry and K partition produces the same fp32 value for an element, whatever the other rows
// hold.
// The verify step relies on this to recompute a proposal's own logit outside the main pass.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <stdint.h>

#include "plm_amd.h"

namespace plm {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

enum { DT_BF16 = 0, DT_F16 = 1 };

template <int DT>
__device__ __forceinline__ f32x4 mfma_16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == DT_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

// fp32 -> 16-bit storage, round to nearest even (what torch's .to(bfloat16/float16) does).
template <int DT>
__device__ __forceinline__ uint16_t to_bits16(float v) {
  if constexpr (DT == DT_BF16) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
  } else {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
  }
}

// 16-bit storage -> fp32 (exact).
template <int DT>
__device__ __forceinline__ float from_bits16(uint16_t h) {
  if constexpr (DT == DT_BF16) {
    return __builtin_bit_cast(float, static_cast<uint32_t>(h) << 16);
  } else {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
  }
}

__device__ __forceinline__ float round_through(float v, int mode) {
  if (mode == 1) return static_cast<float>(static_cast<__bf16>(v));
  if (mode == 2) return static_cast<float>(static_cast<_Float16>(v));
  return v;
}

// Buffer resource over `bytes` bytes at `base`. A raw buffer load whose byte offset is at or past
// `bytes` returns zeros, which masks rows past the end of a tile, padded X rows and the K tail
// without branches around the loads.
constexpr uint32_t kOutOfRange = 0x80000000u;
// Cache-policy bit of the buffer intrinsics that makes an access device-coherent (sc1 on gfx950):
// stores are written through the XCD's L2, loads never hit a stale L2 line.
constexpr int kCoherent = 16;
constexpr int kBufferWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                           kBufferWord3);
}

__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 0));
}

// Packed weights (plm_pack_weight). Fragment (f, s) is weight rows [16f, 16f+16) x K [32s, 32s+32),
// 64 lanes x 16 bytes in the MFMA A-operand order. The fragment rows are padded with zero
// fragments to R = a multiple of 16 (every tile's rows then lie inside the weight, whatever its
// height), the K steps to a multiple of 8, and fragment (f, s) lies at
//   (s / 8) * R * 8 KiB + f * 8 KiB + (s % 8) KiB:
// each fragment row keeps 8 KiB of consecutive K steps together, and the next 8 steps of every
// row follow after all rows. The workgroups of a launch stream their own rows at about the same K
// step at once; in this order they read one contiguous stretch per group of steps, where with
// whole rows stored one after the other (2K bytes apart) the same-step reads landed on few HBM
// channels (measured, a plain stream of the 50257-row LM head: 6.2 against 5.4 TB/s; MLP up 4.7
// against 4.3; the other 1.3B block shapes within a few % either way).
constexpr int kPackGroup = 8;      // K steps of a fragment row stored together
constexpr int kPackRowAlign = 16;  // fragment rows padded to a multiple of this
constexpr uint32_t kPackFragBytes = 1024;
__host__ __device__ constexpr int64_t packed_steps(int64_t Ks) { return (Ks + kPackGroup - 1) / kPackGroup * kPackGroup; }
__host__ __device__ constexpr int64_t pack_rows(int64_t N) {
  return ((N + 15) / 16 + kPackRowAlign - 1) / kPackRowAlign * kPackRowAlign;
}
// Bytes of the packed weight of W[N, K] with Ks = ceil(K / 32) K steps.
__host__ __device__ constexpr int64_t pack_bytes(int64_t N, int64_t Ks) { return pack_rows(N) * packed_steps(Ks) * kPackFragBytes; }
// Bytes from one group of K steps (of every row) to the next.
__host__ __device__ constexpr uint32_t pack_group_bytes(int64_t N) {
  return static_cast<uint32_t>(pack_rows(N)) * kPackGroup * kPackFragBytes;
}
// Offset of fragment row f at K step 0, and the offset K step s adds to it.
__host__ __device__ constexpr uint32_t pack_row_offset(int f) { return static_cast<uint32_t>(f) * kPackGroup * kPackFragBytes; }
__host__ __device__ constexpr uint32_t pack_step_offset(int s, uint32_t group_bytes) {
  return (static_cast<uint32_t>(s) / kPackGroup) * group_bytes + (static_cast<uint32_t>(s) % kPackGroup) * kPackFragBytes;
}

// Workspace layout common to every entry point: the counter area (zero between calls), then scratch.
// Ints of the counter area, so that every entry point can share one workspace:
//   0, 1      streaming chain: launch epoch, workgroups exited
//   2         error flag (PLM_WORKSPACE_ERROR_INDEX), any chain
//   8         verify: workgroups finished (packed verify: groups of workgroups finished)
//   10, 11    packed chain: launch epoch (int64)
//   [16, 48)  packed verify: workgroups finished, per group of kVerifyGroupSize
//   [64, 32768)      streaming kernel: split-K arrival counters
//   [32768, 49152)   streaming chain: tile-done flags
//   [49152, 61440)   packed kernel: split-K arrival counters
//   [61440, 65536)   packed chain: progress flags, an int64 per workgroup
constexpr size_t kCounterBytes = PLM_WORKSPACE_COUNTER_BYTES;
constexpr int64_t kMaxCounters = static_cast<int64_t>(kCounterBytes / sizeof(int));
constexpr int kVerifyCounter = 8;
constexpr int kVerifyOwnDone = 9;  // the fused verify's own-logit workgroups that have counted in
constexpr int kVerifyGroupBase = 16;
constexpr int kVerifyGroupSize = 32;
constexpr int kStreamDoneEnd = 32768 + 16384;
constexpr int kPackedArriveBase = 49152;
constexpr int kPackedBarrierBase = 61440;

inline bool aligned16_ptr(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Workgroups of `kern` (with `threads` threads and `dynamic_lds` bytes of dynamic LDS) that one CU
// holds at once: the runtime's occupancy figure, capped by the LDS count with each workgroup's
// LDS (static and dynamic) rounded up to the 512-byte allocation granule. A launch whose
// workgroups wait on each other relies on this count being exact or low, and the runtime's
// figure has been seen to ignore the granule. Returns 0 on error.
inline int resident_per_cu(const void* kern, int threads, size_t dynamic_lds) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, threads, dynamic_lds) != hipSuccess || n < 1) return 0;
  hipFuncAttributes attr{};
  if (hipFuncGetAttributes(&attr, kern) != hipSuccess) return 0;
  int dev = 0, capacity = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&capacity, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess ||
      capacity <= 0)
    capacity = 160 * 1024;
  const size_t per_group = (dynamic_lds + attr.sharedSizeBytes + 511) / 512 * 512;
  if (per_group > 0) n = std::min<int>(n, static_cast<int>(static_cast<size_t>(capacity) / per_group));
  return n;
}

// Cross-workgroup hand-off (split-K partials, per-workgroup row states) without cache-wide
// maintenance. The MI355X has one L2 per XCD and they are not coherent with each other for
// ordinary accesses, which is why __threadfence() costs a full L2 writeback + invalidate in every
// wavefront. Instead the producer writes with device-coherent stores (written through its L2),
// waits for them to complete, and only then counts itself in with a device-scope atomic; the
// consumer reads with device-coherent loads, which never return a stale L2 line.
template <typename T>
__device__ __forceinline__ void publish(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T>
__device__ __forceinline__ T collect(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Called by every thread of the workgroup after its publish() calls. Returns true in the
// workgroup that arrives last out of `expected`; that workgroup also resets the counter to zero
// for the next launch.
__device__ __forceinline__ bool arrive_last(int* counter, int expected) {
  __shared__ int last;
  __builtin_amdgcn_s_waitcnt(0);  // this wavefront's published stores have completed
  __syncthreads();
  if (threadIdx.x == 0) {
    const int before = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = before == expected - 1;
    if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  return last != 0;
}

// Half-open K-step range [st0, st1) of slice `piece` out of `pieces`, over ceil(K/32) steps.
__device__ __forceinline__ void k_slice(int K, int piece, int pieces, int& st0, int& st1) {
  const int steps = (K + 31) >> 5;
  st0 = static_cast<int>((static_cast<int64_t>(piece) * steps) / pieces);
  st1 = static_cast<int>((static_cast<int64_t>(piece + 1) * steps) / pieces);
}

// Per-lane byte offsets of the operand rows this lane feeds. Rows outside [lo, hi) get an
// out-of-range offset and load as zeros.
template <int NROW16>
__device__ __forceinline__ void row_offsets(int64_t ld, int lo, int hi, int lane, uint32_t (&off)[NROW16]) {
  const int row = lane & 15;
  const int kq = (lane >> 4) << 3;
#pragma unroll
  for (int i = 0; i < NROW16; ++i) {
    const int r = 16 * i + row;
    off[i] = (r >= lo && r < hi) ? static_cast<uint32_t>((r * ld + kq) * 2) : kOutOfRange;
  }
}

template <int MT, int NF, int U>
struct Chunk {
  u32x4 w[NF][U];
  u32x4 x[MT][U];
};

// Loads K steps [st, st+n) (n <= U; steps past n are not loaded). Lanes whose K index is past K
// read zeros.
template <int MT, int NF, int U>
__device__ __forceinline__ void load_chunk(Chunk<MT, NF, U>& c, __amdgpu_buffer_rsrc_t xr, const uint32_t (&xoff)[MT],
                                           __amdgpu_buffer_rsrc_t wr, const uint32_t (&woff)[NF], int K, int st,
                                           int n, int lane) {
  const int kq = (lane >> 4) << 3;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (u < n) {
      const int k = (st + u) * 32;
      const uint32_t kb = static_cast<uint32_t>(k) * 2u;
      const bool kin = k + kq < K;
#pragma unroll
      for (int f = 0; f < NF; ++f) c.w[f][u] = buffer_load16(wr, kin ? woff[f] + kb : kOutOfRange);
#pragma unroll
      for (int t = 0; t < MT; ++t) c.x[t][u] = buffer_load16(xr, kin ? xoff[t] + kb : kOutOfRange);
    }
  }
}

template <int DT, int MT, int NF, int U>
__device__ __forceinline__ void mma_chunk(const Chunk<MT, NF, U>& c, int n, f32x4 (&acc)[NF][MT]) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (u < n) {
#pragma unroll
      for (int f = 0; f < NF; ++f)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[f][t] = mfma_16x16x32<DT>(c.w[f][u], c.x[t][u], acc[f][t]);
    }
  }
}

// acc[f][t] += Wtile[16f .. 16f+16, steps] · X[16t .. 16t+16, steps]^T over K steps [st0, st1),
// in ascending step order. `wr` covers the weight tile (rows past its end read as zeros), `xr`
// covers X. st0/st1 must be wave-uniform.
//   PIPE = false: batches of U steps, each loaded in full before its MFMAs (one register buffer;
//                 the right choice when a wavefront's slice is at most U steps).
//   PIPE = true : two register buffers; the next batch's loads are in flight while the current
//                 batch's MFMAs run, so long slices stream without a latency bubble per batch.
template <int DT, int MT, int NF, int U, bool PIPE>
__device__ __forceinline__ void wave_mma(__amdgpu_buffer_rsrc_t xr, const uint32_t (&xoff)[MT],
                                         __amdgpu_buffer_rsrc_t wr, const uint32_t (&woff)[NF], int K, int st0,
                                         int st1, int lane, f32x4 (&acc)[NF][MT]) {
  int st = st0;
  int left = st1 - st0;
  if constexpr (!PIPE) {
    Chunk<MT, NF, U> c;
    while (left > 0) {
      const int n = left < U ? left : U;
      load_chunk<MT, NF, U>(c, xr, xoff, wr, woff, K, st, n, lane);
      mma_chunk<DT, MT, NF, U>(c, n, acc);
      st += n;
      left -= n;
    }
  } else {
    if (left <= 0) return;
    Chunk<MT, NF, U> ca, cb;
    int na = left < U ? left : U;
    load_chunk<MT, NF, U>(ca, xr, xoff, wr, woff, K, st, na, lane);
    while (true) {
      st += na;
      left -= na;
      const int nb = left < U ? left : U;
      if (nb > 0) load_chunk<MT, NF, U>(cb, xr, xoff, wr, woff, K, st, nb, lane);
      mma_chunk<DT, MT, NF, U>(ca, na, acc);
      if (nb <= 0) break;
      st += nb;
      left -= nb;
      na = left < U ? left : U;
      if (na > 0) load_chunk<MT, NF, U>(ca, xr, xoff, wr, woff, K, st, na, lane);
      mma_chunk<DT, MT, NF, U>(cb, nb, acc);
      if (na <= 0) break;
    }
  }
}

// LDS layout of the wavefront partials: red[((w*NF*MT + f*MT + t)*4 + r)*64 + lane].
template <int MT, int NF>
__device__ __forceinline__ void wave_spill(float* red, int wave, int lane, const f32x4 (&acc)[NF][MT]) {
#pragma unroll
  for (int f = 0; f < NF; ++f)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[((wave * NF * MT + f * MT + t) * 4 + r) * 64 + lane] = acc[f][t][r];
}

// LDS offset (within one wavefront's block) of tile element (n_local, m_local).
template <int MT, int NF>
__device__ __forceinline__ int red_offset(int n_local, int m_local) {
  const int f = n_local >> 4, i = n_local & 15, t = m_local >> 4, mm = m_local & 15;
  return ((f * MT + t) * 4 + (i & 3)) * 64 + (i >> 2) * 16 + mm;
}

// Sum of the wavefronts' partials of one element, in wave order starting from the first: the order
// in which the streaming GEMM's split-K combine adds the partials of the same K slices, so the
// verify step's logits are bit for bit plm_gemm_f32out's with split_k = k_waves.
template <int MT, int NF>
__device__ __forceinline__ float wg_sum(const float* red, int k_waves, int off) {
  constexpr int per_wave = NF * MT * 256;
  float s = red[off];
  for (int w = 1; w < k_waves; ++w) s += red[w * per_wave + off];
  return s;
}

}  // namespace plm
