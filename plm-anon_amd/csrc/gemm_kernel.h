// Skinny split-K GEMM kernel template for the PLM round's dense linears on gfx950 (MI355X).
//
// Y[M,N] = X[M,K] · W[N,K]^T, fp32 accumulation, Y in the input dtype. M is the round width
// (k verify rows + k^2 proposal tokens: 42 at k=6, 56 at k=7, up to 128), N and K are model
// dimensions, so the weight dominates the bytes and the kernel is an HBM stream of W.
//
// Work decomposition (one launch, no second reduction kernel):
//   * workgroup  = one 16*NF-row tile of W (all M rows of X) x one of `split` K ranges;
//   * wavefront  = one of KW contiguous K slices of that range; it streams its slice of the
//                  weight tile from HBM with 16-byte loads straight into MFMA operands;
//   * LDS        = the KW wavefront partials, summed in wave order;
//   * split > 1  = each workgroup publishes an fp32 partial, the last one of the tile to arrive
//                  (integer counter) sums the partials in split order and writes Y. The sum
//                  order is fixed, so results are bitwise reproducible run to run, as in the
//                  reference's two-kernel split-K (plm/fast_gemm.py:3-4, 48, 51-61).
#pragma once

#include <hip/hip_runtime.h>

#include "plm_amd.h"
#include "tile.h"

namespace plm {

struct GemmArgs {
  const uint16_t* x;
  const uint16_t* w;
  uint16_t* y;
  int64_t ldx, ldw, ldy;
  int M, N, K, split;
  int out_f32;     // 1: Y is fp32 (the unrounded accumulator), 0: Y is in the input dtype
  float* partial;  // [split][M][N] fp32, only when split > 1
  int* counter;    // [n_tiles], zero between launches
};

template <int DT>
__device__ __forceinline__ void store_y(const GemmArgs& a, int64_t idx, float v) {
  if (a.out_f32)
    reinterpret_cast<float*>(a.y)[idx] = v;
  else
    a.y[idx] = to_bits16<DT>(v);
}

template <int DT, int MT, int NF, int U, bool PIPE, int KW>
__global__ __launch_bounds__(64 * KW) void skinny_gemm_kernel(GemmArgs a) {
  extern __shared__ float red[];
  constexpr int TN = 16 * NF;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = blockIdx.x / a.split;
  const int s = blockIdx.x - tile * a.split;
  const int n0 = tile * TN;

  const int tn = min(TN, a.N - n0);
  const auto xr = make_rsrc(a.x, static_cast<uint32_t>(a.M * a.ldx * 2));
  const auto wr = make_rsrc(a.w + static_cast<int64_t>(n0) * a.ldw, static_cast<uint32_t>(tn * a.ldw * 2));
  uint32_t xoff[MT], woff[NF];
  row_offsets<MT>(a.ldx, 0, a.M, lane, xoff);
  row_offsets<NF>(a.ldw, 0, tn, lane, woff);

  int st0, st1;
  k_slice(a.K, s * KW + wave, a.split * KW, st0, st1);
  f32x4 acc[NF][MT];
#pragma unroll
  for (int f = 0; f < NF; ++f)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[f][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  wave_mma<DT, MT, NF, U, PIPE>(xr, xoff, wr, woff, a.K, st0, st1, lane, acc);
  wave_spill<MT, NF>(red, wave, lane, acc);
  __syncthreads();

  const int elems = a.M * TN;
  if (a.split == 1) {
    for (int e = threadIdx.x; e < elems; e += 64 * KW) {
      const int m = e / TN, nl = e - m * TN;
      if (nl < tn) store_y<DT>(a, m * a.ldy + n0 + nl, wg_sum<MT, NF>(red, KW, red_offset<MT, NF>(nl, m)));
    }
    return;
  }

  const int64_t plane = static_cast<int64_t>(a.M) * a.N;
  float* part = a.partial + s * plane;
  for (int e = threadIdx.x; e < elems; e += 64 * KW) {
    const int m = e / TN, nl = e - m * TN;
    if (nl < tn) publish(part + static_cast<int64_t>(m) * a.N + n0 + nl, wg_sum<MT, NF>(red, KW, red_offset<MT, NF>(nl, m)));
  }
  if (!arrive_last(a.counter + tile, a.split)) return;
  for (int e = threadIdx.x; e < elems; e += 64 * KW) {
    const int m = e / TN, nl = e - m * TN;
    if (nl < tn) {
      const int64_t idx = static_cast<int64_t>(m) * a.N + n0 + nl;
      float v = collect(a.partial + idx);
      for (int q = 1; q < a.split; ++q) v += collect(a.partial + q * plane + idx);
      store_y<DT>(a, m * a.ldy + n0 + nl, v);
    }
  }
}

// The compiled tile set. MT = ceil(M/16) is picked from M at run time; PIPE is picked from the
// number of K steps per wavefront (pipelined when a wavefront has more than `unroll` steps).
template <int MT, int NF, int U, bool PIPE, int KW>
constexpr bool gemm_compiled() {
  if (KW != 4 && KW != 8) return false;
  const bool u_ok = PIPE ? (U == 2 || U == 4) : (U == 2 || U == 4 || U == 8);
  if (!u_ok) return false;
  // Register budget: (PIPE ? 2 : 1) * U * (NF + MT) 16-byte operands must fit beside the
  // accumulators without spilling at 256 VGPRs (KW = 8) or 512 (KW = 4).
  const int operand_vgprs = (PIPE ? 2 : 1) * U * (NF + MT) * 4;
  const int acc_vgprs = NF * MT * 4;
  const int budget = KW == 8 ? 256 : 512;
  if (operand_vgprs + acc_vgprs + 24 > budget) return false;
  if (MT <= 4) return NF == 1 || NF == 2 || NF == 4;
  return NF == 1 || NF == 2;
}

template <int DT, int MT, int NF, int U, bool PIPE, int KW>
hipError_t launch_gemm(const GemmArgs& a, hipStream_t stream) {
  auto kern = skinny_gemm_kernel<DT, MT, NF, U, PIPE, KW>;
  constexpr size_t lds = static_cast<size_t>(KW) * NF * MT * 256 * sizeof(float);
  if constexpr (lds > 65536) {
    static const hipError_t attr =
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != hipSuccess) return attr;
  }
  const int n_tiles = (a.N + 16 * NF - 1) / (16 * NF);
  hipLaunchKernelGGL(kern, dim3(n_tiles * a.split), dim3(64 * KW), lds, stream, a);
  return hipGetLastError();
}

template <int DT, int MT, int NF, int U, bool PIPE>
hipError_t pick_kw(const GemmArgs& a, int kw, hipStream_t s, bool dry) {
  switch (kw) {
    case 4:
      if constexpr (gemm_compiled<MT, NF, U, PIPE, 4>()) return dry ? hipSuccess : launch_gemm<DT, MT, NF, U, PIPE, 4>(a, s);
      break;
    case 8:
      if constexpr (gemm_compiled<MT, NF, U, PIPE, 8>()) return dry ? hipSuccess : launch_gemm<DT, MT, NF, U, PIPE, 8>(a, s);
      break;
  }
  return hipErrorInvalidConfiguration;
}

template <int DT, int MT, int NF>
hipError_t pick_u(const GemmArgs& a, int u, bool pipe, int kw, hipStream_t s, bool dry) {
  switch (u) {
    case 2: return pipe ? pick_kw<DT, MT, NF, 2, true>(a, kw, s, dry) : pick_kw<DT, MT, NF, 2, false>(a, kw, s, dry);
    case 4: return pipe ? pick_kw<DT, MT, NF, 4, true>(a, kw, s, dry) : pick_kw<DT, MT, NF, 4, false>(a, kw, s, dry);
    case 8: return pipe ? pick_kw<DT, MT, NF, 8, true>(a, kw, s, dry) : pick_kw<DT, MT, NF, 8, false>(a, kw, s, dry);
  }
  return hipErrorInvalidConfiguration;
}

template <int DT, int MT>
hipError_t pick_nf(const GemmArgs& a, int nf, int u, bool pipe, int kw, hipStream_t s, bool dry) {
  switch (nf) {
    case 1: return pick_u<DT, MT, 1>(a, u, pipe, kw, s, dry);
    case 2: return pick_u<DT, MT, 2>(a, u, pipe, kw, s, dry);
    case 4: return pick_u<DT, MT, 4>(a, u, pipe, kw, s, dry);
  }
  return hipErrorInvalidConfiguration;
}

// True when some wavefront has more K steps than one batch of `unroll`.
inline bool needs_pipeline(const GemmArgs& a, const plm_tile& t) {
  const int64_t steps = (a.K + 31) / 32;
  const int64_t pieces = static_cast<int64_t>(t.split_k) * t.k_waves;
  return (steps + pieces - 1) / pieces > t.unroll;
}

template <int DT>
hipError_t pick_mt(const GemmArgs& a, int mt, const plm_tile& t, hipStream_t s, bool dry) {
  const bool pipe = needs_pipeline(a, t);
  switch (mt) {
    case 1: return pick_nf<DT, 1>(a, t.wave_frags, t.unroll, pipe, t.k_waves, s, dry);
    case 2: return pick_nf<DT, 2>(a, t.wave_frags, t.unroll, pipe, t.k_waves, s, dry);
    case 3: return pick_nf<DT, 3>(a, t.wave_frags, t.unroll, pipe, t.k_waves, s, dry);
    case 4: return pick_nf<DT, 4>(a, t.wave_frags, t.unroll, pipe, t.k_waves, s, dry);
    case 5: return pick_nf<DT, 5>(a, t.wave_frags, t.unroll, pipe, t.k_waves, s, dry);
    case 6: return pick_nf<DT, 6>(a, t.wave_frags, t.unroll, pipe, t.k_waves, s, dry);
    case 7: return pick_nf<DT, 7>(a, t.wave_frags, t.unroll, pipe, t.k_waves, s, dry);
    case 8: return pick_nf<DT, 8>(a, t.wave_frags, t.unroll, pipe, t.k_waves, s, dry);
  }
  return hipErrorInvalidConfiguration;
}

// Launches the compiled kernel for dtype DT matching (M, tile), or reports that none exists
// (dry = true only checks).
template <int DT>
hipError_t gemm_dispatch(const GemmArgs& a, const plm_tile& t, hipStream_t s, bool dry) {
  return pick_mt<DT>(a, (a.M + 15) / 16, t, s, dry);
}

hipError_t gemm_dispatch_bf16(const GemmArgs& a, const plm_tile& t, hipStream_t s, bool dry);
hipError_t gemm_dispatch_f16(const GemmArgs& a, const plm_tile& t, hipStream_t s, bool dry);

}  // namespace plm
