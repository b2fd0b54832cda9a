// Fused LM-head verify step on gfx950: logits = X · W^T, then per row softmax statistics, argmax
// and top-p nucleus membership of the proposed ids, without writing the logits to memory.
//
// Reference semantics (plm/decoder.py:71-75, 351-362):
//   probs  = softmax(logits.float()); own = probs[pending]
//   accept = sum(probs * (probs > own)) < p  |  (own >= max(probs) & p > 0)
//   argmax = logits.argmax(-1)   (lowest index among equal maxima)
// Restated over logits l with row maximum mx and e_j = exp(l_j - mx):
//   accept = (sum_{j: l_j > l_own} e_j) / (sum_j e_j) < p  |  (l_own >= mx & p > 0)
// exp is monotone, so "probs > own" and "l > l_own" select the same set except where exp/divide
// rounding makes two distinct logits produce equal probabilities.
// The floor rule (plm/decoder.py:78-82), accept = l_own - logsumexp(l) > log(eps), reads the same
// row state: logsumexp(l) = mx + log(sum_j e_j).
//
// Two launches:
//   1. own_logit_kernel: one workgroup per row r recomputes the single logit l[r, pending[r]] with
//      the same tile geometry, K partition and reduction order as the main pass, so the value is
//      bit-identical to the one the main pass forms for that column.
//   2. verify_main_kernel: G workgroups, each streaming tiles b, b+G, b+2G, ... of W. For every
//      tile it forms the [TN x R] logits in LDS, then each row's tile max / argmax / sum of
//      exponentials / sum above l_own, merged into a running per-row state (online rescaling).
//      The states go to the workspace; the last workgroup to finish (integer counter) merges them
//      in a fixed tree and writes accept[] and argmax[]. No float atomics; bitwise reproducible.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>

#include "epilogue.h"
#include "packed_gemm.h"
#include "plm_amd.h"
#include "tile.h"

namespace plm {

struct VerifyArgs {
  const uint16_t* x;
  const uint16_t* w;
  int64_t ldx, ldw;
  int R, V, K, G;
  const int64_t* pending;
  int pending_rows;  // rows r >= pending_rows propose no id (never accepted)
  float p;           // top-p for PLM_RULE_NUCLEUS, epsilon for PLM_RULE_FLOOR
  int rule;
  int round_mode;
  uint8_t* accept;
  int64_t* argmax;
  int* counter;      // [1], zero between launches
  float* own;        // [R]
  float* state;      // [G][R][3]: row max, sum of exp, sum of exp above own
  int* state_idx;    // [G][R]: argmax
  int* group_counter;  // packed verify: [G / kVerifyGroupSize], zero between launches
  float* gstate;       // packed verify: [groups][R][3], the merged state of each group
  int* gstate_idx;     // packed verify: [groups][R]
  // Packed verify: the row states as 16-byte records {max, sum, sum above own, argmax bits}, one
  // coherent store each and one coherent load each per merge: rec[G][R] over the state and
  // state_idx areas, grec[groups][R] over gstate and gstate_idx.
  f32x4* rec;
  f32x4* grec;
  RoundEpilogue round;  // packed verify: k > 0 runs the round's epilogue after the last merge
  uint16_t* logits;     // packed verify: rows [0, logit_rows) of the logits in the model dtype, or null
  int64_t ld_logits;
  int logit_rows;
  // packed verify: the first own_groups workgroups compute the proposals' own logits (four rows
  // each) and count themselves into *own_done; the others wait for that count before their first
  // fold (bounded; a wait that gives up sets *error).
  int own_groups;
  int* own_done;
  int* error;
};

// Online-softmax state of one row: maximum, sum of exp(l - max), sum of exp(l - max) over l > l_own,
// and the lowest index attaining the maximum. merge() is commutative bit for bit (no contraction,
// symmetric formulas), so a butterfly over lanes leaves every lane with the same result.
struct RowState {
  float mx, se, ab;
  int ai;
};

__device__ __forceinline__ RowState empty_state() { return RowState{-INFINITY, 0.f, 0.f, INT_MAX}; }

// The acceptance decision for a proposal with logit `own` (NaN: not a vocabulary id, never
// accepted) in a row with merged state t.
__device__ __forceinline__ bool accept_proposal(const VerifyArgs& a, float own, const RowState& t) {
  if (!(own == own)) return false;
  if (a.rule == PLM_RULE_FLOOR) return (own - (t.mx + logf(t.se))) > logf(a.p);
  const bool in_nucleus = (t.ab / t.se) < a.p;
  const bool is_max = (own >= t.mx) && (a.p > 0.f);
  return in_nucleus || is_max;
}

// e^d for d = a logit less its row's maximum (d <= 0): the hardware exp2 of d log2(e), exactly 1 at
// d = 0; its error is about an ulp where the terms matter (|d| small) and grows with |d| only
// for terms far below the row's largest.
__device__ __forceinline__ float exp_below_max(float d) { return __builtin_amdgcn_exp2f(d * 1.4426950408889634f); }

// An empty state (maximum -inf) leaves the other unchanged; selects rather than branches, as the
// lanes of a wavefront merge states of different rows.
#pragma clang fp contract(off)
__device__ __forceinline__ RowState merge(RowState a, RowState b) {
  RowState r;
  r.ai = (b.mx > a.mx || (b.mx == a.mx && b.ai < a.ai)) ? b.ai : a.ai;
  const float mx = fmaxf(a.mx, b.mx);
  const float fa = exp_below_max(a.mx - mx), fb = exp_below_max(b.mx - mx);
  const float se = a.se * fa + b.se * fb;
  const float ab = a.ab * fa + b.ab * fb;
  const bool a_empty = a.mx == -INFINITY, b_empty = b.mx == -INFINITY;
  r.mx = b_empty ? a.mx : (a_empty ? b.mx : mx);
  r.se = b_empty ? a.se : (a_empty ? b.se : se);
  r.ab = b_empty ? a.ab : (a_empty ? b.ab : ab);
  return r;
}
#pragma clang fp contract(on)

__device__ __forceinline__ RowState shfl_xor_state(const RowState& s, int off) {
  return RowState{__shfl_xor(s.mx, off, 64), __shfl_xor(s.se, off, 64), __shfl_xor(s.ab, off, 64),
                  __shfl_xor(s.ai, off, 64)};
}

__device__ __forceinline__ RowState wave_merge(RowState s) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s = merge(s, shfl_xor_state(s, off));
  return s;
}

template <int DT, int MT, int NF, int U, bool PIPE, int KW>
__global__ __launch_bounds__(64 * KW) void own_logit_kernel(VerifyArgs a) {
  extern __shared__ float red[];
  constexpr int TN = 16 * NF;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = blockIdx.x;
  const int64_t pid64 = r < a.pending_rows ? a.pending[r] : -1;
  if (pid64 < 0 || pid64 >= a.V) {  // not a vocabulary id: no logit, and the row accepts nothing
    if (threadIdx.x == 0) a.own[r] = NAN;
    return;
  }
  const int pid = static_cast<int>(pid64);
  const int n0 = (pid / TN) * TN;
  const int tn = min(TN, a.V - n0);
  const auto xr = make_rsrc(a.x, static_cast<uint32_t>(a.R * a.ldx * 2));
  const auto wr = make_rsrc(a.w + static_cast<int64_t>(n0) * a.ldw, static_cast<uint32_t>(tn * a.ldw * 2));
  uint32_t xoff[MT], woff[NF];
  row_offsets<MT>(a.ldx, r, r + 1, lane, xoff);
  row_offsets<NF>(a.ldw, pid - n0, pid - n0 + 1, lane, woff);
  int st0, st1;
  k_slice(a.K, wave, KW, st0, st1);
  f32x4 acc[NF][MT];
#pragma unroll
  for (int f = 0; f < NF; ++f)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[f][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  wave_mma<DT, MT, NF, U, PIPE>(xr, xoff, wr, woff, a.K, st0, st1, lane, acc);
  wave_spill<MT, NF>(red, wave, lane, acc);
  __syncthreads();
  if (threadIdx.x == 0) a.own[r] = round_through(wg_sum<MT, NF>(red, KW, red_offset<MT, NF>(pid - n0, r)), a.round_mode);
}

template <int DT, int MT, int NF, int U, bool PIPE, int KW>
__global__ __launch_bounds__(64 * KW) void verify_main_kernel(VerifyArgs a) {
  extern __shared__ float red[];
  constexpr int TN = 16 * NF;
  static_assert(TN <= 64, "one lane per tile column");
  constexpr int RPW = (16 * MT + KW - 1) / KW;  // rows of X per wavefront in the epilogue
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n_tiles = (a.V + TN - 1) / TN;

  const auto xr = make_rsrc(a.x, static_cast<uint32_t>(a.R * a.ldx * 2));
  uint32_t xoff[MT];
  row_offsets<MT>(a.ldx, 0, a.R, lane, xoff);
  int st0, st1;
  k_slice(a.K, wave, KW, st0, st1);

  RowState rs[RPW];
  float own_l[RPW];
#pragma unroll
  for (int j = 0; j < RPW; ++j) {
    rs[j] = empty_state();
    const int m = wave + KW * j;
    own_l[j] = m < a.R ? a.own[m] : 0.f;
  }

  for (int tile = blockIdx.x; tile < n_tiles; tile += a.G) {
    const int n0 = tile * TN;
    const int tn = min(TN, a.V - n0);
    const auto wr = make_rsrc(a.w + static_cast<int64_t>(n0) * a.ldw, static_cast<uint32_t>(tn * a.ldw * 2));
    uint32_t woff[NF];
    row_offsets<NF>(a.ldw, 0, tn, lane, woff);
    f32x4 acc[NF][MT];
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[f][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    wave_mma<DT, MT, NF, U, PIPE>(xr, xoff, wr, woff, a.K, st0, st1, lane, acc);
    __syncthreads();  // the previous tile's epilogue has finished reading LDS
    wave_spill<MT, NF>(red, wave, lane, acc);
    __syncthreads();
    const bool valid = lane < tn;
    const int col = valid ? lane : 0;  // lanes past the tile read column 0 and discard it
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
      const int m = wave + KW * j;
      if (m < a.R) {
        const float lv = round_through(wg_sum<MT, NF>(red, KW, red_offset<MT, NF>(col, m)), a.round_mode);
        const float l = valid ? lv : -INFINITY;
        // Tile maximum with lowest-index tie-break, then the two exponential sums against it.
        RowState t{l, 0.f, 0.f, valid ? n0 + lane : INT_MAX};
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
          const float omx = __shfl_xor(t.mx, off, 64);
          const int oai = __shfl_xor(t.ai, off, 64);
          if (omx > t.mx || (omx == t.mx && oai < t.ai)) {
            t.mx = omx;
            t.ai = oai;
          }
        }
        float e = valid ? exp_below_max(l - t.mx) : 0.f;
        float ab = (valid && l > own_l[j]) ? e : 0.f;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
          e += __shfl_xor(e, off, 64);
          ab += __shfl_xor(ab, off, 64);
        }
        t.se = e;
        t.ab = ab;
        rs[j] = merge(rs[j], t);
      }
    }
  }

  // Publish this workgroup's row states.
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
      const int m = wave + KW * j;
      if (m < a.R) {
        const int64_t slot = static_cast<int64_t>(blockIdx.x) * a.R + m;
        publish(a.state + slot * 3 + 0, rs[j].mx);
        publish(a.state + slot * 3 + 1, rs[j].se);
        publish(a.state + slot * 3 + 2, rs[j].ab);
        publish(a.state_idx + slot, rs[j].ai);
      }
    }
  }
  if (!arrive_last(a.counter, a.G)) return;

  // Last workgroup: merge the G states of every row (lane-strided, then a butterfly).
  for (int j = 0; j < RPW; ++j) {
    const int m = wave + KW * j;
    if (m >= a.R) continue;
    RowState s = empty_state();
    for (int g = lane; g < a.G; g += 64) {
      const int64_t slot = static_cast<int64_t>(g) * a.R + m;
      s = merge(s, RowState{collect(a.state + slot * 3 + 0), collect(a.state + slot * 3 + 1),
                            collect(a.state + slot * 3 + 2), collect(a.state_idx + slot)});
    }
    s = wave_merge(s);
    if (lane == 0) {
      a.accept[m] = accept_proposal(a, a.own[m], s) ? 1 : 0;
      a.argmax[m] = s.ai;
    }
  }
}

template <int MT, int NF, int U, bool PIPE, int KW>
constexpr bool verify_compiled() {
  if (KW != 4) return false;  // the K partition of the streaming GEMM (plm_gemm_f32out gives the same logits)
  if (NF != 2 && NF != 4) return false;
  if (MT < 1 || MT > 4) return false;
  const bool u_ok = PIPE ? (U == 2 || U == 4) : (U == 4 || U == 8);
  if (!u_ok) return false;
  const int operand_vgprs = (PIPE ? 2 : 1) * U * (NF + MT) * 4;
  const int budget = KW == 8 ? 256 : 512;
  return operand_vgprs + NF * MT * 4 + 80 <= budget;
}

constexpr int kMaxVerifyGroups = 1024;

template <int DT, int MT, int NF, int U, bool PIPE, int KW>
hipError_t launch_verify(VerifyArgs a, int cu_count, hipStream_t stream, bool dry) {
  if constexpr (!verify_compiled<MT, NF, U, PIPE, KW>()) {
    return hipErrorInvalidConfiguration;
  } else {
    if (dry) return hipSuccess;
    auto own_kern = own_logit_kernel<DT, MT, NF, U, PIPE, KW>;
    auto main_kern = verify_main_kernel<DT, MT, NF, U, PIPE, KW>;
    constexpr size_t lds = static_cast<size_t>(KW) * NF * MT * 256 * sizeof(float);
    if constexpr (lds > 65536) {
      static const hipError_t attr1 =
          hipFuncSetAttribute(reinterpret_cast<const void*>(own_kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
      static const hipError_t attr2 =
          hipFuncSetAttribute(reinterpret_cast<const void*>(main_kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
      if (attr1 != hipSuccess) return attr1;
      if (attr2 != hipSuccess) return attr2;
    }
    static int per_cu = 0;
    if (per_cu == 0) {
      int blocks = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, reinterpret_cast<const void*>(main_kern), 64 * KW, lds) !=
              hipSuccess ||
          blocks < 1)
        blocks = 1;
      per_cu = blocks;
    }
    const int n_tiles = (a.V + 16 * NF - 1) / (16 * NF);
    a.G = min(n_tiles, min(kMaxVerifyGroups, cu_count * per_cu));
    hipLaunchKernelGGL(own_kern, dim3(a.R), dim3(64 * KW), lds, stream, a);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(main_kern, dim3(a.G), dim3(64 * KW), lds, stream, a);
    return hipGetLastError();
  }
}

template <int DT, int MT, int NF>
hipError_t verify_pick_u(const VerifyArgs& a, const plm_tile& t, bool pipe, int cu, hipStream_t s, bool dry) {
#define PLM_VERIFY_KW(U_, P_)                                                        \
  if (t.unroll == U_ && pipe == P_) {                                                \
    if (t.k_waves == 4) return launch_verify<DT, MT, NF, U_, P_, 4>(a, cu, s, dry);  \
  }
  PLM_VERIFY_KW(2, true)
  PLM_VERIFY_KW(4, true)
  PLM_VERIFY_KW(4, false)
  PLM_VERIFY_KW(8, false)
#undef PLM_VERIFY_KW
  return hipErrorInvalidConfiguration;
}

template <int DT>
hipError_t verify_dispatch(const VerifyArgs& a, const plm_tile& t, int cu, hipStream_t s, bool dry) {
  const int64_t steps = (a.K + 31) / 32;
  const bool pipe = (steps + t.k_waves - 1) / t.k_waves > t.unroll;
  const int mt = (a.R + 15) / 16;
#define PLM_VERIFY_NF(MT_)                                                  \
  if (mt == MT_) {                                                          \
    if (t.wave_frags == 2) return verify_pick_u<DT, MT_, 2>(a, t, pipe, cu, s, dry); \
    if (t.wave_frags == 4) return verify_pick_u<DT, MT_, 4>(a, t, pipe, cu, s, dry); \
  }
  PLM_VERIFY_NF(1)
  PLM_VERIFY_NF(2)
  PLM_VERIFY_NF(3)
  PLM_VERIFY_NF(4)
#undef PLM_VERIFY_NF
  return hipErrorInvalidConfiguration;
}

// ---------------------------------------------------------------------------------------------
// The same step over packed weights (plm_pack_weight), on the packed GEMM's row-split pipeline
// (csrc/packed_gemm.h, KW = 1): a workgroup's four wavefronts each own 16*NF vocabulary rows of a
// 64*NF-row tile over the whole K range, share one copy of X through LDS, and accumulate every
// logit in one MFMA chain over the K steps in ascending order. No cross-wavefront reduction is
// needed, so each wavefront folds its own logits into per-row states right after its K steps.
//
// The proposal logit of row r is recomputed by one wavefront with exactly that MFMA chain (the
// packed fragment row holding pending[r] as A, row r's X fragment as B, K steps ascending), which
// makes it bit-identical to the main pass's value for that column; plm_gemm_packed_f32out with a
// row-split tile (k_waves = 1, split_k = 1) returns the same logits. It runs in the same launch:
// the first ceil(R / 4) workgroups compute four proposals each (one per wavefront) and count
// themselves in; the main workgroups need the proposals' logits only at their first fold, after
// streaming their first tile, and wait for that count there.

// One wavefront per row: own[r] = logit[r, pending[r]] (NaN for an id outside [0, V)), `D` K steps of
// loads in flight. Written device-coherently: in the fused verify the main workgroups read it.
template <int DT, int D>
__device__ __forceinline__ void own_logit_wave(const VerifyArgs& a, int r, int lane) {
  const int64_t pid64 = r < a.pending_rows ? a.pending[r] : -1;
  if (pid64 < 0 || pid64 >= a.V) {
    if (lane == 0) publish(a.own + r, NAN);
    return;
  }
  // The same in every lane (row r is the wavefront's): made a scalar so that the weight's buffer
  // resource is one, and its loads are not wrapped in loops over the lanes' values.
  const int pid = __builtin_amdgcn_readfirstlane(static_cast<int>(pid64));
  const int Ks = (a.K + 31) >> 5;
  const int k_last = a.K - 32 * (Ks - 1);
  // The packed fragment row (16 vocabulary rows) holding pid, and row r's X fragment in the MFMA
  // operand order: lane l = X row 16*(r/16) + l%16, K elements 8*(l/16) .. +8 of each step.
  const uint32_t wgroup = pack_group_bytes(a.V);
  const auto wr = make_rsrc(a.w, static_cast<uint32_t>(pack_bytes(a.V, Ks)));
  const auto xr = make_rsrc(a.x, static_cast<uint32_t>(a.R * a.ldx * 2));
  const int xrow = 16 * (r >> 4) + (lane & 15);
  const uint32_t xo = xrow < a.R ? static_cast<uint32_t>(xrow * a.ldx * 2 + (lane >> 4) * 16) : kOutOfRange;
  const uint32_t xo_last = 8 * (lane >> 4) < k_last ? xo : kOutOfRange;
  const uint32_t wo = pack_row_offset(pid >> 4) + static_cast<uint32_t>(lane * 16);
  u32x4 wb[D], xb[D];
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const bool live = j < Ks;
    wb[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                          wr, wo, static_cast<int>(live ? pack_step_offset(j, wgroup) : kNoLoad), 0));
    xb[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                          xr, j == Ks - 1 ? xo_last : xo, static_cast<int>(live ? j * 64 : kNoLoad), 0));
  }
  for (int s0 = 0; s0 < Ks; s0 += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      acc = mfma_16x16x32<DT>(wb[j], xb[j], acc);
      const int n = s0 + D + j;
      const bool live = n < Ks;
      wb[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            wr, wo, static_cast<int>(live ? pack_step_offset(n, wgroup) : kNoLoad), 0));
      xb[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            xr, n == Ks - 1 ? xo_last : xo, static_cast<int>(live ? n * 64 : kNoLoad), 0));
    }
  }
  // Element (vocabulary row pid%16, column r%16) of the 16x16 result: lane r%16 + 16*((pid%16)/4),
  // component pid%4.
  const int v = pid & 15;
  if (lane == (r & 15) + 16 * (v >> 2)) publish(a.own + r, round_through(acc[v & 3], a.round_mode));
}

// K steps in flight in the fused verify's own-logit workgroups (the main kernel's register budget
// has room for 16 at every compiled tile).
constexpr int kOwnDepth = 16;

// The fused prologue: workgroup g < own_groups computes rows 4g .. 4g+3, one per wavefront, then
// counts itself in once its stores have completed.
template <int DT>
__device__ __forceinline__ void own_logit_group(const VerifyArgs& a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = 4 * static_cast<int>(blockIdx.x) + wave;
  if (r < a.R) own_logit_wave<DT, kOwnDepth>(a, r, lane);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(a.own_done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Polls before a main workgroup gives up waiting for the own logits (several seconds).
constexpr int kOwnSpinLimit = 1 << 22;

__device__ __forceinline__ void wait_own_logits(const VerifyArgs& a) {
  for (int i = 0;; ++i) {
    if (__builtin_amdgcn_readfirstlane(collect(a.own_done)) >= a.own_groups) return;
    if (i >= kOwnSpinLimit) {
      if ((threadIdx.x & 63) == 0) publish(a.error, 1);
      return;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// The final merges run once per launch, on its critical path, so their code is kept short (rolled
// loops: code executed once is fetched cold) and their loads are issued in one batch.
//
// gather_records: the workgroup's threads load member (first + i), i < count <= 32, of every row
// (device-coherent: other workgroups wrote them) into grid[i][m] in LDS; absent entries are left
// unread.
__device__ __forceinline__ void gather_records(const f32x4* rec, int first, int count, int R, f32x4* grid) {
  const auto rr = make_rsrc(rec, static_cast<uint32_t>(first + kVerifyGroupSize) * R * sizeof(f32x4));
  constexpr int kPer = kVerifyGroupSize * 64 / (64 * kPackedWaves);  // entries per thread
  f32x4 v[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int i = static_cast<int>(threadIdx.x) + 64 * kPackedWaves * k;
    const int mem = i >> 6, m = i & 63;
    const bool ok = mem < count && m < R;
    const uint32_t slot = static_cast<uint32_t>((first + mem) * R + m);
    v[k] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rr, ok ? slot * 16 : kOutOfRange, 0, kCoherent));
  }
#pragma unroll
  for (int k = 0; k < kPer; ++k) grid[static_cast<int>(threadIdx.x) + 64 * kPackedWaves * k] = v[k];
  __syncthreads();
}

// Record `slot` of `slots` set to s, written device-coherent (read by gather_records in another
// workgroup).
__device__ __forceinline__ void publish_record(f32x4* rec, int slot, int slots, const RowState& s) {
  const auto rr = make_rsrc(rec, static_cast<uint32_t>(slots) * sizeof(f32x4));
  const f32x4 v{s.mx, s.se, s.ab, __builtin_bit_cast(float, s.ai)};
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rr, static_cast<uint32_t>(slot) * 16, 0, kCoherent);
}

// Every row's state merged over members 0..count-1 of grid: lane = row; wavefront w merges
// members [8w, 8w+8) in order, then wavefront 0 merges the four partial states in wavefront order
// (through the part_* LDS arrays). The result is valid in wavefront 0, lanes < R.
__device__ __forceinline__ RowState merge_rows(const f32x4* grid, int count, int wave, int lane,
                                               float (*part_mx)[64], float (*part_se)[64], float (*part_ab)[64],
                                               int (*part_ai)[64]) {
  constexpr int kPerWave = kVerifyGroupSize / kPackedWaves;
  RowState s = empty_state();
  const int n = count - wave * kPerWave;  // members of this wavefront (the rest of grid is unread)
  f32x4 g[kPerWave];
#pragma unroll
  for (int j = 0; j < kPerWave; ++j) g[j] = grid[(wave * kPerWave + j) * 64 + lane];
#pragma unroll
  for (int j = 0; j < kPerWave; ++j) {
    if (j >= n) break;
    const float idx_bits = g[j][3];  // (a bit cast applied to the vector element itself read element 0)
    s = merge(s, RowState{g[j][0], g[j][1], g[j][2], __builtin_bit_cast(int, idx_bits)});
  }
  part_mx[wave][lane] = s.mx;
  part_se[wave][lane] = s.se;
  part_ab[wave][lane] = s.ab;
  part_ai[wave][lane] = s.ai;
  __syncthreads();
  if (wave == 0) {
#pragma unroll 1
    for (int w = 1; w < kPackedWaves; ++w)
      s = merge(s, RowState{part_mx[w][lane], part_se[w][lane], part_ab[w][lane], part_ai[w][lane]});
  }
  return s;
}

// Folds a wavefront's logits into its row states: column n holds vocabulary rows
// n0 + 16f + i of acc[f][t][i] for row 16t + lane%16; the four lanes of a row (lane%16 equal)
// combine through two butterflies. Tile maximum with lowest-index ties, then the two exponential
// sums against it, merged into the running state.
template <int MODE>
__device__ __forceinline__ float round_logit(float v) {
  if constexpr (MODE == PLM_ROUND_BF16) return static_cast<float>(static_cast<__bf16>(v));
  if constexpr (MODE == PLM_ROUND_F16) return static_cast<float>(static_cast<_Float16>(v));
  return v;
}

// Branch-free: a lane visits its columns in increasing order, so a strict comparison keeps the
// lowest index among its equal maxima (NaN never wins). With CHECK (a wavefront whose columns run
// past V: the last tile) columns past V read as -inf, which neither wins nor adds: e^(-inf - mx) = 0
// once the row maximum is finite, and a row whose maximum is -inf is not merged.
template <int MT, int NF, int MODE, bool CHECK>
__device__ __forceinline__ void fold_columns(const f32x4 (&acc)[NF][MT], int n0, int V, const float (&own_l)[MT],
                                             RowState (&rs)[MT]) {
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    float lv[NF][4];
    float mx = -INFINITY;
    int ai = INT_MAX;
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = n0 + 16 * f + i;
        float l = round_logit<MODE>(acc[f][t][i]);
        if constexpr (CHECK) l = n < V ? l : -INFINITY;
        lv[f][i] = l;
        const bool up = l > mx;
        mx = up ? l : mx;
        ai = up ? n : ai;
      }
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
      const float omx = __shfl_xor(mx, off, 64);
      const int oai = __shfl_xor(ai, off, 64);
      const bool take = omx > mx || (omx == mx && oai < ai);
      mx = take ? omx : mx;
      ai = take ? oai : ai;
    }
    float e = 0.f, ab = 0.f;
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float l = lv[f][i];
        const float ex = exp_below_max(l - mx);
        e += ex;
        ab += l > own_l[t] ? ex : 0.f;
      }
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
      e += __shfl_xor(e, off, 64);
      ab += __shfl_xor(ab, off, 64);
    }
    if (mx != -INFINITY) rs[t] = merge(rs[t], RowState{mx, e, ab, ai});
  }
}

// Writes the logits of rows [0, logit_rows) that this wavefront's accumulators hold, rounded to the
// model dtype (the values the decision reads when the round mode is the model dtype's): lane l
// holds vocabulary rows n0 + 16f + i, i = 0..3, of row 16t + l%16, one 8-byte store each.
template <int DT, int MT, int NF>
__device__ __forceinline__ void store_logits(const f32x4 (&acc)[NF][MT], int n0, const VerifyArgs& a) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    if (16 * t >= a.logit_rows) break;
    const int m = 16 * t + (lane & 15);
    if (m >= a.logit_rows) continue;
    uint16_t* dst = a.logits + static_cast<int64_t>(m) * a.ld_logits;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const int n = n0 + 16 * f;
      if (n + 3 < a.V) {
        u32x2 v;
        v[0] = static_cast<uint32_t>(to_bits16<DT>(acc[f][t][0])) | (static_cast<uint32_t>(to_bits16<DT>(acc[f][t][1])) << 16);
        v[1] = static_cast<uint32_t>(to_bits16<DT>(acc[f][t][2])) | (static_cast<uint32_t>(to_bits16<DT>(acc[f][t][3])) << 16);
        *reinterpret_cast<u32x2*>(dst + n) = v;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (n + i < a.V) dst[n + i] = to_bits16<DT>(acc[f][t][i]);
      }
    }
  }
}

template <int MT, int NF, int D>
constexpr bool verify_packed_compiled() {
  return MT >= 1 && MT <= 4 && (NF == 2 || NF == 4) && (D == 2 || D == 4 || D == 8) && packed_compiled<MT, NF, D, 1>();
}

template <int DT, int MT, int NF, int D>
__global__ __launch_bounds__(64 * kPackedWaves, (packed_waves_per_simd<MT, NF, D, 1>())) void verify_packed_main_kernel(
    VerifyArgs a) {
  if (static_cast<int>(blockIdx.x) < a.own_groups) {
    own_logit_group<DT>(a);
    return;
  }
  const int b = static_cast<int>(blockIdx.x) - a.own_groups;  // this workgroup among the main ones
  constexpr int KW = 1;
  constexpr int XN = x_per_wave<MT, KW>();
  __shared__ float st_mx[kPackedWaves][64], st_se[kPackedWaves][64], st_ab[kPackedWaves][64];
  __shared__ int st_ai[kPackedWaves][64];
  __shared__ f32x4 grid[kVerifyGroupSize * 64];  // final merges: [member][row]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  char* xt = reinterpret_cast<char*>(packed_lds);
  const int xt_write = x_tile_write_offset<true>(lane);
  const int xt_read = x_tile_read_offset<true>(lane);

  PLinear L{};
  L.x = a.x;
  L.wp = a.w;
  L.ldx = a.ldx;
  L.N = a.V;
  L.Ks = (a.K + 31) >> 5;
  L.k_last = a.K - 32 * (L.Ks - 1);
  L.wgroup = pack_group_bytes(a.V);
  L.split = 1;
  L.tiles = (((a.V + 15) >> 4) + tile_frags<NF, KW>() - 1) / tile_frags<NF, KW>();
  L.items = L.tiles;
  POffsets<MT, NF, XN> o;
  packed_offsets<MT, NF, KW>(L, a.R, lane, wave, o);
  const auto wr = make_rsrc(L.wp, static_cast<uint32_t>(pack_bytes(L.N, L.Ks)));
  const auto xr = make_rsrc(L.x, static_cast<uint32_t>(a.R * L.ldx * 2));

  // Row states of the rows this lane's accumulators hold: row 16t + lane%16.
  RowState rs[MT];
  float own_l[MT];
  // Own logits: already there when a separate pass ran first, else read at the first fold, after
  // the own-logit workgroups have counted in (they run while this workgroup streams its first tile).
  bool own_ready = a.own_groups == 0;
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    rs[t] = empty_state();
    const int m = 16 * t + (lane & 15);
    own_l[t] = (own_ready && m < a.R) ? a.own[m] : 0.f;
  }

  u32x4 wb[D][NF], xb[D][XN];
  int xhalf = 0;  // the half of the X tile sets the next pair of K steps uses
  PCursor ld{b, 0, 0, 0, 0};
  pc_enter<NF, D, KW>(L, wave, ld);
  PCursor cp = ld;
  if (ld.item < L.items) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      issue_w<NF>(wr, ld, L.items, L.wgroup, o.wo, wb[j]);
      issue_x_stage<MT, NF, XN, KW, D>(j, xr, ld, L.items, L.Ks, o, xb);
      pc_advance<NF, D, KW>(L, a.G, wave, ld);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (;;) {
      f32x4 acc[NF][MT];
#pragma unroll
      for (int f = 0; f < NF; ++f)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[f][t] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int steps = cp.pend - cp.st;  // a multiple of D, at least D
      auto stage = [&](int j) __attribute__((always_inline)) {
        u32x4 xop[MT];
        stage_x_rows<MT, XN, D>(j, xt, wave, xt_write, xt_read, xb, xop, xhalf);
#pragma unroll
        for (int f = 0; f < NF; ++f)
#pragma unroll
          for (int t = 0; t < MT; ++t) acc[f][t] = mfma_16x16x32<DT>(wb[j][f], xop[t], acc[f][t]);
        issue_w<NF>(wr, ld, L.items, L.wgroup, o.wo, wb[j]);
        issue_x_stage<MT, NF, XN, KW, D>(j, xr, ld, L.items, L.Ks, o, xb);
        pc_advance<NF, D, KW>(L, a.G, wave, ld);
        __builtin_amdgcn_sched_barrier(0);
      };
      // The first D steps peeled off the loop, as in packed_gemm_kernel: the loop is entered only
      // with its own load order in flight, so its load-count waits stay exact.
#pragma unroll
      for (int j = 0; j < D; ++j) stage(j);
      for (int i = D; i < steps; i += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) stage(j);
      }
      // Fold this wavefront's 16*NF columns into the row states (rounding mode resolved once per
      // item, not per element).
      const int n0 = (cp.item * kPackedWaves + wave) * NF * 16 + 4 * (lane >> 4);
      if (!own_ready) {
        wait_own_logits(a);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const int m = 16 * t + (lane & 15);
          own_l[t] = m < a.R ? collect(a.own + m) : 0.f;
        }
        own_ready = true;
      }
      if (a.logit_rows > 0) store_logits<DT, MT, NF>(acc, n0, a);
      const bool full = (cp.item * kPackedWaves + wave + 1) * NF * 16 <= a.V;  // no column past V
      if (a.round_mode == PLM_ROUND_BF16) {
        if (full) fold_columns<MT, NF, PLM_ROUND_BF16, false>(acc, n0, a.V, own_l, rs);
        else fold_columns<MT, NF, PLM_ROUND_BF16, true>(acc, n0, a.V, own_l, rs);
      } else if (a.round_mode == PLM_ROUND_F16) {
        if (full) fold_columns<MT, NF, PLM_ROUND_F16, false>(acc, n0, a.V, own_l, rs);
        else fold_columns<MT, NF, PLM_ROUND_F16, true>(acc, n0, a.V, own_l, rs);
      } else {
        if (full) fold_columns<MT, NF, PLM_ROUND_F32, false>(acc, n0, a.V, own_l, rs);
        else fold_columns<MT, NF, PLM_ROUND_F32, true>(acc, n0, a.V, own_l, rs);
      }
      cp.item += a.G;
      if (cp.item >= L.items) break;
      pc_enter<NF, D, KW>(L, wave, cp);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);

  // The workgroup's state of each row: its four wavefronts merged in wavefront order.
  if (lane < 16) {
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = 16 * t + lane;
      st_mx[wave][m] = rs[t].mx;
      st_se[wave][m] = rs[t].se;
      st_ab[wave][m] = rs[t].ab;
      st_ai[wave][m] = rs[t].ai;
    }
  }
  __syncthreads();
  if (threadIdx.x < a.R) {
    const int m = threadIdx.x;
    RowState s0 = RowState{st_mx[0][m], st_se[0][m], st_ab[0][m], st_ai[0][m]};
#pragma unroll
    for (int w = 1; w < kPackedWaves; ++w) s0 = merge(s0, RowState{st_mx[w][m], st_se[w][m], st_ab[w][m], st_ai[w][m]});
    publish_record(a.rec, b * a.R + m, a.G * a.R, s0);
  }
  // Two-level merge: the last workgroup of each group of kVerifyGroupSize merges the group's
  // states, the last group to finish merges the group states. Each level is one batch of
  // device-coherent loads into LDS and a fixed-order merge with one lane per row.
  const int group = b / kVerifyGroupSize;
  const int gsize = min(kVerifyGroupSize, a.G - group * kVerifyGroupSize);
  if (!arrive_last(a.group_counter + group, gsize)) return;
  gather_records(a.rec, group * kVerifyGroupSize, gsize, a.R, grid);
  {
    const RowState t = merge_rows(grid, gsize, wave, lane, st_mx, st_se, st_ab, st_ai);
    if (wave == 0 && lane < a.R) publish_record(a.grec, group * a.R + lane, (group + 1) * a.R, t);
  }
  const int groups = (a.G + kVerifyGroupSize - 1) / kVerifyGroupSize;
  if (!arrive_last(a.counter, groups)) return;
  // The proposals' own logits (complete before any workgroup's first fold) load with the records.
  const float own_v = (wave == 0 && lane < a.R) ? collect(a.own + lane) : 0.f;
  gather_records(a.grec, 0, groups, a.R, grid);
  const RowState t = merge_rows(grid, groups, wave, lane, st_mx, st_se, st_ab, st_ai);
  if (wave == 0) {
    if (lane == 0 && a.own_groups > 0) publish(a.own_done, 0);  // every workgroup has counted in and read it
    const bool acc = lane < a.R && accept_proposal(a, own_v, t);
    if (lane < a.R) {
      if (a.accept != nullptr) a.accept[lane] = acc ? 1 : 0;
      if (a.argmax != nullptr) a.argmax[lane] = t.ai;
    }
    if (a.round.k > 0) {
      // Rows 0..k-1 verify, rows k.. are the proposal blocks: lane i holds row i's decision and
      // argmax, so hypothesis j is lane k + j's argmax.
      const int ai = t.ai;
      const int k = a.round.k;
      round_epilogue_wave(a.round, lane, acc, [&](int j) { return static_cast<int64_t>(__shfl(ai, k + j)); });
    }
  }
}

template <int DT, int MT, int NF, int D>
hipError_t launch_verify_packed(VerifyArgs a, int cu_count, hipStream_t stream, bool dry) {
  if constexpr (!verify_packed_compiled<MT, NF, D>()) {
    return hipErrorInvalidConfiguration;
  } else {
    if (dry) return hipSuccess;
    auto main_kern = verify_packed_main_kernel<DT, MT, NF, D>;
    constexpr size_t lds = packed_lds_body<MT, NF, 1>();
    static int per_cu = 0;
    if (per_cu == 0) {
      per_cu = resident_per_cu(reinterpret_cast<const void*>(main_kern), 64 * kPackedWaves, lds);
      if (per_cu < 1) return hipErrorInvalidConfiguration;
    }
    const int tiles = ((a.V + 15) / 16 + kPackedWaves * NF - 1) / (kPackedWaves * NF);
    // The own-logit workgroups first (lowest indices: dispatched first, and they wait for nothing),
    // then the main ones, all resident together when the GPU is otherwise idle.
    a.own_groups = (a.R + kPackedWaves - 1) / kPackedWaves;
    a.G = min(tiles, min(kMaxVerifyGroups, max(1, cu_count * per_cu - a.own_groups)));
    hipLaunchKernelGGL(main_kern, dim3(a.own_groups + a.G), dim3(64 * kPackedWaves), lds, stream, a);
    return hipGetLastError();
  }
}

template <int DT, int MT, int NF>
hipError_t verify_packed_pick_d(const VerifyArgs& a, int d, int cu, hipStream_t s, bool dry) {
  if (d == 2) return launch_verify_packed<DT, MT, NF, 2>(a, cu, s, dry);
  if (d == 4) return launch_verify_packed<DT, MT, NF, 4>(a, cu, s, dry);
  if (d == 8) return launch_verify_packed<DT, MT, NF, 8>(a, cu, s, dry);
  return hipErrorInvalidConfiguration;
}

template <int DT>
hipError_t verify_packed_dispatch(const VerifyArgs& a, const plm_tile& t, int cu, hipStream_t s, bool dry) {
  if (t.k_waves != 1 || t.split_k != 1) return hipErrorInvalidConfiguration;
  const int mt = (a.R + 15) / 16;
#define PLM_VERIFY_PACKED(MT_)                                                           \
  if (mt == MT_) {                                                                       \
    if (t.wave_frags == 2) return verify_packed_pick_d<DT, MT_, 2>(a, t.unroll, cu, s, dry); \
    if (t.wave_frags == 4) return verify_packed_pick_d<DT, MT_, 4>(a, t.unroll, cu, s, dry); \
  }
  PLM_VERIFY_PACKED(1)
  PLM_VERIFY_PACKED(2)
  PLM_VERIFY_PACKED(3)
  PLM_VERIFY_PACKED(4)
#undef PLM_VERIFY_PACKED
  return hipErrorInvalidConfiguration;
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// Workspace layout: counter area (ints kVerifyCounter, kVerifyOwnDone, kPkErrorSlot and
// [kVerifyGroupBase, +groups) used) |
// own[R] | state[kMaxVerifyGroups][R][3] | state_idx[kMaxVerifyGroups][R] | gstate[groups][R][3] |
// gstate_idx[groups][R], groups = kMaxVerifyGroups / kVerifyGroupSize. The packed verify keeps its
// 16-byte records over the same bytes: rec[kMaxVerifyGroups][R] from state, grec[groups][R] from
// gstate (each pair of areas holds 12 + 4 bytes per entry).
constexpr int kMaxVerifyGroupSets = kMaxVerifyGroups / kVerifyGroupSize;
static_assert(kVerifyGroupBase + kMaxVerifyGroupSets <= 64, "group counters fit before the streaming counters");
void verify_layout(int64_t R, size_t& own_off, size_t& state_off, size_t& idx_off, size_t& gstate_off,
                   size_t& gidx_off, size_t& total) {
  own_off = kCounterBytes;
  state_off = own_off + align256(static_cast<size_t>(R) * sizeof(float));
  idx_off = state_off + align256(static_cast<size_t>(kMaxVerifyGroups) * R * 3 * sizeof(float));
  gstate_off = idx_off + align256(static_cast<size_t>(kMaxVerifyGroups) * R * sizeof(int));
  gidx_off = gstate_off + align256(static_cast<size_t>(kMaxVerifyGroupSets) * R * 3 * sizeof(float));
  total = gidx_off + align256(static_cast<size_t>(kMaxVerifyGroupSets) * R * sizeof(int));
}

int device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  static int cached_dev = -1, cached_cus = 0;
  if (dev != cached_dev) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cached_dev = dev;
    cached_cus = cus;
  }
  return cached_cus;
}

}  // namespace plm

extern "C" {

size_t plm_lm_head_verify_workspace_bytes(int64_t R, int64_t V, int64_t K, const plm_tile* tile) {
  (void)V;
  (void)K;
  (void)tile;
  if (R < 1) return 0;
  size_t own_off, state_off, idx_off, gstate_off, gidx_off, total;
  plm::verify_layout(R, own_off, state_off, idx_off, gstate_off, gidx_off, total);
  return total;
}

int plm_lm_head_verify(int32_t dtype, const void* x, int64_t ldx, const void* w, int64_t ldw, int64_t R, int64_t V,
                       int64_t K, const int64_t* pending, int32_t rule, float p, int32_t round_mode, uint8_t* accept,
                       int64_t* argmax, const plm_tile* tile, void* workspace, size_t workspace_bytes, void* stream) {
  if (x == nullptr || w == nullptr || pending == nullptr || accept == nullptr || argmax == nullptr || tile == nullptr)
    return PLM_ERR_ARGUMENT;
  if (dtype != PLM_BF16 && dtype != PLM_F16) return PLM_ERR_ARGUMENT;
  if (round_mode < PLM_ROUND_F32 || round_mode > PLM_ROUND_F16) return PLM_ERR_ARGUMENT;
  if (rule != PLM_RULE_NUCLEUS && rule != PLM_RULE_FLOOR) return PLM_ERR_ARGUMENT;
  if (R < 1 || R > 64 || V < 1 || V > (int64_t(1) << 30) || K < 8 || K % 8 != 0 || K > (int64_t(1) << 30))
    return PLM_ERR_ARGUMENT;
  if (ldx < K || ldw < K || tile->split_k != 1 || tile->k_waves < 1) return PLM_ERR_ARGUMENT;
  if (R * ldx * 2 >= (int64_t(1) << 31) || 16 * tile->wave_frags * ldw * 2 >= (int64_t(1) << 31)) return PLM_ERR_ARGUMENT;
  if (ldx % 8 != 0 || ldw % 8 != 0 || !plm::aligned16_ptr(x) || !plm::aligned16_ptr(w)) return PLM_ERR_ALIGNMENT;
  size_t own_off, state_off, idx_off, gstate_off, gidx_off, total;
  plm::verify_layout(R, own_off, state_off, idx_off, gstate_off, gidx_off, total);
  if (workspace == nullptr || workspace_bytes < total || !plm::aligned16_ptr(workspace)) return PLM_ERR_WORKSPACE;

  plm::VerifyArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(w);
  a.ldx = ldx;
  a.ldw = ldw;
  a.R = static_cast<int>(R);
  a.V = static_cast<int>(V);
  a.K = static_cast<int>(K);
  a.pending = pending;
  a.pending_rows = static_cast<int>(R);
  a.p = p;
  a.rule = rule;
  a.round_mode = round_mode;
  a.accept = accept;
  a.argmax = argmax;
  char* ws = static_cast<char*>(workspace);
  a.counter = reinterpret_cast<int*>(ws) + plm::kVerifyCounter;
  a.own = reinterpret_cast<float*>(ws + own_off);
  a.state = reinterpret_cast<float*>(ws + state_off);
  a.state_idx = reinterpret_cast<int*>(ws + idx_off);
  a.group_counter = reinterpret_cast<int*>(ws) + plm::kVerifyGroupBase;
  a.gstate = reinterpret_cast<float*>(ws + gstate_off);
  a.gstate_idx = reinterpret_cast<int*>(ws + gidx_off);

  const int cu = plm::device_cu_count();
  if (cu <= 0) return PLM_ERR_LAUNCH;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t err = dtype == PLM_BF16 ? plm::verify_dispatch<plm::DT_BF16>(a, *tile, cu, s, true)
                                     : plm::verify_dispatch<plm::DT_F16>(a, *tile, cu, s, true);
  if (err != hipSuccess) return PLM_ERR_TILE;
  err = dtype == PLM_BF16 ? plm::verify_dispatch<plm::DT_BF16>(a, *tile, cu, s, false)
                          : plm::verify_dispatch<plm::DT_F16>(a, *tile, cu, s, false);
  return err == hipSuccess ? PLM_OK : PLM_ERR_LAUNCH;
}

}  // extern "C"

namespace {

// The packed verify launch behind plm_lm_head_verify_packed and plm_round_verify_packed.
int packed_verify_entry(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, int64_t R, int64_t V,
                        int64_t K, const int64_t* pending, int64_t pending_rows, int32_t rule, float p,
                        int32_t round_mode, uint8_t* accept, int64_t* argmax, const plm::RoundEpilogue& round,
                        const plm_tile* tile, void* workspace, size_t workspace_bytes, void* stream,
                        void* logits = nullptr, int64_t ld_logits = 0, int64_t logit_rows = 0) {
  if (logit_rows < 0 || logit_rows > R || (logit_rows > 0 && logits == nullptr)) return PLM_ERR_ARGUMENT;
  if (logit_rows > 0) {
    // The logits handed out are the ones the decision reads: the round mode is the model dtype.
    if (round_mode != (dtype == PLM_BF16 ? PLM_ROUND_BF16 : PLM_ROUND_F16) || ld_logits < V) return PLM_ERR_ARGUMENT;
    if (ld_logits % 8 != 0 || !plm::aligned16_ptr(logits)) return PLM_ERR_ALIGNMENT;
  }
  if (x == nullptr || packed_w == nullptr || (pending_rows > 0 && pending == nullptr) || tile == nullptr)
    return PLM_ERR_ARGUMENT;
  if (dtype != PLM_BF16 && dtype != PLM_F16) return PLM_ERR_ARGUMENT;
  if (round_mode < PLM_ROUND_F32 || round_mode > PLM_ROUND_F16) return PLM_ERR_ARGUMENT;
  if (rule != PLM_RULE_NUCLEUS && rule != PLM_RULE_FLOOR) return PLM_ERR_ARGUMENT;
  if (R < 1 || R > 64 || V < 1 || V > (int64_t(1) << 30) || K < 8 || K % 8 != 0 || K > (int64_t(1) << 24))
    return PLM_ERR_ARGUMENT;
  if (ldx < K || R * ldx * 2 >= (int64_t(1) << 31)) return PLM_ERR_ARGUMENT;
  // 32-bit buffer offsets over the packed weight (its padding rows and steps included).
  const int64_t ks = (K + 31) / 32;
  if (plm::pack_bytes(V, ks) >= (int64_t(1) << 31)) return PLM_ERR_ARGUMENT;
  if (ldx % 8 != 0 || !plm::aligned16_ptr(x) || !plm::aligned16_ptr(packed_w)) return PLM_ERR_ALIGNMENT;
  size_t own_off, state_off, idx_off, gstate_off, gidx_off, total;
  plm::verify_layout(R, own_off, state_off, idx_off, gstate_off, gidx_off, total);
  if (workspace == nullptr || workspace_bytes < total || !plm::aligned16_ptr(workspace)) return PLM_ERR_WORKSPACE;

  plm::VerifyArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(packed_w);
  a.ldx = ldx;
  a.ldw = K;
  a.R = static_cast<int>(R);
  a.V = static_cast<int>(V);
  a.K = static_cast<int>(K);
  a.pending = pending;
  a.pending_rows = static_cast<int>(pending_rows);
  a.p = p;
  a.rule = rule;
  a.round_mode = round_mode;
  a.accept = accept;
  a.argmax = argmax;
  a.round = round;
  a.logits = logit_rows > 0 ? static_cast<uint16_t*>(logits) : nullptr;
  a.ld_logits = ld_logits;
  a.logit_rows = static_cast<int>(logit_rows);
  char* ws = static_cast<char*>(workspace);
  a.counter = reinterpret_cast<int*>(ws) + plm::kVerifyCounter;
  a.own = reinterpret_cast<float*>(ws + own_off);
  a.state = reinterpret_cast<float*>(ws + state_off);
  a.state_idx = reinterpret_cast<int*>(ws + idx_off);
  a.group_counter = reinterpret_cast<int*>(ws) + plm::kVerifyGroupBase;
  a.gstate = reinterpret_cast<float*>(ws + gstate_off);
  a.gstate_idx = reinterpret_cast<int*>(ws + gidx_off);
  a.rec = reinterpret_cast<plm::f32x4*>(ws + state_off);
  a.grec = reinterpret_cast<plm::f32x4*>(ws + gstate_off);
  a.own_done = reinterpret_cast<int*>(ws) + plm::kVerifyOwnDone;
  a.error = reinterpret_cast<int*>(ws) + plm::kPkErrorSlot;

  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t err = dtype == PLM_BF16 ? plm::verify_packed_dispatch<plm::DT_BF16>(a, *tile, 1, s, true)
                                     : plm::verify_packed_dispatch<plm::DT_F16>(a, *tile, 1, s, true);
  if (err != hipSuccess) return PLM_ERR_TILE;
  const int cu = plm::device_cu_count();
  if (cu <= 0) return PLM_ERR_LAUNCH;
  err = dtype == PLM_BF16 ? plm::verify_packed_dispatch<plm::DT_BF16>(a, *tile, cu, s, false)
                          : plm::verify_packed_dispatch<plm::DT_F16>(a, *tile, cu, s, false);
  return err == hipSuccess ? PLM_OK : PLM_ERR_LAUNCH;
}

}  // namespace

extern "C" {

int plm_lm_head_verify_packed(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, int64_t R, int64_t V,
                              int64_t K, const int64_t* pending, int32_t rule, float p, int32_t round_mode, uint8_t* accept,
                              int64_t* argmax, const plm_tile* tile, void* workspace, size_t workspace_bytes,
                              void* stream) {
  if (pending == nullptr || accept == nullptr || argmax == nullptr) return PLM_ERR_ARGUMENT;
  return packed_verify_entry(dtype, x, ldx, packed_w, R, V, K, pending, R, rule, p, round_mode, accept, argmax,
                             plm::RoundEpilogue{}, tile, workspace, workspace_bytes, stream);
}

int plm_lm_head_verify_packed_logits(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, int64_t R,
                                     int64_t V, int64_t K, const int64_t* pending, int64_t pending_rows, int32_t rule,
                                     float p, int32_t round_mode, uint8_t* accept, int64_t* argmax, void* logits,
                                     int64_t ld_logits, int64_t logit_rows, const plm_tile* tile, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  if (accept == nullptr || argmax == nullptr || pending_rows < 0 || pending_rows > R) return PLM_ERR_ARGUMENT;
  return packed_verify_entry(dtype, x, ldx, packed_w, R, V, K, pending, pending_rows, rule, p, round_mode, accept,
                             argmax, plm::RoundEpilogue{}, tile, workspace, workspace_bytes, stream, logits, ld_logits,
                             logit_rows);
}

int plm_round_verify_packed(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, int64_t k, int64_t V,
                            int64_t K, int32_t rule, float p, int32_t round_mode, const int64_t* verify,
                            int64_t* pending, int64_t* anchor, int64_t* out, int64_t out_len, int64_t* base,
                            int64_t* offset, int64_t* round_sequence, int64_t sequence_len, int64_t* sequence_step,
                            uint8_t* accept, int64_t* argmax, uint8_t* accepted, int64_t* num_correct,
                            const plm_tile* tile, void* workspace, size_t workspace_bytes, void* stream) {
  if (k < 1 || k + k * k > 64 || out_len < 0) return PLM_ERR_ARGUMENT;
  if (verify == nullptr || anchor == nullptr || out == nullptr || base == nullptr || offset == nullptr)
    return PLM_ERR_ARGUMENT;
  if (k > 1 && pending == nullptr) return PLM_ERR_ARGUMENT;
  if ((round_sequence == nullptr) != (sequence_step == nullptr)) return PLM_ERR_ARGUMENT;
  if (round_sequence != nullptr && sequence_len < 1) return PLM_ERR_ARGUMENT;
  plm::RoundEpilogue e{};
  e.k = static_cast<int>(k);
  e.verify = verify;
  e.pending = pending;
  e.anchor = anchor;
  e.out = out;
  e.out_len = out_len;
  e.base = base;
  e.offset = offset;
  e.round_sequence = round_sequence;
  e.sequence_len = sequence_len;
  e.sequence_step = sequence_step;
  e.accepted = accepted;
  e.num_correct = num_correct;
  return packed_verify_entry(dtype, x, ldx, packed_w, k + k * k, V, K, pending, k - 1, rule, p, round_mode, accept,
                             argmax, e, tile, workspace, workspace_bytes, stream);
}

}  // extern "C"
