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

#include "plm_amd.h"
#include "tile.h"

namespace plm {

struct VerifyArgs {
  const uint16_t* x;
  const uint16_t* w;
  int64_t ldx, ldw;
  int R, V, K, G;
  const int64_t* pending;
  float p;
  int round_mode;
  uint8_t* accept;
  int64_t* argmax;
  int* counter;      // [1], zero between launches
  float* own;        // [R]
  float* state;      // [G][R][3]: row max, sum of exp, sum of exp above own
  int* state_idx;    // [G][R]: argmax
};

// Online-softmax state of one row: maximum, sum of exp(l - max), sum of exp(l - max) over l > l_own,
// and the lowest index attaining the maximum. merge() is commutative bit for bit (no contraction,
// symmetric formulas), so a butterfly over lanes leaves every lane with the same result.
struct RowState {
  float mx, se, ab;
  int ai;
};

__device__ __forceinline__ RowState empty_state() { return RowState{-INFINITY, 0.f, 0.f, INT_MAX}; }

#pragma clang fp contract(off)
__device__ __forceinline__ RowState merge(RowState a, RowState b) {
  RowState r;
  r.ai = (b.mx > a.mx || (b.mx == a.mx && b.ai < a.ai)) ? b.ai : a.ai;
  if (b.mx == -INFINITY) return RowState{a.mx, a.se, a.ab, r.ai};
  if (a.mx == -INFINITY) return RowState{b.mx, b.se, b.ab, r.ai};
  r.mx = fmaxf(a.mx, b.mx);
  const float fa = expf(a.mx - r.mx), fb = expf(b.mx - r.mx);
  r.se = a.se * fa + b.se * fb;
  r.ab = a.ab * fa + b.ab * fb;
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
  const int64_t pid64 = a.pending[r];
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
        float e = valid ? expf(l - t.mx) : 0.f;
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
      const float own = a.own[m];
      const bool in_nucleus = (s.ab / s.se) < a.p;
      const bool is_max = (own >= s.mx) && (a.p > 0.f);
      const bool valid_id = own == own;  // NaN marks a pending id outside [0, V)
      a.accept[m] = (valid_id && (in_nucleus || is_max)) ? 1 : 0;
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

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// Workspace layout: counter area (int kVerifyCounter used) | own[R] | state[kMaxVerifyGroups][R][3] |
// state_idx[kMaxVerifyGroups][R]
void verify_layout(int64_t R, size_t& own_off, size_t& state_off, size_t& idx_off, size_t& total) {
  own_off = kCounterBytes;
  state_off = own_off + align256(static_cast<size_t>(R) * sizeof(float));
  idx_off = state_off + align256(static_cast<size_t>(kMaxVerifyGroups) * R * 3 * sizeof(float));
  total = idx_off + align256(static_cast<size_t>(kMaxVerifyGroups) * R * sizeof(int));
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
  size_t own_off, state_off, idx_off, total;
  plm::verify_layout(R, own_off, state_off, idx_off, total);
  return total;
}

int plm_lm_head_verify(int32_t dtype, const void* x, int64_t ldx, const void* w, int64_t ldw, int64_t R, int64_t V,
                       int64_t K, const int64_t* pending, float p, int32_t round_mode, uint8_t* accept,
                       int64_t* argmax, const plm_tile* tile, void* workspace, size_t workspace_bytes, void* stream) {
  if (x == nullptr || w == nullptr || pending == nullptr || accept == nullptr || argmax == nullptr || tile == nullptr)
    return PLM_ERR_ARGUMENT;
  if (dtype != PLM_BF16 && dtype != PLM_F16) return PLM_ERR_ARGUMENT;
  if (round_mode < PLM_ROUND_F32 || round_mode > PLM_ROUND_F16) return PLM_ERR_ARGUMENT;
  if (R < 1 || R > 64 || V < 1 || V > (int64_t(1) << 30) || K < 8 || K % 8 != 0 || K > (int64_t(1) << 30))
    return PLM_ERR_ARGUMENT;
  if (ldx < K || ldw < K || tile->split_k != 1 || tile->k_waves < 1) return PLM_ERR_ARGUMENT;
  if (R * ldx * 2 >= (int64_t(1) << 31) || 16 * tile->wave_frags * ldw * 2 >= (int64_t(1) << 31)) return PLM_ERR_ARGUMENT;
  if (ldx % 8 != 0 || ldw % 8 != 0 || !plm::aligned16_ptr(x) || !plm::aligned16_ptr(w)) return PLM_ERR_ALIGNMENT;
  size_t own_off, state_off, idx_off, total;
  plm::verify_layout(R, own_off, state_off, idx_off, total);
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
  a.p = p;
  a.round_mode = round_mode;
  a.accept = accept;
  a.argmax = argmax;
  char* ws = static_cast<char*>(workspace);
  a.counter = reinterpret_cast<int*>(ws) + plm::kVerifyCounter;
  a.own = reinterpret_cast<float*>(ws + own_off);
  a.state = reinterpret_cast<float*>(ws + state_off);
  a.state_idx = reinterpret_cast<int*>(ws + idx_off);

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
