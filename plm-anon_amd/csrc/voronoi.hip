// Logit-Voronoi auxiliary decode on gfx950: the token a verify row's auxiliary value decodes to,
// from that row's logits and the (V, A) cost table (plm/auxiliary.py:67-75 over the ``iterate``
// engine, plm/iterate.py:176-342).
//
// A problem is one verify row. Per problem:
//   1. voronoi_shortlist_kernel, one 1024-thread workgroup: the row's softmax normaliser, its
//      n_targets largest logits (value descending, token id ascending), their largest-remainder
//      quotas of the A items, the cost unit and the prior factor (iterate.py:248-290) in one launch.
//      The row stays in registers as 16-bit order keys; a threshold (the n_targets-th largest
//      per-thread maximum, found by bisection over the 16-bit key space) keeps every element of
//      the top n_targets, and only the few elements above it are sorted (bitonic, in LDS).
//   2. voronoi_condense_kernel, items spread over workgroups: each item's k cheapest packed keys
//      of cost + offset (iterate.py:87-107).
//   3. voronoi_fit_kernel, one 1024-thread workgroup: the annealed Sinkhorn sweeps on the condensed
//      problem (iterate.py:110-159). Each thread owns items and all their k slots, so an item's
//      softmax needs no exchange. The per-token loads are exact integer sums: each weight enters
//      as round(w 2^31) into a 64-bit LDS counter per target, so the sums, and the fitted factors,
//      are the same bit for bit on every run whatever order the adds land in (the reference adds
//      fp32 atomics in arrival order, which is not, iterate.py:8-9).
//   2-3 repeat per round; the last fit also resolves the problem's one auxiliary value.
//   4. voronoi_argmin_kernel (only when sigma is asked for): the assignment of every item.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>

#include "plm_amd.h"
#include "tile.h"

namespace plm {
namespace {

constexpr int kRowThreads = 1024;  // shortlist and fit workgroups
constexpr int kRowWaves = kRowThreads / 64;
constexpr int kCandidateCap = 2048;
constexpr int kMaxTargets = 128;   // the packed key keeps the target in its low 7 bits
constexpr int kMaxVocab = 65528;   // token ids ride in the low 16 bits of the sort key; the row + 7
                                   // tokens of alignment fits 64 elements per thread
constexpr int kMaxItems = 8192;
constexpr int kMinItems = 64;
constexpr int kMaxSlots = 16;
constexpr int kItemThreads = 256;  // condense and argmin workgroups
constexpr int kSpreadSample = 64;  // iterate.py:275
constexpr float kBlocked = 1e3f;   // iterate.py:25
constexpr float kLoadFloor = 1e-2f;
constexpr float kEmpty = -1e30f;   // iterate.py:26

// Order-preserving 16-bit keys of bf16 or fp16 values (both keep the sign in bit 15): a larger
// value has a larger key, -0 and +0 share 0x8000, and no value has key 0, which marks a position
// outside the vocabulary. A negative value maps to 0x10000 - bits, the rest to bits | 0x8000. Two
// keys per 32-bit word, in packed 16-bit integer instructions.
typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t order_keys2(uint32_t w) {
  const uint32_t negative = __builtin_bit_cast(uint32_t, __builtin_bit_cast(s16x2, w) >> (s16x2){15, 15});
  const uint32_t flipped = __builtin_bit_cast(uint32_t, (u16x2){0, 0} - __builtin_bit_cast(u16x2, w));
  return (flipped & negative) | ((w | 0x80008000u) & ~negative);
}
__device__ __forceinline__ uint32_t max_keys2(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b)));
}
__device__ __forceinline__ uint32_t order_key16(uint32_t bits) { return order_keys2(bits & 0xFFFFu) & 0xFFFFu; }
__device__ __forceinline__ uint32_t key16_bits(uint32_t key) {
  return key >= 0x8000u ? key & 0x7FFFu : (0x10000u - key) & 0xFFFFu;
}

// A caller's token id as a table row, clamped into [0, V) so no input reads outside the table.
__device__ __forceinline__ int64_t table_row(int64_t token, int V) { return token < 0 ? 0 : (token >= V ? V - 1 : token); }

// -------------------------------------------------------------------------- reductions
// Wavefront reductions run on the VALU: DPP lane permutations inside each row of 16 lanes, then the
// four rows' results read out and combined in row order. A butterfly step adds a + b on one lane
// and b + a on its partner, equal bit for bit, so every lane ends with the same value and the
// summation order is fixed.

constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7 - i within each half row
constexpr int kDppMirror = 0x140;     // lane i <-> 15 - i within each row
constexpr int kDppShr1 = 0x111, kDppShr2 = 0x112, kDppShr4 = 0x114, kDppShr8 = 0x118;
constexpr int kDppBcast15 = 0x142, kDppBcast31 = 0x143;

template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ int dpp(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWS, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, dpp<CTRL>(__builtin_bit_cast(int, v)));
}
template <int CTRL>
__device__ __forceinline__ unsigned long long dpp(unsigned long long v) {
  const uint32_t lo = static_cast<uint32_t>(dpp<CTRL>(static_cast<int>(v)));
  const uint32_t hi = static_cast<uint32_t>(dpp<CTRL>(static_cast<int>(v >> 32)));
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}
__device__ __forceinline__ int lane_value(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }
__device__ __forceinline__ float lane_value(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Every lane of a fully active wavefront gets the sum / maximum of all 64 lanes.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppMirror>(v);
  return ((lane_value(v, 0) + lane_value(v, 16)) + lane_value(v, 32)) + lane_value(v, 48);
}
__device__ __forceinline__ int wave_sum(int v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppMirror>(v);
  return lane_value(v, 0) + lane_value(v, 16) + lane_value(v, 32) + lane_value(v, 48);
}
__device__ __forceinline__ uint32_t wave_max(uint32_t u) {
  int v = static_cast<int>(u);
  v = static_cast<int>(max(static_cast<uint32_t>(v), static_cast<uint32_t>(dpp<kDppXor1>(v))));
  v = static_cast<int>(max(static_cast<uint32_t>(v), static_cast<uint32_t>(dpp<kDppXor2>(v))));
  v = static_cast<int>(max(static_cast<uint32_t>(v), static_cast<uint32_t>(dpp<kDppHalfMirror>(v))));
  v = static_cast<int>(max(static_cast<uint32_t>(v), static_cast<uint32_t>(dpp<kDppMirror>(v))));
  return max(max(static_cast<uint32_t>(lane_value(v, 0)), static_cast<uint32_t>(lane_value(v, 16))),
             max(static_cast<uint32_t>(lane_value(v, 32)), static_cast<uint32_t>(lane_value(v, 48))));
}
// Inclusive prefix sum over the 64 lanes (row-wise shifts, then the row carries broadcast).
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  v += dpp<kDppShr1>(v);
  v += dpp<kDppShr2>(v);
  v += dpp<kDppShr4>(v);
  v += dpp<kDppShr8>(v);
  v += dpp<kDppBcast15, 0xA>(v);
  v += dpp<kDppBcast31, 0xC>(v);
  return v;
}

// Block-wide versions for 1024 threads: every thread gets the result. Each wavefront reduces its
// lanes, lane 0 posts the wavefront's value, and after one barrier every wavefront reads the 16
// posts (one per lane) and reduces them the same way. Calls alternate between two scratch rows,
// so consecutive calls need no barrier between them.
struct BlockScratch {
  int i[2][kRowWaves];
  float f[2][kRowWaves];
  uint32_t u[2][kRowWaves];
};

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x & 63); }

__device__ __forceinline__ int block_sum_int(int v, BlockScratch& s, int& parity) {
  v = wave_sum(v);
  if (lane_id() == 0) s.i[parity][threadIdx.x >> 6] = v;
  __syncthreads();
  const int total = wave_sum(lane_id() < kRowWaves ? s.i[parity][lane_id()] : 0);
  parity ^= 1;
  return total;
}

__device__ __forceinline__ float block_sum_float(float v, BlockScratch& s, int& parity) {
  v = wave_sum(v);
  if (lane_id() == 0) s.f[parity][threadIdx.x >> 6] = v;
  __syncthreads();
  const float total = wave_sum(lane_id() < kRowWaves ? s.f[parity][lane_id()] : 0.f);
  parity ^= 1;
  return total;
}

__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, BlockScratch& s, int& parity) {
  v = wave_max(v);
  if (lane_id() == 0) s.u[parity][threadIdx.x >> 6] = v;
  __syncthreads();
  const uint32_t total = wave_max(lane_id() < kRowWaves ? s.u[parity][lane_id()] : 0u);
  parity ^= 1;
  return total;
}

// Exclusive prefix sum over the workgroup in thread order; `total` gets the sum.
__device__ __forceinline__ int block_exclusive_scan(int v, int& total, BlockScratch& s, int& parity) {
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int inc = wave_inclusive_scan(v);
  if (lane == 63) s.i[parity][wave] = inc;
  __syncthreads();
  const int c = lane < kRowWaves ? s.i[parity][lane] : 0;
  const int base = wave_sum(lane < wave ? c : 0);
  total = wave_sum(c);
  parity ^= 1;
  return base + inc - v;
}

// Descending bitonic sort of s[0, n), n a power of two.
__device__ void bitonic_descending(uint32_t* s, int n) {
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < (n >> 1); i += kRowThreads) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool descending = (lo & size) == 0;
        const uint32_t x = s[lo], y = s[hi];
        if ((x < y) == descending) {
          s[lo] = y;
          s[hi] = x;
        }
      }
      __syncthreads();
    }
  }
}

template <int DT>
__device__ __forceinline__ float round_model(float v) {
  if constexpr (DT == DT_BF16) return static_cast<float>(static_cast<__bf16>(v));
  return static_cast<float>(static_cast<_Float16>(v));
}

// Spread (iterate.py:275-284): the mean over the first min(sample, A) items of the gap between the
// worst and best of the M targets, the gap rounded to the table's dtype as the reference subtracts
// in it. In three steps, all 1024 threads taking part, so a caller can work while the reads are in
// flight:
// spread_reads issues this thread's table reads (column min(lane, cols - 1) of the rows of targets
// wave + 16 i, clamped to M - 1: no conditions, all in flight at once, each an HBM round trip);
// spread_post posts each wavefront's column minima and maxima; after a barrier, spread_mean gives
// wavefront 0 the mean over the columns of the rounded gap.
constexpr int kSpreadReads = kMaxTargets / kRowWaves;
__device__ __forceinline__ int spread_cols(int A, int sample) { return min(min(sample, kSpreadSample), A); }

template <typename RowOf>
__device__ __forceinline__ void spread_reads(const uint16_t* table, int A, int M, int sample, RowOf row_of,
                                             uint16_t (&raw)[kSpreadReads]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cols = spread_cols(A, sample);
#pragma unroll
  for (int i = 0; i < kSpreadReads; ++i)
    raw[i] = table[static_cast<int64_t>(row_of(min(wave + kRowWaves * i, M - 1))) * A + min(lane, cols - 1)];
}

template <int DT>
__device__ __forceinline__ void spread_post(const uint16_t (&raw)[kSpreadReads], int A, int M, int sample,
                                            float (*lo_s)[kSpreadSample], float (*hi_s)[kSpreadSample]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cols = spread_cols(A, sample);
  float lo = INFINITY, hi = -INFINITY;
#pragma unroll
  for (int i = 0; i < kSpreadReads; ++i) {
    if (lane < cols && wave + kRowWaves * i < M) {
      const float v = from_bits16<DT>(raw[i]);
      lo = fminf(lo, v);
      hi = fmaxf(hi, v);
    }
  }
  lo_s[wave][lane] = lo;
  hi_s[wave][lane] = hi;
}

template <int DT>
__device__ __forceinline__ float spread_mean(int A, int sample, const float (*lo_s)[kSpreadSample],
                                             const float (*hi_s)[kSpreadSample]) {
  const int lane = threadIdx.x & 63;
  const int cols = spread_cols(A, sample);
  float lo = lo_s[0][lane], hi = hi_s[0][lane];
#pragma unroll
  for (int g = 1; g < kRowWaves; ++g) {
    lo = fminf(lo, lo_s[g][lane]);
    hi = fmaxf(hi, hi_s[g][lane]);
  }
  return wave_sum(lane < cols ? round_model<DT>(hi - lo) : 0.f) / static_cast<float>(cols);
}

// Prior (iterate.py:286-290), in the reference's operation order.
__device__ __forceinline__ float prior_factor(int64_t count, float unit, int A, float weight) {
  const float share = fmaxf(static_cast<float>(count) / static_cast<float>(A), 1e-9f);
  const float scale = -weight * unit;
  return count > 0 ? scale * logf(share) : kBlocked * unit;
}

// -------------------------------------------------------------------------- 1. shortlist

struct ShortArgs {
  const uint16_t* logits;
  int64_t ld;
  const uint16_t* table;
  int V, A, M;
  float weight;
  int64_t* tokens;   // [N][M]
  int64_t* counts;   // [N][M]
  float* values;     // [N][M] or null
  float* unit;       // [N]
  float* prior;      // [N][M]
  float* normaliser; // [N] or null
};

// Candidate sets up to this size are ranked by counting (each candidate counts the larger ones);
// larger ones go through a bitonic sort.
constexpr int kRankCap = 256;

// Threads whose largest key reaches the threshold hand their keys to the workgroup through LDS, up
// to this many (more only when many equal values sit at the threshold: then each scans its own).
constexpr int kQualifyCap = 256;

// Adds one to hist[bin] for every active lane of the wavefront, one LDS add per distinct bin (the
// group's lowest lane adds the group's size). For bins that few values share: adds of one
// instruction that land on the same counter are carried out one after another, and the per-thread
// maxima of a row fall into a handful of high-byte bins.
__device__ __forceinline__ void wave_bin_add(int* hist, uint32_t bin, bool active) {
  const int lane = threadIdx.x & 63;
  uint64_t pending = __ballot(active);
  while (pending) {
    const int leader = __builtin_ctzll(pending);
    const uint32_t b = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(bin), leader));
    const uint64_t same = __ballot(active && bin == b);
    if (lane == leader) atomicAdd(&hist[b], __popcll(same));
    pending &= ~same;
  }
}

// Wavefront 0 over a 256-bin histogram: the largest bin b whose count of bins >= b reaches `need`.
// out[0] = b, out[1] = need less the count of bins above b (>= 1).
__device__ __forceinline__ void select_bin(const int* hist, int need, int* out) {
  const int lane = threadIdx.x & 63;
  const int c0 = hist[4 * lane], c1 = hist[4 * lane + 1], c2 = hist[4 * lane + 2], c3 = hist[4 * lane + 3];
  const int inc = wave_inclusive_scan(c0 + c1 + c2 + c3);
  const int above = lane_value(inc, 63) - inc;  // bins past 4 lane + 3
  const int s3 = above + c3, s2 = s3 + c2, s1 = s2 + c1, s0 = s1 + c0;
  if (s0 >= need && above < need) {
    const int b = s3 >= need ? 3 : (s2 >= need ? 2 : (s1 >= need ? 1 : 0));
    out[0] = 4 * lane + b;
    out[1] = need - (b == 3 ? above : (b == 2 ? s3 : (b == 1 ? s2 : s1)));
  }
}

// JT = elements per thread (a multiple of 8 covering V / 1024).
template <int DT, int JT>
__global__ __launch_bounds__(kRowThreads) void voronoi_shortlist_kernel(ShortArgs a) {
  constexpr int W = JT / 2;  // key words per thread
  __shared__ __align__(16) uint32_t cand[kCandidateCap];
  __shared__ __align__(16) uint32_t qkeys[kQualifyCap][W];
  __shared__ int qowner[kQualifyCap];
  __shared__ int hist[2][256];
  __shared__ int sel[4];
  __shared__ int counters[2];  // threads that reach the threshold, candidates
  __shared__ uint32_t top[kMaxTargets];
  __shared__ BlockScratch red;
  __shared__ float lo_s[kRowWaves][kSpreadSample], hi_s[kRowWaves][kSpreadSample];
  __shared__ __align__(16) float rem_s[kMaxTargets];
  __shared__ int rank_s[kMaxTargets];
  int parity = 0;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int64_t p = blockIdx.x;
  const int M = a.M;
  const uint16_t* row = a.logits + p * a.ld;
  if (t < 512) (&hist[0][0])[t] = 0;
  if (t < 2) counters[t] = 0;
  if (t < kRankCap + 4) cand[t] = 0u;  // the ranking reads up to a multiple of four past the last candidate

  // The row as order keys, two per register (element j of this thread in half j % 2 of word j / 2);
  // key 0 marks a position outside the vocabulary. The row is read in 16-byte pieces from the
  // 16-byte boundary at or below its start, which lies `shift` tokens before it: element j of this
  // thread is token 8 (t + 1024 (j / 8)) + j % 8 - shift. Pieces [first, last] lie wholly inside the
  // row. Every thread reads all of its pieces at once with no condition, a piece outside that range
  // re-reading one inside it; then the (at most two) pieces straddling an end are read again token
  // by token.
  uint32_t kk[W];
  uint32_t kmax2 = 0;
  const int shift = static_cast<int>((reinterpret_cast<uintptr_t>(row) & 15u) >> 1);
  const uint16_t* base = row - shift;
  const int first = shift > 0 ? 1 : 0, last = (shift + a.V) / 8 - 1;
  const bool any_whole = first <= last;
  auto token_of = [&](int j) -> int { return 8 * (t + kRowThreads * (j >> 3)) + (j & 7) - shift; };
  u32x4 piece[JT / 8];
  if (any_whole) {
#pragma unroll
    for (int c = 0; c < JT / 8; ++c)
      piece[c] = *reinterpret_cast<const u32x4*>(base + 8 * min(max(t + kRowThreads * c, first), last));
  }
#pragma unroll
  for (int c = 0; c < JT / 8; ++c) {
    const int i0 = 8 * (t + kRowThreads * c) - shift;
    if (any_whole && i0 >= 0 && i0 + 8 <= a.V) {
#pragma unroll
      for (int e = 0; e < 4; ++e) kk[4 * c + e] = order_keys2(piece[c][e]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = i0 + 2 * e;
        const uint32_t lo = (i >= 0 && i < a.V) ? order_key16(row[i]) : 0u;
        const uint32_t hi = (i + 1 >= 0 && i + 1 < a.V) ? order_key16(row[i + 1]) : 0u;
        kk[4 * c + e] = lo | (hi << 16);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) kmax2 = max_keys2(kmax2, kk[4 * c + e]);
  }
  const uint32_t kmax = max(kmax2 & 0xFFFFu, kmax2 >> 16);
  auto key_of = [&](int j) -> uint32_t { return (kk[j >> 1] >> (16 * (j & 1))) & 0xFFFFu; };

  // The normaliser max + log(sum exp(l - max)) (iterate.py:56-80, values clamped to the reference's
  // finite stand-in for -inf), only when the caller asks for it: the quotas below use the shortlist's
  // softmax directly, which the normaliser cancels out of (iterate.py:272-273).
  if (a.normaliser != nullptr) {
    const uint32_t bmax = block_max_u32(kmax, red, parity);
    const float mx = fmaxf(from_bits16<DT>(static_cast<uint16_t>(key16_bits(bmax))), kEmpty);
    float se = 0.f;
#pragma unroll
    for (int j = 0; j < JT; ++j) {
      const uint32_t k = key_of(j);
      if (k != 0) se += __expf(fmaxf(from_bits16<DT>(static_cast<uint16_t>(key16_bits(k))), kEmpty) - mx);
    }
    se = block_sum_float(se, red, parity);
    if (t == 0) a.normaliser[p] = mx + logf(se);
  }

  // Threshold: the M-th largest per-thread maximum. At least M elements reach it, so the M largest
  // elements all do. Found as a radix selection over the 1024 maxima: a histogram of their high
  // bytes picks the high byte, a histogram of the low bytes of the maxima in that bin the low one.
  __syncthreads();  // the histograms and counters are zero
  wave_bin_add(hist[0], kmax >> 8, true);
  __syncthreads();
  if (wave == 0) select_bin(hist[0], M, &sel[0]);
  __syncthreads();
  if ((kmax >> 8) == static_cast<uint32_t>(sel[0])) atomicAdd(&hist[1][kmax & 0xFFu], 1);
  __syncthreads();
  if (wave == 0) select_bin(hist[1], sel[1], &sel[2]);
  __syncthreads();
  const uint32_t tau = (static_cast<uint32_t>(sel[0]) << 8) | static_cast<uint32_t>(sel[2]);

  // Candidates: every element at or above the threshold, as sort keys (value key above, 0xFFFF -
  // token below, so equal values order by ascending token id). Their order in cand[] is the order
  // the LDS counter hands out slots in; the ranking below depends only on the set.
  const bool reaches = kmax != 0 && kmax >= tau;
  if (reaches) {
    const int slot = atomicAdd(&counters[0], 1);
    if (slot < kQualifyCap) {
      qowner[slot] = t;
#pragma unroll
      for (int w = 0; w < W; w += 4)
        *reinterpret_cast<u32x4*>(&qkeys[slot][w]) = u32x4{kk[w], kk[w + 1], kk[w + 2], kk[w + 3]};
    }
  }
  __syncthreads();
  auto is_candidate = [&](uint32_t k) { return k != 0 && k >= tau; };
  auto take = [&](uint32_t k, int token) {
    if (is_candidate(k)) {
      const int pos = atomicAdd(&counters[1], 1);
      if (pos < kCandidateCap) cand[pos] = (k << 16) | (0xFFFFu - static_cast<uint32_t>(token));
    }
  };
  const int n_reach = counters[0];
  if (n_reach <= kQualifyCap) {
    for (int f = t; f < n_reach * W; f += kRowThreads) {
      const int slot = f / W, w = f - slot * W;
      const uint32_t k2 = qkeys[slot][w];
      const int token = 8 * (qowner[slot] + kRowThreads * (w >> 2)) + 2 * (w & 3) - shift;
      take(k2 & 0xFFFFu, token);
      take(k2 >> 16, token + 1);
    }
  } else if (reaches) {
#pragma unroll
    for (int j = 0; j < JT; ++j) take(key_of(j), token_of(j));
  }
  __syncthreads();
  int total = counters[1];
  // The spread reads the first kSpreadSample columns (one 128-byte line) of the M targets' table
  // rows; the candidates include the targets, so each candidate's line is requested now and is in
  // the cache by the time the spread's reads go out. The value read is not used.
  uint16_t warm = 0;
  if (total <= kRankCap && t < total)
    warm = a.table[table_row(0xFFFF - static_cast<int>(cand[t] & 0xFFFFu), a.V) * a.A];
  if (total > kCandidateCap) {
    // Many elements tie at the threshold (flat logits): bisect the full 32-bit sort key instead,
    // which leaves exactly M elements at or above it. Rare, so the passes re-read the row rather
    // than hold sort keys in registers.
    auto sort_key = [&](int i) -> uint32_t {
      const uint32_t k = order_key16(row[i]);
      return k == 0 ? 0u : ((k << 16) | (0xFFFFu - static_cast<uint32_t>(i)));
    };
    uint32_t kappa = 0;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t c = kappa | (1u << bit);
      int n = 0;
      for (int i = t; i < a.V; i += kRowThreads) n += sort_key(i) >= c ? 1 : 0;
      if (block_sum_int(n, red, parity) >= M) kappa = c;
    }
    int mine = 0;
    for (int i = t; i < a.V; i += kRowThreads) mine += sort_key(i) >= kappa ? 1 : 0;
    int off = block_exclusive_scan(mine, total, red, parity);
    for (int i = t; i < a.V; i += kRowThreads) {
      const uint32_t sk = sort_key(i);
      if (sk >= kappa && sk != 0) cand[off++] = sk;
    }
    if (t >= total && t < kRankCap + 4) cand[t] = 0u;  // total == M here: clear the first pass's rest
    __syncthreads();
  }
  if (total <= kRankCap) {
    // Rank by counting: sort keys are unique, so a candidate's rank is the number of larger ones.
    const int padded = (total + 3) & ~3;
    // Thread 4 i + g counts, for candidate i, the larger keys among every fourth group of four.
    {
      const int i = t >> 2, g = t & 3;
      const uint32_t key = i < total ? cand[i] : 0xFFFFFFFFu;
      int rank = 0;
      for (int j = 4 * g; j < padded; j += 16) {
        const u32x4 c4 = *reinterpret_cast<const u32x4*>(&cand[j]);
        rank += (c4[0] > key) + (c4[1] > key) + (c4[2] > key) + (c4[3] > key);
      }
      rank += dpp<kDppXor1>(rank);
      rank += dpp<kDppXor2>(rank);
      if (g == 0 && i < total && rank < M) top[rank] = key;
    }
    // every in-row element has a nonzero key and V >= M, so this only guards the slots
    if (t < M && t >= total) top[t] = 0u;
  } else {
    int n_sort = M;
    while (n_sort < total) n_sort <<= 1;
    for (int i = total + t; i < n_sort; i += kRowThreads) cand[i] = 0u;
    __syncthreads();
    bitonic_descending(cand, n_sort);
    if (t < M) top[t] = cand[t];
  }
  __syncthreads();

  // The spread's reads go out first (every wavefront takes its targets' tokens from top[]); the
  // quotas run while they are in flight.
  auto top_token = [&](int m) { return min(static_cast<int>(0xFFFFu - (top[m] & 0xFFFFu)), a.V - 1); };
  uint16_t spread_raw[kSpreadReads];
  spread_reads(a.table, a.A, M, kSpreadSample, top_token, spread_raw);
  // Quotas (iterate.py:214-223, 272-273) by wavefront 0, lane l holding targets l and l + 64. The
  // shortlist's softmax is formed against its largest logit.
  float val[2] = {0.f, 0.f};
  int cnt[2] = {0, 0};
  int remaining = 0;
  if (wave == 0) {
    const int lane = t;
    const float v0 = from_bits16<DT>(static_cast<uint16_t>(key16_bits(top[0] >> 16)));
    float pr[2] = {0.f, 0.f};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int m = lane + 64 * h;
      if (m < M) {
        val[h] = from_bits16<DT>(static_cast<uint16_t>(key16_bits(top[m] >> 16)));
        pr[h] = expf(val[h] - v0);
      }
    }
    const float psum = wave_sum(pr[0] + pr[1]);
    int floors = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int m = lane + 64 * h;
      if (m < M) {
        const float exact = (pr[h] / psum) * static_cast<float>(a.A);
        const float fl = floorf(exact);
        cnt[h] = static_cast<int>(fl);
        rem_s[m] = exact - fl;
        floors += cnt[h];
      }
    }
    remaining = a.A - wave_sum(floors);
  }
  spread_post<DT>(spread_raw, a.A, M, kSpreadSample, lo_s, hi_s);
  asm volatile("" ::"v"(warm));  // older than the spread's reads, so back before them
  __syncthreads();  // rem_s, the spread's minima and maxima
  // Remainder ranks: thread 8 m + g compares target m's remainder with targets [16 g, 16 g + 16);
  // the eight partial counts of m sit in one lane octet and add up there.
  {
    const int m = t >> 3, g = t & 7;
    int part = 0;
    if (m < M) {
      const float mine_rem = rem_s[m];
#pragma unroll
      for (int j = 16 * g; j < 16 * g + 16; j += 4) {
        const f32x4 r4 = *reinterpret_cast<const f32x4*>(&rem_s[j]);
#pragma unroll
        for (int u = 0; u < 4; ++u)
          part += (j + u < M && (r4[u] > mine_rem || (r4[u] == mine_rem && j + u < m))) ? 1 : 0;
      }
    }
    part += dpp<kDppXor1>(part);
    part += dpp<kDppXor2>(part);
    part += dpp<kDppHalfMirror>(part);
    if (g == 0 && m < M) rank_s[m] = part;
  }
  float unit = 0.f;
  if (wave == 0) unit = spread_mean<DT>(a.A, kSpreadSample, lo_s, hi_s);
  __syncthreads();  // rank_s
  if (wave == 0) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int m = t + 64 * h;
      if (m < M) {
        const int c = cnt[h] + (rank_s[m] < remaining ? 1 : 0);
        const int64_t o = p * M + m;
        a.prior[o] = prior_factor(c, unit, a.A, a.weight);
        a.tokens[o] = top_token(m);
        a.counts[o] = c;
        if (a.values != nullptr) a.values[o] = val[h];
      }
    }
    if (t == 0) a.unit[p] = unit;
  }
}

// Standalone spread and prior, for callers that run the engine's steps one by one.
struct SpreadArgs {
  const uint16_t* table;
  const int64_t* tokens;
  float* unit;
  int V, M, A, sample;
};

template <int DT>
__global__ __launch_bounds__(kRowThreads) void voronoi_spread_kernel(SpreadArgs a) {
  __shared__ float lo_s[kRowWaves][kSpreadSample], hi_s[kRowWaves][kSpreadSample];
  const int64_t p = blockIdx.x;
  uint16_t raw[kSpreadReads];
  spread_reads(a.table, a.A, a.M, a.sample, [&](int m) { return table_row(a.tokens[p * a.M + m], a.V); }, raw);
  spread_post<DT>(raw, a.A, a.M, a.sample, lo_s, hi_s);
  __syncthreads();
  if (threadIdx.x < 64) {
    const float unit = spread_mean<DT>(a.A, a.sample, lo_s, hi_s);
    if (threadIdx.x == 0) a.unit[p] = unit;
  }
}

__global__ __launch_bounds__(kMaxTargets) void voronoi_prior_kernel(const int64_t* counts, const float* unit,
                                                                     float* prior, int M, int A, float weight) {
  const int64_t p = blockIdx.x;
  if (threadIdx.x < M) prior[p * M + threadIdx.x] = prior_factor(counts[p * M + threadIdx.x], unit[p], A, weight);
}

// -------------------------------------------------------------------------- 2. condense

struct CondenseArgs {
  const uint16_t* table;
  const int64_t* tokens;  // [N][M]
  const float* offset;    // [N][M]
  int32_t* key;           // [N][K][A]
  int V, M, A;
};

__device__ __forceinline__ int32_t pack_cost(float c, int target) {
  const int32_t bits = __builtin_bit_cast(int32_t, c);
  const int32_t ordered = bits >= 0 ? bits : (bits ^ 0x7FFFFFFF);
  return (ordered & ~0x7F) | target;
}

// A workgroup takes 64 items; its four wavefronts each rank a quarter of the targets for them, and
// the four sorted lists merge pairwise in LDS. Lane b of a wavefront fetches its b-th target's row
// offset and cost offset; every table read then takes them from that lane as scalars, so the reads
// carry no condition and all of a lane's reads are in flight at once.
constexpr int kCondenseItems = 64;
constexpr int kCondenseWaves = kItemThreads / 64;
constexpr int kTargetsPerWave = kMaxTargets / kCondenseWaves;

template <int K>
__device__ __forceinline__ void insert_key(int32_t (&best)[K], int32_t x) {
#pragma unroll
  for (int s = 0; s < K; ++s) {
    const int32_t lo = min(best[s], x);
    x = max(best[s], x);
    best[s] = lo;
  }
}

// The K smallest of two ascending lists, ascending, into a: min(a[i], b[K-1-i]) holds them as an
// ascending-then-descending sequence, which the bitonic half-cleaners sort.
template <int K>
__device__ __forceinline__ void merge_lists(int32_t (&a)[K], const int32_t (&b)[K]) {
#pragma unroll
  for (int i = 0; i < K; ++i) a[i] = min(a[i], b[K - 1 - i]);
#pragma unroll
  for (int d = K / 2; d >= 1; d >>= 1)
#pragma unroll
    for (int i = 0; i < K; ++i)
      if ((i & d) == 0) {
        const int32_t lo = min(a[i], a[i + d]), hi = max(a[i], a[i + d]);
        a[i] = lo;
        a[i + d] = hi;
      }
}

// Bitonic sorting network over K registers, ascending.
template <int K>
__device__ __forceinline__ void sort_ascending(int32_t (&v)[K]) {
#pragma unroll
  for (int size = 2; size <= K; size <<= 1)
#pragma unroll
    for (int stride = size / 2; stride >= 1; stride >>= 1)
#pragma unroll
      for (int i = 0; i < K; ++i) {
        const int j = i ^ stride;
        if (j > i) {
          const int32_t lo = min(v[i], v[j]), hi = max(v[i], v[j]);
          const bool up = (i & size) == 0;
          v[i] = up ? lo : hi;
          v[j] = up ? hi : lo;
        }
      }
}

template <int DT, int K>
__global__ __launch_bounds__(kItemThreads) void voronoi_condense_kernel(CondenseArgs a) {
  __shared__ int32_t part[2][K][kCondenseItems];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int64_t p = blockIdx.y;
  const int per = (a.M + kCondenseWaves - 1) / kCondenseWaves;
  const int m0 = wave * per, m1 = min(a.M, m0 + per);
  // V * A <= 65528 * 8192 elements, so element offsets fit an int and byte offsets its double.
  const int mb = min(m0 + (lane & (kTargetsPerWave - 1)), a.M - 1);
  const int row_bytes = 2 * static_cast<int>(table_row(a.tokens[p * a.M + mb], a.V)) * a.A;
  const float off = a.offset[p * a.M + mb];
  const int item = blockIdx.x * kCondenseItems + lane;
  const uint32_t item_bytes = 2u * static_cast<uint32_t>(min(item, a.A - 1));
  const __amdgpu_buffer_rsrc_t table = make_rsrc(a.table, 2u * static_cast<uint32_t>(a.V) * static_cast<uint32_t>(a.A));
  uint16_t raw[kTargetsPerWave];
#pragma unroll
  for (int b = 0; b < kTargetsPerWave; ++b)
    raw[b] = __builtin_amdgcn_raw_buffer_load_b16(table, static_cast<int>(item_bytes),
                                                  __builtin_amdgcn_readlane(row_bytes, b), 0);
  int32_t best[K];
#pragma unroll
  for (int s = 0; s < K; ++s) best[s] = INT_MAX;
  // The lane's keys K at a time: each group sorted by a network and merged into the list (about
  // 40 % fewer min/max operations than inserting the keys one by one from K = 4 on). Keys are
  // unique (the target sits in their low bits), so either way gives the same K smallest.
  if constexpr (K >= 4) {
    static_assert(kTargetsPerWave % K == 0, "groups of K keys");
#pragma unroll
    for (int c = 0; c < kTargetsPerWave; c += K) {
      int32_t group[K];
#pragma unroll
      for (int i = 0; i < K; ++i) {
        const int b = c + i;
        group[i] = m0 + b < m1 ? pack_cost(from_bits16<DT>(raw[b]) + lane_value(off, b), m0 + b) : INT_MAX;
      }
      sort_ascending<K>(group);
      merge_lists<K>(best, group);
    }
  } else {
#pragma unroll
    for (int b = 0; b < kTargetsPerWave; ++b)
      if (m0 + b < m1) insert_key<K>(best, pack_cost(from_bits16<DT>(raw[b]) + lane_value(off, b), m0 + b));
  }
  // Waves 1 and 3 hand their lists to 0 and 2, then 2 to 0 (through the slot it read itself).
  if (wave & 1) {
#pragma unroll
    for (int s = 0; s < K; ++s) part[wave >> 1][s][lane] = best[s];
  }
  __syncthreads();
  int32_t other[K];
  if ((wave & 1) == 0) {
#pragma unroll
    for (int s = 0; s < K; ++s) other[s] = part[wave >> 1][s][lane];
    merge_lists<K>(best, other);
    if (wave == 2) {
#pragma unroll
      for (int s = 0; s < K; ++s) part[1][s][lane] = best[s];
    }
  }
  __syncthreads();
  if (wave != 0 || item >= a.A) return;
#pragma unroll
  for (int s = 0; s < K; ++s) other[s] = part[1][s][lane];
  merge_lists<K>(best, other);
#pragma unroll
  for (int s = 0; s < K; ++s) a.key[(p * K + s) * a.A + item] = best[s];
}

// -------------------------------------------------------------------------- 3. fit

struct FitArgs {
  const int32_t* key;     // [N][K][A]
  const int64_t* counts;  // [N][M]
  const float* offset;    // [N][M]
  const float* unit;      // [N]
  float* out;             // [N][M]
  int V, M, A, iterations;
  float epsilon, anneal, relax, limit;
  // Resolve one item per problem after the sweeps (null table: no).
  const uint16_t* table;
  const int64_t* tokens;  // [N][M]
  const int64_t* values;  // [N]
  int64_t* decoded;       // [N]
};

// The loads are sums of up to k * A <= 32768 weights. Each weight w (in [0, 1]) enters as the
// integer round(w 2^31) into one of its target's 64-bit LDS counters (integer adds: the sum is
// exact, so it is the same whatever order the workgroup's adds land in); the factor step reads it
// back as sum 2^-31. Rounding moves a weight by at most 2^-32, and a load by at most its entry count
// times that, which the load floor (1e-2) dwarfs.
constexpr float kFixedScale = 2147483648.0f;  // 2^31: w = 1 is 2^31, a u32
constexpr double kFixedUnit = 1.0 / 2147483648.0;
// The adds of one instruction that land on the same counter are carried out one after another, and
// the popular targets sit in most items' slots: so each target has kLoadCopies counters, laid out
// [target][copy], and lane l adds into copy l % kLoadCopies (at most four lanes of an instruction
// share a counter). The counters are never cleared: the factor step keeps the previous sweep's
// total and takes the difference, exact in unsigned 64-bit arithmetic whatever the running total.
constexpr int kLoadCopies = 16;
constexpr int kCopiesPerThread = kLoadCopies * kMaxTargets / kRowThreads;  // the factor step's share
static_assert(kCopiesPerThread == 2, "the factor step reads one 16-byte pair per thread");

template <int DT, int K, int IPT>
__global__ __launch_bounds__(kRowThreads) void voronoi_fit_kernel(FitArgs a) {
  __shared__ __align__(16) unsigned long long load_fx[kMaxTargets * kLoadCopies];
  __shared__ float corr[kMaxTargets];
  __shared__ float share_s[kMaxTargets];
  __shared__ int live_s[kMaxTargets];
  __shared__ float scale_s;
  __shared__ float best_v[kMaxTargets / 64];
  __shared__ int best_i[kMaxTargets / 64];
  __shared__ int64_t token_s[kMaxTargets];
  const int t = threadIdx.x, lane = t & 63;
  const int64_t p = blockIdx.x;
  const int M = a.M, A = a.A;
  const float u = a.unit[p];
  float temperature = a.epsilon * u;
  const float bound = a.limit * u;
  // A sweep's cost scale -log2(e) / T, formed by one thread and read by all.
  constexpr float kNegLog2e = -1.4426950408889634f;
  if (t < kMaxTargets) {
    const int64_t c = t < M ? a.counts[p * M + t] : 0;
    live_s[t] = c > 0;
    share_s[t] = logf(fmaxf(static_cast<float>(c), 1e-9f));
    corr[t] = 0.f;
    if (t == 0) scale_s = kNegLog2e / temperature;
  }
#pragma unroll
  for (int i = 0; i < kCopiesPerThread; ++i) load_fx[kCopiesPerThread * t + i] = 0ull;
  const int copy = lane % kLoadCopies;

  // What the end reads from memory is requested now, so its round trips overlap the sweeps: the
  // target's offset and, when the problem's one item is resolved, its token and the item.
  const bool resolve = a.table != nullptr;
  float offset_t = 0.f;
  int64_t token = 0, decode_item = 0;
  if (t < M) {
    offset_t = a.offset[p * M + t];
    if (resolve) {
      token = a.tokens[p * M + t];
      decode_item = a.values[p];
    }
  }

  // The condensed problem, decoded once (iterate.py:130-134): thread t holds items t + 1024 q and
  // their K slots: base cost and target.
  float base[IPT][K];
  int target[IPT][K];
  bool valid[IPT];
#pragma unroll
  for (int q = 0; q < IPT; ++q) {
    const int item = t + kRowThreads * q;
    valid[q] = item < A;
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const int32_t key = a.key[(p * K + j) * A + min(item, A - 1)];
      const int32_t carried = key & ~0x7F;
      base[q][j] = __builtin_bit_cast(float, carried >= 0 ? carried : (carried ^ 0x7FFFFFFF));
      target[q][j] = key & 0x7F;
    }
  }
  // The target's table cost at the item (auxiliary.py:70-75), requested behind the keys. Every
  // thread issues this one load (the others from an in-bounds stand-in address, the value unused),
  // so the waits for the keys below leave it in flight on every path.
  decode_item = decode_item < 0 ? 0 : (decode_item > A - 1 ? A - 1 : decode_item);
  const uint16_t* cost_src = resolve ? a.table + table_row(token, a.V) * A + decode_item
                                     : reinterpret_cast<const uint16_t*>(a.counts + p * M);
  uint32_t cost_bits = *cost_src;
  if (resolve && t < M) token_s[t] = token;
  __syncthreads();

  unsigned long long load_before = 0;  // this lane octet's target's counter total after the last sweep
  for (int it = 0; it < a.iterations; ++it) {
    // Each item's softmax over its K slots (iterate.py:142-145), added into the loads
    // (iterate.py:146-149). exp(-cost / T - max) as exp2 of cost * (-log2(e) / T) less its maximum;
    // the scale is negative, so the maximum is the cheapest cost times it (rounding is monotone).
    const float scale = scale_s;
#pragma unroll
    for (int q = 0; q < IPT; ++q) {
      if (!valid[q]) continue;
      float x[K];
      float cmin = INFINITY;
#pragma unroll
      for (int j = 0; j < K; ++j) {
        x[j] = base[q][j] + corr[target[q][j]];
        cmin = fminf(cmin, x[j]);
      }
      const float xm = cmin * scale;
      float se = 0.f;
#pragma unroll
      for (int j = 0; j < K; ++j) {
        x[j] = __builtin_amdgcn_exp2f(fmaf(x[j], scale, -xm));
        se += x[j];
      }
      const float r = __builtin_amdgcn_rcpf(se) * kFixedScale;
#pragma unroll
      for (int j = 0; j < K; ++j) {
        const uint32_t w = static_cast<uint32_t>(fmaf(x[j], r, 0.5f));
        __hip_atomic_fetch_add(&load_fx[target[q][j] * kLoadCopies + copy], static_cast<unsigned long long>(w),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
    __syncthreads();
    // The factor step (iterate.py:150-154). Target m's load: threads 8 m .. 8 m + 7 each add two of
    // its counters, the eight partial sums are joined by DPP inside the lane octet, and the sweep's
    // load is the total less the previous sweep's.
    {
      const int m = t >> 3;
      unsigned long long total = load_fx[kCopiesPerThread * t] + load_fx[kCopiesPerThread * t + 1];
      total += dpp<kDppXor1>(total);
      total += dpp<kDppXor2>(total);
      total += dpp<kDppHalfMirror>(total);
      const unsigned long long fx = total - load_before;
      load_before = total;
      if ((t & 7) == 0 && m < M) {
        const float load = static_cast<float>(static_cast<double>(fx) * kFixedUnit);
        float step = temperature * (logf(fmaxf(load, kLoadFloor)) - share_s[m]);
        step = fminf(fmaxf(step, -bound), bound);
        const float c = corr[m] + a.relax * step;
        corr[m] = live_s[m] ? c : 0.f;
      }
      if (t == 0) scale_s = kNegLog2e / (temperature * a.anneal);
    }
    __syncthreads();
    temperature *= a.anneal;
  }

  // The cost's load is used here on every path, so it stays in flight through the sweeps (no
  // earlier wait, no conversion hoisted above them).
  asm volatile("" : "+v"(cost_bits));
  float bias = 0.f;
  if (t < M) {
    bias = offset_t + corr[t];
    a.out[p * M + t] = bias;
  }
  if (!resolve) return;
  // auxiliary.py:70-75 for this problem's one value: argmin_m C[m, a] + b[m], lowest m on ties.
  if (t < ((M + 63) & ~63)) {
    float v = INFINITY;
    int idx = INT_MAX;
    if (t < M) {
      v = from_bits16<DT>(static_cast<uint16_t>(cost_bits)) + bias;
      idx = t;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(v, off, 64);
      const int oi = __shfl_xor(idx, off, 64);
      if (ov < v || (ov == v && oi < idx)) {
        v = ov;
        idx = oi;
      }
    }
    if (lane == 0) {
      best_v[t >> 6] = v;
      best_i[t >> 6] = idx;
    }
  }
  __syncthreads();
  if (t == 0) {
    float v = best_v[0];
    int idx = best_i[0];
    for (int w = 1; w < (M + 63) / 64; ++w)
      if (best_v[w] < v || (best_v[w] == v && best_i[w] < idx)) {
        v = best_v[w];
        idx = best_i[w];
      }
    a.decoded[p] = token_s[idx];
  }
}

// -------------------------------------------------------------------------- 4. argmin

struct ArgminArgs {
  const uint16_t* table;
  const int64_t* tokens;  // [N][M]
  const float* bias;      // [N][M]
  int64_t* sigma;         // [N][A]
  int V, M, A;
};

template <int DT>
__global__ __launch_bounds__(kItemThreads) void voronoi_argmin_kernel(ArgminArgs a) {
  __shared__ int64_t row_s[kMaxTargets];
  __shared__ float bias_s[kMaxTargets];
  const int t = threadIdx.x;
  const int64_t p = blockIdx.y;
  if (t < a.M) {
    row_s[t] = table_row(a.tokens[p * a.M + t], a.V) * a.A;
    bias_s[t] = a.bias[p * a.M + t];
  }
  __syncthreads();
  const int item = blockIdx.x * kItemThreads + t;
  if (item >= a.A) return;
  float best = from_bits16<DT>(a.table[row_s[0] + item]) + bias_s[0];
  int arg = 0;
  for (int m = 1; m < a.M; ++m) {
    const float c = from_bits16<DT>(a.table[row_s[m] + item]) + bias_s[m];
    if (c < best) {
      best = c;
      arg = m;
    }
  }
  a.sigma[p * a.A + item] = arg;
}

// -------------------------------------------------------------------------- host side

bool pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

template <int DT>
hipError_t launch_shortlist(const ShortArgs& a, int64_t n, hipStream_t s) {
  // elements per thread: the row plus up to 7 tokens before it (the aligned start), in multiples of 8
  const int jt = static_cast<int>((a.V + 7 + kRowThreads - 1) / kRowThreads + 7) / 8 * 8;
  const dim3 grid(static_cast<unsigned>(n)), block(kRowThreads);
  switch (jt) {
#define PLM_VOR_JT(J) \
  case J: hipLaunchKernelGGL((voronoi_shortlist_kernel<DT, J>), grid, block, 0, s, a); break;
    PLM_VOR_JT(8)
    PLM_VOR_JT(16)
    PLM_VOR_JT(24)
    PLM_VOR_JT(32)
    PLM_VOR_JT(40)
    PLM_VOR_JT(48)
    PLM_VOR_JT(56)
    PLM_VOR_JT(64)
#undef PLM_VOR_JT
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int DT>
hipError_t launch_condense(const CondenseArgs& a, int k, int64_t n, hipStream_t s) {
  const dim3 grid((a.A + kCondenseItems - 1) / kCondenseItems, static_cast<unsigned>(n)), block(kItemThreads);
  switch (k) {
    case 1: hipLaunchKernelGGL((voronoi_condense_kernel<DT, 1>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((voronoi_condense_kernel<DT, 2>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((voronoi_condense_kernel<DT, 4>), grid, block, 0, s, a); break;
    case 8: hipLaunchKernelGGL((voronoi_condense_kernel<DT, 8>), grid, block, 0, s, a); break;
    case 16: hipLaunchKernelGGL((voronoi_condense_kernel<DT, 16>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int DT, int K, int IPT>
hipError_t launch_fit_kt(const FitArgs& a, int64_t n, hipStream_t s) {
  if constexpr (K * IPT > 32) {
    return hipErrorInvalidValue;
  } else {
    hipLaunchKernelGGL((voronoi_fit_kernel<DT, K, IPT>), dim3(static_cast<unsigned>(n)), dim3(kRowThreads), 0, s, a);
    return hipGetLastError();
  }
}

template <int DT, int K>
hipError_t launch_fit_k(const FitArgs& a, int64_t n, hipStream_t s) {
  switch (a.A > kRowThreads ? a.A / kRowThreads : 1) {
    case 1: return launch_fit_kt<DT, K, 1>(a, n, s);
    case 2: return launch_fit_kt<DT, K, 2>(a, n, s);
    case 4: return launch_fit_kt<DT, K, 4>(a, n, s);
    case 8: return launch_fit_kt<DT, K, 8>(a, n, s);
    default: return hipErrorInvalidValue;
  }
}

template <int DT>
hipError_t launch_fit(const FitArgs& a, int k, int64_t n, hipStream_t s) {
  switch (k) {
    case 1: return launch_fit_k<DT, 1>(a, n, s);
    case 2: return launch_fit_k<DT, 2>(a, n, s);
    case 4: return launch_fit_k<DT, 4>(a, n, s);
    case 8: return launch_fit_k<DT, 8>(a, n, s);
    case 16: return launch_fit_k<DT, 16>(a, n, s);
    default: return hipErrorInvalidValue;
  }
}

template <int DT>
hipError_t launch_argmin(const ArgminArgs& a, int64_t n, hipStream_t s) {
  const dim3 grid((a.A + kItemThreads - 1) / kItemThreads, static_cast<unsigned>(n)), block(kItemThreads);
  hipLaunchKernelGGL((voronoi_argmin_kernel<DT>), grid, block, 0, s, a);
  return hipGetLastError();
}

int to_status(hipError_t e) { return e == hipSuccess ? PLM_OK : (e == hipErrorInvalidValue ? PLM_ERR_ARGUMENT : PLM_ERR_LAUNCH); }

// Sizes the engine supports (the reference's own limits, auxiliary.py:24-25 and iterate.py:298-300,
// plus the ones this implementation adds): n_targets and k powers of two with k <= n_targets <= 128,
// k <= 16; A a power of two in [64, 8192] with k * max(1, A / 1024) <= 32 (the fit holds a thread's
// k * A / 1024 condensed entries in registers); n_targets <= V <= 65536.
bool sizes_ok(int64_t n, int64_t V, int64_t A, int64_t M, int64_t k) {
  if (n < 1 || n > 65535) return false;
  if (!pow2(M) || M > kMaxTargets || V < M || V > kMaxVocab) return false;
  if (!pow2(A) || A < kMinItems || A > kMaxItems) return false;
  if (k != 0 && (!pow2(k) || k > M || k > kMaxSlots || k * std::max<int64_t>(1, A / kRowThreads) > 32)) return false;
  return true;
}

float anneal_factor(double endpoint, double epsilon, int64_t iterations) {
  return static_cast<float>(std::pow(endpoint / epsilon, 1.0 / static_cast<double>(std::max<int64_t>(iterations, 1))));
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

struct AssignLayout {
  size_t tokens, counts, unit, bias0, bias1, key, total;
};

// After the shared workspace's counter area (left untouched), like every other entry point's.
AssignLayout assign_layout(int64_t n, int64_t M, int64_t k, int64_t A) {
  AssignLayout l{};
  size_t o = kCounterBytes;
  l.tokens = o;
  o += align256(n * M * sizeof(int64_t));
  l.counts = o;
  o += align256(n * M * sizeof(int64_t));
  l.unit = o;
  o += align256(n * sizeof(float));
  l.bias0 = o;
  o += align256(n * M * sizeof(float));
  l.bias1 = o;
  o += align256(n * M * sizeof(float));
  l.key = o;
  o += align256(n * k * A * sizeof(int32_t));
  l.total = o;
  return l;
}

}  // namespace
}  // namespace plm

extern "C" {

int plm_voronoi_shortlist(int32_t dtype, const void* logits, int64_t ld_logits, const void* table, int64_t n_problems,
                          int64_t n_vocab, int64_t n_items, int64_t n_targets, float weight, int64_t* tokens,
                          int64_t* counts, float* values, float* unit, float* prior, float* normaliser, void* stream) {
  if (logits == nullptr || table == nullptr || tokens == nullptr || counts == nullptr || unit == nullptr ||
      prior == nullptr)
    return PLM_ERR_ARGUMENT;
  if (dtype != PLM_BF16 && dtype != PLM_F16) return PLM_ERR_ARGUMENT;
  if (!plm::sizes_ok(n_problems, n_vocab, n_items, n_targets, 0) || ld_logits < n_vocab) return PLM_ERR_ARGUMENT;
  plm::ShortArgs a{static_cast<const uint16_t*>(logits), ld_logits, static_cast<const uint16_t*>(table),
                   static_cast<int>(n_vocab), static_cast<int>(n_items), static_cast<int>(n_targets), weight,
                   tokens, counts, values, unit, prior, normaliser};
  const hipStream_t s = static_cast<hipStream_t>(stream);
  return plm::to_status(dtype == PLM_BF16 ? plm::launch_shortlist<plm::DT_BF16>(a, n_problems, s)
                                          : plm::launch_shortlist<plm::DT_F16>(a, n_problems, s));
}

int plm_voronoi_spread(int32_t dtype, const void* table, int64_t n_vocab, int64_t n_items, const int64_t* tokens,
                       int64_t n_problems, int64_t n_targets, int64_t sample, float* unit, void* stream) {
  if (table == nullptr || tokens == nullptr || unit == nullptr) return PLM_ERR_ARGUMENT;
  if (dtype != PLM_BF16 && dtype != PLM_F16) return PLM_ERR_ARGUMENT;
  if (!plm::sizes_ok(n_problems, n_vocab, n_items, n_targets, 0) || sample < 1 || sample > 64) return PLM_ERR_ARGUMENT;
  plm::SpreadArgs a{static_cast<const uint16_t*>(table), tokens, unit, static_cast<int>(n_vocab),
                    static_cast<int>(n_targets), static_cast<int>(n_items), static_cast<int>(sample)};
  const dim3 grid(static_cast<unsigned>(n_problems)), block(1024);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == PLM_BF16)
    hipLaunchKernelGGL((plm::voronoi_spread_kernel<plm::DT_BF16>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((plm::voronoi_spread_kernel<plm::DT_F16>), grid, block, 0, s, a);
  return plm::to_status(hipGetLastError());
}

int plm_voronoi_prior(const int64_t* counts, const float* unit, int64_t n_problems, int64_t n_targets, int64_t n_items,
                      float weight, float* prior, void* stream) {
  if (counts == nullptr || unit == nullptr || prior == nullptr) return PLM_ERR_ARGUMENT;
  if (!plm::sizes_ok(n_problems, n_targets, n_items, n_targets, 0)) return PLM_ERR_ARGUMENT;
  hipLaunchKernelGGL(plm::voronoi_prior_kernel, dim3(static_cast<unsigned>(n_problems)), dim3(128), 0,
                     static_cast<hipStream_t>(stream), counts, unit, prior, static_cast<int>(n_targets),
                     static_cast<int>(n_items), weight);
  return plm::to_status(hipGetLastError());
}

int plm_voronoi_condense(int32_t dtype, const void* table, int64_t n_vocab, int64_t n_items, const int64_t* tokens,
                         const float* offset, int64_t n_problems, int64_t n_targets, int64_t k, int32_t* key,
                         void* stream) {
  if (table == nullptr || tokens == nullptr || offset == nullptr || key == nullptr) return PLM_ERR_ARGUMENT;
  if (dtype != PLM_BF16 && dtype != PLM_F16) return PLM_ERR_ARGUMENT;
  if (!plm::sizes_ok(n_problems, n_vocab, n_items, n_targets, k) || k < 1) return PLM_ERR_ARGUMENT;
  plm::CondenseArgs a{static_cast<const uint16_t*>(table), tokens, offset, key, static_cast<int>(n_vocab),
                      static_cast<int>(n_targets), static_cast<int>(n_items)};
  const hipStream_t s = static_cast<hipStream_t>(stream);
  return plm::to_status(dtype == PLM_BF16 ? plm::launch_condense<plm::DT_BF16>(a, static_cast<int>(k), n_problems, s)
                                          : plm::launch_condense<plm::DT_F16>(a, static_cast<int>(k), n_problems, s));
}

int plm_voronoi_fit(const int32_t* key, const int64_t* counts, const float* offset, const float* unit,
                    int64_t n_problems, int64_t n_targets, int64_t k, int64_t n_items, int64_t iterations,
                    float epsilon, float relax, float endpoint, float limit, float* out, void* stream) {
  if (key == nullptr || counts == nullptr || offset == nullptr || unit == nullptr || out == nullptr)
    return PLM_ERR_ARGUMENT;
  if (!plm::sizes_ok(n_problems, n_targets, n_items, n_targets, k) || k < 1 || iterations < 0 ||
      iterations > (1 << 20) || !(epsilon > 0.f) || !(endpoint > 0.f))
    return PLM_ERR_ARGUMENT;
  plm::FitArgs a{};
  a.key = key;
  a.counts = counts;
  a.offset = offset;
  a.unit = unit;
  a.out = out;
  a.M = static_cast<int>(n_targets);
  a.A = static_cast<int>(n_items);
  a.iterations = static_cast<int>(iterations);
  a.epsilon = epsilon;
  a.anneal = plm::anneal_factor(endpoint, epsilon, iterations);
  a.relax = relax;
  a.limit = limit;
  return plm::to_status(plm::launch_fit<plm::DT_BF16>(a, static_cast<int>(k), n_problems, static_cast<hipStream_t>(stream)));
}

int plm_voronoi_argmin(int32_t dtype, const void* table, int64_t n_vocab, int64_t n_items, const int64_t* tokens,
                       const float* bias, int64_t n_problems, int64_t n_targets, int64_t* sigma, void* stream) {
  if (table == nullptr || tokens == nullptr || bias == nullptr || sigma == nullptr) return PLM_ERR_ARGUMENT;
  if (dtype != PLM_BF16 && dtype != PLM_F16) return PLM_ERR_ARGUMENT;
  if (!plm::sizes_ok(n_problems, n_vocab, n_items, n_targets, 0)) return PLM_ERR_ARGUMENT;
  plm::ArgminArgs a{static_cast<const uint16_t*>(table), tokens, bias, sigma, static_cast<int>(n_vocab),
                    static_cast<int>(n_targets), static_cast<int>(n_items)};
  const hipStream_t s = static_cast<hipStream_t>(stream);
  return plm::to_status(dtype == PLM_BF16 ? plm::launch_argmin<plm::DT_BF16>(a, n_problems, s)
                                          : plm::launch_argmin<plm::DT_F16>(a, n_problems, s));
}

size_t plm_voronoi_assign_workspace_bytes(int64_t n_problems, int64_t n_targets, int64_t k, int64_t n_items) {
  if (n_problems < 1 || n_targets < 1 || k < 1 || n_items < 1) return 0;
  return plm::assign_layout(n_problems, n_targets, k, n_items).total;
}

int plm_voronoi_assign(int32_t dtype, const void* logits, int64_t ld_logits, const void* table, int64_t n_problems,
                       int64_t n_vocab, int64_t n_items, int64_t n_targets, int64_t k, int64_t rounds,
                       int64_t iterations, float weight, float epsilon, float refocus, float relax, float endpoint,
                       float limit, const int64_t* values, int64_t* decoded, int64_t* tokens_out,
                       int64_t* counts_out, float* bias_out, int64_t* sigma, void* workspace, size_t workspace_bytes,
                       void* stream) {
  if (logits == nullptr || table == nullptr) return PLM_ERR_ARGUMENT;
  if (dtype != PLM_BF16 && dtype != PLM_F16) return PLM_ERR_ARGUMENT;
  if ((values == nullptr) != (decoded == nullptr)) return PLM_ERR_ARGUMENT;
  if (!plm::sizes_ok(n_problems, n_vocab, n_items, n_targets, k) || k < 1 || ld_logits < n_vocab) return PLM_ERR_ARGUMENT;
  if (rounds < 1 || rounds > 64 || iterations < 0 || iterations > (1 << 20) || !(epsilon > 0.f) || !(endpoint > 0.f) ||
      !(refocus > 0.f))
    return PLM_ERR_ARGUMENT;
  const plm::AssignLayout l = plm::assign_layout(n_problems, n_targets, k, n_items);
  if (workspace == nullptr || workspace_bytes < l.total || !plm::aligned16_ptr(workspace)) return PLM_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  int64_t* tokens = tokens_out != nullptr ? tokens_out : reinterpret_cast<int64_t*>(ws + l.tokens);
  int64_t* counts = counts_out != nullptr ? counts_out : reinterpret_cast<int64_t*>(ws + l.counts);
  float* unit = reinterpret_cast<float*>(ws + l.unit);
  float* bias[2] = {reinterpret_cast<float*>(ws + l.bias0), reinterpret_cast<float*>(ws + l.bias1)};
  int32_t* key = reinterpret_cast<int32_t*>(ws + l.key);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf16 = dtype == PLM_BF16;

  plm::ShortArgs sa{static_cast<const uint16_t*>(logits), ld_logits, static_cast<const uint16_t*>(table),
                    static_cast<int>(n_vocab), static_cast<int>(n_items), static_cast<int>(n_targets), weight,
                    tokens, counts, nullptr, unit, bias[0], nullptr};
  hipError_t err = bf16 ? plm::launch_shortlist<plm::DT_BF16>(sa, n_problems, s)
                        : plm::launch_shortlist<plm::DT_F16>(sa, n_problems, s);
  if (err != hipSuccess) return plm::to_status(err);
  // iterate.py:336-340: each round condenses against the current factors and refits them; the
  // second and later rounds anneal from epsilon * refocus.
  for (int64_t r = 0; r < rounds; ++r) {
    float* offset = bias[r & 1];
    const bool last = r == rounds - 1;
    float* out = last && bias_out != nullptr ? bias_out : bias[(r + 1) & 1];
    plm::CondenseArgs ca{static_cast<const uint16_t*>(table), tokens, offset, key, static_cast<int>(n_vocab),
                         static_cast<int>(n_targets), static_cast<int>(n_items)};
    err = bf16 ? plm::launch_condense<plm::DT_BF16>(ca, static_cast<int>(k), n_problems, s)
               : plm::launch_condense<plm::DT_F16>(ca, static_cast<int>(k), n_problems, s);
    if (err != hipSuccess) return plm::to_status(err);
    const double eps = r == 0 ? static_cast<double>(epsilon) : static_cast<double>(epsilon) * static_cast<double>(refocus);
    plm::FitArgs fa{};
    fa.key = key;
    fa.counts = counts;
    fa.offset = offset;
    fa.unit = unit;
    fa.out = out;
    fa.V = static_cast<int>(n_vocab);
    fa.M = static_cast<int>(n_targets);
    fa.A = static_cast<int>(n_items);
    fa.iterations = static_cast<int>(iterations);
    fa.epsilon = static_cast<float>(eps);
    fa.anneal = plm::anneal_factor(endpoint, eps, iterations);
    fa.relax = relax;
    fa.limit = limit;
    if (last && values != nullptr) {
      fa.table = static_cast<const uint16_t*>(table);
      fa.tokens = tokens;
      fa.values = values;
      fa.decoded = decoded;
    }
    err = bf16 ? plm::launch_fit<plm::DT_BF16>(fa, static_cast<int>(k), n_problems, s)
               : plm::launch_fit<plm::DT_F16>(fa, static_cast<int>(k), n_problems, s);
    if (err != hipSuccess) return plm::to_status(err);
    if (last && out != bias[(r + 1) & 1]) bias[(r + 1) & 1] = out;
  }
  if (sigma != nullptr) {
    plm::ArgminArgs aa{static_cast<const uint16_t*>(table), tokens, bias[rounds & 1], sigma,
                       static_cast<int>(n_vocab), static_cast<int>(n_targets), static_cast<int>(n_items)};
    err = bf16 ? plm::launch_argmin<plm::DT_BF16>(aa, n_problems, s) : plm::launch_argmin<plm::DT_F16>(aa, n_problems, s);
    if (err != hipSuccess) return plm::to_status(err);
  }
  return PLM_OK;
}

}  // extern "C"
