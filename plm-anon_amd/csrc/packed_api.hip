// C ABI of the packed-weight GEMM: weight packing (plm_pack_weight) and the GEMM over packed
// weights (plm_gemm_packed), declared in include/plm_amd.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "packed_gemm.h"
#include "plm_amd.h"
#include "wide_gemm.h"

namespace plm {

// The fragment (row f, K step s) stored at fragment index `frag` of a packed weight with `rows`
// fragment rows (the order tile.h describes: groups of kPackGroup steps, all rows per group).
__device__ __forceinline__ void packed_frag_at(int64_t frag, int rows, int& f, int& s) {
  const int64_t per_group = static_cast<int64_t>(rows) * kPackGroup;
  const int g = static_cast<int>(frag / per_group);
  const int rem = static_cast<int>(frag - g * per_group);
  f = rem / kPackGroup;
  s = g * kPackGroup + rem % kPackGroup;
}

// Weight packing: thread i writes lane (i % 64) of the fragment stored at i / 64 (16 bytes, zeros
// past N or K, so the padding rows and steps are zero fragments).
__global__ __launch_bounds__(256) void pack_weight_kernel(const uint16_t* __restrict__ w, int64_t ldw, int N, int K,
                                                         int rows, int64_t lanes, u32x4* __restrict__ out) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < lanes;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int lane = static_cast<int>(i & 63);
    int f, s;
    packed_frag_at(i >> 6, rows, f, s);
    const int n = 16 * f + (lane & 15), k = 32 * s + 8 * (lane >> 4);
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (n < N && k < K) v = *reinterpret_cast<const u32x4*>(w + static_cast<int64_t>(n) * ldw + k);
    out[i] = v;
  }
}

// The inverse of pack_weight_kernel: thread i writes lane (i % 64) of the fragment stored at i / 64
// back to its 16 bytes of the row-major W (padding past N or K is dropped).
__global__ __launch_bounds__(256) void unpack_weight_kernel(const u32x4* __restrict__ packed, int N, int K, int rows,
                                                           int64_t lanes, uint16_t* __restrict__ w, int64_t ldw) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < lanes;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int lane = static_cast<int>(i & 63);
    int f, s;
    packed_frag_at(i >> 6, rows, f, s);
    const int n = 16 * f + (lane & 15), k = 32 * s + 8 * (lane >> 4);
    if (n < N && k < K) *reinterpret_cast<u32x4*>(w + static_cast<int64_t>(n) * ldw + k) = packed[i];
  }
}

namespace {

constexpr int64_t kPackedMaxM = 128;

int packed_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  static int cached_dev = -1, cached = 0;
  if (dev != cached_dev) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cached_dev = dev;
    cached = cus;
  }
  return cached;
}

int64_t ksteps(int64_t K) { return (K + 31) / 32; }

int64_t packed_bytes(int64_t N, int64_t K) { return pack_bytes(N, ksteps(K)); }

// k_waves = 4, 8, 16: the workgroup's k_waves wavefronts split the tile's K range (tile =
// 16*wave_frags rows); k_waves = 1: each of four wavefronts takes its own 16*wave_frags rows
// (tile = 64*wave_frags rows).
bool packed_tile_valid(const plm_tile* t) {
  return t != nullptr && (t->wave_frags == 1 || t->wave_frags == 2 || t->wave_frags == 4) &&
         (t->k_waves == 1 || t->k_waves == 4 || t->k_waves == 8 || t->k_waves == 16) && t->split_k >= 1 &&
         t->split_k <= 64 &&
         (t->unroll == 2 || t->unroll == 4 || t->unroll == 6 || t->unroll == 8);
}

// The compiled kernels of one (epilogue, dtype, workgroup layout), per translation unit.
using PackedDispatch = hipError_t (*)(PackedArgs&, int, int, int, hipStream_t, bool);

hipError_t packed_dispatch_dt(int32_t dtype, PackedArgs& a, const plm_tile& t, int cus, hipStream_t s, bool dry,
                              int epi = kEpiPlain) {
  static const PackedDispatch table[3][2][4] = {
      {{packed_dispatch_bf16_k1, packed_dispatch_bf16_k4, packed_dispatch_bf16_k8, packed_dispatch_bf16_k16},
       {packed_dispatch_f16_k1, packed_dispatch_f16_k4, packed_dispatch_f16_k8, packed_dispatch_f16_k16}},
      {{packed_dispatch_lora_bf16_k1, packed_dispatch_lora_bf16_k4, packed_dispatch_lora_bf16_k8,
        packed_dispatch_lora_bf16_k16},
       {packed_dispatch_lora_f16_k1, packed_dispatch_lora_f16_k4, packed_dispatch_lora_f16_k8,
        packed_dispatch_lora_f16_k16}},
      {{packed_dispatch_act_bf16_k1, packed_dispatch_act_bf16_k4, packed_dispatch_act_bf16_k8,
        packed_dispatch_act_bf16_k16},
       {packed_dispatch_act_f16_k1, packed_dispatch_act_f16_k4, packed_dispatch_act_f16_k8,
        packed_dispatch_act_f16_k16}}};
  const int di = dtype == PLM_BF16 ? 0 : (dtype == PLM_F16 ? 1 : -1);
  const int ki = t.k_waves == 1 ? 0 : t.k_waves == 4 ? 1 : t.k_waves == 8 ? 2 : t.k_waves == 16 ? 3 : -1;
  if (di < 0 || ki < 0 || epi < kEpiPlain || epi > kEpiAct) return hipErrorInvalidConfiguration;
  return table[epi][di][ki](a, t.wave_frags, t.unroll, cus, s, dry);
}

// Weight fragments (16 rows each) of one workgroup tile.
int64_t tile_fragments(const plm_tile& t) { return t.k_waves == 1 ? kPackedWaves * t.wave_frags : t.wave_frags; }

int64_t packed_tiles(int64_t N, const plm_tile& t) { return ((N + 15) / 16 + tile_fragments(t) - 1) / tile_fragments(t); }

// Workspace: the counter area, then (split > 1) one fp32 fragment per (tile, split, fragment).
int64_t packed_workspace(int64_t M, int64_t N, const plm_tile& t) {
  if (t.split_k <= 1) return 0;
  const int64_t mt = (M + 15) / 16;
  return static_cast<int64_t>(kCounterBytes) + packed_tiles(N, t) * t.split_k * tile_fragments(t) * mt * kFragBytes;
}

// Gated-LoRA launch (one launch: the h linear's items, then the base linear's). The h linear runs
// on the base linear's tile with its own K split, so that each wavefront of an h item keeps at
// least one pipeline's depth of K steps (at most 8 splits); its few items then end early.
// Workspace: the counter area, the base linear's split partials, the h linear's, then h in the
// model dtype for every row ([M][shards*rank], 256-aligned).
struct LoraLayout {
  int64_t h_split, h_tiles, h_partial, h_offset, bytes;  // h_partial: float offset of h's partials
};

LoraLayout lora_layout(int64_t M, int64_t N, int64_t K, int64_t width, const plm_tile& t) {
  LoraLayout l{};
  const int64_t waves = t.k_waves == 1 ? 1 : t.k_waves;
  l.h_split = std::min<int64_t>(8, std::max<int64_t>(1, ksteps(K) / (waves * t.unroll)));
  l.h_tiles = packed_tiles(width, t);
  const int64_t mt = (M + 15) / 16, per_tile = tile_fragments(t) * mt * (kFragBytes / 4);
  const int64_t base = t.split_k > 1 ? packed_tiles(N, t) * t.split_k * per_tile : 0;
  const int64_t h = l.h_split > 1 ? l.h_tiles * l.h_split * per_tile : 0;
  l.h_partial = base;
  l.h_offset = (static_cast<int64_t>(kCounterBytes) + (base + h) * 4 + 255) / 256 * 256;
  l.bytes = l.h_offset + M * width * 2;
  return l;
}

constexpr int kPackedSpinLimit = 1 << 20;  // polls (each one device round trip) before a wait gives up
// Counter area of a packed launch: split arrival counters from kPackedArriveBase, progress flags
// of a chain (an int64 per workgroup) from kPackedBarrierBase.

// Y columns of a linear: N, or N/2 for the SiLU-and-multiply epilogue.
int64_t out_cols(const plm_chain_gemm& g) { return g.out_f32 == PLM_OUT_SILU_MUL ? g.N / 2 : g.N; }

// Checks one linear's operands (W packed); returns PLM_OK or the status to report. `tile` given:
// the SiLU-and-multiply epilogue is allowed (gate and up fragments pair up inside a wavefront's
// or a tile's fragments, and the output's 16-column blocks are whole).
int packed_check_linear(int32_t dtype, const plm_chain_gemm& g, int64_t M, const plm_tile* tile = nullptr) {
  if (g.x == nullptr || g.w == nullptr || g.y == nullptr) return PLM_ERR_ARGUMENT;
  if (dtype != PLM_BF16 && dtype != PLM_F16) return PLM_ERR_ARGUMENT;
  const bool act = g.out_f32 == PLM_OUT_SILU_MUL;
  if (g.out_f32 != PLM_OUT_MODEL && g.out_f32 != PLM_OUT_F32 && !(act && tile != nullptr)) return PLM_ERR_ARGUMENT;
  if (act && (tile->wave_frags % 2 != 0 || g.N % 32 != 0 || g.ldy % 4 != 0)) return PLM_ERR_ARGUMENT;
  if (M < 1 || M > kPackedMaxM || g.N < 1 || g.K < 8 || g.K > (1 << 24) || g.K % 8 != 0 || g.ldx < g.K ||
      g.ldy < out_cols(g))
    return PLM_ERR_ARGUMENT;
  if (g.split_k < 1 || g.split_k > 64) return PLM_ERR_ARGUMENT;
  if (act && (reinterpret_cast<uintptr_t>(g.y) & 7) != 0) return PLM_ERR_ALIGNMENT;
  // 32-bit buffer offsets: X and the packed weights must each span less than 2 GiB.
  if (M * g.ldx * 2 >= (int64_t(1) << 31) || packed_bytes(g.N, g.K) >= (int64_t(1) << 31)) return PLM_ERR_ARGUMENT;
  if (g.ldx % 8 != 0 || (reinterpret_cast<uintptr_t>(g.x) & 15) != 0 || (reinterpret_cast<uintptr_t>(g.w) & 15) != 0)
    return PLM_ERR_ALIGNMENT;
  return PLM_OK;
}

int packed_launch_args(int32_t dtype, PackedArgs& a, const plm_tile& t, void* workspace, size_t workspace_bytes,
                       int64_t need, hipStream_t s, int epi = kEpiPlain) {
  if (need > 0 && (workspace == nullptr || static_cast<int64_t>(workspace_bytes) < need ||
                   (reinterpret_cast<uintptr_t>(workspace) & 15) != 0))
    return PLM_ERR_WORKSPACE;
  const int cus = packed_cus();
  if (cus <= 0) return PLM_ERR_LAUNCH;
  a.counters = need > 0 ? static_cast<int*>(workspace) : nullptr;
  a.partial = need > 0 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes) : nullptr;
  a.spin_limit = kPackedSpinLimit;
  if (packed_dispatch_dt(dtype, a, t, cus, s, true, epi) != hipSuccess) return PLM_ERR_TILE;
  return packed_dispatch_dt(dtype, a, t, cus, s, false, epi) == hipSuccess ? PLM_OK : PLM_ERR_LAUNCH;
}

int packed_entry(int32_t dtype, const void* x, int64_t ldx, const void* wp, void* y, int64_t ldy, int64_t M, int64_t N,
                 int64_t K, const plm_tile* tile, void* workspace, size_t workspace_bytes, void* stream, int out_f32) {
  if (!packed_tile_valid(tile)) return PLM_ERR_TILE;
  const plm_tile& t = *tile;
  if (N < 1 || N > (int64_t(1) << 30) || K > (int64_t(1) << 30)) return PLM_ERR_ARGUMENT;
  plm_chain_gemm g{};
  g.x = x;
  g.w = wp;
  g.y = y;
  g.ldx = ldx;
  g.ldw = K;
  g.ldy = ldy;
  g.N = static_cast<int32_t>(N);
  g.K = static_cast<int32_t>(K);
  g.split_k = t.split_k;
  g.dep = -1;
  g.out_f32 = out_f32;
  const int status = packed_check_linear(dtype, g, M);
  if (status != PLM_OK) return status;
  const int64_t tiles = packed_tiles(N, t);
  if (t.split_k > 1 && tiles > kPackedBarrierBase - kPackedArriveBase) return PLM_ERR_ARGUMENT;
  g.arrive_base = kPackedArriveBase;
  PackedArgs a{};
  a.single = g;
  a.count = 1;
  a.M = static_cast<int>(M);
  a.G = static_cast<int>(tiles * t.split_k);
  return packed_launch_args(dtype, a, t, workspace, workspace_bytes, packed_workspace(M, N, t),
                            static_cast<hipStream_t>(stream));
}

// Widths past 128 rows (prefill chunks, plm/rounds.py:16, which the reference hands to F.linear)
// run on the wide kernel (csrc/wide_gemm.hip: 128 x 128 tiles staged through LDS, K split for thin
// shapes); the tile configuration applies to the skinny kernel only and is checked for validity.
// Every argument is checked before the launch.
int packed_rows(int32_t dtype, const void* x, int64_t ldx, const void* wp, void* y, int64_t ldy, int64_t M, int64_t N,
                int64_t K, const plm_tile* tile, void* workspace, size_t workspace_bytes, void* stream, int out_f32,
                int64_t cap = kNoCap) {
  if (M <= kPackedMaxM) return packed_entry(dtype, x, ldx, wp, y, ldy, M, N, K, tile, workspace, workspace_bytes, stream, out_f32);
  if (!packed_tile_valid(tile)) return PLM_ERR_TILE;
  if (N < 1 || N > (int64_t(1) << 30) || K > (int64_t(1) << 30)) return PLM_ERR_ARGUMENT;
  plm_chain_gemm g{};
  g.x = x;
  g.w = wp;
  g.y = y;
  g.ldx = ldx;
  g.ldw = K;
  g.ldy = ldy;
  g.N = static_cast<int32_t>(N);
  g.K = static_cast<int32_t>(K);
  g.split_k = 1;
  g.out_f32 = out_f32;
  const int status = packed_check_linear(dtype, g, kPackedMaxM);  // the checks but the width's
  if (status != PLM_OK) return status;
  if (M > (int64_t(1) << 24) || M * ldx * 2 >= (int64_t(1) << 31)) return PLM_ERR_ARGUMENT;
  return wide_gemm(dtype, x, ldx, wp, y, ldy, M, N, K, workspace, workspace_bytes, static_cast<hipStream_t>(stream),
                   out_f32, cap);
}

// How the linears of a chain wait for the ones they read: 0 (none reads another), 2 (every linear
// after the first reads the one before it, none that is read has more tiles than a parity set of
// tile flags holds, and every Y that is read starts on a 128-byte boundary with rows a multiple of
// 128 bytes apart: per-wavefront waits on the producer's tile-done flags, widened to whole
// 128-byte lines of one row; the last linear, read by none, raises no flags), or 1 (otherwise: a
// grid barrier after every linear that is read).
int packed_chain_mode(const plm_chain_gemm* g, int32_t count, const plm_tile& t) {
  bool any = false, pure = count > 1;
  for (int32_t i = 0; i < count; ++i) {
    any = any || g[i].dep >= 0;
    if (i > 0 && g[i].dep != i - 1) pure = false;
    if (i + 1 < count) {
      if (packed_tiles(g[i].N, t) > kPkTileFlags) pure = false;
      if ((reinterpret_cast<uintptr_t>(g[i].y) & 127) != 0 || g[i].ldy % 64 != 0) pure = false;
    }
  }
  return pure ? 2 : (any ? 1 : 0);
}

// Derived fields of a packed chain; returns the workspace bytes or a negative status. Consumed
// linears are numbered 1, 2, ... (done_base): the progress-flag value (grid-barrier mode) or the
// tile-flag value and parity set (tile-flag mode). Grid-barrier mode reuses the split arrival
// counters and partials after every barrier (all earlier linears are finished there); tile-flag
// mode has no point where every workgroup is past a linear, so each linear gets its own.
int64_t packed_prepare(plm_chain_gemm* g, int32_t count, int64_t M, const plm_tile& t) {
  for (int32_t i = 0; i < count; ++i) g[i].consumed = 0;
  for (int32_t i = 0; i < count; ++i) {
    if (g[i].dep < -1 || g[i].dep >= i) return PLM_ERR_ARGUMENT;
    if (g[i].dep >= 0) g[g[i].dep].consumed = 1;
    if (g[i].N < 1 || g[i].split_k < 1 || g[i].split_k > 64) return PLM_ERR_ARGUMENT;
  }
  const int mode = packed_chain_mode(g, count, t);
  const int64_t mt = (M + 15) / 16;
  int64_t arrive = kPackedArriveBase, seq = 0, partial = 0, most_partial = 0;
  for (int32_t i = 0; i < count; ++i) {
    plm_tile ti = t;
    ti.split_k = g[i].split_k;
    const int64_t tiles = packed_tiles(g[i].N, ti);
    g[i].arrive_base = 0;
    g[i].done_base = 0;
    g[i].partial_offset = 0;
    if (g[i].split_k > 1) {
      g[i].arrive_base = static_cast<int32_t>(arrive);
      g[i].partial_offset = partial;
      arrive += tiles;
      const int64_t floats = tiles * g[i].split_k * tile_fragments(t) * mt * (kFragBytes / 4);
      if (floats * 4 >= (int64_t(1) << 31)) return PLM_ERR_ARGUMENT;
      partial += floats;
      most_partial = std::max(most_partial, partial);
      if (arrive > kPackedBarrierBase) return PLM_ERR_ARGUMENT;
    }
    if (g[i].consumed) {
      g[i].done_base = static_cast<int32_t>(++seq);
      if (seq >= (1 << 16)) return PLM_ERR_ARGUMENT;
      if (mode == 1) {
        arrive = kPackedArriveBase;  // everything before the barrier is finished
        partial = 0;
      }
    }
  }
  return static_cast<int64_t>(kCounterBytes) + most_partial * 4;
}

struct PSpan {
  uintptr_t lo, hi;
  bool overlaps(const PSpan& o) const { return lo < o.hi && o.lo < hi; }
};
PSpan pspan(const void* p, int64_t rows, int64_t ld, int64_t cols, int64_t elem) {
  const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
  return PSpan{lo, lo + static_cast<uintptr_t>(((rows - 1) * ld + cols) * elem)};
}

}  // namespace

int packed_gemm_call(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, void* y, int64_t ldy, int64_t M,
                     int64_t N, int64_t K, const plm_tile* tile, void* workspace, size_t workspace_bytes, void* stream,
                     int out_f32, int64_t cap) {
  return packed_rows(dtype, x, ldx, packed_w, y, ldy, M, N, K, tile, workspace, workspace_bytes, stream, out_f32, cap);
}

int64_t packed_gemm_workspace(int64_t M, int64_t N, int64_t K, const plm_tile* tile, int64_t cap) {
  if (!packed_tile_valid(tile) || M < 1 || N < 1 || K < 1) return -1;
  return M > kPackedMaxM ? wide_workspace(M, N, K, cap) : packed_workspace(M, N, *tile);
}

}  // namespace plm

extern "C" {

size_t plm_packed_weight_bytes(int64_t N, int64_t K) {
  if (N < 1 || K < 1) return 0;
  return static_cast<size_t>(plm::packed_bytes(N, K));
}

int plm_pack_weight(int32_t dtype, const void* w, int64_t ldw, int64_t N, int64_t K, void* packed, size_t packed_bytes,
                    void* stream) {
  if (w == nullptr || packed == nullptr || (dtype != PLM_BF16 && dtype != PLM_F16)) return PLM_ERR_ARGUMENT;
  if (N < 1 || K < 8 || K % 8 != 0 || ldw < K) return PLM_ERR_ARGUMENT;
  if (ldw % 8 != 0 || (reinterpret_cast<uintptr_t>(w) & 15) != 0 || (reinterpret_cast<uintptr_t>(packed) & 15) != 0)
    return PLM_ERR_ALIGNMENT;
  const int64_t bytes = plm::packed_bytes(N, K);
  if (static_cast<int64_t>(packed_bytes) < bytes) return PLM_ERR_WORKSPACE;
  if (N > (int64_t(1) << 30) || K > (int64_t(1) << 30)) return PLM_ERR_ARGUMENT;
  const int64_t lanes = bytes / 16;
  const int64_t blocks = std::min<int64_t>((lanes + 255) / 256, 65536);
  hipLaunchKernelGGL(plm::pack_weight_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(w), ldw, static_cast<int>(N),
                     static_cast<int>(K), static_cast<int>(plm::pack_rows(N)), lanes, static_cast<plm::u32x4*>(packed));
  return hipGetLastError() == hipSuccess ? PLM_OK : PLM_ERR_LAUNCH;
}

int plm_unpack_weight(int32_t dtype, const void* packed, size_t packed_bytes, int64_t N, int64_t K, void* w, int64_t ldw,
                      void* stream) {
  if (w == nullptr || packed == nullptr || (dtype != PLM_BF16 && dtype != PLM_F16)) return PLM_ERR_ARGUMENT;
  if (N < 1 || K < 8 || K % 8 != 0 || ldw < K || N > (int64_t(1) << 30) || K > (int64_t(1) << 30))
    return PLM_ERR_ARGUMENT;
  if (ldw % 8 != 0 || (reinterpret_cast<uintptr_t>(w) & 15) != 0 || (reinterpret_cast<uintptr_t>(packed) & 15) != 0)
    return PLM_ERR_ALIGNMENT;
  const int64_t bytes = plm::packed_bytes(N, K);
  if (static_cast<int64_t>(packed_bytes) < bytes) return PLM_ERR_ARGUMENT;
  const int64_t lanes = bytes / 16;
  const int64_t blocks = std::min<int64_t>((lanes + 255) / 256, 65536);
  hipLaunchKernelGGL(plm::unpack_weight_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const plm::u32x4*>(packed), static_cast<int>(N),
                     static_cast<int>(K), static_cast<int>(plm::pack_rows(N)), lanes, static_cast<uint16_t*>(w), ldw);
  return hipGetLastError() == hipSuccess ? PLM_OK : PLM_ERR_LAUNCH;
}

size_t plm_gemm_packed_workspace_bytes(int64_t M, int64_t N, int64_t K, const plm_tile* tile) {
  const int64_t n = plm::packed_gemm_workspace(M, N, K, tile);
  return n < 0 ? 0 : static_cast<size_t>(n);
}

int plm_gemm_packed_tile_supported(int32_t dtype, int64_t M, int64_t K, const plm_tile* tile) {
  if (!plm::packed_tile_valid(tile) || M < 1 || K < 8) return 0;
  if (M > plm::kPackedMaxM) return dtype == PLM_BF16 || dtype == PLM_F16 ? 1 : 0;  // the wide kernel
  plm::PackedArgs a{};
  a.M = static_cast<int>(M);
  return plm::packed_dispatch_dt(dtype, a, *tile, 1, nullptr, true) == hipSuccess ? 1 : 0;
}

int plm_gemm_packed(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, void* y, int64_t ldy, int64_t M,
                    int64_t N, int64_t K, const plm_tile* tile, void* workspace, size_t workspace_bytes, void* stream) {
  return plm::packed_rows(dtype, x, ldx, packed_w, y, ldy, M, N, K, tile, workspace, workspace_bytes, stream, 0);
}

int plm_gemm_packed_f32out(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, float* y, int64_t ldy,
                           int64_t M, int64_t N, int64_t K, const plm_tile* tile, void* workspace,
                           size_t workspace_bytes, void* stream) {
  return plm::packed_rows(dtype, x, ldx, packed_w, y, ldy, M, N, K, tile, workspace, workspace_bytes, stream, 1);
}

int plm_gemm_packed_resident_workgroups(int32_t dtype, int64_t M, const plm_tile* tile) {
  if (!plm::packed_tile_valid(tile) || M < 1 || M > plm::kPackedMaxM) return PLM_ERR_TILE;
  const int cus = plm::packed_cus();
  if (cus <= 0) return PLM_ERR_LAUNCH;
  plm::PackedArgs a{};
  a.M = static_cast<int>(M);
  a.count = 0;
  if (plm::packed_dispatch_dt(dtype, a, *tile, cus, nullptr, false) != hipSuccess) return PLM_ERR_TILE;
  return a.G;
}

int64_t plm_gemm_chain_packed_prepare(plm_chain_gemm* gemms, int32_t count, int64_t M, const plm_tile* tile) {
  if (gemms == nullptr || count < 1 || M < 1 || M > plm::kPackedMaxM) return PLM_ERR_ARGUMENT;
  if (!plm::packed_tile_valid(tile)) return PLM_ERR_TILE;
  return plm::packed_prepare(gemms, count, M, *tile);
}

int plm_gemm_chain_packed_sync_mode(const plm_chain_gemm* gemms, int32_t count, const plm_tile* tile) {
  if (gemms == nullptr || count < 1) return PLM_ERR_ARGUMENT;
  if (!plm::packed_tile_valid(tile)) return PLM_ERR_TILE;
  return plm::packed_chain_mode(gemms, count, *tile);
}

int plm_gemm_chain_packed(int32_t dtype, const plm_chain_gemm* host_gemms, const plm_chain_gemm* device_gemms,
                          int32_t count, int64_t M, const plm_tile* tile, void* workspace, size_t workspace_bytes,
                          void* stream) {
  if (host_gemms == nullptr || device_gemms == nullptr || count < 1) return PLM_ERR_ARGUMENT;
  if (!plm::packed_tile_valid(tile)) return PLM_ERR_TILE;
  if (M < 1 || M > plm::kPackedMaxM) return PLM_ERR_ARGUMENT;
  // The derived fields must be what plm_gemm_chain_packed_prepare computes for this chain.
  std::vector<plm_chain_gemm> check(host_gemms, host_gemms + count);
  const int64_t need = plm::packed_prepare(check.data(), count, M, *tile);
  if (need < 0) return static_cast<int>(need);
  bool sync = false, any_split = false, any_act = false;
  int64_t most_items = 0;
  std::vector<plm::PSpan> ys(count), xs(count), ws(count);
  for (int32_t i = 0; i < count; ++i) {
    const plm_chain_gemm& g = host_gemms[i];
    if (g.consumed != check[i].consumed || g.arrive_base != check[i].arrive_base ||
        g.done_base != check[i].done_base || g.partial_offset != check[i].partial_offset)
      return PLM_ERR_ARGUMENT;
    const int status = plm::packed_check_linear(dtype, g, M, tile);
    if (status != PLM_OK) return status;
    plm_tile ti = *tile;
    ti.split_k = g.split_k;
    most_items = std::max(most_items, plm::packed_tiles(g.N, ti) * g.split_k);
    any_split = any_split || g.split_k > 1;
    any_act = any_act || g.out_f32 == PLM_OUT_SILU_MUL;
    ys[i] = plm::pspan(g.y, M, g.ldy, plm::out_cols(g), g.out_f32 == PLM_OUT_F32 ? 4 : 2);
    xs[i] = plm::pspan(g.x, M, g.ldx, g.K, 2);
    ws[i] = plm::PSpan{reinterpret_cast<uintptr_t>(g.w),
                       reinterpret_cast<uintptr_t>(g.w) + static_cast<uintptr_t>(plm::packed_bytes(g.N, g.K))};
    if (g.dep >= 0) {
      sync = true;
      const plm_chain_gemm& p = host_gemms[g.dep];
      if (g.x != p.y || g.ldx != p.ldy || g.K > plm::out_cols(p) || p.out_f32 == PLM_OUT_F32) return PLM_ERR_ARGUMENT;
    }
  }
  // No linear writes what another linear writes, or reads before it is written.
  for (int32_t i = 0; i < count; ++i)
    for (int32_t j = 0; j < count; ++j) {
      if (i != j && ys[i].overlaps(ys[j])) return PLM_ERR_ARGUMENT;
      if (ys[i].overlaps(ws[j])) return PLM_ERR_ARGUMENT;
      if (ys[i].overlaps(xs[j]) && host_gemms[j].dep != i) return PLM_ERR_ARGUMENT;
    }
  plm::PackedArgs a{};
  a.chain = device_gemms;
  a.single = host_gemms[0];
  a.count = count;
  a.M = static_cast<int>(M);
  a.G = static_cast<int>(most_items);
  a.sync = sync ? plm::packed_chain_mode(host_gemms, count, *tile) : 0;
  const int64_t needed = (sync || any_split) ? need : 0;
  return plm::packed_launch_args(dtype, a, *tile, workspace, workspace_bytes, needed,
                                 static_cast<hipStream_t>(stream), any_act ? plm::kEpiAct : plm::kEpiPlain);
}

size_t plm_gemm_packed_lora_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t gated_from, int64_t rank,
                                            int32_t shards, const plm_tile* tile) {
  if (!plm::packed_tile_valid(tile) || M < 1 || N < 1 || K < 1 || rank < 1 || shards < 1) return 0;
  if (gated_from >= M) return static_cast<size_t>(plm::packed_workspace(M, N, *tile));
  return static_cast<size_t>(plm::lora_layout(M, N, K, shards * rank, *tile).bytes);
}

int plm_gemm_packed_lora(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, void* y, int64_t ldy, int64_t M,
                         int64_t N, int64_t K, int64_t gated_from, const void* packed_a, const void* lora_b, int64_t rank,
                         int32_t shards, const int64_t* shard_sizes, const plm_tile* tile, void* workspace,
                         size_t workspace_bytes, void* stream) {
  if (gated_from < 0 || rank < 8 || rank > 1024 || rank % 8 != 0 || shards < 1 || shards > 3 || shard_sizes == nullptr)
    return PLM_ERR_ARGUMENT;
  if (gated_from >= M)  // no gated row: the base linear alone (plm/gated_lora.py:47-48)
    return plm::packed_entry(dtype, x, ldx, packed_w, y, ldy, M, N, K, tile, workspace, workspace_bytes, stream, 0);
  if (packed_a == nullptr || lora_b == nullptr) return PLM_ERR_ARGUMENT;
  if (!plm::packed_tile_valid(tile)) return PLM_ERR_TILE;
  if (N < 1 || N > (int64_t(1) << 30) || K > (int64_t(1) << 30)) return PLM_ERR_ARGUMENT;
  const plm_tile& t = *tile;
  const int64_t width = shards * rank;  // h columns
  plm::PackedLora z{};
  int64_t end = 0;
  for (int i = 0; i < 3; ++i) z.shard_end[i] = static_cast<int>(N);
  for (int32_t i = 0; i < shards; ++i) {
    if (shard_sizes[i] < 1) return PLM_ERR_ARGUMENT;
    end += shard_sizes[i];
    if (i + 1 < shards) z.shard_end[i] = static_cast<int>(end);
  }
  if (end != N) return PLM_ERR_ARGUMENT;
  if ((reinterpret_cast<uintptr_t>(lora_b) & 15) != 0) return PLM_ERR_ALIGNMENT;
  if (N * rank * 2 >= (int64_t(1) << 31)) return PLM_ERR_ARGUMENT;  // B is read through a 32-bit buffer offset
  const plm::LoraLayout l = plm::lora_layout(M, N, K, width, t);
  if (workspace == nullptr || static_cast<int64_t>(workspace_bytes) < l.bytes ||
      (reinterpret_cast<uintptr_t>(workspace) & 15) != 0)
    return PLM_ERR_WORKSPACE;
  // The base linear: Y = X W^T for every row (the reference's base output, plm/gated_lora.py:52).
  plm_chain_gemm g{};
  g.x = x;
  g.w = packed_w;
  g.y = y;
  g.ldx = ldx;
  g.ldw = K;
  g.ldy = ldy;
  g.N = static_cast<int32_t>(N);
  g.K = static_cast<int32_t>(K);
  g.split_k = t.split_k;
  g.dep = -1;
  g.arrive_base = plm::kPackedArriveBase;
  int status = plm::packed_check_linear(dtype, g, M);
  if (status != PLM_OK) return status;
  // The h linear: h = X A^T in the model dtype (the reference's second GEMM, 54), every row; its
  // stores are written through to the device-coherent level for the base tiles to read.
  plm_chain_gemm gh = g;
  gh.w = packed_a;
  gh.y = static_cast<char*>(workspace) + l.h_offset;
  gh.ldy = width;
  gh.N = static_cast<int32_t>(width);
  gh.split_k = static_cast<int32_t>(l.h_split);
  gh.consumed = 1;
  const int64_t base_tiles = plm::packed_tiles(N, t);
  gh.arrive_base = static_cast<int32_t>(plm::kPackedArriveBase + base_tiles);
  gh.partial_offset = l.h_partial;
  status = plm::packed_check_linear(dtype, gh, M);
  if (status != PLM_OK) return status;
  if (base_tiles + l.h_tiles > plm::kPackedBarrierBase - plm::kPackedArriveBase) return PLM_ERR_ARGUMENT;
  z.pre = gh;
  z.b = static_cast<const uint16_t*>(lora_b);
  z.rank = static_cast<int>(rank);
  z.gated_from = static_cast<int>(gated_from);
  z.h_tiles = static_cast<int>(l.h_tiles);
  z.base_tiles = static_cast<int>(base_tiles);
  z.h_items = static_cast<int>(l.h_tiles * l.h_split);
  plm::PackedArgs a{};
  a.single = g;
  a.count = 2;
  a.M = static_cast<int>(M);
  a.G = static_cast<int>(z.h_items + base_tiles * t.split_k);
  a.sync = 0;
  a.lora = z;
  return plm::packed_launch_args(dtype, a, t, workspace, workspace_bytes, l.bytes, static_cast<hipStream_t>(stream),
                                 plm::kEpiLora);
}

int plm_gemm_packed_silu_mul(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, void* y, int64_t ldy,
                             int64_t M, int64_t N, int64_t K, const plm_tile* tile, void* workspace,
                             size_t workspace_bytes, void* stream) {
  if (!plm::packed_tile_valid(tile)) return PLM_ERR_TILE;
  const plm_tile& t = *tile;
  if (N < 32 || N > (int64_t(1) << 30) || K > (int64_t(1) << 30)) return PLM_ERR_ARGUMENT;
  plm_chain_gemm g{};
  g.x = x;
  g.w = packed_w;
  g.y = y;
  g.ldx = ldx;
  g.ldw = K;
  g.ldy = ldy;
  g.N = static_cast<int32_t>(N);
  g.K = static_cast<int32_t>(K);
  g.split_k = t.split_k;
  g.dep = -1;
  g.out_f32 = PLM_OUT_SILU_MUL;
  const int status = plm::packed_check_linear(dtype, g, M, &t);
  if (status != PLM_OK) return status;
  const int64_t tiles = plm::packed_tiles(N, t);
  if (t.split_k > 1 && tiles > plm::kPackedBarrierBase - plm::kPackedArriveBase) return PLM_ERR_ARGUMENT;
  g.arrive_base = plm::kPackedArriveBase;
  plm::PackedArgs a{};
  a.single = g;
  a.count = 1;
  a.M = static_cast<int>(M);
  a.G = static_cast<int>(tiles * t.split_k);
  return plm::packed_launch_args(dtype, a, t, workspace, workspace_bytes, plm::packed_workspace(M, N, t),
                                 static_cast<hipStream_t>(stream), plm::kEpiAct);
}

}  // extern "C"
