// C ABI of the streaming GEMM: one linear (plm_gemm) or a chain of linears (plm_gemm_chain),
// declared in include/plm_amd.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "plm_amd.h"
#include "stream_gemm.h"

namespace plm {
namespace {

constexpr int kSpinLimit = 1 << 20;  // polls (each one device round trip) before a wait gives up
constexpr int64_t kMaxM = 128;

bool tile_valid(const plm_tile* t) {
  return t != nullptr && (t->wave_frags == 1 || t->wave_frags == 2 || t->wave_frags == 4) &&
         t->k_waves == kStreamKW && t->unroll == kStreamU && t->split_k >= 1 && t->split_k <= 64;
}

hipError_t dispatch(int32_t dtype, StreamArgs& a, const plm_tile& t, int cus, hipStream_t s, bool dry) {
  if (dtype == PLM_BF16) return stream_dispatch_bf16(a, t.wave_frags, cus, s, dry);
  if (dtype == PLM_F16) return stream_dispatch_f16(a, t.wave_frags, cus, s, dry);
  return hipErrorInvalidConfiguration;
}

int device_cus() {
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

// Tiles of a linear: 64 * wave_frags weight rows each (16 * wave_frags per compute wavefront).
int64_t tiles_of(int64_t N, const plm_tile& t) { return (N + 64 * t.wave_frags - 1) / (64 * t.wave_frags); }

// Checks one linear's operands; returns PLM_OK or the status to report.
int check_linear(int32_t dtype, const plm_chain_gemm& g, int64_t M, const plm_tile& t) {
  if (g.x == nullptr || g.w == nullptr || g.y == nullptr) return PLM_ERR_ARGUMENT;
  if (dtype != PLM_BF16 && dtype != PLM_F16) return PLM_ERR_ARGUMENT;
  if (M < 1 || M > kMaxM || g.N < 1 || g.K < 8 || g.K % 8 != 0) return PLM_ERR_ARGUMENT;
  if (g.ldx < g.K || g.ldw < g.K || g.ldy < g.N) return PLM_ERR_ARGUMENT;
  if (g.split_k < 1 || g.split_k > 64 || (g.out_f32 != 0 && g.out_f32 != 1)) return PLM_ERR_ARGUMENT;
  // Buffer offsets are 31-bit: X and one wavefront's weight rows must each span less than 2 GiB.
  if (M * g.ldx * 2 >= (int64_t(1) << 31) || 16 * t.wave_frags * g.ldw * 2 >= (int64_t(1) << 31)) return PLM_ERR_ARGUMENT;
  if (g.ldx % 8 != 0 || g.ldw % 8 != 0 || !aligned16_ptr(g.x) || !aligned16_ptr(g.w)) return PLM_ERR_ALIGNMENT;
  return PLM_OK;
}

struct Span {
  uintptr_t lo, hi;
  bool overlaps(const Span& o) const { return lo < o.hi && o.lo < hi; }
};

Span span_of(const void* p, int64_t rows, int64_t ld, int64_t cols, int64_t elem) {
  const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
  return Span{lo, lo + static_cast<uintptr_t>(((rows - 1) * ld + cols) * elem)};
}

// Derived fields and workspace size of a chain (see plm_gemm_chain_prepare).
int64_t prepare(plm_chain_gemm* g, int32_t count, int64_t M, const plm_tile& t) {
  for (int32_t i = 0; i < count; ++i) g[i].consumed = 0;
  for (int32_t i = 0; i < count; ++i) {
    if (g[i].dep < -1 || g[i].dep >= i) return PLM_ERR_ARGUMENT;
    if (g[i].dep >= 0) g[g[i].dep].consumed = 1;
  }
  int64_t arrive = kArriveBase, done = kDoneBase, partial = 0;
  for (int32_t i = 0; i < count; ++i) {
    if (g[i].N < 1 || g[i].split_k < 1) return PLM_ERR_ARGUMENT;
    const int64_t tiles = tiles_of(g[i].N, t);
    g[i].arrive_base = 0;
    g[i].partial_offset = 0;
    g[i].done_base = 0;
    if (g[i].split_k > 1) {
      g[i].arrive_base = static_cast<int32_t>(arrive);
      g[i].partial_offset = partial;
      arrive += tiles;
      // [split][M][Np] fp32 planes, Np = N rounded up to 4; one buffer resource spans them.
      const int64_t floats = static_cast<int64_t>(g[i].split_k) * M * ((g[i].N + 3) / 4 * 4);
      if (floats * 4 >= (int64_t(1) << 31)) return PLM_ERR_ARGUMENT;
      partial += (floats + 63) / 64 * 64;
    }
    if (g[i].consumed) {
      g[i].done_base = static_cast<int32_t>(done);
      done += tiles;
    }
    if (arrive > kDoneBase || done > kStreamDoneEnd) return PLM_ERR_ARGUMENT;
  }
  return static_cast<int64_t>(kCounterBytes) + partial * static_cast<int64_t>(sizeof(float));
}

int launch(int32_t dtype, StreamArgs& a, const plm_tile& t, void* workspace, size_t workspace_bytes, size_t need,
           hipStream_t stream) {
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || !aligned16_ptr(workspace))) return PLM_ERR_WORKSPACE;
  const int cus = device_cus();
  if (cus <= 0) return PLM_ERR_LAUNCH;
  if (dispatch(dtype, a, t, cus, stream, true) != hipSuccess) return PLM_ERR_TILE;
  a.counters = static_cast<int*>(workspace);
  a.partial = workspace != nullptr ? reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes) : nullptr;
  a.spin_limit = kSpinLimit;
  return dispatch(dtype, a, t, cus, stream, false) == hipSuccess ? PLM_OK : PLM_ERR_LAUNCH;
}

int gemm_entry(int32_t dtype, const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy, int64_t M,
               int64_t N, int64_t K, const plm_tile* tile, void* workspace, size_t workspace_bytes, void* stream,
               int out_f32) {
  if (!tile_valid(tile)) return tile == nullptr ? PLM_ERR_ARGUMENT : PLM_ERR_TILE;
  if (N > (int64_t(1) << 30) || K > (int64_t(1) << 30) || N < 1 || K < 1) return PLM_ERR_ARGUMENT;
  plm_chain_gemm g{};
  g.x = x;
  g.w = w;
  g.y = y;
  g.ldx = ldx;
  g.ldw = ldw;
  g.ldy = ldy;
  g.N = static_cast<int32_t>(N);
  g.K = static_cast<int32_t>(K);
  g.split_k = tile->split_k;
  g.dep = -1;
  g.out_f32 = out_f32;
  const int status = check_linear(dtype, g, M, *tile);
  if (status != PLM_OK) return status;
  const int64_t need = prepare(&g, 1, M, *tile);
  if (need < 0) return static_cast<int>(need);
  StreamArgs a{};
  a.chain = nullptr;
  a.single = g;
  a.count = 1;
  a.M = static_cast<int>(M);
  a.G = static_cast<int>(tiles_of(N, *tile) * g.split_k);
  a.sync = 0;
  return launch(dtype, a, *tile, workspace, workspace_bytes, g.split_k > 1 ? static_cast<size_t>(need) : 0,
                static_cast<hipStream_t>(stream));
}

}  // namespace
}  // namespace plm

extern "C" {

size_t plm_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, const plm_tile* tile) {
  (void)K;
  if (tile == nullptr || tile->split_k <= 1 || M <= 0 || N <= 0) return 0;
  const int64_t floats = static_cast<int64_t>(tile->split_k) * M * ((N + 3) / 4 * 4);
  return plm::kCounterBytes + static_cast<size_t>((floats + 63) / 64 * 64) * sizeof(float);
}

int plm_gemm_tile_supported(int32_t dtype, int64_t M, int64_t K, const plm_tile* tile) {
  if (!plm::tile_valid(tile) || M < 1 || M > plm::kMaxM || K < 1 || K > (int64_t(1) << 30)) return 0;
  plm::StreamArgs a{};
  a.M = static_cast<int>(M);
  return plm::dispatch(dtype, a, *tile, 1, nullptr, true) == hipSuccess ? 1 : 0;
}

int plm_gemm(int32_t dtype, const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy, int64_t M,
             int64_t N, int64_t K, const plm_tile* tile, void* workspace, size_t workspace_bytes, void* stream) {
  return plm::gemm_entry(dtype, x, ldx, w, ldw, y, ldy, M, N, K, tile, workspace, workspace_bytes, stream, 0);
}

int plm_gemm_f32out(int32_t dtype, const void* x, int64_t ldx, const void* w, int64_t ldw, float* y, int64_t ldy,
                    int64_t M, int64_t N, int64_t K, const plm_tile* tile, void* workspace, size_t workspace_bytes,
                    void* stream) {
  return plm::gemm_entry(dtype, x, ldx, w, ldw, y, ldy, M, N, K, tile, workspace, workspace_bytes, stream, 1);
}

int64_t plm_gemm_chain_prepare(plm_chain_gemm* gemms, int32_t count, int64_t M, const plm_tile* tile) {
  if (gemms == nullptr || count < 1 || plm::table_bytes(count) > plm::kTableReserve || M < 1 || M > plm::kMaxM ||
      tile == nullptr)
    return PLM_ERR_ARGUMENT;
  plm_tile t = *tile;
  t.split_k = 1;
  if (!plm::tile_valid(&t)) return PLM_ERR_TILE;
  return plm::prepare(gemms, count, M, t);
}

int plm_gemm_chain(int32_t dtype, const plm_chain_gemm* host_gemms, const plm_chain_gemm* device_gemms, int32_t count,
                   int64_t M, const plm_tile* tile, void* workspace, size_t workspace_bytes, void* stream) {
  if (host_gemms == nullptr || device_gemms == nullptr || count < 1 || tile == nullptr) return PLM_ERR_ARGUMENT;
  plm_tile t = *tile;
  t.split_k = 1;
  if (!plm::tile_valid(&t)) return PLM_ERR_TILE;
  if (M < 1 || M > plm::kMaxM) return PLM_ERR_ARGUMENT;
  // The kernel keeps the chain's descriptors in LDS next to its staging area.
  if (plm::table_bytes(count) > plm::kTableReserve) return PLM_ERR_ARGUMENT;
  // The derived fields must be what prepare() computes for this chain.
  std::vector<plm_chain_gemm> check(host_gemms, host_gemms + count);
  const int64_t need = plm::prepare(check.data(), count, M, t);
  if (need < 0) return static_cast<int>(need);
  bool sync = false;
  int64_t most_items = 0;
  std::vector<plm::Span> ys(count), xs(count), ws(count);
  for (int32_t i = 0; i < count; ++i) {
    const plm_chain_gemm& g = host_gemms[i];
    if (g.consumed != check[i].consumed || g.arrive_base != check[i].arrive_base ||
        g.done_base != check[i].done_base || g.partial_offset != check[i].partial_offset)
      return PLM_ERR_ARGUMENT;
    const int status = plm::check_linear(dtype, g, M, t);
    if (status != PLM_OK) return status;
    most_items = std::max(most_items, plm::tiles_of(g.N, t) * g.split_k);
    ys[i] = plm::span_of(g.y, M, g.ldy, g.N, g.out_f32 ? 4 : 2);
    xs[i] = plm::span_of(g.x, M, g.ldx, g.K, 2);
    ws[i] = plm::span_of(g.w, g.N, g.ldw, g.K, 2);
    if (g.dep >= 0) {
      sync = true;
      const plm_chain_gemm& p = host_gemms[g.dep];
      if (g.x != p.y || g.ldx != p.ldy || g.K > p.N) return PLM_ERR_ARGUMENT;
    }
    if (g.consumed) {
      // Every 128-byte line of a consumed Y is written by one tile: tiles of 64 * wave_frags
      // columns of 16-bit values on 128-byte aligned rows.
      if (g.out_f32) return PLM_ERR_ARGUMENT;
      if ((reinterpret_cast<uintptr_t>(g.y) & 127) != 0 || g.ldy % 64 != 0) return PLM_ERR_ALIGNMENT;
    }
  }
  for (int32_t i = 0; i < count; ++i)
    for (int32_t j = 0; j < count; ++j) {
      if (i != j && ys[i].overlaps(ys[j])) return PLM_ERR_ARGUMENT;
      if (ys[i].overlaps(ws[j])) return PLM_ERR_ARGUMENT;
      if (ys[i].overlaps(xs[j]) && host_gemms[j].dep != i) return PLM_ERR_ARGUMENT;
    }
  plm::StreamArgs a{};
  a.chain = device_gemms;
  a.single = host_gemms[0];
  a.count = count;
  a.M = static_cast<int>(M);
  a.G = static_cast<int>(most_items);
  a.sync = sync ? 1 : 0;
  bool any_split = false;
  for (int32_t i = 0; i < count; ++i) any_split = any_split || host_gemms[i].split_k > 1;
  const size_t needed = (sync || any_split) ? static_cast<size_t>(need) : 0;
  return plm::launch(dtype, a, t, workspace, workspace_bytes, needed, static_cast<hipStream_t>(stream));
}

const char* plm_status_string(int32_t status) {
  switch (status) {
    case PLM_OK: return "ok";
    case PLM_ERR_ARGUMENT: return "invalid argument (size, stride, dtype, null pointer or chain layout)";
    case PLM_ERR_ALIGNMENT: return "pointer or leading dimension not aligned";
    case PLM_ERR_TILE: return "no compiled kernel for this tile configuration and M";
    case PLM_ERR_WORKSPACE: return "workspace missing or too small";
    case PLM_ERR_LAUNCH: return "HIP kernel launch failed";
  }
  return "unknown status";
}

}  // extern "C"
