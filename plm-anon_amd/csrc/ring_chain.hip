// The round's linears as one persistent launch with the weight stream on a wavefront of its own
// (gfx950, MI355X): plm_ring_chain / plm_ring_chain_prepare in include/plm_amd.h.
//
// A chained round is a sequence of skinny linears Y_i = X_i · W_i^T where X_i is the output of an
// earlier linear. Its weights never depend on the activations, so one workgroup per compute unit
// splits into two roles:
//   * a loader wavefront streams the workgroup's packed weight fragments (plm_pack_weight's 1 KiB
//     MFMA operands) from HBM into a ring of LDS slots by buffer-to-LDS DMA, about 16 KiB in
//     flight (one such wavefront per CU measured 5.9 TB/s over the device, and a load from another
//     wavefront of the CU still returns in ~0.7 us), in the order the compute wavefronts consume
//     them, across item and linear boundaries: while the compute wavefronts wait for the linear
//     they read, the next linear's weights are already on their way;
//   * four compute wavefronts each take a quarter of the current item's K steps, read the weights
//     from the ring, X straight from memory into MFMA operands (v_mfma_f32_16x16x32_{bf16,f16}),
//     sum their four partial tiles in LDS in a fixed order, and write Y.
// The loader never waits for another workgroup; the roles meet only in LDS counters (no workgroup
// barrier inside the chain, so neither role holds the other up).
//
// Hand-off between linears. A linear whose Y a later one reads also writes it to a mailbox in the
// workspace in the MFMA operand layout of the reader's X (fragment (k step s, row block t) of
// 64 lanes x 16 bytes at ((s * MT + t) * 64 + lane) * 16): the reader's X loads are then whole,
// contiguous KiB that land in registers as operands. Each tile raises a per-linear flag (the launch
// epoch + 1, so flags only grow and are never cleared) once its mailbox stores have completed; a
// compute wavefront waits only for the producer tiles covering its own K steps. The caller's Y is
// written as well (row-major). The first linear, and any linear whose X comes from outside the
// chain, reads its X row-major.
//
// K split across workgroups (split > 1): every item writes its tile's fp32 partial, and the last
// item of the tile to arrive (device-scope counter, reset by that item) sums the partials in split
// order 0..split-1 and writes Y. No float atomics: results are reproducible bit for bit, and a
// linear's output depends only on its own tile geometry (rows per tile, split), not on the chain it
// runs in.
//
// Sums: within an item, wavefront w accumulates its K steps in ascending order; the four partial
// tiles are combined as (p0 + p2) + (p1 + p3); the split partials in split order.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "plm_amd.h"
#include "tile.h"

namespace plm {
namespace ring {

constexpr int kComputeWaves = 4;
constexpr int kThreads = 64 * (kComputeWaves + 1);
constexpr int kMaxRows = 4;                  // 16-row fragments per tile
constexpr int kRingSlots = 120;              // 1 KiB fragments the ring holds
constexpr int kMaxWaveSteps = 16;            // K steps of one compute wavefront per item
constexpr int kXAhead = 4;                   // K steps of X loads a compute wavefront keeps in flight
constexpr int kMaxMT = 4;                    // row blocks of X (M <= 64)
constexpr int kDmaDepth = 16;                // loader DMAs in flight
constexpr int kFrag = 1024;
constexpr uint32_t kRingBytes = kRingSlots * kFrag;
constexpr uint32_t kRedBytes = 2 * kMaxRows * kMaxMT * kFrag;  // two wavefronts' partial tiles
constexpr uint32_t kCtlBytes = 256;
constexpr uint32_t kLdsBytes = kRingBytes + kRedBytes + kCtlBytes;
constexpr uint32_t kNoLoad = 0x80000000u;

// LDS pointers keep their address space explicitly: through a generic pointer the compiler emits
// flat accesses, which count as vector memory operations and turn every wait for an LDS value into
// a wait for all of the wavefront's loads in flight.
#define LDS __attribute__((address_space(3)))
typedef LDS char LdsChar;
typedef LDS f32x4 LdsF4;
typedef LDS int LdsInt;
typedef LDS void LdsVoid;
// Global pointers likewise (stores through a generic pointer would be flat stores, which count
// against the LDS counter too).
typedef __attribute__((address_space(1))) float GF32;
typedef __attribute__((address_space(1))) f32x4 GF4;
typedef __attribute__((address_space(1))) uint16_t GU16;
typedef __attribute__((address_space(1))) uint64_t GU64;

// Counter-area ints of this launch (apart from those of the other kernels).
constexpr int kEpochSlot = 48;  // int64 at 48-49: ring-chain launches completed on this workspace
constexpr int kExitSlot = 50;   // workgroups that have finished the current launch

// LDS control words (ints), zeroed at kernel start; all counters only grow during a launch. Ring
// positions count fragments over the whole launch: a batch (one K step of every compute wavefront)
// is 4 * tile_rows consecutive positions, wavefront w's rows at w * tile_rows + r, and position q
// lives in slot q % kRingSlots.
struct Ctl {
  int filled;      // ring positions landed in LDS (loader)
  int pad0[3];
  int done[4];     // ring positions compute wavefront w has finished with (a batch end)
  int l1;          // wavefronts 2, 3: partial tiles written (level 1)
  int l2;          // wavefronts 0, 1: level-2 halves written
  int red_free;    // wavefronts 0, 1: reduction area read (level 2 done)
  int parted;      // wavefronts 0, 1: split partial stored and complete
  int decided;     // wavefront 0: split arrival known
  int decision;    // 1 if this workgroup's item was the tile's last split
  int stored;      // wavefronts: Y / mailbox stores complete
  int bail;        // 1 once a wait of this workgroup gave up: every later wait ends at once
};

struct Args {
  const plm_ring_link* links;  // device table
  int count;
  int M;
  int G;
  int spin_limit;
  char* ws;
};

__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int64_t uni64(int64_t v) {
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v >> 32)));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}
template <typename T>
__device__ __forceinline__ T* uptr(T* p) {
  return reinterpret_cast<T*>(uni64(reinterpret_cast<int64_t>(p)));
}
template <typename T>
__device__ __forceinline__ T cload(const T* p) {
  return *((const __attribute__((address_space(4))) T*)p);
}

// Waits on this wavefront's outstanding memory operations that also keep the compiler from moving
// memory accesses across them (the hand-offs below depend on that order).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N <= 63, "vmcnt is six bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// One linear as the kernel reads it (wave-uniform).
struct Link {
  const char* x;        // row-major X (xmode 0) or the producer's mailbox (xmode 1)
  int64_t ldx;
  int xmode;
  uint32_t xbytes;
  const char* w;
  uint32_t wbytes;
  int K, Ks, nfr;       // K, its 32-wide steps, 16-row weight fragments
  char* y;
  int64_t ldy;
  int N, out_f32;
  int tr, split, tiles, items;
  char* mbox;           // this linear's output mailbox (consumed), else nullptr
  uint32_t* flags;      // its tile flags (consumed)
  const uint32_t* pflags;  // the producer's tile flags (xmode 1)
  int ptr;              // the producer's rows per tile (16-row fragments)
  int ptiles;
  float* part;          // split partials [tile][split][row][t] of 1 KiB
  int* arrive;          // split arrival counters, one per tile
};

__device__ __forceinline__ Link load_link(const Args& a, int i) {
  const plm_ring_link* p = a.links + i;
  Link L;
  L.x = uptr(static_cast<const char*>(cload(&p->x)));
  L.ldx = uni64(cload(&p->ldx));
  L.w = uptr(static_cast<const char*>(cload(&p->w)));
  L.y = uptr(static_cast<char*>(cload(&p->y)));
  L.ldy = uni64(cload(&p->ldy));
  L.N = uni(cload(&p->N));
  L.K = uni(cload(&p->K));
  L.Ks = (L.K + 31) >> 5;
  L.nfr = (L.N + 15) >> 4;
  L.wbytes = static_cast<uint32_t>(L.nfr) * static_cast<uint32_t>(L.Ks) * kFrag;
  L.out_f32 = uni(cload(&p->out_f32));
  L.tr = uni(cload(&p->tile_rows));
  L.split = uni(cload(&p->split_k));
  L.tiles = uni(cload(&p->tiles));
  L.items = L.tiles * L.split;
  const int dep = uni(cload(&p->dep));
  const int consumed = uni(cload(&p->consumed));
  L.mbox = consumed ? a.ws + uni64(cload(&p->mbox_offset)) : nullptr;
  L.flags = consumed ? reinterpret_cast<uint32_t*>(a.ws + uni64(cload(&p->flag_offset))) : nullptr;
  L.part = L.split > 1 ? reinterpret_cast<float*>(a.ws + uni64(cload(&p->partial_offset))) : nullptr;
  L.arrive = L.split > 1 ? reinterpret_cast<int*>(a.ws + uni64(cload(&p->arrive_offset))) : nullptr;
  const int MT = (a.M + 15) >> 4;
  if (dep >= 0) {
    const plm_ring_link* q = a.links + dep;
    L.xmode = 1;
    L.x = a.ws + uni64(cload(&q->mbox_offset));
    const int pN = uni(cload(&q->N));
    L.xbytes = static_cast<uint32_t>((pN + 31) >> 5) * static_cast<uint32_t>(MT) * kFrag;
    L.pflags = reinterpret_cast<const uint32_t*>(a.ws + uni64(cload(&q->flag_offset)));
    L.ptr = uni(cload(&q->tile_rows));
    L.ptiles = uni(cload(&q->tiles));
  } else {
    L.xmode = 0;
    L.xbytes = static_cast<uint32_t>(a.M * L.ldx * 2);
    L.pflags = nullptr;
    L.ptr = 1;
    L.ptiles = 0;
  }
  return L;
}

// Geometry of item `item` of L: its tile, split index and K steps [k0, k0 + n); wavefront w takes
// steps [k0 + n*w/4, k0 + n*(w+1)/4) and the item has ceil(n/4) ring batches.
struct Item {
  int tile, s, k0, n, nb;
};
__device__ __forceinline__ Item item_of(const Link& L, int item) {
  Item it;
  if (L.split == 1) {
    it.tile = item;
    it.s = 0;
    it.k0 = 0;
    it.n = L.Ks;
  } else {
    it.tile = static_cast<int>(static_cast<uint32_t>(item) / static_cast<uint32_t>(L.split));
    it.s = item - it.tile * L.split;
    it.k0 = static_cast<int>(static_cast<uint32_t>(it.s * L.Ks) / static_cast<uint32_t>(L.split));
    it.n = static_cast<int>(static_cast<uint32_t>((it.s + 1) * L.Ks) / static_cast<uint32_t>(L.split)) - it.k0;
  }
  it.nb = it.n - ((it.n * 3) >> 2);
  return it;
}
__device__ __forceinline__ void wave_range(const Item& it, int w, int& b, int& c) {
  b = it.k0 + ((it.n * w) >> 2);
  c = it.k0 + ((it.n * (w + 1)) >> 2) - b;
}

__device__ __forceinline__ bool failed(const Args& a) {
  return uni(collect(reinterpret_cast<const int*>(a.ws) + PLM_WORKSPACE_ERROR_INDEX)) != 0;
}
__device__ __forceinline__ void set_failed(const Args& a, int lane) {
  if (lane == 0) publish(reinterpret_cast<int*>(a.ws) + PLM_WORKSPACE_ERROR_INDEX, 1);
}

// Polls an LDS counter until it reaches `target` (every partner's own waits are bounded, so this
// ends; the bound is a second guard that flags the launch). Nothing after it is read early.
// Once any wait of the launch has given up, the loader's waits end within kErrorPolls polls (and
// every LDS wait of the workgroup at once, through Ctl::bail).
constexpr int kErrorPolls = 4096;
__device__ __forceinline__ void wait_lds(const Args& a, volatile LDS Ctl* ctl, const volatile LdsInt* p, int target,
                                         int lane) {
  // No global memory access in here: the compute wavefronts' load-count waits must not see one
  // (a timeout is reported through Ctl::bail and published at the end of the kernel).
  for (int i = 0; uni(*p) < target; ++i) {
    if (uni(ctl->bail)) break;
    if (i > (a.spin_limit << 6)) {
      if (lane == 0) ctl->bail = 1;
      break;
    }
  }
  asm volatile("" ::: "memory");
}
// Counts this wavefront in at an LDS counter once its earlier LDS accesses have completed.
__device__ __forceinline__ void add_lds(volatile LdsInt* p, int lane) {
  wait_lgkm0();
  if (lane == 0) __hip_atomic_fetch_add(const_cast<LdsInt*>(p), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------------------------------------
// Loader wavefront: one DMA per ring position (absent fragments get an out-of-range offset: they
// write zeros into their own slot and touch no memory), so after the vmcnt wait that follows a DMA
// every position but the last kDmaDepth has landed.

__device__ void loader(const Args& a, LdsChar* ring, volatile LDS Ctl* ctl, int lane) {
  int F = 0;     // next ring position
  int cmin = 0;  // positions every compute wavefront has finished with (cached)
  auto min_done = [&]() {
    const int d0 = ctl->done[0], d1 = ctl->done[1], d2 = ctl->done[2], d3 = ctl->done[3];
    return uni(min(min(d0, d1), min(d2, d3)));
  };
  for (int li = 0; li < a.count; ++li) {
    const Link L = load_link(a, li);
    const auto wr = make_rsrc(L.w, L.wbytes);
    const int bf = kComputeWaves * L.tr;  // positions per batch
    for (int item = blockIdx.x; item < L.items; item += a.G) {
      const Item it = item_of(L, item);
      int b[kComputeWaves], c[kComputeWaves];
#pragma unroll
      for (int w = 0; w < kComputeWaves; ++w) wave_range(it, w, b[w], c[w]);
      const int nbatch = (it.nb + kXAhead - 1) / kXAhead * kXAhead;  // padded to whole groups
      for (int j = 0; j < nbatch; ++j) {
        // The batch's slots are free once every position kRingSlots before its end is done with.
        const int need = F + bf - kRingSlots;
        if (need > cmin) {
          cmin = min_done();
          if (need > cmin) {
            // Ring full: everything issued has to be visible before waiting for a free slot.
            wait_vm<0>();
            if (lane == 0) ctl->filled = F;
            for (int i = 0;; ++i) {
              cmin = min_done();
              if (need <= cmin) break;
              if (i > (a.spin_limit << 4)) {
                set_failed(a, lane);
                break;
              }
              if (uni(ctl->bail) || (i % kErrorPolls == kErrorPolls - 1 && failed(a))) break;
              __builtin_amdgcn_s_sleep(1);
            }
          }
        }
#pragma unroll
        for (int w = 0; w < kComputeWaves; ++w) {
          for (int r = 0; r < L.tr; ++r) {
            const uint32_t off =
                j < c[w] ? (static_cast<uint32_t>(it.tile * L.tr + r) * static_cast<uint32_t>(L.Ks) +
                            static_cast<uint32_t>(b[w] + j)) * kFrag
                         : kNoLoad;
            const int slot = (F + w * L.tr + r) % kRingSlots;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (LdsVoid*)(ring + slot * kFrag), 16, lane * 16,
                                                     uni(static_cast<int>(off)), 0, 0);
            wait_vm<kDmaDepth>();
          }
        }
        F += bf;
        // Every DMA but the last kDmaDepth has landed (each position is exactly one DMA).
        if (lane == 0 && F > kDmaDepth) ctl->filled = F - kDmaDepth;
      }
    }
  }
  wait_vm<0>();
  if (lane == 0) ctl->filled = F;
}

// ---------------------------------------------------------------------------------------------
// Compute wavefronts.

// After the reduction, wavefront 0 holds rows 0-1 of the tile and wavefront 1 rows 2-3.
__device__ __forceinline__ bool keeps(int w, int r) { return w == 0 ? r < 2 : r >= 2; }

// Where a compute wavefront's X comes from for one item: K steps [b, b + c) through `r`, step j at
// scalar offset j * step over the per-lane row offsets.
struct XSource {
  __amdgpu_buffer_rsrc_t r;
  uint32_t step;
  int b, c, K, kq;
};

// This wavefront's K steps of one item, TR weight rows per step from the ring, multiplied into acc.
// Steps go in groups of kXAhead with no branch inside a group, so the compiler's load-count waits
// stay exact: the next group's X is requested while this group's MFMAs run. Steps past the
// wavefront's count c multiply the zeros the loader wrote into their slots by zero X
// (out-of-range loads), which adds nothing.
template <int DT, int MT, int TR>
__device__ __forceinline__ void item_mma(const Args& a, const LdsChar* ring, volatile LDS Ctl* ctl, int w, int lane,
                                         int ngroups, const XSource& xs, const uint32_t (&xo)[MT], int& F, int& seen,
                                         f32x4 (&acc)[kMaxRows][MT]) {
  u32x4 x[kXAhead][MT];
  auto load_x = [&](int j, int slot) __attribute__((always_inline)) {
    const bool live = j < xs.c;
    const int st = xs.b + j;
    const uint32_t so = live ? static_cast<uint32_t>(st) * xs.step : 0u;
    const bool kin = live && 32 * st + xs.kq < xs.K;
#pragma unroll
    for (int t = 0; t < MT; ++t)
      x[slot][t] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(xs.r, kin ? xo[t] : kNoLoad, uni(static_cast<int>(so)), 0));
  };
  auto group = [&](int g) __attribute__((always_inline)) {
    const int end = F + kXAhead * kComputeWaves * TR;  // the group's last ring position + 1
    if (seen < end) {
      wait_lds(a, ctl, &ctl->filled, end, lane);
      seen = uni(ctl->filled);
    }
#pragma unroll
    for (int jj = 0; jj < kXAhead; ++jj) {
      const int q0 = F + (jj * kComputeWaves + w) * TR;
      u32x4 wf[TR];
#pragma unroll
      for (int r = 0; r < TR; ++r)
        wf[r] = *reinterpret_cast<const LDS u32x4*>(ring + ((q0 + r) % kRingSlots) * kFrag + lane * 16);
#pragma unroll
      for (int r = 0; r < TR; ++r)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[r][t] = mfma_16x16x32<DT>(wf[r], x[jj][t], acc[r][t]);
      load_x(kXAhead * (g + 1) + jj, jj);
    }
    F = end;
    wait_lgkm0();
    if (lane == 0) ctl->done[w] = end;
  };
#pragma unroll
  for (int jj = 0; jj < kXAhead; ++jj) load_x(jj, jj);
  // The first group is peeled off the loop: the loop is then entered only with the loads in flight
  // in its own order, and the compiler's waits at its head stay exact (entered from the prologue,
  // it drained every load at the top of each group).
  if (ngroups > 0) group(0);
  for (int g = 1; g < ngroups; ++g) group(g);
}

// Waits until every producer tile covering K steps [b, b + c) of L has raised its flag.
__device__ __forceinline__ void wait_producer(const Args& a, const Link& L, int b, int c, uint32_t target, int lane) {
  if (c <= 0) return;
  const int cols = 16 * L.ptr;
  const int t0 = (32 * b) / cols;
  const int t1 = min((32 * (b + c) - 1) / cols, L.ptiles - 1);
  const auto fr = make_rsrc(L.pflags, static_cast<uint32_t>(L.ptiles) * 4u);
  if (failed(a)) return;
  for (int i = 0;; ++i) {
    bool ok = true;
    for (int t = t0; t <= t1; t += 64) {
      const int tt = t + lane;
      const uint32_t v = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(
          fr, tt <= t1 ? static_cast<uint32_t>(tt) * 4u : kNoLoad, 0, kCoherent));
      ok = ok && (tt > t1 || v >= target);
    }
    if (__all(ok)) return;
    if (i >= a.spin_limit) {
      set_failed(a, lane);
      return;
    }
    if ((i & 255) == 255 && failed(a)) return;
    __builtin_amdgcn_s_sleep(1);
  }
}

// Row-major Y: rows m of four columns n..n+3 (fewer at N's end), in the model dtype or fp32.
template <int DT>
__device__ __forceinline__ void store_y(const Link& L, int m, int n, f32x4 v) {
  const int left = L.N - n;
  if (L.out_f32 == PLM_OUT_F32) {
    GF32* y = (GF32*)(L.y) + static_cast<int64_t>(m) * L.ldy + n;
    if (left >= 4 && (reinterpret_cast<uintptr_t>(y) & 15) == 0) {
      *(GF4*)(y) = v;
    } else {
      for (int j = 0; j < 4 && j < left; ++j) y[j] = v[j];
    }
    return;
  }
  GU16* y = (GU16*)(L.y) + static_cast<int64_t>(m) * L.ldy + n;
  const uint16_t h[4] = {to_bits16<DT>(v[0]), to_bits16<DT>(v[1]), to_bits16<DT>(v[2]), to_bits16<DT>(v[3])};
  if (left >= 4 && (reinterpret_cast<uintptr_t>(y) & 7) == 0) {
    const uint64_t bits = (static_cast<uint64_t>(h[0]) | (static_cast<uint64_t>(h[1]) << 16)) |
                          ((static_cast<uint64_t>(h[2]) | (static_cast<uint64_t>(h[3]) << 16)) << 32);
    *(GU64*)(y) = bits;
  } else {
    for (int j = 0; j < 4 && j < left; ++j) y[j] = h[j];
  }
}

// Final values of fragment (row r, block t) of `tile`: the caller's Y and, for a linear a later one
// reads, the mailbox (written through to the device-coherent level). Lane l holds Y[16t + l%16]
// [n0 + 16r + 4(l/16) + 0..3]; in the reader's operand layout those four values are elements
// e0..e0+3 of lane (l%16) + 16*g of the fragment of K step s, with g and e0 from the column.
template <int DT, int MT>
__device__ __forceinline__ void store_final(const Args& a, const Link& L, int tile, int r, int t, int lane, f32x4 v) {
  const int m = 16 * t + (lane & 15);
  const int n = (tile * L.tr + r) * 16 + 4 * (lane >> 4);
  if (m >= a.M || n >= L.N) return;
  store_y<DT>(L, m, n, v);
  if (L.mbox != nullptr) {
    const int s = n >> 5, kk = n & 31;
    const int lp = (lane & 15) + 16 * (kk >> 3);
    const uint64_t bits =
        (static_cast<uint64_t>(to_bits16<DT>(v[0])) | (static_cast<uint64_t>(to_bits16<DT>(v[1])) << 16)) |
        ((static_cast<uint64_t>(to_bits16<DT>(v[2])) | (static_cast<uint64_t>(to_bits16<DT>(v[3])) << 16)) << 32);
    char* p = L.mbox + (static_cast<int64_t>(s) * MT + t) * kFrag + lp * 16 + (kk & 7) * 2;
    publish(reinterpret_cast<uint64_t*>(p), bits);
  }
}

template <int DT, int MT>
__device__ void compute(const Args& a, LdsChar* ring, LdsF4* red, volatile LDS Ctl* ctl, int w, int lane,
                        uint32_t flag_value) {
  int F = 0;             // ring position of the current batch
  int seen = 0;          // the loader's filled count as last read
  int n_items = 0;       // items of this workgroup so far
  int n_split = 0;       // of them with split > 1
  int stored_target = 0; // expected Ctl::stored
  const int kq = 8 * (lane >> 4);
  for (int li = 0; li < a.count; ++li) {
    const Link L = load_link(a, li);
    const auto xr = make_rsrc(L.x, L.xbytes);
    // Per-lane X offsets of row block t at step 0: mailbox fragments, or row-major rows.
    uint32_t xo[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = 16 * t + (lane & 15);
      if (m >= a.M)
        xo[t] = kNoLoad;
      else
        xo[t] = L.xmode ? static_cast<uint32_t>((t * 64 + lane) * 16)
                        : static_cast<uint32_t>(m * L.ldx * 2 + kq * 2);
    }
    const uint32_t xstep = L.xmode ? static_cast<uint32_t>(MT * kFrag) : 64u;
    for (int item = blockIdx.x; item < L.items; item += a.G, ++n_items) {
      const Item it = item_of(L, item);
      int b, c;
      wave_range(it, w, b, c);
      if (L.xmode) wait_producer(a, L, b, c, flag_value, lane);
      f32x4 acc[kMaxRows][MT];
#pragma unroll
      for (int r = 0; r < kMaxRows; ++r)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[r][t] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int ngroups = (it.nb + kXAhead - 1) / kXAhead;
      const XSource xs{xr, xstep, b, c, L.K, kq};
      switch (L.tr) {
        case 1: item_mma<DT, MT, 1>(a, ring, ctl, w, lane, ngroups, xs, xo, F, seen, acc); break;
        case 2: item_mma<DT, MT, 2>(a, ring, ctl, w, lane, ngroups, xs, xo, F, seen, acc); break;
        case 3: item_mma<DT, MT, 3>(a, ring, ctl, w, lane, ngroups, xs, xo, F, seen, acc); break;
        default: item_mma<DT, MT, 4>(a, ring, ctl, w, lane, ngroups, xs, xo, F, seen, acc); break;
      }

      // Sum of the four partial tiles: wavefronts 2 and 3 hand theirs to 0 and 1, which then swap
      // halves: wavefront 0 ends with rows 0-1 and 1 with rows 2-3, each (p0 + p2) + (p1 + p3).
      LdsF4* red0 = red;                               // [row][t][lane]
      LdsF4* red1 = red + kMaxRows * kMaxMT * 64;
      if (w >= 2) {
        if (n_items > 0) wait_lds(a, ctl, &ctl->red_free, 2 * n_items, lane);
        LdsF4* dst = w == 2 ? red0 : red1;
#pragma unroll
        for (int r = 0; r < kMaxRows; ++r)
          if (r < L.tr)
#pragma unroll
            for (int t = 0; t < MT; ++t) dst[(r * kMaxMT + t) * 64 + lane] = acc[r][t];
        add_lds(&ctl->l1, lane);
      } else {
        wait_lds(a, ctl, &ctl->l1, 2 * (n_items + 1), lane);
        const LdsF4* src = w == 0 ? red0 : red1;
#pragma unroll
        for (int r = 0; r < kMaxRows; ++r)
          if (r < L.tr)
#pragma unroll
            for (int t = 0; t < MT; ++t) acc[r][t] += src[(r * kMaxMT + t) * 64 + lane];
        // Level 2: wavefront 0 passes rows 2-3 (into the area it just read), wavefront 1 rows 0-1.
        LdsF4* mine = w == 0 ? red0 : red1;
#pragma unroll
        for (int r = 0; r < kMaxRows; ++r)
          if (!keeps(w, r) && r < L.tr)
#pragma unroll
            for (int t = 0; t < MT; ++t) mine[(r * kMaxMT + t) * 64 + lane] = acc[r][t];
        add_lds(&ctl->l2, lane);
        wait_lds(a, ctl, &ctl->l2, 2 * (n_items + 1), lane);
        const LdsF4* other = w == 0 ? red1 : red0;
#pragma unroll
        for (int r = 0; r < kMaxRows; ++r)
          if (keeps(w, r) && r < L.tr)
#pragma unroll
            for (int t = 0; t < MT; ++t) acc[r][t] += other[(r * kMaxMT + t) * 64 + lane];
        add_lds(&ctl->red_free, lane);
      }

      int last = 1;  // whether this workgroup writes the tile's Y
      if (L.split == 1) {
        if (w < 2) {
#pragma unroll
          for (int r = 0; r < kMaxRows; ++r)
            if (keeps(w, r) && r < L.tr)
#pragma unroll
              for (int t = 0; t < MT; ++t) store_final<DT, MT>(a, L, it.tile, r, t, lane, acc[r][t]);
          wait_vm<0>();
          add_lds(&ctl->stored, lane);
        }
        stored_target += 2;
      } else {
        // This item's partial (rows of wavefront 0 and 1), then the tile's arrival count.
        const int Q = L.tr * MT;
        float* pt = L.part + (static_cast<int64_t>(it.tile) * L.split) * Q * 256;
        const auto prs = make_rsrc(pt, static_cast<uint32_t>(L.split * Q) * kFrag);
        if (w < 2) {
#pragma unroll
          for (int r = 0; r < kMaxRows; ++r)
            if (keeps(w, r) && r < L.tr)
#pragma unroll
              for (int t = 0; t < MT; ++t)
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(u32x4, acc[r][t]), prs,
                    static_cast<uint32_t>(((it.s * L.tr + r) * MT + t) * kFrag + lane * 16), 0, kCoherent);
          wait_vm<0>();
          add_lds(&ctl->parted, lane);
        }
        ++n_split;
        if (w == 0) {
          wait_lds(a, ctl, &ctl->parted, 2 * n_split, lane);
          if (lane == 0) {
            const int before = __hip_atomic_fetch_add(L.arrive + it.tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int is_last = before == L.split - 1;
            if (is_last) __hip_atomic_store(L.arrive + it.tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ctl->decision = is_last;
          }
          add_lds(&ctl->decided, lane);
        }
        wait_lds(a, ctl, &ctl->decided, n_split, lane);
        last = uni(ctl->decision);
        if (last) {
          // Wavefront w sums row w over the splits in order.
          if (w < L.tr) {
            u32x4 pv[MT][4];
            f32x4 sum[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t) sum[t] = f32x4{0.f, 0.f, 0.f, 0.f};
            for (int s0 = 0; s0 < L.split; s0 += 4) {
#pragma unroll
              for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                  pv[t][q] = __builtin_bit_cast(
                      u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                 prs,
                                 s0 + q < L.split ? static_cast<uint32_t>((((s0 + q) * L.tr + w) * MT + t) * kFrag + lane * 16)
                                                  : kNoLoad,
                                 0, kCoherent));
#pragma unroll
              for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                  if (s0 + q < L.split) sum[t] += __builtin_bit_cast(f32x4, pv[t][q]);
            }
#pragma unroll
            for (int t = 0; t < MT; ++t) store_final<DT, MT>(a, L, it.tile, w, t, lane, sum[t]);
            wait_vm<0>();
          }
          add_lds(&ctl->stored, lane);
          stored_target += 4;
        }
      }
      // The tile's Y is complete once every storing wavefront's stores are: raise its flag.
      if (L.flags != nullptr && w == 0 && last) {
        wait_lds(a, ctl, &ctl->stored, stored_target, lane);
        if (lane == 0) publish(L.flags + it.tile, flag_value);
      }
    }
  }
}

template <int DT, int MT>
__global__ __launch_bounds__(kThreads, 1) void ring_chain_kernel(Args a) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  LdsChar* ring = (LdsChar*)lds;
  LdsF4* red = (LdsF4*)(ring + kRingBytes);
  volatile LDS Ctl* ctl = (volatile LDS Ctl*)(ring + kRingBytes + kRedBytes);
  const int lane = threadIdx.x & 63;
  const int wave = uni(threadIdx.x >> 6);
  if (threadIdx.x < kCtlBytes / 4) ((volatile LdsInt*)ctl)[threadIdx.x] = 0;
  const int64_t epoch = uni64(collect(reinterpret_cast<const int64_t*>(a.ws) + kEpochSlot / 2));
  __syncthreads();
  if (wave == kComputeWaves)
    loader(a, ring, ctl, lane);
  else
    compute<DT, MT>(a, ring, red, ctl, wave, lane, static_cast<uint32_t>(epoch + 1));
  wait_vm<0>();
  __syncthreads();
  if (threadIdx.x == 0 && ctl->bail) publish(reinterpret_cast<int*>(a.ws) + PLM_WORKSPACE_ERROR_INDEX, 1);
  // The last workgroup out advances the epoch (every workgroup read it before its first wait, and
  // counts itself out only here, so none of this launch sees the new value).
  if (threadIdx.x == 0) {
    int* exitc = reinterpret_cast<int*>(a.ws) + kExitSlot;
    if (__hip_atomic_fetch_add(exitc, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.G - 1) {
      __hip_atomic_store(exitc, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      int64_t* ep = reinterpret_cast<int64_t*>(a.ws) + kEpochSlot / 2;
      publish(ep, collect(ep) + 1);
    }
  }
}

}  // namespace ring
}  // namespace plm

// ---------------------------------------------------------------------------------------------
// Host side.

namespace plm {
namespace ring {
namespace {

int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return cus;
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
int64_t align256(int64_t v) { return (v + 255) / 256 * 256; }

// Rows per tile and K split of a linear: the pair with the least estimated time (us) for the
// busiest workgroup: its weights at its share of HBM (~23 KiB/us; streamed ahead, so a floor
// rather than a sum), or its X at the compute unit's load rate (~100 KiB/us, after the producer)
// plus a fixed cost per item, whichever is longer; a K split adds about three dependent memory
// round trips (partial written through, arrival count, the last item's reads).
void choose(int64_t N, int64_t K, int64_t MT, int64_t G, int32_t& tr_out, int32_t& split_out) {
  const int64_t Ks = ceil_div(K, 32), nfr = ceil_div(N, 16);
  double best = 1e30;
  for (int tr = kMaxRows; tr >= 1; --tr) {
    const int64_t tiles = ceil_div(nfr, tr);
    for (int64_t s = std::max<int64_t>(1, ceil_div(Ks, kComputeWaves * kMaxWaveSteps)); s <= std::min<int64_t>(Ks, 64);
         ++s) {
      const int64_t steps = ceil_div(Ks, s);
      if (steps > kComputeWaves * kMaxWaveSteps) continue;
      const int64_t per_wg = ceil_div(tiles * s, G);
      const double w_kib = static_cast<double>(per_wg * steps * tr), x_kib = static_cast<double>(per_wg * steps * MT);
      double cost = std::max(w_kib / 23.0, x_kib / 100.0 + 0.4 * per_wg);
      if (s > 1) cost += 3.0 + 0.1 * s;
      if (cost < best - 1e-9) {
        best = cost;
        tr_out = tr;
        split_out = static_cast<int32_t>(s);
      }
    }
  }
}

int64_t prepare(plm_ring_link* g, int32_t count, int64_t M, int64_t G) {
  if (g == nullptr || count < 1 || M < 1 || M > 16 * kMaxMT || G < 1) return PLM_ERR_ARGUMENT;
  const int64_t MT = ceil_div(M, 16);
  for (int32_t i = 0; i < count; ++i) g[i].consumed = 0;
  for (int32_t i = 0; i < count; ++i) {
    plm_ring_link& L = g[i];
    if (L.x == nullptr || L.w == nullptr || L.y == nullptr) return PLM_ERR_ARGUMENT;
    if (L.N < 1 || L.K < 8 || L.K % 8 != 0 || L.K > (1 << 24) || L.ldy < L.N) return PLM_ERR_ARGUMENT;
    if (L.out_f32 != PLM_OUT_MODEL && L.out_f32 != PLM_OUT_F32) return PLM_ERR_ARGUMENT;
    if (L.dep < -1 || L.dep >= i) return PLM_ERR_ARGUMENT;
    if (L.dep >= 0) {
      const plm_ring_link& P = g[L.dep];
      // X is the leading K columns of the producer's Y.
      if (L.x != P.y || L.ldx != P.ldy || L.K > P.N || P.out_f32 != PLM_OUT_MODEL || P.N % 8 != 0)
        return PLM_ERR_ARGUMENT;
      g[L.dep].consumed = 1;
    } else {
      if (L.ldx < L.K || L.ldx % 8 != 0 || (reinterpret_cast<uintptr_t>(L.x) & 15) != 0) return PLM_ERR_ALIGNMENT;
      if (M * L.ldx * 2 >= (int64_t(1) << 31)) return PLM_ERR_ARGUMENT;
    }
    if ((reinterpret_cast<uintptr_t>(L.w) & 15) != 0) return PLM_ERR_ALIGNMENT;
    if (ceil_div(L.N, 16) * ceil_div(L.K, 32) * kFrag >= (int64_t(1) << 31)) return PLM_ERR_ARGUMENT;
    if (ceil_div(L.N, 32) * MT * kFrag >= (int64_t(1) << 31)) return PLM_ERR_ARGUMENT;  // its mailbox
    if (L.tile_rows == 0 || L.split_k == 0) {
      int32_t tr = 1, s = 1;
      choose(L.N, L.K, MT, G, tr, s);
      if (L.tile_rows == 0) L.tile_rows = tr;
      if (L.split_k == 0) L.split_k = s;
    }
    if (L.tile_rows < 1 || L.tile_rows > kMaxRows || L.split_k < 1 || L.split_k > 64) return PLM_ERR_TILE;
    const int64_t Ks = ceil_div(L.K, 32);
    if (L.split_k > Ks || ceil_div(Ks, L.split_k) > kComputeWaves * kMaxWaveSteps) return PLM_ERR_TILE;
    L.tiles = static_cast<int32_t>(ceil_div(ceil_div(L.N, 16), L.tile_rows));
    if (static_cast<int64_t>(L.tiles) * L.split_k >= (int64_t(1) << 30)) return PLM_ERR_ARGUMENT;
  }
  // Workspace: counter area, tile flags, arrival counters (both must start at zero and stay
  // consistent across launches), split partials, mailboxes.
  int64_t off = PLM_WORKSPACE_COUNTER_BYTES;
  for (int32_t i = 0; i < count; ++i) {
    g[i].flag_offset = g[i].consumed ? off : 0;
    if (g[i].consumed) off = align256(off + 4 * int64_t(g[i].tiles));
  }
  for (int32_t i = 0; i < count; ++i) {
    g[i].arrive_offset = g[i].split_k > 1 ? off : 0;
    if (g[i].split_k > 1) off = align256(off + 4 * int64_t(g[i].tiles));
  }
  for (int32_t i = 0; i < count; ++i) {
    g[i].partial_offset = g[i].split_k > 1 ? off : 0;
    if (g[i].split_k > 1) off = align256(off + int64_t(g[i].tiles) * g[i].split_k * g[i].tile_rows * MT * kFrag);
  }
  for (int32_t i = 0; i < count; ++i) {
    g[i].mbox_offset = g[i].consumed ? off : 0;
    if (g[i].consumed) off = align256(off + ceil_div(g[i].N, 32) * MT * kFrag);
  }
  return off;
}

template <int DT, int MT>
hipError_t launch(Args& a, hipStream_t s) {
  auto kern = ring_chain_kernel<DT, MT>;
  static bool attr = false;
  if (!attr) {
    const hipError_t e =
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess) return e;
    attr = true;
  }
  hipLaunchKernelGGL(kern, dim3(a.G), dim3(kThreads), kLdsBytes, s, a);
  return hipGetLastError();
}

template <int DT>
hipError_t launch_mt(Args& a, hipStream_t s) {
  switch ((a.M + 15) / 16) {
    case 1: return launch<DT, 1>(a, s);
    case 2: return launch<DT, 2>(a, s);
    case 3: return launch<DT, 3>(a, s);
    case 4: return launch<DT, 4>(a, s);
  }
  return hipErrorInvalidConfiguration;
}

}  // namespace
}  // namespace ring
}  // namespace plm

extern "C" {

int64_t plm_ring_chain_prepare(plm_ring_link* links, int32_t count, int64_t M, int32_t workgroups) {
  const int64_t G = workgroups > 0 ? workgroups : plm::ring::device_cus();
  if (G < 1) return PLM_ERR_LAUNCH;
  return plm::ring::prepare(links, count, M, G);
}

int plm_ring_chain_workgroups(void) {
  const int cus = plm::ring::device_cus();
  return cus > 0 ? cus : PLM_ERR_LAUNCH;
}

int plm_ring_chain(int32_t dtype, const plm_ring_link* host_links, const plm_ring_link* device_links, int32_t count,
                   int64_t M, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace plm::ring;
  if (host_links == nullptr || device_links == nullptr || count < 1 || M < 1 || M > 16 * kMaxMT)
    return PLM_ERR_ARGUMENT;
  if (dtype != PLM_BF16 && dtype != PLM_F16) return PLM_ERR_ARGUMENT;
  const int G = device_cus();
  if (G < 1) return PLM_ERR_LAUNCH;
  // The host table must be prepared for this grid: re-derive and compare the layout.
  int64_t need = PLM_WORKSPACE_COUNTER_BYTES;
  const int64_t MT = ceil_div(M, 16);
  for (int32_t i = 0; i < count; ++i) {
    const plm_ring_link& L = host_links[i];
    if (L.tile_rows < 1 || L.tile_rows > kMaxRows || L.split_k < 1 || L.tiles != ceil_div(ceil_div(L.N, 16), L.tile_rows))
      return PLM_ERR_ARGUMENT;
    if (L.consumed) need = std::max(need, L.mbox_offset + ceil_div(L.N, 32) * MT * kFrag);
    if (L.split_k > 1)
      need = std::max(need, L.partial_offset + int64_t(L.tiles) * L.split_k * L.tile_rows * MT * kFrag);
  }
  if (workspace == nullptr || static_cast<int64_t>(workspace_bytes) < need ||
      (reinterpret_cast<uintptr_t>(workspace) & 255) != 0)
    return PLM_ERR_WORKSPACE;
  Args a{};
  a.links = device_links;
  a.count = count;
  a.M = static_cast<int>(M);
  a.G = G;
  a.spin_limit = 1 << 20;
  a.ws = static_cast<char*>(workspace);
  const hipError_t e = dtype == PLM_BF16 ? launch_mt<plm::DT_BF16>(a, static_cast<hipStream_t>(stream))
                                         : launch_mt<plm::DT_F16>(a, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? PLM_OK : PLM_ERR_LAUNCH;
}

}  // extern "C"
