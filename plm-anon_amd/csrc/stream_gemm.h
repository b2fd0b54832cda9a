// Streaming skinny GEMM for the PLM round's dense linears on gfx950 (MI355X).
//
// Y[M,N] = X[M,K] · W[N,K]^T with fp32 accumulation, for a single linear or for a chain of linears
// in one launch, where a linear may read an earlier one's output (the round's linears back to
// back). M is the round width (k verify rows + k^2 proposal tokens, 56 at k=7), so the weights are
// almost all of the bytes and the kernel is an HBM stream of W.
//
// Work: item = one 16*NF-row tile of W x one of `split` K ranges. Each workgroup is persistent and
// takes items blockIdx.x, blockIdx.x + G, ... of every linear in turn.
//
// Workgroup = KW compute wavefronts + 1 epilogue wavefront.
//   * Compute wavefronts each own a contiguous K slice of the item. They stream their slice of
//     the weight tile from HBM in chunks of U 32-wide K steps, 16-byte loads straight into MFMA
//     operands (v_mfma_f32_16x16x32_{bf16,f16}), with the next chunk's weight loads always in
//     flight, across item and linear boundaries. X comes from L2 one chunk at a time. At the end
//     of an item they spill their fp32 partial tiles to LDS (double-buffered) and meet the
//     epilogue wavefront at one s_barrier.
//   * The epilogue wavefront sums the KW partials in wave order, writes Y (or, with split > 1, an
//     fp32 partial that the last workgroup of the tile to arrive sums in split order), marks
//     tiles finished, and waits for the tiles an item's X depends on. Only it stores to memory
//     or waits on other workgroups, so the compute wavefronts never wait on a store (on gfx9
//     vmcnt covers loads and stores in issue order: waiting on a store would also drain the
//     weight prefetch).
//
// Chains: a linear whose X is an earlier linear's Y waits, per item, only for the producer tiles
// covering its K range (tile-done flags), so consecutive linears overlap and the weight stream
// does not stop at linear boundaries. Producer Y and all cross-workgroup data go through
// device-coherent stores/loads; a consumer reads X through L2, which is safe because every
// 128-byte line of a consumed Y is written by one workgroup and read by nobody before its
// done flag is set (the host validates the layout that guarantees it).
//
// Results are bitwise reproducible: fixed K partition, K steps in ascending order inside a
// wavefront, wavefront partials summed in wave order, split partials in split order.
#pragma once

#include <hip/hip_runtime.h>

#include "plm_amd.h"
#include "tile.h"

namespace plm {

// Counter-area layout (ints), shared by every launch on one workspace.
constexpr int kEpochSlot = 0;     // chained launches completed on this workspace (tile-done epoch)
constexpr int kExitSlot = 1;      // workgroups finished in the current chained launch
constexpr int kErrorSlot = 2;     // 1 once a bounded wait gave up (results are then invalid)
constexpr int kArriveBase = 64;   // split-K arrival counters, one per (linear, tile)
constexpr int kDoneBase = 32768;  // tile-done flags of linears read later in the chain
constexpr int kArriveCapacity = kDoneBase - kArriveBase;
constexpr int kDoneCapacity = static_cast<int>(kMaxCounters) - kDoneBase;
constexpr int kStreamKW = 4;      // compute wavefronts per workgroup
constexpr size_t kMaxLdsBytes = 160 * 1024 - 256;  // dynamic LDS: 160 KiB per CU on gfx950, less static

struct StreamArgs {
  const plm_chain_gemm* chain;  // device array of `count` linears, or nullptr: use `single`
  plm_chain_gemm single;
  int count;
  int M;
  int G;           // workgroups in the grid
  int sync;        // some linear reads an earlier one's output
  int spin_limit;  // polls before a wait gives up
  int* counters;
  float* partial;
};

// Dynamic LDS: the launch's linear descriptors (copied from the kernel arguments or the device
// table at kernel start, 16-byte aligned), then the spill buffers.
extern __shared__ __attribute__((aligned(16))) float stream_lds[];

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int64_t uniform(int64_t v) {
  const int lo = __builtin_amdgcn_readfirstlane(static_cast<int>(v));
  const int hi = __builtin_amdgcn_readfirstlane(static_cast<int>(v >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo));
}
template <typename T>
__device__ __forceinline__ T* uniform(T* p) {
  return reinterpret_cast<T*>(uniform(reinterpret_cast<int64_t>(p)));
}

// Descriptor of linear gi, in scalar registers: every field is wave-uniform, and buffer
// resources built from it must not be in vector registers (that would cost a waterfall loop
// around every load).
__device__ __forceinline__ plm_chain_gemm gemm_at(int gi) {
  plm_chain_gemm g = reinterpret_cast<const plm_chain_gemm*>(stream_lds)[gi];
  g.x = uniform(g.x);
  g.w = uniform(g.w);
  g.y = uniform(g.y);
  g.ldx = uniform(g.ldx);
  g.ldw = uniform(g.ldw);
  g.ldy = uniform(g.ldy);
  g.N = uniform(g.N);
  g.K = uniform(g.K);
  g.split_k = uniform(g.split_k);
  g.dep = uniform(g.dep);
  g.out_f32 = uniform(g.out_f32);
  g.consumed = uniform(g.consumed);
  g.arrive_base = uniform(g.arrive_base);
  g.done_base = uniform(g.done_base);
  g.partial_offset = uniform(g.partial_offset);
  return g;
}

// The item hand-off flag between the epilogue and the compute wavefronts, typed as LDS so that
// polling it is a ds_read (lgkmcnt) and never a flat load, whose wait would also drain the
// compute wavefronts' outstanding weight prefetch (vmcnt).
typedef __attribute__((address_space(3))) volatile int LdsFlag;

constexpr size_t table_bytes(int count) { return (static_cast<size_t>(count) * sizeof(plm_chain_gemm) + 15) / 16 * 16; }

// K-step range [lo, hi) of split `s` out of `split` (ceil(K/32) steps in all).
__device__ __forceinline__ void split_range(int K, int s, int split, int& lo, int& hi) {
  const int steps = (K + 31) >> 5;
  lo = static_cast<int>(static_cast<int64_t>(s) * steps / split);
  hi = static_cast<int>(static_cast<int64_t>(s + 1) * steps / split);
}

// Where a compute wavefront is in its stream of chunks.
template <int NF>
struct Cursor {
  int gi, item, c, C;  // linear, item, chunk within the item, chunks per item
  int items, split, dep;
  int n0, tn;          // weight rows [n0, n0 + tn) of the item's tile
  int st, ns;          // this wavefront's K steps [st, st + ns)
  int N, K;
  int64_t ldw, ldx;
  const uint16_t* w;
  const uint16_t* x;
};

// Tile, K slice and chunk count of item q.item for compute wavefront `wave`. Every wavefront of
// the workgroup gets the same chunk count (at least one), so they all reach the item's end
// together; a wavefront whose slice is shorter loads nothing in its surplus chunks.
template <int NF, int U>
__device__ __forceinline__ void locate(Cursor<NF>& q, int wave) {
  constexpr int TN = 16 * NF;
  const int tile = q.item / q.split;
  const int s = q.item - tile * q.split;
  q.n0 = tile * TN;
  q.tn = min(TN, q.N - q.n0);
  int lo, hi;
  split_range(q.K, s, q.split, lo, hi);
  const int n = hi - lo;
  const int per = (n + kStreamKW - 1) / kStreamKW;
  q.C = per > 0 ? (per + U - 1) / U : 1;
  q.c = 0;
  q.st = lo + static_cast<int>(static_cast<int64_t>(wave) * n / kStreamKW);
  q.ns = lo + static_cast<int>(static_cast<int64_t>(wave + 1) * n / kStreamKW) - q.st;
}

// Positions `q` on linear gi's first item for this workgroup; false if it has none there.
template <int NF, int U>
__device__ __forceinline__ bool enter(const StreamArgs& a, int gi, Cursor<NF>& q, int wave) {
  constexpr int TN = 16 * NF;
  const plm_chain_gemm g = gemm_at(gi);
  q.gi = gi;
  q.split = g.split_k;
  q.items = ((g.N + TN - 1) / TN) * g.split_k;
  q.item = blockIdx.x;
  if (q.item >= q.items) return false;
  q.dep = g.dep;
  q.N = g.N;
  q.K = g.K;
  q.ldw = g.ldw;
  q.ldx = g.ldx;
  q.w = static_cast<const uint16_t*>(g.w);
  q.x = static_cast<const uint16_t*>(g.x);
  locate<NF, U>(q, wave);
  return true;
}

template <int NF, int U>
__device__ __forceinline__ bool first(const StreamArgs& a, Cursor<NF>& q, int wave) {
  for (int gi = 0; gi < a.count; ++gi)
    if (enter<NF, U>(a, gi, q, wave)) return true;
  return false;
}

template <int NF, int U>
__device__ __forceinline__ bool advance(const StreamArgs& a, Cursor<NF>& q, int wave) {
  if (++q.c < q.C) return true;
  q.item += a.G;
  if (q.item < q.items) {
    locate<NF, U>(q, wave);
    return true;
  }
  for (int gi = q.gi + 1; gi < a.count; ++gi)
    if (enter<NF, U>(a, gi, q, wave)) return true;
  return false;
}

// ------------------------------------------------------------------ compute wavefronts
//
// Operands travel HBM/L2 -> LDS by DMA (buffer_load ... lds: 16 bytes per lane, written to LDS in
// lane order, so reading slot + 16*lane back gives every lane exactly the MFMA operand it loaded)
// and LDS -> VGPRs by ds_read_b128. No vector register is the destination of a load in flight,
// so the compiler never inserts a vmcnt wait of its own in the compute loop; the single wait per
// chunk is explicit, and it leaves the weight ring's later chunks in flight.
//
// Per compute wavefront (all in LDS):
//   * weight ring: R slots of one chunk (U steps x NF fragments, 1 KiB each), filled R-1 chunks
//     ahead of the chunk being multiplied, across item and linear boundaries;
//   * X ring: 2 slots of one chunk (U steps x MT fragments), filled one chunk ahead (or, for the
//     first chunk of an item that depends on earlier linears, once the epilogue wavefront
//     publishes it may be read).
// The four wavefronts' partial tiles are summed pairwise through a spill area of two tiles:
// (w0 + w1) + (w2 + w3), the last sum by the epilogue wavefront.

typedef __attribute__((address_space(3))) u32x4 LdsVec;
typedef __attribute__((address_space(3))) void LdsVoid;

template <int MT, int NF>
constexpr size_t spill_bytes() {  // two partial tiles
  return static_cast<size_t>(2) * NF * MT * 64 * sizeof(f32x4);
}
template <int NF, int U>
constexpr size_t wslot_bytes() {
  return static_cast<size_t>(NF) * U * 1024;
}
template <int MT, int U>
constexpr size_t xslot_bytes() {
  return static_cast<size_t>(MT) * U * 1024;
}
constexpr size_t kTableReserve = 16 * 1024;  // descriptors of a chain of up to 186 linears
// Weight-ring depth that fits beside the spill area, the X rings and the descriptor reserve.
template <int MT, int NF, int U>
constexpr int ring_slots() {
  const long avail = static_cast<long>(kMaxLdsBytes) - static_cast<long>(kTableReserve) -
                     static_cast<long>(spill_bytes<MT, NF>()) -
                     static_cast<long>(kStreamKW * 2 * xslot_bytes<MT, U>());
  const long r = avail / static_cast<long>(kStreamKW * wslot_bytes<NF, U>());
  return r > 8 ? 8 : static_cast<int>(r);
}
// Dynamic LDS bytes past the descriptor table: spill area, weight rings, X rings.
template <int MT, int NF, int U>
constexpr size_t stream_lds_bytes() {
  return spill_bytes<MT, NF>() + kStreamKW * (ring_slots<MT, NF, U>() * wslot_bytes<NF, U>() + 2 * xslot_bytes<MT, U>());
}

struct Rings {
  char* spill;  // two partial tiles, float4 [2][NF][MT][64]
  char* w;      // this wavefront's weight ring
  char* x;      // this wavefront's X ring
};

template <int MT, int NF, int U>
__device__ __forceinline__ Rings rings_of(float* base, int wave) {
  constexpr int R = ring_slots<MT, NF, U>();
  char* b = reinterpret_cast<char*>(base);
  Rings r;
  r.spill = b;
  r.w = b + spill_bytes<MT, NF>() + static_cast<size_t>(wave) * R * wslot_bytes<NF, U>();
  r.x = b + spill_bytes<MT, NF>() + static_cast<size_t>(kStreamKW) * R * wslot_bytes<NF, U>() +
        static_cast<size_t>(wave) * 2 * xslot_bytes<MT, U>();
  return r;
}

// Steps of chunk q.c that this wavefront owns (0..U).
template <int NF, int U>
__device__ __forceinline__ int chunk_steps(const Cursor<NF>& q) {
  const int left = q.ns - q.c * U;
  return left < 0 ? 0 : (left < U ? left : U);
}

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, char* lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (LdsVoid*)(lds), 16, static_cast<int>(off), 0, 0, 0);
}

// Every (step, fragment) load is issued; steps past the wavefront's slice, K past the end and rows
// past the tile get an out-of-range offset, which writes zeros and touches no memory. A fixed
// number of loads per chunk is what makes the explicit wait counts exact.
template <int NF, int U>
__device__ __forceinline__ void dma_w(char* slot, const Cursor<NF>& q, bool live, int lane) {
  const int n = live ? chunk_steps<NF, U>(q) : 0;
  const auto rsrc = make_rsrc(q.w + static_cast<int64_t>(q.n0) * q.ldw, static_cast<uint32_t>(q.tn * q.ldw * 2));
  const int row = lane & 15;
  const int kq = (lane >> 4) << 3;
  const int st = q.st + q.c * U;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int k = (st + u) * 32 + kq;
    const bool kin = u < n && k < q.K;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const int r = 16 * f + row;
      const uint32_t off = (kin && r < q.tn) ? static_cast<uint32_t>((r * q.ldw + k) * 2) : kOutOfRange;
      dma16(rsrc, slot + (u * NF + f) * 1024, off);
    }
  }
}

template <int MT, int NF, int U>
__device__ __forceinline__ void dma_x(char* slot, const StreamArgs& a, const Cursor<NF>& q, bool live, int lane) {
  const int n = live ? chunk_steps<NF, U>(q) : 0;
  const auto rsrc = make_rsrc(q.x, static_cast<uint32_t>(a.M * q.ldx * 2));
  const int row = lane & 15;
  const int kq = (lane >> 4) << 3;
  const int st = q.st + q.c * U;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int k = (st + u) * 32 + kq;
    const bool kin = u < n && k < q.K;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = 16 * t + row;
      const uint32_t off = (kin && m < a.M) ? static_cast<uint32_t>((m * q.ldx + k) * 2) : kOutOfRange;
      dma16(rsrc, slot + (u * MT + t) * 1024, off);
    }
  }
}

// vmcnt(n) with the other counters left alone (gfx9 encoding: vmcnt[3:0] | vmcnt_hi[15:14],
// expcnt[6:4] = 7, lgkmcnt[11:8] = 15).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt is six bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Multiplies the chunk in `wslot` / `xslot` into acc.
template <int DT, int MT, int NF, int U>
__device__ __forceinline__ void mma_lds(const char* wslot, const char* xslot, f32x4 (&acc)[NF][MT], int lane) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    u32x4 wv[NF], xv[MT];
#pragma unroll
    for (int f = 0; f < NF; ++f)
      wv[f] = *(const LdsVec*)(wslot + (u * NF + f) * 1024 + lane * 16);
#pragma unroll
    for (int t = 0; t < MT; ++t)
      xv[t] = *(const LdsVec*)(xslot + (u * MT + t) * 1024 + lane * 16);
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[f][t] = mfma_16x16x32<DT>(wv[f], xv[t], acc[f][t]);
  }
}

// Spill slot of tile `half` (0, 1): lane l's acc[f][t] holds weight rows 16f + 4(l/16) .. +3
// (four consecutive Y columns) for X row 16t + l%16.
template <int MT, int NF>
__device__ __forceinline__ f32x4* spill_slot(char* spill, int half, int f, int t, int lane) {
  return reinterpret_cast<f32x4*>(spill) + ((half * NF + f) * MT + t) * 64 + lane;
}

// The first X chunk of an item that depends on earlier linears may only be read once the
// epilogue wavefront has seen the producer tiles finished; it publishes the item's sequence
// number in `ready` after this workgroup's previous item is through its barriers.
template <int NF>
__device__ __forceinline__ bool deferred_x(const Cursor<NF>& q) {
  return q.c == 0 && q.dep >= 0;
}

__device__ __forceinline__ void wait_ready(LdsFlag* ready, int seq) {
  // The epilogue wavefront's own waits are bounded, so this one ends too; the bound here is a
  // second guard.
  for (int i = 0; *ready < seq && i < (1 << 26); ++i) __builtin_amdgcn_s_sleep(2);
}

// Workgroup barrier for the item hand-off through LDS: this wavefront's LDS writes are complete,
// then s_barrier. Unlike __syncthreads() it does not wait for outstanding vector memory
// operations, so the weight ring's DMA stays in flight across it (a workgroup-scope release
// fence would also wait for the DMA writes into LDS). The memory clobber keeps the compiler
// from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// End of an item: the four partial tiles become (w0 + w1) and (w2 + w3) in the spill area.
//   B1: wavefronts 1 and 3 have spilled; 0 and 2 add them and spill the sums in their place.
//   B2: both sums are in LDS; the epilogue wavefront reads them.
//   B3: the epilogue wavefront has read them; the area is free for the next item.
template <int MT, int NF>
__device__ __forceinline__ void reduce_item(f32x4 (&acc)[NF][MT], char* spill, int wave, int lane) {
  const int half = wave >> 1;
  if (wave & 1) {
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
      for (int t = 0; t < MT; ++t) *spill_slot<MT, NF>(spill, half, f, t, lane) = acc[f][t];
  }
  lds_barrier();  // B1
  if (!(wave & 1)) {
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        f32x4* slot = spill_slot<MT, NF>(spill, half, f, t, lane);
        *slot = acc[f][t] + *slot;
      }
  }
  lds_barrier();  // B2
#pragma unroll
  for (int f = 0; f < NF; ++f)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[f][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  lds_barrier();  // B3
}

template <int DT, int MT, int NF, int U>
__device__ void compute_role(const StreamArgs& a, int wave, int lane, float* lds, LdsFlag* ready) {
  constexpr int R = ring_slots<MT, NF, U>();
  // Loads issued per chunk: X for the next chunk, then weights R-1 chunks ahead. Iteration i
  // issues X(i+1) and W(i+R-1), so chunk i's X and weights have at least kPerChunk loads issued
  // after them. When X(i) went out in iteration i-1 ahead of that iteration's weights W(i+R-2),
  // another NF*U loads follow it, and W(i) itself is older than X(i) only if it was not among
  // them, i.e. if R >= 3; a two-slot ring always waits for the late count.
  constexpr int kPerChunk = (MT + NF) * U;
  constexpr int kWaitLate = kPerChunk > 63 ? 63 : kPerChunk;
  constexpr int kWaitEarly = R < 3 ? kWaitLate : (kPerChunk + NF * U > 63 ? 63 : kPerChunk + NF * U);
  const Rings rg = rings_of<MT, NF, U>(lds, wave);
  Cursor<NF> q, nq, lq;
  f32x4 acc[NF][MT];
#pragma unroll
  for (int f = 0; f < NF; ++f)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[f][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  int seq = 0;
  if (!first<NF, U>(a, q, wave)) return;
  // Prologue: weights of the first R-1 chunks, X of the first.
  lq = q;
  bool lq_live = true;
#pragma unroll
  for (int i = 0; i < R - 1; ++i) {
    dma_w<NF, U>(rg.w + i * wslot_bytes<NF, U>(), lq, lq_live, lane);
    if (lq_live) lq_live = advance<NF, U>(a, lq, wave);
  }
  if (deferred_x<NF>(q)) wait_ready(ready, 0);
  dma_x<MT, NF, U>(rg.x, a, q, true, lane);
  bool x_late = true;  // X of chunk 0 was issued after every weight load before it
  for (int i = 0;; ++i) {
    nq = q;
    const bool has_next = advance<NF, U>(a, nq, wave);
    const bool defer = has_next && deferred_x<NF>(nq);
    char* xnext = rg.x + ((i + 1) & 1) * xslot_bytes<MT, U>();
    __builtin_amdgcn_sched_barrier(0);
    dma_x<MT, NF, U>(xnext, a, nq, has_next && !defer, lane);
    dma_w<NF, U>(rg.w + ((i + R - 1) % R) * wslot_bytes<NF, U>(), lq, lq_live, lane);
    if (lq_live) lq_live = advance<NF, U>(a, lq, wave);
    // This chunk's X and weights are in LDS once at most this many later loads are pending:
    // this iteration's, plus the previous iteration's weights when X was issued before them.
    if (x_late)
      wait_vmcnt<kWaitLate>();
    else
      wait_vmcnt<kWaitEarly>();
    x_late = defer;
    __builtin_amdgcn_sched_barrier(0);
    mma_lds<DT, MT, NF, U>(rg.w + (i % R) * wslot_bytes<NF, U>(), rg.x + (i & 1) * xslot_bytes<MT, U>(), acc, lane);
    __builtin_amdgcn_sched_barrier(0);
    if (q.c == q.C - 1) {
      reduce_item<MT, NF>(acc, rg.spill, wave, lane);
      ++seq;
    }
    if (!has_next) break;
    if (defer) {
      wait_ready(ready, seq);
      dma_x<MT, NF, U>(xnext, a, nq, true, lane);
    }
    q = nq;
  }
  wait_vmcnt<0>();  // no DMA into LDS may outlive the wavefront
}

// ------------------------------------------------------------------ epilogue wavefront

__device__ __forceinline__ int lane0_broadcast(int v) { return __shfl(v, 0, 64); }

// Polls until every lane's `ok` is true or the poll budget runs out (then flags an error).
template <typename Pred>
__device__ __forceinline__ void bounded_wait(const StreamArgs& a, Pred pred) {
  for (int i = 0;; ++i) {
    if (__all(pred())) return;
    if (i >= a.spin_limit) {
      if ((threadIdx.x & 63) == 0) publish(a.counters + kErrorSlot, 1);
      return;
    }
    __builtin_amdgcn_s_sleep(4);
  }
}

template <int DT>
__device__ __forceinline__ void store_y4(const plm_chain_gemm& g, int m, int n, int tn_left, f32x4 v, bool coherent) {
  // Four consecutive columns n..n+3 of row m; tn_left = valid columns from n (may be < 4 at N's end).
  if (g.out_f32) {
    float* y = static_cast<float*>(g.y) + static_cast<int64_t>(m) * g.ldy + n;
    if (tn_left >= 4 && (reinterpret_cast<uintptr_t>(y) & 15) == 0) {
      *reinterpret_cast<f32x4*>(y) = v;
    } else {
      for (int j = 0; j < 4 && j < tn_left; ++j) y[j] = v[j];
    }
    return;
  }
  uint16_t* y = static_cast<uint16_t*>(g.y) + static_cast<int64_t>(m) * g.ldy + n;
  const uint32_t lo = static_cast<uint32_t>(to_bits16<DT>(v[0])) | (static_cast<uint32_t>(to_bits16<DT>(v[1])) << 16);
  const uint32_t hi = static_cast<uint32_t>(to_bits16<DT>(v[2])) | (static_cast<uint32_t>(to_bits16<DT>(v[3])) << 16);
  if (tn_left >= 4 && (reinterpret_cast<uintptr_t>(y) & 7) == 0) {
    const uint64_t bits = static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32);
    if (coherent)
      publish(reinterpret_cast<uint64_t*>(y), bits);
    else
      *reinterpret_cast<uint64_t*>(y) = bits;
  } else {
    const uint16_t h[4] = {static_cast<uint16_t>(lo), static_cast<uint16_t>(lo >> 16), static_cast<uint16_t>(hi),
                           static_cast<uint16_t>(hi >> 16)};
    for (int j = 0; j < 4 && j < tn_left; ++j) {
      if (coherent)
        publish(y + j, h[j]);
      else
        y[j] = h[j];
    }
  }
}

template <int DT, int MT, int NF>
__device__ void epilogue_role(const StreamArgs& a, int lane, float* lds, LdsFlag* ready) {
  constexpr int TN = 16 * NF;
  constexpr int GROUPS = TN / 4;         // four-column groups per tile row
  constexpr int ROWS_PER_PASS = 64 / GROUPS;
  constexpr int PASSES = (16 * MT + ROWS_PER_PASS - 1) / ROWS_PER_PASS;
  char* spill = reinterpret_cast<char*>(lds);
  const int epoch = a.sync ? lane0_broadcast(lane == 0 ? collect(a.counters + kEpochSlot) : 0) : 0;
  const int cg = lane % GROUPS;          // this lane's column group
  const int f = cg / 4, qd = cg % 4;     // fragment and lane quarter that hold it
  int seq = 0;
  for (int gi = 0; gi < a.count; ++gi) {
    const plm_chain_gemm g = gemm_at(gi);
    const int tiles = (g.N + TN - 1) / TN;
    const int items = tiles * g.split_k;
    for (int item = blockIdx.x; item < items; item += a.G) {
      const int tile = item / g.split_k;
      const int s = item - tile * g.split_k;
      const int n0 = tile * TN;
      const int tn = min(TN, g.N - n0);
      if (g.dep >= 0) {
        // X columns [k0, k1) come from the producer's tiles k0/TN .. (k1-1)/TN.
        const plm_chain_gemm p = gemm_at(g.dep);
        int lo, hi;
        split_range(g.K, s, g.split_k, lo, hi);
        const int k0 = lo * 32, k1 = min(hi * 32, g.K);
        if (k1 > k0) {
          const int t0 = k0 / TN, t1 = (k1 - 1) / TN;
          const int* done = a.counters + p.done_base;
          bounded_wait(a, [&] {
            bool ok = true;
            for (int t = t0 + lane; t <= t1; t += 64) ok = ok && collect(done + t) == epoch + 1;
            return ok;
          });
        }
      }
      if (lane == 0) *ready = seq;
      lds_barrier();  // B1: wavefronts 1 and 3 have spilled
      lds_barrier();  // B2: the pair sums are in LDS
      ++seq;
      // The item's tile is (w0 + w1) + (w2 + w3). Pass p covers rows ROWS_PER_PASS * p + lane /
      // GROUPS, columns 4 * cg .. +3. Its stores are issued before B3 releases the spill area.
      const bool coherent = g.consumed != 0;
      const int n = 4 * cg;
      const int Np = (g.N + 3) & ~3;  // split partial planes are [M][Np] fp32
      const uint32_t plane = static_cast<uint32_t>(a.M) * Np * 4u;
      const auto prs = make_rsrc(a.partial + g.partial_offset, g.split_k > 1 ? plane * g.split_k : 0u);
#pragma unroll
      for (int p = 0; p < PASSES; ++p) {
        const int m = p * ROWS_PER_PASS + lane / GROUPS;
        if (m < a.M && n < tn) {
          const int t = m >> 4, l = 16 * qd + (m & 15);
          const f32x4 v = *spill_slot<MT, NF>(spill, 0, f, t, l) + *spill_slot<MT, NF>(spill, 1, f, t, l);
          if (g.split_k == 1) {
            store_y4<DT>(g, m, n0 + n, tn - n, v, coherent);
          } else {
            // Every four-column group of a partial is one 16-byte device-coherent store.
            const uint32_t off = s * plane + (static_cast<uint32_t>(m) * Np + n0 + n) * 4u;
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), prs, off, 0, kCoherent);
          }
        }
      }
      lds_barrier();  // B3: the spill area is free again
      if (g.split_k > 1) {
        // The last of the tile's splits to arrive sums all of them in split order.
        __builtin_amdgcn_s_waitcnt(0);  // the partial is written through before we count in
        int* counter = a.counters + g.arrive_base + tile;
        int before = 0;
        if (lane == 0) {
          before = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (before == g.split_k - 1) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        before = lane0_broadcast(before);
        if (before != g.split_k - 1) continue;
        // Four passes at a time, each summing its splits in order; the four passes' loads of one
        // split are in flight together.
        constexpr int BATCH = 4;
        for (int p0 = 0; p0 < PASSES; p0 += BATCH) {
          f32x4 sum[BATCH];
          uint32_t off[BATCH];
#pragma unroll
          for (int b = 0; b < BATCH; ++b) {
            const int m = (p0 + b) * ROWS_PER_PASS + lane / GROUPS;
            off[b] = (m < a.M && n < tn) ? (static_cast<uint32_t>(m) * Np + n0 + n) * 4u : kOutOfRange;
            sum[b] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
          for (int q = 0; q < g.split_k; ++q) {
            u32x4 part[BATCH];
#pragma unroll
            for (int b = 0; b < BATCH; ++b)
              part[b] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      prs, off[b] == kOutOfRange ? kOutOfRange : off[b] + q * plane, 0,
                                                      kCoherent));
#pragma unroll
            for (int b = 0; b < BATCH; ++b) sum[b] += __builtin_bit_cast(f32x4, part[b]);
          }
#pragma unroll
          for (int b = 0; b < BATCH; ++b) {
            const int m = (p0 + b) * ROWS_PER_PASS + lane / GROUPS;
            if (m < a.M && n < tn) store_y4<DT>(g, m, n0 + n, tn - n, sum[b], coherent);
          }
        }
      }
      if (g.consumed) {
        __builtin_amdgcn_s_waitcnt(0);  // every store of the tile is written through
        if (lane == 0) publish(a.counters + g.done_base + tile, epoch + 1);
      }
    }
  }
  if (a.sync) {
    __builtin_amdgcn_s_waitcnt(0);
    if (lane == 0) {
      const int before = __hip_atomic_fetch_add(a.counters + kExitSlot, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (before == a.G - 1) {
        __hip_atomic_store(a.counters + kExitSlot, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.counters + kEpochSlot, epoch + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

template <int DT, int MT, int NF, int U>
__global__ __launch_bounds__(64 * (kStreamKW + 1)) void stream_gemm_kernel(StreamArgs a) {
  __shared__ int ready;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  {
    // Descriptors into LDS: from the device table for a chain, from the kernel arguments else.
    const int* src = a.chain != nullptr ? reinterpret_cast<const int*>(a.chain) : reinterpret_cast<const int*>(&a.single);
    int* dst = reinterpret_cast<int*>(stream_lds);
    const int words = a.count * static_cast<int>(sizeof(plm_chain_gemm) / sizeof(int));
    for (int i = threadIdx.x; i < words; i += blockDim.x) dst[i] = src[i];
  }
  float* lds = stream_lds + table_bytes(a.count) / sizeof(float);
  if (threadIdx.x == 0) ready = -1;
  __syncthreads();
  LdsFlag* flag = (LdsFlag*)&ready;
  if (wave < kStreamKW)
    compute_role<DT, MT, NF, U>(a, wave, lane, lds, flag);
  else
    epilogue_role<DT, MT, NF>(a, lane, lds, flag);
}

// Compiled tile set: the weight ring is at least two chunks deep beside the spill area and the X
// rings, and the compute wavefronts' registers (accumulators, one step's operands) fit in 256
// VGPRs so that the epilogue wavefront can share a SIMD with a compute wavefront.
template <int MT, int NF, int U>
constexpr bool stream_compiled() {
  if (MT < 1 || MT > 8) return false;
  if (NF != 1 && NF != 2 && NF != 4) return false;
  if (U != 1 && U != 2 && U != 4) return false;
  if (ring_slots<MT, NF, U>() < 2) return false;
  return NF * MT * 4 + (NF + MT) * 4 + 64 <= 256;
}

hipError_t stream_dispatch_bf16(StreamArgs& a, int nf, int u, int cus, hipStream_t s, bool dry);
hipError_t stream_dispatch_f16(StreamArgs& a, int nf, int u, int cus, hipStream_t s, bool dry);

// Workgroups of one launch: persistent, at most what fits on the device at once.
template <int DT, int MT, int NF, int U>
hipError_t stream_launch(StreamArgs& a, int cus, hipStream_t stream, bool dry) {
  if constexpr (!stream_compiled<MT, NF, U>()) {
    return hipErrorInvalidConfiguration;
  } else {
    if (dry) return hipSuccess;
    auto kern = stream_gemm_kernel<DT, MT, NF, U>;
    const size_t lds = table_bytes(a.count) + stream_lds_bytes<MT, NF, U>();
    if (lds > kMaxLdsBytes) return hipErrorInvalidConfiguration;
    static size_t lds_allowed = 64 * 1024;  // the default dynamic LDS limit
    if (lds > lds_allowed) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
      if (e != hipSuccess) return e;
      lds_allowed = lds;
    }
    // Workgroups resident per CU at this LDS size (cached for the one-linear size).
    static int single_per_cu = 0;
    int per_cu = a.count == 1 ? single_per_cu : 0;
    if (per_cu == 0) {
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kern),
                                                       64 * (kStreamKW + 1), lds) != hipSuccess ||
          per_cu < 1)
        return hipErrorInvalidConfiguration;
      if (a.count == 1) single_per_cu = per_cu;
    }
    // a.G arrives as the most items any linear has; a chained launch needs every workgroup
    // resident at once (they wait on each other), a single linear needs no more than its items.
    const int resident = cus * per_cu;
    a.G = a.sync ? resident : min(resident, a.G);
    hipLaunchKernelGGL(kern, dim3(a.G), dim3(64 * (kStreamKW + 1)), lds, stream, a);
    return hipGetLastError();
  }
}

template <int DT, int MT>
hipError_t stream_pick(StreamArgs& a, int nf, int u, int cus, hipStream_t s, bool dry) {
#define PLM_STREAM_CASE(NF_, U_) \
  if (nf == NF_ && u == U_) return stream_launch<DT, MT, NF_, U_>(a, cus, s, dry);
  PLM_STREAM_CASE(1, 1)
  PLM_STREAM_CASE(1, 2)
  PLM_STREAM_CASE(1, 4)
  PLM_STREAM_CASE(2, 1)
  PLM_STREAM_CASE(2, 2)
  PLM_STREAM_CASE(2, 4)
  PLM_STREAM_CASE(4, 1)
  PLM_STREAM_CASE(4, 2)
  PLM_STREAM_CASE(4, 4)
#undef PLM_STREAM_CASE
  return hipErrorInvalidConfiguration;
}

template <int DT>
hipError_t stream_dispatch(StreamArgs& a, int nf, int u, int cus, hipStream_t s, bool dry) {
  switch ((a.M + 15) / 16) {
    case 1: return stream_pick<DT, 1>(a, nf, u, cus, s, dry);
    case 2: return stream_pick<DT, 2>(a, nf, u, cus, s, dry);
    case 3: return stream_pick<DT, 3>(a, nf, u, cus, s, dry);
    case 4: return stream_pick<DT, 4>(a, nf, u, cus, s, dry);
    case 5: return stream_pick<DT, 5>(a, nf, u, cus, s, dry);
    case 6: return stream_pick<DT, 6>(a, nf, u, cus, s, dry);
    case 7: return stream_pick<DT, 7>(a, nf, u, cus, s, dry);
    case 8: return stream_pick<DT, 8>(a, nf, u, cus, s, dry);
  }
  return hipErrorInvalidConfiguration;
}

}  // namespace plm
