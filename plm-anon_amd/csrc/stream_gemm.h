// Streaming skinny GEMM for the PLM round's dense linears on gfx950 (MI355X).
//
// Y[M,N] = X[M,K] · W[N,K]^T with fp32 accumulation, for a single linear or for a chain of linears
// in one launch, where a linear may read an earlier one's output (the round's linears back to
// back). M is the round width (k verify rows + k^2 proposal tokens, 56 at k=7), so the weights are
// almost all of the bytes and the kernel is an HBM stream of W.
//
// Work: item = one tile of 64*NF weight rows x one of `split` K ranges. Each workgroup is
// persistent and takes items blockIdx.x, blockIdx.x + G, ... of every linear in turn.
//
// Workgroup = 4 compute wavefronts + kLoaders loader wavefronts + 1 epilogue wavefront.
//   * The loaders stream the workgroup's chunks into a ring of R slots in LDS by buffer-to-LDS DMA,
//     up to R-1 chunks ahead, across item and linear boundaries: a chunk is two 32-wide K steps,
//     i.e. one 128-byte line of each of the tile's weight rows and X rows, and each DMA
//     instruction moves 8 rows x 128 bytes (whole lines). It waits only on its own loads and on
//     slots being free, so the memory stream never stops for the arithmetic.
//   * Compute wavefront w owns weight rows [16*NF*w, 16*NF*(w+1)) of the tile and the item's whole
//     K range, so it accumulates its rows to the end with no reduction across wavefronts; all four
//     share the chunk's one copy of X. It reads the chunk from LDS into MFMA operands
//     (v_mfma_f32_16x16x32_{bf16,f16}) and hands the slot back.
//   * At an item's end each compute wavefront writes its rows of Y (or, with split > 1, of an fp32
//     partial) straight from its accumulators: it issues no memory loads, so its stores hold
//     nothing up. The epilogue wavefront counts split arrivals (the last workgroup of a tile sums
//     the partials in split order), marks tiles finished, and checks, while the others work,
//     whether the next item's X is ready. The loaders never store or wait on other workgroups: on
//     gfx9 vmcnt covers loads and stores in issue order, so that would drain their stream.
// LDS counters carry the hand-offs (chunks landed, chunks multiplied, tiles written).
//
// Chains: a linear whose X is an earlier linear's Y waits, per item, only for the producer tiles
// covering its K range (tile-done flags), so consecutive linears overlap and the weight stream
// does not stop at linear boundaries. Producer Y and all cross-workgroup data go through
// device-coherent stores/loads; a consumer reads X through L2, which is safe because every
// 128-byte line of a consumed Y is written by one workgroup and read by nobody before its
// done flag is set (the host validates the layout that guarantees it).
//
// Results are bitwise reproducible: every output element is one wavefront's MFMA accumulation
// over its item's K steps in ascending order, and split partials are summed in split order.
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
constexpr int kDoneCapacity = kStreamDoneEnd - kDoneBase;
constexpr int kStreamKW = 4;      // compute wavefronts per workgroup
constexpr int kStreamU = 2;       // 32-wide K steps per chunk: one 128-byte line per row
#ifndef PLM_STREAM_LOADERS
#define PLM_STREAM_LOADERS 4
#endif
constexpr int kLoaders = PLM_STREAM_LOADERS;  // loader wavefronts per workgroup (1, 2 or 4)
static_assert(kLoaders == 1 || kLoaders == 2 || kLoaders == 4, "loaders split 8*NF weight row groups evenly");
constexpr int kStreamWaves = kStreamKW + kLoaders + 1;
constexpr size_t kMaxLdsBytes = 160 * 1024 - 256;  // dynamic LDS: 160 KiB per CU on gfx950, less static

struct StreamArgs {
  const plm_chain_gemm* chain;  // device array of `count` linears, or nullptr: use `single`
  plm_chain_gemm single;
  int count;
  int M;
  int G;           // workgroups in the grid
  int sync;        // some linear reads an earlier one's output
  int spin_limit;  // polls before a wait gives up
  int ring;        // chunk slots of the ring (2..8)
  int* counters;
  float* partial;
};

// Dynamic LDS: the launch's linear descriptors (copied from the kernel arguments or the device
// table at kernel start, 16-byte aligned), then the ring.
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

// Hand-off flags between the wavefronts, typed as LDS so that polling one is a ds_read
// (lgkmcnt) and never a flat load, whose wait would also drain the compute wavefronts' DMA.
typedef __attribute__((address_space(3))) volatile int LdsFlag;
typedef __attribute__((address_space(3))) int LdsInt;
typedef __attribute__((address_space(3))) u32x4 LdsVec;
typedef __attribute__((address_space(3))) void LdsVoid;

__device__ __forceinline__ int lds_uniform(LdsFlag* p) { return __builtin_amdgcn_readfirstlane(*p); }
__device__ __forceinline__ void lds_count(LdsFlag* p) {
  __hip_atomic_fetch_add((LdsInt*)p, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

constexpr size_t table_bytes(int count) { return (static_cast<size_t>(count) * sizeof(plm_chain_gemm) + 15) / 16 * 16; }

// K-step range [lo, hi) of split `s` out of `split` (ceil(K/32) steps in all).
__device__ __forceinline__ void split_range(int K, int s, int split, int& lo, int& hi) {
  const int steps = (K + 31) >> 5;
  lo = static_cast<int>(static_cast<int64_t>(s) * steps / split);
  hi = static_cast<int>(static_cast<int64_t>(s + 1) * steps / split);
}

// ------------------------------------------------------------------ LDS layout
//
// Ring slot: the chunk's X (16*MT rows of 128 bytes) then the tile's weights (64*NF rows of 128
// bytes; compute wavefront w's 16*NF rows at offset w * 2*NF KiB). Rows are stored in groups of 8
// (one DMA instruction, 1 KiB): row r of a group at byte 128*(r%8), its 16-byte piece p (K
// elements 8p..8p+7 of the chunk) at 16*(p ^ swizzle(r)), with r counted inside the compute
// wavefront's rows. The swizzle makes the MFMA operand reads (16 rows x one piece per
// instruction) hit distinct banks.
// X row groups per loader per chunk: the chunk's 2*MT groups dealt round-robin, padded to a
// multiple of the loader count (padding groups receive zeros and are never read).
template <int MT>
constexpr int x_loads() {
  return (2 * MT + kLoaders - 1) / kLoaders;
}
template <int MT>
constexpr size_t xpart_bytes() {
  return static_cast<size_t>(x_loads<MT>()) * kLoaders * 1024;
}
template <int NF>
constexpr size_t wpart_bytes() {  // one compute wavefront's weights
  return static_cast<size_t>(NF) * 16 * 128;
}
template <int MT, int NF>
constexpr size_t slot_bytes() {
  return xpart_bytes<MT>() + kStreamKW * wpart_bytes<NF>();
}
// DMA instructions per loader per chunk: its share of the 8*NF weight row groups and of the X row
// groups, 1 KiB each.
template <int NF>
constexpr int w_loads() {
  return 8 * NF / kLoaders;
}
template <int MT, int NF>
constexpr int chunk_loads() {
  return w_loads<NF>() + x_loads<MT>();
}
constexpr size_t kTableReserve = 16 * 1024;  // descriptors of a chain of up to 186 linears
constexpr int kMaxRing = 8;
// Ring depth that fits in `lds_free` bytes (0 if under two).
template <int MT, int NF>
constexpr int ring_slots(size_t lds_free) {
  long r = static_cast<long>(lds_free / slot_bytes<MT, NF>());
  if (r > kMaxRing) r = kMaxRing;
  return r < 2 ? 0 : static_cast<int>(r);
}
// Ring depth when `table` bytes of descriptors precede the ring.
template <int MT, int NF>
constexpr int ring_for_table(size_t table) {
  return table >= kMaxLdsBytes ? 0 : ring_slots<MT, NF>(kMaxLdsBytes - table);
}
// Chunks a loader keeps in flight: two slots short of the ring, so that a landed chunk waits in
// LDS for the compute wavefronts while the next slot is already free to refill (with one slot
// short, every issue would wait on the multiplication of the oldest landed chunk), and at most
// what vmcnt's six bits can count.
template <int MT, int NF>
constexpr int flight_depth(int ring) {
  const int by_vmcnt = 63 / chunk_loads<MT, NF>();
  const int by_ring = ring > 2 ? ring - 2 : 1;
  return by_ring < by_vmcnt ? by_ring : by_vmcnt;
}

__device__ __forceinline__ int swizzle(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// ------------------------------------------------------------------ item cursor

// Where a wavefront is in the workgroup's stream of chunks.
struct Cursor {
  int gi, item, c, C;  // linear, item, chunk within the item, chunks per item
  int seq;             // items this workgroup started before this one (across the chain)
  int items, split, dep;
  int r0, rows;        // the tile's weight rows [r0, r0 + rows) (rows <= 64*NF)
  int st, ns;          // the item's K steps [st, st + ns)
  int K;
  int64_t ldw, ldx;
  const uint16_t* w;
  const uint16_t* x;
};

// Tile, K range and chunk count of item q.item (at least one chunk, so that every item has an
// end the epilogue sees).
template <int NF>
__device__ __forceinline__ void locate(Cursor& q, int N) {
  const int tile = q.item / q.split;
  const int s = q.item - tile * q.split;
  q.r0 = tile * 64 * NF;
  q.rows = min(64 * NF, N - q.r0);
  int lo, hi;
  split_range(q.K, s, q.split, lo, hi);
  q.st = lo;
  q.ns = hi - lo;
  q.C = q.ns > 0 ? (q.ns + kStreamU - 1) / kStreamU : 1;
  q.c = 0;
}

template <int NF>
__device__ __forceinline__ int items_of(const plm_chain_gemm& g) {
  return ((g.N + 64 * NF - 1) / (64 * NF)) * g.split_k;
}

// Positions `q` on linear gi's first item for this workgroup; false if it has none there.
template <int NF>
__device__ __forceinline__ bool enter(const StreamArgs& a, int gi, Cursor& q) {
  const plm_chain_gemm g = gemm_at(gi);
  q.gi = gi;
  q.split = g.split_k;
  q.items = items_of<NF>(g);
  q.item = blockIdx.x;
  if (q.item >= q.items) return false;
  q.dep = g.dep;
  q.K = g.K;
  q.ldw = g.ldw;
  q.ldx = g.ldx;
  q.w = static_cast<const uint16_t*>(g.w);
  q.x = static_cast<const uint16_t*>(g.x);
  locate<NF>(q, g.N);
  return true;
}

template <int NF>
__device__ __forceinline__ bool first(const StreamArgs& a, Cursor& q) {
  q.seq = 0;
  for (int gi = 0; gi < a.count; ++gi)
    if (enter<NF>(a, gi, q)) return true;
  return false;
}

template <int NF>
__device__ __forceinline__ bool advance(const StreamArgs& a, Cursor& q) {
  if (++q.c < q.C) return true;
  ++q.seq;
  q.item += a.G;
  if (q.item < q.items) {
    locate<NF>(q, gemm_at(q.gi).N);
    return true;
  }
  for (int gi = q.gi + 1; gi < a.count; ++gi)
    if (enter<NF>(a, gi, q)) return true;
  return false;
}

// ------------------------------------------------------------------ wavefront hand-offs

// The wavefront-shared state in LDS.
struct Flags {
  LdsFlag* ready;     // items whose X may be read (sequence number), set by the epilogue
  LdsFlag* staged;    // compute wavefronts that have written their part of the tile (4 per item)
  LdsFlag* consumed;  // chunks the compute wavefronts have multiplied (4 per chunk)
  LdsFlag* loaded;    // per loader: chunks it has landed in LDS
};

// Polls an LDS value until it reaches `target`. The partner wavefronts' own waits are bounded,
// so this one ends too; the bound here is a second guard.
__device__ __forceinline__ void wait_lds(LdsFlag* p, int target) {
  for (int i = 0; lds_uniform(p) < target && i < (1 << 26); ++i) __builtin_amdgcn_s_sleep(1);
}

// The same without sleeping, where the wait is normally short.
__device__ __forceinline__ void spin_lds(LdsFlag* p, int target) {
  for (int i = 0; lds_uniform(p) < target && i < (1 << 28); ++i) {
  }
}

__device__ __forceinline__ int next_slot(int s, int R) { return s + 1 == R ? 0 : s + 1; }

// ------------------------------------------------------------------ loader wavefront
//
// Streams the chunks of the workgroup's items into the ring: weights HBM -> LDS and X L2 -> LDS
// by buffer-to-LDS DMA (16 bytes per lane; lane l's bytes land at 16*l of the 1 KiB block, so
// lane l loads the piece that belongs there). Every chunk is the same number of DMA instructions
// (masked lanes get an out-of-range offset: they write zeros and touch no memory), so the one
// vmcnt wait per chunk is an exact count that leaves the later chunks in flight. Only this
// wavefront issues vector memory operations for the ring; the compute wavefronts only read LDS.

// Cache policy of the weight stream: non-temporal (read once, should not displace X in L2).
constexpr int kStreaming = 2;

template <int AUX>
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, char* lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (LdsVoid*)(lds), 16, static_cast<int>(off), 0, 0, AUX);
}

// Byte offset of the piece that belongs at piece slot lane%8 of a row in 8-row group j (within a
// compute wavefront's rows, or of X): piece (lane%8) ^ swizzle(row), row % 8 = lane / 8 and
// (row / 8) % 2 = j % 2.
__device__ __forceinline__ uint32_t piece_bytes(int j, int lane) {
  return 16u * static_cast<uint32_t>((lane & 7) ^ (lane >> 3) ^ (j & 1));
}

// Per-lane byte offsets, relative to the chunk's K position, of one chunk's loads for the current
// item: row offset + swizzled piece, out of range for rows past the tile or past M. Computed once
// per item; a full chunk then needs scalar work only (its K position moves the buffer base).
// Loader l takes weight row groups l, l + kLoaders, ... (group g: compute wavefront g / (2NF), its
// group g % (2NF)) and X row groups likewise.
template <int MT, int NF>
struct ChunkOffsets {
  uint32_t w[w_loads<NF>()];
  uint32_t x[x_loads<MT>()];
};

template <int MT, int NF>
__device__ __forceinline__ void item_offsets(ChunkOffsets<MT, NF>& io, const StreamArgs& a, const Cursor& q, int ld,
                                             int lane) {
#pragma unroll
  for (int i = 0; i < w_loads<NF>(); ++i) {
    const int g = ld + kLoaders * i;
    const int r = 8 * g + (lane >> 3);
    io.w[i] = r < q.rows ? static_cast<uint32_t>(r * q.ldw * 2) + piece_bytes(g, lane) : kOutOfRange;
  }
#pragma unroll
  for (int i = 0; i < x_loads<MT>(); ++i) {
    const int j = ld + kLoaders * i;
    const int m = 8 * j + (lane >> 3);
    io.x[i] = (j < 2 * MT && m < a.M) ? static_cast<uint32_t>(m * q.ldx * 2) + piece_bytes(j, lane) : kOutOfRange;
  }
}

// Byte offset (within a row) of the piece lane `lane` loads for chunk q.c in row group j, or
// kOutOfRange past the item's K range (the item's last, partial chunk).
__device__ __forceinline__ uint32_t partial_piece(const Cursor& q, int j, int lane) {
  const int p = (lane & 7) ^ (lane >> 3) ^ (j & 1);
  const int step = q.c * kStreamU + (p >> 2);
  const int k = (q.st + step) * 32 + 8 * (p & 3);
  return (step < q.ns && k < q.K) ? static_cast<uint32_t>(k * 2) : kOutOfRange;
}

// Issues loader ld's share of chunk q into `slot`: weights, and X if `with_x` (else zeros).
template <int MT, int NF>
__device__ __forceinline__ void issue_chunk(char* slot, const StreamArgs& a, const Cursor& q, bool with_x, int ld,
                                            int lane, const ChunkOffsets<MT, NF>& io) {
  char* wpart = slot + xpart_bytes<MT>();
  const uint32_t wbytes = static_cast<uint32_t>(q.rows * q.ldw * 2);
  const uint32_t xbytes = with_x ? static_cast<uint32_t>(a.M * q.ldx * 2) : 0u;
  const char* wbase = reinterpret_cast<const char*>(q.w + static_cast<int64_t>(q.r0) * q.ldw);
  const char* xbase = reinterpret_cast<const char*>(q.x);
  if ((q.c + 1) * kStreamU <= q.ns && (q.st + (q.c + 1) * kStreamU) * 32 <= q.K) {
    // Wholly inside the item's K range: the per-item offsets from a base at the chunk's K position.
    const uint32_t kbyte = static_cast<uint32_t>(q.st + q.c * kStreamU) * 64u;
    const auto wr = make_rsrc(wbase + kbyte, wbytes > kbyte ? wbytes - kbyte : 0u);
    const auto xr = make_rsrc(xbase + kbyte, xbytes > kbyte ? xbytes - kbyte : 0u);
#pragma unroll
    for (int i = 0; i < w_loads<NF>(); ++i) dma16<kStreaming>(wr, wpart + (ld + kLoaders * i) * 1024, io.w[i]);
#pragma unroll
    for (int i = 0; i < x_loads<MT>(); ++i) dma16<0>(xr, slot + (ld + kLoaders * i) * 1024, io.x[i]);
  } else {
    const auto wr = make_rsrc(wbase, wbytes);
    const auto xr = make_rsrc(xbase, xbytes);
#pragma unroll
    for (int i = 0; i < w_loads<NF>(); ++i) {
      const int g = ld + kLoaders * i;
      const uint32_t k = partial_piece(q, g, lane);
      dma16<kStreaming>(wr, wpart + g * 1024, (k == kOutOfRange || io.w[i] == kOutOfRange) ? kOutOfRange
                                                                                          : io.w[i] - piece_bytes(g, lane) + k);
    }
#pragma unroll
    for (int i = 0; i < x_loads<MT>(); ++i) {
      const int j = ld + kLoaders * i;
      const uint32_t k = partial_piece(q, j, lane);
      dma16<0>(xr, slot + j * 1024, (k == kOutOfRange || io.x[i] == kOutOfRange) ? kOutOfRange
                                                                                 : io.x[i] - piece_bytes(j, lane) + k);
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

// The chunk issued D chunks ago is in LDS once at most D chunks of loads are outstanding.
template <int L>
__device__ __forceinline__ void wait_depth(int D) {
  switch (D) {
    case 1: wait_vmcnt<L>(); break;
    case 2: wait_vmcnt<(2 * L > 63 ? 0 : 2 * L)>(); break;
    case 3: wait_vmcnt<(3 * L > 63 ? 0 : 3 * L)>(); break;
    case 4: wait_vmcnt<(4 * L > 63 ? 0 : 4 * L)>(); break;
    case 5: wait_vmcnt<(5 * L > 63 ? 0 : 5 * L)>(); break;
    case 6: wait_vmcnt<(6 * L > 63 ? 0 : 6 * L)>(); break;
    default: wait_vmcnt<(7 * L > 63 ? 0 : 7 * L)>(); break;
  }
}

// Issues only loader ld's share of chunk q's X into `slot` (per-lane offsets; the slow path that
// fills in X for chunks issued before their producer tiles were finished).
template <int MT>
__device__ __forceinline__ void issue_x(char* slot, const StreamArgs& a, const Cursor& q, int ld, int lane) {
  const auto xr = make_rsrc(q.x, static_cast<uint32_t>(a.M * q.ldx * 2));
#pragma unroll
  for (int i = 0; i < x_loads<MT>(); ++i) {
    const int j = ld + kLoaders * i;
    const int m = 8 * j + (lane >> 3);
    const uint32_t k = partial_piece(q, j, lane);
    dma16<0>(xr, slot + j * 1024,
             (j < 2 * MT && m < a.M && k != kOutOfRange) ? static_cast<uint32_t>(m * q.ldx * 2) + k : kOutOfRange);
  }
}

// Chunks of a loader whose X has not been issued yet (their items read earlier linears whose
// tiles were not finished when the weights went out): from chunk `first` (cursor `q`, ring slot
// `slot`) up to the last chunk issued.
struct MissingX {
  int first;  // chunk index, or -1 when every issued chunk has its X
  int slot;
  Cursor q;
};

// Issues the X of the missing chunks whose items may now be read, in order, and lands everything:
// afterwards every issued chunk before `m.first` (all of them when m.first == -1) is complete in LDS.
template <int MT, int NF>
__device__ void fill_missing_x(char* ring, const StreamArgs& a, int issued, int R, int ld, int lane, const Flags& fl,
                               MissingX& m) {
  constexpr size_t SLOT = slot_bytes<MT, NF>();
  wait_vmcnt<0>();  // the zeros written in place of the missing X have landed before the real X
  Cursor t = m.q;
  int slot = m.slot;
  int c = m.first;
  m.first = -1;
  const int ready = lds_uniform(fl.ready);
  for (; c < issued; ++c) {
    if (t.dep >= 0 && ready < t.seq) {
      m.first = c;
      m.slot = slot;
      m.q = t;
      break;
    }
    issue_x<MT>(ring + slot * SLOT, a, t, ld, lane);
    slot = next_slot(slot, R);
    if (!advance<NF>(a, t)) break;
  }
  wait_vmcnt<0>();
}

template <int MT, int NF>
__device__ void loader_role(const StreamArgs& a, int ld, int lane, char* lds, const Flags& fl) {
  constexpr size_t SLOT = slot_bytes<MT, NF>();
  constexpr int L = chunk_loads<MT, NF>();
  static_assert(L <= 63, "one chunk's loads fit in vmcnt");
  const int R = a.ring;
  const int D = flight_depth<MT, NF>(R);
  char* ring = lds;
  Cursor q;
  if (!first<NF>(a, q)) return;
  ChunkOffsets<MT, NF> io;
  MissingX miss;
  miss.first = -1;
  int slot = 0, issued = 0, landed = 0;
  // Publishes how many chunks are complete in LDS (weights and X).
  auto publish_loaded = [&]() { fl.loaded[ld] = miss.first >= 0 ? min(landed, miss.first) : landed; };
  for (;;) {
    if (issued >= R) {
      // The slot's previous chunk must have been multiplied by all four compute wavefronts. If it
      // still lacks its X, wait for its producer tiles (the epilogue publishes them in `ready`)
      // and fill it in first: the compute wavefronts cannot get past it before.
      if (miss.first >= 0 && miss.first <= issued - R) {
        // Publish every complete chunk before blocking: the producer tiles may be this
        // workgroup's own earlier items, which the compute wavefronts must be able to finish.
        wait_vmcnt<0>();
        landed = issued;
        publish_loaded();
        wait_lds(fl.ready, miss.q.seq);
        fill_missing_x<MT, NF>(ring, a, issued, R, ld, lane, fl, miss);
        landed = issued;
        publish_loaded();
      }
      spin_lds(fl.consumed, kStreamKW * (issued - R + 1));
    }
    if (q.c == 0) item_offsets<MT, NF>(io, a, q, ld, lane);
    // Weights go out regardless; X only once every earlier chunk has its X and this item's
    // producer tiles are finished.
    const bool with_x = miss.first < 0 && (q.dep < 0 || lds_uniform(fl.ready) >= q.seq);
    if (!with_x && miss.first < 0) {
      miss.first = issued;
      miss.slot = slot;
      miss.q = q;
    }
    issue_chunk<MT, NF>(ring + slot * SLOT, a, q, with_x, ld, lane, io);
    ++issued;
    slot = next_slot(slot, R);
    if (miss.first >= 0 && lds_uniform(fl.ready) >= miss.q.seq) {
      fill_missing_x<MT, NF>(ring, a, issued, R, ld, lane, fl, miss);
      landed = issued;
    } else if (issued - landed > D) {
      wait_depth<L>(D);
      landed = issued - D;
    }
    publish_loaded();
    if (!advance<NF>(a, q)) break;
  }
  // Every complete chunk is published before any wait for producer tiles (see above).
  wait_vmcnt<0>();
  landed = issued;
  publish_loaded();
  while (miss.first >= 0) {
    wait_lds(fl.ready, miss.q.seq);
    fill_missing_x<MT, NF>(ring, a, issued, R, ld, lane, fl, miss);
    publish_loaded();
  }
}

// ------------------------------------------------------------------ compute wavefronts

// Byte offset inside an 8-row-group block of the piece lane `lane` feeds to an MFMA operand at
// step u: row lane%16 of the fragment, piece 4u + lane/16.
__device__ __forceinline__ uint32_t operand_offset(int u, int lane) {
  const int r = lane & 15;
  const int p = 4 * u + (lane >> 4);
  return (r >> 3) * 1024 + 128 * (r & 7) + 16 * (p ^ swizzle(r));
}

// Multiplies the chunk in `slot` into acc: this wavefront's 16*NF weight rows by the 16*MT X rows.
template <int DT, int MT, int NF>
__device__ __forceinline__ void mma_chunk(const char* slot, int wave, f32x4 (&acc)[NF][MT], const uint32_t (&op)[kStreamU]) {
  const char* wp = slot + xpart_bytes<MT>() + wave * wpart_bytes<NF>();
#pragma unroll
  for (int u = 0; u < kStreamU; ++u) {
    u32x4 wv[NF], xv[MT];
#pragma unroll
    for (int f = 0; f < NF; ++f) wv[f] = *(const LdsVec*)(wp + f * 2048 + op[u]);
#pragma unroll
    for (int t = 0; t < MT; ++t) xv[t] = *(const LdsVec*)(slot + t * 2048 + op[u]);
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[f][t] = mfma_16x16x32<DT>(wv[f], xv[t], acc[f][t]);
  }
}

// Stores this wavefront's part of the item's tile: fp32 accumulator register r of lane l for
// fragment (f, t) is Y[16t + l%16][r0 + 16*NF*wave + 16f + 4(l/16) + r], four consecutive columns.
// With split > 1 it is the split's fp32 partial instead (planes [split][M][Np], Np = N rounded up
// to 4; each four-column group is one 16-byte device-coherent store).
template <int DT>
__device__ __forceinline__ void store_y4(const plm_chain_gemm& g, int m, int n, int tn_left, f32x4 v, bool coherent);

template <int DT, int MT, int NF>
__device__ __forceinline__ void store_tile(const StreamArgs& a, const Cursor& q, int wave, int lane,
                                           const f32x4 (&acc)[NF][MT]) {
  const plm_chain_gemm g = gemm_at(q.gi);
  const int s = q.item % q.split;
  const int n_base = q.r0 + 16 * NF * wave + 4 * (lane >> 4);
  const bool coherent = g.consumed != 0;
  const int Np = (g.N + 3) & ~3;
  const uint32_t plane = static_cast<uint32_t>(a.M) * Np * 4u;
  const auto prs = make_rsrc(a.partial + g.partial_offset, q.split > 1 ? plane * q.split : 0u);
#pragma unroll
  for (int f = 0; f < NF; ++f)
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = 16 * t + (lane & 15);
      const int n = n_base + 16 * f;
      if (q.split == 1) {
        if (m < a.M && n < g.N) store_y4<DT>(g, m, n, g.N - n, acc[f][t], coherent);
      } else {
        const uint32_t off = (m < a.M && n < g.N) ? s * plane + (static_cast<uint32_t>(m) * Np + n) * 4u : kOutOfRange;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[f][t]), prs, off, 0, kCoherent);
      }
    }
}

template <int DT, int MT, int NF>
__device__ void compute_role(const StreamArgs& a, int wave, int lane, char* lds, const Flags& fl) {
  constexpr size_t SLOT = slot_bytes<MT, NF>();
  const int R = a.ring;
  char* ring = lds;
  const uint32_t op[kStreamU] = {operand_offset(0, lane), operand_offset(1, lane)};
  Cursor q;
  f32x4 acc[NF][MT];
#pragma unroll
  for (int f = 0; f < NF; ++f)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[f][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (!first<NF>(a, q)) return;
  int slot = 0, done = 0;
  // The compute wavefronts issue no memory loads (they only read LDS), so their stores hold
  // nothing up. The epilogue's split-K arrival and tile-done flag need the tile written through,
  // which a wait on this wavefront's stores guarantees; the wait comes a couple of chunks after
  // the stores (`unreported` counts down), when they have long completed, or at once when the
  // next chunk is not in LDS yet: the loader may be waiting for exactly that tile-done flag.
  int unreported = 0;
  for (;;) {
    if (unreported > 0) {
      bool avail = true;
#pragma unroll
      for (int ld = 0; ld < kLoaders; ++ld) avail = avail && lds_uniform(fl.loaded + ld) >= done + 1;
      if (!avail) {
        __builtin_amdgcn_s_waitcnt(0);
        if (lane == 0) lds_count(fl.staged);
        unreported = 0;
      }
    }
#pragma unroll
    for (int ld = 0; ld < kLoaders; ++ld) spin_lds(fl.loaded + ld, done + 1);
    mma_chunk<DT, MT, NF>(ring + slot * SLOT, wave, acc, op);
    // The chunk's LDS reads are complete (the MFMAs consumed them): release the slot.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (lane == 0) lds_count(fl.consumed);
    ++done;
    slot = next_slot(slot, R);
    if (unreported > 0 && (--unreported == 0 || q.c == q.C - 1)) {
      __builtin_amdgcn_s_waitcnt(0);
      if (lane == 0) lds_count(fl.staged);
      unreported = 0;
    }
    if (q.c == q.C - 1) {
      store_tile<DT, MT, NF>(a, q, wave, lane, acc);
#pragma unroll
      for (int f = 0; f < NF; ++f)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[f][t] = f32x4{0.f, 0.f, 0.f, 0.f};
      unreported = 2;
    }
    if (!advance<NF>(a, q)) break;
  }
  if (unreported > 0) {
    __builtin_amdgcn_s_waitcnt(0);
    if (lane == 0) lds_count(fl.staged);
  }
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

// Position of the epilogue wavefront in the workgroup's item sequence (the same sequence the
// compute wavefronts' cursors walk).
struct ItemPos {
  int gi, item;
};

template <int NF>
__device__ __forceinline__ bool item_from(const StreamArgs& a, ItemPos& p, int gi) {
  for (; gi < a.count; ++gi)
    if (static_cast<int>(blockIdx.x) < items_of<NF>(gemm_at(gi))) {
      p.gi = gi;
      p.item = blockIdx.x;
      return true;
    }
  return false;
}

template <int NF>
__device__ __forceinline__ bool item_next(const StreamArgs& a, ItemPos& p) {
  if (p.item + a.G < items_of<NF>(gemm_at(p.gi))) {
    p.item += a.G;
    return true;
  }
  return item_from<NF>(a, p, p.gi + 1);
}

// Whether the producer tiles that item p's X columns come from are all finished (one poll).
template <int NF>
__device__ __forceinline__ bool deps_done(const StreamArgs& a, const ItemPos& p, int epoch, int lane) {
  const plm_chain_gemm g = gemm_at(p.gi);
  if (g.dep < 0) return true;
  constexpr int TN = 64 * NF;
  const plm_chain_gemm pg = gemm_at(g.dep);
  const int s = p.item % g.split_k;
  int lo, hi;
  split_range(g.K, s, g.split_k, lo, hi);
  const int k0 = lo * 32, k1 = min(hi * 32, g.K);
  if (k1 <= k0) return true;
  // X columns [k0, k1) come from the producer's tiles k0/TN .. (k1-1)/TN.
  const int t0 = k0 / TN, t1 = (k1 - 1) / TN;
  const int* done = a.counters + pg.done_base;
  bool ok = true;
  for (int t = t0 + lane; t <= t1; t += 64) ok = ok && collect(done + t) == epoch + 1;
  return __all(ok);
}

// Sums a tile's split partials in split order 0..split-1 and writes Y. Lane layout: four-column
// group lane % GROUPS, row lane / GROUPS + ROWS_PER_PASS * pass. A round loads every split of
// 16 / split passes at once (16 loads in flight); the sum order stays ascending.
template <int DT, int MT, int NF>
__device__ void combine_tile(const StreamArgs& a, const plm_chain_gemm& g, int n0, int tn, int lane) {
  constexpr int TN = 64 * NF;
  constexpr int GROUPS = TN / 4;
  constexpr int ROWS_PER_PASS = 64 / GROUPS;
  constexpr int PASSES = 16 * MT / ROWS_PER_PASS;
  constexpr int SLOTS = 16;  // loads per round
  const int n = 4 * (lane % GROUPS);
  const bool coherent = g.consumed != 0;
  const int Np = (g.N + 3) & ~3;
  const uint32_t plane = static_cast<uint32_t>(a.M) * Np * 4u;
  const auto prs = make_rsrc(a.partial + g.partial_offset, plane * g.split_k);
  const int S = g.split_k;
  if (S <= SLOTS) {
    const int per_round = SLOTS / S;  // passes per round
    for (int p0 = 0; p0 < PASSES; p0 += per_round) {
      u32x4 part[SLOTS];
#pragma unroll
      for (int i = 0; i < SLOTS; ++i) {
        const int b = i / S, q = i - b * S;  // pass p0 + b, split q
        const int m = (p0 + b) * ROWS_PER_PASS + lane / GROUPS;
        const bool ok = b < per_round && p0 + b < PASSES && m < a.M && n < tn;
        part[i] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       prs, ok ? (static_cast<uint32_t>(m) * Np + n0 + n) * 4u + q * plane : kOutOfRange, 0, kCoherent));
      }
      for (int b = 0; b < per_round && p0 + b < PASSES; ++b) {
        const int m = (p0 + b) * ROWS_PER_PASS + lane / GROUPS;
        f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < SLOTS; ++i)
          if (i / S == b) sum += __builtin_bit_cast(f32x4, part[i]);
        if (m < a.M && n < tn) store_y4<DT>(g, m, n0 + n, tn - n, sum, coherent);
      }
    }
  } else {
    for (int p = 0; p < PASSES; ++p) {
      const int m = p * ROWS_PER_PASS + lane / GROUPS;
      const bool ok = m < a.M && n < tn;
      f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int q0 = 0; q0 < S; q0 += SLOTS) {
        u32x4 part[SLOTS];
#pragma unroll
        for (int i = 0; i < SLOTS; ++i)
          part[i] = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         prs, (ok && q0 + i < S) ? (static_cast<uint32_t>(m) * Np + n0 + n) * 4u + (q0 + i) * plane
                                                 : kOutOfRange,
                         0, kCoherent));
#pragma unroll
        for (int i = 0; i < SLOTS; ++i)
          if (q0 + i < S) sum += __builtin_bit_cast(f32x4, part[i]);
      }
      if (ok) store_y4<DT>(g, m, n0 + n, tn - n, sum, coherent);
    }
  }
}

template <int DT, int MT, int NF>
__device__ void epilogue_role(const StreamArgs& a, int lane, char* lds, const Flags& fl) {
  constexpr int TN = 64 * NF;
  (void)lds;
  const int epoch = a.sync ? lane0_broadcast(lane == 0 ? collect(a.counters + kEpochSlot) : 0) : 0;
  ItemPos cur;
  if (item_from<NF>(a, cur, 0)) {
    bounded_wait(a, [&] { return deps_done<NF>(a, cur, epoch, lane); });
    if (lane == 0) *fl.ready = 0;
    ItemPos nxt = cur;
    bool has_next = item_next<NF>(a, nxt);
    for (int seq = 0;; ++seq) {
      // While the compute wavefronts work on item `seq`, see whether the next item's X is ready.
      bool next_ready = !has_next;
      for (;;) {
        if (!next_ready && deps_done<NF>(a, nxt, epoch, lane)) {
          next_ready = true;
          if (lane == 0) *fl.ready = seq + 1;
        }
        if (lds_uniform(fl.staged) >= kStreamKW * (seq + 1)) break;
        __builtin_amdgcn_s_sleep(2);
      }
      const plm_chain_gemm g = gemm_at(cur.gi);
      const int tile = cur.item / g.split_k;
      const int n0 = tile * TN;
      const int tn = min(TN, g.N - n0);
      bool last = true;  // the tile's final values are written
      if (g.split_k > 1) {
        // The compute wavefronts have written this split's partial through. The last of the
        // tile's splits to arrive sums all of them in split order.
        int* counter = a.counters + g.arrive_base + tile;
        int before = 0;
        if (lane == 0) {
          before = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (before == g.split_k - 1) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        before = lane0_broadcast(before);
        last = before == g.split_k - 1;
        if (last) combine_tile<DT, MT, NF>(a, g, n0, tn, lane);
      }
      if (g.consumed && last) {
        __builtin_amdgcn_s_waitcnt(0);  // every store of the tile is written through
        if (lane == 0) publish(a.counters + g.done_base + tile, epoch + 1);
      }
      if (!has_next) break;
      if (!next_ready) {
        bounded_wait(a, [&] { return deps_done<NF>(a, nxt, epoch, lane); });
        if (lane == 0) *fl.ready = seq + 1;
      }
      cur = nxt;
      has_next = item_next<NF>(a, nxt);
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

template <int DT, int MT, int NF>
__global__ __launch_bounds__(64 * kStreamWaves) void stream_gemm_kernel(StreamArgs a) {
  __shared__ int flags[3 + kLoaders];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  {
    // Descriptors into LDS: from the device table for a chain, from the kernel arguments else.
    const int* src = a.chain != nullptr ? reinterpret_cast<const int*>(a.chain) : reinterpret_cast<const int*>(&a.single);
    int* dst = reinterpret_cast<int*>(stream_lds);
    const int words = a.count * static_cast<int>(sizeof(plm_chain_gemm) / sizeof(int));
    for (int i = threadIdx.x; i < words; i += blockDim.x) dst[i] = src[i];
  }
  char* lds = reinterpret_cast<char*>(stream_lds) + table_bytes(a.count);
  if (threadIdx.x == 0) {
    flags[0] = -1;  // ready
    flags[1] = 0;   // staged
    flags[2] = 0;   // consumed
    for (int ld = 0; ld < kLoaders; ++ld) flags[3 + ld] = 0;  // loaded
  }
  __syncthreads();
  const Flags fl{(LdsFlag*)&flags[0], (LdsFlag*)&flags[1], (LdsFlag*)&flags[2], (LdsFlag*)&flags[3]};
  if (wave < kStreamKW)
    compute_role<DT, MT, NF>(a, wave, lane, lds, fl);
  else if (wave < kStreamKW + kLoaders)
    loader_role<MT, NF>(a, wave - kStreamKW, lane, lds, fl);
  else
    epilogue_role<DT, MT, NF>(a, lane, lds, fl);
}

// Compiled tile set: a ring at least two chunks deep beside the largest descriptor table, and at
// most 64 accumulator VGPRs per compute wavefront.
template <int MT, int NF>
constexpr bool stream_compiled() {
  if (MT < 1 || MT > 8) return false;
  if (NF != 1 && NF != 2 && NF != 4) return false;
  if (ring_for_table<MT, NF>(kTableReserve) < 2) return false;
  return NF * MT <= 16;
}

hipError_t stream_dispatch_bf16(StreamArgs& a, int nf, int cus, hipStream_t s, bool dry);
hipError_t stream_dispatch_f16(StreamArgs& a, int nf, int cus, hipStream_t s, bool dry);

// Workgroups of one launch: persistent, at most what fits on the device at once. The ring is as
// deep as the LDS left by the descriptor table allows.
template <int DT, int MT, int NF>
hipError_t stream_launch(StreamArgs& a, int cus, hipStream_t stream, bool dry) {
  if constexpr (!stream_compiled<MT, NF>()) {
    return hipErrorInvalidConfiguration;
  } else {
    if (dry) return hipSuccess;
    auto kern = stream_gemm_kernel<DT, MT, NF>;
    const size_t table = table_bytes(a.count);
    if (table > kTableReserve) return hipErrorInvalidConfiguration;
    a.ring = ring_for_table<MT, NF>(table);
    if (a.ring < 2) return hipErrorInvalidConfiguration;
    const size_t lds = table + static_cast<size_t>(a.ring) * slot_bytes<MT, NF>();
    static bool lds_raised = false;
    if (!lds_raised) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kMaxLdsBytes));
      if (e != hipSuccess) return e;
      lds_raised = true;
    }
    // Workgroups resident per CU at this LDS size (cached for the last size asked).
    static size_t cached_lds = 0;
    static int cached_per_cu = 0;
    if (cached_lds != lds) {
      const int per_cu = resident_per_cu(reinterpret_cast<const void*>(kern), 64 * kStreamWaves, lds);
      if (per_cu < 1) return hipErrorInvalidConfiguration;
      cached_lds = lds;
      cached_per_cu = per_cu;
    }
    // a.G arrives as the most items any linear has; a chained launch needs every workgroup
    // resident at once (they wait on each other), a single linear needs no more than its items.
    const int resident = cus * cached_per_cu;
    a.G = a.sync ? resident : min(resident, a.G);
    hipLaunchKernelGGL(kern, dim3(a.G), dim3(64 * kStreamWaves), lds, stream, a);
    return hipGetLastError();
  }
}

template <int DT, int MT>
hipError_t stream_pick(StreamArgs& a, int nf, int cus, hipStream_t s, bool dry) {
  if (nf == 1) return stream_launch<DT, MT, 1>(a, cus, s, dry);
  if (nf == 2) return stream_launch<DT, MT, 2>(a, cus, s, dry);
  if (nf == 4) return stream_launch<DT, MT, 4>(a, cus, s, dry);
  return hipErrorInvalidConfiguration;
}

template <int DT>
hipError_t stream_dispatch(StreamArgs& a, int nf, int cus, hipStream_t s, bool dry) {
  switch ((a.M + 15) / 16) {
    case 1: return stream_pick<DT, 1>(a, nf, cus, s, dry);
    case 2: return stream_pick<DT, 2>(a, nf, cus, s, dry);
    case 3: return stream_pick<DT, 3>(a, nf, cus, s, dry);
    case 4: return stream_pick<DT, 4>(a, nf, cus, s, dry);
    case 5: return stream_pick<DT, 5>(a, nf, cus, s, dry);
    case 6: return stream_pick<DT, 6>(a, nf, cus, s, dry);
    case 7: return stream_pick<DT, 7>(a, nf, cus, s, dry);
    case 8: return stream_pick<DT, 8>(a, nf, cus, s, dry);
  }
  return hipErrorInvalidConfiguration;
}

}  // namespace plm
