// Skinny GEMM over pre-packed weights for the PLM round's dense linears on gfx950 (MI355X).
//
// Y[M,N] = X[M,K] · W[N,K]^T with fp32 accumulation, for one linear or for a chain of linears in
// one launch (the round's linears back to back, a later one reading an earlier one's Y). M is the
// round width (56 at k=7), so W is almost all of the bytes and the kernel is an HBM stream of W.
//
// Packed weights. v_mfma_f32_16x16x32_{bf16,f16} takes its A operand as lane l = row l%16, K
// elements [8*(l/16), 8*(l/16)+8) of a 32-wide K step: 16 bytes per lane from 16 different rows.
// Loaded from a row-major W, every quad of lanes touches four rows, so one load instruction is
// 64 separate cache-line requests and the vector memory pipeline, not HBM, sets the speed. The
// weights are therefore rearranged once (plm_pack_weight) into fragments: fragment (f, s) is rows
// [16f, 16f+16) x K [32s, 32s+32) stored as 64 lanes x 16 bytes in exactly that lane order, in
// groups of eight K steps per row (tile.h: pack_row_offset, pack_step_offset). Every weight load
// is then one contiguous, aligned KiB that lands in the registers as the MFMA operand, with no LDS
// staging.
// X (small, L2-resident) is loaded row-major and coalesced, and turned into the operand layout
// through a wavefront-private LDS tile.
//
// Work: item = a tile x one of `split` K ranges. Workgroups are persistent and take items
// blockIdx.x, blockIdx.x + G, ... of each linear in turn. Two workgroup layouts (KW):
//   * KW = 4: a tile is NF fragments (16*NF weight rows); each of the 4 wavefronts owns a quarter
//     of the item's K range, and at the item's end the four partial tiles are summed in LDS in
//     wavefront order (the verify kernel's K partition, so its logits can be reproduced).
//   * KW = 1: a tile is 4*NF fragments; each wavefront owns NF of them over the item's whole K
//     range, and the workgroup shares one copy of X: per K step each wavefront loads a quarter of
//     the X fragments, writes them into a double-buffered LDS tile, and after a barrier reads all
//     of them. Four times fewer X loads per weight byte: the vector-memory pipeline, not HBM, is
//     what a wavefront's load rate runs into (about one KiB load per 60 ns per wavefront).
// Each wavefront streams its weight (and X) fragments through a D-stage register pipeline that
// runs across the linear's item boundaries. With split > 1 a tile's result is an fp32 partial and
// the last workgroup of the tile to arrive (device-scope counter) adds the partials in split
// order and writes Y.
//
// Chains: after a linear whose Y a later linear reads, every workgroup writes its part of Y
// through to the device-coherent level and then raises its own progress flag (one 64-bit word per
// workgroup: launch epoch and the number of such linears it has finished, so flags only grow and
// need no reset). It requests the next linear's first weight fragments, so the weight stream
// overlaps the wait, and then polls every workgroup's flag until all have finished the linear: a
// grid barrier made of plain stores and loads, with no contended atomic. The last workgroup to
// finish a chained launch advances the epoch (chain_exit). All workgroups of a chained launch are resident
// at once; every wait is bounded and sets the error flag if it gives up.
//
// Results are bitwise reproducible run to run: every sum has a fixed order (K steps ascending
// within a wavefront, wavefronts 0..3, splits 0..split-1).
#pragma once

#include <hip/hip_runtime.h>

#include "plm_amd.h"
#include "tile.h"

namespace plm {

constexpr int kPackedWaves = 4;            // wavefronts per workgroup of the row-split layout (KW = 1)
constexpr int kFragBytes = 1024;           // one packed fragment: 64 lanes x 16 bytes
constexpr uint32_t kNoLoad = 0x80000000u;  // scalar offset that puts a load out of range (zeros)
constexpr int kXTileBytes = 16 * 80;       // LDS transpose tile of one X fragment (16 rows of up to 80 B)

// Where a lane writes and reads its 16 bytes of an X transpose tile. A fragment row holds 32 K
// values (64 B, four 16-byte chunks); lane l writes chunk l % 4 of row l / 4 (its X load) and reads
// chunk l / 16 of row l % 16 (the MFMA operand). Swizzled: rows 64 B apart, chunk c of row r at slot
// c ^ ((r >> 2) & 3), so the 16 lanes of an LDS cycle hit 16 different bank groups in both
// directions. Padded: rows 80 B apart, reads conflict-free but writes two-way (kept where the
// swizzled offsets would cost registers the kernel does not have).
template <bool kSwizzle>
__device__ __forceinline__ int x_tile_write_offset(int lane) {
  return kSwizzle ? (lane >> 2) * 64 + (((lane & 3) ^ ((lane >> 4) & 3)) * 16) : (lane >> 2) * 80 + (lane & 3) * 16;
}
template <bool kSwizzle>
__device__ __forceinline__ int x_tile_read_offset(int lane) {
  return kSwizzle ? (lane & 15) * 64 + (((lane >> 4) ^ ((lane >> 2) & 3)) * 16) : (lane & 15) * 80 + (lane >> 4) * 16;
}

// Counter-area layout of a packed launch (int indices).
constexpr int kPkErrorSlot = 2;      // 1 once a bounded wait gave up
constexpr int kPkEpochSlot = 10;     // int64 at ints 10-11: packed chained launches completed
constexpr int kPkMaxWorkgroups = 2048;  // progress flags: int64 per workgroup at kPackedBarrierBase
// Tile-flag mode uses the same 2048 int64 as two parity sets of tile-done flags: consumed linear
// number q (1, 2, ...) raises flag (q & 1) * kPkTileFlags + tile to ((epoch + 1) << 16) + q once
// the tile's Y is written. In a chain where every linear reads the one before it, a set is only
// rewritten (by linear q + 2) after every tile of linear q that a later linear reads is done,
// and values only grow, so no flag needs clearing.
constexpr int kPkTileFlags = 1024;
constexpr int kPkLoraHDone = 12;   // gated-LoRA launch: tiles of h written
constexpr int kPkLoraPast = 13;    // gated-LoRA launch: base tiles past their wait for h
constexpr int kPkExitSlot = 14;    // chained launch: workgroups that have finished it

// Gated low-rank correction inside one launch (plm_gemm_packed_lora, plm/gated_lora.py:45-57):
// linear 0 forms h = X A^T in the model dtype for every row (each tile counts itself in once
// written), linear 1 is the base linear, whose tiles wait for every h tile and then store rows
// m >= gated_from as round(round(acc) + sum_j h[m, s*rank + j] * B[n, j]), s the shard of column
// n: the reference's base output and one addmm_ per shard. The last base tile to pass its wait
// resets both counters for the next launch.
// Store epilogues of packed_gemm_kernel (its EPI template parameter).
constexpr int kEpiPlain = 0;  // Y = X W^T
constexpr int kEpiLora = 1;   // the gated-LoRA launch (PackedLora)
constexpr int kEpiAct = 2;    // a fused gate/up projection's SiLU-and-multiply (act_store)

struct PackedLora {
  plm_chain_gemm pre;   // the h linear (y = h, ldy = its row stride)
  const uint16_t* b;    // [N][rank], the shards' up-projections stacked by output column
  int rank, gated_from;
  int shard_end[3];     // exclusive column ends of the first three shards (N past the last)
  int h_tiles, base_tiles;
  int h_items;          // the base linear's items start at workgroup h_items (mod the grid)
};

struct PackedArgs {
  const plm_chain_gemm* chain;  // device array of `count` linears, or nullptr: use `single`
  plm_chain_gemm single;
  int count;
  int M;
  int G;           // workgroups in the grid
  int sync;        // 0: no linear reads another's output; 1: grid barriers after such linears
                   // (progress flags); 2: tile flags (every linear after the first reads the one
                   // before it: each wavefront waits only for the producer tiles it reads)
  int spin_limit;  // polls before a wait gives up
  int* counters;
  float* partial;
  PackedLora lora;  // packed_gemm_kernel<..., EPI = kEpiLora> only
};

__device__ __forceinline__ int sgpr(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int64_t sgpr64(int64_t v) {
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v >> 32)));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}
template <typename T>
__device__ __forceinline__ T* sgpr_ptr(T* p) {
  return reinterpret_cast<T*>(sgpr64(reinterpret_cast<int64_t>(p)));
}

// One linear as the kernel uses it (all wave-uniform).
struct PLinear {
  const void* x;
  const void* wp;
  void* y;
  int64_t ldx, ldy;
  int N, Ks, k_last, split, tiles, items;  // tiles of 16*NF (KW = 4) or 64*NF (KW = 1) rows
  uint32_t wgroup;  // packed weight: bytes from one group of K steps to the next (pack_group_bytes)
  int out_f32, consumed;
  int* arrive;     // split arrival counters, one per tile
  int seq;         // consumed linears up to and including this one
  float* partial;  // split partials
  int64_t* flag;   // sync == 2 and consumed: this linear's tile-done flags (else nullptr)
  int64_t flag_value;  // the value they get: ((epoch + 1) << 16) + seq
  int role;        // gated-LoRA launch: 1 the h linear, 2 the corrected base linear; else 0
};

// Wavefronts per workgroup: KW for the K-split layouts, four for the row-split one.
template <int KW>
constexpr int packed_waves() {
  return KW == 1 ? kPackedWaves : KW;
}

// Weight fragments of a tile.
template <int NF, int KW>
constexpr int tile_frags() {
  return KW == 1 ? kPackedWaves * NF : NF;
}

// A load through the constant address space: the chain table does not change while the kernel
// runs, so its fields can be fetched with scalar loads.
template <typename T>
__device__ __forceinline__ T const_load(const T* p) {
  return *((const __attribute__((address_space(4))) T*)p);
}

// A linear's descriptor: a chain's from its table, a single linear's from the kernel arguments
// (a gated-LoRA launch: linear 0 is the h linear, linear 1 the base).
template <int NF, int KW, int EPI = kEpiPlain>
__device__ __forceinline__ PLinear load_linear(const PackedArgs& a, int gi, int64_t epoch = 0) {
  plm_chain_gemm g = a.single;
  if constexpr (EPI == kEpiLora) {
    if (gi == 0) g = a.lora.pre;
  } else if (a.chain != nullptr) {
    const plm_chain_gemm* c = a.chain + gi;
    g.x = const_load(&c->x);
    g.w = const_load(&c->w);
    g.y = const_load(&c->y);
    g.ldx = const_load(&c->ldx);
    g.ldy = const_load(&c->ldy);
    g.N = const_load(&c->N);
    g.K = const_load(&c->K);
    g.split_k = const_load(&c->split_k);
    g.out_f32 = const_load(&c->out_f32);
    g.consumed = const_load(&c->consumed);
    g.arrive_base = const_load(&c->arrive_base);
    g.done_base = const_load(&c->done_base);
    g.partial_offset = const_load(&c->partial_offset);
  }
  PLinear L;
  L.x = sgpr_ptr(g.x);
  L.wp = sgpr_ptr(g.w);
  L.y = sgpr_ptr(g.y);
  L.ldx = sgpr64(g.ldx);
  L.ldy = sgpr64(g.ldy);
  L.N = sgpr(g.N);
  const int K = sgpr(g.K);
  L.Ks = (K + 31) >> 5;
  L.k_last = K - 32 * (L.Ks - 1);
  L.split = sgpr(g.split_k);
  L.wgroup = pack_group_bytes(L.N);
  L.tiles = (((L.N + 15) >> 4) + tile_frags<NF, KW>() - 1) / tile_frags<NF, KW>();
  L.items = L.tiles * L.split;
  L.out_f32 = sgpr(g.out_f32);
  L.consumed = sgpr(g.consumed);
  L.arrive = a.counters + sgpr(g.arrive_base);
  L.seq = sgpr(g.done_base);
  L.partial = a.partial + sgpr64(g.partial_offset);
  L.flag = (a.sync == 2 && L.consumed)
               ? reinterpret_cast<int64_t*>(a.counters + kPackedBarrierBase) + (L.seq & 1) * kPkTileFlags
               : nullptr;
  L.flag_value = ((epoch + 1) << 16) + L.seq;
  L.role = EPI == kEpiLora ? (gi == 0 ? 1 : 2) : 0;
  return L;
}

// The first item of linear gi this workgroup takes (then every G-th): the gated-LoRA launch gives
// the h linear's items to workgroups 0, 1, ... and starts the base linear's after them.
template <int EPI>
__device__ __forceinline__ int first_item(const PackedArgs& a, int gi) {
  if constexpr (EPI == kEpiLora) {
    if (gi == 1) return sgpr((static_cast<int>(blockIdx.x) + a.G - a.lora.h_items % a.G) % a.G);
  }
  return static_cast<int>(blockIdx.x);
}

// Whether an earlier bounded wait of this launch (or of an earlier launch whose flag nobody
// cleared) gave up. Every wait checks it on entry and every kErrorCheckPolls polls, so once one wait
// times out the rest of the chain drains at once instead of each link spinning its own limit.
constexpr int kErrorCheckPolls = 256;
__device__ __forceinline__ bool chain_failed(const PackedArgs& a) {
  return __builtin_amdgcn_readfirstlane(collect(a.counters + kPkErrorSlot)) != 0;
}

// sync == 2: raises the tile-done flag of `tile` once every wavefront's stores of it have
// completed (device-coherent Y stores: visible to every workgroup once complete). An atomic
// maximum: a tile of linear q that no later linear reads may finish after linear q + 2 has
// raised the same flag, and must not lower it.
__device__ __forceinline__ void publish_tile(const PLinear& L, int tile) {
  if (L.flag == nullptr) return;
  __builtin_amdgcn_s_waitcnt(0);
  asm volatile("s_barrier" ::: "memory");
  if (threadIdx.x == 0)
    __hip_atomic_fetch_max(L.flag + tile, L.flag_value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// K-step range [b, e) of split s: wavefront w's share of it (K-split layouts: 1/KW) or all of it
// (KW = 1).
// 32-bit unsigned arithmetic (K <= 2^24, split <= 64), without a division when split == 1 and
// with shifts for the power-of-two KW: this runs once per item and is on the critical path.
template <int KW>
__device__ __forceinline__ void packed_range(int Ks, int s, int split, int w, int& b, int& e) {
  int lo = 0, hi = Ks;
  if (split != 1) {
    lo = static_cast<int>(static_cast<uint32_t>(s * Ks) / static_cast<uint32_t>(split));
    hi = static_cast<int>(static_cast<uint32_t>((s + 1) * Ks) / static_cast<uint32_t>(split));
  }
  if constexpr (KW == 1) {
    b = lo;
    e = hi;
  } else {
    const uint32_t n = static_cast<uint32_t>(hi - lo);
    b = lo + static_cast<int>(n * static_cast<uint32_t>(w) / KW);
    e = lo + static_cast<int>(n * static_cast<uint32_t>(w + 1) / KW);
  }
}

// Item -> (tile, split index), without a division when split == 1.
__device__ __forceinline__ void item_tile(int item, int split, int& tile, int& s) {
  if (split == 1) {
    tile = item;
    s = 0;
  } else {
    tile = static_cast<int>(static_cast<uint32_t>(item) / static_cast<uint32_t>(split));
    s = item - tile * split;
  }
}

// A wavefront's position in its stream of (item, K step). A wavefront's steps of an item are
// padded with all-zero steps (out-of-range loads) to a multiple of the pipeline depth D, at least
// D: item boundaries then always fall on pipeline stage 0, so the end-of-item work sits outside
// the unrolled stages and the compiler's load-count waits stay exact across items.
struct PCursor {
  int item;   // >= items once past the linear's last item of this workgroup
  int st;     // current K step
  int end;    // end of the steps that load data
  int pend;   // end of the padded steps
  uint32_t wbase;  // byte offset of the item's first weight fragment at step 0
};

template <int NF, int D, int KW>
__device__ __forceinline__ void pc_enter(const PLinear& L, int wave, PCursor& c) {
  if (c.item >= L.items) return;
  int tile, s;
  item_tile(c.item, L.split, tile, s);
  int b, e;
  packed_range<KW>(L.Ks, s, L.split, wave, b, e);
  c.st = b;
  c.end = e;
  c.pend = b + max(D, (e - b + D - 1) / D * D);
  c.wbase = pack_row_offset(tile * tile_frags<NF, KW>() + (KW == 1 ? wave * NF : 0));
}

template <int NF, int D, int KW>
__device__ __forceinline__ void pc_advance(const PLinear& L, int G, int wave, PCursor& c) {
  if (++c.st == c.pend) {
    c.item += G;
    pc_enter<NF, D, KW>(L, wave, c);
  }
}

__device__ __forceinline__ void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// X fragments a wavefront loads per K step: all MT (KW = 4), or fragments wave, wave + 4, ...
// (KW = 1: the workgroup's four wavefronts load one copy between them).
template <int MT, int KW>
constexpr int x_per_wave() {
  return KW == 1 ? (MT + 3) / 4 : MT;
}

// Per-lane operand offsets of one linear.
template <int MT, int NF, int XN>
struct POffsets {
  uint32_t wo[NF];       // weight fragment f at step 0 (plus the item's wbase, the step's KiB)
  uint32_t xo[XN];       // coalesced X: row 16t + lane/4, bytes 16*(lane%4) of the step's 64
  uint32_t xo_last[XN];  // the same with lanes past K (last step) out of range
};

template <int MT, int NF, int KW>
__device__ __forceinline__ void packed_offsets(const PLinear& L, int M, int lane, int wave,
                                               POffsets<MT, NF, x_per_wave<MT, KW>()>& o) {
#pragma unroll
  for (int f = 0; f < NF; ++f) o.wo[f] = pack_row_offset(f) + static_cast<uint32_t>(lane * 16);
#pragma unroll
  for (int i = 0; i < x_per_wave<MT, KW>(); ++i) {
    const int t = KW == 1 ? wave + 4 * i : i;
    const int m = 16 * t + (lane >> 2);
    o.xo[i] = (t < MT && m < M) ? static_cast<uint32_t>(m * L.ldx * 2 + (lane & 3) * 16) : kOutOfRange;
    o.xo_last[i] = 8 * (lane & 3) < L.k_last ? o.xo[i] : kOutOfRange;
  }
}

// Loads the weight half of one pipeline stage (the cursor's K step). The cursor is the same in
// every lane of a wavefront; its offset goes to the load's scalar operand through readfirstlane,
// so that the compiler, which cannot always prove the cursor uniform, does not wrap each load in a
// loop over the lanes' distinct values (such loops also leave its load-count waits conservative:
// a full drain of the pipeline once per D steps).
template <int NF>
__device__ __forceinline__ void issue_w(__amdgpu_buffer_rsrc_t wr, const PCursor& c, int items, uint32_t wgroup,
                                        const uint32_t (&wo)[NF], u32x4 (&wb)[NF]) {
  const bool live = c.item < items && c.st < c.end;
  const int ws = __builtin_amdgcn_readfirstlane(
      static_cast<int>(live ? c.wbase + pack_step_offset(c.st, wgroup) : kNoLoad));
#pragma unroll
  for (int f = 0; f < NF; ++f)
    wb[f] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, wo[f], ws, 0));
}

// Loads the X half of one pipeline stage. X lanes past K in the last step load zeros (the packed
// weights are zero there, but X past K is another row's data or padding, and 0 * NaN is NaN).
template <int MT, int NF, int XN>
__device__ __forceinline__ void issue_x(__amdgpu_buffer_rsrc_t xr, const PCursor& c, int items, int Ks,
                                        const POffsets<MT, NF, XN>& o, u32x4 (&xb)[XN]) {
  const bool live = c.item < items && c.st < c.end;
  const int xs = __builtin_amdgcn_readfirstlane(static_cast<int>(live ? static_cast<uint32_t>(c.st * 64) : kNoLoad));
  const bool last = c.st == Ks - 1;
#pragma unroll
  for (int t = 0; t < XN; ++t)
    xb[t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, last ? o.xo_last[t] : o.xo[t], xs, 0));
}

// Whether X is loaded and staged for two K steps at a time: always in the row split (KW = 1, one
// barrier per pair), and with eight wavefronts at widths of four to seven X fragments (two private
// X tile sets per wavefront fit the LDS up to seven). A pair's two loads read the two halves of the
// same 128-byte lines of X. Measured on the 1.3B round: at M = 56 the chained round 1049 -> 1027 us
// and the per-GEMM round 1291 -> 1237 us; at M <= 42 (fewer X fragments per weight fragment) the
// chained round lost 1-11 %, so narrower widths stage one step at a time.
template <int MT, int KW>
constexpr bool packed_pair_x() {
  if constexpr (KW == 1) return true;
  if constexpr (KW == 8) return MT >= 4 && static_cast<size_t>(2) * KW * MT * kXTileBytes + kFragBytes <= 160 * 1024;
  return false;
}

// The X loads of pipeline stage j, at the cursor's K step. Paired (packed_pair_x): the X of two
// steps is loaded at the even stage, right behind that stage's weights and ahead of the odd
// stage's (the next step lies in the same item: items start at stage 0 and pad to a multiple of
// the even D), so that the even stage finds both steps' X arrived and stages them together.
template <int MT, int NF, int XN, int KW, int D>
__device__ __forceinline__ void issue_x_stage(int j, __amdgpu_buffer_rsrc_t xr, const PCursor& c, int items, int Ks,
                                              const POffsets<MT, NF, XN>& o, u32x4 (&xb)[D][XN]) {
  if constexpr (!packed_pair_x<MT, KW>()) {
    issue_x<MT, NF, XN>(xr, c, items, Ks, o, xb[j]);
  } else if ((j & 1) == 0) {
    issue_x<MT, NF, XN>(xr, c, items, Ks, o, xb[j]);
    PCursor n = c;
    ++n.st;
    issue_x<MT, NF, XN>(xr, n, items, Ks, o, xb[j + 1]);
  }
}

// Row split (KW = 1): the workgroup's shared X tiles of stage j into the MFMA operand layout. The
// even stage of a pair stores both steps' tile sets and meets the barrier; the odd stage reads its
// set without one. Four tile sets: consecutive pairs use alternate halves (`half` flips per pair),
// so a pair's stores never meet a slower wavefront still reading the pair before: it read those
// before it reached the barrier in between.
template <int MT, int XN, int D>
__device__ __forceinline__ void stage_x_rows(int j, char* xt, int wave, int xt_write, int xt_read,
                                             const u32x4 (&xb)[D][XN], u32x4 (&xop)[MT], int& half) {
  const int h = D % 4 == 0 ? (j >> 1) & 1 : half;  // D % 4 == 0: a D-stage block holds whole pairs of pairs
  char* xs = xt + (2 * h + (j & 1)) * MT * kXTileBytes;
  if ((j & 1) == 0) {
#pragma unroll
    for (int i = 0; i < XN; ++i)
      if (wave + 4 * i < MT) {
        *reinterpret_cast<u32x4*>(xs + (wave + 4 * i) * kXTileBytes + xt_write) = xb[j][i];
        *reinterpret_cast<u32x4*>(xs + (MT + wave + 4 * i) * kXTileBytes + xt_write) = xb[j + 1][i];
      }
    lds_sync();
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) xop[t] = *reinterpret_cast<const u32x4*>(xs + t * kXTileBytes + xt_read);
  if (D % 4 != 0 && (j & 1) == 1) half ^= 1;
}

// Four columns n..n+3 of Y row m (fewer at N's end); written through to the device-coherent level
// when a later linear of the chain reads this Y.
template <int DT>
__device__ __forceinline__ void packed_store4(const PLinear& L, int m, int n, f32x4 v) {
  const int left = L.N - n;
  if (L.out_f32 == PLM_OUT_F32) {
    float* y = static_cast<float*>(L.y) + static_cast<int64_t>(m) * L.ldy + n;
    if (left >= 4 && (reinterpret_cast<uintptr_t>(y) & 15) == 0) {
      *reinterpret_cast<f32x4*>(y) = v;
    } else {
      for (int j = 0; j < 4 && j < left; ++j) y[j] = v[j];
    }
    return;
  }
  uint16_t* y = static_cast<uint16_t*>(L.y) + static_cast<int64_t>(m) * L.ldy + n;
  const uint16_t h0 = to_bits16<DT>(v[0]), h1 = to_bits16<DT>(v[1]), h2 = to_bits16<DT>(v[2]), h3 = to_bits16<DT>(v[3]);
  if (left >= 4 && (reinterpret_cast<uintptr_t>(y) & 7) == 0) {
    const uint64_t bits = (static_cast<uint64_t>(h0) | (static_cast<uint64_t>(h1) << 16)) |
                          ((static_cast<uint64_t>(h2) | (static_cast<uint64_t>(h3) << 16)) << 32);
    if (L.consumed)
      publish(reinterpret_cast<uint64_t*>(y), bits);
    else
      *reinterpret_cast<uint64_t*>(y) = bits;
  } else {
    const uint16_t h[4] = {h0, h1, h2, h3};
    for (int j = 0; j < 4 && j < left; ++j) {
      if (L.consumed)
        publish(y + j, h[j]);
      else
        y[j] = h[j];
    }
  }
}

// Gated LoRA, base tile: a first read of the h counter, issued when the tile's K steps end so that
// it arrives while the tile's sums are formed (and, with split > 1, exchanged).
__device__ __forceinline__ int lora_probe(const PackedArgs& a) { return collect(a.counters + kPkLoraHDone); }

// Gated LoRA, base tile: every wavefront waits (bounded) until every h tile is written, polling
// only if the early read was short.
__device__ __forceinline__ void lora_wait_h(const PackedArgs& a, int lane, int probe) {
  if (__builtin_amdgcn_readfirstlane(probe) >= a.lora.h_tiles || chain_failed(a)) return;
  for (int i = 0;; ++i) {
    if (__builtin_amdgcn_readfirstlane(collect(a.counters + kPkLoraHDone)) >= a.lora.h_tiles) return;
    if (i >= a.spin_limit) {
      if (lane == 0) publish(a.counters + kPkErrorSlot, 1);
      return;
    }
    if (i % kErrorCheckPolls == kErrorCheckPolls - 1 && chain_failed(a)) return;
    __builtin_amdgcn_s_sleep(1);
  }
}

// Eight products of 16-bit pairs added to acc in order.
template <int DT>
__device__ __forceinline__ float lora_dot8(u32x4 a, u32x4 b, float acc) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    acc += from_bits16<DT>(static_cast<uint16_t>(a[w] & 0xffffu)) * from_bits16<DT>(static_cast<uint16_t>(b[w] & 0xffffu));
    acc += from_bits16<DT>(static_cast<uint16_t>(a[w] >> 16)) * from_bits16<DT>(static_cast<uint16_t>(b[w] >> 16));
  }
  return acc;
}

// Gated LoRA: rows n..n+3 of gated column m, the base values rounded to the model dtype plus their
// correction (h read device-coherently: other workgroups wrote it). Per group of eight rank
// elements, the four rows' h and B loads are all issued before any is used; rows at or past N load
// zeros and are not stored.
template <int DT>
__device__ __forceinline__ f32x4 lora_correct(const PackedLora& z, int N, int M, int m, int n, f32x4 v) {
  const auto hr = make_rsrc(z.pre.y, static_cast<uint32_t>(M * z.pre.ldy * 2));
  const auto brs = make_rsrc(z.b, static_cast<uint32_t>(N * z.rank * 2));
  const uint32_t hrow = static_cast<uint32_t>(m * z.pre.ldy * 2);
  uint32_t ho[4], bo[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int c = n + r;
    const int s = (c >= z.shard_end[0]) + (c >= z.shard_end[1]) + (c >= z.shard_end[2]);
    ho[r] = c < N ? hrow + static_cast<uint32_t>(s * z.rank * 2) : kOutOfRange;
    bo[r] = c < N ? static_cast<uint32_t>(c * z.rank * 2) : kOutOfRange;
  }
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < z.rank / 8; ++j) {
    u32x4 hv[4], bv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      hv[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(hr, static_cast<int>(ho[r] + 16u * j), 0, kCoherent));
      bv[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(brs, static_cast<int>(bo[r] + 16u * j), 0, 0));
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = lora_dot8<DT>(hv[r], bv[r], acc[r]);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) v[r] = from_bits16<DT>(to_bits16<DT>(v[r])) + acc[r];
  return v;
}

// Fragment q = f*MT + t of a tile, as lane `lane` holds it: rows n0 + 16f + 4*(lane/16) + r
// (r = 0..3) of column m = 16t + lane%16.
template <int DT, int MT, int EPI>
__device__ __forceinline__ void packed_store_frag(const PackedArgs& a, const PLinear& L, int M, int n0, int q, int lane,
                                                  f32x4 v) {
  const int f = q / MT, t = q - f * MT;
  const int m = 16 * t + (lane & 15);
  const int n = n0 + 16 * f + 4 * (lane >> 4);
  if (m >= M || n >= L.N) return;
  if constexpr (EPI == kEpiLora) {
    if (L.role == 2 && m >= a.lora.gated_from) v = lora_correct<DT>(a.lora, L.N, M, m, n, v);
  }
  packed_store4<DT>(L, m, n, v);
}

// A tile's Y is stored: raises its tile-done flag (sync == 2), or in a gated-LoRA launch counts an
// h tile in (once every wavefront's stores of it have completed), or counts a base tile past its
// wait for h; the last base tile of the launch resets both counters for the next launch.
template <int EPI>
__device__ __forceinline__ void tile_done(const PackedArgs& a, const PLinear& L, int tile) {
  if constexpr (EPI == kEpiLora) {
    if (L.role == 1) __builtin_amdgcn_s_waitcnt(0);
    asm volatile("s_barrier" ::: "memory");
    if (threadIdx.x == 0) {
      if (L.role == 1) {
        __hip_atomic_fetch_add(a.counters + kPkLoraHDone, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else if (__hip_atomic_fetch_add(a.counters + kPkLoraPast, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 a.lora.base_tiles - 1) {
        publish(a.counters + kPkLoraHDone, 0);
        publish(a.counters + kPkLoraPast, 0);
      }
    }
  } else {
    publish_tile(L, tile);
  }
}

// SiLU-and-multiply epilogue (kEpiAct) of a fused gate/up projection packed with its gate and up
// rows interleaved by fragment: fragment 2j holds gate rows [16j, 16j+16) and fragment 2j+1 the
// up rows [16j, 16j+16) of the same output columns. Column block `cblk` (16 columns of the [M, N/2]
// output) of X row 16t + lane%16, columns 16*cblk + 4*(lane/16) + r: the gate and up values rounded
// to the model dtype (the projection's output), then vLLM's SiluAndMul on them (its silu_and_mul
// kernel, which the rounds run with enforce_eager): silu(g) = g / (1 + e^-g) in fp32 rounded to the
// model dtype, times u, rounded again (the product of two 16-bit values is exact in fp32).
template <int DT, int MT>
__device__ __forceinline__ void act_store(const PLinear& L, int M, int cblk, int t, int lane, f32x4 g, f32x4 u) {
  const int m = 16 * t + (lane & 15);
  const int n = 16 * cblk + 4 * (lane >> 4);
  if (m >= M || n >= (L.N >> 1)) return;  // N/2 is a multiple of 16: all four columns are in range
  uint16_t h[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float gr = from_bits16<DT>(to_bits16<DT>(g[r])), ur = from_bits16<DT>(to_bits16<DT>(u[r]));
    h[r] = to_bits16<DT>(from_bits16<DT>(to_bits16<DT>(gr / (1.0f + expf(-gr)))) * ur);
  }
  uint64_t* y = reinterpret_cast<uint64_t*>(static_cast<uint16_t*>(L.y) + static_cast<int64_t>(m) * L.ldy + n);
  const uint64_t bits = (static_cast<uint64_t>(h[0]) | (static_cast<uint64_t>(h[1]) << 16)) |
                        ((static_cast<uint64_t>(h[2]) | (static_cast<uint64_t>(h[3]) << 16)) << 32);
  if (L.consumed)
    publish(y, bits);  // a later linear of the chain reads it
  else
    *y = bits;
}

// kEpiAct end of an item for a K-split workgroup (the wavefronts' tiles already in LDS): each
// wavefront takes fragment pairs (gate, up) of the tile, sums both over the KW wavefronts, and
// stores the activation, or with split > 1 writes the two partials; the last split to arrive sums
// each pair's partials in split order and stores the activation.
template <int DT, int MT, int NF, int KW>
__device__ __forceinline__ void packed_finish_act(const PackedArgs& a, const PLinear& L, int M, int tile, int s,
                                                  int wave, int lane, const f32x4* red, int* last_flag) {
  constexpr int Q = NF * MT, QP = Q / 2, I = (QP + KW - 1) / KW;
  f32x4 g[I], u[I];
#pragma unroll
  for (int i = 0; i < I; ++i) {
    const int p = wave + KW * i;
    if (p < QP) {
      const int j = p / MT, t = p - j * MT, qg = 2 * j * MT + t, qu = qg + MT;
      f32x4 vg = red[qg * 64 + lane], vu = red[qu * 64 + lane];
#pragma unroll
      for (int w = 1; w < KW; ++w) {
        vg += red[(w * Q + qg) * 64 + lane];
        vu += red[(w * Q + qu) * 64 + lane];
      }
      g[i] = vg;
      u[i] = vu;
    }
  }
  lds_sync();  // every wavefront has read the tiles; LDS is free for the next item
  if (L.split == 1) {
#pragma unroll
    for (int i = 0; i < I; ++i) {
      const int p = wave + KW * i;
      if (p < QP) {
        const int j = p / MT, t = p - j * MT;
        act_store<DT, MT>(L, M, tile * (NF / 2) + j, t, lane, g[i], u[i]);
      }
    }
    tile_done<kEpiAct>(a, L, tile);
    return;
  }
  const uint32_t tile_bytes = static_cast<uint32_t>(L.split) * Q * kFragBytes;
  const auto prs = make_rsrc(L.partial + static_cast<int64_t>(tile) * L.split * Q * 256, tile_bytes);
#pragma unroll
  for (int i = 0; i < I; ++i) {
    const int p = wave + KW * i;
    if (p < QP) {
      const int j = p / MT, t = p - j * MT, qg = 2 * j * MT + t, qu = qg + MT;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, g[i]), prs,
                                             static_cast<uint32_t>((s * Q + qg) * kFragBytes + lane * 16), 0, kCoherent);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, u[i]), prs,
                                             static_cast<uint32_t>((s * Q + qu) * kFragBytes + lane * 16), 0, kCoherent);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this wavefront's partials are written through
  lds_sync();
  if (threadIdx.x == 0) {
    int* counter = L.arrive + tile;
    const int before = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = before == L.split - 1;
    if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *last_flag = last;
  }
  lds_sync();
  if (*last_flag == 0) return;
#pragma unroll 1
  for (int i = 0; i < I; ++i) {
    const int p = wave + KW * i;
    if (p < QP) {
      const int j = p / MT, t = p - j * MT, qg = 2 * j * MT + t, qu = qg + MT;
      f32x4 vg = f32x4{0.f, 0.f, 0.f, 0.f}, vu = vg;
      for (int s0 = 0; s0 < L.split; ++s0) {
        vg += __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            prs, static_cast<uint32_t>((s0 * Q + qg) * kFragBytes + lane * 16), 0, kCoherent));
        vu += __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            prs, static_cast<uint32_t>((s0 * Q + qu) * kFragBytes + lane * 16), 0, kCoherent));
      }
      act_store<DT, MT>(L, M, tile * (NF / 2) + j, t, lane, vg, vu);
    }
  }
  tile_done<kEpiAct>(a, L, tile);
}

// End of an item for a K-split workgroup: sums the KW wavefronts' tiles (LDS, wavefront order)
// and writes Y, or with split > 1 the fp32 partial, then the last split to arrive writes Y. With
// KW > 4 the tiles overlay the wavefronts' X transpose tiles, so the workgroup first waits until
// every wavefront is past its last K step.
template <int DT, int MT, int NF, int KW, int EPI>
__device__ __forceinline__ void packed_finish(const PackedArgs& a, const PLinear& L, int M, int item, int wave, int lane,
                                              f32x4 (&acc)[NF][MT], f32x4* red, int* last_flag) {
  constexpr int Q = NF * MT;
  int probe = 0;
  if constexpr (EPI == kEpiLora) {
    if (L.role == 2) probe = lora_probe(a);
  }
  if constexpr (KW > 4) lds_sync();
#pragma unroll
  for (int f = 0; f < NF; ++f)
#pragma unroll
    for (int t = 0; t < MT; ++t) red[(wave * Q + f * MT + t) * 64 + lane] = acc[f][t];
  lds_sync();
  int tile, s;
  item_tile(item, L.split, tile, s);
  if constexpr (EPI == kEpiAct) {
    if (L.out_f32 == PLM_OUT_SILU_MUL) {
      packed_finish_act<DT, MT, NF, KW>(a, L, M, tile, s, wave, lane, red, last_flag);
      return;
    }
  }
  const int n0 = tile * NF * 16;
  f32x4 sum[(Q + KW - 1) / KW];
#pragma unroll
  for (int i = 0; i * KW < Q; ++i) {
    const int q = wave + KW * i;
    if (q < Q) {
      f32x4 v = red[q * 64 + lane];
#pragma unroll
      for (int w = 1; w < KW; ++w) v += red[(w * Q + q) * 64 + lane];
      sum[i] = v;
    }
  }
  lds_sync();  // every wavefront has read the tiles; LDS is free for the next item
  if (L.split == 1) {
    if constexpr (EPI == kEpiLora) {
      if (L.role == 2) lora_wait_h(a, lane, probe);
    }
#pragma unroll
    for (int i = 0; i * KW < Q; ++i) {
      const int q = wave + KW * i;
      if (q < Q) packed_store_frag<DT, MT, EPI>(a, L, M, n0, q, lane, sum[i]);
    }
    tile_done<EPI>(a, L, tile);
    return;
  }
  // Split partial: one KiB block per fragment (an fp32 fragment is 64 lanes x 16 bytes), written
  // through to the device-coherent level.
  const uint32_t tile_bytes = static_cast<uint32_t>(L.split) * Q * kFragBytes;
  const auto prs = make_rsrc(L.partial + static_cast<int64_t>(tile) * L.split * Q * 256, tile_bytes);
#pragma unroll
  for (int i = 0; i * KW < Q; ++i) {
    const int q = wave + KW * i;
    if (q < Q)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sum[i]), prs,
                                             static_cast<uint32_t>((s * Q + q) * kFragBytes + lane * 16), 0, kCoherent);
  }
  __builtin_amdgcn_s_waitcnt(0);  // this wavefront's partial is written through
  lds_sync();
  if (threadIdx.x == 0) {
    int* counter = L.arrive + tile;
    const int before = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = before == L.split - 1;
    if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *last_flag = last;
  }
  lds_sync();
  if (*last_flag == 0) return;
  if constexpr (EPI == kEpiLora) {
    if (L.role == 2) lora_wait_h(a, lane, probe);
  }
#pragma unroll
  for (int i = 0; i * KW < Q; ++i) {
    const int q = wave + KW * i;
    if (q < Q) {
      f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int s0 = 0; s0 < L.split; s0 += 8) {
        u32x4 part[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
          part[j] = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         prs, s0 + j < L.split ? static_cast<uint32_t>(((s0 + j) * Q + q) * kFragBytes + lane * 16) : kOutOfRange,
                         0, kCoherent));
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (s0 + j < L.split) v += __builtin_bit_cast(f32x4, part[j]);
      }
      packed_store_frag<DT, MT, EPI>(a, L, M, n0, q, lane, v);
    }
  }
  tile_done<EPI>(a, L, tile);
}

// End of an item for a row-split workgroup (KW = 1): each wavefront owns its NF fragments of the
// tile outright and writes them (Y, or with split > 1 its fp32 partials; the last split of the
// tile to arrive sums each wavefront's partials in split order and writes Y).
template <int DT, int MT, int NF, int EPI>
__device__ __forceinline__ void packed_finish_rows(const PackedArgs& a, const PLinear& L, int M, int item, int wave,
                                                   int lane, f32x4 (&acc)[NF][MT], int* last_flag) {
  constexpr int QW = NF * MT;               // fragments of one wavefront
  constexpr int Q = kPackedWaves * QW;      // fragments of the tile
  int tile, s;
  item_tile(item, L.split, tile, s);
  const int n0 = (tile * 4 + wave) * NF * 16;
  int probe = 0;
  if constexpr (EPI == kEpiLora) {
    if (L.role == 2) probe = lora_probe(a);
  }
  if (L.split == 1) {
    if constexpr (EPI == kEpiLora) {
      if (L.role == 2) lora_wait_h(a, lane, probe);
    }
    if (EPI == kEpiAct && L.out_f32 == PLM_OUT_SILU_MUL) {
#pragma unroll
      for (int j = 0; j < NF / 2; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t)
          act_store<DT, MT>(L, M, (tile * 4 + wave) * (NF / 2) + j, t, lane, acc[2 * j][t], acc[2 * j + 1][t]);
    } else {
#pragma unroll
      for (int f = 0; f < NF; ++f)
#pragma unroll
        for (int t = 0; t < MT; ++t) packed_store_frag<DT, MT, EPI>(a, L, M, n0, f * MT + t, lane, acc[f][t]);
    }
    tile_done<EPI>(a, L, tile);
    return;
  }
  const uint32_t tile_bytes = static_cast<uint32_t>(L.split) * Q * kFragBytes;
  const auto prs = make_rsrc(L.partial + static_cast<int64_t>(tile) * L.split * Q * 256, tile_bytes);
#pragma unroll
  for (int f = 0; f < NF; ++f)
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int q = wave * QW + f * MT + t;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[f][t]), prs,
                                             static_cast<uint32_t>((s * Q + q) * kFragBytes + lane * 16), 0, kCoherent);
    }
  __builtin_amdgcn_s_waitcnt(0);  // this wavefront's partial is written through
  lds_sync();
  if (threadIdx.x == 0) {
    int* counter = L.arrive + tile;
    const int before = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = before == L.split - 1;
    if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *last_flag = last;
  }
  lds_sync();
  if (*last_flag == 0) return;
  if constexpr (EPI == kEpiLora) {
    if (L.role == 2) lora_wait_h(a, lane, probe);
  }
  if (EPI == kEpiAct && L.out_f32 == PLM_OUT_SILU_MUL) {
    // Each of the wavefront's (gate, up) pairs: both partials summed in split order.
#pragma unroll 1
    for (int pw = 0; pw < QW / 2; ++pw) {
      const int j = pw / MT, t = pw - j * MT, qg = wave * QW + 2 * j * MT + t, qu = qg + MT;
      f32x4 vg = f32x4{0.f, 0.f, 0.f, 0.f}, vu = vg;
      for (int s0 = 0; s0 < L.split; ++s0) {
        vg += __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            prs, static_cast<uint32_t>((s0 * Q + qg) * kFragBytes + lane * 16), 0, kCoherent));
        vu += __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            prs, static_cast<uint32_t>((s0 * Q + qu) * kFragBytes + lane * 16), 0, kCoherent));
      }
      act_store<DT, MT>(L, M, (tile * 4 + wave) * (NF / 2) + j, t, lane, vg, vu);
    }
    tile_done<EPI>(a, L, tile);
    return;
  }
  // A rolled loop over the wavefront's fragments: unrolled, the compiler would keep every
  // fragment's partial loads in flight at once and run out of registers.
#pragma unroll 1
  for (int qw = 0; qw < QW; ++qw) {
    const int q = wave * QW + qw;
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < L.split; s0 += 8) {
      u32x4 part[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        part[j] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       prs, s0 + j < L.split ? static_cast<uint32_t>(((s0 + j) * Q + q) * kFragBytes + lane * 16) : kOutOfRange,
                       0, kCoherent));
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (s0 + j < L.split) v += __builtin_bit_cast(f32x4, part[j]);
    }
    packed_store_frag<DT, MT, EPI>(a, L, M, n0, qw, lane, v);
  }
  tile_done<EPI>(a, L, tile);
}

extern __shared__ __attribute__((aligned(16))) f32x4 packed_lds[];

// Grid barrier after the consumed linear with sequence number `seq`, in two halves so that the
// wait can overlap weight traffic: barrier_arrive raises this workgroup's progress flag (its
// stores are written through: the caller waited for them), barrier_wait polls every workgroup's
// flag until all are at least as far (bounded).
__device__ __forceinline__ void barrier_arrive(const PackedArgs& a, int64_t epoch, int seq) {
  int64_t* flags = reinterpret_cast<int64_t*>(a.counters + kPackedBarrierBase);
  lds_sync();
  if (threadIdx.x == 0) publish(flags + blockIdx.x, ((epoch + 1) << 16) + seq);
}

__device__ __forceinline__ void barrier_wait(const PackedArgs& a, int64_t epoch, int seq, int lane) {
  const int64_t target = ((epoch + 1) << 16) + seq;
  if (threadIdx.x < 64 && !chain_failed(a)) {
    // Each lane polls G/64 flags with device-coherent loads, issued in batches of eight (one
    // batch covers 512 workgroups) before any of the batch is examined.
    const auto frs = make_rsrc(a.counters + kPackedBarrierBase, static_cast<uint32_t>(a.G) * 8u);
    for (int i = 0;; ++i) {
      int64_t low = INT64_MAX;
      for (int j0 = 0; j0 * 64 < a.G; j0 += 8) {
#pragma unroll
        for (int j = j0; j < j0 + 8; ++j) {
          if (j * 64 < a.G) {
            const u32x2 v = __builtin_bit_cast(
                u32x2, __builtin_amdgcn_raw_buffer_load_b64(frs, static_cast<uint32_t>((j * 64 + lane) * 8), 0, kCoherent));
            const int64_t f = static_cast<int64_t>((static_cast<uint64_t>(v.y) << 32) | v.x);
            low = j * 64 + lane < a.G ? min(low, f) : low;
          }
        }
      }
      if (__all(low >= target)) break;
      if (i >= a.spin_limit) {
        if (lane == 0) publish(a.counters + kPkErrorSlot, 1);
        break;
      }
      if (i % kErrorCheckPolls == kErrorCheckPolls - 1 && chain_failed(a)) break;
      __builtin_amdgcn_s_sleep(1);
    }
  }
  lds_sync();
}

typedef __attribute__((address_space(3))) void PkLdsVoid;

// Cache warming during a barrier: requests up to kWarmFragments more of the next linear's weight
// fragments this wavefront will stream (after the D stages already in registers) into a sink KiB
// of LDS that nothing reads (kept apart from the X tiles: the wavefronts' sink writes may land
// after another wavefront has written its next X tile), so that they are on their way from HBM
// into the caches while the workgroup waits; the pipeline then finds them in L2 / the Infinity
// Cache.
constexpr int kWarmFragments = 32;

template <int NF, int D, int KW>
__device__ __forceinline__ void warm_weights(const PLinear& Ln, int G, int wave, int lane, PCursor nx,
                                             __amdgpu_buffer_rsrc_t wr, const uint32_t* wo, PkLdsVoid* dst) {
  for (int n = 0; n < kWarmFragments / NF && nx.item < Ln.items; ++n) {
    if (nx.st < nx.end) {
      const int ws = __builtin_amdgcn_readfirstlane(static_cast<int>(nx.wbase + pack_step_offset(nx.st, Ln.wgroup)));
#pragma unroll
      for (int f = 0; f < NF; ++f) __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, dst, 16, wo[f], ws, 0, 0);
    }
    pc_advance<NF, D, KW>(Ln, G, wave, nx);
  }
  (void)lane;
}

// sync == 2: waits until every tile of the producer linear P that this wavefront's items of L
// read has raised its flag (bounded; error flag on timeout). The range covers every 128-byte
// line the X loads touch, not only the columns they use: a line holding a column of an
// unfinished neighbour tile would otherwise enter this XCD's L2 with that column's old value and
// be served later to a wavefront that waited for the neighbour. The widening by 63 columns is
// exact because the host picks this mode only when every consumed Y starts on a 128-byte boundary
// and its rows are a multiple of 128 bytes apart, so no line spans two rows.
template <int NF, int KW>
__device__ __forceinline__ void wait_producer_tiles(const PackedArgs& a, const PLinear& L, const PLinear& P, int wave,
                                                    int lane) {
  int lo = L.Ks, hi = 0;
  for (int item = blockIdx.x; item < L.items; item += a.G) {
    int tile, s, b, e;
    item_tile(item, L.split, tile, s);
    packed_range<KW>(L.Ks, s, L.split, wave, b, e);
    if (b < e) {
      lo = min(lo, b);
      hi = max(hi, e);
    }
  }
  if (lo >= hi || chain_failed(a)) return;
  // Y columns of one producer tile (half its rows when its epilogue is the SiLU-and-multiply)
  const int cols = P.out_f32 == PLM_OUT_SILU_MUL ? 8 * tile_frags<NF, KW>() : 16 * tile_frags<NF, KW>();
  constexpr int kLineCols = 64;  // bf16 columns of a 128-byte line
  const int t0 = max(32 * lo - (kLineCols - 1), 0) / cols;
  const int t1 = min((32 * hi - 1 + (kLineCols - 1)) / cols, P.tiles - 1);
  const auto frs = make_rsrc(P.flag, static_cast<uint32_t>(P.tiles) * 8u);
  for (int i = 0;; ++i) {
    bool done = true;
    for (int b = t0; b <= t1; b += 64) {
      const int t = b + lane;
      const u32x2 v = __builtin_bit_cast(
          u32x2, __builtin_amdgcn_raw_buffer_load_b64(frs, t <= t1 ? static_cast<uint32_t>(t) * 8u : kOutOfRange, 0, kCoherent));
      const int64_t f = static_cast<int64_t>((static_cast<uint64_t>(v.y) << 32) | v.x);
      done = done && (t > t1 || f >= P.flag_value);
    }
    if (__all(done)) break;
    if (i >= a.spin_limit) {
      if (lane == 0) publish(a.counters + kPkErrorSlot, 1);
      break;
    }
    if (i % kErrorCheckPolls == kErrorCheckPolls - 1 && chain_failed(a)) break;
    __builtin_amdgcn_s_sleep(1);
  }
}

// End of a chained launch: the last workgroup to finish advances the epoch, so that the next
// launch's flags exceed every flag of this one. Every workgroup reads the epoch when it starts and
// counts itself out only after all its wavefronts are past the end, so no workgroup of this
// launch reads the advanced value; the counter is left at zero for the next launch.
__device__ __forceinline__ void chain_exit(const PackedArgs& a) {
  __syncthreads();
  if (threadIdx.x == 0) {
    if (__hip_atomic_fetch_add(a.counters + kPkExitSlot, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.G - 1) {
      __hip_atomic_store(a.counters + kPkExitSlot, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      int64_t* epoch = reinterpret_cast<int64_t*>(a.counters + kPkEpochSlot);
      publish(epoch, collect(epoch) + 1);
    }
  }
}

// Registers per lane of the operand pipeline and the accumulators (with KW = 1 also the MT X
// operands read back from the shared tile, which cannot reuse the pipeline's X registers).
// Configurations below a measured bound (the largest without scratch at 256 VGPRs) run two
// workgroups per CU; larger ones run one, with the AGPR half of the register file available.
template <int MT, int NF, int D, int KW>
constexpr int packed_regs() {
  return (D * (NF + x_per_wave<MT, KW>()) + NF * MT + (KW == 1 ? MT : 0)) * 4;
}
template <int MT, int NF, int D, int KW>
constexpr bool packed_two_per_cu() {
  if constexpr (KW == 1) return packed_regs<MT, NF, D, KW>() <= 100;
  if constexpr (KW > 4) return false;
  return packed_regs<MT, NF, D, KW>() <= 128 && (MT <= 6 || packed_regs<MT, NF, D, KW>() <= 104);
}
// Minimum wavefronts per SIMD the kernel is compiled for (the register budget: 512 per lane
// divided by it): two or one 4-wavefront workgroups per CU (KW = 1, 4), one 8- or 16-wavefront
// workgroup per CU (KW = 8: 2 per SIMD; KW = 16: 4 per SIMD, 128 registers).
template <int MT, int NF, int D, int KW>
constexpr int packed_waves_per_simd() {
  if constexpr (KW > 4) return KW / 4;
  return packed_two_per_cu<MT, NF, D, KW>() ? 2 : 1;
}

// LDS bytes before the warm-up sink: KW = 1: four shared X tile sets (two K steps, double-buffered);
// KW = 4: the four wavefronts' fp32 tiles (reduction), then a private X transpose tile set per
// wavefront; KW > 4: the reduction tiles overlaying the private X tile sets (two per wavefront
// when paired).
template <int MT, int NF, int KW>
constexpr size_t packed_lds_body() {
  constexpr size_t red = static_cast<size_t>(KW) * NF * MT * kFragBytes;
  constexpr size_t xts = static_cast<size_t>(KW) * MT * kXTileBytes * (KW != 1 && packed_pair_x<MT, KW>() ? 2 : 1);
  if constexpr (KW == 1) return static_cast<size_t>(4) * MT * kXTileBytes;
  if constexpr (KW == 4) return red + xts;
  return red > xts ? red : xts;
}

template <int DT, int MT, int NF, int D, int KW, int EPI>
__global__ __launch_bounds__(64 * packed_waves<KW>(), (packed_waves_per_simd<MT, NF, D, KW>())) void packed_gemm_kernel(PackedArgs a) {
  constexpr int XN = x_per_wave<MT, KW>();
  __shared__ int last_flag;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  f32x4* red = packed_lds;
  constexpr int kXSets = KW != 1 && packed_pair_x<MT, KW>() ? 2 : 1;  // private X tile sets per wavefront
  char* xt = reinterpret_cast<char*>(packed_lds) +
             (KW == 1 ? 0
                      : (KW == 4 ? static_cast<size_t>(4) * NF * MT * kFragBytes : 0) +
                            static_cast<size_t>(wave) * kXSets * MT * kXTileBytes);
  PkLdsVoid* sink = (PkLdsVoid*)(reinterpret_cast<char*>(packed_lds) + packed_lds_body<MT, NF, KW>());
  constexpr bool kSwizzleX = !(KW == 8 && MT * NF >= 14);  // the eight-wavefront tiles at 14+ fragments spill
  const int xt_write = x_tile_write_offset<kSwizzleX>(lane);
  const int xt_read = x_tile_read_offset<kSwizzleX>(lane);
  const int64_t epoch = a.sync ? sgpr64(collect(reinterpret_cast<const int64_t*>(a.counters + kPkEpochSlot))) : 0;

  u32x4 wb[D][NF], xb[D][XN];
  [[maybe_unused]] int xhalf = 0;  // KW = 1: the half of the X tile sets the next pair of K steps uses
  // The first weight stages of linear `gi` may already be in flight (requested before the last
  // grid barrier): then only X is still to be loaded for them.
  bool w_ready = false;
  for (int gi = 0; gi < a.count; ++gi) {
    const PLinear L = load_linear<NF, KW, EPI>(a, gi, epoch);
    POffsets<MT, NF, XN> o;
    packed_offsets<MT, NF, KW>(L, a.M, lane, wave, o);
    const auto wr = make_rsrc(L.wp, static_cast<uint32_t>(pack_bytes(L.N, L.Ks)));
    const auto xr = make_rsrc(L.x, static_cast<uint32_t>(a.M * L.ldx * 2));
    PCursor ld{first_item<EPI>(a, gi), 0, 0, 0, 0};
    pc_enter<NF, D, KW>(L, wave, ld);
    PCursor cp = ld;
    if (ld.item < L.items) {
      if (a.sync == 2 && gi > 0) {
        // The first weight stages and more of the weights into the caches, which do not depend
        // on the producer; then the wait for the producer tiles this wavefront reads; then X.
        PCursor lw = ld;
#pragma unroll
        for (int j = 0; j < D; ++j) {
          issue_w<NF>(wr, lw, L.items, L.wgroup, o.wo, wb[j]);
          pc_advance<NF, D, KW>(L, a.G, wave, lw);
          __builtin_amdgcn_sched_barrier(0);
        }
        warm_weights<NF, D, KW>(L, a.G, wave, lane, lw, wr, o.wo, sink);
        wait_producer_tiles<NF, KW>(a, L, load_linear<NF, KW>(a, gi - 1, epoch), wave, lane);
#pragma unroll
        for (int j = 0; j < D; ++j) {
          issue_x_stage<MT, NF, XN, KW, D>(j, xr, ld, L.items, L.Ks, o, xb);
          pc_advance<NF, D, KW>(L, a.G, wave, ld);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else if (!w_ready) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
          issue_w<NF>(wr, ld, L.items, L.wgroup, o.wo, wb[j]);
          issue_x_stage<MT, NF, XN, KW, D>(j, xr, ld, L.items, L.Ks, o, xb);
          pc_advance<NF, D, KW>(L, a.G, wave, ld);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int j = 0; j < D; ++j) {
          issue_x_stage<MT, NF, XN, KW, D>(j, xr, ld, L.items, L.Ks, o, xb);
          pc_advance<NF, D, KW>(L, a.G, wave, ld);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      for (;;) {
        f32x4 acc[NF][MT];
#pragma unroll
        for (int f = 0; f < NF; ++f)
#pragma unroll
          for (int t = 0; t < MT; ++t) acc[f][t] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int steps = cp.pend - cp.st;  // a multiple of D, at least D
        // One pipeline stage: stage j's X into the MFMA operand layout, its MFMAs, then stage j's
        // loads for D steps ahead.
        auto stage = [&](int j) __attribute__((always_inline)) {
          u32x4 xop[MT];
          if constexpr (KW != 1 && kXSets == 2) {
            // The even stage stores both steps' X into the wavefront's two tile sets.
            if ((j & 1) == 0) {
#pragma unroll
              for (int t = 0; t < MT; ++t) {
                *reinterpret_cast<u32x4*>(xt + t * kXTileBytes + xt_write) = xb[j][t];
                *reinterpret_cast<u32x4*>(xt + (MT + t) * kXTileBytes + xt_write) = xb[j + 1][t];
              }
            }
            const char* xs = xt + (j & 1) * MT * kXTileBytes;
#pragma unroll
            for (int t = 0; t < MT; ++t) xop[t] = *reinterpret_cast<const u32x4*>(xs + t * kXTileBytes + xt_read);
          } else if constexpr (KW != 1) {
#pragma unroll
            for (int t = 0; t < MT; ++t) *reinterpret_cast<u32x4*>(xt + t * kXTileBytes + xt_write) = xb[j][t];
#pragma unroll
            for (int t = 0; t < MT; ++t) xop[t] = *reinterpret_cast<const u32x4*>(xt + t * kXTileBytes + xt_read);
          } else {
            stage_x_rows<MT, XN, D>(j, xt, wave, xt_write, xt_read, xb, xop, xhalf);
          }
#pragma unroll
          for (int f = 0; f < NF; ++f)
#pragma unroll
            for (int t = 0; t < MT; ++t) acc[f][t] = mfma_16x16x32<DT>(wb[j][f], xop[t], acc[f][t]);
          issue_w<NF>(wr, ld, L.items, L.wgroup, o.wo, wb[j]);
          issue_x_stage<MT, NF, XN, KW, D>(j, xr, ld, L.items, L.Ks, o, xb);
          pc_advance<NF, D, KW>(L, a.G, wave, ld);
          __builtin_amdgcn_sched_barrier(0);
        };
        // The item's first D steps are peeled off the loop: the loop is then entered only from a
        // block that leaves the loads in flight in the loop's own order, so the compiler's
        // load-count waits inside it stay exact (entered straight from the item's start, where
        // paths with other load orders meet, it waited for every load once per D steps).
#pragma unroll
        for (int j = 0; j < D; ++j) stage(j);
        for (int i = D; i < steps; i += D) {
#pragma unroll
          for (int j = 0; j < D; ++j) stage(j);
        }
        if constexpr (KW != 1)
          packed_finish<DT, MT, NF, KW, EPI>(a, L, a.M, cp.item, wave, lane, acc, red, &last_flag);
        else
          packed_finish_rows<DT, MT, NF, EPI>(a, L, a.M, cp.item, wave, lane, acc, &last_flag);
        cp.item += a.G;
        if (cp.item >= L.items) break;
        pc_enter<NF, D, KW>(L, wave, cp);
      }
    }
    w_ready = false;
    if (a.sync == 1 && L.consumed && gi + 1 < a.count) {
      // Arrive, request the next linear's first weight stages into registers and more of its
      // weights into the caches (weights never depend on the barrier), then wait for every
      // workgroup's part of this Y.
      __builtin_amdgcn_s_waitcnt(0);
      barrier_arrive(a, epoch, L.seq);
      const PLinear Ln = load_linear<NF, KW, EPI>(a, gi + 1);
      PCursor nx{first_item<EPI>(a, gi + 1), 0, 0, 0, 0};
      pc_enter<NF, D, KW>(Ln, wave, nx);
      if (nx.item < Ln.items) {
        POffsets<MT, NF, XN> on;
        packed_offsets<MT, NF, KW>(Ln, a.M, lane, wave, on);
        const auto wrn = make_rsrc(Ln.wp, static_cast<uint32_t>(pack_bytes(Ln.N, Ln.Ks)));
#pragma unroll
        for (int j = 0; j < D; ++j) {
          issue_w<NF>(wrn, nx, Ln.items, Ln.wgroup, on.wo, wb[j]);
          pc_advance<NF, D, KW>(Ln, a.G, wave, nx);
          __builtin_amdgcn_sched_barrier(0);
        }
        w_ready = true;
        warm_weights<NF, D, KW>(Ln, a.G, wave, lane, nx, wrn, on.wo, sink);
      }
      barrier_wait(a, epoch, L.seq, lane);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  if (a.sync) chain_exit(a);
}

// Compiled configurations (all without scratch): 1 <= MT <= 8, NF in {1, 2, 4}, D in
// {2, 4, 6, 8}, at most 20 accumulator fragments, and either two workgroups per CU or one
// workgroup per CU with the pipeline's registers within 320 of a lane's 512.
template <int MT, int NF, int D, int KW>
constexpr bool packed_compiled() {
  if (MT < 1 || MT > 8 || (NF != 1 && NF != 2 && NF != 4) || (D != 2 && D != 4 && D != 6 && D != 8)) return false;
  if ((KW != 1 && KW != 4 && KW != 8 && KW != 16) || NF * MT > 20) return false;
  if constexpr (KW > 4) {
    // One workgroup per CU; the pipeline within the per-wavefront budget (measured without scratch).
    return packed_lds_body<MT, NF, KW>() + kFragBytes <= 160 * 1024 &&
           packed_regs<MT, NF, D, KW>() <= (KW == 8 ? 144 : 60);
  }
  return packed_two_per_cu<MT, NF, D, KW>() || packed_regs<MT, NF, D, KW>() <= 320;
}

// Whether a configuration's epilogue fits the registers its pipeline leaves (measured: no scratch
// in the compiler's resource report for either element type). KW = 1 configurations are held to
// 256 VGPRs, KW = 16 ones to 128; the LoRA epilogue keeps the low-rank correction's operands beside
// the pipeline. A configuration that does not fit runs at a lower pipeline depth D (packed_pick_d):
// the K steps are summed in the same order at every depth, so the results are the same. At D = 2
// only the LoRA epilogue on 16-wavefront tiles with 4 accumulator fragments does not fit; those
// tiles are not compiled for it.
template <int MT, int NF, int D, int KW, int EPI>
constexpr bool packed_fits() {
  constexpr int r = packed_regs<MT, NF, D, KW>();
  if constexpr (KW == 1) return r <= 240 || (EPI == kEpiAct && r <= 292);
  if constexpr (KW == 16) return EPI == kEpiLora ? r <= 48 : (r <= 52 || MT == 1 || D == 2);
  if constexpr (EPI != kEpiLora) return true;
  if constexpr (KW == 4) return packed_two_per_cu<MT, NF, D, KW>() || r <= 288;
  return true;
}

template <int MT, int NF, int KW>
constexpr size_t packed_lds_bytes() {
  return packed_lds_body<MT, NF, KW>() + kFragBytes;  // + the warm-up sink
}

// Launches with G = min(a.G, resident workgroups), where a.G arrives as the most items of any
// linear; a chained launch with grid barriers (a.sync) uses every resident workgroup. `dry` only
// checks that the kernel exists.
template <int DT, int MT, int NF, int D, int KW, int EPI>
hipError_t packed_launch(PackedArgs& a, int cus, hipStream_t stream, bool dry) {
  if constexpr (!packed_compiled<MT, NF, D, KW>() || !packed_fits<MT, NF, D, KW, EPI>()) {
    return hipErrorInvalidConfiguration;
  } else {
    if (dry) return hipSuccess;
    auto kern = packed_gemm_kernel<DT, MT, NF, D, KW, EPI>;
    constexpr size_t lds = packed_lds_bytes<MT, NF, KW>();
    static int per_cu = 0;
    if (per_cu == 0) {
      if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (e != hipSuccess) return e;
      }
      const int n = resident_per_cu(reinterpret_cast<const void*>(kern), 64 * packed_waves<KW>(), lds);
      if (n < 1) return hipErrorInvalidConfiguration;
      per_cu = n;
    }
    const int resident = min(cus * per_cu, kPkMaxWorkgroups);
    if (a.count == 0) {  // query: the resident workgroups a chained launch would use
      a.G = resident;
      return hipSuccess;
    }
    a.G = a.sync ? resident : min(a.G, resident);
    if (a.G < 1) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(kern, dim3(a.G), dim3(64 * packed_waves<KW>()), lds, stream, a);
    return hipGetLastError();
  }
}

template <int DT, int MT, int NF, int KW, int EPI>
hipError_t packed_pick_d(PackedArgs& a, int d, int cus, hipStream_t s, bool dry) {
  // The depth of a compiled tile is a cap: lowered to one whose epilogue fits (packed_fits).
  if (d == 8 && packed_compiled<MT, NF, 8, KW>() && !packed_fits<MT, NF, 8, KW, EPI>()) d = 6;
  if (d == 6 && packed_compiled<MT, NF, 6, KW>() && !packed_fits<MT, NF, 6, KW, EPI>()) d = 4;
  if (d == 4 && packed_compiled<MT, NF, 4, KW>() && !packed_fits<MT, NF, 4, KW, EPI>()) d = 2;
  if (d == 2) return packed_launch<DT, MT, NF, 2, KW, EPI>(a, cus, s, dry);
  if (d == 4) return packed_launch<DT, MT, NF, 4, KW, EPI>(a, cus, s, dry);
  if (d == 6) return packed_launch<DT, MT, NF, 6, KW, EPI>(a, cus, s, dry);
  if (d == 8) return packed_launch<DT, MT, NF, 8, KW, EPI>(a, cus, s, dry);
  return hipErrorInvalidConfiguration;
}

template <int DT, int MT, int KW, int EPI>
hipError_t packed_pick(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry) {
  if (nf == 1) {
    if constexpr (EPI == kEpiAct) return hipErrorInvalidConfiguration;  // gate and up fragments come in pairs
    else return packed_pick_d<DT, MT, 1, KW, EPI>(a, d, cus, s, dry);
  }
  if (nf == 2) return packed_pick_d<DT, MT, 2, KW, EPI>(a, d, cus, s, dry);
  if (nf == 4) return packed_pick_d<DT, MT, 4, KW, EPI>(a, d, cus, s, dry);
  return hipErrorInvalidConfiguration;
}

// EPI: the store epilogue (kEpiPlain; kEpiLora: the gated-LoRA launch, PackedArgs::lora: two linears,
// the base tiles corrected).
template <int DT, int KW, int EPI = kEpiPlain>
hipError_t packed_dispatch_kw(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry) {
  switch ((a.M + 15) / 16) {
    case 1: return packed_pick<DT, 1, KW, EPI>(a, nf, d, cus, s, dry);
    case 2: return packed_pick<DT, 2, KW, EPI>(a, nf, d, cus, s, dry);
    case 3: return packed_pick<DT, 3, KW, EPI>(a, nf, d, cus, s, dry);
    case 4: return packed_pick<DT, 4, KW, EPI>(a, nf, d, cus, s, dry);
    case 5: return packed_pick<DT, 5, KW, EPI>(a, nf, d, cus, s, dry);
    case 6: return packed_pick<DT, 6, KW, EPI>(a, nf, d, cus, s, dry);
    case 7: return packed_pick<DT, 7, KW, EPI>(a, nf, d, cus, s, dry);
    case 8: return packed_pick<DT, 8, KW, EPI>(a, nf, d, cus, s, dry);
  }
  return hipErrorInvalidConfiguration;
}

// The single-linear entry behind plm_gemm_packed / plm_gemm_packed_f32out (argument checks, then
// the launch), and the workspace bytes it needs for a shape and tile (-1 for an invalid tile): for
// other translation units that launch the same kernel over their own scratch. `cap` bounds the
// scratch a wide call (M > 128) may use: its K split, which only sets the speed, is chosen to fit.
int packed_gemm_call(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, void* y, int64_t ldy, int64_t M,
                     int64_t N, int64_t K, const plm_tile* tile, void* workspace, size_t workspace_bytes, void* stream,
                     int out_f32, int64_t cap = INT64_MAX);
int64_t packed_gemm_workspace(int64_t M, int64_t N, int64_t K, const plm_tile* tile, int64_t cap = INT64_MAX);

// One translation unit per (dtype, workgroup layout) so that they build in parallel.
hipError_t packed_dispatch_bf16_k1(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_bf16_k4(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_bf16_k8(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_bf16_k16(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_f16_k1(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_f16_k4(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_f16_k8(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_f16_k16(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
// The same translation units' gated-LoRA launches.
hipError_t packed_dispatch_lora_bf16_k1(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_lora_bf16_k4(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_lora_bf16_k8(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_lora_bf16_k16(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_lora_f16_k1(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_lora_f16_k4(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_lora_f16_k8(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_lora_f16_k16(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
// ... and the SiLU-and-multiply launches (wave_frags 2 or 4).
hipError_t packed_dispatch_act_bf16_k1(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_act_bf16_k4(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_act_bf16_k8(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_act_bf16_k16(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_act_f16_k1(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_act_f16_k4(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_act_f16_k8(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);
hipError_t packed_dispatch_act_f16_k16(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry);

}  // namespace plm
