/*
 * plm_amd.h — C ABI of the MI355X (gfx950) kernels for the PLM round's dense linears.
 *
 * Plain pointers, sizes and a stream handle; no torch types. Every entry point launches on the
 * caller's HIP stream, performs no host synchronisation and allocates nothing, so it can be
 * recorded into a HIP graph. Status codes are PLM_OK (0) or a negative PLM_ERR_* value;
 * plm_status_string() names them.
 *
 * Layouts follow the reference's GEMM: Y[M,N] = X[M,K] · W[N,K]^T, all row-major with the
 * last dimension contiguous (plm/fast_gemm.py:3, 17-48). Leading dimensions are in elements.
 */
#ifndef PLM_AMD_H
#define PLM_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of X, W and Y (the reference's HALF_DTYPES, plm/fast_gemm.py:66). */
enum plm_dtype { PLM_BF16 = 0, PLM_F16 = 1 };

/* Rounding applied to the fp32 logits before the verify epilogue reads them.
 * PLM_ROUND_F32 keeps the fp32 accumulator; PLM_ROUND_BF16 / PLM_ROUND_F16 round to the model
 * dtype first, which is what the reference's decoder sees (plm/fast_gemm.py:46 casts the
 * accumulator, plm/decoder.py:73 upcasts it again). */
enum plm_round_mode { PLM_ROUND_F32 = 0, PLM_ROUND_BF16 = 1, PLM_ROUND_F16 = 2 };

/* Acceptance rule of the verify step (RoundDecoder's accept_rule, plm/decoder.py:88-89, 353):
 * PLM_RULE_NUCLEUS is nucleus_acceptance (plm/decoder.py:71-75) with threshold = top-p;
 * PLM_RULE_FLOOR is floor_acceptance (plm/decoder.py:78-82) with threshold = epsilon. */
enum plm_accept_rule { PLM_RULE_NUCLEUS = 0, PLM_RULE_FLOOR = 1 };

/* What a chain linear writes (plm_chain_gemm.out_f32): Y in the input dtype, the fp32
 * accumulator, or — packed chains only — the SiLU-and-multiply of a fused gate/up projection
 * (plm_gemm_packed_silu_mul's epilogue: Y[M, N/2], W packed with its halves interleaved). */
enum plm_out_kind { PLM_OUT_MODEL = 0, PLM_OUT_F32 = 1, PLM_OUT_SILU_MUL = 2 };

/* Every workspace starts with this many bytes of integer arrival counters, which must be zero
 * before the first call and which every kernel leaves zero; the rest of a workspace is scratch
 * that needs no initialisation. One workspace may therefore serve every entry point in turn on
 * one stream (calls that overlap on different streams need separate workspaces). */
#define PLM_WORKSPACE_COUNTER_BYTES (1u << 18)

enum plm_status {
  PLM_OK = 0,
  PLM_ERR_ARGUMENT = -1,      /* bad size, stride, dtype or null pointer */
  PLM_ERR_ALIGNMENT = -2,     /* a pointer or leading dimension is not 16-byte aligned */
  PLM_ERR_TILE = -3,          /* no compiled kernel for this tile / M combination */
  PLM_ERR_WORKSPACE = -4,     /* workspace missing or smaller than the query function says */
  PLM_ERR_LAUNCH = -5         /* the HIP launch itself failed */
};

/* Index (in ints) of the error flag inside the counter area: a chained launch sets it to 1 when a
 * bounded wait for another workgroup gave up (the launch's results are then invalid). */
#define PLM_WORKSPACE_ERROR_INDEX 2

/*
 * Tile configuration of one GEMM shape: the MI355X counterpart of the reference's
 * {BLOCK_M, BLOCK_N, BLOCK_K, SPLIT_K, num_warps, num_stages} dict (plm/fast_gemm.py:64).
 * The fields mean different things to the two kernel families:
 *   packed-weight kernel (plm_gemm_packed, plm_gemm_chain_packed, the verify over packed W):
 *     wave_frags : 16-row weight fragments each wavefront streams per K step (1, 2 or 4).
 *     k_waves    : workgroup layout. 4, 8 or 16: that many wavefronts split the K range of a
 *                  16*wave_frags-row tile and their fp32 tiles are summed in LDS in wavefront order;
 *                  1: four wavefronts each own 16*wave_frags rows of a 64*wave_frags-row tile over
 *                  the whole K range and share one copy of X through LDS.
 *     split_k    : workgroups splitting K (1..64); their fp32 partials are summed in split order
 *                  0..split_k-1 by the last workgroup of the tile to finish (no float atomics).
 *     unroll     : K steps of loads in flight per wavefront (2, 4, 6 or 8).
 *   row-major streaming kernel (plm_gemm, plm_gemm_chain, plm_lm_head_verify):
 *     wave_frags : 16-row fragments per compute wavefront; a workgroup has four compute wavefronts
 *                  (tile = 64*wave_frags rows), four loader wavefronts and one epilogue wavefront.
 *     k_waves    : 4 (the compute wavefronts).
 *     split_k    : as above.
 *     unroll     : 2 (one 128-byte line of every weight row per streamed chunk).
 */
typedef struct plm_tile {
  int32_t wave_frags;
  int32_t k_waves;
  int32_t split_k;
  int32_t unroll;
} plm_tile;

/*
 * Packed weights. plm_pack_weight rearranges a row-major W[N,K] (ldw elements per row) into the
 * operand order of gfx950's 16x16x32 MFMA: fragment (f, s) = rows [16f, 16f+16) x K [32s, 32s+32)
 * as 64 lanes x 16 bytes, lane l holding row 16f + l%16, elements 32s + 8*(l/16) .. +8. With the
 * fragment rows zero-padded to R (a multiple of 16) and the K steps to a multiple of 8, fragment
 * (f, s) lies at KiB (s/8)*8R + 8f + s%8: eight K steps of a row together, then the next eight of
 * every row. Each weight load of plm_gemm_packed is then one contiguous KiB, and workgroups that
 * stream their rows at the same K step read one contiguous stretch between them. The format is
 * this library's own, read only by its kernels and plm_unpack_weight. Packing is a one-time pass
 * per weight (the reference reads its weights as they
 * are, plm/fast_gemm.py:17-48; a caller keeps the packed copy next to the weight).
 * plm_packed_weight_bytes gives the size; `packed` must be 16-byte aligned.
 */
size_t plm_packed_weight_bytes(int64_t N, int64_t K);
int plm_pack_weight(int32_t dtype, const void* w, int64_t ldw, int64_t N, int64_t K, void* packed, size_t packed_bytes,
                    void* stream);

/*
 * The inverse of plm_pack_weight: writes the row-major W[N,K] (row stride ldw, 16-byte aligned,
 * ldw % 8 == 0) back from its packed copy, bit for bit. No counterpart in the reference, which
 * keeps only the row-major weight and hands the widths it does not tune (prefill chunks,
 * plm/rounds.py:16) to F.linear (plm/fast_gemm.py:108-111): a caller that keeps only the packed
 * copy unpacks a weight into a transient buffer for such a call.
 */
int plm_unpack_weight(int32_t dtype, const void* packed, size_t packed_bytes, int64_t N, int64_t K, void* w, int64_t ldw,
                      void* stream);

/*
 * Y[M,N] = X[M,K] · W[N,K]^T over a packed W, fp32 accumulation, Y in the input dtype: the fast
 * path behind triton_linear (plm/fast_gemm.py:82-97, with gemm_kernel 17-48 and
 * splitk_reduce_kernel 51-61). Tile fields for this kernel: wave_frags = 16-row fragments per
 * wavefront (1, 2, 4); k_waves = 4: a workgroup tile is 16*wave_frags rows and its four
 * wavefronts split the tile's K range (summed in LDS in wavefront order), or k_waves = 1: a
 * workgroup tile is 64*wave_frags rows, each wavefront owns 16*wave_frags of them over the whole
 * K range, and the four share one copy of X through LDS; split_k = workgroups splitting K (1..64,
 * partials summed in split order); unroll = K steps of loads in flight per wavefront (2, 4, 6,
 * 8). Requirements as plm_gemm (K % 8 == 0, K <= 2^24, ldx % 8 == 0, x 16-byte aligned) except
 * that M may exceed 128: wider calls (prefill chunks, plm/rounds.py:16, which the reference hands to
 * F.linear) run on a compute-oriented wide kernel (128 x 128 tiles staged through LDS, K split in
 * fixed order for shapes with few tiles) whose tiling is its own: `tile` must be valid but is not
 * used. Workspace: plm_gemm_packed_workspace_bytes.
 */
int plm_gemm_packed(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, void* y, int64_t ldy, int64_t M,
                    int64_t N, int64_t K, const plm_tile* tile, void* workspace, size_t workspace_bytes, void* stream);

/* As plm_gemm_packed with an fp32 Y (the accumulator before the cast, plm/fast_gemm.py:46). */
int plm_gemm_packed_f32out(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, float* y, int64_t ldy,
                           int64_t M, int64_t N, int64_t K, const plm_tile* tile, void* workspace,
                           size_t workspace_bytes, void* stream);

/*
 * plm_gemm_packed without a workspace argument and without allocating: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). The split-K scratch is a device array inside the
 * library, PLM_NOALLOC_SCRATCH_BYTES per device, held until the process ends; a shape and tile whose
 * plm_gemm_packed_workspace_bytes exceeds it is rejected with PLM_ERR_WORKSPACE. Every call on one
 * device shares that array, so calls that overlap on one device (other streams, other threads) race.
 * Otherwise as plm_gemm_packed: same kernel, same results bit for bit.
 */
#define PLM_NOALLOC_SCRATCH_BYTES (PLM_WORKSPACE_COUNTER_BYTES + (8u << 20))
int plm_gemm_packed_noalloc(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, void* y, int64_t ldy,
                            int64_t M, int64_t N, int64_t K, const plm_tile* tile, void* stream);

/* Workspace bytes plm_gemm_packed needs for this shape and tile (0 without split-K), and whether a
 * kernel is compiled for the tile at this M. */
size_t plm_gemm_packed_workspace_bytes(int64_t M, int64_t N, int64_t K, const plm_tile* tile);
int plm_gemm_packed_tile_supported(int32_t dtype, int64_t M, int64_t K, const plm_tile* tile);

/*
 * Y[M,N] = X[M,K] · W[N,K]^T with fp32 accumulation, Y in the input dtype.
 * Replaces triton_linear (plm/fast_gemm.py:82-97) together with gemm_kernel (17-48) and
 * splitk_reduce_kernel (51-61). Requirements: 1 <= M <= 128, K % 8 == 0, ldx/ldw % 8 == 0,
 * x and w 16-byte aligned. `workspace` may be NULL when plm_gemm_workspace_bytes() is 0;
 * otherwise its counter area must be zero before its first use (it is left zero).
 */
int plm_gemm(int32_t dtype, const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy,
             int64_t M, int64_t N, int64_t K, const plm_tile* tile, void* workspace, size_t workspace_bytes,
             void* stream);

/*
 * As plm_gemm, but Y is fp32: the accumulator before the cast to the input dtype (the value the
 * reference's gemm_kernel holds at plm/fast_gemm.py:46 before `.to(c dtype)`). With split_k == 1
 * and the tile plm_lm_head_verify uses, these are bit for bit the logits the verify step reads.
 */
int plm_gemm_f32out(int32_t dtype, const void* x, int64_t ldx, const void* w, int64_t ldw, float* y, int64_t ldy,
                    int64_t M, int64_t N, int64_t K, const plm_tile* tile, void* workspace, size_t workspace_bytes,
                    void* stream);

/*
 * One linear of a chain run by plm_gemm_chain: Y[M,N] = X[M,K] · W[N,K]^T. The first block is the
 * caller's; plm_gemm_chain_prepare fills the second.
 */
typedef struct plm_chain_gemm {
  const void* x;
  const void* w;
  void* y;
  int64_t ldx, ldw, ldy;
  int32_t N, K;
  int32_t split_k;        /* workgroups splitting K (>= 1) */
  int32_t dep;            /* -1, or the index of an earlier linear whose Y this X is (x == that y,
                             ldx == its ldy, K <= its Y's columns): the linear then waits for those tiles */
  int32_t out_f32;        /* a plm_out_kind: PLM_OUT_F32 (1) the fp32 accumulator, PLM_OUT_MODEL (0) Y in
                             the input dtype; PLM_OUT_SILU_MUL (2, packed chains, even wave_frags) the
                             SiLU-and-multiply, Y[M, N/2] with N % 32 == 0, ldy % 4 == 0, y 8-byte aligned */
  /* filled by plm_gemm_chain_prepare */
  int32_t consumed;       /* 1 when a later linear reads this Y */
  int32_t arrive_base;    /* counter-area index of this linear's split-K arrival counters */
  int32_t done_base;      /* plm_gemm_chain: counter-area index of this linear's tile-done flags;
                             plm_gemm_chain_packed: the progress-flag value that marks its Y written */
  int64_t partial_offset; /* float offset of this linear's split partials in the workspace */
} plm_chain_gemm;

/*
 * A chain of linears over packed weights in one launch (the round's linears back to back,
 * replacing the per-GEMM graph nodes of plm/decoder.py:312-324): plm_chain_gemm entries with
 * `w` a packed weight (ldw is ignored). After every linear whose Y a later one reads, all
 * workgroups meet at a grid barrier, so such a linear must not write fp32. The tile gives
 * wave_frags, k_waves and unroll for every linear; each linear's split_k is its own. The launch
 * (one kernel; its last workgroup to finish advances the workspace's launch epoch) needs
 * every workgroup resident at once (the device to itself while it runs); a barrier that does not
 * complete in about a second sets the int at PLM_WORKSPACE_ERROR_INDEX to 1.
 * plm_gemm_chain_packed_prepare fills the derived fields and returns the workspace bytes.
 */
int64_t plm_gemm_chain_packed_prepare(plm_chain_gemm* gemms, int32_t count, int64_t M, const plm_tile* tile);
/* Workgroups a packed launch with this tile keeps resident on the current device (the grid of a
 * chained launch), or a negative status. Needs a device. */
int plm_gemm_packed_resident_workgroups(int32_t dtype, int64_t M, const plm_tile* tile);
int plm_gemm_chain_packed(int32_t dtype, const plm_chain_gemm* host_gemms, const plm_chain_gemm* device_gemms,
                          int32_t count, int64_t M, const plm_tile* tile, void* workspace, size_t workspace_bytes,
                          void* stream);
/* How plm_gemm_chain_packed would make the linears of this chain wait for each other (host only,
 * no device needed): 0 none reads another; 2 per-wavefront waits on the producer's tile-done flags
 * (every linear after the first reads the one before it and every Y that is read starts on a
 * 128-byte boundary with ldy a multiple of 64 elements); 1 a grid barrier after every linear that
 * is read (any other pattern). A negative status for an invalid chain or tile. */
int plm_gemm_chain_packed_sync_mode(const plm_chain_gemm* gemms, int32_t count, const plm_tile* tile);

/*
 * Fills the derived fields of gemms[0..count) for the tile configuration (whose split_k is
 * ignored: each linear has its own) and returns the workspace bytes plm_gemm_chain needs, or a
 * negative status if the chain is invalid.
 */
int64_t plm_gemm_chain_prepare(plm_chain_gemm* gemms, int32_t count, int64_t M, const plm_tile* tile);

/*
 * Runs a chain of linears in one launch: the round's linears back to back (the reference's replayed
 * round calls fast_gemm 4L+1 times, plm/decoder.py:312-324). A linear with dep >= 0
 * starts each of its tiles as soon as the producer tiles covering that tile's K range are written,
 * so consecutive linears overlap. `host_gemms` is the prepared array, `device_gemms` a copy of it in
 * device memory (read by the kernel). Requirements as plm_gemm, plus: a consumed Y is 16-bit,
 * 128-byte aligned with ldy a multiple of 64, and no
 * Y overlaps another Y or any X or W of the chain except through dep. Workgroups wait on each
 * other, so the launch needs the device to itself (nothing else running on it).
 */
int plm_gemm_chain(int32_t dtype, const plm_chain_gemm* host_gemms, const plm_chain_gemm* device_gemms, int32_t count,
                   int64_t M, const plm_tile* tile, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes plm_gemm needs for this shape and tile (the reference's _partial_buffer,
 * plm/fast_gemm.py:70-79): PLM_WORKSPACE_COUNTER_BYTES plus the fp32 split partials. 0 when
 * split_k == 1. */
size_t plm_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, const plm_tile* tile);

/* 1 when a kernel is compiled for this tile at this M and K, else 0. */
int plm_gemm_tile_supported(int32_t dtype, int64_t M, int64_t K, const plm_tile* tile);

/*
 * Fused LM-head verify step: logits[R,V] = X[R,K] · W[V,K]^T are formed tile by tile and never
 * written to memory. For every row r:
 *   accept[r] = the acceptance rule's decision for pending[r] (enum plm_accept_rule):
 *               PLM_RULE_NUCLEUS, as nucleus_acceptance (plm/decoder.py:71-75): mass strictly
 *               above the proposal's own probability < p, or the proposal is the row maximum and
 *               p > 0; p <= 0 accepts nothing (exact matching, plm/decoder.py:115).
 *               PLM_RULE_FLOOR, as floor_acceptance (plm/decoder.py:78-82): logit[pending[r]] -
 *               logsumexp(logits[r]) > log(p), with p = epsilon.
 *               An id outside [0, V) is never accepted.
 *   argmax[r] = index of the row maximum, lowest index on ties (plm/decoder.py:362).
 * `round_mode` (enum plm_round_mode) fixes the logits the decision reads. Requirements as
 * plm_gemm. `tile` uses split_k == 1.
 */
int plm_lm_head_verify(int32_t dtype, const void* x, int64_t ldx, const void* w, int64_t ldw, int64_t R, int64_t V,
                       int64_t K, const int64_t* pending, int32_t rule, float p, int32_t round_mode, uint8_t* accept,
                       int64_t* argmax, const plm_tile* tile, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes plm_lm_head_verify and plm_lm_head_verify_packed need (counter area first, as for
 * plm_gemm). */
size_t plm_lm_head_verify_workspace_bytes(int64_t R, int64_t V, int64_t K, const plm_tile* tile);

/*
 * plm_lm_head_verify over a packed W (plm_pack_weight; the same decision rule and outputs) on the
 * packed GEMM's row-split pipeline: `tile` has k_waves = 1, split_k = 1, wave_frags 2 or 4 and
 * unroll 2, 4 or 8. The logits it decides on are bit for bit those plm_gemm_packed_f32out returns
 * with any such tile. Requirements: 1 <= R <= 64, K % 8 == 0, K <= 2^24, ldx % 8 == 0, x and
 * packed_w 16-byte aligned.
 */
int plm_lm_head_verify_packed(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, int64_t R, int64_t V,
                              int64_t K, const int64_t* pending, int32_t rule, float p, int32_t round_mode, uint8_t* accept,
                              int64_t* argmax, const plm_tile* tile, void* workspace, size_t workspace_bytes,
                              void* stream);

/*
 * plm_lm_head_verify_packed for a round whose verify rows decode through the auxiliary scheme
 * (RoundDecoder._steady_round, plm/decoder.py:316-322): only rows r < pending_rows decide on
 * pending[r] (the others are never accepted), and the logits of rows [0, logit_rows) are written
 * to `logits` (row stride ld_logits) in the model dtype, rounded from the same fp32 accumulators
 * the decision reads — the `logits[:K]` the decode takes (decoder.py:318-320), without writing the
 * other rows'. round_mode must be the model dtype's (PLM_ROUND_BF16 for bf16, PLM_ROUND_F16 for
 * fp16); ld_logits % 8 == 0, logits 16-byte aligned. Workspace as plm_lm_head_verify_workspace_bytes.
 */
int plm_lm_head_verify_packed_logits(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, int64_t R,
                                     int64_t V, int64_t K, const int64_t* pending, int64_t pending_rows, int32_t rule,
                                     float p, int32_t round_mode, uint8_t* accept, int64_t* argmax, void* logits,
                                     int64_t ld_logits, int64_t logit_rows, const plm_tile* tile, void* workspace,
                                     size_t workspace_bytes, void* stream);

/*
 * One round's bookkeeping after the verify step, on the device: RoundDecoder._epilogue
 * (plm/decoder.py:351-365) from the verify kernel's outputs. With k proposals per round
 * (round width k + k*k):
 *   widened[k-1]     the acceptance rule's decision for verify rows 0..k-2 (accept[] of the verify
 *                    step over those rows with the proposals as pending ids)
 *   hypotheses[k*k]  argmax of the proposal rows k..k+k*k-1 (argmax[] of the verify step)
 *   verify[k]        the verify rows' decoded tokens
 *   accepted[i]   = verify[i] == pending[i] || widened[i]; num_correct = leading accepted count
 *   out[base + i] = pending[i] for i < num_correct and verify[num_correct] at i == num_correct
 *                   (slots outside [0, out_len) are not written)
 *   round_sequence[min(step, sequence_len - 1)] = num_correct; step += 1 (both may be NULL)
 *   pending       = hypotheses[num_correct*k + 1 .. num_correct*k + k-1]   (updated in place)
 *   anchor[0] = verify[num_correct]; base += num_correct + 1; offset += num_correct + 1
 * `accepted` (k-1 bytes) and `num_correct` (one int64) are optional outputs (NULL: not written).
 * All pointers are device pointers; 1 <= k <= 64. One wavefront, no workspace.
 */
int plm_round_epilogue(int64_t k, const uint8_t* widened, const int64_t* hypotheses, const int64_t* verify,
                       int64_t* pending, int64_t* anchor, int64_t* out, int64_t out_len, int64_t* base,
                       int64_t* offset, int64_t* round_sequence, int64_t sequence_len, int64_t* sequence_step,
                       uint8_t* accepted, int64_t* num_correct, void* stream);

/*
 * The round's whole LM-head end in one verify launch pair: plm_lm_head_verify_packed over the round's
 * R = k + k*k rows (rows 0..k-2 decide on pending[0..k-2], the other rows propose nothing) with
 * plm_round_epilogue's bookkeeping run by the last workgroup after its final merge (widened = the
 * rule's decisions of rows 0..k-2, hypotheses = the argmax of rows k..R-1), so neither the
 * decisions nor the hypotheses make a round trip through memory. Arguments as those two entry
 * points; 1 <= k <= 7 (R <= 64); `accept[R]` and `argmax[R]` (every row's decision and argmax) are
 * optional outputs (NULL: not written), `pending` is read for the decisions and rewritten with
 * the next round's proposals. Workspace as plm_lm_head_verify_workspace_bytes(R, V, K, tile).
 */
int plm_round_verify_packed(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, int64_t k, int64_t V,
                            int64_t K, int32_t rule, float p, int32_t round_mode, const int64_t* verify,
                            int64_t* pending, int64_t* anchor, int64_t* out, int64_t out_len, int64_t* base,
                            int64_t* offset, int64_t* round_sequence, int64_t sequence_len, int64_t* sequence_step,
                            uint8_t* accept, int64_t* argmax, uint8_t* accepted, int64_t* num_correct,
                            const plm_tile* tile, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Gated LoRA linear over a packed W (GatedLoraMethod.apply, plm/gated_lora.py:45-57): Y = X W^T for
 * every row, and for rows m >= gated_from the rank-r correction of the rows that carry the adapter:
 *   h = round(X[gated_from:] A^T)                 [M - gated_from, shards*rank]  (54)
 *   Y[m, n] = round(round(X W^T)[m, n] + h[m - gated_from, s*rank .. +rank] . B[n, :])   (55-58)
 * with A the shards' down-projections stacked ([shards*rank, K], packed by plm_pack_weight), B the
 * shards' up-projections stacked by output column (lora_b: [N, rank] row-major), and shard s owning
 * the next shard_sizes[s] output columns (1 <= shards <= 3: a fused q/k/v or gate/up projection;
 * rank a multiple of 8, 8 <= rank <= 1024; lora_b 16-byte aligned). One launch on `tile`: its first
 * workgroups form h (every row, into the workspace), the others run the base GEMM and, once every h
 * tile is written, add the correction to their gated rows before storing them. The workgroups wait
 * on each other (bounded: a wait that gives up sets the int at PLM_WORKSPACE_ERROR_INDEX, and the
 * launch's results are then invalid and the workspace's counter area must be zeroed again before
 * its next use); two such launches must not run at once on one workspace. gated_from >= M is
 * plm_gemm_packed. Workspace: plm_gemm_packed_lora_workspace_bytes.
 */
int plm_gemm_packed_lora(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, void* y, int64_t ldy,
                         int64_t M, int64_t N, int64_t K, int64_t gated_from, const void* packed_a, const void* lora_b,
                         int64_t rank, int32_t shards, const int64_t* shard_sizes, const plm_tile* tile,
                         void* workspace, size_t workspace_bytes, void* stream);
size_t plm_gemm_packed_lora_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t gated_from, int64_t rank,
                                            int32_t shards, const plm_tile* tile);

/*
 * A fused gate/up projection followed by its activation, in one launch. Replaces two launches of
 * the reference's Llama-style rounds: the gate_up_proj GEMM (plm/fast_gemm.py:104-110, or F.linear)
 * and vLLM 0.26.0's SiluAndMul on its output (uv.lock:3123-3125; the rounds run with
 * enforce_eager, plm/decoder.py:37, so its silu_and_mul kernel), with the same roundings:
 *   Y[m, n] = round(round(silu(g)) * u),  g = round((X W^T)[m, n]),  u = round((X W^T)[m, N/2 + n])
 * for 0 <= n < N/2, silu(g) = g / (1 + e^-g) in fp32, round() to the model dtype. `packed_w` is
 * W[N, K] (gate rows 0..N/2-1, up rows N/2..N-1) packed with the two halves interleaved by 16-row
 * fragment — fragment 2j = gate rows [16j, 16j+16), fragment 2j+1 = up rows [16j, 16j+16) — i.e.
 * plm_pack_weight of the rows in that order. N a multiple of 32, tile.wave_frags 2 or 4, Y [M, N/2]
 * with ldy % 4 == 0 and y 8-byte aligned; otherwise as plm_gemm_packed (M <= 128). Workspace as
 * plm_gemm_packed_workspace_bytes(M, N, K, tile).
 */
int plm_gemm_packed_silu_mul(int32_t dtype, const void* x, int64_t ldx, const void* packed_w, void* y, int64_t ldy,
                             int64_t M, int64_t N, int64_t K, const plm_tile* tile, void* workspace,
                             size_t workspace_bytes, void* stream);

/*
 * The verify rows' auxiliary decode, logit-Voronoi scheme with the `iterate` engine
 * (LogitVoronoiAuxiliary.decode_unmasked, plm/auxiliary.py:67-75, over Voronoi.assign,
 * plm/iterate.py:322-342). A problem is one row of logits[n_problems, n_vocab] (bf16 or fp16,
 * row stride ld_logits); `table` is the engine's contiguous [n_vocab, n_items] cost table in the
 * same dtype (auxiliary.py:62-63: -(auxiliary_vocabulary . W^T)^T).
 *
 * Sizes (the reference's limits, auxiliary.py:24-25 and iterate.py:298-300, and this build's):
 * n_targets and k powers of two, k <= n_targets <= 128, k <= 16; n_items a power of two in
 * [64, 8192] with k * max(1, n_items / 1024) <= 32; n_targets <= n_vocab <= 65528;
 * 1 <= n_problems <= 65535. All pointers are device pointers. `table` has n_vocab rows; token ids
 * handed in (tokens[]) are clamped into [0, n_vocab), so no input reads outside it.
 *
 * Ties the reference leaves to torch (topk, an unstable argsort) are fixed: the shortlist is the
 * n_targets largest logits by (value descending, token id ascending); equal quota remainders rank
 * by shortlist position. The fit's per-token loads are exact integer sums of the weights in units
 * of 2^-31 (no float atomics), so every output is reproducible bit for bit.
 */

/* Voronoi.shortlist + spread + prior (iterate.py:248-290) in one launch: tokens[N, M] (int64),
 * counts[N, M] (int64, summing to n_items per row), unit[N], prior[N, M] (float; weight is the
 * prior's weight, 0.1 in assign); values[N, M] (the shortlisted logits) and normaliser[N]
 * (max + log sum exp) are optional (NULL: not written). */
int plm_voronoi_shortlist(int32_t dtype, const void* logits, int64_t ld_logits, const void* table, int64_t n_problems,
                          int64_t n_vocab, int64_t n_items, int64_t n_targets, float weight, int64_t* tokens,
                          int64_t* counts, float* values, float* unit, float* prior, float* normaliser, void* stream);

/* Voronoi.spread (iterate.py:275-284): unit[N] = mean over the first min(sample, 64, n_items)
 * items of the gap between the worst and best of the row's targets, the gap in the table's dtype.
 * Voronoi.prior (iterate.py:286-290): prior[N, M] = -weight * unit * log(max(counts / n_items,
 * 1e-9)) for counts > 0, else 1000 * unit. plm_voronoi_shortlist computes both in its launch. */
int plm_voronoi_spread(int32_t dtype, const void* table, int64_t n_vocab, int64_t n_items, const int64_t* tokens,
                       int64_t n_problems, int64_t n_targets, int64_t sample, float* unit, void* stream);
int plm_voronoi_prior(const int64_t* counts, const float* unit, int64_t n_problems, int64_t n_targets, int64_t n_items,
                      float weight, float* prior, void* stream);

/* condense (iterate.py:195-211): key[N, k, n_items] (int32), each item's k smallest packed keys of
 * table[tokens[m], item] + offset[m] (the cost's order-preserving bits with the low 7 replaced by
 * m), ascending. */
int plm_voronoi_condense(int32_t dtype, const void* table, int64_t n_vocab, int64_t n_items, const int64_t* tokens,
                         const float* offset, int64_t n_problems, int64_t n_targets, int64_t k, int32_t* key,
                         void* stream);

/* Voronoi.fit (iterate.py:292-312): `iterations` annealed Sinkhorn sweeps from temperature
 * epsilon * unit down by (endpoint / epsilon)^(1/iterations) per sweep, each factor's step clamped
 * to +-limit * unit and over-relaxed by `relax`; out[N, M] = offset + correction. The reference's
 * defaults are relax 1.9, endpoint 0.0087, limit 0.25. */
int plm_voronoi_fit(const int32_t* key, const int64_t* counts, const float* offset, const float* unit,
                    int64_t n_problems, int64_t n_targets, int64_t k, int64_t n_items, int64_t iterations,
                    float epsilon, float relax, float endpoint, float limit, float* out, void* stream);

/* Voronoi.argmin (iterate.py:314-320): sigma[N, n_items] = argmin_m table[tokens[m], a] + bias[m]
 * (int64, lowest m on ties). */
int plm_voronoi_argmin(int32_t dtype, const void* table, int64_t n_vocab, int64_t n_items, const int64_t* tokens,
                       const float* bias, int64_t n_problems, int64_t n_targets, int64_t* sigma, void* stream);

/*
 * Voronoi.assign (iterate.py:322-342) and decode_unmasked (auxiliary.py:67-75): shortlist, then
 * `rounds` of condense + fit (the first from epsilon, later ones from epsilon * refocus), all on
 * `stream`. Outputs, each optional (NULL: not written): decoded[N] = tokens[sigma[values[n]]] with
 * values clamped to [0, n_items) (values and decoded go together); tokens_out[N, M], counts_out[N, M],
 * bias_out[N, M] (the fitted factors); sigma[N, n_items] (one more launch). The reference's defaults
 * are n_targets 128, k 8, rounds 2, iterations 12, weight 0.1, epsilon 0.15, refocus 0.35, relax 1.9,
 * endpoint 0.0087, limit 0.25. Workspace: plm_voronoi_assign_workspace_bytes, 16-byte aligned; its
 * counter area is not touched (the scratch after it is), so the GEMMs' workspace can be shared.
 */
int plm_voronoi_assign(int32_t dtype, const void* logits, int64_t ld_logits, const void* table, int64_t n_problems,
                       int64_t n_vocab, int64_t n_items, int64_t n_targets, int64_t k, int64_t rounds,
                       int64_t iterations, float weight, float epsilon, float refocus, float relax, float endpoint,
                       float limit, const int64_t* values, int64_t* decoded, int64_t* tokens_out,
                       int64_t* counts_out, float* bias_out, int64_t* sigma, void* workspace, size_t workspace_bytes,
                       void* stream);
size_t plm_voronoi_assign_workspace_bytes(int64_t n_problems, int64_t n_targets, int64_t k, int64_t n_items);

/* Human-readable name of a status code. */
const char* plm_status_string(int32_t status);

#ifdef __cplusplus
}
#endif

#endif /* PLM_AMD_H */
