// Round bookkeeping after the verify step (plm/decoder.py:351-365), for one wavefront: used by the
// standalone epilogue kernel (csrc/epilogue.hip) and by the fused verify's last merge
// (csrc/verify.hip). With k proposals per round:
//
//   accepted[i]  = verify[i] == pending[i] || widened[i]                     (i < k-1, 354)
//   num_correct  = length of the leading run of accepted proposals           (cumprod().sum(), 355)
//   picked       = verify[num_correct]                                       (357)
//   out[base+i]  = pending[i] for i < num_correct, picked at i == num_correct (358-359)
//   round_sequence[min(step, capacity-1)] = num_correct; step += 1          (360-361)
//   pending      = hypotheses[num_correct][1:k]                             (362)
//   anchor = picked; base += num_correct + 1; offset += num_correct + 1     (363-365)
//
// Lane i owns proposal i (k <= 64); the leading run is the position of the lowest rejected lane in
// a wavefront ballot.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace plm {

struct RoundEpilogue {
  int k;
  const int64_t* verify;   // [k] the verify rows' decoded tokens
  int64_t* pending;        // [k-1] this round's proposals in, the next round's out
  int64_t* anchor;         // [1]
  int64_t* out;            // [out_len] committed tokens; slots outside it are not written
  int64_t out_len;
  int64_t* base;           // [1]
  int64_t* offset;         // [1]
  int64_t* round_sequence;  // [sequence_len] or nullptr (then sequence_step too)
  int64_t sequence_len;
  int64_t* sequence_step;  // [1]
  uint8_t* accepted;       // [k-1] or nullptr
  int64_t* num_correct;    // [1] or nullptr
};

// Called by all 64 lanes of one wavefront. `widened` is the acceptance rule's decision for verify
// row `lane` (read for lanes < k-1); `hyp(j)` returns entry j of the k*k proposal-row argmaxes and
// is called by every lane with the same control flow (it may be a cross-lane read), with
// 1 <= j < k*k.
template <class Hyp>
__device__ __forceinline__ void round_epilogue_wave(const RoundEpilogue& e, int lane, bool widened, Hyp hyp) {
  const int k = e.k;
  const bool proposal = lane < k - 1;
  const int64_t proposed = proposal ? e.pending[lane] : 0;
  const bool acc = proposal && (e.verify[lane] == proposed || widened);
  const unsigned long long rejected = __ballot(proposal && !acc);
  const int nc = rejected != 0ull ? __ffsll(static_cast<long long>(rejected)) - 1 : k - 1;
  const int64_t picked = e.verify[nc];
  const int64_t base = *e.base;
  const int64_t next = k > 1 ? hyp(nc * k + 1 + (proposal ? lane : 0)) : 0;
  // Every lane has read pending, base and verify before any lane writes below (one wavefront,
  // loads return before the ballot's result is used).
  if (lane < k) {
    const int64_t slot = base + lane;
    if (slot >= 0 && slot < e.out_len) {
      if (lane < nc) e.out[slot] = proposed;
      else if (lane == nc) e.out[slot] = picked;
    }
  }
  if (proposal) {
    e.pending[lane] = next;
    if (e.accepted != nullptr) e.accepted[lane] = acc ? 1 : 0;
  }
  if (lane == 0) {
    *e.anchor = picked;
    *e.base = base + nc + 1;
    *e.offset += nc + 1;
    if (e.num_correct != nullptr) *e.num_correct = nc;
    if (e.round_sequence != nullptr) {
      const int64_t step = *e.sequence_step;
      e.round_sequence[step < e.sequence_len - 1 ? step : e.sequence_len - 1] = nc;
      *e.sequence_step = step + 1;
    }
  }
}

}  // namespace plm
