// Round bookkeeping after the verify step on gfx950 (plm/decoder.py:351-365), in one wavefront:
//
//   accepted[i]  = verify[i] == pending[i] || widened[i]                     (i < k-1, 354)
//   num_correct  = length of the leading run of accepted proposals           (cumprod().sum(), 355)
//   picked       = verify[num_correct]                                       (357)
//   out[base+i]  = pending[i] for i < num_correct, picked at i == num_correct (358-359)
//   round_sequence[min(step, capacity-1)] = num_correct; step += 1          (360-361)
//   pending      = hypotheses[num_correct][1:k]                             (362)
//   anchor = picked; base += num_correct + 1; offset += num_correct + 1     (363-365)
//
// `widened` is the acceptance rule's decision for the first k-1 verify rows and `hypotheses` the
// argmax of the k*k proposal rows, both as the fused verify kernel writes them. Lane i owns slot i
// (k <= 64); the leading run is the position of the lowest rejected lane in a wavefront ballot.
#include <hip/hip_runtime.h>

#include "plm_amd.h"

namespace plm {

struct EpilogueArgs {
  int k;
  const uint8_t* widened;
  const int64_t* hypotheses;
  const int64_t* verify;
  int64_t* pending;
  int64_t* anchor;
  int64_t* out;
  int64_t out_len;
  int64_t* base;
  int64_t* offset;
  int64_t* round_sequence;
  int64_t sequence_len;
  int64_t* sequence_step;
  uint8_t* accepted;
  int64_t* num_correct;
};

__global__ __launch_bounds__(64) void round_epilogue_kernel(EpilogueArgs a) {
  const int i = threadIdx.x;
  const int k = a.k;
  const bool proposal = i < k - 1;
  const int64_t proposed = proposal ? a.pending[i] : 0;
  const bool acc = proposal && (a.verify[i] == proposed || a.widened[i] != 0);
  const unsigned long long rejected = __ballot(proposal && !acc);
  const int nc = rejected != 0ull ? __ffsll(static_cast<long long>(rejected)) - 1 : k - 1;
  const int64_t picked = a.verify[nc];
  const int64_t base = *a.base;
  // Every lane has read pending, base and verify before any lane writes below (one wavefront,
  // loads return before the ballot's result is used).
  if (i < k) {
    const int64_t slot = base + i;
    if (slot >= 0 && slot < a.out_len) {
      if (i < nc) a.out[slot] = proposed;
      else if (i == nc) a.out[slot] = picked;
    }
  }
  if (proposal) {
    a.pending[i] = a.hypotheses[static_cast<int64_t>(nc) * k + 1 + i];
    if (a.accepted != nullptr) a.accepted[i] = acc ? 1 : 0;
  }
  if (i == 0) {
    *a.anchor = picked;
    *a.base = base + nc + 1;
    *a.offset += nc + 1;
    if (a.num_correct != nullptr) *a.num_correct = nc;
    if (a.round_sequence != nullptr) {
      const int64_t step = *a.sequence_step;
      a.round_sequence[step < a.sequence_len - 1 ? step : a.sequence_len - 1] = nc;
      *a.sequence_step = step + 1;
    }
  }
}

}  // namespace plm

extern "C" {

int plm_round_epilogue(int64_t k, const uint8_t* widened, const int64_t* hypotheses, const int64_t* verify,
                       int64_t* pending, int64_t* anchor, int64_t* out, int64_t out_len, int64_t* base,
                       int64_t* offset, int64_t* round_sequence, int64_t sequence_len, int64_t* sequence_step,
                       uint8_t* accepted, int64_t* num_correct, void* stream) {
  if (k < 1 || k > 64 || out_len < 0) return PLM_ERR_ARGUMENT;
  if (hypotheses == nullptr || verify == nullptr || anchor == nullptr || out == nullptr || base == nullptr ||
      offset == nullptr)
    return PLM_ERR_ARGUMENT;
  if (k > 1 && (widened == nullptr || pending == nullptr)) return PLM_ERR_ARGUMENT;
  if ((round_sequence == nullptr) != (sequence_step == nullptr)) return PLM_ERR_ARGUMENT;
  if (round_sequence != nullptr && sequence_len < 1) return PLM_ERR_ARGUMENT;
  plm::EpilogueArgs a{};
  a.k = static_cast<int>(k);
  a.widened = widened;
  a.hypotheses = hypotheses;
  a.verify = verify;
  a.pending = pending;
  a.anchor = anchor;
  a.out = out;
  a.out_len = out_len;
  a.base = base;
  a.offset = offset;
  a.round_sequence = round_sequence;
  a.sequence_len = sequence_len;
  a.sequence_step = sequence_step;
  a.accepted = accepted;
  a.num_correct = num_correct;
  hipLaunchKernelGGL(plm::round_epilogue_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), a);
  return hipGetLastError() == hipSuccess ? PLM_OK : PLM_ERR_LAUNCH;
}

}  // extern "C"
