// Round bookkeeping after the verify step on gfx950 (plm/decoder.py:351-365), in one wavefront
// (the arithmetic is in epilogue.h, shared with the fused verify): `widened` is the acceptance
// rule's decision for the first k-1 verify rows and `hypotheses` the argmax of the k*k proposal
// rows, both as the verify kernel writes them.
#include <hip/hip_runtime.h>

#include "epilogue.h"
#include "plm_amd.h"

namespace plm {

__global__ __launch_bounds__(64) void round_epilogue_kernel(RoundEpilogue e, const uint8_t* widened,
                                                            const int64_t* hypotheses) {
  const int lane = threadIdx.x;
  const bool w = lane < e.k - 1 && widened[lane] != 0;
  round_epilogue_wave(e, lane, w, [&](int j) { return hypotheses[j]; });
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
  plm::RoundEpilogue e{};
  e.k = static_cast<int>(k);
  e.verify = verify;
  e.pending = pending;
  e.anchor = anchor;
  e.out = out;
  e.out_len = out_len;
  e.base = base;
  e.offset = offset;
  e.round_sequence = round_sequence;
  e.sequence_len = sequence_len;
  e.sequence_step = sequence_step;
  e.accepted = accepted;
  e.num_correct = num_correct;
  hipLaunchKernelGGL(plm::round_epilogue_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), e, widened,
                     hypotheses);
  return hipGetLastError() == hipSuccess ? PLM_OK : PLM_ERR_LAUNCH;
}

}  // extern "C"
