// bf16 instantiations of the packed-weight GEMM with workgroup layout KW = 1
// (rows split across the four wavefronts); one translation unit per (dtype, layout) so that they build in
// parallel. Each also holds the layout's gated-LoRA and SiLU-and-multiply launches.
#include "packed_gemm.h"

namespace plm {

hipError_t packed_dispatch_bf16_k1(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry) {
  return packed_dispatch_kw<DT_BF16, 1>(a, nf, d, cus, s, dry);
}

hipError_t packed_dispatch_lora_bf16_k1(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry) {
  return packed_dispatch_kw<DT_BF16, 1, kEpiLora>(a, nf, d, cus, s, dry);
}

hipError_t packed_dispatch_act_bf16_k1(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry) {
  return packed_dispatch_kw<DT_BF16, 1, kEpiAct>(a, nf, d, cus, s, dry);
}

}  // namespace plm
