// bf16 instantiations of the packed-weight GEMM (one translation unit per dtype so they build in parallel).
#include "packed_gemm.h"

namespace plm {

hipError_t packed_dispatch_bf16(PackedArgs& a, int nf, int d, int cus, hipStream_t s, bool dry) {
  return packed_dispatch<DT_BF16>(a, nf, d, cus, s, dry);
}

}  // namespace plm
