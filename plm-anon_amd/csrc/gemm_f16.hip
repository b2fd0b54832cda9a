// f16 instantiations of the skinny GEMM (one translation unit per dtype so they build in parallel).
#include "gemm_kernel.h"

namespace plm {

hipError_t gemm_dispatch_f16(const GemmArgs& a, const plm_tile& t, hipStream_t s, bool dry) {
  return gemm_dispatch<DT_F16>(a, t, s, dry);
}

}  // namespace plm
