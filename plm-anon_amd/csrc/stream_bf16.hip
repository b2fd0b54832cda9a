// bf16 instantiations of the streaming GEMM (one translation unit per dtype so they build in parallel).
#include "stream_gemm.h"

namespace plm {

hipError_t stream_dispatch_bf16(StreamArgs& a, int nf, int cus, hipStream_t s, bool dry) {
  return stream_dispatch<DT_BF16>(a, nf, cus, s, dry);
}

}  // namespace plm
