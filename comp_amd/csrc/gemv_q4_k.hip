// GEMV launches for Q4_K weights (q8_K activations in: unfused, and fused with the quantizer); the kernel template is
// in gemv_kernel.h.  A translation unit of their own, so the library's instantiations compile in parallel.
#include "gemv_kernel.h"

namespace komp {

hipError_t launch_gemv_q4_k(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  return gemv_impl::by_mode<FMT_Q4_K, false>(c, p, stream);
}

}  // namespace komp
