// Fused quantize-and-GEMV launches (f32 activations in); the kernel template is in gemv_kernel.h.
#include "gemv_kernel.h"

namespace komp {

hipError_t launch_gemv_fused(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  if (c.fmt == FMT_Q4_0) return gemv_impl::by_mode<FMT_Q4_0, true>(c, p, stream);
  return gemv_impl::by_mode<FMT_TQ2_0, true>(c, p, stream);
}

}  // namespace komp
