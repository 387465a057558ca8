// Fused quantize-and-GEMV launches for the Q8_0 and IQ4_NL weight formats (f32 activations in); the kernel template
// is in gemv_kernel.h.
#include "gemv_kernel.h"

namespace komp {

hipError_t launch_gemv_more_fused(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  if (c.fmt == FMT_Q8_0)
    return q8_lean_eligible(c, p) ? launch_gemv_q8_lean(c, p, stream) : gemv_impl::by_mode<FMT_Q8_0, true>(c, p, stream);
  if (c.fmt == FMT_IQ4_NL)
    return q4_lean_eligible(c, p) ? launch_gemv_q4_lean(c, p, stream) : gemv_impl::by_mode<FMT_IQ4_NL, true>(c, p, stream);
  if (c.fmt == FMT_Q4_K)
    return q4k_lean_eligible(c, p) ? launch_gemv_q4k_lean(c, p, stream) : launch_gemv_q4_k_fused(c, p, stream);
  return hipErrorInvalidValue;
}

}  // namespace komp
