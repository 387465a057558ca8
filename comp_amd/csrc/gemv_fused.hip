// Fused quantize-and-GEMV launches (f32 activations in); the kernel template is in gemv_kernel.h.
#include "gemv_kernel.h"

namespace komp {

hipError_t launch_gemv_fused(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  switch (c.fmt) {
    case FMT_Q4_0:
      if (q4_lean_eligible(c, p)) return launch_gemv_q4_lean(c, p, stream);
      return gemv_impl::by_mode<FMT_Q4_0, true>(c, p, stream);
    case FMT_TQ2_0:
      if (tq2_lean_eligible(c, p)) return launch_gemv_tq2_lean(c, p, stream);
      return gemv_impl::by_mode<FMT_TQ2_0, true>(c, p, stream);
    default: return launch_gemv_more_fused(c, p, stream);  // Q8_0, IQ4_NL (gemv_more_fused.hip)
  }
}

}  // namespace komp
