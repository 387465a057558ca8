// Unfused GEMV launches (q8 activations in) and the shared helpers; the kernel template is in gemv_kernel.h.
#include "gemv_kernel.h"

namespace komp {

size_t gemv_lds_bytes(int fmt, int m, int k) {
  if (fmt == FMT_Q4_K) return static_cast<size_t>(m) * (k / 256) * (256 + 8 + 32);  // + 8 int32 sub-block sums
  if (fmt != FMT_TQ2_0) return static_cast<size_t>(m) * (k / 32) * (32 + 8);
  return static_cast<size_t>(m) * (k / 256) * (256 + 8);
}

hipError_t launch_gemv(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  if (c.x != nullptr) return launch_gemv_fused(c, p, stream);
  switch (c.fmt) {
    case FMT_Q4_0:
      if (q4_lean_eligible(c, p)) return launch_gemv_q4_lean(c, p, stream);
      return gemv_impl::by_mode<FMT_Q4_0, false>(c, p, stream);
    case FMT_TQ2_0:
      if (tq2_lean_eligible(c, p)) return launch_gemv_tq2_lean(c, p, stream);
      return gemv_impl::by_mode<FMT_TQ2_0, false>(c, p, stream);
    default: return launch_gemv_more(c, p, stream);  // Q8_0, IQ4_NL (gemv_more.hip)
  }
}

}  // namespace komp
