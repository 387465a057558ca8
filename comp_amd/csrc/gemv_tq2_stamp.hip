// The TQ2_0 lean kernels' stamped instantiations (gemv_tq2.h, STAMP): dp4a, one pass and one K step.  Only the
// tuning harness's span timing runs them (komp_stamps_begin / komp_stamps_end).
#include "gemv_tq2.h"

namespace komp {

hipError_t launch_gemv_tq2_lean_stamped(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  return gemv_tq2::launch_mode<false, true>(c, p, stream);
}

}  // namespace komp
