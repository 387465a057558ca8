// The Q4_0 lean kernels' bytes-mode instantiations (the kernels: gemv_q4.h), in a translation unit of their own so
// that they compile beside the dp4a ones.
#include "gemv_q4.h"

namespace komp {

hipError_t launch_gemv_q4_lean_bytes(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  return gemv_q4::launch_mode<FMT_Q4_0, true>(c, p, stream);
}

}  // namespace komp
