// The TQ2_0 lean kernels' bytes-mode instantiations (the kernels: gemv_tq2.h), in a translation unit of their own so
// that they compile beside the dp4a ones.
#include "gemv_tq2.h"

namespace komp {

hipError_t launch_gemv_tq2_lean_bytes(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  return gemv_tq2::launch_mode<true>(c, p, stream);
}

}  // namespace komp
