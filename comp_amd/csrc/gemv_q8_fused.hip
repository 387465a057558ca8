// The Q8_0 lean kernels' fused instantiations (f32 activations in, quantized to q8_0 in every workgroup; the kernels:
// gemv_q8.h).
#include "gemv_q8.h"

namespace komp {

hipError_t launch_gemv_q8_lean_fused(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  return gemv_q8::launch_fused<true>(c, p, stream);
}

}  // namespace komp
