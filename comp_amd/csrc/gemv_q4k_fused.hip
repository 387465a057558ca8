// The Q4_K lean kernels' fused instantiations (f32 activations in, quantized to q8_K in every workgroup; the kernels:
// gemv_q4k.h).
#include "gemv_q4k.h"

namespace komp {

hipError_t launch_gemv_q4k_lean_fused(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  return gemv_q4k::launch_fused<true>(c, p, stream);
}

}  // namespace komp
