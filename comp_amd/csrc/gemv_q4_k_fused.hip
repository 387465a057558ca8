// Fused quantize-and-GEMV launches for Q4_K weights (f32 activations in, quantized to q8_K in every workgroup).
#include "gemv_kernel.h"

namespace komp {

hipError_t launch_gemv_q4_k_fused(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  return gemv_impl::by_mode<FMT_Q4_K, true>(c, p, stream);
}

}  // namespace komp
