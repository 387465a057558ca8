// The Q8_0 lean kernels' unfused instantiations, their plan check and their LDS size (the kernels: gemv_q8.h; the
// fused instantiations: gemv_q8_fused.hip).
#include "gemv_q8.h"

namespace komp {

size_t q8_lean_lds_bytes(int lpr, int nb, int mc, int k) {
  const int bstep = (lpr / 2) * nb;
  const int64_t nblk = k / 32;
  const int64_t pad = (nblk + bstep - 1) / bstep * bstep;
  return static_cast<size_t>(mc) * pad * (16 + 16 + 4);  // two 16-byte halves and d_x per block
}

bool q8_lean_eligible(const GemvCall& c, const GemvPlan& p) {
  // dp4a mode, one column with nb up to 8, two or three with nb up to 4 (the instantiations)
  const bool nb_ok = p.nb == 1 || p.nb == 2 || p.nb == 4 || (p.nb == 8 && c.m == 1);
  return c.fmt == FMT_Q8_0 && c.m >= 1 && c.m <= 3 && c.mode == MODE_DP4A && p.lpr_log2 >= 2 && p.lpr_log2 <= 6 &&
         nb_ok && p.waves >= 1 && p.waves <= 16 && p.rows_per_wave == (64 >> p.lpr_log2) * p.passes &&
         lean_strides_fit(c, 64 >> p.lpr_log2) && q8_lean_lds_bytes(1 << p.lpr_log2, p.nb, c.m, c.k) <= gemv_q8::kLdsLimit;
}

hipError_t launch_gemv_q8_lean(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  if (p.waves * p.rows_per_wave < p.block_n) return hipErrorInvalidConfiguration;
  if (c.x != nullptr) return launch_gemv_q8_lean_fused(c, p, stream);
  return gemv_q8::launch_fused<false>(c, p, stream);
}

}  // namespace komp
