// The Q4_0 / IQ4_NL lean kernels' dp4a instantiations, their plan checks and their LDS sizes (the kernels:
// gemv_q4.h).
#include "gemv_q4.h"

namespace komp {

size_t q4_lean_lds_bytes(int g, int nb, int mc, int k, bool bytes) {
  const int bstep = g * nb;
  const int64_t nblk = k / 32;
  const int64_t pad = (nblk + bstep - 1) / bstep * bstep;
  return static_cast<size_t>(mc) * pad * ((bytes ? 2 : 1) * (16 + 16) + 8);  // bytes mode: 16-bit activations
}

bool q4_lean_eligible(const GemvCall& c, const GemvPlan& p) {
  // one column with nb up to 8, two or three columns with nb up to 4 (the instantiations); 1024 threads hold at most
  // 128 VGPRs, which three columns at nb 4 stay within.  dp4a mode, and Q4_0 in bytes mode
  const bool nb_ok = p.nb == 1 || p.nb == 2 || p.nb == 4 || (p.nb == 8 && c.m == 1);
  const bool mode_ok = c.mode == MODE_DP4A || (c.mode == MODE_BYTES && c.fmt == FMT_Q4_0);
  return (c.fmt == FMT_Q4_0 || c.fmt == FMT_IQ4_NL) && c.m >= 1 && c.m <= 3 && mode_ok && p.lpr_log2 >= 2 &&
         p.lpr_log2 <= 6 && nb_ok && p.waves >= 1 && p.waves <= 16 && p.rows_per_wave == (64 >> p.lpr_log2) * p.passes &&
         lean_strides_fit(c, 64 >> p.lpr_log2) &&
         q4_lean_lds_bytes(1 << p.lpr_log2, p.nb, c.m, c.k, c.mode == MODE_BYTES) <= gemv_impl::kLdsLimit;
}

hipError_t launch_gemv_q4_lean(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  if (p.waves * p.rows_per_wave < p.block_n) return hipErrorInvalidConfiguration;
  if (c.mode == MODE_BYTES) return launch_gemv_q4_lean_bytes(c, p, stream);
  return c.fmt == FMT_Q4_0 ? gemv_q4::launch_mode<FMT_Q4_0, false>(c, p, stream)
                           : gemv_q4::launch_mode<FMT_IQ4_NL, false>(c, p, stream);
}

}  // namespace komp
