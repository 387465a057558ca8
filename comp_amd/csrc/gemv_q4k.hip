// The Q4_K lean kernels' unfused instantiations, their plan check and their LDS size (the kernels: gemv_q4k.h; the
// fused instantiations: gemv_q4k_fused.hip).
#include "gemv_q4k.h"

namespace komp {

size_t q4k_lean_lds_bytes(int lpr, int nb, int mc, int k) {
  const int bstep = (lpr / 4) * nb;
  const int64_t nblk = k / 256;
  const int64_t pad = (nblk + bstep - 1) / bstep * bstep;
  return static_cast<size_t>(mc) * pad * (gemv_q4k::kBlockStride + 8 * 4 + 4);  // values, sub-block sums, d_x
}

bool q4k_lean_eligible(const GemvCall& c, const GemvPlan& p) {
  // dp4a mode, 1-3 columns, nb 1, 2 or 4 (the instantiations: 12 VGPRs of weights and scales per slot), 16-byte
  // aligned scale planes (each block's 16-byte entry is one load)
  bool ws_aligned = reinterpret_cast<uintptr_t>(c.ws) % 16 == 0;
  for (int i = 0; c.nseg > 1 && i < c.nseg; ++i) ws_aligned = ws_aligned && reinterpret_cast<uintptr_t>(c.segs.ws[i]) % 16 == 0;
  return c.fmt == FMT_Q4_K && c.m >= 1 && c.m <= 3 && c.mode == MODE_DP4A && ws_aligned && p.lpr_log2 >= 2 &&
         p.lpr_log2 <= 6 && (p.nb == 1 || p.nb == 2 || p.nb == 4) && p.waves >= 1 && p.waves <= 16 &&
         p.rows_per_wave == (64 >> p.lpr_log2) * p.passes && lean_strides_fit(c, 64 >> p.lpr_log2) &&
         q4k_lean_lds_bytes(1 << p.lpr_log2, p.nb, c.m, c.k) <= gemv_q4k::kLdsLimit;
}

hipError_t launch_gemv_q4k_lean(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  if (p.waves * p.rows_per_wave < p.block_n) return hipErrorInvalidConfiguration;
  if (c.x != nullptr) return launch_gemv_q4k_lean_fused(c, p, stream);
  return gemv_q4k::launch_fused<false>(c, p, stream);
}

}  // namespace komp
