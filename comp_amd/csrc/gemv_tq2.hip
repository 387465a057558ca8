// The TQ2_0 lean kernels' dp4a instantiations, their plan checks and their LDS sizes (the kernels: gemv_tq2.h).
#include "gemv_tq2.h"

namespace komp {

namespace {
size_t tq2_staged_bytes(int lpr, int nb, int mc, int k, bool bytes) {  // bytes mode: two planes of 16-bit values
  const int bstep = (lpr / 4) * nb;
  const int64_t nblk = k / 256;
  const int64_t pad = (nblk + bstep - 1) / bstep * bstep;
  return static_cast<size_t>(mc) * pad * ((bytes ? 2 : 1) * gemv_tq2::kBlockStride + 8);
}
size_t tq2_raw_bytes(int mc, int k, bool fused) {  // the columns as they are in memory (f32, or q8 bytes and d_x)
  return fused ? static_cast<size_t>(mc) * k * 4 : static_cast<size_t>(mc) * k + static_cast<size_t>(mc) * (k / 256) * 4;
}
}  // namespace

bool tq2_lean_dma(int lpr, int nb, int mc, int k, bool fused, int threads, bool bytes) {
  // q8 columns in dp4a mode only.  Fused, every workgroup reads all of the f32 columns (21 MB from L2 over the chip at 2560x6912
  // and 3 columns), and through LDS that cost more than the register passes, copied ahead of the weights (3 columns
  // 5.7 -> 6.8 us, 2 columns 4.5 -> 5.4) or behind them (7.1, 5.6); with q8 in, 3 columns 4.8 -> 4.6, 2 columns
  // 4.2 -> 3.9
  return !fused && !bytes && mc > 1 && static_cast<int64_t>(mc) * (k / 256) * 16 > threads &&
         ((tq2_staged_bytes(lpr, nb, mc, k, false) + 15) & ~size_t{15}) + tq2_raw_bytes(mc, k, fused) <= gemv_tq2::kLdsLimit;
}

size_t tq2_lean_lds_bytes(int lpr, int nb, int mc, int k, bool fused, int threads, bool bytes) {
  const size_t staged = tq2_staged_bytes(lpr, nb, mc, k, bytes);
  if (!tq2_lean_dma(lpr, nb, mc, k, fused, threads, bytes)) return staged;
  return ((staged + 15) & ~size_t{15}) + tq2_raw_bytes(mc, k, fused);  // the raw columns follow, 16-byte aligned
}

bool tq2_lean_eligible(const GemvCall& c, const GemvPlan& p) {
  // one column with nb up to 8, two or three with nb up to 4 (the instantiations); dp4a and bytes modes
  const bool nb_ok = p.nb == 1 || p.nb == 2 || p.nb == 4 || (p.nb == 8 && c.m == 1);
  return c.fmt == FMT_TQ2_0 && c.m >= 1 && c.m <= 3 && (c.mode == MODE_DP4A || c.mode == MODE_BYTES) &&
         p.lpr_log2 >= 2 && p.lpr_log2 <= 6 &&
         nb_ok && p.waves >= 1 && p.waves <= 16 && p.rows_per_wave == (64 >> p.lpr_log2) * p.passes &&
         lean_strides_fit(c, 64 >> p.lpr_log2) &&
         tq2_lean_lds_bytes(1 << p.lpr_log2, p.nb, c.m, c.k, c.x != nullptr, 64 * p.waves, c.mode == MODE_BYTES) <=
             gemv_tq2::kLdsLimit;
}

bool tq2_lean_stampable(const GemvCall& c, const GemvPlan& p) {
  const int lpr = 1 << p.lpr_log2;
  return c.mode == MODE_DP4A && c.nseg <= 1 && p.passes == 1 && c.k / 256 <= (lpr / 4) * p.nb &&
         !tq2_lean_dma(lpr, p.nb, c.m, c.k, c.x != nullptr, 64 * p.waves, false);
}

hipError_t launch_gemv_tq2_lean(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  if (p.waves * p.rows_per_wave < p.block_n) return hipErrorInvalidConfiguration;
  if (stamps_on() && tq2_lean_stampable(c, p)) {  // the tuning harness's wave stamps, while there is room for them
    const int64_t groups = (c.n + p.block_n - 1) / p.block_n;
    if (uint32_t* slot = stamp_slot(4 + 4 * groups * p.waves)) {
      GemvCall cs = c;
      cs.segs.stamps = slot;
      return launch_gemv_tq2_lean_stamped(cs, p, stream);
    }
  }
  return c.mode == MODE_BYTES ? launch_gemv_tq2_lean_bytes(c, p, stream) : gemv_tq2::launch_mode<false>(c, p, stream);
}

}  // namespace komp
