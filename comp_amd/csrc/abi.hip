// extern "C" entry points of libkomp_hip.so (declared in include/komp_abi.h): argument validation, the mapping of
// the reference's tune knobs to a launch plan, column chunking, and the dispatch timing of the tuning harness.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/komp_abi.h"
#include "komp_internal.h"

namespace komp {
namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return KOMP_OK;
  return fail(KOMP_EHIP, "%s: HIP error %d (%s)", what, static_cast<int>(e), hipGetErrorString(e));
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

bool in_set(int v, const int* set, int n) {
  for (int i = 0; i < n; ++i)
    if (set[i] == v) return true;
  return false;
}

const int kBlockN[] = {8, 16, 32, 64, 128};
const int kNb[] = {1, 2, 4, 8, 16};
const int kWarps[] = {1, 2, 4, 8};
constexpr size_t kLdsMax = 160 * 1024;

// ---- dispatch timing ------------------------------------------------------------------------------------------------
struct TimingState {
  std::mutex mu;
  std::atomic<bool> on{false};
  int64_t max = 0;
  int64_t used = 0;
  std::vector<hipEvent_t> events;  // pairs (start, stop)
  std::vector<int> kinds;
};
TimingState g_timing;

// ---- in-kernel wave stamps ------------------------------------------------------------------------------------------
struct StampState {
  std::mutex mu;
  std::atomic<bool> on{false};
  uint32_t* buf = nullptr;
  int64_t words = 0;
  int64_t used = 0;
};
StampState g_stamps;

// ---- auto plan ------------------------------------------------------------------------------------------------------
// The plan gemv uses when block_n == 0.
//   Throughput regime (N >= 16384 rows, several workgroups per CU; one unfused Q4_0 / IQ4_NL column from 12288).  Each
//   row is read in ONE K step: the lean kernels then run their single-step form (a straight-line weight stream).
//   One Q4_0 / IQ4_NL column: nb 4, lanes per row = chunks / 4 within 16..64, 8 rows a workgroup (4 waves of two rows
//   at 32 lanes, 8 of one at 64); 2-7% faster than the earlier multi-step plans at Llama-3-8B shapes (gate+up 28672 x
//   4096 11.84 -> 11.37 us, 28672 x 8192 21.4 -> 20.7, IQ4_NL 28672 x 8192 23.4 -> 22.9).  Other Q4_0 launches:
//   whole rows in one K step, each wave walking two rows in sequence, nb 4 (8 past 256 chunks), lanes per row =
//   chunks / nb within 16..64, 4 waves; reading whole rows keeps the DRAM accesses of the grid in long runs (plans
//   that read each row in 1 KB pieces over several steps ran 5-17% slower).  TQ2_0: nb 4 and as many lanes per row
//   (16..64) as give each lane quad one block per chunk slot, 8 waves: at 32768 x 8192, 32 lanes per row ran 12.0-12.4
//   us against 16.2 for 16 lanes in two K steps (whose instance needs more than 64 VGPRs, 7 waves a SIMD).
//   Latency regime (fewer rows: every wave of the grid is resident at once), dp4a mode (TQ2_0: and bytes mode), fused
//   launches of one column, TQ2_0 with 1-3 columns and Q4_0 with 2-3: one workgroup per CU with ceil(N / CUs) rows,
//   one row group per wave, one K step where nb allows.  A grid of at most one workgroup per CU is spread one to a
//   CU, so no CU stages (and, fused, quantizes) the activations twice or runs two workgroups' dots on the same SIMDs;
//   9-24% faster at the BitNet-2B and Llama-3-8B shapes than 8-wave workgroups of 8-16 rows.  Lanes per row start at
//   64 and halve while the rows would need more than 16 waves or a lane would get fewer than 1.5 of the row's 16-byte
//   chunks.
//   Otherwise (one unfused Q4_0 column, other modes, 2-3 columns of the other formats): 8 waves per workgroup, as
//   many lanes per row as the row has 16-byte chunks (at most 64; the fused launch halves that, since every workgroup
//   pays for quantizing the input), and nb just large enough for one K step (Q4_0 caps it at 4), because each extra
//   step adds a full HBM round trip to a wave's critical path.
// The knob-mapped plans are knob sets of the explicit tune space; the two-pass Q4_0 throughput plan and the
// one-workgroup-per-CU plans are beyond the knob mapping.
int pow2_ceil(int64_t v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

GemvPlan plan_of(int block_n, int nb, int waves, int lpr, int passes) {
  GemvPlan plan;
  plan.block_n = block_n;
  plan.nb = nb;
  plan.waves = waves;
  plan.lpr_log2 = 0;
  while ((1 << plan.lpr_log2) < lpr) ++plan.lpr_log2;
  plan.passes = passes;
  plan.rows_per_wave = (64 / lpr) * passes;
  return plan;
}

std::atomic<int> g_cus[kMaxDevices];

// CUs of the current device (256 on MI355X; also the answer when no device can be queried)
int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  int c = g_cus[dev].load(std::memory_order_relaxed);
  if (c > 0) return c;
  if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
  g_cus[dev].store(c, std::memory_order_relaxed);
  return c;
}

// sw: the largest row stride of the launch's matrices (bytes; 0: dense rows), which decides whether the lean kernels
// can take a plan of more than 8 waves (their 32-bit per-pass buffer ranges, lean_strides_fit).
GemvPlan auto_plan(int fmt, bool fused, int mode, int64_t m, int64_t n, int64_t k, int64_t sw = 0) {
  const int bpb = fmt_info(fmt).qbytes / (fmt == FMT_Q4_K ? 32 : 16);  // lane slots per block (Q4_K: 32-byte groups)
  const int64_t nblk = k / fmt_info(fmt).block;
  const int64_t chunks = nblk * bpb;                      // lane slots per row (16-byte chunks; Q4_K 32-byte groups)
  // one unfused Q4_0 / IQ4_NL column (the lean kernel) over many rows: each row in one K step of nb 4, as few lanes
  // per row as that allows (16..64), 8 rows a workgroup (4 waves at least); the lean kernel's single-step form
  const bool lean_q4 = (fmt == FMT_Q4_0 || fmt == FMT_IQ4_NL) && m == 1 &&
                       (mode == KOMP_MODE_DP4A || (fmt == FMT_Q4_0 && mode == KOMP_MODE_BYTES));
  if (lean_q4 && !fused && n >= 12288 && chunks <= 256) {
    int lpr = pow2_ceil((chunks + 3) / 4);
    lpr = lpr < 16 ? 16 : lpr;
    const int rpw = 64 / lpr;
    const int w = 8 / rpw < 4 ? 4 : 8 / rpw;
    return plan_of(w * rpw, 4, w, lpr, 1);
  }
  if (n >= 16384) {
    if (fmt == FMT_TQ2_0) {
      // nb 4, as many lanes per row as give every row one K step (16..64, lanes of a quad share a block), 8 waves;
      // the single-step form of the lean kernel
      int lpr = pow2_ceil(nblk);
      lpr = lpr < 16 ? 16 : (lpr > 64 ? 64 : lpr);
      return plan_of(8 * (64 / lpr), 4, 8, lpr, 1);
    }
    if (lean_q4 && chunks <= 128)
      // one fused column of rows of up to 128 blocks: 16 lanes per row, nb 2, 8 waves; 3-7% faster than the rule
      // below at 28672-128256 rows x 4096 columns
      return plan_of(32, 2, 8, 16, 1);
    const bool lean_q4_cols = (fmt == FMT_Q4_0 || fmt == FMT_IQ4_NL) && (m == 2 || m == 3) &&
                              (mode == KOMP_MODE_DP4A || (fmt == FMT_Q4_0 && mode == KOMP_MODE_BYTES));
    if (lean_q4_cols && chunks <= 128) {
      // two or three Q4_0 / IQ4_NL columns of rows of up to 128 blocks: each row in one K step of nb 4, 8 waves of
      // two rows, the lean kernel's single-pass form (Llama-3-8B gate+up 28672 x 4096: 3 columns 14.6 -> 12.5 us,
      // 2 columns 12.3 -> 11.9, against two passes of 4 waves)
      int lpr = pow2_ceil((chunks + 3) / 4);
      lpr = lpr < 16 ? 16 : lpr;
      return plan_of(8 * (64 / lpr), 4, 8, lpr, 1);
    }
    const int nb = chunks > 256 ? 8 : 4;
    int lpr = pow2_ceil((chunks + nb - 1) / nb);
    lpr = lpr < 16 ? 16 : (lpr > 64 ? 64 : lpr);
    return plan_of(4 * (64 / lpr) * 2, nb, 4, lpr, 2);  // 4 waves, two passes each
  }
  // the lean kernels' modes: dp4a, and bytes for TQ2_0 and Q4_0
  const bool lean_mode = mode == KOMP_MODE_DP4A || ((fmt == FMT_TQ2_0 || fmt == FMT_Q4_0) && mode == KOMP_MODE_BYTES);
  if (lean_mode && m <= 3 && (fmt == FMT_TQ2_0 || (m == 1 && fused) || (fmt == FMT_Q4_0 && m > 1))) {
    const int cus = device_cus();
    const int64_t rows = n < 1 ? 1 : (n + cus - 1) / cus;
    const int lpr_min = bpb > 4 ? bpb : 4;  // a row group holds whole blocks
    int lpr = 64;
    while (lpr > lpr_min && ((rows + 64 / lpr - 1) / (64 / lpr) > 16 || 2 * chunks < 3 * lpr)) lpr >>= 1;
    const int rpp = 64 / lpr;
    int64_t waves = (rows + rpp - 1) / rpp;
    // TQ2_0 with 2-3 columns stages 16 threads per block and column: enough waves for one staging pass, when that
    // costs at most a quarter more rows per workgroup (a second pass of the q8_K staging costs more than the rows;
    // measured at BitNet-2B shapes: 6912x2560, 3 columns, 8 waves of 4 rows 4.17 us against 4.83 for 7 waves and
    // 5.2 for the 16-row plan below; 2560x6912 keeps 10 waves, 2 columns 4.6 against 4.9 for 14)
    const int64_t stage_waves = (m * nblk * 16 + 63) / 64;
    int64_t wg_rows = rows;
    if (fmt == FMT_TQ2_0 && m > 1 && stage_waves > waves && stage_waves <= waves + waves / 4) {
      waves = stage_waves;
      wg_rows = waves * rpp;  // fewer, fuller workgroups
    }
    // One column over few rows a CU (at most 8 waves of them), TQ2_0 or f32 in: as many waves as one staging pass
    // takes (16 threads a block of q8_K activations, 8 a block of q8_0 ones; at most 16), each with its full rows
    // (fewer, fuller workgroups), instead of one wave staging in several passes.  TQ2_0: 127 x 2816 2.81 -> 2.16 us
    // (f32 in 3.30 -> 2.17, bytes 3.23 -> 2.50), 127 x 6912 3.46 -> 2.28 (f32 in 4.96 -> 2.52), 300 x 2560 2.79 ->
    // 2.21, 2048 x 2560 2.63 -> 2.34 (f32 in 2.88 -> 2.31).  f32 in: Q4_0 127 x 4192 7.12 -> 3.36, 300 x 4096 4.31 ->
    // 2.53, 1000 x 4096 3.33 -> 2.62, 2048 x 4096 3.29 -> 2.87; IQ4_NL 127 x 4096 6.35 -> 2.93; Q8_0 6.27 -> 3.20;
    // Q4_K 4.11 -> 2.59.  The Llama-3-8B plans (4096-6144 rows: 9-16 waves) keep theirs.
    if (m == 1 && (fmt == FMT_TQ2_0 || fused) && waves <= 8) {
      const int per_block = (fmt == FMT_TQ2_0 || fmt == FMT_Q4_K) ? 16 : 8;
      int64_t one_pass = (nblk * per_block + 63) / 64;
      one_pass = one_pass < 16 ? one_pass : 16;
      if (one_pass > waves) {
        waves = one_pass;
        wg_rows = waves * rpp;
      }
    }
    // two or three columns only with two waves on most SIMDs: with fewer, the 8-wave plans below, two workgroups
    // a CU, stage and dot faster (TQ2_0 4097 x 2816, 3 columns: 4.16 against 4.32 us; 127 x 2816: 3.0 against 4.8).
    // Q4_0 at Llama-3-8B shapes, 2-3 columns: 8-36% faster than those plans, the fused launches most (4096 x 14336,
    // 3 columns: 15.8 against 24.7 us fused, 9.3 against 10.2 with q8 in).
    if (waves <= 16 && (m == 1 || waves >= 7)) {
      const int64_t blocks_per_slot = lpr / bpb;
      // the 16-wave instantiations: nb up to 8 for one column, 4 for two and three; Q4_K 2 (its lean kernel's rows
      // of 56 blocks in two steps of 32 ran 9.0 us at 4096 x 14336 fused, in one of 64 10.0)
      const int nb_max = fmt == FMT_Q4_K ? 2 : (m > 1 ? 4 : 8);
      int nb = pow2_ceil((nblk + blocks_per_slot - 1) / blocks_per_slot);
      nb = nb < 1 ? 1 : (nb > nb_max ? nb_max : nb);
      if (fmt == FMT_Q4_0 && m > 1 && !fused && mode == KOMP_MODE_DP4A && nblk > blocks_per_slot * nb && nblk <= 256)
        // two or three Q4_0 columns with q8 in whose rows this plan takes in two K steps but 64 lanes of nb 4 in
        // one (a few blocks past 128: K = 4192): the one-column plan's shape, 8 waves of one row in one step
        // (4097 x 4192, 3 columns 5.21 -> 4.58 us, 2 columns 4.68 -> 4.06; 6913 x 4192 6.58 -> 6.08).  Fused
        // launches were slower so (8.8 -> 9.4 us), and IQ4_NL no faster.
        return plan_of(8, pow2_ceil((nblk + 63) / 64), 8, 64, 1);
      // past 8 waves, two or three columns (and bytes mode) run this plan on the lean kernels only: the general kernel
      // takes at most 8 waves there
      const size_t lean_lds = fmt == FMT_TQ2_0 ? tq2_lean_lds_bytes(lpr, nb, static_cast<int>(m), static_cast<int>(k), fused,
                                                                    static_cast<int>(64 * waves), mode == KOMP_MODE_BYTES)
                                               : q4_lean_lds_bytes(lpr, nb, static_cast<int>(m), static_cast<int>(k),
                                                                   mode == KOMP_MODE_BYTES);
      // and only where the lean kernels' 32-bit per-pass buffer ranges hold a pass's rows (else the 8-wave plans)
      const int64_t row_bytes = sw > 0 ? sw : nblk * fmt_info(fmt).qbytes;
      const bool lean_fit = rpp * row_bytes <= 0x7FFFFFF0;
      if (waves <= 8 || (lean_fit && ((m == 1 && mode == KOMP_MODE_DP4A) || lean_lds <= kLdsMax)))
        return plan_of(static_cast<int>(wg_rows), nb, static_cast<int>(waves), lpr, 1);
    }
  }
  if (fmt == FMT_Q4_K && mode == KOMP_MODE_DP4A && m <= 3) {
    // the Q4_K lean kernel (32-byte slots, 4 lanes a block): nb 2, 32 lanes a row for rows of up to 16 blocks (one
    // K step), 64 for longer ones; the long rows in one workgroup of one row a wave per CU when that is at most 16
    // waves; otherwise one column over 4 waves, two and three over 8.  Measured on MI355X against the other lean
    // plans (1 column: 4096 x 4096 3.8 us, 14336 x 4096 7.6, 4096 x 14336 8.1; 3 columns at 14336 x 4096 10.2, at
    // 4096 x 14336 11.7 against 12.5 over 8 waves), from 4.6 / 8.9 / 10.3 / 13.9 on the general kernel's plans
    const int lq = chunks <= 64 ? 32 : 64;
    int nbq = pow2_ceil((chunks + lq - 1) / lq);
    nbq = nbq > 2 ? 2 : nbq;
    const int64_t per_cu = (n + device_cus() - 1) / device_cus();
    if (lq == 64 && per_cu <= 16) return plan_of(static_cast<int>(per_cu), nbq, static_cast<int>(per_cu), 64, 1);
    const int wq = m > 1 ? 8 : 4;
    return plan_of(wq * (64 / lq), nbq, wq, lq, 1);
  }
  if (fmt == FMT_Q4_K) {
    // Q4_K (32-byte slots) on the general kernel (bytes and emulated modes): about two slots per lane (four from
    // 12288 rows on), nb <= 2, and 8-16 rows per workgroup of at least 4 waves.  Measured on MI355X at 4096-14336
    // rows x 2560-14336 columns, 1 column: 10-25% faster than the 16-byte-chunk rules below.
    int lq = pow2_ceil(n >= 12288 ? (chunks + 3) / 4 : (chunks + 1) / 2);
    lq = lq < bpb ? bpb : (lq > 64 ? 64 : lq);
    int nbq = pow2_ceil((chunks + lq - 1) / lq);
    nbq = nbq > 2 ? 2 : nbq;
    const int rpw = 64 / lq;
    const int wq = 8 / rpw < 4 ? 4 : 8 / rpw;
    return plan_of(wq * rpw, nbq, wq, lq, 1);
  }
  if (!fused && fmt == FMT_Q8_0 && mode == KOMP_MODE_DP4A && m <= 3 && n >= 12288 && chunks <= 256)
    // Q8_0 on its lean kernel, many rows with short rows: 64 lanes a row (a lane pair per block), rows of up to 128
    // blocks in one K step of nb 4, 8 waves of one row (14336 x 4096: 11.7 -> 10.7 us against the rule below on the
    // same kernel, 3 columns 12.5 -> 12.2)
    return plan_of(8, pow2_ceil((nblk + 31) / 32), 8, 64, 1);
  if (!fused && fmt != FMT_TQ2_0 && n >= 12288 && chunks <= 256)
    // many rows per CU with short rows (Llama-3-8B's gate and up projections, 14336 x 4096): 4-wave workgroups of 8
    // rows, two rows per wave with 32 lanes each, nb 2 (2-4 K steps); 10-15% faster than one K step of 64 lanes
    return plan_of(8, 2, 4, 32, 1);
  if (fmt == FMT_TQ2_0 && m == 3 && mode == KOMP_MODE_DP4A && nblk <= 16) {
    // three TQ2_0 columns over few rows (these plans): the lean kernel stages 16 threads per block and column, and a
    // second staging pass of 8 waves costs more than a wider workgroup; one row a wave, as many waves as one pass
    // takes (127 x 2816: 3.21 -> 2.75 us, f32 in 3.71 -> 3.33; 2048 x 2816: 3.47 -> 3.01; 1000 x 4096, 12 waves: 3.08
    // -> 2.92; at 2560 columns 8 waves already stage in one pass).  Longer rows (6912 columns) keep 8 waves: 16 of
    // them in two passes ran slower.
    const int64_t stage_waves = (m * nblk * 16 + 63) / 64;
    if (stage_waves > 8) return plan_of(static_cast<int>(stage_waves), 1, static_cast<int>(stage_waves), 64, 1);
  }
  int lpr = pow2_ceil(fused ? (chunks + 1) / 2 : chunks);
  lpr = lpr < 4 ? 4 : (lpr > 64 ? 64 : lpr);
  if (lpr < bpb) lpr = bpb;  // a row group holds whole blocks
  const int64_t blocks_per_slot = lpr / bpb;
  int nb = pow2_ceil((nblk + blocks_per_slot - 1) / blocks_per_slot);
  nb = nb < 1 ? 1 : (nb > 16 ? 16 : nb);
  if (fmt != FMT_TQ2_0 && nb > 4) nb = 4;
  int w = 8;
  const int rpw = 64 / lpr;
  while (w * rpw > 128) w >>= 1;
  while (w * rpw < 8) w <<= 1;
  return plan_of(w * rpw, nb, w, lpr, 1);
}

// Unfused single Q4_0 / IQ4_NL columns in the lean kernel's modes (dp4a; Q4_0 bytes too): the launches whose knob
// programs may run one workgroup a wave (gemv_entry).
bool knob_waves_apart(int fmt, bool fused, int mode, int64_t m) {
  return !fused && m == 1 &&
         ((fmt == FMT_Q4_0 && (mode == KOMP_MODE_DP4A || mode == KOMP_MODE_BYTES)) ||
          (fmt == FMT_IQ4_NL && mode == KOMP_MODE_DP4A));
}

GemvPlan knob_plan(int fmt, int block_n, int nb, int num_warps) {
  GemvPlan plan;
  plan.block_n = block_n;
  plan.nb = nb;
  plan.waves = num_warps;
  const int rpw = block_n / num_warps;
  const int rpp = rpw < 16 ? rpw : 16;
  plan.lpr_log2 = 0;
  while ((64 >> plan.lpr_log2) > rpp) ++plan.lpr_log2;
  plan.passes = rpw / rpp;
  plan.rows_per_wave = rpw;
  // TQ2_0 (64-byte blocks): a K step of fewer than 256 bytes a row (lanes a row x nb x 16) leaves every load
  // instruction half a cache line of each row, and the few workgroups of such knob sets (one per block_n rows) are
  // bound by the misses each CU keeps in flight.  The step is widened to 256 bytes a row (nb 1 or 2 -> 4 at 4 lanes a
  // row, 1 -> 2 at 8): the same rows a workgroup and waves, S the same, Y within the same bound.  The reference's spec
  // defaults (block_n 64, nb 1, num_warps 4) at BitNet-2B 2560 x 6912: 9.95 -> 7.46 us; 6912 x 2560 4.93 -> 4.22.
  if (fmt == FMT_TQ2_0)
    while ((1 << plan.lpr_log2) * plan.nb < 16 && plan.nb < 4) plan.nb *= 2;
  return plan;
}

// ---- matrix-core GEMM ----------------------------------------------------------------------------------------------
// From kGemmMinM activation columns on, block_n == 0 in dp4a mode (unfused) runs the matrix-core GEMM, which reads the
// weights once per 64 columns, instead of the GEMV in column chunks of 3 (which reads them once for up to 3 columns,
// in one launch).  At 4 columns the GEMM is 1.2-1.8x faster at Llama-3-8B and BitNet-2B shapes; at 3 the lean GEMVs
// are as fast or faster (TQ2_0 6912 x 2560: 5.6 against 5.8 us, 2560 x 6912: 5.7 against 5.2, 32768 x 8192: 22.5
// against 23.9; Q4_0 4096 x 14336: 9.9 against 13.9).
constexpr int64_t kGemmMinM = 4;
constexpr int64_t kGemmMaxCols = int64_t{1} << 20;  // columns per GEMM launch (grid.y = columns / 64 at most 16384)

// The GEMM's plan for m columns (one launch) and n rows.  Columns go in groups of at most 64 (4 tiles of 16), split
// evenly.  The waves of a workgroup split K (wk) and rows (wr) by how many 16-row tiles each CU gets (r, counting
// column groups): with about one per CU every wave of a CU must share the tile's K, so K is split 8 ways; with a few
// per CU, 2-4 ways; with many, each wave owns its rows and no partial sums meet.  Measured on MI355X at Llama-3-8B
// (4096x4096, 14336x4096, 4096x14336, 128256x4096) and BitNet-2B shapes, 1..64 columns.  False when the shape is past
// the kernel's 32-bit buffer offsets (64 * K and 32 * SW below 2^31) or its scale slab does not fit in LDS.
bool gemm_plan(int fmt, int64_t m, int64_t n, int64_t k, int64_t sw, GemmPlan* p) {
  if (64 * k > INT32_MAX || 32 * sw > INT32_MAX) return false;
  if (fmt == FMT_Q4_K) {
    // Q4_K: the same families with one row tile per wave (each output also holds the block's two integer sums);
    // long rows move down the family list until the unpacked scale slab fits in LDS
    const int64_t c16 = (m + 15) / 16;
    const int64_t groups = (c16 + 3) / 4;
    const int cn = static_cast<int>(groups > 0 ? (c16 + groups - 1) / groups : 1);
    const double r = static_cast<double>((n + 15) / 16) * groups / device_cus();
    static const int kFam[4][2] = {{1, 8}, {2, 4}, {4, 2}, {8, 1}};  // (wk, wr)
    int f = r > 8.0 ? 0 : (r > 2.0 ? 1 : (r > 1.25 && cn > 1 ? 2 : 3));
    for (;; ++f) {
      if (f == 2 && cn == 1) continue;  // (4, 2) only with 2+ column tiles
      const GemmPlan q = {kFam[f][0], kFam[f][1], 1, cn, f == 0 && cn > 2 ? 1 : 2};
      if (gemm_lds_bytes(fmt, q, static_cast<int>(k)) <= kLdsMax || f == 3) {
        *p = q;
        return gemm_lds_bytes(fmt, q, static_cast<int>(k)) <= kLdsMax;
      }
    }
  }
  const int64_t c16 = (m + 15) / 16;
  int64_t groups = (c16 + 3) / 4;
  int cn = static_cast<int>(groups > 0 ? (c16 + groups - 1) / groups : 1);
  const int64_t tiles = (n + 15) / 16;
  double r = static_cast<double>(tiles) * groups / device_cus();
  // Few row tiles a CU: fewer column tiles a workgroup, in more column groups (each reads its rows' weights again,
  // mostly from L2).  4 column tiles and at most 2 row tiles a CU: halve until each CU has more than 2; at 64 columns
  // Q4_0 4096 x 4096 16.3 -> 15.0 us, 4096 x 14336 46.0 -> 40.2, TQ2_0 2560 x 6912 18.6 -> 14.7 (one column tile a
  // workgroup), TQ2_0 6912 x 2560 14.7 -> 12.0 (two).  3 column tiles with idle CUs: one column tile a workgroup
  // (TQ2_0 2560 x 6912 at 48 columns 14.5 -> 11.9 us; at 4096 rows, one tile a CU, splitting measured slower).
  const auto regroup = [&](int to) {
    cn = to;
    groups = (c16 + cn - 1) / cn;
    r = static_cast<double>(tiles) * groups / device_cus();
  };
  if (cn == 4)
    while (r <= 2.0 && cn > 1) regroup(cn / 2);
  else if (cn == 3 && r < 1.0)
    regroup(1);
  GemmPlan q = {8, 1, 1, cn, 2};
  if (r > 8.0)
    q = cn == 1 ? GemmPlan{1, 8, m > 8 && fmt != FMT_Q8_0 ? 2 : 1, 1, 2} : GemmPlan{1, 8, 1, cn, cn == 2 ? 2 : 1};
  else if (r > 2.0 && cn == 1)
    q = GemmPlan{4, 2, 2, 1, 4};
  else if (r > 2.0 && fmt == FMT_Q8_0)  // Q8_0's two row tiles a wave would need more than 256 VGPRs
    q = GemmPlan{2, 4, 1, cn, 2};
  else if (r > 2.0)
    // two row tiles a wave: each activation load feeds twice the MFMAs (the activations are re-read for every row
    // tile, 8x the weight bytes a step at 64 columns); 4 waves from 4 row tiles a CU.  Q4_0 14336 x 4096 at 32 / 48 /
    // 64 columns: 32.0 / 44.2 / 56.1 -> 23.7 / 30.3 / 37.7 us; 28672 x 4096 at 64: 108 -> 67 us; TQ2_0 14336 x 4096
    // at 64: 44.6 -> 27.2 us.  Past 3 tiles a CU, K split 2 ways (4 waves a workgroup, fewer partial sums to add):
    // Q4_0 14336 x 4096 at 64 columns 35.4 -> 34.3 us
    q = r > 3.0 ? GemmPlan{2, 2, 2, cn, 2} : GemmPlan{4, 2, 2, cn, 2};
  else if (r > 1.25 && cn > 1)
    q = GemmPlan{4, 2, 1, cn, 2};
  while (gemm_lds_bytes(fmt, q, static_cast<int>(k)) > kLdsMax && q.wn * q.wr > 1) {  // long rows: fewer rows a group
    if (q.wn > 1 && (q.wk == 1 || (q.wk == 4 && q.cn > 1)))
      q.wn = 1;  // (1, 8, 2, 1, 2) -> (1, 8, 1, 1, 2); (4, 2, 2, cn, 2) -> (4, 2, 1, cn, 2)
    else
      q = GemmPlan{8, 1, 1, cn, 2};
  }
  *p = q;
  return gemm_lds_bytes(fmt, q, static_cast<int>(k)) <= kLdsMax;
}

// The matrix-core GEMV (gemv_tq2_mfma.hip) for kMfmaM TQ2_0 columns, block_n == 0 in dp4a mode.  Measured on MI355X
// against the lean kernel's plans (graph replays, cold weights), three columns with q8_K in: BitNet-2B 6912 x 2560
// 3.95 -> 3.84 us, 2560 x 6912 4.44 -> 4.22, 6913 x 2816 4.5 -> 3.9, 4097 x 2816 4.2 -> 3.3, 32768 x 8192 23.3 ->
// 18.4; f32 in (each wave quantizing its own blocks): 32768 x 8192 32.4 -> 24.0, but 1.1-1.3 us slower at the
// BitNet-2B shapes, where every workgroup reading all 3 x K f32 inputs costs more than the dots save (there the lean
// kernel's fewer, fuller workgroups stay), so fused launches take it from 4 row tiles a CU on.  Up to 8 rows a CU the
// lean kernel is faster (0.3-0.9 us at 64-2048 rows x 2560-8192 columns): every workgroup reads all 3 x K
// activations for few rows.  Two columns stay on the lean kernel (as fast or faster at every shape measured).
// Plans: rows spread evenly over the CUs, at most 16 a workgroup (2560 rows: 256 workgroups of 10, 4.22 us against
// 4.39 for 160 of 16); one block a wave (up to 16 waves a workgroup) for rows of up to 16 blocks, else about two; from
// 4 row tiles a CU, two tiles a workgroup (each activation load serves both) and four blocks a wave.  False when the
// shape is past it (rows of more than 64 blocks, or past its 32-bit descriptor ranges).
constexpr int64_t kMfmaM = 3;
bool tq2_mfma_plan(int64_t m, int64_t n, int64_t k, int64_t sw, bool fused, MfmaPlan* p) {
  if (m != kMfmaM || k <= 0 || k % 256 || n < 1) return false;
  const int64_t nblk = k / 256;
  const int64_t cus = device_cus();
  const int64_t tiles = (n + 15) / 16;
  const bool big = tiles >= 4 * cus;
  if (n <= 8 * cus || (fused && !big)) return false;
  int64_t waves = big ? (nblk + 3) / 4 : (nblk <= 16 ? nblk : (nblk + 1) / 2);
  waves = waves > 16 ? 16 : waves;
  const int64_t nbw = (nblk + waves - 1) / waves;
  if (nbw > 4 || 16 * sw > 0x7FFFFFF0 || 4 * k > 0x7FFFFFF0) return false;
  if (sw < 64 * nblk || sw % 16 != 0) return false;  // its 16-byte weight loads need 16-byte aligned rows
  const int64_t even = (n + cus - 1) / cus;  // rows a CU: more than 8
  const int64_t rows = big ? 32 : (even < 16 ? even : 16);
  *p = MfmaPlan{big ? 2 : 1, static_cast<int>(waves), static_cast<int>(nbw), static_cast<int>(rows)};
  return true;
}

enum Route { kRouteAuto = 0, kRouteGemm = 1 };

struct GemvMat {
  const uint8_t* wq;
  const int16_t* ws;
  float* y;
  int32_t* s;
  int64_t n;
  int64_t sw;
};

struct GemvArgs {
  const GemvMat* mats;  // 1..kMaxSegs matrices sharing the activation input
  int count;
  const int8_t* xq;     // unfused
  const float* xd;
  const float* x;       // fused
  int8_t* xq_out;
  float* xd_out;
  int16_t* xb_out;
};

int gemv_entry(int fmt, bool fused, const char* name, const GemvArgs& a, int64_t M, int64_t K, int block_n, int nb,
               int mode, int num_warps, void* stream, int route = kRouteAuto) {
  const FmtInfo fi = fmt_info(fmt);
  const int blk = fi.block;
  const int64_t row_bytes = K / blk * fi.qbytes;
  if (a.count < 1 || a.count > kMaxSegs || a.mats == nullptr)
    return fail(KOMP_EINVAL, "%s: count=%d must be 1..%d", name, a.count, kMaxSegs);
  if (M < 0 || K < 0) return fail(KOMP_EINVAL, "%s: negative size (M=%lld K=%lld)", name, (long long)M, (long long)K);
  if (K > INT32_MAX) return fail(KOMP_EINVAL, "%s: K must be < 2^31", name);
  if (K % blk) return fail(KOMP_EINVAL, "%s: K=%lld is not a multiple of the %d-value block", name, (long long)K, blk);
  int64_t total_rows = 0;
  for (int i = 0; i < a.count; ++i) {
    const GemvMat& w = a.mats[i];
    if (w.n < 0 || w.n > INT32_MAX) return fail(KOMP_EINVAL, "%s: N=%lld out of range", name, (long long)w.n);
    if (w.n > 0 && (w.sw < row_bytes || w.sw % 16))  // (a matrix without rows has no row stride)
      return fail(KOMP_EINVAL, "%s: SW=%lld must be a multiple of 16 and >= %lld (the quant bytes of a row)", name,
                  (long long)w.sw, (long long)row_bytes);
    total_rows += w.n;
  }
  if (total_rows > INT32_MAX) return fail(KOMP_EINVAL, "%s: the matrices' rows must total < 2^31", name);
  if (mode < KOMP_MODE_BYTES || mode > KOMP_MODE_DP4A) return fail(KOMP_EINVAL, "%s: mode=%d not in {0,1,2}", name, mode);
  if (block_n != 0) {
    if (!in_set(block_n, kBlockN, 5)) return fail(KOMP_EINVAL, "%s: block_n=%d not in {8,16,32,64,128}", name, block_n);
    if (!in_set(nb, kNb, 5)) return fail(KOMP_EINVAL, "%s: nb=%d not in {1,2,4,8,16}", name, nb);
    if (!in_set(num_warps, kWarps, 4)) return fail(KOMP_EINVAL, "%s: num_warps=%d not in {1,2,4,8}", name, num_warps);
    if (fmt == FMT_Q4_K && nb > 8)  // a q4_k lane slot is a 32-byte group, twice the other formats' chunk
      return fail(KOMP_EINVAL, "%s: nb=%d; q4_k takes nb <= 8 (32-byte groups per lane)", name, nb);
  }
  if (fused && blk != 256 && a.xb_out != nullptr)
    return fail(KOMP_EINVAL, "%s: XB (bsums) is a q8_K plane; pass NULL for q8_0 activations", name);
  if (fused && a.xq_out == nullptr && (a.xd_out != nullptr || a.xb_out != nullptr))
    return fail(KOMP_EINVAL, "%s: XD / XB outputs need XQ as well", name);
  if (fused && a.xq_out != nullptr && a.xd_out == nullptr)
    return fail(KOMP_EINVAL, "%s: the XQ output needs XD as well", name);
  if (M == 0 || total_rows == 0) return KOMP_OK;
  if (K > 0 && !fused && (a.xq == nullptr || a.xd == nullptr))
    return fail(KOMP_EINVAL, "%s: XQ and XD must not be NULL", name);
  if (K > 0 && fused && a.x == nullptr) return fail(KOMP_EINVAL, "%s: X must not be NULL", name);
  if (!aligned(a.xq, 16) || !aligned(a.x, 16)) return fail(KOMP_EINVAL, "%s: XQ and X must be 16-byte aligned", name);
  if (!aligned(a.xd, 4) || !aligned(a.xq_out, 4) || !aligned(a.xd_out, 4) || !aligned(a.xb_out, 2))
    return fail(KOMP_EINVAL, "%s: XD and the q8 outputs must be aligned to their element size", name);
  GemvMat mats[kMaxSegs];  // the matrices with rows
  int count = 0;
  for (int i = 0; i < a.count; ++i) {
    const GemvMat& w = a.mats[i];
    if (w.n == 0) continue;
    if (K > 0 && (w.wq == nullptr || w.ws == nullptr)) return fail(KOMP_EINVAL, "%s: WQ and WS must not be NULL", name);
    if (w.y == nullptr) return fail(KOMP_EINVAL, "%s: Y must not be NULL", name);
    if (!aligned(w.wq, 16)) return fail(KOMP_EINVAL, "%s: WQ must be 16-byte aligned", name);
    if (!aligned(w.ws, 2) || !aligned(w.y, 4) || !aligned(w.s, 4))
      return fail(KOMP_EINVAL, "%s: WS, Y and S must be aligned to their element size", name);
    if (fmt == FMT_Q4_K && !aligned(w.ws, 16))  // its 16-byte scale-plane entries are read whole
      return fail(KOMP_EINVAL, "%s: WS must be 16-byte aligned for q4_k", name);
    mats[count++] = w;
  }
  const int64_t nblk = K / blk;
  if (route == kRouteGemm || (!fused && block_n == 0 && mode == KOMP_MODE_DP4A && M >= kGemmMinM)) {
    GemmPlan gp;
    bool fits = true;
    for (int i = 0; i < count; ++i)
      fits = fits && gemm_plan(fmt, M < kGemmMaxCols ? M : kGemmMaxCols, mats[i].n, K, mats[i].sw, &gp);
    if (fits) {
      for (int i = 0; i < count; ++i) {
        for (int64_t m0 = 0; m0 < M; m0 += kGemmMaxCols) {
          const int64_t mc = M - m0 < kGemmMaxCols ? M - m0 : kGemmMaxCols;
          gemm_plan(fmt, mc, mats[i].n, K, mats[i].sw, &gp);
          GemmCall c = {};
          c.fmt = fmt;
          c.wq = mats[i].wq;
          c.ws = mats[i].ws;
          c.xq = a.xq != nullptr ? a.xq + m0 * K : nullptr;
          c.xd = a.xd != nullptr ? a.xd + m0 * nblk : nullptr;
          c.y = mats[i].y + m0 * mats[i].n;
          c.s = mats[i].s != nullptr ? mats[i].s + m0 * mats[i].n * nblk * s_per_block(fmt) : nullptr;
          c.m = static_cast<int>(mc);
          c.n = static_cast<int>(mats[i].n);
          c.k = static_cast<int>(K);
          c.sw = mats[i].sw;
          const int st = hip_status(launch_gemm(c, gp, static_cast<hipStream_t>(stream)), name);
          if (st != KOMP_OK) return st;
        }
      }
      return KOMP_OK;
    }
    if (route == kRouteGemm)
      return fail(KOMP_EINVAL, "%s: K=%lld / SW past the GEMM's limits (64*K and 32*SW below 2^31, scale slab in LDS)",
                  name, (long long)K);
  }
  MfmaPlan mp;
  if (block_n == 0 && mode == KOMP_MODE_DP4A && fmt == FMT_TQ2_0 && count == 1 &&
      tq2_mfma_plan(M, mats[0].n, K, mats[0].sw, fused, &mp)) {
    GemvCall c = {};
    c.fmt = fmt;
    c.wq = mats[0].wq;
    c.ws = mats[0].ws;
    c.xq = fused ? nullptr : a.xq;
    c.xd = fused ? nullptr : a.xd;
    c.x = fused ? a.x : nullptr;
    c.xq_out = a.xq_out;
    c.xd_out = a.xd_out;
    c.xb_out = a.xb_out;
    c.y = mats[0].y;
    c.s = mats[0].s;
    c.m = static_cast<int>(M);
    c.n = static_cast<int>(mats[0].n);
    c.k = static_cast<int>(K);
    c.sw = mats[0].sw;
    c.mode = mode;
    c.nseg = 1;
    if (tq2_mfma_eligible(c, mp)) return hip_status(launch_gemv_tq2_mfma(c, mp, static_cast<hipStream_t>(stream)), name);
  }
  int mc = static_cast<int>(M < 3 ? M : 3);
  while (mc > 1 && gemv_lds_bytes(fmt, mc, static_cast<int>(K)) > kLdsMax) --mc;
  if (gemv_lds_bytes(fmt, mc, static_cast<int>(K)) > kLdsMax)
    return fail(KOMP_EINVAL, "%s: K=%lld needs more than 160 KiB of LDS for one activation column", name, (long long)K);

  int64_t sw_max = 0;
  for (int i = 0; i < count; ++i) sw_max = mats[i].sw > sw_max ? mats[i].sw : sw_max;
  GemvPlan plan =
      block_n == 0 ? auto_plan(fmt, fused, mode, M, total_rows, K, sw_max) : knob_plan(fmt, block_n, nb, num_warps);
  if (block_n != 0 && num_warps > 1 && knob_waves_apart(fmt, fused, mode, M)) {
    // The knobs fix each wave's rows (block_n / num_warps), lanes per row and nb, and with them every output bit: a
    // program's waves share no rows.  How the waves group into workgroups is the launch's: when the programs hold no
    // more waves than the device has CUs, each wave runs as a workgroup of its own, so the programs' rows spread over
    // a CU a wave instead of a CU a program (Q4_0 4096 x 4096 at 64/4/4: 64 workgroups of 4 waves 7.45 us,
    // 256 of one 6.25; 4096 x 14336 22.0 -> 17.0; 128/4/8 12.4 -> 6.3; IQ4_NL 8.55 -> 8.15).  Unfused Q4_0 / IQ4_NL
    // columns on the lean kernel only: a fused launch's workgroups each quantize all of K, which one wave does slower
    // (8.7 -> 10.5 us), and TQ2_0's each stage all of K (2560 x 6912 at 64/1/4: 7.45 -> 7.52, bytes 10.3 -> 10.8).
    int64_t programs = 0;
    for (int i = 0; i < count; ++i) programs += (mats[i].n + block_n - 1) / block_n;
    if (programs * num_warps <= device_cus()) plan = knob_plan(fmt, block_n / num_warps, nb, 1);
  }

  for (int64_t m0 = 0; m0 < M; m0 += mc) {
    GemvCall c = {};
    c.fmt = fmt;
    c.wq = mats[0].wq;
    c.ws = mats[0].ws;
    c.xq = fused ? nullptr : a.xq + m0 * K;
    c.xd = fused ? nullptr : a.xd + m0 * nblk;
    c.x = fused ? a.x + m0 * K : nullptr;
    c.xq_out = a.xq_out != nullptr ? a.xq_out + m0 * K : nullptr;
    c.xd_out = a.xd_out != nullptr ? a.xd_out + m0 * nblk : nullptr;
    c.xb_out = a.xb_out != nullptr ? a.xb_out + m0 * (K / 16) : nullptr;
    c.y = mats[0].y + m0 * mats[0].n;
    c.s = mats[0].s != nullptr ? mats[0].s + m0 * mats[0].n * nblk * s_per_block(fmt) : nullptr;
    c.m = static_cast<int>(M - m0 < mc ? M - m0 : mc);
    c.n = static_cast<int>(mats[0].n);
    c.k = static_cast<int>(K);
    c.sw = mats[0].sw;
    c.mode = mode;
    c.nseg = count;
    for (int i = 0; count > 1 && i < count; ++i) {
      c.segs.wq[i] = mats[i].wq;
      c.segs.ws[i] = mats[i].ws;
      c.segs.y[i] = mats[i].y + m0 * mats[i].n;
      c.segs.sw[i] = mats[i].sw;
      c.segs.n[i] = static_cast<int>(mats[i].n);
    }
    const int st = hip_status(launch_gemv(c, plan, static_cast<hipStream_t>(stream)), name);
    if (st != KOMP_OK) return st;
  }
  return KOMP_OK;
}

int gemv_multi_entry(int fmt, int count, const uint8_t* const* WQ, const int16_t* const* WS, float* const* Y,
                     const int64_t* N, const int64_t* SW, const int8_t* XQ, const float* XD, const float* X, int64_t M,
                     int64_t K, int block_n, int nb, int mode, int num_warps, void* stream) {
  static const char* const names[] = {"komp_q4_0_gemv_multi", "komp_tq2_0_gemv_multi", "komp_q8_0_gemv_multi",
                                      "komp_iq4_nl_gemv_multi", "komp_q4_k_gemv_multi"};
  const char* name = names[fmt];
  if (count < 1 || count > kMaxSegs) return fail(KOMP_EINVAL, "%s: count=%d must be 1..%d", name, count, kMaxSegs);
  if (WQ == nullptr || WS == nullptr || Y == nullptr || N == nullptr || SW == nullptr)
    return fail(KOMP_EINVAL, "%s: the WQ, WS, Y, N and SW arrays must not be NULL", name);
  if ((X != nullptr) == (XQ != nullptr || XD != nullptr))
    return fail(KOMP_EINVAL, "%s: give either XQ and XD (q8 input) or X (f32 input)", name);
  GemvMat mats[kMaxSegs];
  for (int i = 0; i < count; ++i) mats[i] = GemvMat{WQ[i], WS[i], Y[i], nullptr, N[i], SW[i]};
  const GemvArgs a{mats, count, XQ, XD, X, nullptr, nullptr, nullptr};
  return gemv_entry(fmt, X != nullptr, name, a, M, K, block_n, nb, mode, num_warps, stream);
}

}  // namespace

Timing timing_slot(int kind) {
  Timing t{false, nullptr, nullptr};
  if (!g_timing.on.load(std::memory_order_relaxed)) return t;
  std::lock_guard<std::mutex> lock(g_timing.mu);
  if (!g_timing.on || g_timing.used >= g_timing.max) return t;
  const size_t i = static_cast<size_t>(g_timing.used);
  while (g_timing.events.size() < 2 * (i + 1)) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return t;
    g_timing.events.push_back(e);
  }
  if (g_timing.kinds.size() <= i) g_timing.kinds.resize(i + 1);
  g_timing.kinds[i] = kind;
  g_timing.used++;
  t.on = true;
  t.start = g_timing.events[2 * i];
  t.stop = g_timing.events[2 * i + 1];
  return t;
}

int device_cu_count() { return device_cus(); }

bool stamps_on() { return g_stamps.on.load(std::memory_order_relaxed); }

uint32_t* stamp_slot(int64_t words) {
  if (!stamps_on()) return nullptr;
  std::lock_guard<std::mutex> lock(g_stamps.mu);
  if (!g_stamps.on || words <= 0 || g_stamps.used + words > g_stamps.words) return nullptr;
  uint32_t* p = g_stamps.buf + g_stamps.used;
  g_stamps.used += (words + 3) & ~int64_t{3};  // the next launch's header stays 16-byte aligned
  return p;
}

}  // namespace komp

using namespace komp;

extern "C" {

int komp_abi_version(void) { return KOMP_ABI_VERSION; }

const char* komp_last_error(void) { return g_error.c_str(); }

int komp_quant_q8_0(const float* X, int8_t* XQ, float* XD, int64_t M, int64_t K, int bb, void* stream) {
  if (M < 0 || K < 0) return fail(KOMP_EINVAL, "komp_quant_q8_0: negative size");
  if (K % 32) return fail(KOMP_EINVAL, "komp_quant_q8_0: K=%lld is not a multiple of 32", (long long)K);
  if (bb < 1) return fail(KOMP_EINVAL, "komp_quant_q8_0: bb=%d must be >= 1", bb);
  const int64_t nblocks = M * (K / 32);
  if (nblocks == 0) return KOMP_OK;
  if (X == nullptr || XQ == nullptr || XD == nullptr) return fail(KOMP_EINVAL, "komp_quant_q8_0: NULL pointer");
  if (!aligned(X, 16) || !aligned(XQ, 4) || !aligned(XD, 4))
    return fail(KOMP_EINVAL, "komp_quant_q8_0: X must be 16-byte aligned, XQ and XD 4-byte aligned");
  return hip_status(launch_quant_q8_0(X, XQ, XD, nblocks, static_cast<hipStream_t>(stream)), "komp_quant_q8_0");
}

int komp_quant_q8_K(const float* X, int8_t* XQ, float* XD, int16_t* XB, int64_t M, int64_t K, void* stream) {
  if (M < 0 || K < 0) return fail(KOMP_EINVAL, "komp_quant_q8_K: negative size");
  if (K % 256) return fail(KOMP_EINVAL, "komp_quant_q8_K: K=%lld is not a multiple of 256", (long long)K);
  const int64_t nblocks = M * (K / 256);
  if (nblocks == 0) return KOMP_OK;
  if (X == nullptr || XQ == nullptr || XD == nullptr) return fail(KOMP_EINVAL, "komp_quant_q8_K: NULL pointer");
  if (!aligned(X, 16) || !aligned(XQ, 16) || !aligned(XD, 4) || !aligned(XB, 2))
    return fail(KOMP_EINVAL, "komp_quant_q8_K: X and XQ must be 16-byte aligned, XD 4-byte, XB 2-byte aligned");
  return hip_status(launch_quant_q8_K(X, XQ, XD, XB, nblocks, static_cast<hipStream_t>(stream)), "komp_quant_q8_K");
}

int komp_q4_0_gemv(const uint8_t* WQ, const int16_t* WS, const int8_t* XQ, const float* XD, float* Y, int32_t* S,
                   int64_t M, int64_t N, int64_t K, int64_t SW, int block_n, int nb, int mode, int num_warps,
                   void* stream) {
  const GemvMat w{WQ, WS, Y, S, N, SW};
  const GemvArgs a{&w, 1, XQ, XD, nullptr, nullptr, nullptr, nullptr};
  return gemv_entry(FMT_Q4_0, false, "komp_q4_0_gemv", a, M, K, block_n, nb, mode, num_warps, stream);
}

int komp_tq2_0_gemv(const uint8_t* WQ, const int16_t* WS, const int8_t* XQ, const float* XD, float* Y, int32_t* S,
                    int64_t M, int64_t N, int64_t K, int64_t SW, int block_n, int nb, int mode, int num_warps,
                    void* stream) {
  const GemvMat w{WQ, WS, Y, S, N, SW};
  const GemvArgs a{&w, 1, XQ, XD, nullptr, nullptr, nullptr, nullptr};
  return gemv_entry(FMT_TQ2_0, false, "komp_tq2_0_gemv", a, M, K, block_n, nb, mode, num_warps, stream);
}

int komp_q4_0_gemv_f32(const uint8_t* WQ, const int16_t* WS, const float* X, float* Y, int32_t* S, int8_t* XQ,
                       float* XD, int16_t* XB, int64_t M, int64_t N, int64_t K, int64_t SW, int block_n, int nb,
                       int mode, int num_warps, void* stream) {
  const GemvMat w{WQ, WS, Y, S, N, SW};
  const GemvArgs a{&w, 1, nullptr, nullptr, X, XQ, XD, XB};
  return gemv_entry(FMT_Q4_0, true, "komp_q4_0_gemv_f32", a, M, K, block_n, nb, mode, num_warps, stream);
}

int komp_tq2_0_gemv_f32(const uint8_t* WQ, const int16_t* WS, const float* X, float* Y, int32_t* S, int8_t* XQ,
                        float* XD, int16_t* XB, int64_t M, int64_t N, int64_t K, int64_t SW, int block_n, int nb,
                        int mode, int num_warps, void* stream) {
  const GemvMat w{WQ, WS, Y, S, N, SW};
  const GemvArgs a{&w, 1, nullptr, nullptr, X, XQ, XD, XB};
  return gemv_entry(FMT_TQ2_0, true, "komp_tq2_0_gemv_f32", a, M, K, block_n, nb, mode, num_warps, stream);
}

namespace {
int split_entry(int fmt, const char* name, const uint8_t* W, uint8_t* WQ, int16_t* WS, int64_t N, int64_t K,
                int64_t SW, void* stream) {
  const int blk = fmt_info(fmt).block;
  const int64_t qbytes = fmt_info(fmt).qbytes;
  if (N < 0 || K < 0) return fail(KOMP_EINVAL, "%s: negative size (N=%lld K=%lld)", name, (long long)N, (long long)K);
  if (K % blk) return fail(KOMP_EINVAL, "%s: K=%lld is not a multiple of the %d-value block", name, (long long)K, blk);
  if (K > INT32_MAX) return fail(KOMP_EINVAL, "%s: K must be < 2^31", name);
  const int64_t row_bytes = K / blk * qbytes;
  if (N > 0 && (SW < row_bytes || SW % 16))
    return fail(KOMP_EINVAL, "%s: SW=%lld must be a multiple of 16 and >= %lld (the quant bytes of a row)", name,
                (long long)SW, (long long)row_bytes);
  if (N == 0 || K == 0) return KOMP_OK;
  if (W == nullptr || WQ == nullptr || WS == nullptr) return fail(KOMP_EINVAL, "%s: NULL pointer", name);
  if (!aligned(W, 4) || !aligned(WQ, 16) || !aligned(WS, fmt == FMT_Q4_K ? 16 : 2))
    return fail(KOMP_EINVAL, "%s: W must be 4-byte aligned, WQ 16-byte aligned, WS %d-byte aligned", name,
                fmt == FMT_Q4_K ? 16 : 2);
  return hip_status(launch_split(fmt, W, WQ, WS, N, K, SW, static_cast<hipStream_t>(stream)), name);
}
}  // namespace

int komp_q4_0_split(const uint8_t* W, uint8_t* WQ, int16_t* WS, int64_t N, int64_t K, int64_t SW, void* stream) {
  return split_entry(FMT_Q4_0, "komp_q4_0_split", W, WQ, WS, N, K, SW, stream);
}

int komp_tq2_0_split(const uint8_t* W, uint8_t* WQ, int16_t* WS, int64_t N, int64_t K, int64_t SW, void* stream) {
  return split_entry(FMT_TQ2_0, "komp_tq2_0_split", W, WQ, WS, N, K, SW, stream);
}

int komp_q4_0_gemm(const uint8_t* WQ, const int16_t* WS, const int8_t* XQ, const float* XD, float* Y, int32_t* S,
                   int64_t M, int64_t N, int64_t K, int64_t SW, void* stream) {
  const GemvMat w{WQ, WS, Y, S, N, SW};
  const GemvArgs a{&w, 1, XQ, XD, nullptr, nullptr, nullptr, nullptr};
  return gemv_entry(FMT_Q4_0, false, "komp_q4_0_gemm", a, M, K, 0, 0, KOMP_MODE_DP4A, 0, stream, kRouteGemm);
}

int komp_tq2_0_gemm(const uint8_t* WQ, const int16_t* WS, const int8_t* XQ, const float* XD, float* Y, int32_t* S,
                    int64_t M, int64_t N, int64_t K, int64_t SW, void* stream) {
  const GemvMat w{WQ, WS, Y, S, N, SW};
  const GemvArgs a{&w, 1, XQ, XD, nullptr, nullptr, nullptr, nullptr};
  return gemv_entry(FMT_TQ2_0, false, "komp_tq2_0_gemm", a, M, K, 0, 0, KOMP_MODE_DP4A, 0, stream, kRouteGemm);
}

int komp_gemm_plan(int fmt, int64_t M, int64_t N, int64_t K, int64_t SW, int* rows_per_wg, int* cols_per_wg,
                   int* waves) {
  if (fmt < FMT_Q4_0 || fmt > FMT_Q4_K) return fail(KOMP_EINVAL, "komp_gemm_plan: fmt=%d", fmt);
  if (M < 1 || N < 0 || K < 0 || SW < 0) return fail(KOMP_EINVAL, "komp_gemm_plan: bad argument");
  GemmPlan p;
  if (!gemm_plan(fmt, M < kGemmMaxCols ? M : kGemmMaxCols, N, K, SW, &p))
    return fail(KOMP_EINVAL, "komp_gemm_plan: K=%lld / SW=%lld past the GEMM's limits", (long long)K, (long long)SW);
  if (rows_per_wg != nullptr) *rows_per_wg = 16 * p.wn * p.wr;
  if (cols_per_wg != nullptr) *cols_per_wg = 16 * p.cn;
  if (waves != nullptr) *waves = p.wk * p.wr;
  return KOMP_OK;
}

int komp_gemv_mfma_plan(int fmt, int fused, int mode, int64_t M, int64_t N, int64_t K, int64_t SW, int* rows_per_wg,
                        int* waves) {
  if (fmt < FMT_Q4_0 || fmt > FMT_Q4_K) return fail(KOMP_EINVAL, "komp_gemv_mfma_plan: fmt=%d", fmt);
  if (M < 0 || N < 0 || K < 0 || SW < 0) return fail(KOMP_EINVAL, "komp_gemv_mfma_plan: bad argument");
  MfmaPlan p;
  const bool on = mode == KOMP_MODE_DP4A && fmt == FMT_TQ2_0 && tq2_mfma_plan(M, N, K, SW, fused != 0, &p);
  if (rows_per_wg != nullptr) *rows_per_wg = on ? p.rows : 0;
  if (waves != nullptr) *waves = on ? p.waves : 0;
  return on ? 1 : 0;
}

int komp_q4_0_gemv_multi(int count, const uint8_t* const* WQ, const int16_t* const* WS, float* const* Y,
                         const int64_t* N, const int64_t* SW, const int8_t* XQ, const float* XD, const float* X,
                         int64_t M, int64_t K, int block_n, int nb, int mode, int num_warps, void* stream) {
  return gemv_multi_entry(FMT_Q4_0, count, WQ, WS, Y, N, SW, XQ, XD, X, M, K, block_n, nb, mode, num_warps, stream);
}

int komp_tq2_0_gemv_multi(int count, const uint8_t* const* WQ, const int16_t* const* WS, float* const* Y,
                          const int64_t* N, const int64_t* SW, const int8_t* XQ, const float* XD, const float* X,
                          int64_t M, int64_t K, int block_n, int nb, int mode, int num_warps, void* stream) {
  return gemv_multi_entry(FMT_TQ2_0, count, WQ, WS, Y, N, SW, XQ, XD, X, M, K, block_n, nb, mode, num_warps, stream);
}

// ---- Q8_0 and IQ4_NL (q8_0 activations): the same entries as Q4_0's ----
#define KOMP_FORMAT_ENTRIES(F, FMT)                                                                                   \
  int komp_##F##_gemv(const uint8_t* WQ, const int16_t* WS, const int8_t* XQ, const float* XD, float* Y, int32_t* S,  \
                      int64_t M, int64_t N, int64_t K, int64_t SW, int block_n, int nb, int mode, int num_warps,      \
                      void* stream) {                                                                                 \
    const GemvMat w{WQ, WS, Y, S, N, SW};                                                                             \
    const GemvArgs a{&w, 1, XQ, XD, nullptr, nullptr, nullptr, nullptr};                                              \
    return gemv_entry(FMT, false, "komp_" #F "_gemv", a, M, K, block_n, nb, mode, num_warps, stream);               \
  }                                                                                                                   \
  int komp_##F##_gemv_f32(const uint8_t* WQ, const int16_t* WS, const float* X, float* Y, int32_t* S, int8_t* XQ,     \
                          float* XD, int64_t M, int64_t N, int64_t K, int64_t SW, int block_n, int nb, int mode,      \
                          int num_warps, void* stream) {                                                              \
    const GemvMat w{WQ, WS, Y, S, N, SW};                                                                             \
    const GemvArgs a{&w, 1, nullptr, nullptr, X, XQ, XD, nullptr};                                                    \
    return gemv_entry(FMT, true, "komp_" #F "_gemv_f32", a, M, K, block_n, nb, mode, num_warps, stream);            \
  }                                                                                                                   \
  int komp_##F##_gemv_multi(int count, const uint8_t* const* WQ, const int16_t* const* WS, float* const* Y,           \
                            const int64_t* N, const int64_t* SW, const int8_t* XQ, const float* XD, const float* X,   \
                            int64_t M, int64_t K, int block_n, int nb, int mode, int num_warps, void* stream) {       \
    return gemv_multi_entry(FMT, count, WQ, WS, Y, N, SW, XQ, XD, X, M, K, block_n, nb, mode, num_warps, stream);   \
  }                                                                                                                   \
  int komp_##F##_gemm(const uint8_t* WQ, const int16_t* WS, const int8_t* XQ, const float* XD, float* Y, int32_t* S,  \
                      int64_t M, int64_t N, int64_t K, int64_t SW, void* stream) {                                    \
    const GemvMat w{WQ, WS, Y, S, N, SW};                                                                             \
    const GemvArgs a{&w, 1, XQ, XD, nullptr, nullptr, nullptr, nullptr};                                              \
    return gemv_entry(FMT, false, "komp_" #F "_gemm", a, M, K, 0, 0, KOMP_MODE_DP4A, 0, stream, kRouteGemm);        \
  }                                                                                                                   \
  int komp_##F##_split(const uint8_t* W, uint8_t* WQ, int16_t* WS, int64_t N, int64_t K, int64_t SW, void* stream) {  \
    return split_entry(FMT, "komp_" #F "_split", W, WQ, WS, N, K, SW, stream);                                        \
  }

KOMP_FORMAT_ENTRIES(q8_0, FMT_Q8_0)
KOMP_FORMAT_ENTRIES(iq4_nl, FMT_IQ4_NL)
#undef KOMP_FORMAT_ENTRIES

// ---- Q4_K (q8_K activations): TQ2_0's entries, S with two int32 per block ----
int komp_q4_k_gemv(const uint8_t* WQ, const int16_t* WS, const int8_t* XQ, const float* XD, float* Y, int32_t* S,
                   int64_t M, int64_t N, int64_t K, int64_t SW, int block_n, int nb, int mode, int num_warps,
                   void* stream) {
  const GemvMat w{WQ, WS, Y, S, N, SW};
  const GemvArgs a{&w, 1, XQ, XD, nullptr, nullptr, nullptr, nullptr};
  return gemv_entry(FMT_Q4_K, false, "komp_q4_k_gemv", a, M, K, block_n, nb, mode, num_warps, stream);
}

int komp_q4_k_gemv_f32(const uint8_t* WQ, const int16_t* WS, const float* X, float* Y, int32_t* S, int8_t* XQ,
                       float* XD, int16_t* XB, int64_t M, int64_t N, int64_t K, int64_t SW, int block_n, int nb,
                       int mode, int num_warps, void* stream) {
  const GemvMat w{WQ, WS, Y, S, N, SW};
  const GemvArgs a{&w, 1, nullptr, nullptr, X, XQ, XD, XB};
  return gemv_entry(FMT_Q4_K, true, "komp_q4_k_gemv_f32", a, M, K, block_n, nb, mode, num_warps, stream);
}

int komp_q4_k_gemv_multi(int count, const uint8_t* const* WQ, const int16_t* const* WS, float* const* Y,
                         const int64_t* N, const int64_t* SW, const int8_t* XQ, const float* XD, const float* X,
                         int64_t M, int64_t K, int block_n, int nb, int mode, int num_warps, void* stream) {
  return gemv_multi_entry(FMT_Q4_K, count, WQ, WS, Y, N, SW, XQ, XD, X, M, K, block_n, nb, mode, num_warps, stream);
}

int komp_q4_k_gemm(const uint8_t* WQ, const int16_t* WS, const int8_t* XQ, const float* XD, float* Y, int32_t* S,
                   int64_t M, int64_t N, int64_t K, int64_t SW, void* stream) {
  const GemvMat w{WQ, WS, Y, S, N, SW};
  const GemvArgs a{&w, 1, XQ, XD, nullptr, nullptr, nullptr, nullptr};
  return gemv_entry(FMT_Q4_K, false, "komp_q4_k_gemm", a, M, K, 0, 0, KOMP_MODE_DP4A, 0, stream, kRouteGemm);
}

int komp_q4_k_split(const uint8_t* W, uint8_t* WQ, int16_t* WS, int64_t N, int64_t K, int64_t SW, void* stream) {
  return split_entry(FMT_Q4_K, "komp_q4_k_split", W, WQ, WS, N, K, SW, stream);
}

int komp_gemv_auto_config(int fmt, int fused, int mode, int64_t M, int64_t N, int64_t K, int* block_n, int* nb,
                          int* num_warps, int* lanes_per_row, int* passes) {
  if (fmt < FMT_Q4_0 || fmt > FMT_Q4_K) return fail(KOMP_EINVAL, "komp_gemv_auto_config: fmt=%d", fmt);
  if (mode < KOMP_MODE_BYTES || mode > KOMP_MODE_DP4A)
    return fail(KOMP_EINVAL, "komp_gemv_auto_config: mode=%d not in {0,1,2}", mode);
  if (M < 1 || N < 0 || K < 0 || block_n == nullptr || nb == nullptr || num_warps == nullptr)
    return fail(KOMP_EINVAL, "komp_gemv_auto_config: bad argument");
  const GemvPlan plan = auto_plan(fmt, fused != 0, mode, M, N, K);
  *block_n = plan.block_n;
  *nb = plan.nb;
  *num_warps = plan.waves;
  if (lanes_per_row != nullptr) *lanes_per_row = 1 << plan.lpr_log2;
  if (passes != nullptr) *passes = plan.passes;
  return KOMP_OK;
}

int komp_dp4a_probe(const int32_t* A, const int32_t* B, const int32_t* C, int32_t* OUT, int64_t n, int mode,
                    void* stream) {
  if (n < 0) return fail(KOMP_EINVAL, "komp_dp4a_probe: negative n");
  if (mode != KOMP_MODE_DP4A && mode != KOMP_MODE_DP4A_EMU)
    return fail(KOMP_EINVAL, "komp_dp4a_probe: mode=%d must be 1 (emulated) or 2 (v_dot4c_i32_i8)", mode);
  if (n == 0) return KOMP_OK;
  if (!A || !B || !C || !OUT) return fail(KOMP_EINVAL, "komp_dp4a_probe: NULL pointer");
  return hip_status(launch_dp4a_probe(A, B, C, OUT, n, mode, static_cast<hipStream_t>(stream)), "komp_dp4a_probe");
}

int komp_stream_read(const void* SRC, int64_t bytes, uint32_t* OUT, void* stream) {
  if (bytes < 0 || bytes % 16) return fail(KOMP_EINVAL, "komp_stream_read: bytes=%lld must be a multiple of 16", static_cast<long long>(bytes));
  if (bytes / 16 > (int64_t{1} << 42)) return fail(KOMP_EINVAL, "komp_stream_read: bytes too large");
  if (bytes == 0) return KOMP_OK;
  if (!SRC || !OUT) return fail(KOMP_EINVAL, "komp_stream_read: NULL pointer");
  if (!aligned(SRC, 16) || !aligned(OUT, 4)) return fail(KOMP_EINVAL, "komp_stream_read: SRC must be 16-byte and OUT 4-byte aligned");
  return hip_status(launch_stream_read(SRC, bytes, OUT, static_cast<hipStream_t>(stream)), "komp_stream_read");
}

int komp_clock(uint64_t* OUT, void* stream) {
  if (!OUT || !aligned(OUT, 8)) return fail(KOMP_EINVAL, "komp_clock: OUT must be an 8-byte aligned device pointer");
  return hip_status(launch_clock(OUT, static_cast<hipStream_t>(stream)), "komp_clock");
}

int komp_clock_khz(int* khz) {
  if (!khz) return fail(KOMP_EINVAL, "komp_clock_khz: NULL pointer");
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, dev);
  return hip_status(e, "komp_clock_khz");
}

int komp_q4_0_decode(const uint8_t* WQ, int32_t* OUT, int64_t R, void* stream) {
  if (R < 0) return fail(KOMP_EINVAL, "komp_q4_0_decode: negative R");
  if (R == 0) return KOMP_OK;
  if (!WQ || !OUT || !aligned(WQ, 16)) return fail(KOMP_EINVAL, "komp_q4_0_decode: WQ must be 16-byte aligned");
  return hip_status(launch_q4_0_decode(WQ, OUT, R, static_cast<hipStream_t>(stream)), "komp_q4_0_decode");
}

int komp_tq2_0_decode(const uint8_t* WQ, int32_t* OUT, int64_t nblk, void* stream) {
  if (nblk < 0) return fail(KOMP_EINVAL, "komp_tq2_0_decode: negative nblk");
  if (nblk == 0) return KOMP_OK;
  if (!WQ || !OUT || !aligned(WQ, 16)) return fail(KOMP_EINVAL, "komp_tq2_0_decode: WQ must be 16-byte aligned");
  return hip_status(launch_tq2_0_decode(WQ, OUT, nblk, static_cast<hipStream_t>(stream)), "komp_tq2_0_decode");
}

int komp_timing_begin(int64_t max_dispatches) {
  if (max_dispatches < 0) return fail(KOMP_EINVAL, "komp_timing_begin: negative max_dispatches");
  std::lock_guard<std::mutex> lock(g_timing.mu);
  g_timing.max = max_dispatches;
  g_timing.used = 0;
  g_timing.on = true;
  return KOMP_OK;
}

int komp_timing_end(double* ms, int64_t* count) {
  std::lock_guard<std::mutex> lock(g_timing.mu);
  g_timing.on = false;
  for (int i = 0; i < KOMP_TIMING_KINDS; ++i) {
    if (ms) ms[i] = 0.0;
    if (count) count[i] = 0;
  }
  for (int64_t i = 0; i < g_timing.used; ++i) {
    hipEvent_t e0 = g_timing.events[2 * i], e1 = g_timing.events[2 * i + 1];
    hipError_t e = hipEventSynchronize(e1);
    if (e != hipSuccess) return hip_status(e, "komp_timing_end");
    float t = 0.0f;
    e = hipEventElapsedTime(&t, e0, e1);
    if (e != hipSuccess) return hip_status(e, "komp_timing_end");
    const int kd = g_timing.kinds[i];
    if (ms) ms[kd] += t;
    if (count) count[kd] += 1;
  }
  g_timing.used = 0;
  return KOMP_OK;
}

int komp_stamps_begin(uint32_t* buf, int64_t words) {
  if (words < 0 || (words > 0 && (buf == nullptr || !aligned(buf, 16))))
    return fail(KOMP_EINVAL, "komp_stamps_begin: buf must be 16-byte aligned and words >= 0");
  std::lock_guard<std::mutex> lock(g_stamps.mu);
  g_stamps.buf = buf;
  g_stamps.words = words;
  g_stamps.used = 0;
  g_stamps.on = true;
  return KOMP_OK;
}

int komp_stamps_end(int64_t* words_used, int* clock_khz) {
  std::lock_guard<std::mutex> lock(g_stamps.mu);
  g_stamps.on = false;
  if (words_used) *words_used = g_stamps.used;
  g_stamps.buf = nullptr;
  g_stamps.words = g_stamps.used = 0;
  if (clock_khz) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(clock_khz, hipDeviceAttributeWallClockRate, dev);
    if (e != hipSuccess) return hip_status(e, "komp_stamps_end");
  }
  return KOMP_OK;
}

}  // extern "C"
