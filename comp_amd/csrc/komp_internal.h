// Internal (C++) interface between the C-ABI layer (abi.hip) and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

namespace komp {

enum Fmt { FMT_Q4_0 = 0, FMT_TQ2_0 = 1, FMT_Q8_0 = 2, FMT_IQ4_NL = 3, FMT_Q4_K = 4 };

// Per-format constants: values per block, ggml block bytes, quant bytes per block and their offset, scale offset,
// scale-plane bytes per block (the f16 scale; Q4_K: d, dmin and the 12 bytes of 6-bit sub-block scales and mins).
struct FmtInfo {
  int block;
  int nbytes;
  int qbytes;
  int qoff;
  int soff;
  int sbytes;
};
inline FmtInfo fmt_info(int fmt) {
  switch (fmt) {
    case FMT_TQ2_0: return FmtInfo{256, 66, 64, 0, 64, 2};
    case FMT_Q8_0: return FmtInfo{32, 34, 32, 2, 0, 2};
    case FMT_Q4_K: return FmtInfo{256, 144, 128, 16, 0, 16};
    default: return FmtInfo{32, 18, 16, 2, 0, 2};  // Q4_0, IQ4_NL
  }
}
// int32 of S per block: the exact block dot, or (Q4_K) the scaled dot and the mins dot
inline int s_per_block(int fmt) { return fmt == FMT_Q4_K ? 2 : 1; }

// Kernel kinds, for the per-dispatch timing of the tuning harness.
enum Kind {
  KIND_QUANT_Q8_0 = 0,
  KIND_QUANT_Q8_K = 1,
  KIND_Q4_0_GEMV = 2,
  KIND_TQ2_0_GEMV = 3,
  KIND_PROBE = 4,
  KIND_Q8_0_GEMV = 5,
  KIND_IQ4_NL_GEMV = 6,
  KIND_Q4_K_GEMV = 7,
  KIND_COUNT = 8
};
// the timing kind of a weight format's GEMV / GEMM launches
constexpr int gemv_kind(int fmt) {
  return fmt == FMT_TQ2_0 ? KIND_TQ2_0_GEMV : fmt == FMT_Q8_0 ? KIND_Q8_0_GEMV
                                           : fmt == FMT_IQ4_NL ? KIND_IQ4_NL_GEMV
                                           : fmt == FMT_Q4_K  ? KIND_Q4_K_GEMV : KIND_Q4_0_GEMV;
}

// Work decomposition of one GEMV launch (gemv_kernel.h describes the mapping of block_n / nb / num_warps).
struct GemvPlan {
  int block_n;        // rows per workgroup
  int nb;             // 16-byte weight chunks each lane loads per row per K step
  int waves;          // wavefronts per workgroup (at most 8)
  int rows_per_wave;  // block_n / waves = (64 >> lpr_log2) * passes
  int lpr_log2;       // log2(lanes per row group)
  int passes;         // row groups each wave walks in sequence
};

// Several weight matrices that share one activation input, in one launch: segment i covers workgroups
// [first_wg[i], first_wg[i + 1]) (the last one up to the grid's end), and no workgroup straddles two matrices.
constexpr int kMaxSegs = 4;
struct GemvSegs {
  const uint8_t* wq[kMaxSegs];
  const int16_t* ws[kMaxSegs];
  float* y[kMaxSegs];
  int64_t sw[kMaxSegs];
  int n[kMaxSegs];
  int first_wg[kMaxSegs];
  uint32_t* stamps;  // the stamped TQ2_0 lean instantiations only: this launch's wave-stamp records (stamp_slot)
};

struct GemvCall {
  int fmt;
  const uint8_t* wq;
  const int16_t* ws;
  const int8_t* xq;   // q8 activations (unfused) ...
  const float* xd;
  const float* x;     // ... or f32 activations, quantized by every workgroup into LDS (fused)
  int8_t* xq_out;     // fused only, optional: the q8 planes as quant_q8_0 / quant_q8_K would write them
  float* xd_out;
  int16_t* xb_out;    // q8_K bsums, optional
  float* y;
  int32_t* s;
  int m;          // activation columns in this launch (1..3)
  int n;
  int k;
  int64_t sw;     // WQ row stride in bytes
  int mode;
  int nseg;       // 1: the single matrix above; 2..kMaxSegs: the matrices in segs (wq / ws / y / n / sw above unused)
  GemvSegs segs;  // first_wg is filled in at launch, from the plan
};

// Matrix-core GEMM (any number of activation columns): a workgroup of wk x wr waves covers wr row groups of wn
// 16-row tiles (wk waves split each group's K) and cn 16-column tiles; d K steps in flight per wave.
struct GemmPlan {
  int wk;
  int wr;
  int wn;
  int cn;
  int d;
};

struct GemmCall {
  int fmt;
  const uint8_t* wq;
  const int16_t* ws;
  const int8_t* xq;
  const float* xd;
  float* y;
  int32_t* s;
  int m;
  int n;
  int k;
  int64_t sw;
};

// The lean kernels' loop forms pipeline their weight loads (a second kernel form) for one column when a wave walks this
// many tiles (passes x K steps) or more: the reference's knob plans, whose small workgroups walk whole rows in narrow
// steps.  With fewer, the second buffer's registers cost more occupancy than the prefetch saves.
constexpr int kPipeMinTiles = 3;

// The lean kernels address one pass of a wave's rows with 32-bit per-lane offsets inside a buffer descriptor whose
// range is capped at 0x7FFFFFF0 bytes, so every matrix's `rows_per_pass` row strides must fit below the cap; other
// strides take the general kernel, which addresses rows in 64 bits.
inline bool lean_strides_fit(const GemvCall& c, int rows_per_pass) {
  constexpr int64_t kCap = 0x7FFFFFF0;
  if (c.nseg <= 1) return rows_per_pass * c.sw <= kCap;
  for (int i = 0; i < c.nseg; ++i)
    if (rows_per_pass * c.segs.sw[i] > kCap) return false;
  return true;
}

// Dynamic LDS above 64 KiB has to be allowed per kernel, on each device.  `limit` is one kernel's cache of the
// largest size allowed so far, per device: the fast path reads it without a lock, and raising it happens under a
// lock, so the allowed size only grows and a thread that sees a large enough value may launch at once.
constexpr int kMaxDevices = 64;
inline std::mutex& dynamic_lds_mutex() {
  static std::mutex mu;
  return mu;
}
inline hipError_t allow_dynamic_lds(const void* kernel, size_t bytes, std::atomic<unsigned> (&limit)[kMaxDevices]) {
  if (bytes <= 64 * 1024) return hipSuccess;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const bool cached = dev >= 0 && dev < kMaxDevices;
  if (cached && limit[dev].load(std::memory_order_acquire) >= bytes) return hipSuccess;
  std::lock_guard<std::mutex> lock(dynamic_lds_mutex());
  if (cached && limit[dev].load(std::memory_order_relaxed) >= bytes) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
  if (e == hipSuccess && cached) limit[dev].store(static_cast<unsigned>(bytes), std::memory_order_release);
  return e;
}

// Dispatch hook: every launch goes through it so the tuning harness can time dispatches with hipExtLaunchKernel events.
struct Timing {
  bool on;
  hipEvent_t start;
  hipEvent_t stop;
};
Timing timing_slot(int kind);   // defined in abi.hip

// In-kernel wave stamps of the tuning harness (komp_stamps_begin / komp_stamps_end in abi.hip): whether stamping is
// on, and a launch's records, `words` words of the caller's stamp buffer (nullptr when stamping is off or the buffer
// has no room left; the launch then runs unstamped).  Record layout: a header {kStampMagic, waves, N, K}, then
// {entry, staged, dots, stored} per wave, each the low 32 bits of the real-time counter.
constexpr uint32_t kStampMagic = 0x4B535450u;
bool stamps_on();
uint32_t* stamp_slot(int64_t words);

int device_cu_count();  // CUs of the current device (256 on MI355X, and when no device can be queried)
size_t gemv_lds_bytes(int fmt, int m, int k);
hipError_t launch_gemv(const GemvCall& c, const GemvPlan& p, hipStream_t stream);
hipError_t launch_gemv_fused(const GemvCall& c, const GemvPlan& p, hipStream_t stream);
hipError_t launch_gemv_more(const GemvCall& c, const GemvPlan& p, hipStream_t stream);
hipError_t launch_gemv_more_fused(const GemvCall& c, const GemvPlan& p, hipStream_t stream);
hipError_t launch_gemv_q4_k(const GemvCall& c, const GemvPlan& p, hipStream_t stream);
hipError_t launch_gemv_q4_k_fused(const GemvCall& c, const GemvPlan& p, hipStream_t stream);
// TQ2_0, 1-3 columns in dp4a and bytes modes (gemv_tq2.hip, gemv_tq2_bytes.hip): the plans it runs, its LDS bytes
// and its launch
bool tq2_lean_eligible(const GemvCall& c, const GemvPlan& p);
size_t tq2_lean_lds_bytes(int lpr, int nb, int mc, int k, bool fused, int threads, bool bytes);
// several q8 columns staged in more than one pass of the workgroup's threads go through LDS as they are in memory
bool tq2_lean_dma(int lpr, int nb, int mc, int k, bool fused, int threads, bool bytes);
hipError_t launch_gemv_tq2_lean(const GemvCall& c, const GemvPlan& p, hipStream_t stream);
hipError_t launch_gemv_tq2_lean_bytes(const GemvCall& c, const GemvPlan& p, hipStream_t stream);
// the stamped instantiations (gemv_tq2_stamp.hip): dp4a plans with one pass and one K step, no global -> LDS copy
bool tq2_lean_stampable(const GemvCall& c, const GemvPlan& p);
hipError_t launch_gemv_tq2_lean_stamped(const GemvCall& c, const GemvPlan& p, hipStream_t stream);
// Q4_0 and IQ4_NL, 1-3 columns in dp4a mode (gemv_q4.hip), and Q4_0 in bytes mode (gemv_q4_bytes.hip)
bool q8_lean_eligible(const GemvCall& c, const GemvPlan& p);
size_t q8_lean_lds_bytes(int lpr, int nb, int mc, int k);
hipError_t launch_gemv_q8_lean(const GemvCall& c, const GemvPlan& p, hipStream_t stream);
hipError_t launch_gemv_q8_lean_fused(const GemvCall& c, const GemvPlan& p, hipStream_t stream);

// TQ2_0, three columns in dp4a mode, q8_K or f32 in, on the matrix cores (gemv_tq2_mfma.hip): workgroups of `rows`
// rows in `tiles` 16-row tiles (rows <= 16 tiles) whose `waves` waves split K into ranges of at most `nbw` blocks
struct MfmaPlan {
  int tiles;
  int waves;
  int nbw;
  int rows;
};
size_t tq2_mfma_lds_bytes(int tiles, int nbw, int mc, bool fused, int waves);
bool tq2_mfma_eligible(const GemvCall& c, const MfmaPlan& p);
hipError_t launch_gemv_tq2_mfma(const GemvCall& c, const MfmaPlan& p, hipStream_t stream);

bool q4k_lean_eligible(const GemvCall& c, const GemvPlan& p);
size_t q4k_lean_lds_bytes(int lpr, int nb, int mc, int k);
hipError_t launch_gemv_q4k_lean(const GemvCall& c, const GemvPlan& p, hipStream_t stream);
hipError_t launch_gemv_q4k_lean_fused(const GemvCall& c, const GemvPlan& p, hipStream_t stream);

bool q4_lean_eligible(const GemvCall& c, const GemvPlan& p);
size_t q4_lean_lds_bytes(int g, int nb, int mc, int k, bool bytes);
hipError_t launch_gemv_q4_lean(const GemvCall& c, const GemvPlan& p, hipStream_t stream);
hipError_t launch_gemv_q4_lean_bytes(const GemvCall& c, const GemvPlan& p, hipStream_t stream);
size_t gemm_lds_bytes(int fmt, const GemmPlan& p, int k);
hipError_t launch_gemm(const GemmCall& c, const GemmPlan& p, hipStream_t stream);
hipError_t launch_split(int fmt, const uint8_t* w, uint8_t* wq, int16_t* ws, int64_t n, int64_t k, int64_t sw,
                        hipStream_t stream);
hipError_t launch_quant_q8_0(const float* x, int8_t* xq, float* xd, int64_t nblocks, hipStream_t stream);
hipError_t launch_quant_q8_K(const float* x, int8_t* xq, float* xd, int16_t* xb, int64_t nblocks, hipStream_t stream);
hipError_t launch_stream_read(const void* src, int64_t bytes, uint32_t* out, hipStream_t stream);
hipError_t launch_clock(uint64_t* out, hipStream_t stream);
hipError_t launch_dp4a_probe(const int32_t* a, const int32_t* b, const int32_t* c, int32_t* out, int64_t n, int mode,
                             hipStream_t stream);
hipError_t launch_q4_0_decode(const uint8_t* wq, int32_t* out, int64_t rows, hipStream_t stream);
hipError_t launch_tq2_0_decode(const uint8_t* wq, int32_t* out, int64_t nblk, hipStream_t stream);

}  // namespace komp
