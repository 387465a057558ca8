// Weight ingestion on the device: ggml block bytes -> KURN's split planes, the device counterpart of the reference's
// host.split (src/komp/host.py:16-22).
//
// W holds N rows of K/blk ggml blocks, each `nbytes` long (Q4_0 and IQ4_NL: f16 d then 16 quant bytes, 18 bytes;
// Q8_0: f16 d then 32 int8, 34 bytes; TQ2_0: 64 quant bytes then f16 d, 66 bytes; Q4_K: f16 d, f16 dmin, 12 scale
// bytes, 128 quant bytes, 144 bytes).  Outputs: WQ u8 [N][SW] (the quant bytes of row r at WQ + r*SW, blocks in
// order) and WS i16 [N][K/blk] (the f16 bit patterns; Q4_K: [N][8 K/256], each block's first 16 bytes).  Pure byte
// movement, so the planes equal host.split's bit for bit.
//
// One thread per 16-byte chunk of WQ (Q4_0, IQ4_NL: one per block, Q8_0: two, TQ2_0: four, Q4_K: eight).  A chunk's 16 source
// bytes start at an address that is 2 mod 4 for every other block (18-, 34- and 66-byte blocks), so the thread loads the aligned words that
// cover them and funnel-shifts them into place (v_alignbyte_b32); consecutive threads read consecutive 16-18 byte
// windows, so each wave's loads cover contiguous memory.  The loads go through a buffer descriptor whose range ends at
// the launch's last byte, so nothing is read past the tensor.
// The thread of chunk 0 also moves the block's scale-plane bytes (2, or Q4_K's 16 in one 16-byte load and store).  HBM-bound: it reads each ggml byte once and writes
// each plane byte once.
#include <hip/hip_ext.h>

#include "komp_device.h"
#include "komp_internal.h"

namespace komp {
namespace split_impl {

constexpr int kRsrcWord3 = 0x00020000;  // buffer descriptor word 3 on gfx9: 32-bit data, no swizzle
constexpr int kThreads = 256;

// chunks: WQ chunks in this launch (blocks * chunks per block); nblk: blocks per row; cpb_log2: log2(chunks per
// block); nbytes, qoff, soff: the ggml block's size, quant offset and scale offset; wbytes: the launch's ggml bytes.
// W, WQ and WS point at the launch's first row.
__global__ void __launch_bounds__(kThreads)
split_kernel(int chunks, int nblk, int cpb_log2, int nbytes, int qoff, int soff, int sbytes, int wbytes, int64_t SW,
             const uint8_t* __restrict__ W, uint8_t* __restrict__ WQ, int16_t* __restrict__ WS) {
  const int t = blockIdx.x * kThreads + threadIdx.x;
  if (t >= chunks) return;
  const auto w = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(W), 0, wbytes, kRsrcWord3);
  const int b = t >> cpb_log2;            // block within the launch
  const int c = t & ((1 << cpb_log2) - 1);  // chunk within the block
  const int row = b / nblk;
  const int col = b - row * nblk;
  // src is even (block sizes and offsets are even), so the window starts 0 or 2 bytes into its first dword and needs
  // at most the low half of a fifth one.  That half is a 2-byte load: a 4-byte load that crosses the descriptor's end
  // returns zero whole, which would drop the last block's last two bytes.
  const unsigned src = static_cast<unsigned>(b * nbytes + qoff + 16 * c);
  const unsigned a = src & ~3u;
  const unsigned sh = src & 3u;
  unsigned d[5];
#pragma unroll
  for (int i = 0; i < 4; ++i) d[i] = __builtin_amdgcn_raw_buffer_load_b32(w, a + 4 * i, 0, 0);
  d[4] = __builtin_amdgcn_raw_buffer_load_b16(w, a + 16, 0, 0);
  u32x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], sh);
  *reinterpret_cast<u32x4*>(WQ + row * SW + (static_cast<int64_t>(col) << (cpb_log2 + 4)) + 16 * c) = o;
  if (c == 0) {
    const unsigned so = static_cast<unsigned>(b * nbytes + soff);
    if (sbytes == 16)  // Q4_K: 144-byte blocks, so the 16 bytes start 16-byte aligned
      *reinterpret_cast<u32x4*>(WS + 8 * b) = __builtin_amdgcn_raw_buffer_load_b128(w, so, 0, 0);
    else
      WS[b] = static_cast<int16_t>(__builtin_amdgcn_raw_buffer_load_b16(w, so, 0, 0));
  }
}

}  // namespace split_impl

// Rows are launched in batches whose ggml bytes stay below 2^31 (32-bit buffer offsets).
hipError_t launch_split(int fmt, const uint8_t* w, uint8_t* wq, int16_t* ws, int64_t n, int64_t k, int64_t sw,
                        hipStream_t stream) {
  const FmtInfo f = fmt_info(fmt);
  const int blk = f.block;
  const int nbytes = f.nbytes;
  const int qoff = f.qoff;
  const int soff = f.soff;
  const int cpb_log2 = f.qbytes == 16 ? 0 : f.qbytes == 32 ? 1 : f.qbytes == 64 ? 2 : 3;  // 16-byte chunks per block
  const int64_t nblk = k / blk;
  const int64_t row_bytes = nblk * nbytes;
  int64_t rows_per = row_bytes > 0 ? (int64_t{1} << 30) / row_bytes : n;
  if (rows_per < 1) rows_per = 1;
  for (int64_t r0 = 0; r0 < n; r0 += rows_per) {
    const int64_t rows = n - r0 < rows_per ? n - r0 : rows_per;
    const int64_t chunks = rows * nblk << cpb_log2;
    if (chunks == 0) continue;
    const dim3 grid(static_cast<unsigned>((chunks + split_impl::kThreads - 1) / split_impl::kThreads));
    const Timing tm = timing_slot(KIND_PROBE);
    hipExtLaunchKernelGGL(split_impl::split_kernel, grid, dim3(split_impl::kThreads), 0, stream, tm.start, tm.stop, 0,
                          static_cast<int>(chunks), static_cast<int>(nblk), cpb_log2, nbytes, qoff, soff, f.sbytes,
                          static_cast<int>(rows * row_bytes), sw, w + r0 * row_bytes, wq + r0 * sw,
                          ws + r0 * nblk * (f.sbytes / 2));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace komp
