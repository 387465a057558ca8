// Activation quantizers (q8_0, q8_K) and the probe kernels, for gfx950.
//
// Replaces src/komp/kernels.py:22-45 (quant_q8_0, quant_q8_K) and :145-170 (dp4a_probe, q4_0_decode, tq2_0_decode).
// The arithmetic is ggml's reference quantizers as restated in patches/0001-language-extra-kurn.patch:104-131, with
// correctly rounded f32 division (v_div_scale/fmas/fixup, never a bare v_rcp_f32), f32 denormals preserved, and
// round-to-nearest-even f32 -> f16 conversion; so the bytes equal the reference's bytes exactly.
#include <hip/hip_ext.h>

#include "komp_device.h"
#include "komp_internal.h"

namespace komp {
namespace {

constexpr int QUANT_THREADS = 256;

// q8_0: 8 lanes per block of 32 (4 values each, one 16-byte load), 32 blocks per 256-lane workgroup.
__global__ void __launch_bounds__(QUANT_THREADS)
quant_q8_0_kernel(const float* __restrict__ X, int8_t* __restrict__ XQ, float* __restrict__ XD, int64_t nblocks) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * QUANT_THREADS + threadIdx.x;
  const int64_t blk = gid >> 3;
  const bool valid = blk < nblocks;  // a group of 8 lanes is wholly valid or not
  const f32x4 v = valid ? reinterpret_cast<const f32x4*>(X)[gid] : f32x4{0.f, 0.f, 0.f, 0.f};
  float d;
  int qsum;
  const unsigned packed = q8_0_group8(v, d, qsum);
  if (valid) {
    reinterpret_cast<unsigned*>(XQ)[gid] = packed;
    if ((gid & 7) == 0) XD[blk] = d;
  }
}

// q8_K: 16 lanes per block of 256 (16 consecutive values each, four 16-byte loads), 16 blocks per 256-lane
// workgroup.  Each lane's 16 values are exactly one bsum group.  bsums (XB) are optional.
__global__ void __launch_bounds__(QUANT_THREADS)
quant_q8_K_kernel(const float* __restrict__ X, int8_t* __restrict__ XQ, float* __restrict__ XD,
                  int16_t* __restrict__ XB, int64_t nblocks) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * QUANT_THREADS + threadIdx.x;  // one 16-value group per lane
  const int64_t blk = gid >> 4;
  if (blk >= nblocks) return;  // rows of 16 lanes leave together: a row is one block
  const int r = static_cast<int>(gid & 15);
  f32x4 v[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) v[t] = reinterpret_cast<const f32x4*>(X)[gid * 4 + t];
  u32x4 q;
  float d;
  int qsum;
  const int bsum = q8_K_row16(v, r, q, d, qsum);
  reinterpret_cast<u32x4*>(XQ)[gid] = q;
  if (XB != nullptr) XB[gid] = static_cast<int16_t>(bsum);
  if (r == 0) XD[blk] = d;
}

__global__ void dp4a_probe_kernel(const int32_t* __restrict__ A, const int32_t* __restrict__ B,
                                  const int32_t* __restrict__ C, int32_t* __restrict__ OUT, int64_t n, int mode) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const unsigned a = static_cast<unsigned>(A[i]);
  const unsigned b = static_cast<unsigned>(B[i]);
  OUT[i] = mode == MODE_DP4A ? dot4<MODE_DP4A>(a, b, C[i]) : dot4<MODE_DP4A_EMU>(a, b, C[i]);
}

// [R][16] q4_0 quant bytes -> [R][32] int32 values, through the GEMV's packed-word nibble split.
__global__ void q4_0_decode_kernel(const uint8_t* __restrict__ WQ, int32_t* __restrict__ OUT, int64_t rows) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const u32x4 w = reinterpret_cast<const u32x4*>(WQ)[r];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const unsigned lo = w[d] & 0x0F0F0F0Fu;
    const unsigned hi = (w[d] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      OUT[r * 32 + 4 * d + e] = static_cast<int>((lo >> (8 * e)) & 0xFFu) - 8;
      OUT[r * 32 + 16 + 4 * d + e] = static_cast<int>((hi >> (8 * e)) & 0xFFu) - 8;
    }
  }
}

// [NBLK][64] tq2_0 quant bytes -> [NBLK][256] int32 values, through the GEMV's packed-word crumb split.
__global__ void tq2_0_decode_kernel(const uint8_t* __restrict__ WQ, int32_t* __restrict__ OUT, int64_t nblk) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;  // one 16-byte chunk per lane
  if (gid >= nblk * 4) return;
  const int64_t b = gid >> 2;
  const int q = static_cast<int>(gid & 3);
  const u32x4 w = reinterpret_cast<const u32x4*>(WQ)[gid];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const unsigned c = (w[d] >> (2 * j)) & 0x03030303u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // chunk q: h = q / 2, i = 16 * (q % 2) + 4d + e; value h*128 + j*32 + i
        const int v = (q >> 1) * 128 + j * 32 + 16 * (q & 1) + 4 * d + e;
        OUT[b * 256 + v] = static_cast<int>((c >> (8 * e)) & 0xFFu) - 1;
      }
    }
  }
}

// Streaming-read probe: every 16 bytes of SRC read once with 16-byte buffer loads (4 per thread, 512 threads per
// workgroup, all in flight together; streaming cache policy: sc0 nt), XOR-folded per wave into OUT[wave]: the time of
// moving the bytes alone, the floor a GEMV over as many bytes is measured against.  Each workgroup's 32 KB lie in
// one buffer descriptor whose range ends at SRC's end, so the loads carry no bounds branches (bytes past the end
// read as zeros).  Like a GEMV, it writes a result: a kernel that stores anything ends ~0.4 us later than one that
// does not (the stores' completion before the kernel's end), at every size.
__global__ void __launch_bounds__(512) stream_read_kernel(const u32x4* __restrict__ SRC, int64_t n16,
                                                          uint32_t* __restrict__ OUT) {
  const int64_t first = static_cast<int64_t>(blockIdx.x) * 2048;  // the workgroup's first 16-byte element
  const int64_t left = (n16 - first) * 16;
  const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<u32x4*>(SRC + first), 0,
                                                    static_cast<int>(left < 32768 ? left : 32768), 0x00020000);
  u32x4 v[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) v[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, (u * 512 + threadIdx.x) * 16, 0, 3);
  unsigned acc = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc ^= static_cast<unsigned>(__shfl_xor(static_cast<int>(acc), o, 64));
  if ((threadIdx.x & 63) == 0) OUT[static_cast<int64_t>(blockIdx.x) * 8 + (threadIdx.x >> 6)] = acc;
}

// One lane writes the device's constant-rate real-time counter (the wave stamps' clock) to OUT[0] with a vector store:
// where the stream reaches it, e.g. around a stretch of work inside a HIP graph.
__global__ void __launch_bounds__(64) clock_kernel(uint64_t* __restrict__ OUT) {
  const uint64_t t = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) OUT[0] = t;
}

template <typename F, typename... Args>
hipError_t launch(int kind, F kern, dim3 grid, dim3 block, hipStream_t stream, Args... args) {
  const Timing tm = timing_slot(kind);
  if (tm.on) {
    hipExtLaunchKernelGGL(kern, grid, block, 0, stream, tm.start, tm.stop, 0, args...);
  } else {
    hipLaunchKernelGGL(kern, grid, block, 0, stream, args...);
  }
  return hipGetLastError();
}

unsigned blocks_for(int64_t threads, int per) { return static_cast<unsigned>((threads + per - 1) / per); }

}  // namespace

hipError_t launch_quant_q8_0(const float* x, int8_t* xq, float* xd, int64_t nblocks, hipStream_t stream) {
  return launch(KIND_QUANT_Q8_0, quant_q8_0_kernel, dim3(blocks_for(nblocks * 8, QUANT_THREADS)), dim3(QUANT_THREADS),
                stream, x, xq, xd, nblocks);
}

hipError_t launch_quant_q8_K(const float* x, int8_t* xq, float* xd, int16_t* xb, int64_t nblocks, hipStream_t stream) {
  return launch(KIND_QUANT_Q8_K, quant_q8_K_kernel, dim3(blocks_for(nblocks * 16, QUANT_THREADS)),
                dim3(QUANT_THREADS), stream, x, xq, xd, xb, nblocks);
}

hipError_t launch_dp4a_probe(const int32_t* a, const int32_t* b, const int32_t* c, int32_t* out, int64_t n, int mode,
                             hipStream_t stream) {
  return launch(KIND_PROBE, dp4a_probe_kernel, dim3(blocks_for(n, 256)), dim3(256), stream, a, b, c, out, n, mode);
}

hipError_t launch_stream_read(const void* src, int64_t bytes, uint32_t* out, hipStream_t stream) {
  const int64_t n16 = bytes / 16;
  return launch(KIND_PROBE, stream_read_kernel, dim3(blocks_for(n16, 2048)), dim3(512), stream,
                static_cast<const u32x4*>(src), n16, out);
}

hipError_t launch_clock(uint64_t* out, hipStream_t stream) {
  return launch(KIND_PROBE, clock_kernel, dim3(1), dim3(64), stream, out);
}

hipError_t launch_q4_0_decode(const uint8_t* wq, int32_t* out, int64_t rows, hipStream_t stream) {
  return launch(KIND_PROBE, q4_0_decode_kernel, dim3(blocks_for(rows, 64)), dim3(64), stream, wq, out, rows);
}

hipError_t launch_tq2_0_decode(const uint8_t* wq, int32_t* out, int64_t nblk, hipStream_t stream) {
  return launch(KIND_PROBE, tq2_0_decode_kernel, dim3(blocks_for(nblk * 4, 64)), dim3(64), stream, wq, out, nblk);
}

}  // namespace komp
