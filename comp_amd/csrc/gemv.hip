// Decode GEMVs for Q4_0 x q8_0 and TQ2_0 x q8_K on gfx950 (CDNA4).
//
// Replaces the reference's Triton kernels src/komp/kernels.py:48-94 (q4_0_gemv) and :97-142 (tq2_0_gemv).
//
// Y[m][n] = sum_b d_w(n, b) * d_x(m, b) * s(m, n, b), where s is the exact int32 dot of weight block b of row n with
// activation block b of column m.  The weights stream once from HBM for all columns (1..3 per launch); the activation
// columns are staged in LDS once per workgroup.
//
// Work decomposition (the reference's tune knobs keep their role; the mapping is this kernel's own):
//   waves per workgroup   = num_warps
//   rows per workgroup    = block_n; each wave owns block_n / num_warps rows ("rows per wave")
//   lanes per row group   = 64 / min(rows per wave, 16); a wave walks its rows in passes of 64 / lanes-per-group rows
//   nb                    = 16-byte weight chunks each lane loads per row per K step
// A 16-byte chunk is one Q4_0 block (32 weights) or a quarter of a TQ2_0 block (64 weights).  Q4_0: lane g of a row
// group takes blocks step*G*nb + u*G + g (u < nb, G = lanes per group), so every load instruction of the group reads
// G*16 contiguous bytes of its row.  TQ2_0: aligned lane quads own a block; lane q of a quad takes bytes 16q..16q+15,
// and the quad's partial dots are added with two DPP steps before the block's scale is applied.
//
// Integer dots (modes 1 and 2): Q4_0 dots the unsigned nibbles (w & 0x0F0F0F0F, (w >> 4) & 0x0F0F0F0F) and starts
// from -8 * sum(x of the block); TQ2_0 dots the crumbs ((w >> 2j) & 0x03030303) and starts from -sum(x of the block)
// (kernels.py:72-88, 122-136).  Both corrections are precomputed per block while the activations are staged.
// Mode 0 unpacks every weight and activation to int32 first (kernels.py:65-71, 115-121).
#include <hip/hip_ext.h>

#include "komp_device.h"
#include "komp_internal.h"

namespace komp {
namespace {

constexpr unsigned NIB = 0x0F0F0F0Fu;
constexpr unsigned CRUMB = 0x03030303u;
constexpr unsigned ONES = 0x01010101u;

// Q4_0: exact int32 dot of one block (16 quant bytes) with its 32 activations; xl = values 0..15, xh = 16..31.
template <int MODE>
__device__ __forceinline__ int q4_0_block_dot(u32x4 w, u32x4 xl, u32x4 xh, int corr) {
  if constexpr (MODE == MODE_BYTES) {
    int s = 0;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int lo = static_cast<int>((w[d] >> (8 * e)) & 15u) - 8;
        const int hi = static_cast<int>((w[d] >> (8 * e + 4)) & 15u) - 8;
        s += lo * sbyte(xl[d], e) + hi * sbyte(xh[d], e);
      }
    }
    return s;
  } else {
    int s = corr;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      s = dot4<MODE>(w[d] & NIB, xl[d], s);
      s = dot4<MODE>((w[d] >> 4) & NIB, xh[d], s);
    }
    return s;
  }
}

// TQ2_0: partial int32 dot of one 16-byte chunk.  Byte t of the chunk holds, at bits 2j, the value whose activation
// is byte t of x[j].
template <int MODE>
__device__ __forceinline__ int tq2_0_chunk_dot(u32x4 w, const u32x4 (&x)[4], int init) {
  int s = init;
  if constexpr (MODE == MODE_BYTES) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const unsigned byte = (w[d] >> (8 * e)) & 0xFFu;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          s += (static_cast<int>((byte >> (2 * j)) & 3u) - 1) * sbyte(x[j][d], e);
        }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int d = 0; d < 4; ++d) s = dot4<MODE>((w[d] >> (2 * j)) & CRUMB, x[j][d], s);
    }
  }
  return s;
}

template <int FMT, int MODE, int MC, int NB>
__global__ void __launch_bounds__(512)
gemv_kernel(const uint8_t* __restrict__ WQ, const int16_t* __restrict__ WS, const int8_t* __restrict__ XQ,
            const float* __restrict__ XD, float* __restrict__ Y, int32_t* __restrict__ S, int N, int K, int64_t SW,
            int rows_per_wg, int lpr_log2, int passes) {
  extern __shared__ __align__(16) unsigned char lds[];
  constexpr int BLK = FMT == FMT_Q4_0 ? 32 : 256;
  const int nblk = K / BLK;
  const int tid = threadIdx.x;
  const int nthreads = blockDim.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lpr = 1 << lpr_log2;
  const int gl = lane & (lpr - 1);
  const int grp = lane >> lpr_log2;
  const int rows_per_pass = 64 >> lpr_log2;
  const int rows_per_wave = rows_per_wg / (nthreads >> 6);
  const int row_base = blockIdx.x * rows_per_wg + wave * rows_per_wave;
  const int bpg = FMT == FMT_Q4_0 ? lpr : (lpr >> 2);  // blocks a row group covers per chunk slot
  const int bstep = bpg * NB;                            // blocks a row group covers per K step
  const int nsteps = (nblk + bstep - 1) / bstep;
  const int q = gl & 3;                                  // TQ2_0: chunk of the block this lane loads
  const int gblk = FMT == FMT_Q4_0 ? gl : (gl >> 2);     // block offset of this lane within a slot
  const int tiles = passes * (nsteps > 0 ? nsteps : 1);

  u32x4 w[NB];
  int16_t sc[NB];
  auto tile_row = [&](int t, int& row) {
    const int p = nsteps > 0 ? t / nsteps : t;
    const int rl = p * rows_per_pass + grp;
    row = row_base + rl;
    return rl < rows_per_wave && row < N;
  };
  auto load_tile = [&](int t) {
    int row;
    const bool rv = tile_row(t, row);
    const int st = nsteps > 0 ? t % nsteps : 0;
    const uint8_t* wrow = WQ + static_cast<int64_t>(row) * SW;
    const int16_t* srow = WS + static_cast<int64_t>(row) * nblk;
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int b = st * bstep + u * bpg + gblk;
      if (rv && b < nblk) {
        w[u] = *reinterpret_cast<const u32x4*>(wrow + (FMT == FMT_Q4_0 ? b * 16 : b * 64 + q * 16));
        sc[u] = srow[b];
      } else {
        w[u] = u32x4{0u, 0u, 0u, 0u};
        sc[u] = 0;
      }
    }
  };

  // Issue the first tile's weight loads before staging the activations, so HBM latency overlaps the staging.
  load_tile(0);

  // ---- stage the activation columns in LDS ----
  // Q4_0: xlo[m][b] = activations 0..15 of block b, xhi[m][b] = 16..31, meta[m][b] = {d_x bits, -8 * sum(x)}.
  // TQ2_0: x4[m][j][b][q] = the 16 activations that pair with crumb j of chunk q; meta[m][b] = {d_x bits, -sum(x)}.
  u32x4* xv = reinterpret_cast<u32x4*>(lds);
  int2* meta;
  if constexpr (FMT == FMT_Q4_0) {
    meta = reinterpret_cast<int2*>(xv + 2 * MC * nblk);
    for (int i = tid; i < MC * nblk; i += nthreads) {
      const int m = i / nblk;
      const int b = i - m * nblk;
      const u32x4* src = reinterpret_cast<const u32x4*>(XQ + static_cast<int64_t>(m) * K + b * 32);
      const u32x4 a = src[0];
      const u32x4 c = src[1];
      xv[i] = a;
      xv[MC * nblk + i] = c;
      int sum = 0;
      if constexpr (MODE != MODE_BYTES) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          sum = dot4<MODE>(a[d], ONES, sum);
          sum = dot4<MODE>(c[d], ONES, sum);
        }
      }
      meta[i] = make_int2(__float_as_int(XD[static_cast<int64_t>(m) * nblk + b]), -8 * sum);
    }
  } else {
    meta = reinterpret_cast<int2*>(xv + 16 * MC * nblk);
    // 16 consecutive lanes stage one block: piece p = 16 contiguous activation bytes at 16p (h = p >> 3,
    // j = (p >> 1) & 3, half = p & 1).  nthreads is a multiple of 64, so the 16-lane groups stay aligned and whole.
    for (int i = tid; i < MC * nblk * 16; i += nthreads) {
      const int p = i & 15;
      const int mb = i >> 4;
      const int m = mb / nblk;
      const int b = mb - m * nblk;
      const u32x4 a = *reinterpret_cast<const u32x4*>(XQ + static_cast<int64_t>(m) * K + b * 256 + p * 16);
      const int j = (p >> 1) & 3;
      const int qq = ((p >> 3) << 1) | (p & 1);
      xv[((m * 4 + j) * nblk + b) * 4 + qq] = a;
      int sum = 0;
      if constexpr (MODE != MODE_BYTES) {
#pragma unroll
        for (int d = 0; d < 4; ++d) sum = dot4<MODE>(a[d], ONES, sum);
        sum = group_sum(sum, 16);
      }
      if (p == 0) meta[mb] = make_int2(__float_as_int(XD[static_cast<int64_t>(m) * nblk + b]), -sum);
    }
  }
  __syncthreads();

  // ---- stream the weights ----
  float acc[MC];
  for (int t = 0; t < tiles; ++t) {
    if (t > 0) load_tile(t);
    int row;
    const bool rv = tile_row(t, row);
    const int st = nsteps > 0 ? t % nsteps : 0;
    if (st == 0) {
#pragma unroll
      for (int m = 0; m < MC; ++m) acc[m] = 0.0f;
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int b = st * bstep + u * bpg + gblk;
      if (b < nblk) {
        const float dw = f16_bits_to_f32(sc[u]);
#pragma unroll
        for (int m = 0; m < MC; ++m) {
          const int2 mt = meta[m * nblk + b];
          const float dx = __int_as_float(mt.x);
          if constexpr (FMT == FMT_Q4_0) {
            const int s = q4_0_block_dot<MODE>(w[u], xv[m * nblk + b], xv[(MC + m) * nblk + b], mt.y);
            if (S != nullptr && rv) S[(static_cast<int64_t>(m) * N + row) * nblk + b] = s;
            acc[m] += static_cast<float>(s) * dw * dx;  // kernels.py:93 order
          } else {
            u32x4 xs[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) xs[j] = xv[((m * 4 + j) * nblk + b) * 4 + q];
            const int init = (MODE != MODE_BYTES && q == 0) ? mt.y : 0;
            const int s = group_sum(tq2_0_chunk_dot<MODE>(w[u], xs, init), 4);
            if (S != nullptr && rv && q == 0) S[(static_cast<int64_t>(m) * N + row) * nblk + b] = s;
            const float f = dx * dw * static_cast<float>(s);  // kernels.py:141 order
            acc[m] += q == 0 ? f : 0.0f;
          }
        }
      }
    }
    if (st == nsteps - 1 || nsteps == 0) {
#pragma unroll
      for (int m = 0; m < MC; ++m) {
        const float v = group_sum(acc[m], lpr);
        if (gl == 0 && rv) Y[static_cast<int64_t>(m) * N + row] = v;
      }
    }
  }
}

template <int FMT, int MODE, int MC, int NB>
hipError_t launch_t(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  auto kern = gemv_kernel<FMT, MODE, MC, NB>;
  const dim3 grid(static_cast<unsigned>((c.n + p.block_n - 1) / p.block_n));
  const dim3 block(static_cast<unsigned>(64 * p.waves));
  const unsigned lds = static_cast<unsigned>(gemv_lds_bytes(FMT, MC, c.k));
  static unsigned lds_attr = 64 * 1024;  // dynamic LDS above 64 KiB must be requested per kernel
  if (lds > lds_attr) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) return e;
    lds_attr = lds;
  }
  const Timing tm = timing_slot(FMT == FMT_Q4_0 ? KIND_Q4_0_GEMV : KIND_TQ2_0_GEMV);
  if (tm.on) {
    hipExtLaunchKernelGGL(kern, grid, block, lds, stream, tm.start, tm.stop, 0, c.wq, c.ws, c.xq, c.xd, c.y, c.s, c.n,
                          c.k, c.sw, p.block_n, p.lpr_log2, p.passes);
  } else {
    hipLaunchKernelGGL(kern, grid, block, lds, stream, c.wq, c.ws, c.xq, c.xd, c.y, c.s, c.n, c.k, c.sw, p.block_n,
                       p.lpr_log2, p.passes);
  }
  return hipGetLastError();
}

template <int FMT, int MODE, int MC>
hipError_t by_nb(const GemvCall& c, const GemvPlan& p, hipStream_t s) {
  switch (p.nb) {
    case 1: return launch_t<FMT, MODE, MC, 1>(c, p, s);
    case 2: return launch_t<FMT, MODE, MC, 2>(c, p, s);
    case 4: return launch_t<FMT, MODE, MC, 4>(c, p, s);
    case 8: return launch_t<FMT, MODE, MC, 8>(c, p, s);
    case 16: return launch_t<FMT, MODE, MC, 16>(c, p, s);
  }
  return hipErrorInvalidValue;
}

template <int FMT, int MODE>
hipError_t by_mc(const GemvCall& c, const GemvPlan& p, hipStream_t s) {
  switch (c.m) {
    case 1: return by_nb<FMT, MODE, 1>(c, p, s);
    case 2: return by_nb<FMT, MODE, 2>(c, p, s);
    case 3: return by_nb<FMT, MODE, 3>(c, p, s);
  }
  return hipErrorInvalidValue;
}

template <int FMT>
hipError_t by_mode(const GemvCall& c, const GemvPlan& p, hipStream_t s) {
  switch (c.mode) {
    case MODE_BYTES: return by_mc<FMT, MODE_BYTES>(c, p, s);
    case MODE_DP4A_EMU: return by_mc<FMT, MODE_DP4A_EMU>(c, p, s);
    case MODE_DP4A: return by_mc<FMT, MODE_DP4A>(c, p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

size_t gemv_lds_bytes(int fmt, int m, int k) {
  if (fmt == FMT_Q4_0) return static_cast<size_t>(m) * (k / 32) * (32 + 8);
  return static_cast<size_t>(m) * (k / 256) * (256 + 8);
}

hipError_t launch_gemv(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  return c.fmt == FMT_Q4_0 ? by_mode<FMT_Q4_0>(c, p, stream) : by_mode<FMT_TQ2_0>(c, p, stream);
}

}  // namespace komp
