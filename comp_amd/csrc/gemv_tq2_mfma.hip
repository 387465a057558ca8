// TQ2_0 decode GEMV of three activation columns on the gfx950 matrix cores (dp4a mode, q8_K activations in), with the
// decode GEMVs' result definition (src/komp/kernels.py:97-142):
//   Y[m][n] = sum_b d_x(m, b) * d_w(n, b) * f32(s(m, n, b)),  s = the exact int32 dot of weight block b of row n with
//   activation block b of column m,
// and the same optional S [M][N][K/256].
//
// Why a separate kernel for a few columns.  The lean dp4a kernel (gemv_tq2.h) spends 16 v_dot4 per 64 weights and
// column: 2.6 VALU per weight at three columns, which is what bounds it once the weights are in.  Here the
// activations are the MFMA's A operand (16 rows, of which the first M are the columns) and the weights its B operand
// (16 columns = 16 weight rows), so a v_mfma_i32_16x16x64_i8 takes 64 weights of each of 16 rows for every column at
// once, and the VALU work per weight (unpacking the crumbs, scaling each block) no longer grows with the columns.
//
// Layout.  Operand lane l holds 16 k slots of group g = l / 16 for A row / B column r = l % 16, the same slots in A and
// B.  Lane (r, g) loads bytes 16g..16g+15 of a weight block of row r (one 16-byte load reads 64 bytes of each of 16
// rows); crumb j of byte 16g + e is value (g/2)*128 + 32j + 16(g%2) + e of the block (kernels.py:102), so the B
// operand of crumb j is (w >> 2j) & 0x03030303 and the A operand the 16 activation bytes of column r at that offset,
// one 16-byte load each.  Crumbs go in unsigned (0..3); the -1 offset times the block's activation sum comes from
// four more MFMAs of the same A pieces with a B of all -1 bytes, which start the accumulator, so every C element is the
// exact block dot s.  C element i of lane (r, g) is column 4g + i, row r: lanes 0-15 hold the 4 columns of row r.
//
// Work split.  A workgroup owns 16*T rows (T row tiles, every wave all of them) and all of K; its waves split K into
// contiguous block ranges, at most NBW blocks a wave.  Every load of a wave is issued up front (no loop, no branch
// between loads): the activations (L2 hits) first, then the weights and the scales; a block past the wave's range, a
// row past the matrix and the lanes of columns past M load zeros through the buffer range check without touching
// memory.  Each block's C is scaled as d_x * d_w * f32(s) (kernels.py:141) and added into the lane's f32 sums in
// block order; the waves' partial sums then meet in LDS and are added in wave order (one barrier), so Y does not
// depend on timing.
#include <hip/hip_ext.h>

#include "komp_device.h"
#include "komp_internal.h"

namespace komp {
namespace gemv_tq2_mfma {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr unsigned kOob = 0x7FFFFFF0u;  // a per-lane offset past every descriptor's range: the load returns zeros
constexpr unsigned kCrumb = 0x03030303u;
constexpr int kMaxWaves = 16;

// A raw buffer descriptor over `bytes` (at most 0x7FFFFFF0; the host keeps every range below it).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// R rows a workgroup (the host's plan, at most 16 T) in T row tiles of 16, at most NBW blocks a wave, MC columns (at
// most 4: the C lanes of row group 0).  The lanes of a tile's rows past R (or past N) load zeros and store nothing, so
// R balances the rows over the CUs (2560 rows: 256 workgroups of 10 rows, not 160 of 16).  The first 15 argument
// dwords (preloaded into SGPRs) are the ones the first loads need.  STAMP: the measurement instantiation; each wave reads the real-time
// counter on entry, once its loads have landed, after its blocks are scaled and once the workgroup's outputs are
// stored, and lane 0 writes the four low words to stamps[4 + 4 * (blockIdx.x * waves + wave)] (header {kStampMagic,
// waves of the grid, N, K} from thread 0 of workgroup 0), the lean kernels' record layout.
// FUSED: X f32 [MC][K] in instead of the q8_K planes; each wave quantizes the blocks of its own range (all columns)
// with the quantizer's arithmetic (q8_K_row16: 16 lanes a block and column, four of them a pass) into a region of LDS
// of its own and reads its A pieces back from there, so no wave waits for another before its dots; the blocks' q8
// sums give the -1 offsets (no offset MFMAs).  Workgroup 0 also writes the q8_K planes when XQo is not NULL.
template <int T, int NBW, int MC, bool FUSED, bool STAMP>
__global__ void __launch_bounds__(64 * kMaxWaves)
tq2_mfma_kernel(const void* __restrict__ XA, const uint8_t* __restrict__ WQ, const int16_t* __restrict__ WS, int N,
                int R, int nblk, int SW, int K, const float* __restrict__ XD, float* __restrict__ Y,
                int32_t* __restrict__ S, uint32_t* __restrict__ stamps, int8_t* __restrict__ XQo,
                float* __restrict__ XDo, int16_t* __restrict__ XBo) {
  extern __shared__ __align__(16) unsigned char lds[];
  uint64_t t_entry = 0, t_in = 0, t_dots = 0;
  if constexpr (STAMP) {
    t_entry = __builtin_amdgcn_s_memrealtime();
    __builtin_amdgcn_sched_barrier(0);
  }
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ks = __builtin_amdgcn_readfirstlane(blockDim.x >> 6);  // waves, each a range of blocks
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int row0 = blockIdx.x * R;
  const int row_end = min(N, row0 + R);  // past the workgroup's last row
  const int b0 = wave * nblk / ks;  // this wave's blocks: [b0, b0 + nbw), nbw <= NBW (the host's plan)
  const int nbw = (wave + 1) * nblk / ks - b0;

  // ---- the activations: piece j of column c (c < MC) of slot i is the 16 bytes at block b0 + i, offset
  // (g/2)*128 + 32j + 16(g%2); one load a slot reads all of them, lane (4j + c, g) taking piece (c, j).  The A operand
  // of crumb j wants it in lane (c, g): a DPP row shift left by 4j (lanes of other A rows, columns past MC, and slots
  // past the wave's range read zeros or are never used) ----
  // Fused: pass pp's 16-lane row q (pair P = 4 pp + q = slot i * MC + column c) loads the 16 f32 values 16 r16.. of
  // that block and column
  constexpr int NP = NBW * MC;         // (slot, column) pairs of the wave
  constexpr int NPASS = (NP + 3) / 4;  // quantizer passes, four pairs each
  u32x4 xl[NBW];
  f32x4 xv[FUSED ? NPASS : 1][4];
  float dx[NBW][MC];
  if constexpr (FUSED) {
    const auto fr = rsrc(XA, static_cast<unsigned>(MC * K * 4));
#pragma unroll
    for (int pp = 0; pp < NPASS; ++pp) {
      const int pr = 4 * pp + g;  // this lane's pair
      const int i = pr / MC, c = pr - i * MC;
      const unsigned vf = pr < NP && i < nbw ? static_cast<unsigned>((c * K + (b0 + i) * 256 + 16 * r16) * 4) : kOob;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        xv[pp][q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(fr, vf + 16 * q, 0, 0));
    }
  } else {
    const auto xr = rsrc(XA, static_cast<unsigned>(MC * K));
    const int xc = r16 & 3, xj = r16 >> 2;
    const unsigned vx = xc < MC ? static_cast<unsigned>(xc * K + (g >> 1) * 128 + (g & 1) * 16 + 32 * xj) : kOob;
#pragma unroll
    for (int i = 0; i < NBW; ++i)
      xl[i] = __builtin_amdgcn_raw_buffer_load_b128(xr, i < nbw ? vx : kOob, static_cast<unsigned>((b0 + i) * 256), 0);
    // d_x of each column and slot: wave-uniform, through the scalar cache
#pragma unroll
    for (int i = 0; i < NBW; ++i)
#pragma unroll
      for (int k = 0; k < MC; ++k) {  // a slot past the range reads the row's last d_x and scales by zero (no branch)
        const float v = XD[k * nblk + min(b0 + i, nblk - 1)];
        dx[i][k] = i < nbw ? v : 0.0f;
      }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- the weights and scales of the T tiles: lane (r16, g) reads bytes 16g.. of each block of row r16, and the
  // scale of block b0 + g of row r16 (one load a tile for the wave's at most 4 blocks) ----
  u32x4 w[T][NBW];
  int16_t sc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int rt = row0 + 16 * t;
    const unsigned rows = __builtin_amdgcn_readfirstlane(min(16, max(0, row_end - rt)));  // wave-uniform
    const auto wr = rsrc(WQ + static_cast<int64_t>(rt) * SW, rows * static_cast<unsigned>(SW));
    const unsigned vw = static_cast<unsigned>(r16 * SW + 16 * g);
#pragma unroll
    for (int i = 0; i < NBW; ++i)
      w[t][i] = __builtin_amdgcn_raw_buffer_load_b128(wr, i < nbw ? vw : kOob, static_cast<unsigned>((b0 + i) * 64), 2);
    const auto sr = rsrc(WS + static_cast<int64_t>(rt) * nblk, rows * static_cast<unsigned>(nblk) * 2);
    const unsigned vs = g < nbw ? static_cast<unsigned>((r16 * nblk + g) * 2) : kOob;
    sc[t] = static_cast<int16_t>(__builtin_amdgcn_raw_buffer_load_b16(sr, vs, static_cast<unsigned>(b0 * 2), 0));
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (STAMP) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __builtin_amdgcn_sched_barrier(0);
    t_in = __builtin_amdgcn_s_memrealtime();
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- the block dots and their scaling, block by block ----
  // d_w of slot i for the lanes of row group 0 (the C lanes that are kept): row i's value, broadcast from lane
  // (r16, i) with permlane swaps (permlane16_swap(v, v) leaves row 0's value in row 0 of the first result and row
  // 1's in row 0 of the second; permlane32_swap(v, v) first brings rows 2-3 down)
  float dws[T][NBW];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const unsigned f = __float_as_uint(f16_bits_to_f32(sc[t]));
    if constexpr (NBW <= 2) {
      const auto p = __builtin_amdgcn_permlane16_swap(f, f, false, false);
      dws[t][0] = __uint_as_float(p[0]);
      if constexpr (NBW == 2) dws[t][1] = __uint_as_float(p[1]);
    } else {
      const auto h = __builtin_amdgcn_permlane32_swap(f, f, false, false);
      const auto lo = __builtin_amdgcn_permlane16_swap(h[0], h[0], false, false);
      const auto hi = __builtin_amdgcn_permlane16_swap(h[1], h[1], false, false);
      dws[t][0] = __uint_as_float(lo[0]);
      dws[t][1] = __uint_as_float(lo[1]);
      dws[t][2] = __uint_as_float(hi[0]);
      if constexpr (NBW == 4) dws[t][3] = __uint_as_float(hi[1]);
    }
  }
  float acc[T][MC];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int k = 0; k < MC; ++k) acc[t][k] = 0.0f;
  // Every slot is computed, with no branch (behind one, the compiler would sink the weight loads to their first use):
  // a slot past the wave's range has zero activations, weights, d_w and d_x, and adds zero.  The MFMAs go in
  // independent chains of four (the offset of each slot, and the crumbs of each slot and tile from zero), interleaved
  // across slots and tiles, so consecutive MFMAs rarely wait for each other's results.
  i32x4 xa[NBW][4];
  int msum[FUSED ? NBW : 1][MC];  // fused: -(the block's q8 sum) of each slot and column
  if constexpr (FUSED) {
    // quantize the wave's pairs into its LDS region (256 bytes a pair, in value order), then read the A pieces back
    unsigned char* const xs = lds + wave * (NP * 256);
#pragma unroll
    for (int pp = 0; pp < NPASS; ++pp) {
      const int pr = 4 * pp + g;
      const int i = pr / MC, c = pr - i * MC;
      u32x4 qv;
      float d;
      int qsum;
      const int bsum = q8_K_row16(xv[pp], r16, qv, d, qsum);
      if (pr < NP) *reinterpret_cast<u32x4*>(xs + pr * 256 + 16 * r16) = qv;
      if (__builtin_expect(blockIdx.x == 0 && XQo != nullptr, 0)) {  // workgroup 0 writes the q8_K planes out
        if (pr < NP && i < nbw) {
          const int b = b0 + i;
          *reinterpret_cast<u32x4*>(XQo + c * K + b * 256 + 16 * r16) = qv;
          if (r16 == 0) XDo[c * nblk + b] = d;
          if (XBo != nullptr) XBo[c * (K / 16) + b * 16 + r16] = static_cast<int16_t>(bsum);
        }
      }
      // pair 4 pp + q's d and sum sit in every lane of row q
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int pq = 4 * pp + q;
        if (pq < NP) {
          dx[pq / MC][pq % MC] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(d), 16 * q));
          msum[pq / MC][pq % MC] = -__builtin_amdgcn_readlane(qsum, 16 * q);
        }
      }
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave's LDS writes are done
    asm volatile("" ::: "memory");
    const int xc = r16 < MC ? r16 : MC - 1;  // the lanes of A rows past MC read a real column (their C is unused)
#pragma unroll
    for (int i = 0; i < NBW; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        xa[i][j] = *reinterpret_cast<const i32x4*>(xs + (i * MC + xc) * 256 + (g >> 1) * 128 + 32 * j + (g & 1) * 16);
  } else {
#pragma unroll
    for (int i = 0; i < NBW; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xa[i][0][e] = static_cast<int>(xl[i][e]);
        xa[i][1][e] = __builtin_amdgcn_update_dpp(0, static_cast<int>(xl[i][e]), 0x104, 0xF, 0xF, false);  // row_shl:4
        xa[i][2][e] = __builtin_amdgcn_update_dpp(0, static_cast<int>(xl[i][e]), 0x108, 0xF, 0xF, false);  // row_shl:8
        xa[i][3][e] = __builtin_amdgcn_update_dpp(0, static_cast<int>(xl[i][e]), 0x10C, 0xF, 0xF, false);  // row_shl:12
      }
  }
  i32x4 corr[NBW], cc[T][NBW];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int i = 0; i < NBW; ++i)
      if constexpr (!FUSED)
        corr[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[i][j], i32x4{-1, -1, -1, -1},
                                                        j ? corr[i] : i32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int i = 0; i < NBW; ++i) {
        const u32x4 cr = (w[t][i] >> (2u * j)) & kCrumb;
        cc[t][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[i][j], reinterpret_cast<const i32x4&>(cr),
                                                         j ? cc[t][i] : i32x4{0, 0, 0, 0}, 0, 0, 0);
      }
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int row = row0 + 16 * t + r16;
#pragma unroll
    for (int i = 0; i < NBW; ++i) {
      i32x4 sb;  // the exact block dots (|s| < 2^17)
      if constexpr (FUSED) {
#pragma unroll
        for (int k = 0; k < 4; ++k) sb[k] = cc[t][i][k] + (k < MC ? msum[i][k] : 0);
      } else {
        sb = cc[t][i] + corr[i];
      }
      if (__builtin_expect(S != nullptr, 0)) {
        if (g == 0 && row < row_end && i < nbw) {
#pragma unroll
          for (int k = 0; k < MC; ++k) S[(static_cast<int64_t>(k) * N + row) * nblk + b0 + i] = sb[k];
        }
      }
#pragma unroll
      for (int k = 0; k < MC; ++k)
        acc[t][k] = __builtin_fmaf(dx[i][k] * dws[t][i], static_cast<float>(sb[k]), acc[t][k]);
    }
  }

  if constexpr (STAMP) {
    __builtin_amdgcn_sched_barrier(0);
    t_dots = __builtin_amdgcn_s_memrealtime();
    __builtin_amdgcn_sched_barrier(0);
  }
  // the stamp record, once the wave's stores have completed
  const auto stamp_out = [&]() {
    if constexpr (STAMP) {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      __builtin_amdgcn_sched_barrier(0);
      const uint64_t t_stored = __builtin_amdgcn_s_memrealtime();
      u32x4* rec = reinterpret_cast<u32x4*>(stamps);
      if (lane == 0)
        rec[1 + blockIdx.x * ks + wave] = u32x4{static_cast<unsigned>(t_entry), static_cast<unsigned>(t_in),
                                                static_cast<unsigned>(t_dots), static_cast<unsigned>(t_stored)};
      if (blockIdx.x == 0 && threadIdx.x == 0)
        rec[0] = u32x4{kStampMagic, gridDim.x * ks, static_cast<unsigned>(N), static_cast<unsigned>(nblk) * 256u};
    }
  };

  // ---- the waves' partial sums, added in wave order ----
  if (ks == 1) {
    if (g == 0) {
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int row = row0 + 16 * t + r16;
        if (row < row_end) {
#pragma unroll
          for (int k = 0; k < MC; ++k) Y[static_cast<int64_t>(k) * N + row] = acc[t][k];
        }
      }
    }
    stamp_out();
    return;
  }
  float* red = reinterpret_cast<float*>(lds + (FUSED ? ks * NP * 256 : 0));  // [wave][t][k][16], past the staging
  if (g == 0) {
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int k = 0; k < MC; ++k) red[((wave * T + t) * MC + k) * 16 + r16] = acc[t][k];
  }
  __syncthreads();
  for (int o = threadIdx.x; o < T * MC * 16; o += blockDim.x) {
    const int r = o & 15;
    const int k = (o >> 4) % MC;
    const int t = (o >> 4) / MC;
    float sum = red[(t * MC + k) * 16 + r];
    for (int p = 1; p < ks; ++p) sum += red[((p * T + t) * MC + k) * 16 + r];
    const int row = row0 + 16 * t + r;
    if (row < row_end) Y[static_cast<int64_t>(k) * N + row] = sum;
  }
  stamp_out();
}

template <int T, int NBW, int MC, bool FUSED>
hipError_t launch_k(const GemvCall& c, const MfmaPlan& p, hipStream_t stream) {
  const int nblk = c.k / 256;
  const unsigned groups = static_cast<unsigned>((c.n + p.rows - 1) / p.rows);
  // the tuning harness's wave stamps, while there is room for them
  uint32_t* const slot = stamps_on() ? stamp_slot(4 + 4 * int64_t{groups} * p.waves) : nullptr;
  const auto kern =
      slot != nullptr ? tq2_mfma_kernel<T, NBW, MC, FUSED, true> : tq2_mfma_kernel<T, NBW, MC, FUSED, false>;
  const size_t lds = tq2_mfma_lds_bytes(T, NBW, MC, FUSED, p.waves);
  const dim3 grid(groups), block(static_cast<unsigned>(64 * p.waves));
  const int sw = static_cast<int>(c.sw);
  const void* xa = FUSED ? static_cast<const void*>(c.x) : static_cast<const void*>(c.xq);
  const Timing tm = timing_slot(KIND_TQ2_0_GEMV);
  if (tm.on)
    hipExtLaunchKernelGGL(kern, grid, block, lds, stream, tm.start, tm.stop, 0, xa, c.wq, c.ws, c.n, p.rows, nblk, sw, c.k,
                          c.xd, c.y, c.s, slot, c.xq_out, c.xd_out, c.xb_out);
  else
    hipLaunchKernelGGL(kern, grid, block, lds, stream, xa, c.wq, c.ws, c.n, p.rows, nblk, sw, c.k, c.xd, c.y, c.s, slot,
                       c.xq_out, c.xd_out, c.xb_out);
  return hipGetLastError();
}

template <int T, int NBW>
hipError_t by_mc(const GemvCall& c, const MfmaPlan& p, hipStream_t s) {
  if (c.m != 3) return hipErrorInvalidValue;  // the column count the library routes here
  return c.x != nullptr ? launch_k<T, NBW, 3, true>(c, p, s) : launch_k<T, NBW, 3, false>(c, p, s);
}

template <int T>
hipError_t by_nbw(const GemvCall& c, const MfmaPlan& p, hipStream_t s) {
  switch (p.nbw) {
    case 1: return by_mc<T, 1>(c, p, s);
    case 2: return by_mc<T, 2>(c, p, s);
    case 3: return by_mc<T, 3>(c, p, s);
    case 4: return by_mc<T, 4>(c, p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace gemv_tq2_mfma

size_t tq2_mfma_lds_bytes(int tiles, int nbw, int mc, bool fused, int waves) {
  const size_t stage = fused ? static_cast<size_t>(waves) * nbw * mc * 256 : 0;  // each wave's quantized blocks
  return stage + (waves > 1 ? static_cast<size_t>(waves) * tiles * mc * 16 * sizeof(float) : 0);
}

bool tq2_mfma_eligible(const GemvCall& c, const MfmaPlan& p) {
  if (c.fmt != FMT_TQ2_0 || c.mode != MODE_DP4A || c.nseg > 1 || c.m != 3) return false;
  if (c.x == nullptr && (c.xq == nullptr || c.xd == nullptr)) return false;
  if (c.k % 256 != 0 || c.k <= 0 || c.n <= 0) return false;
  if (p.tiles < 1 || p.tiles > 2 || p.rows < 1 || p.rows > 16 * p.tiles || p.waves < 1 || p.waves > gemv_tq2_mfma::kMaxWaves || p.nbw < 1 || p.nbw > 4)
    return false;
  const int64_t nblk = c.k / 256;
  if ((nblk + p.waves - 1) / p.waves > p.nbw) return false;                   // each wave's range fits its slots
  if (16 * c.sw > 0x7FFFFFF0 || int64_t{4} * c.k > 0x7FFFFFF0) return false;  // the descriptors' ranges
  return c.sw >= 64 * nblk && c.sw % 16 == 0;
}

hipError_t launch_gemv_tq2_mfma(const GemvCall& c, const MfmaPlan& p, hipStream_t stream) {
  if (!tq2_mfma_eligible(c, p)) return hipErrorInvalidConfiguration;
  return p.tiles == 2 ? gemv_tq2_mfma::by_nbw<2>(c, p, stream) : gemv_tq2_mfma::by_nbw<1>(c, p, stream);
}

}  // namespace komp
