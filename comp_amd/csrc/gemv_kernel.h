// Decode GEMVs for Q4_0 x q8_0 and TQ2_0 x q8_K on gfx950 (CDNA4), and for the ggml formats Q8_0 and IQ4_NL (x q8_0)
// and Q4_K (x q8_K) with the same structure (their lanes and dots are described where they are computed).  In dp4a
// mode, 1-3 Q4_0 / IQ4_NL columns run the lean kernel of gemv_q4.h instead (Q4_0 in bytes mode too), and 1-3 TQ2_0
// columns (dp4a and bytes modes) that of gemv_tq2.h, which take the same plans and give the same S (and Y within the
// same bound).
//
// Replaces the reference's Triton kernels src/komp/kernels.py:48-94 (q4_0_gemv) and :97-142 (tq2_0_gemv).
//
// Y[m][n] = sum_b d_w(n, b) * d_x(m, b) * s(m, n, b), where s is the exact int32 dot of weight block b of row n with
// activation block b of column m.  The weights stream once from HBM for all columns (1..3 per launch), with
// non-temporal 16-byte loads (they are read once); the activation columns are staged in LDS once per workgroup, and
// so is the workgroup's slab of weight scales when it is small and aligned (copied global -> LDS directly), so the
// weight stream issues only 16-byte quant loads instead of a 2-byte scale load beside each of them.
// The fused variant stages f32 activations instead: every workgroup quantizes them itself (q8_0 / q8_K, with the
// same device functions as the quantizer kernels, so the bytes are identical) and one workgroup also writes the q8
// planes out; that removes the separate quantizer dispatch from a decode step.
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
// from -8 * sum(x of the block); TQ2_0 dots the crumbs and starts from -sum(x of the block) (kernels.py:72-88,
// 122-136).  TQ2_0 masks three crumb fields in place (weights x1, x4, x16 in three accumulators) and shifts only the
// fourth, which the x16 accumulator also takes; the block dot is (a1 * 16 + a4 * 4 + a16) / 16, exact in int32.
// Mode 0 unpacks every weight and activation to int32 first (kernels.py:65-71, 115-121).
#pragma once

#include <hip/hip_ext.h>

#include <type_traits>

#include "komp_device.h"
#include "komp_internal.h"

namespace komp {
namespace gemv_impl {

constexpr size_t kScaleSlabMax = 16 * 1024;  // largest scale slab staged in LDS
constexpr size_t kLdsLimit = 160 * 1024;      // LDS per workgroup on gfx950

constexpr unsigned NIB = 0x0F0F0F0Fu;
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

// IQ4_NL: exact int32 dot of one block (16 quant bytes, Q4_0's nibble order) with its 32 activations; the nibbles
// index ggml's value table (signed values, no offset).
template <int MODE>
__device__ __forceinline__ int iq4_nl_block_dot(u32x4 w, u32x4 xl, u32x4 xh) {
  int s = 0;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    unsigned lo, hi;
    iq4_nl_lut(w[d], lo, hi);
    if constexpr (MODE == MODE_BYTES) {
#pragma unroll
      for (int e = 0; e < 4; ++e) s += sbyte(lo, e) * sbyte(xl[d], e) + sbyte(hi, e) * sbyte(xh[d], e);
    } else {
      s = dot4<MODE>(lo, xl[d], s);
      s = dot4<MODE>(hi, xh[d], s);
    }
  }
  return s;
}

// Q8_0: partial int32 dot of one 16-byte chunk (16 int8 weights) with the 16 activations of the same half block.
template <int MODE>
__device__ __forceinline__ int q8_0_chunk_dot(u32x4 w, u32x4 x) {
  int s = 0;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    if constexpr (MODE == MODE_BYTES) {
#pragma unroll
      for (int e = 0; e < 4; ++e) s += sbyte(w[d], e) * sbyte(x[d], e);
    } else {
      s = dot4<MODE>(w[d], x[d], s);
    }
  }
  return s;
}

// Q4_K: the two int32 dots of one 32-byte group of a block (16-byte halves wa, wb), whose low nibbles are the 32
// values of one sub-block (activation pieces xa, xb) and whose high nibbles the 32 values of the next (xc, xd); the
// nibbles are unsigned, the sub-blocks' mins enter through their own term.
template <int MODE>
__device__ __forceinline__ int2 q4_k_group_dots(u32x4 wa, u32x4 wb, u32x4 xa, u32x4 xb, u32x4 xc, u32x4 xd) {
  int lo = 0, hi = 0;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    if constexpr (MODE == MODE_BYTES) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lo += static_cast<int>((wa[d] >> (8 * e)) & 15u) * sbyte(xa[d], e) +
              static_cast<int>((wb[d] >> (8 * e)) & 15u) * sbyte(xb[d], e);
        hi += static_cast<int>((wa[d] >> (8 * e + 4)) & 15u) * sbyte(xc[d], e) +
              static_cast<int>((wb[d] >> (8 * e + 4)) & 15u) * sbyte(xd[d], e);
      }
    } else {
      lo = dot4<MODE>(wa[d] & NIB, xa[d], lo);
      lo = dot4<MODE>(wb[d] & NIB, xb[d], lo);
      hi = dot4<MODE>((wa[d] >> 4) & NIB, xc[d], hi);
      hi = dot4<MODE>((wb[d] >> 4) & NIB, xd[d], hi);
    }
  }
  return make_int2(lo, hi);
}

// Q4_K: the 6-bit scales and mins of sub-blocks 2j and 2j+1 from a block's 16 scale-plane bytes (dword 0: f16 d and
// dmin; dwords 1..3: the 12 packed bytes), as {scale 2j, scale 2j+1, min 2j, min 2j+1} in bytes 0..3.  Sub-blocks
// 0..3 keep their scale and min in the low 6 bits of bytes 0..3 and 4..7; sub-blocks 4..7 in the low and high nibble
// of bytes 8..11, with the top two bits of bytes 0..3 (scales) and 4..7 (mins) above them (ggml get_scale_min_k4).
// hi: all ones for j >= 2; sel: the v_perm selector that takes bytes 2(j&1), 2(j&1)+1 of the scales, then of the
// mins.  Both are constants of the lane; the two forms are blended bit-wise (v_bfi_b32), so the wave never branches.
__device__ __forceinline__ unsigned q4_k_scale_pair(u32x4 meta, unsigned hi, unsigned sel) {
  const unsigned u0 = meta[1], u1 = meta[2], u2 = meta[3];
  const unsigned sc_lo = u0 & 0x3F3F3F3Fu, mn_lo = u1 & 0x3F3F3F3Fu;
  const unsigned sc_hi = (u2 & 0x0F0F0F0Fu) | ((u0 >> 2) & 0x30303030u);
  const unsigned mn_hi = ((u2 >> 4) & 0x0F0F0F0Fu) | ((u1 >> 2) & 0x30303030u);
  const unsigned sc = (sc_hi & hi) | (sc_lo & ~hi);
  const unsigned mn = (mn_hi & hi) | (mn_lo & ~hi);
  return __builtin_amdgcn_perm(mn, sc, sel);
}

// TQ2_0: partial int32 dot of one 16-byte chunk.  Byte t of the chunk holds, at bits 2j, the value whose activation
// is byte t of x[j].  `init` joins the x1 accumulator.
template <int MODE>
__device__ __forceinline__ int tq2_0_chunk_dot(u32x4 w, const u32x4 (&x)[4], int init) {
  if constexpr (MODE == MODE_BYTES) {
    int s = init;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const unsigned byte = (w[d] >> (8 * e)) & 0xFFu;
#pragma unroll
        for (int j = 0; j < 4; ++j) s += (static_cast<int>((byte >> (2 * j)) & 3u) - 1) * sbyte(x[j][d], e);
      }
    }
    return s;
  } else {
    int a1 = init, a4 = 0, a16 = 0;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      a1 = dot4<MODE>(w[d] & 0x03030303u, x[0][d], a1);
      a4 = dot4<MODE>(w[d] & 0x0C0C0C0Cu, x[1][d], a4);
      a16 = dot4<MODE>(w[d] & 0x30303030u, x[2][d], a16);
      a16 = dot4<MODE>((w[d] >> 2) & 0x30303030u, x[3][d], a16);
    }
    return ((a1 << 4) + (a4 << 2) + a16) >> 4;
  }
}

// Largest workgroup an instantiation is built for.  One activation column in dp4a mode with nb <= 8 (Q4_K, whose
// 16-byte scale entries take 4 VGPRs per chunk slot: nb <= 4) fits 16 waves (at most 128 VGPRs per wave), which the
// one-workgroup-per-CU plans of small GEMVs use; the others stay at 8.
template <int FMT, int MODE, int MC, int NB, bool FUSED>
constexpr int max_threads() {
  return (MC == 1 && MODE == MODE_DP4A && NB <= (FMT == FMT_Q4_K ? 4 : 8)) ? 1024 : 512;
}

template <int FMT, int MODE, int MC, int NB, bool FUSED>
__global__ void __launch_bounds__((max_threads<FMT, MODE, MC, NB, FUSED>()))
gemv_kernel(int N1, int nblk, int64_t SW1, int rows_per_wg, int rows_per_wave, int lpr_log2, int sc_mode, int nseg,
            int passes, const uint8_t* __restrict__ WQ1, const int16_t* __restrict__ WS1, int K, int nsteps,
            const int8_t* __restrict__ XQ, const float* __restrict__ XD, const float* __restrict__ X,
            int8_t* __restrict__ XQo, float* __restrict__ XDo, int16_t* __restrict__ XBo, float* __restrict__ Y1,
            int32_t* __restrict__ S, const GemvSegs segs) {
  // The host precomputes every quotient (nblk = K / block, rows per wave, K steps), and what the first weight and
  // scale loads need comes first: gfx950 preloads the first 14 argument dwords into SGPRs (16 user SGPRs, 2 of them
  // the argument pointer), so those loads are issued without waiting for an argument fetch from memory and the
  // prologue does no integer division.
  //
  // sc_mode 1: the workgroup's weight scales WS[row0 .. row0 + rows_per_wg) (one contiguous slab, 16-byte aligned, a
  // multiple of 8 scales) are staged in LDS with the activations, and the weight stream issues only quant loads.
  // sc_mode 0: each lane loads its scales beside its quants (one 2-byte load per 16-byte chunk), for slabs that are
  // too large for LDS or not 16-byte aligned.
  //
  // nseg > 1: several matrices sharing the input; the workgroup takes its matrix from segs (scalar compares on the
  // argument block) and from there on works as for one matrix, on its row range within it.
  extern __shared__ __align__(16) unsigned char lds[];
  constexpr bool QK = FMT == FMT_Q4_K;
  constexpr bool BLK32 = FMT != FMT_TQ2_0 && !QK;  // 32-value blocks with q8_0 activations (Q4_0, Q8_0, IQ4_NL)
  constexpr int BB = FMT == FMT_TQ2_0 ? 64 : QK ? 128 : (FMT == FMT_Q8_0 ? 32 : 16);  // quant bytes per block
  // log2(lane slots per block): a slot is 16 bytes of the block, or (Q4_K) a 32-byte group loaded as two halves
  constexpr int CPB_LOG2 = FMT == FMT_TQ2_0 ? 2 : QK ? 2 : (FMT == FMT_Q8_0 ? 1 : 0);
  constexpr int LB = QK ? 32 : 16;  // bytes of a lane slot
  constexpr int SCW = QK ? 8 : 1;  // int16 of the scale plane per block (Q4_K: d, dmin and 12 scale bytes)
  constexpr int SPB = QK ? 2 : 1;  // int32 of S per block (Q4_K: the scaled dot and the mins dot)
  int N = N1;
  int64_t SW = SW1;
  const uint8_t* __restrict__ WQ = WQ1;
  const int16_t* __restrict__ WS = WS1;
  float* __restrict__ Y = Y1;
  int wg = blockIdx.x;  // workgroup index within its matrix
  if (nseg > 1) {
    int sg = 0;
#pragma unroll
    for (int i = 1; i < kMaxSegs; ++i)
      if (i < nseg && wg >= segs.first_wg[i]) sg = i;
    N = segs.n[sg];
    SW = segs.sw[sg];
    WQ = segs.wq[sg];
    WS = segs.ws[sg];
    Y = segs.y[sg];
    wg -= segs.first_wg[sg];
  }
  const int tid = threadIdx.x;
  const int nthreads = blockDim.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lpr = 1 << lpr_log2;
  const int gl = lane & (lpr - 1);
  const int grp = lane >> lpr_log2;
  const int rows_per_pass = 64 >> lpr_log2;
  const int row_base = wg * rows_per_wg + wave * rows_per_wave;  // wave-uniform
  // this wave's rows inside the workgroup's (a plan may give the waves more row slots than the workgroup has rows)
  const int wave_rows = min(rows_per_wave, rows_per_wg - wave * rows_per_wave);  // wave-uniform, may be <= 0
  const int bpg = lpr >> CPB_LOG2;                       // blocks a row group covers per chunk slot
  const int bstep = bpg * NB;                            // blocks a row group covers per K step
  const int q = gl & ((1 << CPB_LOG2) - 1);              // Q8_0, TQ2_0, Q4_K: chunk of the block this lane loads
  const int gblk = gl >> CPB_LOG2;                       // block offset of this lane within a slot
  const int tiles = passes * nsteps;
  // per-lane byte offsets within a row group's tile (row grp of the group, block gblk, chunk q)
  const int64_t lane_w = static_cast<int64_t>(grp) * SW + gblk * BB + q * LB;
  const int64_t lane_s = (static_cast<int64_t>(grp) * nblk + gblk) * SCW;

  using ScT = std::conditional_t<QK, u32x4, int16_t>;  // one block's scale-plane entry
  u32x4 w[NB];
  u32x4 w2[QK ? NB : 1];  // Q4_K: the second 16-byte half of each slot
  ScT sc[NB];
  const bool sc_global = sc_mode == 0;
  auto load_tile = [&](int t) {
    const int p = t / nsteps;
    const int st = t - p * nsteps;
    const int rl = p * rows_per_pass + grp;
    const bool rv = rl < wave_rows && row_base + rl < N;
    const int64_t row0 = static_cast<int64_t>(row_base) + p * rows_per_pass;  // wave-uniform
    const uint8_t* wt = WQ + row0 * SW + static_cast<int64_t>(st) * bstep * BB + lane_w;
    const int16_t* stp = WS + (row0 * nblk + st * bstep) * SCW + lane_s;
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int b = st * bstep + u * bpg + gblk;
      if (rv && b < nblk) {
        w[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wt + static_cast<int64_t>(u) * bpg * BB));
        if constexpr (QK) {
          w2[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wt + static_cast<int64_t>(u) * bpg * BB + 16));
          sc[u] = sc_global ? *reinterpret_cast<const u32x4*>(stp + u * bpg * SCW) : u32x4{0u, 0u, 0u, 0u};
        } else {
          sc[u] = sc_global ? stp[u * bpg] : static_cast<int16_t>(0);
        }
      } else {
        w[u] = u32x4{0u, 0u, 0u, 0u};
        if constexpr (QK) w2[u] = u32x4{0u, 0u, 0u, 0u};
        sc[u] = ScT{};
      }
    }
  };

  // Issue the first tile's weight loads before staging the activations, so HBM latency overlaps the staging.
  load_tile(0);

  // ---- LDS layout ----
  // Q4_0: xlo[m][b] = activations 0..15 of block b, xhi[m][b] = 16..31, meta[m][b] = {d_x bits, -8 * sum(x)}.
  // TQ2_0: x4[m][j][b][q] = the 16 activations that pair with crumb j of chunk q; meta[m][b] = {d_x bits, -sum(x)}.
  // Then (sc_mode 1) the scale slab [waves * rows_per_wave][nblk] (rows past the workgroup's are never loaded nor
  // used), 16-byte aligned (the activation bytes are a multiple of 8).
  // Q4_K: xk[m][p][b] = activation piece p (bytes 16p..16p+15) of block b, meta[m][b] = {d_x bits, 0}, then
  // bs[m][b][i] = the int32 sum of sub-block i's 32 activations (two q8_K bsums).
  u32x4* xv = reinterpret_cast<u32x4*>(lds);
  int2* meta = reinterpret_cast<int2*>(xv + (BLK32 ? 2 : 16) * MC * nblk);
  int* bs = reinterpret_cast<int*>(meta + MC * nblk);  // Q4_K only
  u32x4* scs16 = xv + ((MC * nblk * (BLK32 ? 40 : QK ? 296 : 264) + 15) >> 4);
  const int16_t* scs = reinterpret_cast<const int16_t*>(scs16);

  // Then the scale slab (sc_mode 1): each wave copies 1 KB pieces of it from global memory straight into LDS
  // (global_load_lds_dwordx4: lane i's 16 bytes land at the wave's LDS base + 16 i), so the copy holds no registers;
  // the barrier after the activation staging waits for it with the other loads.
  if (sc_mode == 1) {
    const int wg_row0 = wg * rows_per_wg;
    const int sc_rows = min(rows_per_wg, N - wg_row0);
    const int pieces = (sc_rows * nblk * SCW) >> 3;  // 16-byte pieces
    const u32x4* src = reinterpret_cast<const u32x4*>(WS + static_cast<int64_t>(wg_row0) * nblk * SCW);
    for (int c = wave * 64; c < pieces; c += nthreads) {  // wave-uniform
      if (c + lane < pieces)
        __builtin_amdgcn_global_load_lds(src + c + lane, reinterpret_cast<__attribute__((address_space(3))) void*>(
                                                             reinterpret_cast<uintptr_t>(scs16 + c)),
                                         16, 0, 0);
    }
  }

  // ---- stage the activation columns in LDS ----
  // Each loop below issues the global loads of up to SU iterations before using any of them, so a workgroup pays one
  // memory round trip per SU iterations of staging rather than one per iteration.  The unfused loops finish in one
  // iteration for every shape that fits LDS with 256+ lanes, and extra staging registers would cut the occupancy of
  // the weight stream, so they use SU = 1.
  constexpr int SU = FUSED ? 2 : 1;
  if constexpr (BLK32 && !FUSED) {
    const int total = MC * nblk;
    for (int i0 = tid; i0 < total; i0 += SU * nthreads) {
      u32x4 a[SU], c[SU];
      float dxs[SU];
#pragma unroll
      for (int u = 0; u < SU; ++u) {
        const int i = i0 + u * nthreads;
        if (i < total) {
          const int m = i / nblk;
          const u32x4* src = reinterpret_cast<const u32x4*>(XQ + static_cast<int64_t>(m) * K + (i - m * nblk) * 32);
          a[u] = src[0];
          c[u] = src[1];
          dxs[u] = XD[i];  // XD [M][nblk] is dense: block (m, b) at m * nblk + b = i
        }
      }
#pragma unroll
      for (int u = 0; u < SU; ++u) {
        const int i = i0 + u * nthreads;
        if (i < total) {
          const int m = i / nblk;
          const int b = i - m * nblk;
          xv[i] = a[u];
          xv[MC * nblk + i] = c[u];
          int sum = 0;
          if constexpr (MODE != MODE_BYTES && FMT == FMT_Q4_0) {  // the -8 offset of the Q4_0 nibbles
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              sum = dot4<MODE>(a[u][d], ONES, sum);
              sum = dot4<MODE>(c[u][d], ONES, sum);
            }
          }
          meta[i] = make_int2(__float_as_int(dxs[u]), -8 * sum);
        }
      }
    }
  } else if constexpr (BLK32) {
    // 8 consecutive lanes quantize one block (lane e holds values 4e..4e+3); groups of 8 stay aligned and whole.
    const int total = MC * nblk * 8;
    for (int i0 = tid; i0 < total; i0 += SU * nthreads) {
      f32x4 v[SU];
#pragma unroll
      for (int u = 0; u < SU; ++u) {
        const int i = i0 + u * nthreads;
        if (i < total) {
          const int mb = i >> 3;
          const int m = mb / nblk;
          v[u] = *reinterpret_cast<const f32x4*>(X + static_cast<int64_t>(m) * K + (mb - m * nblk) * 32 + (i & 7) * 4);
        }
      }
#pragma unroll
      for (int u = 0; u < SU; ++u) {
        const int i = i0 + u * nthreads;
        if (i < total) {
          const int e = i & 7;
          const int mb = i >> 3;
          const int m = mb / nblk;
          const int b = mb - m * nblk;
          float d;
          int qsum;
          const unsigned packed = q8_0_group8(v[u], d, qsum);
          reinterpret_cast<unsigned*>(xv + (e < 4 ? mb : MC * nblk + mb))[e & 3] = packed;
          if (e == 0) meta[mb] = make_int2(__float_as_int(d), FMT == FMT_Q4_0 ? -8 * qsum : 0);
          if (blockIdx.x == 0 && XQo != nullptr) {
            reinterpret_cast<unsigned*>(XQo + static_cast<int64_t>(m) * K + b * 32)[e] = packed;
            if (e == 0) XDo[static_cast<int64_t>(m) * nblk + b] = d;
          }
        }
      }
    }
  } else if constexpr (!FUSED) {
    // 16 consecutive lanes stage one block: piece p = 16 contiguous activation bytes at 16p (h = p >> 3,
    // j = (p >> 1) & 3, half = p & 1).  nthreads is a multiple of 64, so the 16-lane groups stay aligned and whole.
    const int total = MC * nblk * 16;
    for (int i0 = tid; i0 < total; i0 += SU * nthreads) {
      u32x4 a[SU];
      float dxs[SU];
#pragma unroll
      for (int u = 0; u < SU; ++u) {
        const int i = i0 + u * nthreads;
        if (i < total) {
          const int mb = i >> 4;
          const int m = mb / nblk;
          a[u] = *reinterpret_cast<const u32x4*>(XQ + static_cast<int64_t>(m) * K + (mb - m * nblk) * 256 + (i & 15) * 16);
          dxs[u] = XD[mb];  // XD [M][nblk] is dense: block (m, b) at m * nblk + b = mb
        }
      }
#pragma unroll
      for (int u = 0; u < SU; ++u) {
        const int i = i0 + u * nthreads;
        if (i < total) {
          const int p = i & 15;
          const int mb = i >> 4;
          const int m = mb / nblk;
          const int b = mb - m * nblk;
          if constexpr (QK) {
            xv[(m * 16 + p) * nblk + b] = a[u];
            int sum = 0;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              if constexpr (MODE == MODE_BYTES) {
#pragma unroll
                for (int e = 0; e < 4; ++e) sum += sbyte(a[u][d], e);
              } else {
                sum = dot4<MODE>(a[u][d], ONES, sum);
              }
            }
            sum = group_sum(sum, 2);  // lanes p, p ^ 1 hold the two halves of sub-block p / 2
            if ((p & 1) == 0) bs[mb * 8 + (p >> 1)] = sum;
            if (p == 0) meta[mb] = make_int2(__float_as_int(dxs[u]), 0);
          } else {
            const int j = (p >> 1) & 3;
            const int qq = ((p >> 3) << 1) | (p & 1);
            xv[((m * 4 + j) * nblk + b) * 4 + qq] = a[u];
            int sum = 0;
            if constexpr (MODE != MODE_BYTES) {
#pragma unroll
              for (int d = 0; d < 4; ++d) sum = dot4<MODE>(a[u][d], ONES, sum);
              sum = group_sum(sum, 16);
            }
            if (p == 0) meta[mb] = make_int2(__float_as_int(dxs[u]), -sum);
          }
        }
      }
    }
  } else {
    // 16 consecutive lanes quantize one block: lane r holds values 16r..16r+15, which are exactly one bsum group and
    // exactly the LDS piece (j = (r % 8) / 2, chunk q = 2 (r / 8) + r % 2); rows of 16 stay aligned and whole.
    const int total = MC * nblk * 16;
    for (int i0 = tid; i0 < total; i0 += SU * nthreads) {
      f32x4 v[SU][4];
#pragma unroll
      for (int u = 0; u < SU; ++u) {
        const int i = i0 + u * nthreads;
        if (i < total) {
          const int mb = i >> 4;
          const int m = mb / nblk;
          const f32x4* src = reinterpret_cast<const f32x4*>(X + static_cast<int64_t>(m) * K + (mb - m * nblk) * 256 +
                                                            (i & 15) * 16);
#pragma unroll
          for (int t = 0; t < 4; ++t) v[u][t] = src[t];
        }
      }
#pragma unroll
      for (int u = 0; u < SU; ++u) {
        const int i = i0 + u * nthreads;
        if (i < total) {
          const int r = i & 15;
          const int mb = i >> 4;
          const int m = mb / nblk;
          const int b = mb - m * nblk;
          u32x4 qv;
          float d;
          int qsum;
          const int bsum = q8_K_row16(v[u], r, qv, d, qsum);
          if constexpr (QK) {
            xv[(m * 16 + r) * nblk + b] = qv;
            const int s32 = group_sum(bsum, 2);  // lanes r, r ^ 1 hold the two halves of sub-block r / 2
            if ((r & 1) == 0) bs[mb * 8 + (r >> 1)] = s32;
            if (r == 0) meta[mb] = make_int2(__float_as_int(d), 0);
          } else {
            const int j = (r & 7) >> 1;
            const int qq = ((r >> 3) << 1) | (r & 1);
            xv[((m * 4 + j) * nblk + b) * 4 + qq] = qv;
            if (r == 0) meta[mb] = make_int2(__float_as_int(d), -qsum);
          }
          if (blockIdx.x == 0 && XQo != nullptr) {
            reinterpret_cast<u32x4*>(XQo + static_cast<int64_t>(m) * K + b * 256)[r] = qv;
            if (r == 0) XDo[static_cast<int64_t>(m) * nblk + b] = d;
            if (XBo != nullptr) XBo[static_cast<int64_t>(mb) * 16 + r] = static_cast<int16_t>(bsum);
          }
        }
      }
    }
  }
  __syncthreads();

  // ---- stream the weights ----
  float acc[MC];
  for (int t = 0; t < tiles; ++t) {
    if (t > 0) load_tile(t);
    const int p = t / nsteps;
    const int st = t - p * nsteps;
    const int rl = p * rows_per_pass + grp;
    const int row = row_base + rl;
    const bool rv = rl < wave_rows && row < N;
    if (st == 0) {
#pragma unroll
      for (int m = 0; m < MC; ++m) acc[m] = 0.0f;
    }
    if (!sc_global) {
      // this tile's scales from the LDS slab (a lane of an idle row reads a slab row that was not loaded; its results
      // are never stored)
      const int16_t* scr = scs + (wave * rows_per_wave + rl) * nblk * SCW;
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const int b = st * bstep + u * bpg + gblk;
        if constexpr (QK)
          sc[u] = b < nblk ? *reinterpret_cast<const u32x4*>(scr + b * SCW) : u32x4{0u, 0u, 0u, 0u};
        else
          sc[u] = b < nblk ? scr[b] : static_cast<int16_t>(0);
      }
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int b = st * bstep + u * bpg + gblk;
      if (b < nblk) {
        float dw, dmin = 0.0f;
        unsigned scm = 0;
        if constexpr (QK) {
          dw = f16_bits_to_f32(static_cast<int16_t>(sc[u][0] & 0xFFFFu));
          dmin = f16_bits_to_f32(static_cast<int16_t>(sc[u][0] >> 16));
          const unsigned jb = 2u * (q & 1);  // byte of sub-block 2q within its dword
          scm = q4_k_scale_pair(sc[u], q >= 2 ? ~0u : 0u, jb | ((jb + 1) << 8) | ((jb + 4) << 16) | ((jb + 5) << 24));
        } else {
          dw = f16_bits_to_f32(sc[u]);
        }
#pragma unroll
        for (int m = 0; m < MC; ++m) {
          const int2 mt = meta[m * nblk + b];
          const float dx = __int_as_float(mt.x);
          if constexpr (FMT == FMT_Q4_0 || FMT == FMT_IQ4_NL) {
            const u32x4 xl = xv[m * nblk + b], xh = xv[(MC + m) * nblk + b];
            const int s = FMT == FMT_Q4_0 ? q4_0_block_dot<MODE>(w[u], xl, xh, mt.y)
                                          : iq4_nl_block_dot<MODE>(w[u], xl, xh);
            if (S != nullptr && rv) S[(static_cast<int64_t>(m) * N + row) * nblk + b] = s;
            acc[m] += static_cast<float>(s) * dw * dx;  // kernels.py:93 order
          } else if constexpr (QK) {
            // lane quad: slot q is the block's 32-byte group q: values 64q + e (sub-block 2q, low nibbles, activation
            // pieces 4q and 4q + 1) and 64q + 32 + e (sub-block 2q + 1, high nibbles, pieces 4q + 2 and 4q + 3)
            const u32x4* xq4 = xv + (m * 16 + 4 * q) * nblk + b;
            const int2 dd = q4_k_group_dots<MODE>(w[u], w2[u], xq4[0], xq4[nblk], xq4[2 * nblk], xq4[3 * nblk]);
            const int2 xs = *reinterpret_cast<const int2*>(bs + (m * nblk + b) * 8 + 2 * q);  // sub-block sums
            // 24-bit multiplies (full rate): |dots| < 2^16, |sums| < 2^13, scales and mins < 64
            const int sd = __mul24(static_cast<int>(scm & 0xFFu), dd.x) + __mul24(static_cast<int>((scm >> 8) & 0xFFu), dd.y);
            const int sm = __mul24(static_cast<int>((scm >> 16) & 0xFFu), xs.x) + __mul24(static_cast<int>(scm >> 24), xs.y);
            const int sdb = group_sum(sd, 4), smb = group_sum(sm, 4);  // the block's exact (sd, sm), every lane
            if (S != nullptr && rv && q == 0) {
              int32_t* sp = S + ((static_cast<int64_t>(m) * N + row) * nblk + b) * SPB;
              sp[0] = sdb;
              sp[1] = smb;
            }
            // y += d * dx * sd - dmin * dx * sm (ggml vec_dot_q4_K_q8_K), once per block (lane 0 of the quad)
            const float t = __builtin_fmaf(static_cast<float>(sdb), dw * dx, acc[m]);
            const float t2 = __builtin_fmaf(-static_cast<float>(smb), dmin * dx, t);
            acc[m] = q == 0 ? t2 : acc[m];
          } else if constexpr (FMT == FMT_Q8_0) {
            // lane pair: chunk q holds the block's values 16q .. 16q+15, dotted with the matching staged half
            const int s = group_sum(q8_0_chunk_dot<MODE>(w[u], xv[(q * MC + m) * nblk + b]), 2);
            if (S != nullptr && rv && q == 0) S[(static_cast<int64_t>(m) * N + row) * nblk + b] = s;
            const float f = static_cast<float>(s) * dw * dx;  // kernels.py:93 order
            acc[m] += q == 0 ? f : 0.0f;
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
    if (st == nsteps - 1) {
#pragma unroll
      for (int m = 0; m < MC; ++m) {
        const float v = group_sum(acc[m], lpr);
        if (gl == 0 && rv) Y[static_cast<int64_t>(m) * N + row] = v;
      }
    }
  }
}

template <int FMT, int MODE, int MC, int NB, bool FUSED>
hipError_t launch_t(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  auto kern = gemv_kernel<FMT, MODE, MC, NB, FUSED>;
  if (64 * p.waves > max_threads<FMT, MODE, MC, NB, FUSED>() || p.waves * p.rows_per_wave < p.block_n)
    return hipErrorInvalidConfiguration;
  GemvSegs segs = c.segs;
  int64_t groups = (c.n + p.block_n - 1) / p.block_n;
  if (c.nseg > 1) {
    groups = 0;
    for (int i = 0; i < c.nseg; ++i) {
      segs.first_wg[i] = static_cast<int>(groups);
      groups += (segs.n[i] + p.block_n - 1) / p.block_n;
    }
  }
  const dim3 grid(static_cast<unsigned>(groups));
  const dim3 block(static_cast<unsigned>(64 * p.waves));
  const int nblk = c.k / fmt_info(FMT).block;
  // the workgroup's scale slab goes to LDS when it is small (the weight stream then issues only quant loads)
  const size_t base = gemv_lds_bytes(FMT, MC, c.k);
  const size_t sc_off = (base + 15) & ~static_cast<size_t>(15);
  const int scw = fmt_info(FMT).sbytes / 2;  // int16 of the scale plane per block
  const size_t sc_bytes = static_cast<size_t>(p.waves) * p.rows_per_wave * nblk * 2 * scw;  // every wave's row slots
  int sc_mode = 0;
  bool ws_aligned = reinterpret_cast<uintptr_t>(c.ws) % 16 == 0;
  for (int i = 0; c.nseg > 1 && i < c.nseg; ++i) ws_aligned = ws_aligned && reinterpret_cast<uintptr_t>(segs.ws[i]) % 16 == 0;
  if (nblk > 0 && (nblk * scw) % 8 == 0 && ws_aligned && sc_bytes <= kScaleSlabMax && sc_off + sc_bytes <= kLdsLimit)
    sc_mode = 1;
  const unsigned lds = static_cast<unsigned>(sc_mode != 0 ? sc_off + sc_bytes : base);
  static std::atomic<unsigned> lds_limit[kMaxDevices];  // this instantiation's allowed dynamic LDS, per device
  const hipError_t le = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds, lds_limit);
  if (le != hipSuccess) return le;
  const Timing tm = timing_slot(gemv_kind(FMT));
  const int cpb = fmt_info(FMT).qbytes / (FMT == FMT_Q4_K ? 32 : 16);  // lane slots per block
  if ((1 << p.lpr_log2) < cpb) return hipErrorInvalidConfiguration;  // a row group holds whole blocks
  const int bstep = ((1 << p.lpr_log2) / cpb) * NB;
  const int nsteps = nblk > 0 ? (nblk + bstep - 1) / bstep : 1;
  const int rows_per_wave = p.rows_per_wave;
  if (tm.on) {
    hipExtLaunchKernelGGL(kern, grid, block, lds, stream, tm.start, tm.stop, 0, c.n, nblk, c.sw, p.block_n,
                          rows_per_wave, p.lpr_log2, sc_mode, c.nseg, p.passes, c.wq, c.ws, c.k, nsteps, c.xq, c.xd,
                          c.x, c.xq_out, c.xd_out, c.xb_out, c.y, c.s, segs);
  } else {
    hipLaunchKernelGGL(kern, grid, block, lds, stream, c.n, nblk, c.sw, p.block_n, rows_per_wave, p.lpr_log2, sc_mode,
                       c.nseg, p.passes, c.wq, c.ws, c.k, nsteps, c.xq, c.xd, c.x, c.xq_out, c.xd_out, c.xb_out, c.y,
                       c.s, segs);
  }
  return hipGetLastError();
}

template <int FMT, int MODE, int MC, bool FUSED>
hipError_t by_nb(const GemvCall& c, const GemvPlan& p, hipStream_t s) {
  switch (p.nb) {
    case 1: return launch_t<FMT, MODE, MC, 1, FUSED>(c, p, s);
    case 2: return launch_t<FMT, MODE, MC, 2, FUSED>(c, p, s);
    case 4: return launch_t<FMT, MODE, MC, 4, FUSED>(c, p, s);
    case 8: return launch_t<FMT, MODE, MC, 8, FUSED>(c, p, s);
    case 16:  // Q4_K slots are 32 bytes: nb 16 would hold 192 VGPRs of weights and scales per lane
      if constexpr (FMT == FMT_Q4_K) return hipErrorInvalidValue;
      else return launch_t<FMT, MODE, MC, 16, FUSED>(c, p, s);
  }
  return hipErrorInvalidValue;
}

template <int FMT, int MODE, bool FUSED>
hipError_t by_mc(const GemvCall& c, const GemvPlan& p, hipStream_t s) {
  switch (c.m) {
    case 1: return by_nb<FMT, MODE, 1, FUSED>(c, p, s);
    case 2: return by_nb<FMT, MODE, 2, FUSED>(c, p, s);
    case 3: return by_nb<FMT, MODE, 3, FUSED>(c, p, s);
  }
  return hipErrorInvalidValue;
}

template <int FMT, bool FUSED>
hipError_t by_mode(const GemvCall& c, const GemvPlan& p, hipStream_t s) {
  switch (c.mode) {
    case MODE_BYTES: return by_mc<FMT, MODE_BYTES, FUSED>(c, p, s);
    case MODE_DP4A_EMU: return by_mc<FMT, MODE_DP4A_EMU, FUSED>(c, p, s);
    case MODE_DP4A: return by_mc<FMT, MODE_DP4A, FUSED>(c, p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace gemv_impl

size_t gemv_lds_bytes(int fmt, int m, int k);

}  // namespace komp
