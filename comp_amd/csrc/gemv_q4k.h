// Q4_K decode GEMVs of 1-3 activation columns in dp4a mode (ggml block_q4_K: 256 values as 128 nibble bytes, with
// f16 d, f16 dmin and 12 bytes of packed 6-bit sub-block scales and mins in the scale plane; q8_K activations),
// unfused and fused with the q8_K quantizer.  The arithmetic is the general kernel's (gemv_kernel.h): a lane quad per
// block, lane q taking the block's 32-byte group q (sub-blocks 2q and 2q + 1), the block's exact (sd, sm) summed over
// the quad and added once per block by the quad's lane 0 as y += d * dx * sd - dmin * dx * sm (ggml
// vec_dot_q4_K_q8_K), so S and Y equal the general kernel's for the same plan.  The structure is the lean kernels'
// (gemv_q4.h, gemv_tq2.h):
//   * weight and scale loads are buffer loads from loop-invariant per-lane offsets, the step and slot offsets being
//     a scalar; a block past the row's end, and every row past the matrix, reads zeros without touching memory, so no
//     load sits behind a branch and each block's dot waits for its own loads only;
//   * the staging's activation loads are issued before the weight loads, and the barrier that publishes the staged
//     columns waits for LDS writes only, so the weights stay in flight through the staging;
//   * a plan of one pass and one K step (the decode shapes) is straight-line code with no loop and no reload.
#pragma once

#include "gemv_kernel.h"

namespace komp {
namespace gemv_q4k {

constexpr unsigned kOob = 0x7FFFFFF0u;   // a buffer offset past every descriptor's range: the load returns zeros
// LDS bytes per staged 256-value block: 80 dwords, so that with the pieces rotated (below) the 16-byte reads of
// consecutive lanes (lane q of a quad reads 64 bytes at 64q of its block, neighbouring quads the next blocks) fall on
// distinct banks, for 32 or 64 banks
constexpr int kBlockStride = 320;
constexpr size_t kLdsLimit = 160 * 1024;

// A raw buffer descriptor over `bytes` (at most 0x7FFFFFF0: one pass's rows, which the plans keep below 2^31 bytes).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// LPR lanes per row group (4 per block), NB 32-byte groups per lane per K step, MC activation columns.  ONE: the plan
// has one pass and one K step.
template <int LPR, int NB, int MC, bool FUSED, bool ONE>
__device__ __forceinline__ void q4k_lean_body(int N1, int nblk, int SW1, int nseg, int rows_per_wg, int passes,
                                              const uint8_t* __restrict__ WQ1, const int16_t* __restrict__ WS1,
                                              const void* __restrict__ XA, const float* __restrict__ XD,
                                              float* __restrict__ Y1, int32_t* __restrict__ S,
                                              int8_t* __restrict__ XQo, float* __restrict__ XDo,
                                              int16_t* __restrict__ XBo, const GemvSegs& segs) {
  constexpr int RPW = 64 / LPR;          // rows per wave and pass
  constexpr int BPG = LPR / 4;           // blocks a row group covers per slot
  constexpr int BSTEP = BPG * NB;        // blocks per K step
  constexpr int XB = kBlockStride;
  extern __shared__ __align__(16) unsigned char lds[];
  const int tid = threadIdx.x;
  // ---- the staging's first loads (16 threads per block: thread r holds values 16r .. 16r + 15, one bsum group),
  // issued first: they need only preloaded arguments, so they go out before anything else and do not queue behind
  // the weights.  Fused: the f32 values; unfused: the q8 bytes, and d_x for the block's first thread.  The columns'
  // blocks in order (X [MC][K], XQ [MC][K] and XD [MC][nblk] are dense) ----
  const int nstage = MC * nblk * 16;
  const int nthreads = blockDim.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool stg = tid < nstage;
  f32x4 xf[4];
  u32x4 x16;
  float xdv = 0.0f;
  if (stg) {
    if constexpr (FUSED) {
      const f32x4* src = reinterpret_cast<const f32x4*>(static_cast<const float*>(XA) + tid * 16);
#pragma unroll
      for (int t = 0; t < 4; ++t) xf[t] = src[t];
    } else {
      x16 = *reinterpret_cast<const u32x4*>(static_cast<const int8_t*>(XA) + tid * 16);
      if ((tid & 15) == 0) xdv = XD[tid >> 4];
    }
  }
  int N = N1;
  unsigned SW = static_cast<unsigned>(SW1);  // a row's bytes: one pass's rows span at most 0x7FFFFFF0 of them
  const uint8_t* WQ = WQ1;
  const int16_t* WS = WS1;
  float* Y = Y1;
  int wg = blockIdx.x;
  if (__builtin_expect(nseg > 1, 0)) {  // several matrices sharing the column: this workgroup's one
    int sg = 0;
#pragma unroll
    for (int i = 1; i < kMaxSegs; ++i)
      if (i < nseg && wg >= segs.first_wg[i]) sg = i;
    N = segs.n[sg];
    SW = static_cast<unsigned>(segs.sw[sg]);
    WQ = segs.wq[sg];
    WS = segs.ws[sg];
    Y = segs.y[sg];
    wg -= segs.first_wg[sg];
  }
  const int q = lane & 3;
  const int gblk = (lane & (LPR - 1)) >> 2;
  const int grp = lane / LPR;
  const int nsteps = ONE ? 1 : (nblk + BSTEP - 1) / BSTEP;
  const int npass = ONE ? 1 : passes;
  const int nblk_pad = nsteps * BSTEP;
  const int rows_per_wave = RPW * npass;
  const int row_base = wg * rows_per_wg + wave * rows_per_wave;  // wave-uniform
  const int wave_rows = min(rows_per_wave, rows_per_wg - wave * rows_per_wave);
  const int vrows = max(0, min(wave_rows, N - row_base));  // rows of this wave inside the matrix
  const unsigned vo_w = grp * SW + gblk * 128 + q * 32;
  const unsigned vo_s = static_cast<unsigned>((grp * nblk + gblk) * 16);

  // ---- weights: tile (p, st) = rows p * RPW + grp of the wave, blocks st * BSTEP + u * BPG + gblk; per slot the
  // lane's 32-byte group (two 16-byte loads) and the block's 16-byte scale entry, which every lane of the quad needs
  // (its own sub-blocks' scales and mins; lane 0 also d and dmin) ----
  u32x4 w[NB], w2[NB], sc[NB];
  auto load = [&](int p, int st) {
    const int prow = p * RPW;  // wave-uniform
    const unsigned rows = __builtin_amdgcn_readfirstlane(min(RPW, max(0, vrows - prow)));  // wave-uniform
    const auto wrs = rsrc(WQ + static_cast<int64_t>(row_base + prow) * SW, rows * SW);
    const auto srs = rsrc(WS + static_cast<int64_t>(row_base + prow) * nblk * 8, rows * static_cast<unsigned>(nblk) * 16);
    const unsigned so_w = static_cast<unsigned>(st * BSTEP * 128);
    const unsigned so_s = static_cast<unsigned>(st * BSTEP * 16);
    const int lim = nblk - st * BSTEP;  // blocks from the tile's first to the row's end (wave-uniform)
#pragma unroll
    for (int u = 0; u < NB; ++u) {  // the scales first: a block's dot then waits for its own weight loads only
      const bool ok = gblk + u * BPG < lim;
      sc[u] = __builtin_amdgcn_raw_buffer_load_b128(srs, ok ? vo_s : kOob, so_s + u * BPG * 16, 0);
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const bool ok = gblk + u * BPG < lim;
      w[u] = __builtin_amdgcn_raw_buffer_load_b128(wrs, ok ? vo_w : kOob, so_w + u * BPG * 128, 2);
      w2[u] = __builtin_amdgcn_raw_buffer_load_b128(wrs, ok ? vo_w + 16 : kOob, so_w + u * BPG * 128, 2);
    }
  };
  load(0, 0);
  int lp = 0, lst = 0;  // the next tile to load
  auto advance = [&](int& p, int& st) {
    if (++st == nsteps) {
      st = 0;
      ++p;
    }
  };
  advance(lp, lst);

  // ---- stage the columns: block b of column m (LDS slot m * nblk_pad + b) = its 256 q8 values at slot * XB, as 16
  // pieces of 16 bytes with piece 4j + i (j = the 64-value group, i its quarter) at position 4j + (i + j) % 4 (lane q
  // reads its group's quarter i at instruction i, so the four lanes of a quad read four different bank ranges);
  // bs[slot][i] = the int32 sum of sub-block i's 32 values (two q8_K bsums); dx[slot] = d_x.  Slots past nblk hold
  // zero sums and d_x, so a block past the row's end (zero weights and scales) adds exact zeros ----
  unsigned char* xs = lds;
  int* bs = reinterpret_cast<int*>(lds + MC * nblk_pad * XB);
  float* dxs = reinterpret_cast<float*>(bs + MC * nblk_pad * 8);
  auto stage_one = [&](int i, const f32x4 (&v)[4], const u32x4& xq16, float dxv) {
    const int r = i & 15;
    const int bi = i >> 4;  // flattened block of the columns
    int b = bi;             // its LDS slot
    if constexpr (MC > 1) b += (bi / nblk) * (nblk_pad - nblk);
    u32x4 qv;
    float d;
    int s16;
    if constexpr (FUSED) {
      int qsum;
      s16 = q8_K_row16(v, r, qv, d, qsum);  // the quant_q8_K arithmetic (byte-identical planes)
      if (__builtin_expect(blockIdx.x == 0 && XQo != nullptr, 0)) {  // one workgroup writes the q8_K planes out
        reinterpret_cast<u32x4*>(XQo)[i] = qv;
        if (r == 0) XDo[bi] = d;
        if (XBo != nullptr) XBo[i] = static_cast<int16_t>(s16);
      }
    } else {
      qv = xq16;
      d = dxv;
      s16 = 0;
#pragma unroll
      for (int t = 0; t < 4; ++t) s16 = __builtin_amdgcn_sdot4(static_cast<int>(qv[t]), 0x01010101, s16, false);
    }
    const int s32 = group_sum(s16, 2);  // lanes r, r ^ 1 hold the two halves of sub-block r / 2
    *reinterpret_cast<u32x4*>(xs + b * XB + ((r & ~3) | (((r & 3) + (r >> 2)) & 3)) * 16) = qv;
    if ((r & 1) == 0) bs[b * 8 + (r >> 1)] = s32;
    if (r == 0) dxs[b] = d;
  };
  if (stg) stage_one(tid, xf, x16, xdv);
  // columns longer than one staging pass of the workgroup (out of line: none at the decode shapes)
  if (__builtin_expect(nstage > nthreads, 0)) {
    for (int i = tid + nthreads; i < nstage; i += nthreads) {
      f32x4 v[4];
      u32x4 xq16;
      float dxv = 0.0f;
      if constexpr (FUSED) {
        const f32x4* src = reinterpret_cast<const f32x4*>(static_cast<const float*>(XA) + i * 16);
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = src[t];
      } else {
        xq16 = *reinterpret_cast<const u32x4*>(static_cast<const int8_t*>(XA) + i * 16);
        if ((i & 15) == 0) dxv = XD[i >> 4];
      }
      stage_one(i, v, xq16, dxv);
    }
  }
  const int npad = nblk_pad - nblk;
  for (int i = tid; i < MC * npad * 8; i += nthreads) {
    const int m = i / (npad * 8);
    const int e = i - m * npad * 8;
    const int b = m * nblk_pad + nblk + (e >> 3);
    bs[b * 8 + (e & 7)] = 0;
    if ((e & 7) == 0) dxs[b] = 0.0f;
  }
  // Publish the LDS writes to the workgroup.  Nothing else needs publishing, so the barrier waits for LDS operations
  // only and the weight loads stay in flight; the compiler fences keep every LDS access on its side of the barrier.
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left as they are
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // ---- stream the weights ----
  const unsigned char* xl = xs + gblk * XB;  // lane q's 64 activations (sub-blocks 2q, 2q + 1): quarter i at xo[i]
  unsigned xo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) xo[i] = static_cast<unsigned>((4 * q + ((i + q) & 3)) * 16);
  const int* bl = bs + gblk * 8 + 2 * q;
  const float* dl = dxs + gblk;
  // the lane's scale selection (gemv_impl::q4_k_scale_pair): sub-blocks 2q, 2q + 1 are bytes 2 (q & 1), +1 of the
  // scales and of the mins, taken from the high-nibble form for q >= 2
  const unsigned hiq = q >= 2 ? ~0u : 0u;
  const unsigned jb = 2u * (q & 1);
  const unsigned sel = jb | ((jb + 1) << 8) | ((jb + 4) << 16) | ((jb + 5) << 24);
  float acc[MC];
  int p = 0, st = 0;  // the tile being dotted: pass p, K step st
  auto tile = [&](bool next) {
    const int rl = p * RPW + grp;
    const int row = row_base + rl;
    const bool rv = rl < wave_rows && row < N;
    if (st == 0) {
#pragma unroll
      for (int m = 0; m < MC; ++m) acc[m] = 0.0f;
    }
    const int tb = st * BSTEP;
    const int lim = nblk - tb;  // blocks from the tile's first to the row's end (wave-uniform)
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      if (u * BPG >= lim) break;  // wave-uniform: no lane of the wave has a block in this slot or the next
      const float dw = f16_bits_to_f32(static_cast<int16_t>(sc[u][0] & 0xFFFFu));
      const float dmin = f16_bits_to_f32(static_cast<int16_t>(sc[u][0] >> 16));
      const unsigned scm = gemv_impl::q4_k_scale_pair(sc[u], hiq, sel);
      const int b = tb + u * BPG + gblk;
#pragma unroll
      for (int m = 0; m < MC; ++m) {
        const int bo = m * nblk_pad + tb + u * BPG;  // the slot's first block (the lane's is bo + gblk)
        const unsigned char* xp = xl + bo * XB;
        const int2 dd = gemv_impl::q4_k_group_dots<MODE_DP4A>(
            w[u], w2[u], *reinterpret_cast<const u32x4*>(xp + xo[0]), *reinterpret_cast<const u32x4*>(xp + xo[1]),
            *reinterpret_cast<const u32x4*>(xp + xo[2]), *reinterpret_cast<const u32x4*>(xp + xo[3]));
        const int2 xsum = *reinterpret_cast<const int2*>(bl + bo * 8);
        // 24-bit multiplies (full rate): |dots| < 2^16, |sums| < 2^13, scales and mins < 64
        const int sd = __mul24(static_cast<int>(scm & 0xFFu), dd.x) + __mul24(static_cast<int>((scm >> 8) & 0xFFu), dd.y);
        const int sm = __mul24(static_cast<int>((scm >> 16) & 0xFFu), xsum.x) + __mul24(static_cast<int>(scm >> 24), xsum.y);
        const int sdb = group_sum(sd, 4), smb = group_sum(sm, 4);  // the block's exact (sd, sm), every lane
        if (__builtin_expect(S != nullptr, 0)) {
          if (q == 0 && rv && b < nblk) {
            int32_t* sp = S + ((static_cast<int64_t>(m) * N + row) * nblk + b) * 2;
            sp[0] = sdb;
            sp[1] = smb;
          }
        }
        // y += d * dx * sd - dmin * dx * sm, once per block (lane 0 of the quad)
        const float dx = dl[bo];
        const float t = __builtin_fmaf(static_cast<float>(sdb), dw * dx, acc[m]);
        const float t2 = __builtin_fmaf(-static_cast<float>(smb), dmin * dx, t);
        acc[m] = q == 0 ? t2 : acc[m];
      }
    }
    if (next && lp < npass) {  // no load past the wave's last tile
      load(lp, lst);
      advance(lp, lst);
    }
    if (st == nsteps - 1) {
#pragma unroll
      for (int m = 0; m < MC; ++m) {
        const float v = group_sum(acc[m], LPR);
        if ((lane & (LPR - 1)) == 0 && rv) Y[static_cast<int64_t>(m) * N + row] = v;
      }
    }
    advance(p, st);
  };
  const int ntiles = ONE ? 1 : npass * nsteps;
  for (int t = 0; t < ntiles; ++t) tile(!ONE);
}

#define KOMP_Q4K_LEAN_ARGS                                                                                        \
  int N1, int nblk, int SW1, int nseg, int rows_per_wg, int passes, const uint8_t *__restrict__ WQ1,                 \
      const int16_t *__restrict__ WS1, const void *__restrict__ XA, const float *__restrict__ XD,                     \
      float *__restrict__ Y1, int32_t *__restrict__ S, int8_t *__restrict__ XQo, float *__restrict__ XDo,            \
      int16_t *__restrict__ XBo, const GemvSegs segs
#define KOMP_Q4K_LEAN_PASS N1, nblk, SW1, nseg, rows_per_wg, passes, WQ1, WS1, XA, XD, Y1, S, XQo, XDo, XBo, segs

template <int LPR, int NB, int MC, bool FUSED, bool ONE>
__global__ void __launch_bounds__(1024) q4k_lean_kernel(KOMP_Q4K_LEAN_ARGS) {
  q4k_lean_body<LPR, NB, MC, FUSED, ONE>(KOMP_Q4K_LEAN_PASS);
}

#undef KOMP_Q4K_LEAN_ARGS
#undef KOMP_Q4K_LEAN_PASS

template <int LPR, int NB, int MC, bool FUSED>
hipError_t launch_k(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  const bool one = p.passes == 1 && c.k / 256 <= (LPR / 4) * NB;
  auto kern = one ? q4k_lean_kernel<LPR, NB, MC, FUSED, true> : q4k_lean_kernel<LPR, NB, MC, FUSED, false>;
  GemvSegs segs = c.segs;
  int64_t groups = (c.n + p.block_n - 1) / p.block_n;
  if (c.nseg > 1) {
    groups = 0;
    for (int i = 0; i < c.nseg; ++i) {
      segs.first_wg[i] = static_cast<int>(groups);
      groups += (segs.n[i] + p.block_n - 1) / p.block_n;
    }
  }
  const int nblk = c.k / 256;
  const size_t lds = q4k_lean_lds_bytes(LPR, NB, MC, c.k);
  static std::atomic<unsigned> lds_limit[2][kMaxDevices];  // each kernel's allowed dynamic LDS, per device
  const hipError_t le = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds, lds_limit[one ? 1 : 0]);
  if (le != hipSuccess) return le;
  const dim3 grid(static_cast<unsigned>(groups));
  const dim3 block(static_cast<unsigned>(64 * p.waves));
  const void* xa = FUSED ? static_cast<const void*>(c.x) : static_cast<const void*>(c.xq);
  const int sw = static_cast<int>(c.nseg > 1 ? 0 : c.sw);  // below 2^31 (q4k_lean_eligible); segments carry theirs
  const Timing tm = timing_slot(gemv_kind(FMT_Q4_K));
  if (tm.on) {
    hipExtLaunchKernelGGL(kern, grid, block, lds, stream, tm.start, tm.stop, 0, c.n, nblk, sw, c.nseg, p.block_n,
                          p.passes, c.wq, c.ws, xa, c.xd, c.y, c.s, c.xq_out, c.xd_out, c.xb_out, segs);
  } else {
    hipLaunchKernelGGL(kern, grid, block, lds, stream, c.n, nblk, sw, c.nseg, p.block_n, p.passes, c.wq, c.ws, xa,
                       c.xd, c.y, c.s, c.xq_out, c.xd_out, c.xb_out, segs);
  }
  return hipGetLastError();
}

template <int LPR, int MC, bool FUSED>
hipError_t by_nb(const GemvCall& c, const GemvPlan& p, hipStream_t s) {
  switch (p.nb) {
    case 1: return launch_k<LPR, 1, MC, FUSED>(c, p, s);
    case 2: return launch_k<LPR, 2, MC, FUSED>(c, p, s);
    case 4: return launch_k<LPR, 4, MC, FUSED>(c, p, s);
  }
  return hipErrorInvalidValue;
}

template <int LPR, bool FUSED>
hipError_t by_mc(const GemvCall& c, const GemvPlan& p, hipStream_t s) {
  switch (c.m) {
    case 1: return by_nb<LPR, 1, FUSED>(c, p, s);
    case 2: return by_nb<LPR, 2, FUSED>(c, p, s);
    case 3: return by_nb<LPR, 3, FUSED>(c, p, s);
  }
  return hipErrorInvalidValue;
}

// The lean Q4_K kernels, unfused (gemv_q4k.hip) or fused (gemv_q4k_fused.hip), each its own translation unit.
template <bool FUSED>
hipError_t launch_fused(const GemvCall& c, const GemvPlan& p, hipStream_t s) {
  switch (p.lpr_log2) {
    case 2: return by_mc<4, FUSED>(c, p, s);
    case 3: return by_mc<8, FUSED>(c, p, s);
    case 4: return by_mc<16, FUSED>(c, p, s);
    case 5: return by_mc<32, FUSED>(c, p, s);
    case 6: return by_mc<64, FUSED>(c, p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace gemv_q4k
}  // namespace komp
