// Q8_0 decode GEMVs of 1-3 activation columns in dp4a mode (ggml block_q8_0: 32 int8 values and an f16 d; q8_0
// activations), unfused and fused with the q8_0 quantizer.  The arithmetic is the general kernel's (gemv_kernel.h): a
// lane pair per block, lane q taking the block's 16-byte half q and its matching staged activation half, the pair's
// dots summed into the block's exact int32 dot and scaled once per block by the pair's lane 0 as f32(s) * d_w * d_x
// (kernels.py:93 order), so S and Y equal the general kernel's for the same plan.  The structure is the lean
// kernels' (gemv_q4.h): branch-free buffer loads from per-lane offsets (a block past the row's end and every row past
// the matrix read zeros without touching memory), the staging's activation loads issued before the weights, a
// barrier that waits for LDS writes only, and straight-line code for one pass and one K step.
#pragma once

#include "gemv_kernel.h"

namespace komp {
namespace gemv_q8 {

constexpr unsigned kOob = 0x7FFFFFF0u;  // a buffer offset past every descriptor's range: the load returns zeros
constexpr size_t kLdsLimit = 160 * 1024;

// A raw buffer descriptor over `bytes` (at most 0x7FFFFFF0: one pass's rows, which the plans keep below 2^31 bytes).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// LPR lanes per row group (2 per block), NB 16-byte slots per lane per K step, MC activation columns.  ONE: the plan
// has one pass and one K step.
template <int LPR, int NB, int MC, bool FUSED, bool ONE>
__device__ __forceinline__ void q8_lean_body(int N1, int nblk, int SW1, int nseg, int rows_per_wg, int passes,
                                             const uint8_t* __restrict__ WQ1, const int16_t* __restrict__ WS1,
                                             const void* __restrict__ XA, const float* __restrict__ XD,
                                             float* __restrict__ Y1, int32_t* __restrict__ S, int8_t* __restrict__ XQo,
                                             float* __restrict__ XDo, const GemvSegs& segs) {
  constexpr int RPW = 64 / LPR;   // rows per wave and pass
  constexpr int BPG = LPR / 2;    // blocks a row group covers per slot
  constexpr int BSTEP = BPG * NB;  // blocks per K step
  extern __shared__ __align__(16) unsigned char lds[];
  const int tid = threadIdx.x;
  // ---- the staging's first loads, issued first: fused, 8 lanes per block with 4 f32 values each; unfused, one lane
  // per block with its 32 q8 bytes and d_x.  The columns' blocks in order (X [MC][K], XQ [MC][K], XD [MC][nblk]
  // dense) ----
  const int nstage = FUSED ? MC * nblk * 8 : MC * nblk;
  const bool stg = tid < nstage;
  f32x4 xf;
  u32x4 xa, xb;
  float xdv = 0.0f;
  if (stg) {
    if constexpr (FUSED) {
      xf = *reinterpret_cast<const f32x4*>(static_cast<const float*>(XA) + tid * 4);
    } else {
      const u32x4* src = reinterpret_cast<const u32x4*>(static_cast<const int8_t*>(XA) + tid * 32);
      xa = src[0];
      xb = src[1];
      xdv = XD[tid];
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
  const int nthreads = blockDim.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = lane & 1;
  const int gblk = (lane & (LPR - 1)) >> 1;
  const int grp = lane / LPR;
  const int nsteps = ONE ? 1 : (nblk + BSTEP - 1) / BSTEP;
  const int npass = ONE ? 1 : passes;
  const int nblk_pad = nsteps * BSTEP;
  const int rows_per_wave = RPW * npass;
  const int row_base = wg * rows_per_wg + wave * rows_per_wave;  // wave-uniform
  const int wave_rows = min(rows_per_wave, rows_per_wg - wave * rows_per_wave);
  const int vrows = max(0, min(wave_rows, N - row_base));  // rows of this wave inside the matrix
  const unsigned vo_w = grp * SW + gblk * 32 + q * 16;
  const unsigned vo_s = static_cast<unsigned>((grp * nblk + gblk) * 2);

  // ---- weights: tile (p, st) = rows p * RPW + grp of the wave, blocks st * BSTEP + u * BPG + gblk; the lane's
  // 16-byte half and the block's scale ----
  u32x4 w[NB];
  int16_t sc[NB];
  auto load = [&](int p, int st) {
    const int prow = p * RPW;  // wave-uniform
    const unsigned rows = __builtin_amdgcn_readfirstlane(min(RPW, max(0, vrows - prow)));  // wave-uniform
    const auto wrs = rsrc(WQ + static_cast<int64_t>(row_base + prow) * SW, rows * SW);
    const auto srs = rsrc(WS + static_cast<int64_t>(row_base + prow) * nblk, rows * static_cast<unsigned>(nblk) * 2);
    const unsigned so_w = static_cast<unsigned>(st * BSTEP * 32);
    const unsigned so_s = static_cast<unsigned>(st * BSTEP * 2);
    const int lim = nblk - st * BSTEP;  // blocks from the tile's first to the row's end (wave-uniform)
#pragma unroll
    for (int u = 0; u < NB; ++u) {  // the scales first: a block's dot then waits for its own weight load only
      const bool ok = gblk + u * BPG < lim;
      sc[u] = static_cast<int16_t>(__builtin_amdgcn_raw_buffer_load_b16(srs, ok ? vo_s : kOob, so_s + u * BPG * 2, 0));
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const bool ok = gblk + u * BPG < lim;
      w[u] = __builtin_amdgcn_raw_buffer_load_b128(wrs, ok ? vo_w : kOob, so_w + u * BPG * 32, 2);
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

  // ---- stage the columns: x2[2 slot] = activations 0..15 of the block in LDS slot m * nblk_pad + b (block b of
  // column m), x2[2 slot + 1] = 16..31 (the halves interleaved, so the lanes of a pair, and neighbouring pairs, read
  // consecutive 16-byte pieces: no bank conflicts), dxs[slot] = d_x, for b < nblk_pad (zeros past nblk, so a block
  // past the row's end adds 0) ----
  u32x4* x2 = reinterpret_cast<u32x4*>(lds);
  float* dxs = reinterpret_cast<float*>(x2 + 2 * MC * nblk_pad);
  auto slot = [&](int i) {  // flattened block i of the columns -> its LDS slot
    if constexpr (MC == 1) return i;
    const int m = i / nblk;
    return i + m * (nblk_pad - nblk);
  };
  auto stage_fused = [&](int i, const f32x4& v) {
    const int e = i & 7;
    const int bi = i >> 3;
    const int b = slot(bi);
    float d;
    int qsum;
    const unsigned packed = q8_0_group8(v, d, qsum);  // the quant_q8_0 arithmetic (byte-identical planes)
    reinterpret_cast<unsigned*>(x2 + 2 * b + (e >> 2))[e & 3] = packed;
    if (e == 0) dxs[b] = d;
    if (__builtin_expect(blockIdx.x == 0 && XQo != nullptr, 0)) {  // one workgroup writes the q8_0 planes out
      reinterpret_cast<unsigned*>(XQo)[i] = packed;
      if (e == 0) XDo[bi] = d;
    }
  };
  auto stage_q8 = [&](int bi, const u32x4& a, const u32x4& c, float dxv) {
    const int b = slot(bi);
    x2[2 * b] = a;
    x2[2 * b + 1] = c;
    dxs[b] = dxv;
  };
  if (stg) {
    if constexpr (FUSED) stage_fused(tid, xf);
    else stage_q8(tid, xa, xb, xdv);
  }
  if (__builtin_expect(nstage > nthreads, 0)) {  // columns longer than one pass of the workgroup (out of line)
    for (int i = tid + nthreads; i < nstage; i += nthreads) {
      if constexpr (FUSED) {
        stage_fused(i, *reinterpret_cast<const f32x4*>(static_cast<const float*>(XA) + i * 4));
      } else {
        const u32x4* src = reinterpret_cast<const u32x4*>(static_cast<const int8_t*>(XA) + i * 32);
        stage_q8(i, src[0], src[1], XD[i]);
      }
    }
  }
  for (int i = tid; i < MC * (nblk_pad - nblk); i += nthreads) {
    const int m = i / (nblk_pad - nblk);
    dxs[m * nblk_pad + nblk + (i - m * (nblk_pad - nblk))] = 0.0f;
  }
  // Publish the LDS writes to the workgroup.  Nothing else needs publishing, so the barrier waits for LDS operations
  // only and the weight loads stay in flight; the compiler fences keep every LDS access on its side of the barrier.
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left as they are
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // ---- stream the weights ----
  const u32x4* xq = x2 + 2 * gblk + q;  // the lane's staged half of its block
  const float* dl = dxs + gblk;
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
      const float dw = f16_bits_to_f32(sc[u]);
      const int b = tb + u * BPG + gblk;
#pragma unroll
      for (int m = 0; m < MC; ++m) {
        const int bo = m * nblk_pad + tb + u * BPG;  // the slot's first block (the lane's is bo + gblk)
        const int s = group_sum(gemv_impl::q8_0_chunk_dot<MODE_DP4A>(w[u], xq[2 * bo]), 2);
        if (__builtin_expect(S != nullptr, 0)) {
          if (q == 0 && rv && b < nblk) S[(static_cast<int64_t>(m) * N + row) * nblk + b] = s;
        }
        const float f = static_cast<float>(s) * dw * dl[bo];  // kernels.py:93 order
        acc[m] += q == 0 ? f : 0.0f;
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

#define KOMP_Q8_LEAN_ARGS                                                                                         \
  int N1, int nblk, int SW1, int nseg, int rows_per_wg, int passes, const uint8_t *__restrict__ WQ1,                 \
      const int16_t *__restrict__ WS1, const void *__restrict__ XA, const float *__restrict__ XD,                     \
      float *__restrict__ Y1, int32_t *__restrict__ S, int8_t *__restrict__ XQo, float *__restrict__ XDo,            \
      const GemvSegs segs
#define KOMP_Q8_LEAN_PASS N1, nblk, SW1, nseg, rows_per_wg, passes, WQ1, WS1, XA, XD, Y1, S, XQo, XDo, segs

template <int LPR, int NB, int MC, bool FUSED, bool ONE>
__global__ void __launch_bounds__(1024) q8_lean_kernel(KOMP_Q8_LEAN_ARGS) {
  q8_lean_body<LPR, NB, MC, FUSED, ONE>(KOMP_Q8_LEAN_PASS);
}

#undef KOMP_Q8_LEAN_ARGS
#undef KOMP_Q8_LEAN_PASS

template <int LPR, int NB, int MC, bool FUSED>
hipError_t launch_k(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  const bool one = p.passes == 1 && c.k / 32 <= (LPR / 2) * NB;
  auto kern = one ? q8_lean_kernel<LPR, NB, MC, FUSED, true> : q8_lean_kernel<LPR, NB, MC, FUSED, false>;
  GemvSegs segs = c.segs;
  int64_t groups = (c.n + p.block_n - 1) / p.block_n;
  if (c.nseg > 1) {
    groups = 0;
    for (int i = 0; i < c.nseg; ++i) {
      segs.first_wg[i] = static_cast<int>(groups);
      groups += (segs.n[i] + p.block_n - 1) / p.block_n;
    }
  }
  const int nblk = c.k / 32;
  const size_t lds = q8_lean_lds_bytes(LPR, NB, MC, c.k);
  static std::atomic<unsigned> lds_limit[2][kMaxDevices];  // each kernel's allowed dynamic LDS, per device
  const hipError_t le = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds, lds_limit[one ? 1 : 0]);
  if (le != hipSuccess) return le;
  const dim3 grid(static_cast<unsigned>(groups));
  const dim3 block(static_cast<unsigned>(64 * p.waves));
  const void* xa = FUSED ? static_cast<const void*>(c.x) : static_cast<const void*>(c.xq);
  const int sw = static_cast<int>(c.nseg > 1 ? 0 : c.sw);  // below 2^31 (q8_lean_eligible); segments carry theirs
  const Timing tm = timing_slot(gemv_kind(FMT_Q8_0));
  if (tm.on) {
    hipExtLaunchKernelGGL(kern, grid, block, lds, stream, tm.start, tm.stop, 0, c.n, nblk, sw, c.nseg, p.block_n,
                          p.passes, c.wq, c.ws, xa, c.xd, c.y, c.s, c.xq_out, c.xd_out, segs);
  } else {
    hipLaunchKernelGGL(kern, grid, block, lds, stream, c.n, nblk, sw, c.nseg, p.block_n, p.passes, c.wq, c.ws, xa,
                       c.xd, c.y, c.s, c.xq_out, c.xd_out, segs);
  }
  return hipGetLastError();
}

template <int LPR, int MC, bool FUSED>
hipError_t by_nb(const GemvCall& c, const GemvPlan& p, hipStream_t s) {
  switch (p.nb) {
    case 1: return launch_k<LPR, 1, MC, FUSED>(c, p, s);
    case 2: return launch_k<LPR, 2, MC, FUSED>(c, p, s);
    case 4: return launch_k<LPR, 4, MC, FUSED>(c, p, s);
    case 8:
      if constexpr (MC == 1) return launch_k<LPR, 8, MC, FUSED>(c, p, s);
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

// The lean Q8_0 kernels, unfused (gemv_q8.hip) or fused (gemv_q8_fused.hip), each its own translation unit.
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

}  // namespace gemv_q8
}  // namespace komp
