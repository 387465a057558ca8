// Q4_0 and IQ4_NL decode GEMVs of 1-3 activation columns in dp4a mode, and Q4_0's in bytes mode (16-byte blocks of 32
// nibbles, q8_0 activations), unfused and fused with the q8_0 quantizer.  Same plans, lanes, accumulation order,
// results and S as the general kernel in gemv_kernel.h (kernels.py:48-94 semantics: lane g of a row group takes blocks
// st * G * nb + u * G + g and adds s * d_w * d_x per block and column, the row group's lanes are added at the end),
// with what the general kernel keeps at run time made compile-time (G lanes per row, nb blocks per lane and K step, MC
// columns):
//   * weight and scale loads are buffer loads from loop-invariant per-lane offsets, the step and block offsets being
//     a scalar and an immediate; a block past the row's end, and every row past the matrix, reads zeros without
//     touching memory, so no load sits behind a branch and each block's dot waits for its own load only;
//   * the staged columns' low halves, high halves and block metadata are three LDS arrays indexed by column and
//     block, so a block's reads are per-lane bases plus immediates.  Bytes mode stages each half as 16-bit integers,
//     its even and its odd bytes in two arrays, and multiply-adds every nibble with its activation two a lane and
//     instruction (v_pk_mad_u16);
//   * the staging's activation loads are issued before the weight loads, and the barrier that publishes the staged
//     column waits for LDS writes only, so the weights stay in flight through the staging.
#pragma once

#include "gemv_kernel.h"

namespace komp {
namespace gemv_q4 {

constexpr unsigned kOob = 0x7FFFFFF0u;  // a buffer offset past every descriptor's range: the load returns zeros

// A raw buffer descriptor over `bytes` (at most 0x7FFFFFF0: one pass's rows, which the plans keep below 2^31 bytes).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// Bytes mode: the exact int32 dot of one Q4_0 block with every nibble and activation unpacked to an integer first,
// from corr = -8 * sum(x of the block).  le / lo: the even / odd bytes of activations 0..15 as 16-bit integers
// (sext_even / sext_odd of each dword), he / ho those of 16..31; the low nibble of byte t pairs with activation t, the
// high one with 16 + t.  Each nibble is isolated into a 16-bit half (bytes 0, 2 or 1, 3 of a weight dword at once):
// a half adds 16 products of at most 15 x 128, so |sum| <= 30720 and the 16-bit sums are exact.
__device__ __forceinline__ int q4_0_block_dot_bytes(const u32x4& w, const u32x4& le, const u32x4& lo, const u32x4& he,
                                                    const u32x4& ho, int corr) {
  s16x2 acc = {0, 0};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    acc += halves(w[d] & 0x000F000Fu) * halves(le[d]);          // low nibbles of bytes 0, 2
    acc += halves((w[d] >> 8) & 0x000F000Fu) * halves(lo[d]);   // low nibbles of bytes 1, 3
    acc += halves((w[d] >> 4) & 0x000F000Fu) * halves(he[d]);   // high nibbles of bytes 0, 2
    acc += halves((w[d] >> 12) & 0x000F000Fu) * halves(ho[d]);  // high nibbles of bytes 1, 3
  }
  return corr + static_cast<int>(acc.x) + static_cast<int>(acc.y);
}

// G lanes per row group, NB blocks per lane per K step, MC activation columns.  The arguments every first load needs,
// and the segment count, fill the 14 preloaded argument dwords (a 32-bit row stride: the plans that run here keep a
// pass's rows below 2^31 bytes).  ONE: the plan has one pass and one K step, so the weight stream is straight-line
// code with no loop and no reload (a launch starts with a cold instruction cache, and every 64-byte line of code on
// the way to the first dot costs tens of nanoseconds of fetch).
// BYTES: Q4_0 in bytes mode (q4_0_block_dot_bytes on 16-bit activations); otherwise dp4a.
// PIPE: the loop form with the weight loads software-pipelined, for waves of many tiles (the reference's knob plans).
template <int FMT, int G, int NB, int MC, bool FUSED, bool ONE, bool BYTES, bool PIPE = false>
__device__ __forceinline__ void q4_lean_body(int N1, int nblk, int SW1, int nseg, int rows_per_wg, int passes,
                                             const uint8_t* __restrict__ WQ1, const int16_t* __restrict__ WS1,
                                             const void* __restrict__ XA, const float* __restrict__ XD,
                                             float* __restrict__ Y1, int32_t* __restrict__ S, int8_t* __restrict__ XQo,
                                             float* __restrict__ XDo, const GemvSegs& segs) {
  constexpr int RPW = 64 / G;   // rows per wave and pass
  constexpr int BSTEP = G * NB;  // blocks per K step
  extern __shared__ __align__(16) unsigned char lds[];
  const int tid = threadIdx.x;
  // ---- the staging's first loads, issued first (they need only preloaded arguments, so they go out before the
  // segment table of a multi-matrix launch is read, and before the weights): fused, 8 lanes per block with 4 f32
  // values each; unfused, one lane per block with its 32 q8 bytes and d_x.  Blocks of all columns in order (X [MC][K]
  // and XQ [MC][K] are dense, so block i of the flattened columns starts at 32 i; XD [MC][nblk] likewise) ----
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
  if (__builtin_expect(nseg > 1, 0)) {  // several matrices sharing the column: this workgroup's one (scalar compares on the arguments)
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
  const int g = lane & (G - 1);
  const int grp = lane / G;
  const int nsteps = ONE ? 1 : (nblk + BSTEP - 1) / BSTEP;
  const int npass = ONE ? 1 : passes;
  const int nblk_pad = nsteps * BSTEP;
  const int rows_per_wave = RPW * npass;
  const int row_base = wg * rows_per_wg + wave * rows_per_wave;  // wave-uniform
  const int wave_rows = min(rows_per_wave, rows_per_wg - wave * rows_per_wave);
  const int vrows = max(0, min(wave_rows, N - row_base));  // rows of this wave inside the matrix
  const unsigned vo_w = grp * SW + g * 16;
  const unsigned vo_s = static_cast<unsigned>((grp * nblk + g) * 2);

  // ---- weights: tile (p, st) = rows p * RPW + grp of the wave, blocks st * BSTEP + u * G + g.  The pipelined form
  // keeps D tiles in flight, 8 chunks a lane: tile t is loaded into buffer t % D while tile t - D + 1 is being dotted,
  // so a K step waits for its own loads only instead of a memory round trip per step (nb 8 keeps one buffer: two
  // would take the kernel past 128 VGPRs; 16 chunks a lane measured slower, 7.5 -> 8.3 us at Q4_0 4096 x 4096 with
  // block_n 64, nb 4, 4 waves).  The other forms keep one buffer, which holds fewer registers: with two tiles a wave
  // or several workgroups a CU that is faster ----
  constexpr int D = (!PIPE || NB >= 8) ? 1 : 8 / NB;
  u32x4 w[D][NB];
  int16_t sc[D][NB];
  // One form for every tile, with no branch: a block past the row's end swaps its per-lane offset for the
  // out-of-range one, and a tile past the wave's last (p = npass) has a descriptor of no rows, so every load of the
  // loop is issued whatever the tile and the compiler counts the loads in flight exactly (behind a branch it waits
  // for all of them at the join).
  auto load = [&](u32x4 (&wb)[NB], int16_t (&sb)[NB], int p, int st) {
    // a descriptor per pass, over the pass's rows inside the matrix: a row past the matrix lies past the range,
    // which the per-lane offset is checked against, and reads zeros; the step goes into the scalar offset, and the
    // per-lane offsets stay the same in every pass
    const int prow = p * RPW;  // wave-uniform
    const unsigned rows = __builtin_amdgcn_readfirstlane(min(RPW, max(0, vrows - prow)));  // wave-uniform
    const auto wrs = rsrc(WQ + static_cast<int64_t>(row_base + prow) * SW, rows * SW);
    const auto srs = rsrc(WS + static_cast<int64_t>(row_base + prow) * nblk, rows * static_cast<unsigned>(nblk) * 2);
    const unsigned so_w = static_cast<unsigned>(st * BSTEP * 16);
    const unsigned so_s = static_cast<unsigned>(st * BSTEP * 2);
    const int lim = nblk - st * BSTEP;  // blocks from the step's first to the row's end (wave-uniform)
#pragma unroll
    for (int u = 0; u < NB; ++u) {  // the scales first: a block's dot then waits for its own weight load only
      const bool ok = g + u * G < lim;
      sb[u] = static_cast<int16_t>(__builtin_amdgcn_raw_buffer_load_b16(srs, ok ? vo_s + u * G * 2 : kOob, so_s, 0));
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const bool ok = g + u * G < lim;
      wb[u] = __builtin_amdgcn_raw_buffer_load_b128(wrs, ok ? vo_w + u * G * 16 : kOob, so_w, 2);
    }
  };
  load(w[0], sc[0], 0, 0);
  int lp = 0, lst = 0;  // the next tile to load
  auto advance = [&](int& p, int& st) {
    if (++st == nsteps) {
      st = 0;
      ++p;
    }
  };
  advance(lp, lst);

  // ---- stage the columns: xl[m][b] = activations 0..15 of block b of column m, xh[m][b] = 16..31, meta[m][b] =
  // {d_x bits, -8 * sum(x) (Q4_0; IQ4_NL 0)} for b < nblk_pad (zeros past nblk, so a block past the row's end adds 0);
  // column m at m * nblk_pad ----
  // bytes mode: xl and xh hold the even bytes as 16-bit integers, xlo and xho the odd ones
  constexpr int PL = BYTES ? 2 : 1;
  u32x4* xl = reinterpret_cast<u32x4*>(lds);
  u32x4* xh = xl + PL * MC * nblk_pad;
  u32x4* xlo = xl + MC * nblk_pad;
  u32x4* xho = xh + MC * nblk_pad;
  int2* meta = reinterpret_cast<int2*>(xh + PL * MC * nblk_pad);
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
    if constexpr (BYTES) {
      reinterpret_cast<unsigned*>(e < 4 ? xl + b : xh + b)[e & 3] = sext_even(packed);
      reinterpret_cast<unsigned*>(e < 4 ? xlo + b : xho + b)[e & 3] = sext_odd(packed);
    } else {
      reinterpret_cast<unsigned*>(e < 4 ? xl + b : xh + b)[e & 3] = packed;
    }
    if (e == 0) meta[b] = make_int2(__float_as_int(d), FMT == FMT_Q4_0 ? -8 * qsum : 0);
    if (__builtin_expect(blockIdx.x == 0 && XQo != nullptr, 0)) {  // one workgroup writes the q8_0 planes out
      reinterpret_cast<unsigned*>(XQo)[i] = packed;
      if (e == 0) XDo[bi] = d;
    }
  };
  auto stage_q8 = [&](int bi, const u32x4& a, const u32x4& c, float dxv) {
    const int b = slot(bi);
    int sum = 0;
    if constexpr (BYTES) {  // the values unpacked to 16-bit integers, stored and added (|sum| <= 32 x 128)
      u32x4 ae, ao, ce, co;
      s16x2 t = {0, 0};
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        ae[d] = sext_even(a[d]);
        ao[d] = sext_odd(a[d]);
        ce[d] = sext_even(c[d]);
        co[d] = sext_odd(c[d]);
        t += halves(ae[d]) + halves(ao[d]) + halves(ce[d]) + halves(co[d]);
      }
      xl[b] = ae;
      xlo[b] = ao;
      xh[b] = ce;
      xho[b] = co;
      sum = static_cast<int>(t.x) + static_cast<int>(t.y);
    } else {
      xl[b] = a;
      xh[b] = c;
      if constexpr (FMT == FMT_Q4_0) {  // the -8 offset of the Q4_0 nibbles
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          sum = __builtin_amdgcn_sdot4(static_cast<int>(a[d]), 0x01010101, sum, false);
          sum = __builtin_amdgcn_sdot4(static_cast<int>(c[d]), 0x01010101, sum, false);
        }
      }
    }
    meta[b] = make_int2(__float_as_int(dxv), -8 * sum);
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
    meta[m * nblk_pad + nblk + (i - m * (nblk_pad - nblk))] = make_int2(0, 0);
  }
  // Publish the LDS writes to the workgroup.  Nothing else needs publishing (no other shared or global data is read
  // back), so the barrier waits for LDS operations only and the weight loads stay in flight; the compiler fences
  // keep every LDS access on its side of the barrier.
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left as they are
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // the loop form's next tiles, issued once the staging is done: a staging pass that loads after them would wait for
  // them too (loads retire in issue order)
#pragma unroll
  for (int d = 1; d < D; ++d) {
    load(w[d], sc[d], lp, lst);
    advance(lp, lst);
  }

  // ---- stream the weights ----
  const u32x4* xlg = xl + g;
  const u32x4* xhg = xh + g;
  const u32x4* xlog = xlo + g;
  const u32x4* xhog = xho + g;
  const int2* mg = meta + g;
  float acc[MC];
  int p = 0, st = 0;  // the tile being dotted: pass p, K step st
  // Dot the tile in buffer (wb, sb), then (next) load tile t + D into it, past the wave's last tile a load of no rows
  // (zeros, no memory touched); the pass's outputs are stored after its last step.
  auto tile = [&](u32x4 (&wb)[NB], int16_t (&sb)[NB], bool next) {
    const int rl = p * RPW + grp;
    const int row = row_base + rl;
    const bool rv = rl < wave_rows && row < N;
    if (st == 0) {
#pragma unroll
      for (int m = 0; m < MC; ++m) acc[m] = 0.0f;
    }
    const int tb = st * BSTEP;
    const int lim = nblk - tb;  // blocks from the step's first to the row's end (wave-uniform)
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      // no lane of the wave has a block in this slot or the next (the row's last step): skipped, except in the
      // pipelined form, which dots them (zero weights and activations), since a branch here would make the compiler
      // wait for every load in flight
      if (D == 1 && u * G >= lim) break;
      const int bo = tb + u * G;
      const float dw = f16_bits_to_f32(sb[u]);
#pragma unroll
      for (int m = 0; m < MC; ++m) {
        const int bm = m * nblk_pad + bo;
        const int2 mt = mg[bm];
        int s;
        if constexpr (BYTES)
          s = q4_0_block_dot_bytes(wb[u], xlg[bm], xlog[bm], xhg[bm], xhog[bm], mt.y);
        else if constexpr (FMT == FMT_Q4_0)
          s = gemv_impl::q4_0_block_dot<MODE_DP4A>(wb[u], xlg[bm], xhg[bm], mt.y);
        else
          s = gemv_impl::iq4_nl_block_dot<MODE_DP4A>(wb[u], xlg[bm], xhg[bm]);
        if (__builtin_expect(S != nullptr, 0) && rv && bo + g < nblk) S[(static_cast<int64_t>(m) * N + row) * nblk + bo + g] = s;
        acc[m] += static_cast<float>(s) * dw * __int_as_float(mt.x);  // kernels.py:93 order
      }
    }
    if (next && (D > 1 || lp < npass)) {  // one buffer: nothing to pipeline, no load past the wave's last tile
      load(wb, sb, lp, lst);
      advance(lp, lst);
    }
    if (st == nsteps - 1) {
#pragma unroll
      for (int m = 0; m < MC; ++m) {
        const float v = group_sum(acc[m], G);
        if (g == 0 && rv) Y[static_cast<int64_t>(m) * N + row] = v;
      }
    }
    advance(p, st);
  };
  // Whole rounds of D tiles in the loop, with no branch that leaves a round midway (behind one, the loads in flight
  // would reach the loop's head in two orders, and the compiler would wait for the stricter of them), then the last
  // T mod D tiles straight-line, with nothing left to load
  const int ntiles = npass * nsteps;
  const int rounds = ONE ? 1 : ntiles / D;
  for (int r = 0; r < rounds; ++r) {
#pragma unroll
    for (int d = 0; d < D; ++d) tile(w[d], sc[d], !ONE);
  }
  if constexpr (D > 1) {
    const int rest = ntiles - rounds * D;  // wave-uniform
#pragma unroll
    for (int d = 0; d < D - 1; ++d)
      if (d < rest) tile(w[d], sc[d], false);
  }
}

#define KOMP_Q4_LEAN_ARGS                                                                                         \
  int N1, int nblk, int SW1, int nseg, int rows_per_wg, int passes, const uint8_t *__restrict__ WQ1,                 \
      const int16_t *__restrict__ WS1, const void *__restrict__ XA, const float *__restrict__ XD,                     \
      float *__restrict__ Y1, int32_t *__restrict__ S, int8_t *__restrict__ XQo, float *__restrict__ XDo,            \
      const GemvSegs segs
#define KOMP_Q4_LEAN_PASS N1, nblk, SW1, nseg, rows_per_wg, passes, WQ1, WS1, XA, XD, Y1, S, XQo, XDo, segs

template <int FMT, int G, int NB, int MC, bool FUSED, bool ONE>
__global__ void __launch_bounds__(1024) q4_lean_kernel(KOMP_Q4_LEAN_ARGS) {
  q4_lean_body<FMT, G, NB, MC, FUSED, ONE, false>(KOMP_Q4_LEAN_PASS);
}

template <int G, int NB, int MC, bool FUSED, bool ONE>
__global__ void __launch_bounds__(1024) q4_lean_bytes_kernel(KOMP_Q4_LEAN_ARGS) {
  q4_lean_body<FMT_Q4_0, G, NB, MC, FUSED, ONE, true>(KOMP_Q4_LEAN_PASS);
}

// The pipelined loop forms (PIPE above) of one column, dp4a and bytes mode.
template <int FMT, int G, int NB, bool FUSED>
__global__ void __launch_bounds__(1024) q4_lean_pipe_kernel(KOMP_Q4_LEAN_ARGS) {
  q4_lean_body<FMT, G, NB, 1, FUSED, false, false, true>(KOMP_Q4_LEAN_PASS);
}
template <int G, int NB, bool FUSED>
__global__ void __launch_bounds__(1024) q4_lean_bytes_pipe_kernel(KOMP_Q4_LEAN_ARGS) {
  q4_lean_body<FMT_Q4_0, G, NB, 1, FUSED, false, true, true>(KOMP_Q4_LEAN_PASS);
}

#undef KOMP_Q4_LEAN_ARGS
#undef KOMP_Q4_LEAN_PASS

template <int FMT, int G, int NB, int MC, bool FUSED, bool BYTES>
hipError_t launch_k(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  // the single-pass, single-step form (a straight-line weight stream) for every plan of one pass and one K step; the
  // pipelined loop form for one column whose waves walk kPipeMinTiles tiles or more
  const bool one = p.passes == 1 && c.k / 32 <= G * NB;
  const bool pipe = MC == 1 && !one && NB < 8 && p.passes * ((c.k / 32 + G * NB - 1) / (G * NB)) >= kPipeMinTiles;
  auto kern = one ? q4_lean_kernel<FMT, G, NB, MC, FUSED, true> : q4_lean_kernel<FMT, G, NB, MC, FUSED, false>;
  if constexpr (BYTES)
    kern = one ? q4_lean_bytes_kernel<G, NB, MC, FUSED, true> : q4_lean_bytes_kernel<G, NB, MC, FUSED, false>;
  if constexpr (MC == 1 && NB < 8) {
    if (pipe) kern = BYTES ? q4_lean_bytes_pipe_kernel<G, NB, FUSED> : q4_lean_pipe_kernel<FMT, G, NB, FUSED>;
  }
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
  const size_t lds = q4_lean_lds_bytes(G, NB, MC, c.k, BYTES);
  static std::atomic<unsigned> lds_limit[3][kMaxDevices];  // each kernel's allowed dynamic LDS, per device
  const hipError_t le = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds, lds_limit[one ? 1 : pipe ? 2 : 0]);
  if (le != hipSuccess) return le;
  const dim3 grid(static_cast<unsigned>(groups));
  const dim3 block(static_cast<unsigned>(64 * p.waves));
  const void* xa = FUSED ? static_cast<const void*>(c.x) : static_cast<const void*>(c.xq);
  const int sw = static_cast<int>(c.nseg > 1 ? 0 : c.sw);  // below 2^31 (q4_lean_eligible); segments carry theirs
  const Timing tm = timing_slot(gemv_kind(FMT));
  if (tm.on) {
    hipExtLaunchKernelGGL(kern, grid, block, lds, stream, tm.start, tm.stop, 0, c.n, nblk, sw, c.nseg, p.block_n,
                          p.passes, c.wq, c.ws, xa, c.xd, c.y, c.s, c.xq_out, c.xd_out, segs);
  } else {
    hipLaunchKernelGGL(kern, grid, block, lds, stream, c.n, nblk, sw, c.nseg, p.block_n, p.passes, c.wq, c.ws, xa,
                       c.xd, c.y, c.s, c.xq_out, c.xd_out, segs);
  }
  return hipGetLastError();
}

template <int FMT, int G, int MC, bool FUSED, bool BYTES>
hipError_t by_nb(const GemvCall& c, const GemvPlan& p, hipStream_t s) {
  switch (p.nb) {
    case 1: return launch_k<FMT, G, 1, MC, FUSED, BYTES>(c, p, s);
    case 2: return launch_k<FMT, G, 2, MC, FUSED, BYTES>(c, p, s);
    case 4: return launch_k<FMT, G, 4, MC, FUSED, BYTES>(c, p, s);
    case 8:
      if constexpr (MC == 1) return launch_k<FMT, G, 8, MC, FUSED, BYTES>(c, p, s);
  }
  return hipErrorInvalidValue;
}

template <int FMT, int G, bool FUSED, bool BYTES>
hipError_t by_mc(const GemvCall& c, const GemvPlan& p, hipStream_t s) {
  switch (c.m) {
    case 1: return by_nb<FMT, G, 1, FUSED, BYTES>(c, p, s);
    case 2: return by_nb<FMT, G, 2, FUSED, BYTES>(c, p, s);
    case 3: return by_nb<FMT, G, 3, FUSED, BYTES>(c, p, s);
  }
  return hipErrorInvalidValue;
}

// The lean kernels of one format and mode (dp4a: gemv_q4.hip; Q4_0 bytes: gemv_q4_bytes.hip, its own translation
// unit).
template <int FMT, bool BYTES>
hipError_t launch_mode(const GemvCall& c, const GemvPlan& p, hipStream_t s) {
  const bool fused = c.x != nullptr;
  switch (p.lpr_log2) {
    case 2: return fused ? by_mc<FMT, 4, true, BYTES>(c, p, s) : by_mc<FMT, 4, false, BYTES>(c, p, s);
    case 3: return fused ? by_mc<FMT, 8, true, BYTES>(c, p, s) : by_mc<FMT, 8, false, BYTES>(c, p, s);
    case 4: return fused ? by_mc<FMT, 16, true, BYTES>(c, p, s) : by_mc<FMT, 16, false, BYTES>(c, p, s);
    case 5: return fused ? by_mc<FMT, 32, true, BYTES>(c, p, s) : by_mc<FMT, 32, false, BYTES>(c, p, s);
    case 6: return fused ? by_mc<FMT, 64, true, BYTES>(c, p, s) : by_mc<FMT, 64, false, BYTES>(c, p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace gemv_q4
}  // namespace komp
