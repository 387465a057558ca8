// TQ2_0 decode GEMV of 1-3 activation columns in dp4a and bytes modes (the BitNet decode step), unfused (q8_K in) and
// fused with the q8_K quantizer.  Same plans, block dots and S as the general kernel in gemv_kernel.h
// (kernels.py:97-142 semantics); the lanes per row group, the chunks per lane and the columns are template arguments
// here, which is what makes it leaner:
//   * weight and scale loads are buffer loads from loop-invariant per-lane offsets, the tile and chunk offsets being
//     a scalar and an immediate.  A chunk past the row's last block, and every row past the matrix, reads zeros
//     without touching memory (the buffer range check), so no load sits behind a branch and the compiler waits for
//     each chunk's own load instead of for the whole tile;
//   * the activation columns lie in LDS in their natural order, 288 bytes per 256-value block (the 32-byte pad puts the
//     four lane quads of a 16-lane row group on disjoint banks), so a chunk's four 16-byte activation pieces are one
//     base address plus immediates.  Bytes mode stages every activation as a 16-bit integer instead, in two planes of
//     that layout (the even and the odd bytes of each dword), so its pieces are read with the same bank pattern;
//   * dp4a mode dots the crumbs in place with v_dot4_i32_i8 (16 x the chunk's dot); bytes mode unpacks every crumb and
//     activation to a 16-bit integer first and multiply-adds them two a lane and instruction (v_pk_mad_u16);
//   * the lane quad's partial dots are added (two DPP adds) into the block's exact dot, and each block is scaled once:
//     chunk slot u of a quad belongs to lane u % 4, which alone loads the block's d_w and meta (d_x, -sum(x)),
//     completes the dot and scales it as d_x * d_w * f32(s) (kernels.py:141).  The general kernel lets lane 0 scale
//     every slot, so the lean kernel adds the same terms in another order (Y within the same f32 error bound; S equal).
//     Both modes compute the same exact block dots, so their Y are bit-identical;
//   * the activation loads of the staging are issued before the weight loads, and the barrier that publishes the
//     staged column waits for LDS writes only, so the weights stay in flight through the staging.
#pragma once

#include <hip/hip_ext.h>

#include "komp_device.h"
#include "komp_internal.h"

namespace komp {
namespace gemv_tq2 {

constexpr int kBlockStride = 288;        // LDS bytes per staged 256-value block
constexpr unsigned kOob = 0x7FFFFFF0u;   // a buffer offset past every descriptor's range: the load returns zeros
constexpr size_t kLdsLimit = 160 * 1024;

// A raw buffer descriptor over `bytes` (at most 0x7FFFFFF0: one pass's rows, which the plans keep below 2^31 bytes).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// The crumb masks, held in SGPRs: each masking AND is then a 4-byte instruction instead of an 8-byte one carrying a
// literal.  A launch runs from a cold instruction cache, where the weight stream's code bytes cost fetch time.
struct CrumbMasks {
  unsigned m1, m4, m16;
};
__device__ __forceinline__ CrumbMasks crumb_masks() {
  CrumbMasks k;
  asm("s_mov_b32 %0, 0x03030303" : "=s"(k.m1));
  asm("s_mov_b32 %0, 0x0c0c0c0c" : "=s"(k.m4));
  asm("s_mov_b32 %0, 0x30303030" : "=s"(k.m16));
  return k;
}

// Sum of the four signed byte products of a and b: v_dot4_i32_i8 with a zero addend, the first dot of a chain (the
// compiler otherwise clears a register for v_dot4c_i32_i8 to accumulate into).
__device__ __forceinline__ int dot4_first(unsigned a, unsigned b) {
  int r;
  asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// 16 x the partial int32 dot of one 16-byte chunk with its four 16-byte activation pieces (piece j pairs with the
// crumbs at bits 2j): three accumulators for the crumbs masked in place (x1, x4, x16) and one shift for the fourth,
// joined as (4 * (4 * a1 + a4) + a16) with two shift-adds.  Every term is a multiple of 16.
__device__ __forceinline__ int chunk_dot16(const u32x4& w, const u32x4 (&x)[4], const CrumbMasks& k) {
  int a1 = dot4_first(w[0] & k.m1, x[0][0]);
  int a4 = dot4_first(w[0] & k.m4, x[1][0]);
  int a16 = dot4_first(w[0] & k.m16, x[2][0]);
  a16 = __builtin_amdgcn_sdot4(static_cast<int>((w[0] >> 2) & k.m16), static_cast<int>(x[3][0]), a16, false);
#pragma unroll
  for (int d = 1; d < 4; ++d) {
    a1 = __builtin_amdgcn_sdot4(static_cast<int>(w[d] & k.m1), static_cast<int>(x[0][d]), a1, false);
    a4 = __builtin_amdgcn_sdot4(static_cast<int>(w[d] & k.m4), static_cast<int>(x[1][d]), a4, false);
    a16 = __builtin_amdgcn_sdot4(static_cast<int>(w[d] & k.m16), static_cast<int>(x[2][d]), a16, false);
    a16 = __builtin_amdgcn_sdot4(static_cast<int>((w[d] >> 2) & k.m16), static_cast<int>(x[3][d]), a16, false);
  }
  return (((a1 << 2) + a4) << 2) + a16;
}

// Bytes mode: the partial int32 dot of one 16-byte chunk with every weight and activation unpacked to an integer
// first.  xe[j] / xo[j]: activation piece j's even / odd bytes as 16-bit integers (sext_even / sext_odd of each
// dword); crumb j of weight byte e pairs with byte e of piece j.  Each crumb is isolated into a 16-bit half (bytes
// 0, 2 or 1, 3 of a weight dword at once) and multiplied with its activation, two products a lane and instruction
// into 16-bit sums: a half adds 32 products of at most 3 x 128, so |sum| <= 12288 and the 16-bit sums are exact
// (the low 16 bits of a product and sum are the same for signed and unsigned halves).
__device__ __forceinline__ int chunk_dot_bytes(const u32x4& w, const u32x4 (&xe)[4], const u32x4 (&xo)[4]) {
  s16x2 acc = {0, 0};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const unsigned ce = (w[d] >> (2 * j)) & 0x00030003u;      // crumb j of bytes 0 and 2
      const unsigned co = (w[d] >> (2 * j + 8)) & 0x00030003u;  // crumb j of bytes 1 and 3
      acc += halves(ce) * halves(xe[j][d]);
      acc += halves(co) * halves(xo[j][d]);
    }
  }
  return static_cast<int>(acc.x) + static_cast<int>(acc.y);
}

// c ? a : b per lane, as one v_cndmask_b32 on a lane mask in SGPRs.  Written out because the compiler turns a chain
// of such selects on the lane's quad position into an array indexed by it, which it keeps in scratch memory.
__device__ __forceinline__ int lane_select(uint64_t c, int a, int b) {
  int r;
  asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(b), "v"(a), "s"(c));
  return r;
}

// Reduce-scatter over a lane quad: p0..p3 are the lane's partial dots of four chunk slots; lane q of the quad gets
// the quad's sum for slot q.  odd / hi: the lanes whose quad position has bit 0 / bit 1 set.  Two exchanges of two
// values and one of one (three DPP adds, six selects) instead of a full quad sum per slot (eight DPP adds).
__device__ __forceinline__ int quad_scatter4(int p0, int p1, int p2, int p3, uint64_t odd, uint64_t hi) {
  // lanes q, q ^ 1: keep the slots whose bit 0 is q's
  const int t1 = lane_select(odd, p1, p0) + dpp_i<KOMP_DPP_XOR1>(lane_select(odd, p0, p1));  // slot q & 1
  const int t2 = lane_select(odd, p3, p2) + dpp_i<KOMP_DPP_XOR1>(lane_select(odd, p2, p3));  // slot (q & 1) + 2
  // lanes q, q ^ 2: keep the slot whose bit 1 is q's
  return lane_select(hi, t2, t1) + dpp_i<KOMP_DPP_XOR2>(lane_select(hi, t1, t2));
}

// The same for two slots: lanes q and q + 2 of the quad both get the quad's sum for slot q & 1.
__device__ __forceinline__ int quad_scatter2(int p0, int p1, uint64_t odd) {
  const int t = lane_select(odd, p1, p0) + dpp_i<KOMP_DPP_XOR1>(lane_select(odd, p0, p1));
  return t + dpp_i<KOMP_DPP_XOR2>(t);
}

// LPR lanes per row group (4 per block: lane q of a quad takes bytes 16q..16q+15 of the block), NB chunks per lane
// per K step, MC activation columns.  The arguments every first load needs, and the segment count, fill the 14
// preloaded argument dwords (a 32-bit row stride: the plans that run here keep a pass's rows below 2^31 bytes).
// ONE: the plan has one pass and one K step (every decode shape whose rows fit one step), so the weight stream is
// straight-line code with no loop and no reload: a launch starts with a cold instruction cache, and every 64-byte
// line of code on the way to the first dot costs tens of nanoseconds of fetch.
// BYTES: bytes mode (the activations staged as 16-bit integers, chunk_dot_bytes); otherwise dp4a (chunk_dot16).
// STAMP: the measurement instantiation.  Each wave reads the real-time counter on entry, once the staged columns are
// published, after its last weight chunk's dot and after its outputs are stored (their stores complete), and lane 0
// writes the four low words to segs.stamps[4 + 4 * (blockIdx.x * waves + wave)]; thread 0 of workgroup 0 writes the
// header {kStampMagic, waves of the grid, N, K}.  Scheduling barriers keep each reading in its place.
// PIPE: the loop form with the weight loads software-pipelined, for waves of many tiles (the reference's knob plans).
template <int LPR, int NB, int MC, bool FUSED, bool ONE, bool DMA, bool BYTES, bool STAMP = false, bool PIPE = false,
          bool PRE = false>
__device__ __forceinline__ void tq2_lean_body(int N1, int nblk, int SW1, int nseg, int rows_per_wg, int passes,
                                              const uint8_t* __restrict__ WQ1, const int16_t* __restrict__ WS1,
                                              const void* __restrict__ XA, const float* __restrict__ XD,
                                              float* __restrict__ Y1, int32_t* __restrict__ S,
                                              int8_t* __restrict__ XQo, float* __restrict__ XDo,
                                              int16_t* __restrict__ XBo, const GemvSegs& segs) {
  constexpr int RPW = 64 / LPR;          // rows per wave and pass
  constexpr int BPG = LPR / 4;           // blocks a row group covers per chunk slot
  constexpr int BSTEP = BPG * NB;        // blocks per K step
  constexpr int XB = kBlockStride;
  extern __shared__ __align__(16) unsigned char lds[];
  const int tid = threadIdx.x;
  uint64_t t_entry = 0, t_staged = 0, t_dots = 0;
  if constexpr (STAMP) {
    t_entry = __builtin_amdgcn_s_memrealtime();
    __builtin_amdgcn_sched_barrier(0);
  }
  // ---- the staging's first loads (16 threads per block), issued first: they need only preloaded arguments, so they
  // go out before anything else (the segment table of a multi-matrix launch included) and do not queue behind the
  // weights.  f32 values 16i .. 16i + 15 (fused) or q8 bytes 16i .. 16i + 15 and d_x (unfused) of the flattened
  // columns (X [MC][K], XQ [MC][K] and XD [MC][nblk] are dense) for thread i.  DMA (several q8 columns needing more
  // than one staging pass, when LDS holds them): the columns are copied global -> LDS instead (global_load_lds: no
  // registers held), every pass ahead of the weights, and staged from there; staged pass by pass from registers,
  // each later pass waits for every weight load issued before it (the load counter retires in issue order).  A
  // template flag, so that each form's wait counts are exact (behind a runtime branch the compiler makes the
  // register staging wait for the weights) ----
  const int nstage = MC * nblk * 16;
  const int nthreads = blockDim.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool stg = !DMA && tid < nstage;
  const int nsteps = ONE ? 1 : (nblk + BSTEP - 1) / BSTEP;
  const int nblk_pad = nsteps * BSTEP;
  constexpr int PL = BYTES ? 2 : 1;  // staged planes: the q8 bytes, or their even and odd bytes as 16-bit integers
  unsigned char* const raw = lds + ((MC * nblk_pad * (PL * XB + 8) + 15) & ~15);  // past the staged columns and meta
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
  if constexpr (DMA) {  // lane i's piece lands at the wave's LDS address + size * i
    typedef __attribute__((address_space(3))) void* lds_ptr;
    const int pieces = FUSED ? nstage * 4 : nstage;  // 16-byte pieces of X (f32) or XQ (q8)
    const u32x4* src = static_cast<const u32x4*>(XA);
    for (int c = wave * 64; c < pieces; c += nthreads)
      if (c + lane < pieces)
        __builtin_amdgcn_global_load_lds(src + c + lane, reinterpret_cast<lds_ptr>(reinterpret_cast<uintptr_t>(raw + c * 16)),
                                         16, 0, 0);
    if constexpr (!FUSED) {  // and d_x, one dword per block, after the q8 bytes
      unsigned char* rawd = raw + nstage * 16;
      for (int c = wave * 64; c < MC * nblk; c += nthreads)
        if (c + lane < MC * nblk)
          __builtin_amdgcn_global_load_lds(XD + c + lane, reinterpret_cast<lds_ptr>(reinterpret_cast<uintptr_t>(rawd + c * 4)),
                                           4, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);  // the copies stay ahead of the weight loads
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
  const int q = lane & 3;
  const int gblk = (lane & (LPR - 1)) >> 2;
  const int grp = lane / LPR;
  const int npass = ONE ? 1 : passes;
  const int rows_per_wave = RPW * npass;
  const int row_base = wg * rows_per_wg + wave * rows_per_wave;  // wave-uniform
  const int wave_rows = min(rows_per_wave, rows_per_wg - wave * rows_per_wave);
  const int vrows = max(0, min(wave_rows, N - row_base));  // rows of this wave inside the matrix
  const unsigned vo_w = grp * SW + gblk * 64 + q * 16;
  const unsigned vo_s = static_cast<unsigned>((grp * nblk + gblk) * 2);


  // ---- weights: tile (p, st) = rows p * RPW + grp of the wave, blocks st * BSTEP + u * BPG + gblk.  Chunk slot u of
  // a quad is scaled by lane u % 4 alone, so a lane loads the scales of its own slots only: q, q + 4 (nb 8); lanes
  // q >= nb own none (nb < 4) and read a zero scale ----
  // The pipelined form keeps D tiles in flight, 8 chunks a lane: tile t is loaded into buffer t % D while tile t - D + 1
  // is being dotted, so a K step waits for its own loads only instead of a memory round trip per step (nb 8 keeps one
  // buffer; 16 chunks a lane measured slower, 5.0 -> 5.7 us at 6912 x 2560 with block_n 64, nb 1, 4 waves).  The
  // other forms keep one buffer, which holds fewer registers.
  constexpr int NOWN = (NB + 3) / 4;
  constexpr int D = (!PIPE || NB >= 8) ? 1 : 8 / NB;
  u32x4 w[D][NB];
  int16_t sc[D][NOWN];
  const bool owner = NB >= 4 || q < NB;
  const unsigned vo_sq = vo_s + static_cast<unsigned>(q * BPG * 2);
  // One form for every tile, with no branch: a chunk past the row's end swaps its per-lane offset for the out-of-range
  // one, and a tile past the wave's last (p = npass) has a descriptor of no rows, so every load of the loop is issued
  // whatever the tile and the compiler counts the loads in flight exactly (behind a branch it waits for all of them at
  // the join).
  auto load = [&](u32x4 (&wb)[NB], int16_t (&sb)[NOWN], int p, int st) {
    // a descriptor per pass, over the pass's rows inside the matrix: a row past the matrix lies past the range,
    // which the per-lane offset is checked against, and reads zeros; the step goes into the scalar offset, and the
    // per-lane offsets stay the same in every pass
    const int prow = p * RPW;  // wave-uniform
    const unsigned rows = __builtin_amdgcn_readfirstlane(min(RPW, max(0, vrows - prow)));  // wave-uniform
    const auto wrs = rsrc(WQ + static_cast<int64_t>(row_base + prow) * SW, rows * SW);
    const auto srs = rsrc(WS + static_cast<int64_t>(row_base + prow) * nblk, rows * static_cast<unsigned>(nblk) * 2);
    const unsigned so_w = static_cast<unsigned>(st * BSTEP * 64);
    const unsigned so_s = static_cast<unsigned>(st * BSTEP * 2);
    const int lim = nblk - st * BSTEP;  // blocks from the tile's first to the row's end (wave-uniform)
    // The chunk's place in the step is wave-uniform and goes into the scalar offset too, so every chunk's load shares
    // the one per-lane offset
#pragma unroll
    for (int i = 0; i < NOWN; ++i) {  // the scales first: a chunk's dot then waits for its own weight load only
      const bool ok = owner && gblk + (q + 4 * i) * BPG < lim;
      sb[i] = static_cast<int16_t>(__builtin_amdgcn_raw_buffer_load_b16(srs, ok ? vo_sq : kOob, so_s + i * 4 * BPG * 2, 0));
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const bool ok = gblk + u * BPG < lim;
      wb[u] = __builtin_amdgcn_raw_buffer_load_b128(wrs, ok ? vo_w : kOob, so_w + u * BPG * 64, 2);
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

  // ---- stage the columns: LDS block b of column m = its 256 q8 values in order at (m * nblk_pad + b) * XB, then
  // meta[m * nblk_pad + b] = {d_x bits, -sum(x of the block)} for b < nblk_pad (zeros past nblk, so a chunk past the
  // row's end adds 0 * 0) ----
  // Bytes mode: plane 0 holds the even bytes of each staged dword and plane 1, opl bytes on, the odd ones, each as
  // two 16-bit integers (a dword of plane p at the staged dword's offset)
  unsigned char* xs = lds;
  const int opl = MC * nblk_pad * XB;
  int2* meta = reinterpret_cast<int2*>(lds + PL * opl);
  auto store_staged = [&](int b, int r, const u32x4& qv) {  // thread r's 16 values of staged block b
    unsigned char* dst = xs + b * XB + r * 16;
    if constexpr (BYTES) {
      u32x4 e, o;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        e[t] = sext_even(qv[t]);
        o[t] = sext_odd(qv[t]);
      }
      *reinterpret_cast<u32x4*>(dst) = e;
      *reinterpret_cast<u32x4*>(dst + opl) = o;
    } else {
      *reinterpret_cast<u32x4*>(dst) = qv;
    }
  };
  auto stage_one = [&](int i, const f32x4 (&v)[4], const u32x4& xq16, float dxv) {
    const int r = i & 15;
    const int bi = i >> 4;  // flattened block of the columns
    int b = bi;             // its LDS slot
    if constexpr (MC > 1) b += (bi / nblk) * (nblk_pad - nblk);
    if constexpr (FUSED) {
      u32x4 qv;
      float d;
      int qsum;
      const int bsum = q8_K_row16(v, r, qv, d, qsum);  // the quant_q8_K arithmetic (byte-identical planes)
      store_staged(b, r, qv);
      if (r == 0) meta[b] = make_int2(__float_as_int(d), -qsum);
      if (__builtin_expect(blockIdx.x == 0 && XQo != nullptr, 0)) {  // one workgroup writes the q8_K planes out
        reinterpret_cast<u32x4*>(XQo)[i] = qv;
        if (r == 0) XDo[bi] = d;
        if (XBo != nullptr) XBo[i] = static_cast<int16_t>(bsum);
      }
    } else {
      int s16 = 0;
      if constexpr (BYTES) {  // the values unpacked to 16-bit integers and added (|sum| <= 16 x 128 a thread)
        s16x2 t = {0, 0};
#pragma unroll
        for (int d = 0; d < 4; ++d)
          t += halves(sext_even(xq16[d])) + halves(sext_odd(xq16[d]));
        s16 = static_cast<int>(t.x) + static_cast<int>(t.y);
      } else {
#pragma unroll
        for (int d = 0; d < 4; ++d) s16 = __builtin_amdgcn_sdot4(static_cast<int>(xq16[d]), 0x01010101, s16, false);
      }
      const int qsum = group_sum(s16, 16);
      store_staged(b, r, xq16);
      if (r == 0) meta[b] = make_int2(__float_as_int(dxv), -qsum);
    }
  };
  if constexpr (DMA) {
    // the copies are older than the first tile's NOWN + NB loads: wait for them only, then let every wave see them
    constexpr int kN = NOWN + NB;
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((kN & 0xF) | 0x70 | 0xF00 | ((kN >> 4) << 14));  // vmcnt(NOWN + NB)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const float* rawd = reinterpret_cast<const float*>(raw + nstage * 16);
    for (int i = tid; i < nstage; i += nthreads) {
      f32x4 v[4];
      u32x4 xq16;
      float dxv = 0.0f;
      if constexpr (FUSED) {
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = *reinterpret_cast<const f32x4*>(raw + i * 64 + t * 16);
      } else {
        xq16 = *reinterpret_cast<const u32x4*>(raw + i * 16);
        if ((i & 15) == 0) dxv = rawd[i >> 4];
      }
      stage_one(i, v, xq16, dxv);
    }
  } else {
    if (stg) stage_one(tid, xf, x16, xdv);
    // one column longer than a staging pass of the workgroup (out of line: none at the decode shapes)
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
  if constexpr (STAMP) {
    __builtin_amdgcn_sched_barrier(0);
    t_staged = __builtin_amdgcn_s_memrealtime();
    __builtin_amdgcn_sched_barrier(0);
  }

  // the loop form's next tiles, issued once the staging is done: a staging pass that loads after them would wait for
  // them too (loads retire in issue order)
#pragma unroll
  for (int d = 1; d < D; ++d) {
    load(w[d], sc[d], lp, lst);
    advance(lp, lst);
  }

  // ---- stream the weights ----
  const unsigned char* xl = xs + gblk * XB + (q >> 1) * 128 + (q & 1) * 16;  // bytes 16q.. pair with x[(q/2)*128 + 32j + 16(q%2) ..]
  const int2* ml = meta + gblk;
  const uint64_t odd = __builtin_amdgcn_ballot_w64((q & 1) != 0), hi = __builtin_amdgcn_ballot_w64((q & 2) != 0);
  const CrumbMasks km = crumb_masks();
  float acc[MC];
  int p = 0, st = 0;  // the tile being dotted: pass p, K step st
  // Dot the tile in buffer (wb, sb), then (next) load tile t + D into it, past the wave's last tile a load of no rows
  // (zeros, no memory touched); the pass's outputs are stored after its last step.
  auto tile = [&](u32x4 (&wb)[NB], int16_t (&sb)[NOWN], bool next) {
    const int rl = p * RPW + grp;
    const int row = row_base + rl;
    const bool rv = rl < wave_rows && row < N;
    if (st == 0) {
#pragma unroll
      for (int m = 0; m < MC; ++m) acc[m] = 0.0f;
    }
    const int tb = st * BSTEP;
    const int lim = nblk - tb;  // blocks from the tile's first to the row's end (wave-uniform)
    // the lane's partial dots of its chunks (16 x them in dp4a mode).  Slots past the row's end hold zero weights and
    // zero scales and d_x, so they add nothing; the slots no lane of the wave has a block in (the row's last step) are
    // skipped, except in the pipelined form, which dots them, since a branch there would make the compiler wait for
    // every load in flight
    int pd[MC][NB];
#pragma unroll
    for (int m = 0; m < MC; ++m)
#pragma unroll
      for (int u = 0; u < NB; ++u) pd[m][u] = 0;
    // PRE: every slot's activation pieces and every owned block's meta are read from LDS before the first dot (slots
    // past the row's end read the zero padding), so their latency overlaps the wait for the weights instead of
    // following it; at the price of 16 VGPRs a slot, so only for launches of at most a workgroup a CU, whose
    // occupancy they do not cost (5-8 slots x columns in workgroups of at most 8 waves: 512-thread bounds)
    // (bytes mode: both planes, 32 VGPRs a slot)
    static_assert(!PRE || NB * MC * (BYTES ? 2 : 1) <= 8, "PRE: tiles of at most 8 slots x columns x planes");
    u32x4 xpre[PRE ? NB : 1][PRE ? MC : 1][4];
    u32x4 xopre[PRE && BYTES ? NB : 1][PRE && BYTES ? MC : 1][4];
    int2 mpre[PRE ? NOWN : 1][PRE ? MC : 1];
    if constexpr (PRE) {
#pragma unroll
      for (int u = 0; u < NB; ++u)
#pragma unroll
        for (int m = 0; m < MC; ++m)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            xpre[u][m][j] = *reinterpret_cast<const u32x4*>(xl + (m * nblk_pad + tb + u * BPG) * XB + 32 * j);
            if constexpr (BYTES)
              xopre[u][m][j] = *reinterpret_cast<const u32x4*>(xl + (m * nblk_pad + tb + u * BPG) * XB + opl + 32 * j);
          }
#pragma unroll
      for (int i = 0; i < NOWN; ++i) {
        const int u = NB >= 4 ? 4 * i + q : (owner ? q : 0);
#pragma unroll
        for (int m = 0; m < MC; ++m) mpre[i][m] = ml[m * nblk_pad + tb + u * BPG];
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      if (D == 1 && u * BPG >= lim) break;
#pragma unroll
      for (int m = 0; m < MC; ++m) {
        const unsigned char* xp = xl + (m * nblk_pad + tb + u * BPG) * XB;
        u32x4 xv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) xv[j] = PRE ? xpre[u][m][j] : *reinterpret_cast<const u32x4*>(xp + 32 * j);
        if constexpr (BYTES) {
          u32x4 xo[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) xo[j] = PRE ? xopre[u][m][j] : *reinterpret_cast<const u32x4*>(xp + opl + 32 * j);
          pd[m][u] = chunk_dot_bytes(wb[u], xv, xo);
        } else {
          pd[m][u] = chunk_dot16(wb[u], xv, km);
        }
        // the dot is computed here, in the slot's own block: sunk to the scaling after the loop it would keep every
        // slot's activation pieces live at once (16 VGPRs a slot and column)
        asm volatile("" : "+v"(pd[m][u]));
      }
    }
    if constexpr (STAMP) {  // the last step's dots issued
      __builtin_amdgcn_sched_barrier(0);
      t_dots = __builtin_amdgcn_s_memrealtime();
      __builtin_amdgcn_sched_barrier(0);
    }
    // lane q completes and scales the blocks of slots q, q + 4: the exact dot s = the quad's sum (/ 16) - sum(x), then
    // d_x * d_w * f32(s) (kernels.py:141 order)
#pragma unroll
    for (int i = 0; i < NOWN; ++i) {
      if (D == 1 && 4 * i * BPG >= lim) break;  // wave-uniform: every slot from 4i on lies past the row's end
      const int u = NB >= 4 ? 4 * i + q : (owner ? q : 0);  // lanes q >= nb (nb < 4) own nothing: slot 0, d_w 0
      const float dw = f16_bits_to_f32(sb[i]);
#pragma unroll
      for (int m = 0; m < MC; ++m) {
        int v;  // the quad's sum for the lane's slot u
        if constexpr (NB == 1)
          v = group_sum(pd[m][0], 4);
        else if constexpr (NB == 2)
          v = quad_scatter2(pd[m][0], pd[m][1], odd);
        else
          v = quad_scatter4(pd[m][4 * i], pd[m][4 * i + 1], pd[m][4 * i + 2], pd[m][4 * i + 3], odd, hi);
        const int2 mt = PRE ? mpre[i][m] : ml[m * nblk_pad + tb + u * BPG];
        const int s = (BYTES ? v : v >> 4) + mt.y;  // the block's exact dot
        if (__builtin_expect(S != nullptr, 0)) {
          const int b = tb + u * BPG + gblk;
          if (owner && rv && b < nblk) S[(static_cast<int64_t>(m) * N + row) * nblk + b] = s;
        }
        const float f = __int_as_float(mt.x) * dw * static_cast<float>(s);
        acc[m] += owner ? f : 0.0f;
      }
    }
    if (next && (D > 1 || lp < npass)) {  // one buffer: nothing to pipeline, no load past the wave's last tile
      load(wb, sb, lp, lst);
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
  if constexpr (STAMP) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the wave's stores have completed
    __builtin_amdgcn_sched_barrier(0);
    const uint64_t t_stored = __builtin_amdgcn_s_memrealtime();
    u32x4* rec = reinterpret_cast<u32x4*>(segs.stamps);
    const unsigned wpg = static_cast<unsigned>(nthreads) >> 6;
    if (lane == 0) {
      const u32x4 v = {static_cast<unsigned>(t_entry), static_cast<unsigned>(t_staged), static_cast<unsigned>(t_dots),
                       static_cast<unsigned>(t_stored)};
      rec[1 + blockIdx.x * wpg + static_cast<unsigned>(wave)] = v;
    }
    if (blockIdx.x == 0 && tid == 0) {
      const u32x4 h = {kStampMagic, gridDim.x * wpg, static_cast<unsigned>(N1), static_cast<unsigned>(nblk) * 256u};
      rec[0] = h;
    }
  }
}

#define KOMP_TQ2_LEAN_ARGS                                                                                        \
  int N1, int nblk, int SW1, int nseg, int rows_per_wg, int passes, const uint8_t *__restrict__ WQ1,                 \
      const int16_t *__restrict__ WS1, const void *__restrict__ XA, const float *__restrict__ XD,                     \
      float *__restrict__ Y1, int32_t *__restrict__ S, int8_t *__restrict__ XQo, float *__restrict__ XDo,            \
      int16_t *__restrict__ XBo, const GemvSegs segs
#define KOMP_TQ2_LEAN_PASS N1, nblk, SW1, nseg, rows_per_wg, passes, WQ1, WS1, XA, XD, Y1, S, XQo, XDo, XBo, segs

template <int LPR, int NB, int MC, bool FUSED, bool ONE, bool DMA>
__global__ void __launch_bounds__(1024) tq2_lean_kernel(KOMP_TQ2_LEAN_ARGS) {
  tq2_lean_body<LPR, NB, MC, FUSED, ONE, DMA, false>(KOMP_TQ2_LEAN_PASS);
}

// The single-pass, single-step dp4a form of one column with every slot's LDS reads ahead of the dots (PRE above), for
// launches of at most one workgroup a CU.
template <int LPR, int NB, int MC, bool FUSED, bool DMA>
__global__ void __launch_bounds__(NB * MC > 4 ? 512 : 1024) tq2_lean_pre_kernel(KOMP_TQ2_LEAN_ARGS) {
  tq2_lean_body<LPR, NB, MC, FUSED, true, DMA, false, false, false, true>(KOMP_TQ2_LEAN_PASS);
}

// The stamped single-pass, single-step dp4a form (STAMP above): the measurement instantiation of the tuning harness,
// with or without the early LDS reads as the plain launch would run them.
template <int LPR, int NB, int MC, bool FUSED, bool PRE>
__global__ void __launch_bounds__(PRE && NB * MC > 4 ? 512 : 1024) tq2_lean_stamped_kernel(KOMP_TQ2_LEAN_ARGS) {
  tq2_lean_body<LPR, NB, MC, FUSED, true, false, false, true, false, PRE>(KOMP_TQ2_LEAN_PASS);
}

template <int LPR, int NB, int MC, bool FUSED, bool ONE>
__global__ void __launch_bounds__(1024) tq2_lean_bytes_kernel(KOMP_TQ2_LEAN_ARGS) {
  tq2_lean_body<LPR, NB, MC, FUSED, ONE, false, true>(KOMP_TQ2_LEAN_PASS);
}

// The single-pass bytes-mode form of one column with both planes' LDS reads ahead of the dots (PRE above), for
// launches of at most one workgroup a CU.
template <int LPR, int NB, bool FUSED>
__global__ void __launch_bounds__(NB * 2 > 4 ? 512 : 1024) tq2_lean_bytes_pre_kernel(KOMP_TQ2_LEAN_ARGS) {
  tq2_lean_body<LPR, NB, 1, FUSED, true, false, true, false, false, true>(KOMP_TQ2_LEAN_PASS);
}

// The pipelined loop forms (PIPE above) of one column, dp4a and bytes mode.
template <int LPR, int NB, bool FUSED, bool BYTES>
__global__ void __launch_bounds__(1024) tq2_lean_pipe_kernel(KOMP_TQ2_LEAN_ARGS) {
  tq2_lean_body<LPR, NB, 1, FUSED, false, false, BYTES, false, true>(KOMP_TQ2_LEAN_PASS);
}

#undef KOMP_TQ2_LEAN_ARGS
#undef KOMP_TQ2_LEAN_PASS

// STAMP: the stamped instantiation (dp4a, one pass and one K step, no global -> LDS copy: tq2_lean_stampable), with
// c.segs.stamps holding the launch's records; only it is instantiated, in its own translation unit.
template <int LPR, int NB, int MC, bool FUSED, bool BYTES, bool STAMP = false>
hipError_t launch_k(const GemvCall& c, const GemvPlan& p, hipStream_t stream) {
  const bool one = p.passes == 1 && c.k / 256 <= (LPR / 4) * NB;
  // the pipelined loop form for one column whose waves walk kPipeMinTiles tiles or more
  const bool pipe = !STAMP && MC == 1 && !one && NB < 8 &&
                    p.passes * ((c.k / 256 + (LPR / 4) * NB - 1) / ((LPR / 4) * NB)) >= kPipeMinTiles;
  decltype(&tq2_lean_kernel<LPR, NB, MC, FUSED, true, false>) kern;
  bool dma = false;
  int64_t groups = (c.n + p.block_n - 1) / p.block_n;
  if (c.nseg > 1) {
    groups = 0;
    for (int i = 0; i < c.nseg; ++i) groups += (c.segs.n[i] + p.block_n - 1) / p.block_n;
  }
  // the early LDS reads for one column's single-pass form when the launch holds at most one workgroup a CU (the
  // decode shapes of a few MB): their registers cost no occupancy there (BitNet-2B 6912 x 2560 fused: span 2.64 ->
  // 2.49 us), while the many-workgroup launches of large matrices lose waves a SIMD to them (TQ2_0 32768 x 8192:
  // 13.3 -> 15.3 us)
  // (bytes mode: one column, nb <= 4, both planes read early: 6912 x 2560 3.72 -> 3.49 us, f32 in 3.67 -> 3.48,
  // 2560 x 6912 3.54 -> 3.48; but f32 in at nb 2, 2560 x 6912, 3.59 -> 3.67, so not there)
  constexpr bool kPreForm = BYTES ? (MC == 1 && NB <= 4 && (!FUSED || NB == 4)) : (NB * MC <= 4 || (MC == 2 && NB == 4));
  constexpr int kPreSlots = NB * MC * (BYTES ? 2 : 1);
  const bool pre = kPreForm && one && groups <= device_cu_count() && (kPreSlots <= 4 || p.waves <= 8);
  if constexpr (STAMP) {
    if (BYTES || !one || tq2_lean_dma(LPR, NB, MC, c.k, FUSED, 64 * p.waves, false) || c.segs.stamps == nullptr)
      return hipErrorInvalidConfiguration;
    kern = tq2_lean_stamped_kernel<LPR, NB, MC, FUSED, false>;
    if constexpr (kPreForm) {
      if (pre) kern = tq2_lean_stamped_kernel<LPR, NB, MC, FUSED, true>;
    }
  } else if constexpr (BYTES) {
    kern = one ? tq2_lean_bytes_kernel<LPR, NB, MC, FUSED, true> : tq2_lean_bytes_kernel<LPR, NB, MC, FUSED, false>;
    if constexpr (MC == 1 && NB < 8) {
      if (pipe) kern = tq2_lean_pipe_kernel<LPR, NB, FUSED, true>;
    }
    if constexpr (kPreForm) {
      if (pre) kern = tq2_lean_bytes_pre_kernel<LPR, NB, FUSED>;
    }
  } else {
    kern = one ? tq2_lean_kernel<LPR, NB, MC, FUSED, true, false> : tq2_lean_kernel<LPR, NB, MC, FUSED, false, false>;
    if constexpr (MC == 1 && NB < 8) {
      if (pipe) kern = tq2_lean_pipe_kernel<LPR, NB, FUSED, false>;
    }
    if constexpr (kPreForm) {
      if (pre) kern = tq2_lean_pre_kernel<LPR, NB, MC, FUSED, false>;
    }
    if constexpr (MC > 1 && !FUSED) {
      dma = tq2_lean_dma(LPR, NB, MC, c.k, FUSED, 64 * p.waves, false);
      if (dma) kern = one ? tq2_lean_kernel<LPR, NB, MC, FUSED, true, true> : tq2_lean_kernel<LPR, NB, MC, FUSED, false, true>;
      if constexpr (kPreForm) {
        if (dma && pre) kern = tq2_lean_pre_kernel<LPR, NB, MC, FUSED, true>;
      }
    }
  }
  GemvSegs segs = c.segs;
  if (c.nseg > 1) {
    int64_t first = 0;
    for (int i = 0; i < c.nseg; ++i) {
      segs.first_wg[i] = static_cast<int>(first);
      first += (segs.n[i] + p.block_n - 1) / p.block_n;
    }
  }
  const int nblk = c.k / 256;
  const size_t lds = tq2_lean_lds_bytes(LPR, NB, MC, c.k, FUSED, 64 * p.waves, BYTES);
  static std::atomic<unsigned> lds_limit[6][kMaxDevices];  // each kernel's allowed dynamic LDS, per device
  const hipError_t le = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds,
                                          lds_limit[pre ? 5 : (pipe ? 4 : (one ? 1 : 0) + (dma ? 2 : 0))]);
  if (le != hipSuccess) return le;
  const dim3 grid(static_cast<unsigned>(groups));
  const dim3 block(static_cast<unsigned>(64 * p.waves));
  const void* xa = FUSED ? static_cast<const void*>(c.x) : static_cast<const void*>(c.xq);
  const int sw = static_cast<int>(c.nseg > 1 ? 0 : c.sw);  // below 2^31 (tq2_lean_eligible); segments carry theirs
  const Timing tm = timing_slot(gemv_kind(FMT_TQ2_0));
  if (tm.on) {
    hipExtLaunchKernelGGL(kern, grid, block, lds, stream, tm.start, tm.stop, 0, c.n, nblk, sw, c.nseg, p.block_n,
                          p.passes, c.wq, c.ws, xa, c.xd, c.y, c.s, c.xq_out, c.xd_out, c.xb_out, segs);
  } else {
    hipLaunchKernelGGL(kern, grid, block, lds, stream, c.n, nblk, sw, c.nseg, p.block_n, p.passes, c.wq, c.ws, xa,
                       c.xd, c.y, c.s, c.xq_out, c.xd_out, c.xb_out, segs);
  }
  return hipGetLastError();
}

template <int LPR, int MC, bool FUSED, bool BYTES, bool STAMP>
hipError_t by_nb(const GemvCall& c, const GemvPlan& p, hipStream_t s) {
  switch (p.nb) {
    case 1: return launch_k<LPR, 1, MC, FUSED, BYTES, STAMP>(c, p, s);
    case 2: return launch_k<LPR, 2, MC, FUSED, BYTES, STAMP>(c, p, s);
    case 4: return launch_k<LPR, 4, MC, FUSED, BYTES, STAMP>(c, p, s);
    case 8:
      if constexpr (MC == 1) return launch_k<LPR, 8, MC, FUSED, BYTES, STAMP>(c, p, s);
  }
  return hipErrorInvalidValue;
}

template <int LPR, bool FUSED, bool BYTES, bool STAMP>
hipError_t by_mc(const GemvCall& c, const GemvPlan& p, hipStream_t s) {
  switch (c.m) {
    case 1: return by_nb<LPR, 1, FUSED, BYTES, STAMP>(c, p, s);
    case 2: return by_nb<LPR, 2, FUSED, BYTES, STAMP>(c, p, s);
    case 3: return by_nb<LPR, 3, FUSED, BYTES, STAMP>(c, p, s);
  }
  return hipErrorInvalidValue;
}

// The lean kernels of one mode (dp4a: gemv_tq2.hip, bytes: gemv_tq2_bytes.hip, the stamped dp4a instantiations:
// gemv_tq2_stamp.hip, each its own translation unit).
template <bool BYTES, bool STAMP = false>
hipError_t launch_mode(const GemvCall& c, const GemvPlan& p, hipStream_t s) {
  const bool fused = c.x != nullptr;
  switch (p.lpr_log2) {
    case 2: return fused ? by_mc<4, true, BYTES, STAMP>(c, p, s) : by_mc<4, false, BYTES, STAMP>(c, p, s);
    case 3: return fused ? by_mc<8, true, BYTES, STAMP>(c, p, s) : by_mc<8, false, BYTES, STAMP>(c, p, s);
    case 4: return fused ? by_mc<16, true, BYTES, STAMP>(c, p, s) : by_mc<16, false, BYTES, STAMP>(c, p, s);
    case 5: return fused ? by_mc<32, true, BYTES, STAMP>(c, p, s) : by_mc<32, false, BYTES, STAMP>(c, p, s);
    case 6: return fused ? by_mc<64, true, BYTES, STAMP>(c, p, s) : by_mc<64, false, BYTES, STAMP>(c, p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace gemv_tq2
}  // namespace komp
