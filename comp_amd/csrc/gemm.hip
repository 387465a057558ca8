// Batched-column GEMMs on the gfx950 matrix cores: Q4_0, Q8_0 and IQ4_NL x q8_0, TQ2_0 and Q4_K x q8_K, for any number
// M of activation columns, with the decode GEMVs' result definition (src/komp/kernels.py:48-94 and :97-142):
//   Y[m][n] = sum_b d_w(n, b) * d_x(m, b) * s(m, n, b),  s = the exact int32 dot of weight block b of row n with
//   activation block b of column m,
// and the same optional S [M][N][K/block] of exact block dots.  The GEMVs stream the weights once per 1..3 columns;
// this kernel streams them once per 64 columns, so a batch of decode tokens reads each weight byte once.
//
// Tiles.  A workgroup (W waves) owns 16*WN weight rows x 16*CN activation columns and all of K.  Its waves split K:
// a K step is 64 contiguous bytes of each weight row (4 Q4_0 blocks or 1 TQ2_0 block) and wave w takes steps
// w, w + W, w + 2W, ...; at the end the waves add their f32 partials in wave order.  Lane (r, g) (r = lane % 16,
// g = lane / 16) loads bytes 16g..16g+15 of a step for row r, so one load instruction reads 64 bytes of each of 16
// rows.  Each wave keeps D steps of activation loads and DW >= D steps of weight loads in flight (register rings;
// the step loop has no branch, so each step waits for its own loads only).  Loads go through buffer descriptors whose
// range ends at the tile's last valid row / column, with the whole offset of a load in its per-lane offset (no scalar
// offset): a load past the range (a block past K in the tile's last row, every load of a step past the wave's last)
// returns zeros without touching memory.
//
// Integer dots.  Operand lane l holds k slots of group l / 16 for row / column l % 16, the same slots in A and B
// (v_mfma_i32_16x16x32_i8: 8 bytes a lane, v_mfma_i32_16x16x64_i8: 16 bytes), so a block dot needs all four lane
// groups to hold pieces of the same block:
//   Q4_0   after the load, group g holds block 4s+g whole.  A 4x4 dword transpose across the groups
//          (v_permlane32_swap, v_permlane16_swap) leaves dword g of each of the four blocks in group g; dword g holds
//          values 4g..4g+3 (low nibbles) and 16+4g..16+4g+3 (high nibbles), so A = {w & 0x0F0F0F0F, (w >> 4) &
//          0x0F0F0F0F}.  The activations are loaded the same way (32 bytes of block 4s+g of column r in group g) and
//          transposed into B = {x[4g..4g+3], x[16+4g..16+4g+3]}.
//   Q8_0   a step is 2 blocks of 32 int8; group g holds half g%2 of block g/2, and the same transpose leaves dword g
//          of each half of each block in group g: A = {w0, w1} as loaded, no offset.
//   IQ4_NL Q4_0's byte layout; the nibbles go through ggml's 16-entry value table (two v_perm_b32 and a byte
//          select per dword), which gives signed values: no offset.
//   TQ2_0  group g holds bytes 16g..16g+15 of the block; crumb j of byte 16g+e is value (g/2)*128 + 32j + 16(g%2) + e
//          (kernels.py:102), so B for crumb j is 16 contiguous activation bytes and nothing is transposed.
//   Q4_K   a step is half a 256-value block (4 sub-blocks of 32); after the transpose sub-block i is the low (even i)
//          or high (odd i) nibbles of pieces 2(i/2) and 2(i/2)+1, i.e. Q4_0's block i; each sub-block's dot is
//          weighted by its 6-bit scale in registers and a second MFMA with the row's 6-bit min in every k slot
//          accumulates the mins term (see compute).
// Nibbles and crumbs go in unsigned (0..15, 0..2).  Their offset (-8, resp. -1, times the block's activation sum)
// comes from one more MFMA of a constant A (every byte -8, resp. -1) with the same B, which starts the accumulator,
// so every C element is the exact block dot s.  C element r of lane (c, g) is row 4g + r, column c.
//
// Scales.  The workgroup's rows of WS (16*WN rows, contiguous in WS) are copied to LDS once and read back per step in
// the C layout; d_x comes with each step's loads.  Per block: Q4_0 acc += (f32(s) * d_w) * d_x, TQ2_0
// acc += (d_x * d_w) * f32(s), each with one fused multiply-add (the GEMVs' operand order, kernels.py:93, :141).
#include <hip/hip_ext.h>

#include "komp_device.h"
#include "komp_internal.h"

namespace komp {
namespace gemm_impl {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kRsrcWord3 = 0x00020000;     // buffer descriptor word 3 on gfx9: 32-bit data, no swizzle
constexpr unsigned kOob = 0x7FFFFFF0u;     // an offset (or offset part) past every descriptor's range: zeros
constexpr unsigned NIB = 0x0F0F0F0Fu;
constexpr unsigned CRUMB = 0x03030303u;

// A raw buffer descriptor over [base, base + bytes), the range clamped to [0, 0x7FFFFFF0] (every offset the kernel
// uses below the cap is also below 2^31, which the host checks).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
  const int n = static_cast<int>(bytes <= 0 ? 0 : (bytes < 0x7FFFFFF0 ? bytes : 0x7FFFFFF0));
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, n, kRsrcWord3);
}


// 4x4 dword transpose across the four 16-lane rows of a wave: on entry row g of v[q] holds element (q, g), on exit
// row g of t[j] holds element (g, j).  permlane32_swap(x, y) exchanges x's rows 2-3 with y's rows 0-1;
// permlane16_swap(x, y) exchanges x's rows 1 and 3 with y's rows 0 and 2.
__device__ __forceinline__ void transpose4(const u32x4& v, unsigned (&t)[4]) {
  const auto a = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
  const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  t[0] = c[0];
  t[1] = c[1];
  t[2] = d[0];
  t[3] = d[1];
}

// Row stride (in floats) of the f32 scale slab: nblk rounded up to a multiple of 4.
__host__ __device__ constexpr int slab_stride(int nblk) { return (nblk + 3) & ~3; }

// Row broadcasts: on exit b[j] holds, in every row, row j of v.  permlane32_swap(v, v) gives rows (0 1 0 1) and
// (2 3 2 3); permlane16_swap of each with itself splits those into single rows.
__device__ __forceinline__ void bcast_rows(float v, float (&b)[4]) {
  const unsigned u = __float_as_uint(v);
  const auto h = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const auto lo = __builtin_amdgcn_permlane16_swap(h[0], h[0], false, false);
  const auto hi = __builtin_amdgcn_permlane16_swap(h[1], h[1], false, false);
  b[0] = __uint_as_float(lo[0]);
  b[1] = __uint_as_float(lo[1]);
  b[2] = __uint_as_float(hi[0]);
  b[3] = __uint_as_float(hi[1]);
}

__device__ __forceinline__ long pack2(unsigned lo, unsigned hi) {
  return static_cast<long>(static_cast<unsigned long>(lo) | (static_cast<unsigned long>(hi) << 32));
}

// FMT: any weight format above.  WK x WR waves: WR row groups of WN 16-row tiles each, every group's K split over WK
// waves.  CN 16-column tiles.  D steps in flight per wave.  STORE_S: also write the block dots to S (a separate
// instantiation, so the plain kernel's step loop has no branch between an MFMA and the scaling of its result).
template <int FMT, int WK, int WR, int WN, int CN, int D, bool STORE_S>
__global__ void __launch_bounds__(64 * WK * WR)
gemm_kernel(int N, int M, int K, int nblk, int64_t SW, const uint8_t* __restrict__ WQ, const int16_t* __restrict__ WS,
            const int8_t* __restrict__ XQ, const float* __restrict__ XD, float* __restrict__ Y,
            int32_t* __restrict__ S) {
  // The arguments every first load needs fill exactly the 14 argument dwords gfx950 preloads into SGPRs (16 user
  // SGPRs, 2 of them the argument pointer), so no load waits for an argument fetch; the step count and the slab
  // stride are shifts of nblk.
  constexpr bool NIB4 = FMT == FMT_Q4_0 || FMT == FMT_IQ4_NL;  // 16 nibble bytes per 32-value block
  constexpr bool Q8 = FMT == FMT_Q8_0;                           // 32 int8 bytes per 32-value block
  constexpr bool BLK32 = NIB4 || Q8;                             // the 32-value blocks (q8_0 activations)
  constexpr bool TQ2 = FMT == FMT_TQ2_0;
  constexpr bool QK = FMT == FMT_Q4_K;                           // 256-value blocks, 4 sub-blocks per 64-byte step
  constexpr int BPS = NIB4 ? 4 : (Q8 ? 2 : 1);                   // blocks per 64-byte K step (Q4_K: half a block)
  const int nsteps = QK ? 2 * nblk : (nblk + BPS - 1) / BPS;     // K steps
  // row stride of the f32 scale slab in LDS: nblk rounded up to a multiple of 4 (so Q4_0 reads a step's four scales
  // of a row with one 16-byte LDS load)
  const int ss = slab_stride(nblk);
  constexpr int W = WK * WR;
  constexpr int XV = (NIB4 || QK) ? 2 : (Q8 ? 1 : 4);            // 16-byte activation loads per column tile per step
  constexpr int WGR = 16 * WN * WR;     // rows per workgroup
  constexpr int RPW = WGR / W;          // slab rows each wave stages
  static_assert(RPW >= 1 && RPW * W == WGR, "the waves split the workgroup's rows evenly");
  extern __shared__ __align__(16) unsigned char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wk = wave % WK;  // this wave's K share ...
  const int wr = wave / WK;  // ... of row group wr
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int n0 = blockIdx.x * WGR;
  if (n0 >= N) return;  // a padding workgroup (see launch_s): the whole workgroup leaves before any barrier
  const int nw = n0 + 16 * WN * wr;  // first row of this wave's tiles
  const int m0 = blockIdx.y * (16 * CN);
  const int rows = max(0, min(16 * WN, N - nw));  // valid rows of this wave's tiles, valid columns of the workgroup
  const int cols = min(16 * CN, M - m0);
  const auto wq = rsrc(WQ + nw * SW, rows * SW);
  const auto xq = rsrc(XQ + static_cast<int64_t>(m0) * K, static_cast<int64_t>(cols) * K);
  const auto xd = rsrc(XD + static_cast<int64_t>(m0) * nblk, static_cast<int64_t>(cols) * nblk * 4);

  // Per-lane offsets are fixed, and a step adds its wave-uniform offset to them, so the whole offset of every load is
  // its per-lane offset (plus an immediate), which the range check covers; the buffer instruction's scalar offset is
  // always 0.  A step past the wave's last adds kOob instead (every per-lane offset is below 2^31, so the sum does
  // not wrap), which makes all of its loads return zeros without touching memory.  In a partial last Q4_0 step the
  // lanes of blocks past K read the next row's (column's) first bytes, or zeros past the tensor's end; those blocks
  // are skipped when the step is computed.
  unsigned va[WN];
#pragma unroll
  for (int t = 0; t < WN; ++t) va[t] = static_cast<unsigned>((16 * t + r16) * SW + 16 * g);
  // 32-value blocks: load v of column c takes bytes 64v + 16g .. +15 of the step's activations (64 contiguous bytes
  // per column per load); after the dword transpose these are exactly the B halves of blocks 2v and 2v + 1 (see
  // compute).  d_x: row group g loads block BPS*s + g's (Q8_0: + g % 2).
  unsigned vx[CN], vd[CN];
#pragma unroll
  for (int u = 0; u < CN; ++u) {
    const int c = 16 * u + r16;
    vx[u] = static_cast<unsigned>((BLK32 || QK) ? c * K + 16 * g : c * K + (g >> 1) * 128 + (g & 1) * 16);
    vd[u] = static_cast<unsigned>(c * nblk * 4 + (NIB4 ? 4 * g : (Q8 ? 4 * (g & 1) : 0)));
  }

  struct WStep {  // a K step's weight loads
    u32x4 a[WN];
  };
  struct Step {  // a K step's activation loads
    u32x4 x[CN][XV];
    float dx[CN];  // 32-value blocks: d_x of row group g's block of the step; TQ2_0: d_x of block s; Q4_K: s / 2
  };
  auto load_w = [&](WStep& w, int s) {
    const unsigned sa = s < nsteps ? 64u * s : kOob;  // wave-uniform
#pragma unroll
    for (int t = 0; t < WN; ++t) w.a[t] = __builtin_amdgcn_raw_buffer_load_b128(wq, va[t] + sa, 0, 2);  // nt: read once
  };
  auto load = [&](Step& st, int s) {
    const bool sv = s < nsteps;  // wave-uniform
    const unsigned sx = sv ? (QK ? 128u : 32u * BPS * (TQ2 ? 8u : 1u)) * s : kOob;  // activation bytes per step
    // d_x: 32-value blocks past K (the lanes of a partial last step) load zero, so such a block adds exact zeros
    const unsigned sd = !sv || (BLK32 && BPS * s + (NIB4 ? g : (g & 1)) >= nblk)
                            ? kOob : (QK ? 4u * (s >> 1) : 4u * BPS * s);  // fmt: skip
#pragma unroll
    for (int u = 0; u < CN; ++u) {
#pragma unroll
      for (int v = 0; v < XV; ++v)
        st.x[u][v] = __builtin_amdgcn_raw_buffer_load_b128(xq, vx[u] + sx + ((BLK32 || QK) ? 64 * v : 32 * v), 0, 0);
      st.dx[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xd, vd[u] + sd, 0, 0));
    }
  };

  // ---- the scale slab: f32 d_w of the workgroup's rows, row stride ss, zero past row N and past block nblk ----
  // Its first batch of loads is issued before the step loads, so converting it waits for nothing else.
  float* slab = reinterpret_cast<float*>(lds);
  constexpr int SCW = QK ? 8 : 1;  // int16 of WS per block (Q4_K: d, dmin and the 12 packed scale bytes)
  const auto ws = rsrc(WS + static_cast<int64_t>(n0) * nblk * SCW,
                       static_cast<int64_t>(max(0, min(WGR, N - n0))) * nblk * 2 * SCW);
  // Q4_K slab: per (row, block) 6 dwords {f32 d, f32 dmin, scales of sub-blocks 0-3, 4-7, mins 0-3, 4-7 (bytes)},
  // unpacked once from the 16 scale-plane bytes (ggml get_scale_min_k4's layout) by one lane
  unsigned* qslab = reinterpret_cast<unsigned*>(lds);
  u32x4 qraw[QK ? RPW : 1];
  auto qk_slab_load = [&](int c0) {
#pragma unroll
    for (int i = 0; i < (QK ? RPW : 0); ++i) {
      const int col = c0 + lane;
      qraw[i] = __builtin_amdgcn_raw_buffer_load_b128(
          ws, col < nblk ? static_cast<unsigned>(((wave * RPW + i) * nblk + col) * 16) : kOob, 0, 0);
    }
  };
  auto qk_slab_store = [&](int c0) {
#pragma unroll
    for (int i = 0; i < (QK ? RPW : 0); ++i) {
      const int col = c0 + lane;
      if (col < nblk) {
        const u32x4 r = qraw[i];
        unsigned* e = qslab + ((wave * RPW + i) * nblk + col) * 6;
        e[0] = __float_as_uint(f16_bits_to_f32(static_cast<int16_t>(r[0] & 0xFFFFu)));
        e[1] = __float_as_uint(f16_bits_to_f32(static_cast<int16_t>(r[0] >> 16)));
        e[2] = r[1] & 0x3F3F3F3Fu;
        e[3] = (r[3] & 0x0F0F0F0Fu) | ((r[1] >> 2) & 0x30303030u);
        e[4] = r[2] & 0x3F3F3F3Fu;
        e[5] = ((r[3] >> 4) & 0x0F0F0F0Fu) | ((r[2] >> 2) & 0x30303030u);
      }
    }
  };
  constexpr int kBatch = 4;  // 64-block column chunks per slab row per batch
  unsigned short h[RPW][kBatch];
  auto slab_load = [&](int c0) {
#pragma unroll
    for (int i = 0; i < RPW; ++i)
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        const int col = c0 + 64 * b + lane;
        h[i][b] = __builtin_amdgcn_raw_buffer_load_b16(
            ws, col < nblk ? static_cast<unsigned>(((wave * RPW + i) * nblk + col) * 2) : kOob, 0, 0);
      }
  };
  auto slab_store = [&](int c0) {  // columns past ss go to a per-lane spill slot after the slab (no branch)
#pragma unroll
    for (int i = 0; i < RPW; ++i)
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        const int col = c0 + 64 * b + lane;
        slab[col < ss ? (wave * RPW + i) * ss + col : WGR * ss + lane] = f16_bits_to_f32(static_cast<int16_t>(h[i][b]));
      }
  };
  if constexpr (QK) qk_slab_load(0); else slab_load(0);

  // Wave wk takes steps wk, wk + WK, ...; Q4_K: both halves of blocks wk, wk + WK, ... (its integer sums then stay
  // within the wave), i.e. steps 2(wk + WK j) and 2(wk + WK j) + 1.
  auto step_of = [&](int i) { return QK ? 2 * (wk + WK * (i >> 1)) + (i & 1) : wk + WK * i; };
  const int my = QK ? 2 * (nblk > wk ? (nblk - wk + WK - 1) / WK : 0)
                    : (nsteps > wk ? (nsteps - wk + WK - 1) / WK : 0);  // this wave's steps (wave-uniform)
  // Two rings: the activations (L2 hits) D steps ahead, the weights (HBM) DW steps ahead.  After step i's compute the
  // wave loads step i + D's activations, then step i + DW's weights.  DW = 2D for TQ2_0's 8-wave plans with one row
  // tile a wave (with two, the extra registers spill), whose steps (4 crumb MFMAs per tile, 16 activation loads)
  // leave the weights' HBM latency exposed at D (TQ2_0 6912 x 2560 at 64 columns: 18.2 -> 15.1 us); elsewhere the
  // deeper weight ring measured no faster (Q4_0 14336 x 4096 at 64 columns) or slower (at 4 and 16 columns).  The
  // first loads go out after the slab's, in the order the step loop
  // keeps (weights of steps 0..DW-D-1, then activations of step d with weights of step DW-D+d), so the compiler's wait
  // counts at the loop's head see the same order on entry as on the back edge: each step waits for its own loads.
  constexpr int DW = (TQ2 && WK * WR == 8 && WN == 1) ? 2 * D : D;
  WStep wring[DW];
  Step ring[D];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int d = 0; d < DW - D; ++d) load_w(wring[d], step_of(d));  // past the wave's steps: zeros
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int d = 0; d < D; ++d) {
    load(ring[d], step_of(d));
    load_w(wring[DW - D + d], step_of(DW - D + d));
    __builtin_amdgcn_sched_barrier(0);
  }

  if constexpr (QK) {
    qk_slab_store(0);
    for (int c0 = 64; c0 < nblk; c0 += 64) {  // rows of more than 64 blocks
      qk_slab_load(c0);
      qk_slab_store(c0);
    }
  } else {
    slab_store(0);
    for (int c0 = 64 * kBatch; c0 < ss; c0 += 64 * kBatch) {  // rows of more than 64 * kBatch blocks
      slab_load(c0);
      slab_store(c0);
    }
  }
  __syncthreads();

  f32x4 acc[WN][CN];
  i32x4 qsd[QK ? WN : 1][QK ? CN : 1], qsm[QK ? WN : 1][QK ? CN : 1];  // Q4_K: a block's (sd, sm) so far
#pragma unroll
  for (int t = 0; t < WN; ++t)
#pragma unroll
    for (int u = 0; u < CN; ++u) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};
  if constexpr (QK) {
#pragma unroll
    for (int t = 0; t < WN; ++t)
#pragma unroll
      for (int u = 0; u < CN; ++u) qsd[t][u] = qsm[t][u] = i32x4{0, 0, 0, 0};
  }

  auto store_s = [&](const i32x4& cc, int t, int u, int b) {
    const int col = m0 + 16 * u + r16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = nw + 16 * t + 4 * g + r;
      if (col < M && row < N) S[(static_cast<int64_t>(col) * N + row) * nblk + b] = cc[r];
    }
  };

  auto compute = [&](const WStep& wt, const Step& st, int s) {
    if constexpr (QK) {
      // Q4_K step s = half s % 2 of block s / 2: 64 quant bytes = 32-byte groups j = 2 (s % 2) + {0, 1}, each the
      // low nibbles of sub-block 2j and the high nibbles of sub-block 2j + 1.  After the transpose ta[t][p] (row
      // group g) is dword g of the step's 16-byte piece p (group p / 2, half p % 2), so sub-block i of the step (the
      // block's 4 (s % 2) + i) is {nib(piece 2 (i / 2)), nib(piece 2 (i / 2) + 1)}, low nibbles for even i, high for
      // odd: the slots of Q4_0's block i, whose B operand the activation loads give unchanged.
      unsigned ta[WN][4], xt[CN][XV][4];
#pragma unroll
      for (int t = 0; t < WN; ++t) transpose4(wt.a[t], ta[t]);
#pragma unroll
      for (int u = 0; u < CN; ++u)
#pragma unroll
        for (int v = 0; v < XV; ++v) transpose4(st.x[u][v], xt[u][v]);
      const int hb = s & 1;
      const int b = s >> 1;
      long bi[CN][4];
#pragma unroll
      for (int u = 0; u < CN; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) bi[u][i] = pack2(xt[u][i >> 1][2 * (i & 1)], xt[u][i >> 1][2 * (i & 1) + 1]);
#pragma unroll
      for (int t = 0; t < WN; ++t) {
        const int row_a = 16 * (WN * wr + t) + r16;  // the A operand's row (mins)
        unsigned scw[4];                             // scales of the C rows 4g + r, this half's 4 sub-blocks
#pragma unroll
        for (int r = 0; r < 4; ++r) scw[r] = qslab[((16 * (WN * wr + t) + 4 * g + r) * nblk + b) * 6 + 2 + hb];
        const unsigned mw = qslab[(row_a * nblk + b) * 6 + 4 + hb];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const unsigned p0 = ta[t][2 * (i >> 1)], p1 = ta[t][2 * (i >> 1) + 1];
          const long ai = (i & 1) ? pack2((p0 >> 4) & NIB, (p1 >> 4) & NIB) : pack2(p0 & NIB, p1 & NIB);
          const unsigned mb = ((mw >> (8 * i)) & 0xFFu) * 0x01010101u;  // the row's min in every k slot
#pragma unroll
          for (int u = 0; u < CN; ++u) {
            const i32x4 cc = __builtin_amdgcn_mfma_i32_16x16x32_i8(ai, bi[u][i], i32x4{0, 0, 0, 0}, 0, 0, 0);
            qsm[t][u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(pack2(mb, mb), bi[u][i], qsm[t][u], 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r)  // |cc| < 2^16, scales < 64: a 24-bit multiply-add
              qsd[t][u][r] += __mul24(static_cast<int>((scw[r] >> (8 * i)) & 0xFFu), cc[r]);
          }
        }
        if (hb == 1) {  // the block is complete: y += d * dx * sd - dmin * dx * sm (ggml vec_dot_q4_K_q8_K)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float2 dd =
                *reinterpret_cast<const float2*>(qslab + ((16 * (WN * wr + t) + 4 * g + r) * nblk + b) * 6);
#pragma unroll
            for (int u = 0; u < CN; ++u) {
              acc[t][u][r] = __builtin_fmaf(static_cast<float>(qsd[t][u][r]), dd.x * st.dx[u], acc[t][u][r]);
              acc[t][u][r] = __builtin_fmaf(-static_cast<float>(qsm[t][u][r]), dd.y * st.dx[u], acc[t][u][r]);
            }
          }
#pragma unroll
          for (int u = 0; u < CN; ++u) {
            if constexpr (STORE_S) {
              const int col = m0 + 16 * u + r16;
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int row = nw + 16 * t + 4 * g + r;
                if (col < M && row < N) {
                  int32_t* sp = S + ((static_cast<int64_t>(col) * N + row) * nblk + b) * 2;
                  sp[0] = qsd[t][u][r];
                  sp[1] = qsm[t][u][r];
                }
              }
            }
            qsd[t][u] = qsm[t][u] = i32x4{0, 0, 0, 0};
          }
        }
      }
    } else if constexpr (BLK32) {
      // weights (Q4_0, IQ4_NL): row group g holds block 4s+g; after the transpose ta[t][j] (row group g) is dword g of
      // block 4s+j.  Q8_0: row group g holds half g%2 of block 2s + g/2; after the transpose ta[t][2j + h] (row group
      // g) is dword g of half h of block 2s+j.
      // activations: load v, row group g holds dwords 0..3 of half g%2 of block 2v + g/2; after the transpose
      // xt[u][v][2i + h] (row group g) is dword g of half h of block 2v + i, i.e. xt[u][j / 2][2 (j % 2) + h] holds
      // x[4g .. 4g+3] (h = 0) and x[16 + 4g .. 16 + 4g+3] (h = 1) of the step's block j.
      // d_x: row group g holds block BPS*s + g's (Q8_0: g % 2); dxb[u][j] is block j's in every row group.
      unsigned ta[WN][4], xt[CN][XV][4];
      float dxb[CN][4];
#pragma unroll
      for (int t = 0; t < WN; ++t) transpose4(wt.a[t], ta[t]);
#pragma unroll
      for (int u = 0; u < CN; ++u) {
#pragma unroll
        for (int v = 0; v < XV; ++v) transpose4(st.x[u][v], xt[u][v]);
        bcast_rows(st.dx[u], dxb[u]);
      }
      float dw[WN][4][BPS];  // [t][r][j] = d_w of row 16t + 4g + r, block BPS*s + j
#pragma unroll
      for (int t = 0; t < WN; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float* row = slab + (16 * (WN * wr + t) + 4 * g + r) * ss + BPS * s;
          if constexpr (BPS == 4) {
            const f32x4 v4 = *reinterpret_cast<const f32x4*>(row);
#pragma unroll
            for (int j = 0; j < 4; ++j) dw[t][r][j] = v4[j];
          } else {
            const float2 v2 = *reinterpret_cast<const float2*>(row);
            dw[t][r][0] = v2.x;
            dw[t][r][1] = v2.y;
          }
        }
#pragma unroll
      for (int j = 0; j < BPS; ++j) {
        const int b = BPS * s + j;
        // the step's last blocks past K (wave-uniform): their d_x is zero, so only S needs the branch
        if (STORE_S && b >= nblk) break;
        long bj[CN];
        i32x4 corr[CN];
#pragma unroll
        for (int u = 0; u < CN; ++u) {
          bj[u] = pack2(xt[u][j >> 1][2 * (j & 1)], xt[u][j >> 1][2 * (j & 1) + 1]);
          if constexpr (FMT == FMT_Q4_0)
            corr[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(static_cast<long>(0xF8F8F8F8F8F8F8F8ull), bj[u],
                                                            i32x4{0, 0, 0, 0}, 0, 0, 0);
          else
            corr[u] = i32x4{0, 0, 0, 0};  // signed weights: no offset
        }
#pragma unroll
        for (int t = 0; t < WN; ++t) {
          long aj;
          if constexpr (FMT == FMT_Q4_0)
            aj = pack2(ta[t][j] & NIB, (ta[t][j] >> 4) & NIB);
          else if constexpr (FMT == FMT_IQ4_NL) {
            unsigned lo, hi;
            iq4_nl_lut(ta[t][j], lo, hi);
            aj = pack2(lo, hi);
          }
          else
            aj = pack2(ta[t][2 * j], ta[t][2 * j + 1]);
#pragma unroll
          for (int u = 0; u < CN; ++u) {
            const i32x4 cc = __builtin_amdgcn_mfma_i32_16x16x32_i8(aj, bj[u], corr[u], 0, 0, 0);
            if constexpr (STORE_S) store_s(cc, t, u, b);
#pragma unroll
            for (int r = 0; r < 4; ++r)
              acc[t][u][r] = __builtin_fmaf(static_cast<float>(cc[r]) * dw[t][r][j], dxb[u][j], acc[t][u][r]);
          }
        }
      }
    } else {
      i32x4 corr[CN];
#pragma unroll
      for (int u = 0; u < CN; ++u) {
        corr[u] = i32x4{0, 0, 0, 0};
#pragma unroll
        for (int v = 0; v < 4; ++v)
          corr[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(i32x4{-1, -1, -1, -1},
                                                          reinterpret_cast<const i32x4&>(st.x[u][v]), corr[u], 0, 0, 0);
      }
#pragma unroll
      for (int t = 0; t < WN; ++t) {
        float dw[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) dw[r] = slab[(16 * (WN * wr + t) + 4 * g + r) * ss + s];
        i32x4 aj[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const u32x4 cr = (wt.a[t] >> (2u * v)) & CRUMB;
          aj[v] = reinterpret_cast<const i32x4&>(cr);
        }
#pragma unroll
        for (int u = 0; u < CN; ++u) {
          i32x4 cc = corr[u];
#pragma unroll
          for (int v = 0; v < 4; ++v)
            cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(aj[v], reinterpret_cast<const i32x4&>(st.x[u][v]), cc, 0, 0,
                                                        0);
          if constexpr (STORE_S) store_s(cc, t, u, s);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[t][u][r] = __builtin_fmaf(st.dx[u] * dw[r], static_cast<float>(cc[r]), acc[t][u][r]);
        }
      }
    }
  };

  // Whole groups of DW steps run with no wave-uniform branch in the loop (a branch there makes the compiler's wait
  // counts conservative: a step would wait for the next steps' loads too); the last my % DW steps follow, unrolled.
  // With S (whose stores branch anyway) every step is guarded instead.
  if constexpr (!STORE_S) {
    int i0 = 0;
    for (; i0 + DW <= my; i0 += DW) {
#pragma unroll
      for (int d = 0; d < DW; ++d) {
        const int i = i0 + d;
        compute(wring[d], ring[d % D], step_of(i));
        __builtin_amdgcn_sched_barrier(0);  // slot order kept: the other slots' loads stay in flight meanwhile
        load(ring[d % D], i + D < my ? step_of(i + D) : nsteps);  // past the wave's last step: zeros, no traffic
        load_w(wring[d], i + DW < my ? step_of(i + DW) : nsteps);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int d = 0; d < ((QK && DW <= 2) ? 0 : DW - 1); ++d) {  // the tail (Q4_K: none, its step count is even)
      const int i = i0 + d;  // every weight load of the tail is in flight already
      if (i < my) {
        compute(wring[d], ring[d % D], step_of(i));
        if (d < DW - D && i + D < my) load(ring[d % D], step_of(i + D));
      }
    }
  } else {
    for (int i0 = 0; i0 < my; i0 += DW) {
#pragma unroll
      for (int d = 0; d < DW; ++d) {
        const int i = i0 + d;
        if (i < my) {
          compute(wring[d], ring[d % D], step_of(i));
          load(ring[d % D], i + D < my ? step_of(i + D) : nsteps);
          load_w(wring[d], i + DW < my ? step_of(i + DW) : nsteps);
        }
      }
    }
  }

  if constexpr (WK == 1) {  // each wave holds whole dots: store them
#pragma unroll
    for (int t = 0; t < WN; ++t)
#pragma unroll
      for (int u = 0; u < CN; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = nw + 16 * t + 4 * g + r;
          const int col = m0 + 16 * u + r16;
          if (row < N && col < M) Y[static_cast<int64_t>(col) * N + row] = acc[t][u][r];
        }
  } else {  // partials of the WK waves of a row group, added in wave order
    __syncthreads();  // every wave is done with the slab
    float* red = reinterpret_cast<float*>(lds);
#pragma unroll
    for (int t = 0; t < WN; ++t)
#pragma unroll
      for (int u = 0; u < CN; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[((((wave * WN + t) * CN + u) * 4 + r) << 6) + lane] = acc[t][u][r];
    __syncthreads();
    for (int idx = wk; idx < WN * CN * 4; idx += WK) {
      const int r = idx & 3;
      const int u = (idx >> 2) % CN;
      const int t = (idx >> 2) / CN;
      float sum = 0.f;
      for (int w = 0; w < WK; ++w) sum += red[(((((wr * WK + w) * WN + t) * CN + u) * 4 + r) << 6) + lane];
      const int row = nw + 16 * t + 4 * g + r;
      const int col = m0 + 16 * u + r16;
      if (row < N && col < M) Y[static_cast<int64_t>(col) * N + row] = sum;
    }
  }
}

}  // namespace gemm_impl

namespace {

template <int FMT, int WK, int WR, int WN, int CN, int D, bool STORE_S>
hipError_t launch_s(const GemmCall& c, const GemmPlan& p, hipStream_t stream) {
  const int nblk = c.k / fmt_info(FMT).block;
  // Workgroups go to the 8 XCDs round-robin by linear id (x fastest).  With several column groups the row groups are
  // padded to a multiple of 8, so every column group of a row group runs on one XCD and reads the rows' weights from
  // that XCD's L2 after the first; the padding workgroups exit at once.
  const unsigned gx = (c.n + 16 * WN * WR - 1) / (16 * WN * WR), gy = (c.m + 16 * CN - 1) / (16 * CN);
  const dim3 grid(gy > 1 ? (gx + 7) / 8 * 8 : gx, gy);
  const dim3 block(64 * WK * WR);
  const size_t lds = gemm_lds_bytes(FMT, p, c.k);
  auto kern = gemm_impl::gemm_kernel<FMT, WK, WR, WN, CN, D, STORE_S>;
  static std::atomic<unsigned> lds_limit[kMaxDevices];  // this instantiation's allowed dynamic LDS, per device
  const hipError_t le = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds, lds_limit);
  if (le != hipSuccess) return le;
  const Timing tm = timing_slot(gemv_kind(FMT));
  hipExtLaunchKernelGGL(kern, grid, block, lds, stream, tm.start, tm.stop, 0, c.n, c.m, c.k, nblk, c.sw, c.wq, c.ws,
                        c.xq, c.xd, c.y, c.s);
  return hipGetLastError();
}

template <int FMT, int WK, int WR, int WN, int CN, int D>
hipError_t launch_t(const GemmCall& c, const GemmPlan& p, hipStream_t stream) {
  if (c.s == nullptr) return launch_s<FMT, WK, WR, WN, CN, D, false>(c, p, stream);
  if constexpr (WN == 2 && CN == 4) {
    // storing S as well, two row tiles a wave with four column tiles would hold more than 256 VGPRs (spilled to
    // scratch): one row tile a wave, twice the workgroups; each output's sums run in the same order, so Y is the same
    GemmPlan q = p;
    q.wn = 1;
    return launch_s<FMT, WK, WR, 1, CN, D, true>(c, q, stream);
  } else {
    return launch_s<FMT, WK, WR, WN, CN, D, true>(c, p, stream);
  }
}

// The instantiated plans (gemm_plan in abi.hip picks one): (wk, wr, wn, cn, d).
template <int FMT>
hipError_t launch_fmt(const GemmCall& c, const GemmPlan& p, hipStream_t stream) {
#define KOMP_GEMM_PLAN(WK, WR, WN, CN, D) \
  if (p.wk == WK && p.wr == WR && p.wn == WN && p.cn == CN && p.d == D) return launch_t<FMT, WK, WR, WN, CN, D>(c, p, stream);
  KOMP_GEMM_PLAN(8, 1, 1, 1, 2)
  KOMP_GEMM_PLAN(8, 1, 1, 2, 2)
  KOMP_GEMM_PLAN(8, 1, 1, 3, 2)
  KOMP_GEMM_PLAN(8, 1, 1, 4, 2)
  KOMP_GEMM_PLAN(4, 2, 1, 2, 2)
  KOMP_GEMM_PLAN(4, 2, 1, 3, 2)
  KOMP_GEMM_PLAN(4, 2, 1, 4, 2)
  KOMP_GEMM_PLAN(4, 2, 2, 1, 4)
  KOMP_GEMM_PLAN(2, 4, 1, 2, 2)
  KOMP_GEMM_PLAN(2, 4, 1, 3, 2)
  KOMP_GEMM_PLAN(2, 4, 1, 4, 2)
  KOMP_GEMM_PLAN(1, 8, 1, 1, 2)
  if constexpr (FMT != FMT_Q8_0) {  // Q8_0's two row tiles a wave need more than 256 VGPRs (the plan never asks)
    KOMP_GEMM_PLAN(1, 8, 2, 1, 2)
  }
  KOMP_GEMM_PLAN(1, 8, 1, 2, 2)
  KOMP_GEMM_PLAN(1, 8, 1, 3, 1)
  KOMP_GEMM_PLAN(1, 8, 1, 4, 1)
  if constexpr (FMT != FMT_Q8_0) {  // two row tiles a wave with 2-4 column tiles (208 VGPRs at 4)
    KOMP_GEMM_PLAN(4, 2, 2, 2, 2)
    KOMP_GEMM_PLAN(4, 2, 2, 3, 2)
    KOMP_GEMM_PLAN(4, 2, 2, 4, 2)
    KOMP_GEMM_PLAN(2, 2, 2, 2, 2)
    KOMP_GEMM_PLAN(2, 2, 2, 3, 2)
    KOMP_GEMM_PLAN(2, 2, 2, 4, 2)
  }
#undef KOMP_GEMM_PLAN
  return hipErrorInvalidConfiguration;
}

// Q4_K's plans (gemm_plan in abi.hip): one row tile per wave, since every output tile also holds the block's two
// integer sums.
hipError_t launch_fmt_q4_k(const GemmCall& c, const GemmPlan& p, hipStream_t stream) {
#define KOMP_GEMM_PLAN(WK, WR, WN, CN, D) \
  if (p.wk == WK && p.wr == WR && p.wn == WN && p.cn == CN && p.d == D) return launch_t<FMT_Q4_K, WK, WR, WN, CN, D>(c, p, stream);
  KOMP_GEMM_PLAN(8, 1, 1, 1, 2)
  KOMP_GEMM_PLAN(8, 1, 1, 2, 2)
  KOMP_GEMM_PLAN(4, 2, 1, 2, 2)
  KOMP_GEMM_PLAN(2, 4, 1, 1, 2)
  KOMP_GEMM_PLAN(2, 4, 1, 2, 2)
  KOMP_GEMM_PLAN(1, 8, 1, 1, 2)
  KOMP_GEMM_PLAN(1, 8, 1, 2, 2)
  KOMP_GEMM_PLAN(8, 1, 1, 3, 2)
  KOMP_GEMM_PLAN(8, 1, 1, 4, 2)
  KOMP_GEMM_PLAN(4, 2, 1, 3, 2)
  KOMP_GEMM_PLAN(4, 2, 1, 4, 2)
  KOMP_GEMM_PLAN(2, 4, 1, 3, 2)
  KOMP_GEMM_PLAN(2, 4, 1, 4, 2)
  KOMP_GEMM_PLAN(1, 8, 1, 3, 1)
  KOMP_GEMM_PLAN(1, 8, 1, 4, 1)
#undef KOMP_GEMM_PLAN
  return hipErrorInvalidConfiguration;
}

}  // namespace

size_t gemm_lds_bytes(int fmt, const GemmPlan& p, int k) {
  const int nblk = k / fmt_info(fmt).block;
  const size_t slab = fmt == FMT_Q4_K ? static_cast<size_t>(16) * p.wn * p.wr * nblk * 24  // 6 dwords a block
                                      : (static_cast<size_t>(16) * p.wn * p.wr * gemm_impl::slab_stride(nblk) + 64) * 4;
  const size_t red = p.wk > 1 ? static_cast<size_t>(p.wk) * p.wr * p.wn * p.cn * 4 * 64 * 4 : 0;
  return slab > red ? slab : red;
}

hipError_t launch_gemm(const GemmCall& c, const GemmPlan& p, hipStream_t stream) {
  switch (c.fmt) {
    case FMT_Q4_0: return launch_fmt<FMT_Q4_0>(c, p, stream);
    case FMT_TQ2_0: return launch_fmt<FMT_TQ2_0>(c, p, stream);
    case FMT_Q8_0: return launch_fmt<FMT_Q8_0>(c, p, stream);
    case FMT_IQ4_NL: return launch_fmt<FMT_IQ4_NL>(c, p, stream);
    case FMT_Q4_K: return launch_fmt_q4_k(c, p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace komp
