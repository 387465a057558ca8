// Device helpers shared by the gfx950 kernels of the COMP decode path.
//
// Format math restated from the reference's Triton helpers (patches/0001-language-extra-kurn.patch:33-131) as
// CDNA4 integer/float code: packed-word dot products map to v_dot4c_i32_i8, cross-lane reductions to DPP.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace komp {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum Mode { MODE_BYTES = 0, MODE_DP4A_EMU = 1, MODE_DP4A = 2 };

// Bytes mode's unpacked integers: two 16-bit values a register (v_pk_* arithmetic).
typedef short s16x2 __attribute__((ext_vector_type(2)));

// A register's two 16-bit halves.  Takes the word by value: a bit cast applied to a vector element itself reads
// element 0 whatever the index.
__device__ __forceinline__ s16x2 halves(unsigned v) { return __builtin_bit_cast(s16x2, v); }

// The signed bytes of q as 16-bit integers: bytes 0 and 2 (even) or 1 and 3 (odd) in the low and high half.
__device__ __forceinline__ unsigned sext_even(unsigned q) {
  return __builtin_bit_cast(unsigned, halves(q << 8) >> 8);
}
__device__ __forceinline__ unsigned sext_odd(unsigned q) {
  return __builtin_bit_cast(unsigned, halves(q) >> 8);
}

// f16 bit pattern -> f32, exact for every pattern (patch:33-36).
__device__ __forceinline__ float f16_bits_to_f32(int16_t bits) {
  return __half2float(__ushort_as_half(static_cast<unsigned short>(bits)));
}

// dp4a.s32.s32 from shifts and multiplies: c + sum of the four signed-byte products (patch:66-70).
__device__ __forceinline__ int dp4a_emu(int a, int b, int c) {
  int p = ((a << 24) >> 24) * ((b << 24) >> 24) + ((a << 16) >> 24) * ((b << 16) >> 24);
  return c + p + ((a << 8) >> 24) * ((b << 8) >> 24) + (a >> 24) * (b >> 24);
}

// dp4a on the hardware: v_dot4c_i32_i8 (no clamp, so int32 wraparound like dp4a.s32.s32).
template <int MODE>
__device__ __forceinline__ int dot4(unsigned a, unsigned b, int c) {
  if constexpr (MODE == MODE_DP4A) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
  } else {
    return dp4a_emu(static_cast<int>(a), static_cast<int>(b), c);
  }
}

// IQ4_NL: a quant word q (4 bytes of Q4_0's nibble order) -> the int8 values of ggml's kvalues_iq4nl table that its
// 8 nibbles index: lo byte j = table[q byte j & 15], hi byte j = table[q byte j >> 4].  Per 4 nibbles, two
// v_perm_b32 look the low 3 index bits up in the table's low and high eight entries, and a third v_perm_b32 keeps
// one of the two per byte by bit 3 of the index (its selector byte j is j, or j + 4 to take the high lookup).
// 13 VALU ops per 8 values.
__device__ __forceinline__ void iq4_nl_lut(unsigned q, unsigned& lo, unsigned& hi) {
  constexpr unsigned T0 = 0xBFAD9881u;  // -127, -104, -83, -65 (bytes 0..3)
  constexpr unsigned T1 = 0xF6EADDCFu;  // -49, -35, -22, -10
  constexpr unsigned T2 = 0x26190D01u;  // 1, 13, 25, 38
  constexpr unsigned T3 = 0x71594535u;  // 53, 69, 89, 113
  // The identity selector lives in a VGPR (a plain v_mov the compiler hoists), so each merge selector is one
  // v_and_or_b32 (a VOP3 encoding holds one literal or SGPR constant, not the two the expression has).
  unsigned ident;
  asm("v_mov_b32 %0, 0x3020100" : "=v"(ident));
  const unsigned r = q >> 4;  // byte j: the high nibble of q byte j in its low 4 bits
  const unsigned sl = q & 0x07070707u;
  const unsigned sh = r & 0x07070707u;
  const unsigned l0 = __builtin_amdgcn_perm(T1, T0, sl), l1 = __builtin_amdgcn_perm(T3, T2, sl);
  const unsigned h0 = __builtin_amdgcn_perm(T1, T0, sh), h1 = __builtin_amdgcn_perm(T3, T2, sh);
  lo = __builtin_amdgcn_perm(l1, l0, ((q >> 1) & 0x04040404u) | ident);
  hi = __builtin_amdgcn_perm(h1, h0, ((r >> 1) & 0x04040404u) | ident);
}

// Signed byte e of a 32-bit word.
__device__ __forceinline__ int sbyte(unsigned w, int e) { return static_cast<int>(w << (24 - 8 * e)) >> 24; }

// ---- DPP cross-lane moves (wave64; a DPP "row" is 16 lanes) ----------------------------------------------------------
// quad_perm [1,0,3,2] = lane ^ 1, [2,3,0,1] = lane ^ 2, row_half_mirror = lane i <- 7-i within 8, row_mirror =
// lane i <- 15-i within 16.  After xor1, xor2, half_mirror and mirror steps every lane of a row holds the row's total.
#define KOMP_DPP_XOR1 0xB1
#define KOMP_DPP_XOR2 0x4E
#define KOMP_DPP_HALF_MIRROR 0x141
#define KOMP_DPP_MIRROR 0x140

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of G lanes (G a power of two, 1..64); every lane of a group receives the group's sum.
template <typename T>
__device__ __forceinline__ T group_sum(T v, int g) {
  if constexpr (sizeof(T) == 4 && __is_same(T, float)) {
    if (g >= 2) v += dpp_f<KOMP_DPP_XOR1>(v);
    if (g >= 4) v += dpp_f<KOMP_DPP_XOR2>(v);
    if (g >= 8) v += dpp_f<KOMP_DPP_HALF_MIRROR>(v);
    if (g >= 16) v += dpp_f<KOMP_DPP_MIRROR>(v);
  } else {
    if (g >= 2) v += dpp_i<KOMP_DPP_XOR1>(v);
    if (g >= 4) v += dpp_i<KOMP_DPP_XOR2>(v);
    if (g >= 8) v += dpp_i<KOMP_DPP_HALF_MIRROR>(v);
    if (g >= 16) v += dpp_i<KOMP_DPP_MIRROR>(v);
  }
  // across rows: v_permlane16_swap(v, v) leaves rows (0 0 2 2) in its first result and (1 1 3 3) in its second,
  // v_permlane32_swap(v, v) rows (0 1 0 1) and (2 3 2 3), so one swap and one add give each lane its own value plus
  // its partner row's (lane ^ 16, lane ^ 32: the same sums, added in the same order up to commutation, as an exchange
  // through LDS, without the LDS round trip)
  if (g >= 32) {
    const auto p = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                    false, false);
    v = __builtin_bit_cast(T, static_cast<unsigned>(p[0])) + __builtin_bit_cast(T, static_cast<unsigned>(p[1]));
  }
  if (g >= 64) {
    const auto p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                    false, false);
    v = __builtin_bit_cast(T, static_cast<unsigned>(p[0])) + __builtin_bit_cast(T, static_cast<unsigned>(p[1]));
  }
  return v;
}

// Exact roundf (halfway away from zero) for every f32 (patch:84-90).
__device__ __forceinline__ float round_half_away(float x) {
  float a = fabsf(x);
  float f = floorf(a);
  float r = (a - f >= 0.5f) ? f + 1.0f : f;
  return copysignf(r, x);
}

// ---- activation quantizers (patch:104-131), shared by the quantizer kernels and the fused GEMV staging -------------

// ggml q8_0 on one block of 32 values held by 8 aligned lanes (4 consecutive values each).  Returns this lane's 4
// quantized values packed in a dword (value e in byte e); d_store receives f32(f16(d)) (the stored scale, RTNE), and
// qsum the block's sum of q (every lane of the group receives it).
__device__ __forceinline__ unsigned q8_0_group8(f32x4 v, float& d_store, int& qsum) {
  // |x| >= 0, whose bit patterns order like the floats, so the 8-lane max runs on integers (single DPP instructions)
  int ab = __float_as_int(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
  ab = max(ab, dpp_i<KOMP_DPP_XOR1>(ab));
  ab = max(ab, dpp_i<KOMP_DPP_XOR2>(ab));
  ab = max(ab, dpp_i<KOMP_DPP_HALF_MIRROR>(ab));
  const float d = __int_as_float(ab) / 127.0f;  // correctly rounded (no fast-math)
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  unsigned packed = 0;
  int sum = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int qv = static_cast<int>(round_half_away(v[e] * id));  // q from the unrounded d
    sum += qv;
    packed |= (static_cast<unsigned>(qv) & 0xFFu) << (8 * e);
  }
  sum += dpp_i<KOMP_DPP_XOR1>(sum);
  sum += dpp_i<KOMP_DPP_XOR2>(sum);
  sum += dpp_i<KOMP_DPP_HALF_MIRROR>(sum);
  qsum = sum;
  d_store = __half2float(__float2half_rn(d));
  return packed;
}

// Sum / max / min over each aligned 16-lane DPP row; every lane of the row receives the row's result.
__device__ __forceinline__ int row16_min_i(int v) {
  v = min(v, dpp_i<KOMP_DPP_XOR1>(v));
  v = min(v, dpp_i<KOMP_DPP_XOR2>(v));
  v = min(v, dpp_i<KOMP_DPP_HALF_MIRROR>(v));
  return min(v, dpp_i<KOMP_DPP_MIRROR>(v));
}

__device__ __forceinline__ int row16_max_i(int v) {
  v = max(v, dpp_i<KOMP_DPP_XOR1>(v));
  v = max(v, dpp_i<KOMP_DPP_XOR2>(v));
  v = max(v, dpp_i<KOMP_DPP_HALF_MIRROR>(v));
  return max(v, dpp_i<KOMP_DPP_MIRROR>(v));
}

// The max of `hi` and the min of `lo` over each aligned 16-lane row, the two reductions interleaved step by step so
// that neither waits on its own previous DPP result.
__device__ __forceinline__ void row16_max_min_i(int& hi, int& lo) {
  hi = max(hi, dpp_i<KOMP_DPP_XOR1>(hi));
  lo = min(lo, dpp_i<KOMP_DPP_XOR1>(lo));
  hi = max(hi, dpp_i<KOMP_DPP_XOR2>(hi));
  lo = min(lo, dpp_i<KOMP_DPP_XOR2>(lo));
  hi = max(hi, dpp_i<KOMP_DPP_HALF_MIRROR>(hi));
  lo = min(lo, dpp_i<KOMP_DPP_HALF_MIRROR>(lo));
  hi = max(hi, dpp_i<KOMP_DPP_MIRROR>(hi));
  lo = min(lo, dpp_i<KOMP_DPP_MIRROR>(lo));
}

// f32 bits -> int32 whose signed order is the float order (-0 just below +0); the map is its own inverse.  Row
// reductions of floats run on these keys because integer max/min fold into single DPP instructions, while float ones
// need NaN-quieting moves around every DPP step.
__device__ __forceinline__ int f32_order_key(int bits) { return bits ^ ((bits >> 31) & 0x7FFFFFFF); }

// ggml q8_K on one block of 256 values held by an aligned 16-lane row (lane r of the row holds values 16r..16r+15 in
// v[0..3]); the whole row must be active and the wave's control flow uniform.  Writes the lane's 16 q into qout (value
// 4t+e in byte e of qout[t]) and returns the lane's sum of its 16 q, which is exactly bsum r of the block; d_out
// receives d (0 for an all-zero block) and qsum the block's sum of q.
//
// mx, the x of largest |x| with the first index winning ties (patch:121-125), is the block's signed maximum hi or its
// signed minimum lo: whichever has the larger magnitude.  Only when both +|mx| and -|mx| occur does the index order
// decide; that rare case takes a wave-uniform branch that finds the sign of the first occurrence.
//
// q = round_half_even(iscale * x) (patch:128, 94-101) without the clamp to 127: |x| <= |mx| and iscale = -127 / mx
// correctly rounded, so |iscale * x| <= 127 (1 + 2^-24)^2 < 127.5 and the rounded value never exceeds 127 in
// magnitude.  Adding 1.5 * 2^23 to the rounded product rounds it to an integer in the default round-to-nearest-even
// mode, exactly as round_half_even does, and the low byte of the sum's bits is that integer's two's-complement byte.
__device__ __forceinline__ int q8_K_row16(const f32x4 (&v)[4], int r, u32x4& qout, float& d_out, int& qsum) {
#pragma clang fp contract(off)
  // three-operand trees (v_max3 / v_min3, depth 3 rather than a chain of 8), which take the loaded values as they are
  auto at = [&](int i) { return v[i >> 2][i & 3]; };
  float hp[5], lp[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    hp[i] = fmaxf(fmaxf(at(3 * i), at(3 * i + 1)), at(3 * i + 2));
    lp[i] = fminf(fminf(at(3 * i), at(3 * i + 1)), at(3 * i + 2));
  }
  float hi = fmaxf(fmaxf(fmaxf(hp[0], hp[1]), hp[2]), fmaxf(fmaxf(hp[3], hp[4]), at(15)));
  float lo = fminf(fminf(fminf(lp[0], lp[1]), lp[2]), fminf(fminf(lp[3], lp[4]), at(15)));
  int hk = f32_order_key(__float_as_int(hi)), lk = f32_order_key(__float_as_int(lo));
  row16_max_min_i(hk, lk);
  hi = __int_as_float(f32_order_key(hk));
  lo = __int_as_float(f32_order_key(lk));
  float mx = hi >= -lo ? hi : lo;
  const bool tie = hi == -lo && hi != 0.0f;
  if (__builtin_expect(__ballot(tie) != 0, 0)) {
    // sign of this lane's first value with |x| == hi (reverse scan), then the lowest lane of the row that has one
    int neg = 2;
#pragma unroll
    for (int t = 3; t >= 0; --t)
#pragma unroll
      for (int e = 3; e >= 0; --e) neg = fabsf(v[t][e]) == hi ? (v[t][e] < 0.0f ? 1 : 0) : neg;
    const int first = row16_min_i(neg < 2 ? 2 * r + neg : 64);
    if (tie) mx = (first & 1) ? lo : hi;
  }
  const bool nz = mx != 0.0f;
  const float iscale = -127.0f / (nz ? mx : 1.0f);  // an all-zero block gives q = 0 through the same arithmetic
  // 1.5 * 2^23 and the all-ones bytes in SGPRs: the 16 adds and 4 dots are then 4-byte instructions rather than
  // 8-byte ones carrying a literal (the fused GEMVs run this code from a cold instruction cache)
  float kRound;
  int ones;
  asm("s_mov_b32 %0, 0x4b400000" : "=s"(kRound));  // 12582912.0f
  asm("s_mov_b32 %0, 0x01010101" : "=s"(ones));
  int s16 = 0;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    unsigned b[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) b[e] = __float_as_uint(iscale * v[t][e] + kRound);
    const unsigned p01 = __builtin_amdgcn_perm(b[1], b[0], 0x0c0c0400u);  // bytes {b0, b1, 0, 0}
    const unsigned p23 = __builtin_amdgcn_perm(b[3], b[2], 0x0c0c0400u);
    qout[t] = p01 | (p23 << 16);
    s16 = __builtin_amdgcn_sdot4(static_cast<int>(qout[t]), ones, s16, false);
  }
  qsum = group_sum(s16, 16);
  d_out = nz ? 1.0f / iscale : 0.0f;
  return s16;
}

}  // namespace komp
