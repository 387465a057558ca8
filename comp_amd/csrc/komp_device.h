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
  if (g >= 32) v += __shfl_xor(v, 16, 64);
  if (g >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

// Exact roundf (halfway away from zero) for every f32 (patch:84-90).
__device__ __forceinline__ float round_half_away(float x) {
  float a = fabsf(x);
  float f = floorf(a);
  float r = (a - f >= 0.5f) ? f + 1.0f : f;
  return copysignf(r, x);
}

}  // namespace komp
