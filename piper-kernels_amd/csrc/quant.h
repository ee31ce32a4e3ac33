// Quantisation arithmetic shared by the prep kernels and the attention prologue (which can
// quantise its own query block): one definition, so every path produces the same codes.  The
// probability-code packers of the two attention kernels live here too, so that the library's
// probe checks the very functions the kernels run.
//
// Reference: sage/reference.py:61-77 (per-group scale amax / 127 + 1e-7, round half to even,
// clamp to +-127) and reference.py:22-32 (the same rule per V row).
#pragma once

#include "common.h"

namespace piper {

template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {  // v of the lane the DPP control names (all lanes valid)
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, false));
}

__device__ __forceinline__ float lane_value(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Max over the 64 lanes of a wave, in every lane: DPP within each row of 16 lanes (quad
// swaps, then rotations by 4 and 8), then the four row maxima read as scalars.  fmaxf drops a
// NaN operand, so the result is the max of the non-NaN values whatever the order.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp<0x124>(v));  // row_ror:4
  v = fmaxf(v, dpp<0x128>(v));  // row_ror:8
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

template <int kLanes>
__device__ __forceinline__ float group_max(float v) {  // max over aligned groups of kLanes lanes
#pragma unroll
  for (int m = kLanes / 2; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

__device__ __forceinline__ float scale_from_amax(float amax) {
  // amax / 127 + 1e-7: correctly rounded FP32 division, then an FP32 add (no contraction).
  const float q = amax / 127.0f;
  return __fadd_rn(q, 1e-7f);
}

// A quantisation scale with its correctly rounded reciprocal, shared by all elements it divides.
struct Divisor {
  float s;  // the scale, or 0 for an infinite scale (see quotient)
  float y;  // RN(1 / scale), IEEE division
  Divisor() = default;
  __device__ explicit Divisor(float scale) : s(__builtin_isinf(scale) ? 0.0f : scale), y(1.0f / scale) {}
  // RN(x / scale) without a per-element division (Markstein: with y = RN(1/s) and a faithful
  // q0 = RN(x y), the remainder x - s q0 is exact in one FMA and RN(q0 + r y) = RN(x / s) for
  // normal x; subnormal x only moves a quotient far below 1/2 by an ulp, so the rounded code is
  // unchanged).  For an infinite scale (non-finite input) y = 0 and s = 0 give x / inf = +-0
  // for finite x and NaN for infinite x, as the division does.
  __device__ float quotient(float x) const {
    const float q0 = __fmul_rn(x, y);
    const float r = fmaf(-s, q0, x);
    return fmaf(r, y, q0);
  }
};

// The code of x as the low byte of a word: the bits of RN(x / scale) + 1.5 * 2^23.  That FP32
// add rounds the quotient to an integer, half to even (its ulp is 1 and 1.5 * 2^23 is even),
// and leaves the integer in two's complement in the low mantissa bits.  The reference's clamp
// to +-127 never acts on a finite input: |x| <= amax and scale >= RN(amax / 127), so
// |x / scale| <= 127 (1 + 2^-23) and the rounded quotient is at most 127 in magnitude.
// (Non-finite inputs: a NaN quotient gives code 0.)
__device__ __forceinline__ uint32_t code_word(float x, const Divisor& d) {
  return __builtin_bit_cast(uint32_t, __fadd_rn(d.quotient(x), kAccBiasValue));
}

__device__ __forceinline__ int code_of(float x, const Divisor& d) {
  return static_cast<int8_t>(code_word(x, d) & 0xffu);
}

// Low bytes of four words, a in byte 0 (v_perm_b32 selectors: 0-3 pick bytes of the second
// operand, 4-7 bytes of the first, 0x0c a zero byte).
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return __builtin_amdgcn_perm(b, a, 0x0c0c0400u) | __builtin_amdgcn_perm(d, c, 0x04000c0cu);
}

// Piper Attention's UINT8 probability codes, e0 in byte 0, as u - 128 in signed INT8 (the PV
// MFMA's operand).  v_cvt_pk_u8_f32 rounds half to even and saturates to [0, 255]: the
// reference's round().clamp(0, 255) (reference.py:104-107) in one instruction per code.
__device__ __forceinline__ uint32_t pack_codes(float e0, float e1, float e2, float e3) {
  uint32_t w = __builtin_amdgcn_cvt_pk_u8_f32(e0, 0, 0u);
  w = __builtin_amdgcn_cvt_pk_u8_f32(e1, 1, w);
  w = __builtin_amdgcn_cvt_pk_u8_f32(e2, 2, w);
  w = __builtin_amdgcn_cvt_pk_u8_f32(e3, 3, w);
  return w ^ 0x80808080u;  // u - 128 as signed INT8
}

// The byte selector of pack_scaled_codes (v_perm_b32: byte 0 of the second operand, byte 0 of
// the first, two zero bytes), held in a VGPR: a VOP3 instruction takes no literal operand, and
// one that reads an SGPR issues at half rate.
__device__ __forceinline__ uint32_t code_selector() {
  uint32_t sel = 0x0c0c0400u;
  asm volatile("" : "+v"(sel));
  return sel;
}

// Piper Attention's UINT8 probability codes of e_i = E_i * c (the same rule as pack_codes, for
// products in [0, 255.5)), e0 in byte 0, as u - 128 in signed INT8.  fma(E, c, 1.5 * 2^23 - 128)
// rounds the exact product once, into the binade [2^23, 2^24) whose spacing is 1: to the nearest
// integer, half to even (1.5 * 2^23 - 128 is even), and the low byte of its bits is u - 128 in
// two's complement.  The multiplier c rides in the FMA, so the caller needs no per-code scaling.
__device__ __forceinline__ uint32_t pack_scaled_codes(float e0, float e1, float e2, float e3, float c, uint32_t sel) {
  constexpr float kMagic = 12582784.0f;  // 1.5 * 2^23 - 128
  const uint32_t a = __builtin_bit_cast(uint32_t, fmaf(e0, c, kMagic));
  const uint32_t b = __builtin_bit_cast(uint32_t, fmaf(e1, c, kMagic));
  const uint32_t d2 = __builtin_bit_cast(uint32_t, fmaf(e2, c, kMagic));
  const uint32_t d3 = __builtin_bit_cast(uint32_t, fmaf(e3, c, kMagic));
  const uint32_t lo = __builtin_amdgcn_perm(b, a, sel);    // [u0, u1, 0, 0] - 128
  const uint32_t hi = __builtin_amdgcn_perm(d3, d2, sel);  // [u2, u3, 0, 0] - 128
  return (hi << 16) | lo;
}

// SageAttention2++'s FP8 E4M3 probability codes, a in byte 0 (round to nearest even, like
// torch's float8_e4m3fn cast).  Both 16-bit halves are written, so the word starts from an
// undefined register (no clearing move).
__device__ __forceinline__ uint32_t pack_fp8(float a, float b, float c, float d) {
  int undef;
  asm volatile("" : "=v"(undef));
  uint32_t w = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, undef, false));
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, static_cast<int>(w), true));
}

}  // namespace piper
