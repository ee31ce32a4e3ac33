// Shared device helpers for the gfx950 Piper Attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace piper {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;
constexpr int kQueryBlock = 32;  // rows per Q scale (sage/reference.py:6)
constexpr int kKeyBlock = 64;    // rows per K scale and keys per P block (reference.py:16)
constexpr float kLog2e = 1.4426950408889634f;
// Integer accumulators that start from kAccBias read, as FP32 bits, 1.5 * 2^23 + value exactly
// while |value| < 2^22: the FP32 mantissa at [2^23, 2^24) has unit spacing.  Subtracting
// kAccBiasValue (exact) replaces an i32 -> f32 conversion with a plain FP32 subtraction.
constexpr int kAccBias = 0x4B400000;
constexpr float kAccBiasValue = 12582912.0f;  // 1.5 * 2^23

__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}

// Exact widening of 8 packed 16-bit floats (one 16-byte load) to float.
template <bool kBf16>
__device__ __forceinline__ void widen8(const uint4 raw, float (&out)[8]) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (kBf16) {
      out[2 * i] = __uint_as_float(w[i] << 16);
      out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    } else {
      out[2 * i] = half_bits_to_float(w[i] & 0xffffu);
      out[2 * i + 1] = half_bits_to_float(w[i] >> 16);
    }
  }
}

// Round-to-nearest-even narrowing of two floats to a packed pair of the 16-bit output formats
// (a in the low half): one gfx950 v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32 per pair.  Finite values
// round exactly as torch's casts do; a NaN becomes a NaN of the format.
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_half2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((float2_t){a, b}, half2_t));
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((float2_t){a, b}, bf16x2_t));
}

// Max / sum of a value over the two 32-lane halves of a wave (lane l and l ^ 32).
// (The final max is one v_max_f32 written as assembly: fmaxf would first quiet each swapped
// operand with a v_max_f32 of itself, since the compiler cannot tell they hold no signalling NaN.)
__device__ __forceinline__ float cross_half_max(float v) {
  const uint32_t u = __float_as_uint(v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  float m;
  asm("v_max_f32 %0, %1, %2" : "=v"(m) : "v"(__uint_as_float(r[0])), "v"(__uint_as_float(r[1])));
  return m;
}

__device__ __forceinline__ float cross_half_sum(float v) {
  const uint32_t u = __float_as_uint(v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2).  Remap the
// hardware block id so that consecutive logical ids -- the query blocks of one head, which
// stream the same K/V tiles -- run on the same XCD.
// The same for `xccs` XCCs (block b runs on XCC b % xccs); xcc_remap(b, n, 8) == xcd_remap(b, n).
__device__ __forceinline__ int xcc_remap(int block, int blocks, int xccs) {
  const int xcc = block % xccs;
  const int local = block / xccs;
  const int base = blocks / xccs;
  const int rem = blocks - base * xccs;
  return xcc * base + (xcc < rem ? xcc : rem) + local;
}

__device__ __forceinline__ int xcd_remap(int block, int blocks) {
  const int xcd = block & 7;
  const int local = block >> 3;
  const int base = blocks >> 3;
  const int rem = blocks & 7;
  return xcd * base + (xcd < rem ? xcd : rem) + local;
}

}  // namespace piper
