// Roofline calibration: dense MFMAs issued back to back on every SIMD, for measuring the
// sustained matrix-core rate of this GPU at its running clock (the attention kernels are
// priced against it next to the published peak).
//
// Each wave keeps four independent accumulator chains so the MFMA pipe never waits on a
// result, and runs `iterations` rounds of four MFMAs on constant operands: every A and B
// element is 1 (INT8 1, or FP8 E4M3 1.0 = 0x38), so after the loop every accumulator element
// is exactly iterations * K (K = 32 for the INT8 instruction, 64 for the FP8 one).  Each lane
// then stores the 32-bit sum of its 64 accumulator registers to sink[global thread index]:
// iterations * 2048 (INT8, modulo 2^32) or iterations * 4096 (FP8, as FP32 bits), a value a
// caller can check so that a fast time cannot come from work the compiler removed.
//
// Two more kinds measure how MFMA execution and VALU issue share a SIMD.  Kind 2 runs 64
// FP32 FMAs per round (16 independent chains f = f * 1 + 1, every result an exact integer)
// and no MFMA; kind 3 runs the INT8 kind's four MFMAs per round with 16 of those FMAs issued
// after each one (scheduling barriers keep the interleave).  Launched like the attention
// kernel (one 8-wave workgroup per compute unit, two waves per SIMD), the three times give
// t(MFMA), t(VALU) and t(both): t(both) = max of the two if the units overlap, their sum if
// they serialise.  Kind 2 stores the FP32 bits of 64 * iterations; kind 3 stores
// iterations * 2048 + 64 * iterations modulo 2^32.  Kinds 4 and 5 time two other instruction
// classes the same way (64 per round on 16 chains): v_max3_f32 (f = max(f, 1, 0), which stays 1;
// stores the bits of 16.0) and v_exp_f32 (f = 2^-f from 0, which converges to the root of
// x = 2^-x, 0.641186; stores the bits of the 16-chain sum).  Kind 6 is kind 2 with a wave-wide
// ds_read_b128 of zeros after every 8 FMAs (the FMA result word, 64 * iterations, is unchanged):
// t(6) - t(2) is what 8 * iterations LDS reads add to a VALU-bound wave.
//
// Kinds 7 and 8 check conversions rather than time them: on entry, the 512 words of each
// workgroup's part of `sink` hold FP32 values; thread t packs values 4 (t % 128) .. + 3 with the
// attention kernels' own probability-code packers (kind 7: Piper Attention's UINT8 codes,
// stored as u - 128 per byte; kind 8: SageAttention2++'s FP8 E4M3 codes) and stores the word
// over word t.  `iterations` is not used.
#include "common.h"
#include "kernels.h"
#include "quant.h"

namespace piper {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

template <int kKind>
__global__ void __launch_bounds__(kProbeThreads, 1) mfma_probe_kernel(uint32_t* sink, int iterations) {
  uint32_t total = 0;
  if constexpr (kKind == 7 || kKind == 8) {
    const float* values = reinterpret_cast<const float*>(sink) + static_cast<long>(blockIdx.x) * kProbeThreads;
    const int i = 4 * (threadIdx.x % (kProbeThreads / 4));
    const float a = values[i], b = values[i + 1], c = values[i + 2], d = values[i + 3];
    __syncthreads();  // every read of this workgroup's words precedes every store over them
    total = kKind == 7 ? pack_codes(a, b, c, d) : pack_fp8(a, b, c, d);
  } else if constexpr (kKind == 0) {
    v4i a = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    asm volatile("" : "+v"(a));  // opaque: the products cannot be folded
    v16i acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = v16i{};
    for (int it = 0; it < iterations; ++it) {
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, a, acc[c], 0, 0, 0);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) total += static_cast<uint32_t>(acc[c][r]);
  } else if constexpr (kKind == 4 || kKind == 5) {
    // instruction-class issue rates: 64 v_max3_f32 (kind 4) or v_exp_f32 (kind 5) per round
    float one = 1.0f, zero = 0.0f;
    asm volatile("" : "+v"(one), "+v"(zero));
    float f[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) f[i] = kKind == 4 ? 1.0f : 0.0f;
    for (int it = 0; it < iterations; ++it) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          if constexpr (kKind == 4) f[i] = fmaxf(fmaxf(f[i], one), zero);  // stays 1
          else f[i] = __builtin_amdgcn_exp2f(-f[i]);  // converges to the root of x = 2^-x
        }
      }
    }
    float fsum = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) fsum += f[i];
    total = __builtin_bit_cast(uint32_t, fsum);
  } else if constexpr (kKind == 6) {
    // kind 2's FMAs with one wave-wide ds_read_b128 after every 8 of them (8 per round, the
    // attention kernel's ratio of LDS reads to VALU work); the LDS words are zero
    __shared__ __attribute__((aligned(16))) float lds[4 * kProbeThreads];
#pragma unroll
    for (int i = 0; i < 4; ++i) lds[4 * threadIdx.x + i] = 0.0f;
    __syncthreads();
    const uint32_t address = static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) float*)(lds + 4 * (threadIdx.x & 63))));
    float one = 1.0f, addend = 1.0f;
    asm volatile("" : "+v"(one), "+v"(addend));
    float f[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) f[i] = 0.0f;
    v4i word = {0, 0, 0, 0};
    for (int it = 0; it < iterations; ++it) {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        // explicit reads (the compiler would hoist or merge loop-invariant loads); their words
        // are waited for once after the loop
        asm volatile("ds_read_b128 %0, %1" : "=v"(word) : "v"(address) : "memory");
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 8; ++i) f[(8 * c + i) & 15] = fmaf(f[(8 * c + i) & 15], one, addend);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(word) : : "memory");
    float fsum = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) fsum += f[i];
    total = __builtin_bit_cast(uint32_t, fsum) + static_cast<uint32_t>(word[0] | word[1] | word[2] | word[3]);
  } else if constexpr (kKind == 2 || kKind == 3) {
    v4i a = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    asm volatile("" : "+v"(a));
    float one = 1.0f, addend = 1.0f;  // two registers: an FMA reading one VGPR twice issues slower
    asm volatile("" : "+v"(one), "+v"(addend));  // opaque: the FMAs cannot be folded
    float f[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) f[i] = 0.0f;
    v16i acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = v16i{};
    for (int it = 0; it < iterations; ++it) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if constexpr (kKind == 3) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, a, acc[c], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 16; ++i) f[i] = fmaf(f[i], one, addend);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    float fsum = 0.0f;  // 16 chains of 4 * iterations: exact while 64 * iterations < 2^24
#pragma unroll
    for (int i = 0; i < 16; ++i) fsum += f[i];
    if constexpr (kKind == 2) {
      total = __builtin_bit_cast(uint32_t, fsum);
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) total += static_cast<uint32_t>(acc[c][r]);
      total += static_cast<uint32_t>(fsum);
    }
  } else {
    v8i a = {0x38383838, 0x38383838, 0x38383838, 0x38383838, 0x38383838, 0x38383838, 0x38383838, 0x38383838};
    asm volatile("" : "+v"(a));
    v16f acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = v16f{};
    for (int it = 0; it < iterations; ++it) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        acc[c] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, a, acc[c], 0, 0, 0, 0, 0, 0);
    }
    float sum = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) sum += acc[c][r];
    total = __builtin_bit_cast(uint32_t, sum);
  }
  sink[static_cast<long>(blockIdx.x) * kProbeThreads + threadIdx.x] = total;
}

hipError_t launch_mfma_probe(int kind, int workgroups, int iterations, uint32_t* sink, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(workgroups));
  const dim3 block(kProbeThreads);
  switch (kind) {
    case 0: hipLaunchKernelGGL(mfma_probe_kernel<0>, grid, block, 0, stream, sink, iterations); break;
    case 1: hipLaunchKernelGGL(mfma_probe_kernel<1>, grid, block, 0, stream, sink, iterations); break;
    case 2: hipLaunchKernelGGL(mfma_probe_kernel<2>, grid, block, 0, stream, sink, iterations); break;
    case 3: hipLaunchKernelGGL(mfma_probe_kernel<3>, grid, block, 0, stream, sink, iterations); break;
    case 4: hipLaunchKernelGGL(mfma_probe_kernel<4>, grid, block, 0, stream, sink, iterations); break;
    case 5: hipLaunchKernelGGL(mfma_probe_kernel<5>, grid, block, 0, stream, sink, iterations); break;
    case 6: hipLaunchKernelGGL(mfma_probe_kernel<6>, grid, block, 0, stream, sink, iterations); break;
    case 7: hipLaunchKernelGGL(mfma_probe_kernel<7>, grid, block, 0, stream, sink, iterations); break;
    default: hipLaunchKernelGGL(mfma_probe_kernel<8>, grid, block, 0, stream, sink, iterations); break;
  }
  return hipGetLastError();
}

}  // namespace piper
