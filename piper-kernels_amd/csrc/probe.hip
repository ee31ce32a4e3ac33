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
#include "common.h"
#include "kernels.h"

namespace piper {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

template <int kKind>
__global__ void __launch_bounds__(kProbeThreads, 1) mfma_probe_kernel(uint32_t* sink, int iterations) {
  uint32_t total = 0;
  if constexpr (kKind == 0) {
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
  if (kind == 0)
    hipLaunchKernelGGL(mfma_probe_kernel<0>, grid, block, 0, stream, sink, iterations);
  else
    hipLaunchKernelGGL(mfma_probe_kernel<1>, grid, block, 0, stream, sink, iterations);
  return hipGetLastError();
}

}  // namespace piper
