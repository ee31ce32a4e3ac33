// libpiper_probe.so: measurement kernels beside the Piper Attention backend (C ABI in
// include/piper_probe.h).  Nothing here is part of the operator.
//
// * piper_mfma_probe: dense MFMAs issued back to back on every SIMD (the sustained matrix-core
//   rate of this GPU at its running clock), and two conversion checks that run the attention
//   kernels' own probability-code packers (quant.h) on caller values.
// * piper_issue_probe: per-wave roles on shared SIMDs, each a fixed inline-assembly loop timed by
//   s_memtime, to measure how MFMA execution, VALU issue and LDS reads of different waves share
//   a SIMD (the issue bound of the attention kernels).
#include <cstdarg>
#include <cstdio>

#include "common.h"
#include "piper_probe.h"
#include "quant.h"

namespace piper {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kProbeThreads = PIPER_MFMA_PROBE_THREADS;  // 8 waves: two per SIMD

// Kinds I8 and F8: four accumulator chains per wave, `iterations` rounds of four MFMAs on
// all-ones operands; each lane stores the 32-bit sum of its 64 accumulator registers.
// Kinds P_CODES_U8 / P_CODES_FP8: thread t packs four of its workgroup's values with the
// kernels' packer and stores the word over word t.  P_CODES_U8_SCALED: thread t packs values
// 4 (t % 64) .. + 3 times the multiplier in word 256 + 4 (t % 64).
template <int kKind>
__global__ void __launch_bounds__(kProbeThreads, 1) mfma_probe_kernel(uint32_t* sink, int iterations) {
  uint32_t total = 0;
  if constexpr (kKind == PIPER_MFMA_PROBE_P_CODES_U8_SCALED) {
    const float* values = reinterpret_cast<const float*>(sink) + static_cast<long>(blockIdx.x) * kProbeThreads;
    const int g = threadIdx.x % 64;
    const float a = values[4 * g], b = values[4 * g + 1], c = values[4 * g + 2], d = values[4 * g + 3];
    const float m = values[256 + 4 * g];
    __syncthreads();  // every read of this workgroup's words precedes every store over them
    total = pack_scaled_codes(a, b, c, d, m, code_selector());
  } else if constexpr (kKind == PIPER_MFMA_PROBE_P_CODES_U8 || kKind == PIPER_MFMA_PROBE_P_CODES_FP8) {
    const float* values = reinterpret_cast<const float*>(sink) + static_cast<long>(blockIdx.x) * kProbeThreads;
    const int i = 4 * (threadIdx.x % (kProbeThreads / 4));
    const float a = values[i], b = values[i + 1], c = values[i + 2], d = values[i + 3];
    __syncthreads();  // every read of this workgroup's words precedes every store over them
    total = kKind == PIPER_MFMA_PROBE_P_CODES_U8 ? pack_codes(a, b, c, d) : pack_fp8(a, b, c, d);
  } else if constexpr (kKind == PIPER_MFMA_PROBE_I8) {
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

// ---------------------------------------------------------------------------------------
// Issue probe.  Loop bodies are inline assembly on independent chains, so the instruction
// stream is fixed: FMA chains f = f * 1 + 1, exp chains x = 2^-x, conversion chains that keep
// writing byte lanes of a word, MFMA chains on AGPR accumulators.
// ---------------------------------------------------------------------------------------
constexpr int kIssueLdsBytes = 100 * 1024;  // more than half of a CU's 160 KiB: one workgroup per CU
constexpr int kInner = 8;                    // rounds between clock reads

__device__ __forceinline__ void fma16(float (&f)[16], float one, float add) {
  asm volatile(
      "v_fma_f32 %0, %0, %16, %17\n\t"
      "v_fma_f32 %1, %1, %16, %17\n\t"
      "v_fma_f32 %2, %2, %16, %17\n\t"
      "v_fma_f32 %3, %3, %16, %17\n\t"
      "v_fma_f32 %4, %4, %16, %17\n\t"
      "v_fma_f32 %5, %5, %16, %17\n\t"
      "v_fma_f32 %6, %6, %16, %17\n\t"
      "v_fma_f32 %7, %7, %16, %17\n\t"
      "v_fma_f32 %8, %8, %16, %17\n\t"
      "v_fma_f32 %9, %9, %16, %17\n\t"
      "v_fma_f32 %10, %10, %16, %17\n\t"
      "v_fma_f32 %11, %11, %16, %17\n\t"
      "v_fma_f32 %12, %12, %16, %17\n\t"
      "v_fma_f32 %13, %13, %16, %17\n\t"
      "v_fma_f32 %14, %14, %16, %17\n\t"
      "v_fma_f32 %15, %15, %16, %17\n\t"
      : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]), "+v"(f[7]), "+v"(f[8]), "+v"(f[9]), "+v"(f[10]), "+v"(f[11]), "+v"(f[12]), "+v"(f[13]), "+v"(f[14]), "+v"(f[15])
      : "v"(one), "v"(add));
}

__device__ __forceinline__ void exp16(float (&f)[16]) {
  asm volatile(
      "v_exp_f32 %0, -%0\n\t"
      "v_exp_f32 %1, -%1\n\t"
      "v_exp_f32 %2, -%2\n\t"
      "v_exp_f32 %3, -%3\n\t"
      "v_exp_f32 %4, -%4\n\t"
      "v_exp_f32 %5, -%5\n\t"
      "v_exp_f32 %6, -%6\n\t"
      "v_exp_f32 %7, -%7\n\t"
      "v_exp_f32 %8, -%8\n\t"
      "v_exp_f32 %9, -%9\n\t"
      "v_exp_f32 %10, -%10\n\t"
      "v_exp_f32 %11, -%11\n\t"
      "v_exp_f32 %12, -%12\n\t"
      "v_exp_f32 %13, -%13\n\t"
      "v_exp_f32 %14, -%14\n\t"
      "v_exp_f32 %15, -%15\n\t"
      : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]), "+v"(f[7]), "+v"(f[8]), "+v"(f[9]), "+v"(f[10]), "+v"(f[11]), "+v"(f[12]), "+v"(f[13]), "+v"(f[14]), "+v"(f[15]));
}

__device__ __forceinline__ void cvt16(uint32_t (&w)[16], float one) {
  asm volatile(
      "v_cvt_pk_u8_f32 %0, %16, 0, %0\n\t"
      "v_cvt_pk_u8_f32 %1, %16, 1, %1\n\t"
      "v_cvt_pk_u8_f32 %2, %16, 2, %2\n\t"
      "v_cvt_pk_u8_f32 %3, %16, 3, %3\n\t"
      "v_cvt_pk_u8_f32 %4, %16, 0, %4\n\t"
      "v_cvt_pk_u8_f32 %5, %16, 1, %5\n\t"
      "v_cvt_pk_u8_f32 %6, %16, 2, %6\n\t"
      "v_cvt_pk_u8_f32 %7, %16, 3, %7\n\t"
      "v_cvt_pk_u8_f32 %8, %16, 0, %8\n\t"
      "v_cvt_pk_u8_f32 %9, %16, 1, %9\n\t"
      "v_cvt_pk_u8_f32 %10, %16, 2, %10\n\t"
      "v_cvt_pk_u8_f32 %11, %16, 3, %11\n\t"
      "v_cvt_pk_u8_f32 %12, %16, 0, %12\n\t"
      "v_cvt_pk_u8_f32 %13, %16, 1, %13\n\t"
      "v_cvt_pk_u8_f32 %14, %16, 2, %14\n\t"
      "v_cvt_pk_u8_f32 %15, %16, 3, %15\n\t"
      : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(w[4]), "+v"(w[5]), "+v"(w[6]), "+v"(w[7]), "+v"(w[8]), "+v"(w[9]), "+v"(w[10]), "+v"(w[11]), "+v"(w[12]), "+v"(w[13]), "+v"(w[14]), "+v"(w[15])
      : "v"(one));
}

// 16 v_fma_f32, 4 v_cvt_pk_u8_f32 and 2 v_exp_f32, interleaved (the attention loop's proportions)
__device__ __forceinline__ void mix22(float (&f)[16], uint32_t (&w)[16], float (&e)[2], float one, float add) {
  asm volatile(
      "v_fma_f32 %0, %0, %22, %23\n\t"
      "v_fma_f32 %1, %1, %22, %23\n\t"
      "v_fma_f32 %2, %2, %22, %23\n\t"
      "v_cvt_pk_u8_f32 %16, %22, 0, %16\n\t"
      "v_fma_f32 %3, %3, %22, %23\n\t"
      "v_fma_f32 %4, %4, %22, %23\n\t"
      "v_fma_f32 %5, %5, %22, %23\n\t"
      "v_exp_f32 %20, -%20\n\t"
      "v_fma_f32 %6, %6, %22, %23\n\t"
      "v_fma_f32 %7, %7, %22, %23\n\t"
      "v_cvt_pk_u8_f32 %17, %22, 1, %17\n\t"
      "v_fma_f32 %8, %8, %22, %23\n\t"
      "v_fma_f32 %9, %9, %22, %23\n\t"
      "v_fma_f32 %10, %10, %22, %23\n\t"
      "v_cvt_pk_u8_f32 %18, %22, 2, %18\n\t"
      "v_fma_f32 %11, %11, %22, %23\n\t"
      "v_fma_f32 %12, %12, %22, %23\n\t"
      "v_exp_f32 %21, -%21\n\t"
      "v_fma_f32 %13, %13, %22, %23\n\t"
      "v_fma_f32 %14, %14, %22, %23\n\t"
      "v_cvt_pk_u8_f32 %19, %22, 3, %19\n\t"
      "v_fma_f32 %15, %15, %22, %23\n\t"
      : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]), "+v"(f[7]), "+v"(f[8]), "+v"(f[9]), "+v"(f[10]), "+v"(f[11]), "+v"(f[12]), "+v"(f[13]), "+v"(f[14]), "+v"(f[15]), "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(e[0]), "+v"(e[1])
      : "v"(one), "v"(add));
}

__device__ __forceinline__ void mfma_agpr(v16i& acc, v4i a) {
  asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %1, %0" : "+a"(acc) : "v"(a));
}

__device__ __forceinline__ void mfma_vgpr(v16i& acc, v4i a) {
  asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %1, %0" : "+v"(acc) : "v"(a));
}

// 16 v_add_f32 (VOP2) on 16 chains whose other operand is a 32-bit literal or an SGPR.
#define PIPER_ADD16(OPND)                                                                                         \
  "v_add_f32_e32 %0, " OPND ", %0\n\tv_add_f32_e32 %1, " OPND ", %1\n\tv_add_f32_e32 %2, " OPND ", %2\n\t"       \
  "v_add_f32_e32 %3, " OPND ", %3\n\tv_add_f32_e32 %4, " OPND ", %4\n\tv_add_f32_e32 %5, " OPND ", %5\n\t"       \
  "v_add_f32_e32 %6, " OPND ", %6\n\tv_add_f32_e32 %7, " OPND ", %7\n\tv_add_f32_e32 %8, " OPND ", %8\n\t"       \
  "v_add_f32_e32 %9, " OPND ", %9\n\tv_add_f32_e32 %10, " OPND ", %10\n\tv_add_f32_e32 %11, " OPND ", %11\n\t"   \
  "v_add_f32_e32 %12, " OPND ", %12\n\tv_add_f32_e32 %13, " OPND ", %13\n\tv_add_f32_e32 %14, " OPND ", %14\n\t" \
  "v_add_f32_e32 %15, " OPND ", %15\n\t"
#define PIPER_F16_OUTS                                                                                             \
  "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]), "+v"(f[7]), "+v"(f[8]),     \
      "+v"(f[9]), "+v"(f[10]), "+v"(f[11]), "+v"(f[12]), "+v"(f[13]), "+v"(f[14]), "+v"(f[15])

__device__ __forceinline__ void add16_literal(float (&f)[16]) { asm volatile(PIPER_ADD16("0xcb400000") : PIPER_F16_OUTS); }

__device__ __forceinline__ void add16_sgpr(float (&f)[16], float b) { asm volatile(PIPER_ADD16("%16") : PIPER_F16_OUTS : "s"(b)); }

// 32 instructions of one form into v72-v79 (four passes), sources in v64-v68 (banks 0, 1, 2, 3, 0):
// fixed registers, so that the banks of the operands are the form's and not the allocator's.  They
// stay below v80: with the 32 AGPRs of the MFMA roles the kernel needs at most 128 registers per
// lane, the most a 1024-thread workgroup (four waves per SIMD) can be given.
#define PIPER_BANK8(FORM)                                                                                     \
  FORM("v72", "v64") FORM("v73", "v65") FORM("v74", "v66") FORM("v75", "v67") FORM("v76", "v64")            \
  FORM("v77", "v65") FORM("v78", "v66") FORM("v79", "v67")
#define PIPER_BANK32(FORM) PIPER_BANK8(FORM) PIPER_BANK8(FORM) PIPER_BANK8(FORM) PIPER_BANK8(FORM)
#define PIPER_FMA_SPLIT(D, S) "v_fma_f32 " D ", v64, v65, v66\n\t"
#define PIPER_FMA_SAME(D, S) "v_fma_f32 " D ", v64, v68, v66\n\t"
#define PIPER_FMAC_SAME(D, S) "v_fmac_f32 " D ", " S ", v69\n\t"  // S: the bank of D
#define PIPER_MAX3(D, S) "v_max3_f32 " D ", v64, v65, v66\n\t"
#define PIPER_PERM(D, S) "v_perm_b32 " D ", v64, v65, v66\n\t"
#define PIPER_BANK_CLOBBERS                                                                                   \
  "v64", "v65", "v66", "v67", "v68", "v69", "v72", "v73", "v74", "v75", "v76", "v77", "v78", "v79"

template <int R>
__device__ __forceinline__ uint32_t issue_loop(uint64_t t0, uint64_t budget, const char* lds, uint32_t& rounds,
                                               uint64_t& t1) {
  constexpr bool kMfma = R == PIPER_ISSUE_MFMA || R == PIPER_ISSUE_MIX || R == PIPER_ISSUE_MFMA_FMA || R == PIPER_ISSUE_CLUSTER;
  constexpr bool kMfmaVgpr = R == PIPER_ISSUE_MIX_VGPR;
  v4i a = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
  asm volatile("" : "+v"(a));
  float one = 1.0f, add = 1.0f;
  asm volatile("" : "+v"(one), "+v"(add));
  float f[16];
  uint32_t w[16];
  float e[2] = {0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    f[i] = 0.0f;
    w[i] = 0u;
  }
  v16i acc0 = {}, acc1 = {};
  if constexpr (kMfma) asm volatile("" : "+a"(acc0), "+a"(acc1));
  if constexpr (kMfmaVgpr) asm volatile("" : "+v"(acc0), "+v"(acc1));
  float negb = -12582912.0f;  // the attention kernels' accumulator bias, in an SGPR
  asm volatile("" : "+s"(negb));
  // LDS reads: lane l reads the 16 bytes at 16 l + 1024 (i % 8), inside the first 8 KiB
  const uint32_t lds_base = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)lds)) + 16u * (threadIdx.x & 63);
  v4i words[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) words[i] = v4i{0, 0, 0, 0};
  do {
    for (int r = 0; r < kInner; ++r) {
      if constexpr (R == PIPER_ISSUE_MFMA) {
        mfma_agpr(acc0, a);
        mfma_agpr(acc1, a);
      } else if constexpr (R == PIPER_ISSUE_FMA) {
        fma16(f, one, add);
        fma16(f, one, add);
      } else if constexpr (R == PIPER_ISSUE_EXP) {
        exp16(f);
        exp16(f);
      } else if constexpr (R == PIPER_ISSUE_CVT) {
        cvt16(w, one);
        cvt16(w, one);
      } else if constexpr (R == PIPER_ISSUE_MIX) {
        mfma_agpr(acc0, a);
        mix22(f, w, e, one, add);
        mfma_agpr(acc1, a);
        mix22(f, w, e, one, add);
      } else if constexpr (R == PIPER_ISSUE_VALU_MIX) {
        mix22(f, w, e, one, add);
        mix22(f, w, e, one, add);
      } else if constexpr (R == PIPER_ISSUE_LDS) {
#pragma unroll
        for (int half = 0; half < 2; ++half) {
#pragma unroll
          for (int i = 0; i < 8; ++i)
            asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(words[i]) : "v"(lds_base), "i"(1024 * i) : "memory");
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
      } else if constexpr (R == PIPER_ISSUE_MFMA_FMA) {
        mfma_agpr(acc0, a);
        fma16(f, one, add);
        mfma_agpr(acc1, a);
        fma16(f, one, add);
      } else if constexpr (R == PIPER_ISSUE_MIX_VGPR) {
        mfma_vgpr(acc0, a);
        mix22(f, w, e, one, add);
        mfma_vgpr(acc1, a);
        mix22(f, w, e, one, add);
      } else if constexpr (R == PIPER_ISSUE_CLUSTER) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          mfma_agpr(acc0, a);
          mfma_agpr(acc1, a);
        }
#pragma unroll
        for (int m = 0; m < 8; ++m) mix22(f, w, e, one, add);
      } else if constexpr (R == PIPER_ISSUE_ADD_LIT) {
        add16_literal(f);
        add16_literal(f);
      } else if constexpr (R == PIPER_ISSUE_ADD_SGPR) {
        add16_sgpr(f, negb);
        add16_sgpr(f, negb);
      } else if constexpr (R == PIPER_ISSUE_FMA_SPLIT) {
        asm volatile(PIPER_BANK32(PIPER_FMA_SPLIT)::: PIPER_BANK_CLOBBERS);
      } else if constexpr (R == PIPER_ISSUE_FMA_SAME) {
        asm volatile(PIPER_BANK32(PIPER_FMA_SAME)::: PIPER_BANK_CLOBBERS);
      } else if constexpr (R == PIPER_ISSUE_FMAC_SAME) {
        asm volatile(PIPER_BANK32(PIPER_FMAC_SAME)::: PIPER_BANK_CLOBBERS);
      } else if constexpr (R == PIPER_ISSUE_MAX3) {
        asm volatile(PIPER_BANK32(PIPER_MAX3)::: PIPER_BANK_CLOBBERS);
      } else if constexpr (R == PIPER_ISSUE_PERM) {
        asm volatile(PIPER_BANK32(PIPER_PERM)::: PIPER_BANK_CLOBBERS);
      }
    }
    rounds += kInner;
    t1 = __builtin_amdgcn_s_memtime();
  } while (t1 - t0 < budget);
  uint32_t check = 0;
  if constexpr (kMfma || kMfmaVgpr) {
    v16i r0, r1;
    asm volatile("" : "=v"(r0) : "0"(acc0));
    asm volatile("" : "=v"(r1) : "0"(acc1));
#pragma unroll
    for (int i = 0; i < 16; ++i) check += static_cast<uint32_t>(r0[i] + r1[i]);
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) check += __float_as_uint(f[i]) + w[i];
#pragma unroll
  for (int i = 0; i < 8; ++i) check += static_cast<uint32_t>(words[i].x ^ words[i].w);
  return check + __float_as_uint(e[0]) + __float_as_uint(e[1]);
}

struct IssueParams {
  piper_issue_record* records;
  uint64_t budget;
  int roles[PIPER_ISSUE_MAX_WAVES_PER_SIMD];
};

// kVgprOnly: the kernel runs MIX_VGPR waves only (its VGPR accumulators get a register
// allocation of their own; beside the AGPR roles' state they would be shuffled through AGPRs).
template <bool kVgprOnly>
__global__ void __attribute__((amdgpu_flat_work_group_size(256, 1024))) issue_probe_kernel(const IssueParams p) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  __shared__ uint32_t slots[4];  // waves of this workgroup that reached each SIMD's counter
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (threadIdx.x < 4) slots[threadIdx.x] = 0;
  __syncthreads();
  const uint32_t hw_id = __builtin_amdgcn_s_getreg((31 << 11) | 4);   // HW_REG_HW_ID, 32 bits
  const uint32_t xcc_id = __builtin_amdgcn_s_getreg((15 << 11) | 20);  // HW_REG_XCC_ID, 16 bits
  uint32_t slot = 0;
  if ((threadIdx.x & 63) == 0) slot = atomicAdd(&slots[(hw_id >> 4) & 3], 1u);
  slot = __builtin_amdgcn_readfirstlane(slot);
  const int role = slot < PIPER_ISSUE_MAX_WAVES_PER_SIMD ? p.roles[slot] : PIPER_ISSUE_IDLE;
  __syncthreads();
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  uint64_t t1 = t0;
  uint32_t rounds = 0, check = 0;
  if constexpr (kVgprOnly) {
    if (role == PIPER_ISSUE_MIX_VGPR) check = issue_loop<PIPER_ISSUE_MIX_VGPR>(t0, p.budget, lds, rounds, t1);
  } else switch (role) {
    case PIPER_ISSUE_MFMA: check = issue_loop<PIPER_ISSUE_MFMA>(t0, p.budget, lds, rounds, t1); break;
    case PIPER_ISSUE_FMA: check = issue_loop<PIPER_ISSUE_FMA>(t0, p.budget, lds, rounds, t1); break;
    case PIPER_ISSUE_EXP: check = issue_loop<PIPER_ISSUE_EXP>(t0, p.budget, lds, rounds, t1); break;
    case PIPER_ISSUE_CVT: check = issue_loop<PIPER_ISSUE_CVT>(t0, p.budget, lds, rounds, t1); break;
    case PIPER_ISSUE_MIX: check = issue_loop<PIPER_ISSUE_MIX>(t0, p.budget, lds, rounds, t1); break;
    case PIPER_ISSUE_VALU_MIX: check = issue_loop<PIPER_ISSUE_VALU_MIX>(t0, p.budget, lds, rounds, t1); break;
    case PIPER_ISSUE_LDS: check = issue_loop<PIPER_ISSUE_LDS>(t0, p.budget, lds, rounds, t1); break;
    case PIPER_ISSUE_MFMA_FMA: check = issue_loop<PIPER_ISSUE_MFMA_FMA>(t0, p.budget, lds, rounds, t1); break;
    case PIPER_ISSUE_CLUSTER: check = issue_loop<PIPER_ISSUE_CLUSTER>(t0, p.budget, lds, rounds, t1); break;
    case PIPER_ISSUE_ADD_LIT: check = issue_loop<PIPER_ISSUE_ADD_LIT>(t0, p.budget, lds, rounds, t1); break;
    case PIPER_ISSUE_ADD_SGPR: check = issue_loop<PIPER_ISSUE_ADD_SGPR>(t0, p.budget, lds, rounds, t1); break;
    case PIPER_ISSUE_FMA_SPLIT: check = issue_loop<PIPER_ISSUE_FMA_SPLIT>(t0, p.budget, lds, rounds, t1); break;
    case PIPER_ISSUE_FMA_SAME: check = issue_loop<PIPER_ISSUE_FMA_SAME>(t0, p.budget, lds, rounds, t1); break;
    case PIPER_ISSUE_FMAC_SAME: check = issue_loop<PIPER_ISSUE_FMAC_SAME>(t0, p.budget, lds, rounds, t1); break;
    case PIPER_ISSUE_MAX3: check = issue_loop<PIPER_ISSUE_MAX3>(t0, p.budget, lds, rounds, t1); break;
    case PIPER_ISSUE_PERM: check = issue_loop<PIPER_ISSUE_PERM>(t0, p.budget, lds, rounds, t1); break;
    default: break;
  }
  if ((threadIdx.x & 63) == 0) {
    piper_issue_record rec;
    rec.hw_id = hw_id;
    rec.xcc_id = xcc_id;
    rec.role = static_cast<uint32_t>(role);
    rec.slot = slot;
    rec.cycles = t1 - t0;
    rec.rounds = rounds;
    rec.check = check;
    p.records[static_cast<long>(blockIdx.x) * PIPER_ISSUE_RECORDS_PER_WORKGROUP + wave] = rec;
  }
}

thread_local char g_last_error[512] = "";

int fail(int status, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
  return status;
}

// Engine clock: each one-wave workgroup reads the shader clock counter (s_memtime, variable
// frequency) and the wall clock counter (s_memrealtime, constant rate) at its start, sleeps until
// the wall clock has advanced by `ticks` (at most kClockProbeMaxSleeps sleeps, so the wave ends
// even if the counter stalled), and reads both again.
constexpr uint32_t kClockProbeMaxSleeps = 1u << 20;

__global__ void __launch_bounds__(64) clock_probe_kernel(uint64_t* records, uint64_t ticks) {
  const uint64_t wall0 = __builtin_amdgcn_s_memrealtime();
  const uint64_t clock0 = __builtin_amdgcn_s_memtime();
  uint64_t wall1 = wall0;
  for (uint32_t i = 0; i < kClockProbeMaxSleeps && wall1 - wall0 < ticks; ++i) {
    __builtin_amdgcn_s_sleep(127);
    wall1 = __builtin_amdgcn_s_memrealtime();
  }
  const uint64_t clock1 = __builtin_amdgcn_s_memtime();
  if (threadIdx.x == 0) {
    uint64_t* r = records + 4 * static_cast<long>(blockIdx.x);
    r[0] = wall0;
    r[1] = clock0;
    r[2] = wall1;
    r[3] = clock1;
  }
}

}  // namespace
}  // namespace piper

extern "C" {

int piper_probe_abi_version(void) { return PIPER_PROBE_ABI_VERSION; }

const char* piper_probe_last_error(void) { return piper::g_last_error; }

int piper_mfma_probe(int32_t kind, int32_t workgroups, int32_t iterations, uint32_t* sink, void* stream) {
  using namespace piper;
  if (kind < PIPER_MFMA_PROBE_I8 || kind > PIPER_MFMA_PROBE_P_CODES_U8_SCALED)
    return fail(2, "unknown MFMA probe kind %d", kind);
  if (workgroups < 1 || workgroups > 65536 || iterations < 1 || iterations > (1 << 24))
    return fail(1, "probe needs 1..65536 workgroups and 1..2^24 iterations, got %d and %d", workgroups, iterations);
  if (sink == nullptr || (reinterpret_cast<uintptr_t>(sink) & 3u) != 0)
    return fail(1, "sink must be a non-NULL 4-byte aligned buffer of workgroups * %d words", PIPER_MFMA_PROBE_THREADS);
  const dim3 grid(static_cast<unsigned>(workgroups));
  const dim3 block(kProbeThreads);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (kind) {
    case PIPER_MFMA_PROBE_I8: hipLaunchKernelGGL(mfma_probe_kernel<PIPER_MFMA_PROBE_I8>, grid, block, 0, s, sink, iterations); break;
    case PIPER_MFMA_PROBE_F8: hipLaunchKernelGGL(mfma_probe_kernel<PIPER_MFMA_PROBE_F8>, grid, block, 0, s, sink, iterations); break;
    case PIPER_MFMA_PROBE_P_CODES_U8:
      hipLaunchKernelGGL(mfma_probe_kernel<PIPER_MFMA_PROBE_P_CODES_U8>, grid, block, 0, s, sink, iterations);
      break;
    case PIPER_MFMA_PROBE_P_CODES_FP8:
      hipLaunchKernelGGL(mfma_probe_kernel<PIPER_MFMA_PROBE_P_CODES_FP8>, grid, block, 0, s, sink, iterations);
      break;
    default:
      hipLaunchKernelGGL(mfma_probe_kernel<PIPER_MFMA_PROBE_P_CODES_U8_SCALED>, grid, block, 0, s, sink, iterations);
      break;
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(3, "probe launch failed: %s", hipGetErrorString(err));
  g_last_error[0] = '\0';
  return 0;
}

int piper_issue_probe(const piper_issue_probe_args* a, void* stream) {
  using namespace piper;
  if (a == nullptr) return fail(1, "args is NULL");
  if (a->waves_per_simd < 1 || a->waves_per_simd > PIPER_ISSUE_MAX_WAVES_PER_SIMD)
    return fail(1, "waves_per_simd must be 1..%d, got %d", PIPER_ISSUE_MAX_WAVES_PER_SIMD, a->waves_per_simd);
  if (a->workgroups < 1 || a->workgroups > 65536) return fail(1, "workgroups must be 1..65536, got %d", a->workgroups);
  if (a->cycle_budget < 1000 || a->cycle_budget > 100000000)
    return fail(1, "cycle_budget must be 1000..10^8, got %lld", (long long)a->cycle_budget);
  if (a->records == nullptr || (reinterpret_cast<uintptr_t>(a->records) & 7u) != 0)
    return fail(1, "records must be a non-NULL 8-byte aligned buffer of workgroups * %d records",
                PIPER_ISSUE_RECORDS_PER_WORKGROUP);
  IssueParams p{};
  p.records = a->records;
  p.budget = static_cast<uint64_t>(a->cycle_budget);
  int vgpr_roles = 0, other_roles = 0;
  for (int s = 0; s < PIPER_ISSUE_MAX_WAVES_PER_SIMD; ++s) {
    const int role = s < a->waves_per_simd ? a->roles[s] : PIPER_ISSUE_IDLE;
    if (role < 0 || role >= PIPER_ISSUE_ROLES) return fail(2, "unknown role %d in slot %d", role, s);
    p.roles[s] = role;
    vgpr_roles += role == PIPER_ISSUE_MIX_VGPR;
    other_roles += role != PIPER_ISSUE_MIX_VGPR && role != PIPER_ISSUE_IDLE;
  }
  if (vgpr_roles > 0 && other_roles > 0) return fail(2, "MIX_VGPR shares a SIMD only with MIX_VGPR or IDLE waves");
  const void* kernel = vgpr_roles > 0 ? reinterpret_cast<const void*>(issue_probe_kernel<true>)
                                      : reinterpret_cast<const void*>(issue_probe_kernel<false>);
  hipError_t err = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kIssueLdsBytes);
  if (err != hipSuccess) return fail(3, "hipFuncSetAttribute failed: %s", hipGetErrorString(err));
  if (vgpr_roles > 0)
    hipLaunchKernelGGL(issue_probe_kernel<true>, dim3(static_cast<unsigned>(a->workgroups)),
                       dim3(256 * a->waves_per_simd), kIssueLdsBytes, static_cast<hipStream_t>(stream), p);
  else
    hipLaunchKernelGGL(issue_probe_kernel<false>, dim3(static_cast<unsigned>(a->workgroups)),
                       dim3(256 * a->waves_per_simd), kIssueLdsBytes, static_cast<hipStream_t>(stream), p);
  err = hipGetLastError();
  if (err != hipSuccess) return fail(3, "issue probe launch failed: %s", hipGetErrorString(err));
  g_last_error[0] = '\0';
  return 0;
}

int piper_clock_probe(int32_t workgroups, int64_t duration_us, uint64_t* records, int32_t* wall_clock_khz,
                      void* stream) {
  using namespace piper;
  if (workgroups < 1 || workgroups > PIPER_CLOCK_PROBE_MAX_WORKGROUPS)
    return fail(1, "clock probe needs 1..%d workgroups, got %d", PIPER_CLOCK_PROBE_MAX_WORKGROUPS, workgroups);
  if (duration_us < 1 || duration_us > 2000000)
    return fail(1, "clock probe duration must be 1..2000000 us, got %lld", (long long)duration_us);
  if (records == nullptr || (reinterpret_cast<uintptr_t>(records) & 7u) != 0 || wall_clock_khz == nullptr)
    return fail(1, "records must be a non-NULL 8-byte aligned buffer of 4 * workgroups words, wall_clock_khz non-NULL");
  int device = 0;
  int khz = 0;
  hipError_t err = hipGetDevice(&device);
  if (err == hipSuccess) err = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device);
  if (err != hipSuccess) return fail(3, "wall clock rate unavailable: %s", hipGetErrorString(err));
  if (khz <= 0) return fail(2, "the device reports no wall clock rate");
  const uint64_t ticks = static_cast<uint64_t>(duration_us) * static_cast<uint64_t>(khz) / 1000u;
  hipLaunchKernelGGL(clock_probe_kernel, dim3(static_cast<unsigned>(workgroups)), dim3(64), 0,
                     static_cast<hipStream_t>(stream), records, ticks);
  err = hipGetLastError();
  if (err != hipSuccess) return fail(3, "clock probe launch failed: %s", hipGetErrorString(err));
  *wall_clock_khz = khz;
  g_last_error[0] = '\0';
  return 0;
}

}  // extern "C"
