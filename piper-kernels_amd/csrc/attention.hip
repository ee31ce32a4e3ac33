// Fused Piper Attention forward for gfx950: INT8 MFMA QK^T, FP32 online softmax, UINT8
// probabilities times INT8 V on signed MFMA through u@v = (u-128)@v + 128*colsum(v).
//
// Behaviour follows the reference recurrence (jumbledpoophj/piper-kernels 0.2.1,
// src/piper_kernels/attention/piper_attention/reference.py:61-118): per 64-key block,
// shifted = s + ln vs, block max bm, p = exp(s - bm), u = round(p * vs * 255) clamped to
// [0, 255], num = num*alpha + (u @ v) * beta / 255, den = den*alpha + sum(p) * beta, and the
// epilogue num / max(den, 1e-30) + mean(V).  Work is done in the log2 domain (the softmax
// scale carries log2(e)) and the numerator is rescaled lazily: only when a block maximum
// exceeds the reference maximum by more than 2^8, which changes rounding, not the formula.
//
// Design (one workgroup = NW waves x 32 queries, K/V streamed in 64-key tiles):
// * S^T = K Q^T on v_mfma_i32_32x32x32_i8: each lane owns one query column, so the row max,
//   row sum and P quantisation run in-lane; the two 32-lane halves are merged with
//   v_permlane32_swap.  K rows are loaded in a permuted order so that each lane ends up with
//   16 consecutive keys -- exactly the B-operand layout of the PV MFMA, so P never leaves
//   registers.
// * O^T = V^T P^T on the same MFMA with the affine correction 128*colsum(v) as the
//   accumulator input; v_cvt_pk_u8_f32 rounds half-to-even and saturates to [0, 255], which
//   is round().clamp(0, 255) of the reference.
// * K, V^T, per-key log2 scales, inverse multipliers and column sums of a tile are staged in
//   LDS (double-buffered, padded rows against bank conflicts) with 16-byte global loads.
#include "common.h"
#include "kernels.h"

namespace piper {

constexpr float kLazyRescale = 8.0f;               // log2 headroom before num/den are rescaled
constexpr float kLog2Of255 = 7.994353436858858f;   // log2(255)

template <int D, int NW>
struct TileLayout {
  static constexpr int kThreads = NW * kWave;
  static constexpr int kKStride = D + 16;       // bytes per K row in LDS
  static constexpr int kVStride = kKeyBlock + 16;  // bytes per V^T row in LDS
  static constexpr int kKBytes = kKeyBlock * kKStride;
  static constexpr int kVBytes = D * kVStride;
  static constexpr int kLogOffset = kKBytes + kVBytes;  // 64 floats: log2 of V row scales
  static constexpr int kInvOffset = kLogOffset + 256;   // 64 floats: 1 / (255 * scale)
  static constexpr int kCorrOffset = kInvOffset + 256;  // D ints: 128 * colsum
  static constexpr int kStageBytes = kCorrOffset + 4 * D;
  static constexpr int kChunksK = kKeyBlock * D / 16;  // 16-byte chunks per region
  static constexpr int kChunksV = D * kKeyBlock / 16;
  static constexpr int kChunks = kChunksK + kChunksV + 16 + 16 + D / 4;
  static constexpr int kRounds = (kChunks + kThreads - 1) / kThreads;
};

template <int D, int NW>
__device__ __forceinline__ void fetch_tile(const AttnParams& p, int bh, int t,
                                           uint4 (&reg)[TileLayout<D, NW>::kRounds]) {
  using L = TileLayout<D, NW>;
  const int8_t* ktile = p.key_code + (static_cast<long>(bh) * p.sk64 + static_cast<long>(t) * kKeyBlock) * D;
  const int8_t* vtile = p.value_code + (static_cast<long>(bh) * p.nkb + t) * static_cast<long>(D * kKeyBlock);
  const float* lk = p.value_log2_scale + static_cast<long>(bh) * p.sk64 + t * kKeyBlock;
  const float* iv = p.value_inv_multiplier + static_cast<long>(bh) * p.sk64 + t * kKeyBlock;
  const int32_t* cr = p.value_correction + (static_cast<long>(bh) * p.nkb + t) * D;
#pragma unroll
  for (int r = 0; r < L::kRounds; ++r) {
    const int i = threadIdx.x + r * L::kThreads;
    if (i >= L::kChunks) break;
    const uint4* src;
    if (i < L::kChunksK) {
      src = reinterpret_cast<const uint4*>(ktile) + i;
    } else if (i < L::kChunksK + L::kChunksV) {
      src = reinterpret_cast<const uint4*>(vtile) + (i - L::kChunksK);
    } else if (i < L::kChunksK + L::kChunksV + 16) {
      src = reinterpret_cast<const uint4*>(lk) + (i - L::kChunksK - L::kChunksV);
    } else if (i < L::kChunksK + L::kChunksV + 32) {
      src = reinterpret_cast<const uint4*>(iv) + (i - L::kChunksK - L::kChunksV - 16);
    } else {
      src = reinterpret_cast<const uint4*>(cr) + (i - L::kChunksK - L::kChunksV - 32);
    }
    reg[r] = *src;
  }
}

template <int D, int NW>
__device__ __forceinline__ void store_tile(char* stage, const uint4 (&reg)[TileLayout<D, NW>::kRounds]) {
  using L = TileLayout<D, NW>;
#pragma unroll
  for (int r = 0; r < L::kRounds; ++r) {
    const int i = threadIdx.x + r * L::kThreads;
    if (i >= L::kChunks) break;
    int dst;
    if (i < L::kChunksK) {
      dst = (i / (D / 16)) * L::kKStride + (i % (D / 16)) * 16;
    } else if (i < L::kChunksK + L::kChunksV) {
      const int j = i - L::kChunksK;
      dst = L::kKBytes + (j >> 2) * L::kVStride + (j & 3) * 16;
    } else {
      dst = L::kLogOffset + (i - L::kChunksK - L::kChunksV) * 16;  // log2, inv and corr are contiguous
    }
    *reinterpret_cast<uint4*>(stage + dst) = reg[r];
  }
}

__device__ __forceinline__ uint32_t pack_codes(float e0, float e1, float e2, float e3) {
  uint32_t w = __builtin_amdgcn_cvt_pk_u8_f32(e0, 0, 0u);
  w = __builtin_amdgcn_cvt_pk_u8_f32(e1, 1, w);
  w = __builtin_amdgcn_cvt_pk_u8_f32(e2, 2, w);
  w = __builtin_amdgcn_cvt_pk_u8_f32(e3, 3, w);
  return w ^ 0x80808080u;  // u - 128 as signed INT8
}

template <int kOut>
__device__ __forceinline__ void store4(void* out, long index, float a, float b, float c, float d) {
  if constexpr (kOut == 2) {
    *reinterpret_cast<float4*>(static_cast<float*>(out) + index) = make_float4(a, b, c, d);
  } else if constexpr (kOut == 1) {
    const uint2 v = make_uint2(float_to_bf16_bits(a) | (float_to_bf16_bits(b) << 16),
                               float_to_bf16_bits(c) | (float_to_bf16_bits(d) << 16));
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + index) = v;
  } else {
    const uint2 v = make_uint2(float_to_half_bits(a) | (float_to_half_bits(b) << 16),
                               float_to_half_bits(c) | (float_to_half_bits(d) << 16));
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + index) = v;
  }
}

template <int D, int NW, bool kCausal, int kOut>
__global__ void __launch_bounds__(NW * 64, 1) attention_kernel(const AttnParams p) {
  using L = TileLayout<D, NW>;
  constexpr int kChunksD = D / 32;
  __shared__ __attribute__((aligned(16))) char smem[2 * L::kStageBytes];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5;  // lane half
  const int n = lane & 31;  // query column within the wave
  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int qtile = logical % p.query_tiles;
  const int bh = logical / p.query_tiles;
  const int q0 = qtile * (NW * 32) + wave * 32;  // first query of this wave
  const bool wave_live = q0 < p.query_length;

  // Q^T fragments (B operand): query q0 + n, bytes [32c + 16h, +16) of each 32-dim chunk.
  v4i qf[kChunksD];
  float cq = 0.0f;
  if (q0 < p.sq32) {
    const int8_t* qrow = p.query_code + (static_cast<long>(bh) * p.sq32 + q0 + n) * D + 16 * h;
#pragma unroll
    for (int c = 0; c < kChunksD; ++c) qf[c] = *reinterpret_cast<const v4i*>(qrow + 32 * c);
    cq = p.query_scale[static_cast<long>(bh) * p.nqb + (q0 >> 5)] * p.scale_log2e;
  } else {
#pragma unroll
    for (int c = 0; c < kChunksD; ++c) qf[c] = v4i{0, 0, 0, 0};
  }

  int tiles = p.nkb;
  int wave_tiles = wave_live ? p.nkb : 0;
  if constexpr (kCausal) {
    const int last_query = min(p.query_length, (qtile + 1) * NW * 32) - 1;
    tiles = last_query / kKeyBlock + 1;
    wave_tiles = wave_live ? (min(p.query_length, q0 + 32) - 1) / kKeyBlock + 1 : 0;
  }

  float num[kChunksD][16];
#pragma unroll
  for (int j = 0; j < kChunksD; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) num[j][r] = 0.0f;
  float den = 0.0f;
  float mref = -__builtin_inff();

  // MFMA row m of the K operand holds key 16*((m>>2)&1) + 4*(m>>3) + (m&3), so that output
  // register r of lane half h holds key 16h + r.
  const int krow = 16 * ((n >> 2) & 1) + 4 * (n >> 3) + (n & 3);
  const float* key_scale = p.key_scale + static_cast<long>(bh) * p.nkb;

  uint4 reg[L::kRounds];
  fetch_tile<D, NW>(p, bh, 0, reg);
  store_tile<D, NW>(smem, reg);
  __syncthreads();

  for (int t = 0; t < tiles; ++t) {
    const char* sb = smem + (t & 1) * L::kStageBytes;
    if (t + 1 < tiles) fetch_tile<D, NW>(p, bh, t + 1, reg);

    if (t < wave_tiles) {
      // ---- integer scores for 64 keys: s0 keys 0..31, s1 keys 32..63 ----
      v16i s0 = {}, s1 = {};
#pragma unroll
      for (int c = 0; c < kChunksD; ++c) {
        const v4i a0 = *reinterpret_cast<const v4i*>(sb + krow * L::kKStride + 32 * c + 16 * h);
        const v4i a1 = *reinterpret_cast<const v4i*>(sb + (32 + krow) * L::kKStride + 32 * c + 16 * h);
        s0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, qf[c], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, qf[c], s1, 0, 0, 0);
      }
      const float ct = cq * key_scale[t];

      // ---- shifted scores x = s * c + log2(vs), in-lane over 32 keys ----
      const float4* lk4 = reinterpret_cast<const float4*>(sb + L::kLogOffset);
      float x[32];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 la = lk4[4 * h + q];
        const float4 lb = lk4[8 + 4 * h + q];
        x[4 * q + 0] = fmaf(static_cast<float>(s0[4 * q + 0]), ct, la.x);
        x[4 * q + 1] = fmaf(static_cast<float>(s0[4 * q + 1]), ct, la.y);
        x[4 * q + 2] = fmaf(static_cast<float>(s0[4 * q + 2]), ct, la.z);
        x[4 * q + 3] = fmaf(static_cast<float>(s0[4 * q + 3]), ct, la.w);
        x[16 + 4 * q + 0] = fmaf(static_cast<float>(s1[4 * q + 0]), ct, lb.x);
        x[16 + 4 * q + 1] = fmaf(static_cast<float>(s1[4 * q + 1]), ct, lb.y);
        x[16 + 4 * q + 2] = fmaf(static_cast<float>(s1[4 * q + 2]), ct, lb.z);
        x[16 + 4 * q + 3] = fmaf(static_cast<float>(s1[4 * q + 3]), ct, lb.w);
      }
      if constexpr (kCausal) {
        if (t * kKeyBlock + kKeyBlock - 1 > q0) {  // tile crosses this wave's diagonal
          const int query = q0 + n;
          const int key_base = t * kKeyBlock + 16 * h;
#pragma unroll
          for (int r = 0; r < 32; ++r) {
            const int key = key_base + (r < 16 ? r : 16 + r);
            if (key > query) x[r] = -__builtin_inff();
          }
        }
      }

      float mx = x[0];
#pragma unroll
      for (int r = 1; r < 32; ++r) mx = fmaxf(mx, x[r]);
      mx = cross_half_max(mx);  // block max of the shifted scores for this query

      const bool grow = mx > mref + kLazyRescale;
      if (__builtin_amdgcn_ballot_w64(grow) != 0) {
        const float alpha = grow ? __builtin_amdgcn_exp2f(mref - mx) : 1.0f;
        if (grow) mref = mx;
#pragma unroll
        for (int j = 0; j < kChunksD; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) num[j][r] *= alpha;
        den *= alpha;
      }
      const bool empty = mx == -__builtin_inff();
      const float beta = empty ? 0.0f : __builtin_amdgcn_exp2f(mx - mref);
      const float shift = empty ? 0.0f : mx - kLog2Of255;

      // ---- e = 255 * vs * p, den += sum(p), UINT8 codes ----
      const float4* iv4 = reinterpret_cast<const float4*>(sb + L::kInvOffset);
      float psum = 0.0f;
      uint32_t pw[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 ia = iv4[4 * h + q];
        const float4 ib = iv4[8 + 4 * h + q];
        const float e0 = __builtin_amdgcn_exp2f(x[4 * q + 0] - shift);
        const float e1 = __builtin_amdgcn_exp2f(x[4 * q + 1] - shift);
        const float e2 = __builtin_amdgcn_exp2f(x[4 * q + 2] - shift);
        const float e3 = __builtin_amdgcn_exp2f(x[4 * q + 3] - shift);
        const float f0 = __builtin_amdgcn_exp2f(x[16 + 4 * q + 0] - shift);
        const float f1 = __builtin_amdgcn_exp2f(x[16 + 4 * q + 1] - shift);
        const float f2 = __builtin_amdgcn_exp2f(x[16 + 4 * q + 2] - shift);
        const float f3 = __builtin_amdgcn_exp2f(x[16 + 4 * q + 3] - shift);
        psum = fmaf(e0, ia.x, psum);
        psum = fmaf(e1, ia.y, psum);
        psum = fmaf(e2, ia.z, psum);
        psum = fmaf(e3, ia.w, psum);
        psum = fmaf(f0, ib.x, psum);
        psum = fmaf(f1, ib.y, psum);
        psum = fmaf(f2, ib.z, psum);
        psum = fmaf(f3, ib.w, psum);
        pw[q] = pack_codes(e0, e1, e2, e3);
        pw[4 + q] = pack_codes(f0, f1, f2, f3);
      }
      psum = cross_half_sum(psum);
      den = fmaf(psum, beta, den);

      // ---- numerator: O^T += (V^T (u - 128) + 128 colsum) * beta / 255 ----
      const v4i p0 = {static_cast<int>(pw[0]), static_cast<int>(pw[1]), static_cast<int>(pw[2]),
                      static_cast<int>(pw[3])};
      const v4i p1 = {static_cast<int>(pw[4]), static_cast<int>(pw[5]), static_cast<int>(pw[6]),
                      static_cast<int>(pw[7])};
      const float weight = beta * (1.0f / 255.0f);
      const char* vsb = sb + L::kKBytes;
      const v4i* corr4 = reinterpret_cast<const v4i*>(sb + L::kCorrOffset);
#pragma unroll
      for (int j = 0; j < kChunksD; ++j) {
        v16i acc;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const v4i c4 = corr4[8 * j + 2 * g + h];
          acc[4 * g + 0] = c4[0];
          acc[4 * g + 1] = c4[1];
          acc[4 * g + 2] = c4[2];
          acc[4 * g + 3] = c4[3];
        }
        const char* vrow = vsb + (32 * j + n) * L::kVStride + 16 * h;
        const v4i a0 = *reinterpret_cast<const v4i*>(vrow);
        const v4i a1 = *reinterpret_cast<const v4i*>(vrow + 32);
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, p0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, p1, acc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 16; ++r) num[j][r] = fmaf(static_cast<float>(acc[r]), weight, num[j][r]);
      }
    }

    if (t + 1 < tiles) store_tile<D, NW>(smem + ((t + 1) & 1) * L::kStageBytes, reg);
    __syncthreads();
  }

  // ---- epilogue: num / max(den, 1e-30) + mean(V), one query per lane ----
  const int query = q0 + n;
  if (!wave_live || query >= p.query_length) return;
  const float rden = 1.0f / fmaxf(den, 1e-30f);
  const float* vmean = p.value_mean + static_cast<long>(bh) * D;
  const long out_row = (static_cast<long>(bh) * p.query_length + query) * D;
#pragma unroll
  for (int j = 0; j < kChunksD; ++j) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * j + 8 * g + 4 * h;
      float4 m = make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (!kCausal) m = *reinterpret_cast<const float4*>(vmean + d0);
      // explicit FMAs: every output dtype rounds the same FP32 value
      store4<kOut>(p.output, out_row + d0, fmaf(num[j][4 * g + 0], rden, m.x), fmaf(num[j][4 * g + 1], rden, m.y),
                   fmaf(num[j][4 * g + 2], rden, m.z), fmaf(num[j][4 * g + 3], rden, m.w));
    }
  }
}

template <int D, int NW, bool kCausal>
static hipError_t launch_out(int out_dtype, const AttnParams& ap, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(ap.query_tiles * ap.batch_heads));
  const dim3 block(NW * 64);
  switch (out_dtype) {
    case 0: hipLaunchKernelGGL((attention_kernel<D, NW, kCausal, 0>), grid, block, 0, stream, ap); break;
    case 1: hipLaunchKernelGGL((attention_kernel<D, NW, kCausal, 1>), grid, block, 0, stream, ap); break;
    default: hipLaunchKernelGGL((attention_kernel<D, NW, kCausal, 2>), grid, block, 0, stream, ap); break;
  }
  return hipGetLastError();
}

template <int D, int NW>
static hipError_t launch_causal(bool causal, int out_dtype, const AttnParams& ap, hipStream_t stream) {
  return causal ? launch_out<D, NW, true>(out_dtype, ap, stream) : launch_out<D, NW, false>(out_dtype, ap, stream);
}

hipError_t launch_attention(int head_dim, bool causal, int out_dtype, int waves, const AttnParams& ap,
                            hipStream_t stream) {
  if (head_dim == 128) {
    return waves == 4 ? launch_causal<128, 4>(causal, out_dtype, ap, stream)
                      : launch_causal<128, 8>(causal, out_dtype, ap, stream);
  }
  return waves == 4 ? launch_causal<64, 4>(causal, out_dtype, ap, stream)
                    : launch_causal<64, 8>(causal, out_dtype, ap, stream);
}

}  // namespace piper
