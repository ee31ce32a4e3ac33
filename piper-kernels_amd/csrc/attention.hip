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
// * K, V^T, per-key log2 scales, inverse multipliers and column sums of a tile form one
//   record laid out exactly like its LDS stage (padded rows against bank conflicts); it is
//   copied with direct global -> LDS loads into a 6-stage ring, 4 blocks ahead.
#include "common.h"
#include "kernels.h"
#include "quant.h"

namespace piper {

constexpr float kLazyRescale = 8.0f;               // log2 headroom before num/den are rescaled
constexpr float kLog2Of255 = 7.994353436858858f;   // log2(255)

template <int D, int NW>
struct TileLayout {
  static constexpr int kKStride = kv_k_stride(D);  // bytes per K row in LDS
  static constexpr int kVStride = kv_v_stride();   // bytes per V^T row in LDS
  static constexpr int kKBytes = kv_v_offset(D);
  static constexpr int kLogOffset = kv_log_offset(D);  // 64 floats: log2 of V row scales
  static constexpr int kInvOffset = kv_inv_offset(D);  // 64 floats: 1 / (255 * scale)
  static constexpr int kCorrOffset = kv_corr_offset(D);  // D ints: biased 128 * colsum
  static constexpr int kStageBytes = kv_tile_bytes(D);  // the tile record is the stage image
  static constexpr int kPieces = kStageBytes / 1024;    // 1 KiB per wave-wide 16-byte load
  static constexpr int kRounds = (kPieces + NW - 1) / NW;
  static constexpr int kFullWaves = kPieces % NW == 0 ? NW : kPieces % NW;  // waves with kRounds pieces
};

// One wave-wide global_load_lds_dwordx4: lane i copies 16 bytes from its global address to
// LDS byte lds + 16 * i.  Issued as inline assembly so that the compiler's wait insertion does
// not treat every later LDS read as dependent on it: the waits are explicit (stage_barrier,
// and a drain before the waves end).
__device__ __forceinline__ void copy_piece(const void* src, uint32_t lds) {
  // s_nop: one wait state between the SALU write of M0 and the LDS DMA that reads it
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds) : "memory");
}

__device__ __forceinline__ uint32_t lds_address(const char* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}

// Direct global -> LDS copy of the tile record of block t into one LDS stage: wave w copies
// 1 KiB pieces w, w + NW, ... (each lane 16 bytes), so the per-lane addresses are loop
// invariant and no VGPRs hold staged data.  Completion is tracked by this wave's vmcnt.
template <int D, int NW>
__device__ __forceinline__ void copy_block(const AttnParams& p, char* stage, int bh, int t, int wave, int lane) {
  using L = TileLayout<D, NW>;
  const char* tile = reinterpret_cast<const char*>(p.kv_tiles) + (static_cast<long>(bh) * p.nkb + t) * L::kStageBytes;
  const uint32_t base = lds_address(stage);
#pragma unroll
  for (int r = 0; r < L::kRounds; ++r) {
    const int piece = wave + r * NW;  // wave-uniform: a scalar branch
    if (piece < L::kPieces) copy_piece(tile + piece * 1024 + lane * 16, base + piece * 1024);
  }
}

// Workgroup barrier that lets this wave's newest kInFlight direct loads stay in flight.
// (__syncthreads would drain every outstanding load.)  LDS reads are waited for as well, so
// a stage is never overwritten under a pending read.
template <int kInFlight>
__device__ __forceinline__ void stage_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kInFlight) : "memory");
}

template <int D, int NW>
__device__ __forceinline__ void stage_barrier_keep_last(int wave) {
  using L = TileLayout<D, NW>;
  if (wave < L::kFullWaves)
    stage_barrier<L::kRounds>();
  else
    stage_barrier<L::kRounds - 1>();
}

// Balanced max over 32 values (depth 4 instead of a 16-long v_max3 chain).
__device__ __forceinline__ float max32(const float (&x)[32]) {
  float t[11];
#pragma unroll
  for (int i = 0; i < 10; ++i) t[i] = fmaxf(fmaxf(x[3 * i], x[3 * i + 1]), x[3 * i + 2]);
  t[10] = fmaxf(x[30], x[31]);
  const float u0 = fmaxf(fmaxf(t[0], t[1]), t[2]);
  const float u1 = fmaxf(fmaxf(t[3], t[4]), t[5]);
  const float u2 = fmaxf(fmaxf(t[6], t[7]), t[8]);
  const float u3 = fmaxf(t[9], t[10]);
  return fmaxf(fmaxf(u0, u1), fmaxf(u2, u3));
}

__device__ __forceinline__ uint32_t pack_codes(float e0, float e1, float e2, float e3) {
  uint32_t w = __builtin_amdgcn_cvt_pk_u8_f32(e0, 0, 0u);
  w = __builtin_amdgcn_cvt_pk_u8_f32(e1, 1, w);
  w = __builtin_amdgcn_cvt_pk_u8_f32(e2, 2, w);
  w = __builtin_amdgcn_cvt_pk_u8_f32(e3, 3, w);
  return w ^ 0x80808080u;  // u - 128 as signed INT8
}

// Keep x as a materialised FP32 value: narrowing must round the FP32 result (as the
// reference casts its FP32 output), not a fused multiply-add to f16 (v_fma_mix).
__device__ __forceinline__ float materialize(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

template <int kOut>
__device__ __forceinline__ void store4(void* out, long index, float a, float b, float c, float d) {
  if constexpr (kOut != 2) {
    a = materialize(a);
    b = materialize(b);
    c = materialize(c);
    d = materialize(d);
  }
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

// Value of an integer accumulator that started from kAccBias: one exact FP32 subtraction.
// (The element arrives as a scalar: this clang's __builtin_bit_cast of an ext_vector
// subscript reads element 0.)
__device__ __forceinline__ float unbias(int bits) { return __builtin_bit_cast(float, bits) - kAccBiasValue; }

// A 16-byte global load the compiler does not track: the caller waits for it with an explicit
// s_waitcnt, which lets later direct LDS copies stay in flight.  (A tracked load would get a
// compiler wait that also drains every copy issued after it: vmcnt completes in order.)
__device__ __forceinline__ v4i load_untracked(const void* src) {
  v4i r;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=&v"(r) : "v"(src) : "memory");
  return r;
}

// Fused query quantisation, part 1: lane (n, h) issues the loads of elements [32c + 16h, +16)
// of query row q0 + n (row q0 for rows past the end: their values are replaced by zeros).
template <int D>
__device__ __forceinline__ void issue_query_loads(const AttnParams& p, int bh, int q0, int n, int h,
                                                  v4i (&raw)[D / 16]) {
  const int b = bh / p.heads;
  const int head = bh - b * p.heads;
  const int row = min(q0 + n, p.query_length - 1);
  const uint16_t* src = static_cast<const uint16_t*>(p.query.data) + b * p.query.stride_batch +
                        head * p.query.stride_head + static_cast<long>(row) * p.query.stride_seq + 16 * h;
#pragma unroll
  for (int c = 0; c < D / 32; ++c) {
    raw[2 * c] = load_untracked(src + 32 * c);
    raw[2 * c + 1] = load_untracked(src + 32 * c + 8);
  }
}

// Part 2, after the wait: the wave's 32-row query block quantised in registers exactly as the
// prep kernel does it (sage/reference.py:61-77: one scale amax / 127 + 1e-7 over the
// zero-padded 32 x D block, codes round-half-even(x / scale) clamped to +-127).  The block amax
// is a wave-wide max; the 16 codes of each chunk are packed in element order, the layout of
// the prepared code rows.  Returns the scale.
template <int D>
__device__ __forceinline__ float quantize_query_block(const AttnParams& p, int q0, int n, const v4i (&raw)[D / 16],
                                                     v4i (&qf)[D / 32]) {
  constexpr int kChunksD = D / 32;
  const bool valid = q0 + n < p.query_length;
  float f[2 * kChunksD][8];
#pragma unroll
  for (int i = 0; i < 2 * kChunksD; ++i) {
    const uint4 bits = valid ? make_uint4(raw[i].x, raw[i].y, raw[i].z, raw[i].w) : make_uint4(0, 0, 0, 0);
    if (p.query_bf16) widen8<true>(bits, f[i]);
    else widen8<false>(bits, f[i]);
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 2 * kChunksD; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(f[i][e]));
  amax = wave_max(amax);
  const float scale = scale_from_amax(amax);
  const Divisor divisor(scale);
#pragma unroll
  for (int c = 0; c < kChunksD; ++c) {
    uint32_t w[4];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      uint32_t code[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) code[e] = code_word(f[2 * c + half][e], divisor);
      w[2 * half] = pack_low_bytes(code[0], code[1], code[2], code[3]);
      w[2 * half + 1] = pack_low_bytes(code[4], code[5], code[6], code[7]);
    }
    qf[c] = v4i{static_cast<int>(w[0]), static_cast<int>(w[1]), static_cast<int>(w[2]), static_cast<int>(w[3])};
  }
  return scale;
}

// Integer scores S^T = K Q^T of one 64-key block: s[0] keys 0..31, s[1] keys 32..63 (each
// lane: its query column, keys 16h + r after the K-row permutation).
template <int D, int NW>
__device__ __forceinline__ void block_scores(const char* stage, const v4i (&qf)[D / 32], int h, int krow,
                                             const v16i& bias, v16i (&s)[2]) {
  using L = TileLayout<D, NW>;
  // accumulators start from the bias: |K Q^T| <= D * 128 * 128 < 2^22, so each result reads as
  // FP32 1.5 * 2^23 + score exactly
  s[0] = s[1] = bias;
#pragma unroll
  for (int c = 0; c < D / 32; ++c) {
    const char* kb = stage + 32 * c + 16 * h;
    const v4i a0 = *reinterpret_cast<const v4i*>(kb + krow * L::kKStride);
    const v4i a1 = *reinterpret_cast<const v4i*>(kb + (32 + krow) * L::kKStride);
    s[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, qf[c], s[0], 0, 0, 0);
    s[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, qf[c], s[1], 0, 0, 0);
  }
}

// Online softmax and PV of one 64-key block (block index t, staged at `stage`) for one wave.
template <int D, int NW, bool kCausal>
__device__ __forceinline__ void block_update(const char* stage, const v16i (&s)[2], float ct, int t, int q0, int n,
                                             int h, float (&num)[D / 32][16], float& den, float& mref) {
  using L = TileLayout<D, NW>;
  constexpr int kChunksD = D / 32;

  // ---- shifted scores x = s * c + log2(vs), in-lane over 32 keys, and the block max ----
  const float4* lk4 = reinterpret_cast<const float4*>(stage + L::kLogOffset);
  float x[32];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 la = lk4[4 * h + q];
    const float4 lb = lk4[8 + 4 * h + q];
    x[4 * q + 0] = fmaf(unbias(s[0][4 * q + 0]), ct, la.x);
    x[4 * q + 1] = fmaf(unbias(s[0][4 * q + 1]), ct, la.y);
    x[4 * q + 2] = fmaf(unbias(s[0][4 * q + 2]), ct, la.z);
    x[4 * q + 3] = fmaf(unbias(s[0][4 * q + 3]), ct, la.w);
    x[16 + 4 * q + 0] = fmaf(unbias(s[1][4 * q + 0]), ct, lb.x);
    x[16 + 4 * q + 1] = fmaf(unbias(s[1][4 * q + 1]), ct, lb.y);
    x[16 + 4 * q + 2] = fmaf(unbias(s[1][4 * q + 2]), ct, lb.z);
    x[16 + 4 * q + 3] = fmaf(unbias(s[1][4 * q + 3]), ct, lb.w);
  }
  if constexpr (kCausal) {
    if (t * kKeyBlock + kKeyBlock - 1 > q0) {  // block crosses this wave's diagonal
      const int query = q0 + n;
      const int key_base = t * kKeyBlock + 16 * h;
#pragma unroll
      for (int r = 0; r < 32; ++r) {
        const int key = key_base + (r < 16 ? r : 16 + r);
        if (key > query) x[r] = -__builtin_inff();
      }
    }
  }
  const float mx = cross_half_max(max32(x));

  // ---- lazy rescale of num/den when the block maximum outgrows the reference by 2^8 ----
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

  // ---- e = 255 * vs * p = exp2(x - bm + log2 255), den += sum(p) * beta, UINT8 codes ----
  const bool empty = mx == -__builtin_inff();
  const float beta = empty ? 0.0f : __builtin_amdgcn_exp2f(mx - mref);
  const float shift = empty ? 0.0f : mx - kLog2Of255;
  const float4* iv4 = reinterpret_cast<const float4*>(stage + L::kInvOffset);
  float ps[4] = {0.0f, 0.0f, 0.0f, 0.0f};
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
    ps[0] = fmaf(e0, ia.x, ps[0]);
    ps[1] = fmaf(e1, ia.y, ps[1]);
    ps[2] = fmaf(e2, ia.z, ps[2]);
    ps[3] = fmaf(e3, ia.w, ps[3]);
    ps[0] = fmaf(f0, ib.x, ps[0]);
    ps[1] = fmaf(f1, ib.y, ps[1]);
    ps[2] = fmaf(f2, ib.z, ps[2]);
    ps[3] = fmaf(f3, ib.w, ps[3]);
    pw[q] = pack_codes(e0, e1, e2, e3);
    pw[4 + q] = pack_codes(f0, f1, f2, f3);
  }
  const float psum = cross_half_sum((ps[0] + ps[1]) + (ps[2] + ps[3]));
  den = fmaf(psum, beta, den);
  const float weight = beta * (1.0f / 255.0f);
  const v4i p0 = {static_cast<int>(pw[0]), static_cast<int>(pw[1]), static_cast<int>(pw[2]), static_cast<int>(pw[3])};
  const v4i p1 = {static_cast<int>(pw[4]), static_cast<int>(pw[5]), static_cast<int>(pw[6]), static_cast<int>(pw[7])};

  // ---- numerator: O^T += (V^T (u - 128) + 128 colsum) * beta / 255 ----
  const v4i* corr4 = reinterpret_cast<const v4i*>(stage + L::kCorrOffset);
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
    const char* vrow = stage + L::kKBytes + (32 * j + n) * L::kVStride + 16 * h;
    const v4i a0 = *reinterpret_cast<const v4i*>(vrow);
    const v4i a1 = *reinterpret_cast<const v4i*>(vrow + 32);
    acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, p0, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, p1, acc, 0, 0, 0);
    // acc started from the biased correction: its bits are 1.5 * 2^23 + (u @ v) exactly.
#pragma unroll
    for (int r = 0; r < 16; ++r) num[j][r] = fmaf(unbias(acc[r]), weight, num[j][r]);
  }
}

// LDS ring of kStages tile records.  Iteration t consumes block t (stage t % kStages), issues
// the QK MFMAs of block t + 1 first so they run under the softmax VALU work, and starts the
// direct copy of block t + kLead.  A workgroup barrier follows every second iteration; the
// barrier after iteration i waits for every copy issued before iteration i.  With 6 stages
// and a lead of 4: a copy issued at iteration t is complete and published by the barrier
// after iteration t + 1 or t + 2, before its first read (QK at iteration t + kLead - 1), and
// the stage it overwrites was last read at iteration t - 2, before the barrier after t - 2
// or t - 1.
constexpr int kStages = 6;
constexpr int kLead = 4;

template <int D, int NW, bool kCausal, bool kBarrier>
__device__ __forceinline__ void pipeline_step(const AttnParams& p, char* smem, int t, int tiles, int wave_tiles, int bh,
                                              int wave, int lane, const v4i (&qf)[D / 32], float cq,
                                              int q0, int n, int h, int krow, const v16i& bias,
                                              const v16i (&s_cur)[2], v16i (&s_next)[2], float (&num)[D / 32][16],
                                              float& den, float& mref) {
  using L = TileLayout<D, NW>;
  // unconditional (clamped) so every iteration issues the same number of copies; a clamped
  // copy lands in a stage no iteration reads before it is written again
  copy_block<D, NW>(p, smem + ((t + kLead) % kStages) * L::kStageBytes, bh, min(t + kLead, tiles - 1), wave, lane);
  if (t < wave_tiles) {
    block_scores<D, NW>(smem + ((t + 1) % kStages) * L::kStageBytes, qf, h, krow, bias, s_next);  // unused past the end
    const char* stage = smem + (t % kStages) * L::kStageBytes;
    const float key_scale = *reinterpret_cast<const float*>(stage + D);  // K scale in row 0's padding
    block_update<D, NW, kCausal>(stage, s_cur, cq * key_scale, t, q0, n, h, num, den, mref);
  }
  if constexpr (kBarrier) stage_barrier_keep_last<D, NW>(wave);
}

template <int D, int NW, bool kCausal, int kOut>
__global__ void __launch_bounds__(NW * 64, 1) attention_kernel(const AttnParams p) {
  using L = TileLayout<D, NW>;
  constexpr int kChunksD = D / 32;
  __shared__ __attribute__((aligned(16))) char smem[kStages * L::kStageBytes];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5;  // lane half
  const int n = lane & 31;  // query column within the wave
  const int logical = p.xcd_remap ? xcd_remap(blockIdx.x, gridDim.x) : static_cast<int>(blockIdx.x);
  // causal: the longest query tiles (most key blocks) are dispatched first
  // wave-uniform in SGPRs (the runtime division is VALU code): per-block key scales then come
  // from scalar loads, which do not share the vmcnt counter with the direct LDS copies
  const int bh = __builtin_amdgcn_readfirstlane(logical / p.query_tiles);
  const int qtile_fwd = __builtin_amdgcn_readfirstlane(logical - bh * p.query_tiles);
  const int qtile = kCausal && !p.causal_forward ? p.query_tiles - 1 - qtile_fwd : qtile_fwd;
  const int q0 = qtile * (NW * 32) + wave * 32;  // first query of this wave
  const bool wave_live = q0 < p.query_length;

  int tiles = p.nkb;
  int wave_tiles = wave_live ? p.nkb : 0;
  if constexpr (kCausal) {
    const int last_query = min(p.query_length, (qtile + 1) * NW * 32) - 1;
    tiles = last_query / kKeyBlock + 1;
    wave_tiles = wave_live ? (min(p.query_length, q0 + 32) - 1) / kKeyBlock + 1 : 0;
  }

  // Q^T fragments (B operand): query q0 + n, bytes [32c + 16h, +16) of each 32-dim chunk.
  v4i qf[kChunksD];
  float cq = 0.0f;
  const bool fused_live = p.fused_query && wave_live;
  v4i raw[D / 16];
  if (fused_live) issue_query_loads<D>(p, bh, q0, n, h, raw);
  if (!p.fused_query && q0 < p.sq32) {
    const int8_t* qrow = p.query_code + (static_cast<long>(bh) * p.sq32 + q0 + n) * D + 16 * h;
#pragma unroll
    for (int c = 0; c < kChunksD; ++c) qf[c] = *reinterpret_cast<const v4i*>(qrow + 32 * c);
    cq = p.query_scale[static_cast<long>(bh) * p.nqb + (q0 >> 5)] * p.scale_log2e;
    // Settle the prepared Q loads inside this branch: a load the compiler still counts as
    // pending at the loop header would get its wait (in-order vmcnt, so a wait for all direct
    // LDS copies in flight) inside every iteration, and a wait at the join would also drain
    // the untracked query loads of the fused path.
#pragma unroll
    for (int c = 0; c < kChunksD; ++c) asm volatile("" ::"v"(qf[c]));
    asm volatile("" ::"v"(cq));
  } else {
#pragma unroll
    for (int c = 0; c < kChunksD; ++c) qf[c] = v4i{0, 0, 0, 0};
  }

  // prologue copies: blocks 0 .. kLead-1 (missing blocks repeat the last one)
#pragma unroll
  for (int b = 0; b < kLead; ++b) copy_block<D, NW>(p, smem + b * L::kStageBytes, bh, min(b, tiles - 1), wave, lane);

  if (fused_live) {
    // wait for the query loads only (issued before this wave's kLead * kRounds or
    // kLead * (kRounds - 1) copies), then quantise while the copies land
    if (wave < L::kFullWaves)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLead * L::kRounds) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLead * (L::kRounds - 1)) : "memory");
#pragma unroll
    for (int i = 0; i < D / 16; ++i) asm volatile("" : "+v"(raw[i]));
    cq = quantize_query_block<D>(p, q0, n, raw, qf) * p.scale_log2e;
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

  stage_barrier<0>();  // all prologue copies landed

  // QK accumulator bias, kept in registers for the whole loop (opaque, so not rematerialised)
  v16i bias = {kAccBias, kAccBias, kAccBias, kAccBias, kAccBias, kAccBias, kAccBias, kAccBias,
               kAccBias, kAccBias, kAccBias, kAccBias, kAccBias, kAccBias, kAccBias, kAccBias};
  asm volatile("" : "+v"(bias));
  v16i s_a[2], s_b[2];  // scores of the current and the next block, alternating
  if (wave_tiles > 0) block_scores<D, NW>(smem, qf, h, krow, bias, s_a);

  // unrolled by two so both score sets keep static names; one barrier per pair
  int t = 0;
  for (; t + 1 < tiles; t += 2) {
    pipeline_step<D, NW, kCausal, false>(p, smem, t, tiles, wave_tiles, bh, wave, lane, qf, cq, q0, n, h,
                                         krow, bias, s_a, s_b, num, den, mref);
    pipeline_step<D, NW, kCausal, true>(p, smem, t + 1, tiles, wave_tiles, bh, wave, lane, qf, cq, q0, n,
                                        h, krow, bias, s_b, s_a, num, den, mref);
  }
  if (t < tiles)
    pipeline_step<D, NW, kCausal, false>(p, smem, t, tiles, wave_tiles, bh, wave, lane, qf, cq, q0, n, h,
                                         krow, bias, s_a, s_b, num, den, mref);
  // no direct copy may still be writing this workgroup's LDS when its waves end
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

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
