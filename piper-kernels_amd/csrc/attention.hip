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
  static_assert(kChunks * 16 == kv_tile_bytes(D), "LDS stage order must match the tile record");
};

// Global -> register -> LDS staging of one 64-key block: kRounds 16-byte chunks per thread.
// Branch-free on purpose: a per-lane branch around a load makes the compiler wait for it at
// the reconvergence point, which would serialise the prefetch.  Threads past the last chunk
// load and store the last chunk again (identical data, benign).
template <int D, int NW>
struct Staging {
  using L = TileLayout<D, NW>;
  static constexpr int kRounds = (L::kChunks + L::kThreads - 1) / L::kThreads;
};

template <int D, int NW>
__device__ __forceinline__ int staging_chunk(int r) {
  using L = TileLayout<D, NW>;
  const int c = threadIdx.x + r * L::kThreads;
  return c < L::kChunks ? c : L::kChunks - 1;
}

// Loads the tile record of block t (t must be a valid block index): a uniform base address
// plus a loop-invariant per-thread offset, so the loop spends no VALU on addressing.
template <int D, int NW>
__device__ __forceinline__ void fetch_block(const AttnParams& p, int bh, int t,
                                            v4i (&reg)[Staging<D, NW>::kRounds]) {
  const v4i* tile = reinterpret_cast<const v4i*>(p.kv_tiles + (static_cast<long>(bh) * p.nkb + t) * kv_tile_bytes(D));
#pragma unroll
  for (int r = 0; r < Staging<D, NW>::kRounds; ++r) reg[r] = tile[staging_chunk<D, NW>(r)];
}

template <int D, int NW>
__device__ __forceinline__ void store_block(char* stage, const v4i (&reg)[Staging<D, NW>::kRounds]) {
  using L = TileLayout<D, NW>;
#pragma unroll
  for (int r = 0; r < Staging<D, NW>::kRounds; ++r) {
    const int i = staging_chunk<D, NW>(r);
    const int j = i - L::kChunksK;
    const int k_dst = (i / (D / 16)) * L::kKStride + (i % (D / 16)) * 16;
    const int v_dst = L::kKBytes + (j >> 2) * L::kVStride + (j & 3) * 16;
    const int x_dst = L::kLogOffset + (j - L::kChunksV) * 16;  // log2, inv and corr are contiguous
    const int dst = i < L::kChunksK ? k_dst : j < L::kChunksV ? v_dst : x_dst;
    *reinterpret_cast<v4i*>(stage + dst) = reg[r];
  }
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

// Integer scores S^T = K Q^T of one 64-key block: s[0] keys 0..31, s[1] keys 32..63 (each
// lane: its query column, keys 16h + r after the K-row permutation).
template <int D, int NW>
__device__ __forceinline__ void block_scores(const char* stage, const v4i (&qf)[D / 32], int h, int krow,
                                             v16i (&s)[2]) {
  using L = TileLayout<D, NW>;
  s[0] = s[1] = v16i{};
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
    x[4 * q + 0] = fmaf(static_cast<float>(s[0][4 * q + 0]), ct, la.x);
    x[4 * q + 1] = fmaf(static_cast<float>(s[0][4 * q + 1]), ct, la.y);
    x[4 * q + 2] = fmaf(static_cast<float>(s[0][4 * q + 2]), ct, la.z);
    x[4 * q + 3] = fmaf(static_cast<float>(s[0][4 * q + 3]), ct, la.w);
    x[16 + 4 * q + 0] = fmaf(static_cast<float>(s[1][4 * q + 0]), ct, lb.x);
    x[16 + 4 * q + 1] = fmaf(static_cast<float>(s[1][4 * q + 1]), ct, lb.y);
    x[16 + 4 * q + 2] = fmaf(static_cast<float>(s[1][4 * q + 2]), ct, lb.z);
    x[16 + 4 * q + 3] = fmaf(static_cast<float>(s[1][4 * q + 3]), ct, lb.w);
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
    // (The element goes through a scalar first: this clang's __builtin_bit_cast of an
    // ext_vector subscript reads element 0.)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int bits = acc[r];
      num[j][r] = fmaf(__builtin_bit_cast(float, bits) - kAccBiasValue, weight, num[j][r]);
    }
  }
}

// LDS ring of kStages tile records.  Iteration t consumes block t (stage t % kStages), issues
// the QK MFMAs of block t + 1 first so they run under the softmax VALU work, writes block
// t + kLead (loaded into `ready` one iteration earlier) and starts loading block t + kLead + 1
// into `loading`.  A workgroup barrier follows every second iteration only: with a write lead
// of 3 and 5 stages, every written stage is separated from its first read (QK at iteration
// t + kLead - 1) and from its previous reads (iteration t + kLead - kStages) by a barrier.
constexpr int kStages = 5;
constexpr int kLead = 3;

template <int D, int NW, bool kCausal, bool kBarrier>
__device__ __forceinline__ void pipeline_step(const AttnParams& p, char* smem, int t, int tiles, int wave_tiles, int bh,
                                              const v4i (&qf)[D / 32], float cq, const float* key_scale, int q0,
                                              int n, int h, int krow, const v16i (&s_cur)[2], v16i (&s_next)[2],
                                              float (&num)[D / 32][16], float& den, float& mref,
                                              v4i (&ready)[Staging<D, NW>::kRounds],
                                              v4i (&loading)[Staging<D, NW>::kRounds]) {
  using L = TileLayout<D, NW>;
  // unconditional (clamped) so every iteration issues the same loads: static vmcnt waits
  fetch_block<D, NW>(p, bh, min(t + kLead + 1, tiles - 1), loading);
  if (t < wave_tiles) {
    block_scores<D, NW>(smem + ((t + 1) % kStages) * L::kStageBytes, qf, h, krow, s_next);  // unused past the end
    block_update<D, NW, kCausal>(smem + (t % kStages) * L::kStageBytes, s_cur, cq * key_scale[t], t, q0, n, h, num,
                                 den, mref);
  }
  if (t + kLead < tiles) store_block<D, NW>(smem + ((t + kLead) % kStages) * L::kStageBytes, ready);
  if constexpr (kBarrier) __syncthreads();
}

template <int D, int NW, bool kCausal, int kOut>
__global__ void __launch_bounds__(NW * 64, 1) attention_kernel(const AttnParams p) {
  using L = TileLayout<D, NW>;
  using S = Staging<D, NW>;
  constexpr int kChunksD = D / 32;
  __shared__ __attribute__((aligned(16))) char smem[kStages * L::kStageBytes];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5;  // lane half
  const int n = lane & 31;  // query column within the wave
  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  // causal: the longest query tiles (most key blocks) are dispatched first
  const int qtile = kCausal ? p.query_tiles - 1 - logical % p.query_tiles : logical % p.query_tiles;
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

  // prologue: blocks 0 .. kLead-1 into LDS (missing blocks repeat the last one), block kLead
  // into registers
  v4i reg_a[S::kRounds];
  v4i reg_b[S::kRounds];
#pragma unroll
  for (int b = 0; b < kLead; ++b) {
    fetch_block<D, NW>(p, bh, min(b, tiles - 1), reg_a);
    store_block<D, NW>(smem + b * L::kStageBytes, reg_a);
  }
  fetch_block<D, NW>(p, bh, min(kLead, tiles - 1), reg_a);
  __syncthreads();

  v16i s_a[2], s_b[2];  // scores of the current and the next block, alternating
  if (wave_tiles > 0) block_scores<D, NW>(smem, qf, h, krow, s_a);

  // Iteration t stores the register set loaded at t - 1 and loads into the other one:
  // unrolled by two so both register sets keep static names; one barrier per pair.
  int t = 0;
  for (; t + 1 < tiles; t += 2) {
    pipeline_step<D, NW, kCausal, false>(p, smem, t, tiles, wave_tiles, bh, qf, cq, key_scale, q0, n, h, krow, s_a,
                                         s_b, num, den, mref, reg_a, reg_b);
    pipeline_step<D, NW, kCausal, true>(p, smem, t + 1, tiles, wave_tiles, bh, qf, cq, key_scale, q0, n, h, krow, s_b,
                                        s_a, num, den, mref, reg_b, reg_a);
  }
  if (t < tiles)
    pipeline_step<D, NW, kCausal, false>(p, smem, t, tiles, wave_tiles, bh, qf, cq, key_scale, q0, n, h, krow, s_a,
                                         s_b, num, den, mref, reg_a, reg_b);

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
