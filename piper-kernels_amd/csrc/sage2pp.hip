// Fused SageAttention2++ forward for gfx950: INT8 MFMA QK^T, FP32 online softmax whose frame
// is shifted by log2(448), FP8 E4M3 probabilities times FP8 E4M3 V on
// v_mfma_f32_32x32x64_f8f6f4, accumulated in FP32 across all key blocks.
//
// Behaviour follows the reference recurrence (jumbledpoophj/piper-kernels 0.2.1,
// src/piper_kernels/attention/sage_attention_2pp/reference.py:58-104; the GPU kernel it
// models is sage_attention_2pp/triton.py:391-510): per 64-key block, bm = max(s) - log2 448,
// m' = max(m, bm), acc = acc * exp2(m - m') + fp8(exp2(s - m')) @ v8, den = den * exp2(m - m')
// + sum(exp2(s - m')), and the epilogue acc * scale_v / max(den, 1e-30).  Scores are in the
// log2 domain (the softmax scale carries log2 e).
//
// By default one arithmetic difference from the reference: its 64-key partial products are
// rounded to FP16 (a model of NVIDIA's FP16-accumulating FP8 MMA, reference.py:95-98).  gfx950's
// FP8 MFMA accumulates in FP32, so the products of every block accumulate in the MFMA's own FP32
// registers, rescaled only when the running maximum moves, and the per-channel V scale is
// applied once at the end.  The kFp16Partials instantiation (PIPER_SAGE_FP16_PARTIALS) keeps the
// reference's rounding: each block's product is formed on its own, rounded to FP16 and added.  This removes all per-block VALU work on the D outputs (the
// reference applies a scale per block): per block and lane, the VALU work is the 32 scores'
// subtraction, max, FMA, exp2, sum and FP8 packing.
//
// Design shared with the Piper Attention kernel (stream.h): one workgroup = NW waves x 32
// queries of one head; S^T = K Q^T with K rows loaded in a permuted order, so each lane owns
// one query and keys {16h .. 16h+15} and {32+16h .. 32+16h+15} of every block -- which, packed
// in that order, is directly the B operand of the FP8 MFMA (which contracts over any key order
// the A operand shares: V^T rows are read at bytes [16h, +16) and [32 + 16h, +16)); the query
// is quantised in the prologue; tile records are copied straight into an LDS ring (two stages per
// workgroup with three workgroups per CU, the default; four or six in the two-waves-per-SIMD plans).
#include "common.h"
#include "kernels.h"
#include "quant.h"
#include "stream.h"

namespace piper {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr float kLog2Of448 = 8.807354922057604f;  // log2(448): probabilities are born in [0, 448]

template <int D, int NW>
struct SageLayout : StagePieces<sage_tile_bytes(D), NW> {  // the tile record is the stage image
  static constexpr int kKStride = kv_k_stride(D);   // bytes per K row in LDS
  static constexpr int kVStride = kv_v_stride();    // bytes per V^T row in LDS
  static constexpr int kVOffset = sage_v_offset(D);
};

// Online softmax and PV of one 64-key block (block index t, staged at `stage`) for one wave,
// in two parts.  Head: raw scores, masks, block maximum and the frame move (rescale of the
// accumulators when the running maximum grows; exact, otherwise the weight is 1).  Tail:
// probabilities, denominator share, FP8 codes and the PV MFMAs.  ct[g] = query scale * key scale
// * softmax scale * log2 e for the keys of K thread group g (keys k with (k % 8) / 2 == g; all
// four equal for per-block K scales); register 4q + i holds key 16h + 4q + i (or 32 + ...), so
// it belongs to group 2 (q % 2) + i / 2.  mrun is the running maximum (log2 units, per query),
// den this lane half's share of the denominator; x carries the raw scores from head to tail.
template <int D, bool kCausal, bool kPerThread>
__device__ __forceinline__ void sage_block_head(const v16i (&s)[2], const float (&ct)[4], int t, int q0, int n,
                                                int h, int key_length, float (&x)[32], v16f (&acc)[D / 32],
                                                float& den, float& mrun) {
  constexpr int kChunksD = D / 32;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    x[r] = unbias_score(s[0][r]);
    x[16 + r] = unbias_score(s[1][r]);
  }
  // Both masks are scalar branches taken by one tile (and the diagonal tiles); the empty asm
  // keeps the compiler from speculating them into per-element compares in every block.
  if (t * kKeyBlock + kKeyBlock > key_length) {  // the last tile: its padding keys score -inf
    asm volatile("");
    const int key_base = t * kKeyBlock + 16 * h;
#pragma unroll
    for (int r = 0; r < 32; ++r) {
      const int key = key_base + (r < 16 ? r : 16 + r);
      if (key >= key_length) x[r] = -__builtin_inff();
    }
  }
  if constexpr (kCausal) {
    if (t * kKeyBlock + kKeyBlock - 1 > q0) {  // block crosses this wave's diagonal
      asm volatile("");
      const int query = q0 + n;
      const int key_base = t * kKeyBlock + 16 * h;
#pragma unroll
      for (int r = 0; r < 32; ++r) {
        const int key = key_base + (r < 16 ? r : 16 + r);
        if (key > query) x[r] = -__builtin_inff();
      }
    }
  }
  // ct > 0, so the maximum commutes with the scaling: max(RN(x ct)) = RN(max(x) ct) -- per K
  // thread group when the groups have their own scales
  float block_max;
  if constexpr (kPerThread) {
    float gmax[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int r = 4 * (g >> 1) + 2 * (g & 1);  // registers r, r+1, r+8, r+9 of each half
      gmax[g] = cross_half_max(fmaxf(fmaxf(fmaxf(x[r], x[r + 1]), fmaxf(x[r + 8], x[r + 9])),
                                     fmaxf(fmaxf(x[16 + r], x[17 + r]), fmaxf(x[24 + r], x[25 + r]))));
    }
    block_max = fmaxf(fmaxf(gmax[0] * ct[0], gmax[1] * ct[1]), fmaxf(gmax[2] * ct[2], gmax[3] * ct[3])) -
                kLog2Of448;
  } else {
    block_max = cross_half_max(max32(x)) * ct[0] - kLog2Of448;
  }
  const float next = fmaxf(mrun, block_max);
  const bool grow = next > mrun;
  if (__builtin_amdgcn_ballot_w64(grow) != 0) {
    const float w = grow ? __builtin_amdgcn_exp2f(mrun - next) : 1.0f;  // exp2(-inf) = 0 at the start
#pragma unroll
    for (int j = 0; j < kChunksD; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][r] *= w;
    den *= w;
    mrun = next;
  }
}

template <int D, int NW, bool kFp16Partials>
__device__ __forceinline__ void sage_block_tail(const char* stage, const float (&x)[32], const float (&ct)[4], int n,
                                                int h, v16f (&acc)[D / 32], float& den, float mrun) {
  using L = SageLayout<D, NW>;
  constexpr int kChunksD = D / 32;
  // ---- p = exp2(s ct - m') in [0, 448], the denominator share and the FP8 codes ----
  float ps[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  uint32_t pw[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const float c01 = ct[2 * (q & 1)], c23 = ct[2 * (q & 1) + 1];
    const float e0 = __builtin_amdgcn_exp2f(fmaf(x[4 * q + 0], c01, -mrun));
    const float e1 = __builtin_amdgcn_exp2f(fmaf(x[4 * q + 1], c01, -mrun));
    const float e2 = __builtin_amdgcn_exp2f(fmaf(x[4 * q + 2], c23, -mrun));
    const float e3 = __builtin_amdgcn_exp2f(fmaf(x[4 * q + 3], c23, -mrun));
    ps[0] += e0;
    ps[1] += e1;
    ps[2] += e2;
    ps[3] += e3;
    pw[q] = pack_fp8(e0, e1, e2, e3);
  }
  den += (ps[0] + ps[1]) + (ps[2] + ps[3]);
  const v8i p = {static_cast<int>(pw[0]), static_cast<int>(pw[1]), static_cast<int>(pw[2]), static_cast<int>(pw[3]),
                 static_cast<int>(pw[4]), static_cast<int>(pw[5]), static_cast<int>(pw[6]), static_cast<int>(pw[7])};

  // ---- O^T += V^T P^T on the FP8 MFMA, accumulating in FP32 (with kFp16Partials, the block's
  // 64-key product is formed on its own and rounded to FP16 before it is added: the reference's
  // partial.to(float16), reference.py:95-98; |partial| <= 64 * 448 * 2.25 < 65504) ----
#pragma unroll
  for (int j = 0; j < kChunksD; ++j) {
    const char* vrow = stage + L::kVOffset + (32 * j + n) * L::kVStride + 16 * h;
    const v4i a0 = *reinterpret_cast<const v4i*>(vrow);
    const v4i a1 = *reinterpret_cast<const v4i*>(vrow + 32);
    const v8i a = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
    if constexpr (kFp16Partials) {
      const v16f zero = {};
      const v16f part = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, p, zero, 0, 0, 0, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][r] += static_cast<float>(static_cast<_Float16>(part[r]));
    } else {
      acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, p, acc[j], 0, 0, 0, 0, 0, 0);
    }
  }
}

template <int D, int NW, bool kCausal, bool kPerThread, bool kFp16Partials, bool kBarrier>
__device__ __forceinline__ void sage_step(const SageParams& p, char* smem, int t, int tiles, int wave_tiles, int bh,
                                          int wave, int lane, const v4i (&qf)[D / 32], float cq, int q0, int n,
                                          int h, int krow, const v16i (&s_cur)[2],
                                          v16i (&s_next)[2], v16f (&acc)[D / 32], float& den, float& mrun) {
  using L = SageLayout<D, NW>;
  using R = Ring<NW>;  // the Piper Attention kernel's ring (stream.h)
  copy_block<L>(p, smem + ((t + R::kLead) % R::kStages) * L::kStageBytes, bh, min(t + R::kLead, tiles - 1), wave,
                lane);
  if (t < wave_tiles) {
    const char* stage = smem + (t % R::kStages) * L::kStageBytes;
    // the K scales of the tile's four thread groups sit in the padding of K row 0
    float ct[4];
    if constexpr (kPerThread) {
      const float4 ks = *reinterpret_cast<const float4*>(stage + D);
      ct[0] = cq * ks.x;
      ct[1] = cq * ks.y;
      ct[2] = cq * ks.z;
      ct[3] = cq * ks.w;
    } else {
      ct[0] = ct[1] = ct[2] = ct[3] = cq * *reinterpret_cast<const float*>(stage + D);
    }
    float x[32];
    // the next block's QK MFMAs first: they run under this block's softmax (issuing them after
    // the frame move, or interleaving them with the softmax, measured 1-5% slower; feeding the
    // biased accumulator bits to the exp FMA with a folded constant saves the 32 subtractions
    // but costs register copies and measured 3% slower)
    block_scores<D, L>(smem + ((t + 1) % R::kStages) * L::kStageBytes, qf, h, krow, s_next);
    sage_block_head<D, kCausal, kPerThread>(s_cur, ct, t, q0, n, h, p.key_length, x, acc, den, mrun);
    sage_block_tail<D, NW, kFp16Partials>(stage, x, ct, n, h, acc, den, mrun);
  }
  if constexpr (kBarrier) stage_barrier_keep_last<L>(wave);
}

template <int D, int NW, bool kCausal, int kOut, bool kPerThread, bool kFp16Partials>
__global__ void __launch_bounds__(NW * 64, 8 / NW) sage_attention_kernel(const SageParams p) {
  using L = SageLayout<D, NW>;
  using R = Ring<NW>;
  constexpr int kChunksD = D / 32;
  constexpr int kSageLead = R::kLead;
  __shared__ __attribute__((aligned(16))) char smem[R::kStages * L::kStageBytes];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5;
  const int n = lane & 31;
  // wave-uniform in SGPRs (the runtime division is VALU code): per-block key scales then come
  // from scalar loads, which do not share the vmcnt counter with the direct LDS copies
  const TileCoord tc = workgroup_tile<kCausal>(p);
  const int bh = __builtin_amdgcn_readfirstlane(tc.bh);
  const int qtile = __builtin_amdgcn_readfirstlane(tc.qtile);
  const int q0 = qtile * (NW * 32) + wave * 32;
  const bool wave_live = q0 < p.query_length;

  int tiles = p.nkb;
  int wave_tiles = wave_live ? p.nkb : 0;
  if constexpr (kCausal) {
    const int last_query = min(p.query_length, (qtile + 1) * NW * 32) - 1;
    tiles = last_query / kKeyBlock + 1;
    wave_tiles = wave_live ? (min(p.query_length, q0 + 32) - 1) / kKeyBlock + 1 : 0;
  }

  // query loads first (untracked), then the prologue copies, then a wait for the query only
  v4i raw[D / 16];
  if (wave_live) issue_query_loads<D>(p, bh, q0, n, h, raw);
#pragma unroll
  for (int b = 0; b < kSageLead; ++b) copy_block<L>(p, smem + b * L::kStageBytes, bh, min(b, tiles - 1), wave, lane);
  v4i qf[kChunksD];
  float cq = 0.0f;
  if (wave_live) {
    if (wave < L::kFullWaves)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kSageLead * L::kRounds) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kSageLead * (L::kRounds - 1)) : "memory");
#pragma unroll
    for (int i = 0; i < D / 16; ++i) asm volatile("" : "+v"(raw[i]));
    cq = quantize_query_block<D, kPerThread>(p, q0, n, raw, qf) * (p.scale_log2e * kScoreUnit);
  } else {
#pragma unroll
    for (int c = 0; c < kChunksD; ++c) qf[c] = v4i{0, 0, 0, 0};
  }

  v16f acc[kChunksD];
#pragma unroll
  for (int j = 0; j < kChunksD; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
  float den = 0.0f;
  float mrun = -__builtin_inff();
  const int krow = 16 * ((n >> 2) & 1) + 4 * (n >> 3) + (n & 3);

  stage_barrier<0>();  // all prologue copies landed

  v16i s_a[2], s_b[2];
  if (wave_tiles > 0) block_scores<D, L>(smem, qf, h, krow, s_a);

  int t = 0;
  for (; t + 1 < tiles; t += 2) {
    if constexpr (!kCausal) progress_priority(t, 2, tiles);  // causal: workgroups differ in length
    sage_step<D, NW, kCausal, kPerThread, kFp16Partials, R::kEveryIteration>(
        p, smem, t, tiles, wave_tiles, bh, wave, lane, qf, cq, q0, n, h, krow, s_a, s_b, acc, den, mrun);
    sage_step<D, NW, kCausal, kPerThread, kFp16Partials, true>(p, smem, t + 1, tiles, wave_tiles, bh, wave, lane, qf, cq,
                                                               q0, n, h, krow, s_b, s_a, acc, den, mrun);
  }
  if (t < tiles)
    sage_step<D, NW, kCausal, kPerThread, kFp16Partials, false>(p, smem, t, tiles, wave_tiles, bh, wave, lane, qf, cq, q0,
                                                                n, h, krow, s_a, s_b, acc, den, mrun);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no copy may outlive the waves

  // ---- epilogue: acc * scale_v / max(den, 1e-30); lane (n, h) holds rows d = 32j + 8g + 4h + i ----
  const float total = cross_half_sum(den);
  const int query = q0 + n;
  if (!wave_live || query >= p.query_length) return;
  const float rden = 1.0f / fmaxf(total, 1e-30f);
  const float* vscale = p.value_scale + static_cast<long>(bh) * D;
  const long out_row = (static_cast<long>(bh) * p.query_length + query) * D;
#pragma unroll
  for (int j = 0; j < kChunksD; ++j) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * j + 8 * g + 4 * h;
      const float4 vs = *reinterpret_cast<const float4*>(vscale + d0);
      store4<kOut>(p.output, out_row + d0, (acc[j][4 * g + 0] * vs.x) * rden, (acc[j][4 * g + 1] * vs.y) * rden,
                   (acc[j][4 * g + 2] * vs.z) * rden, (acc[j][4 * g + 3] * vs.w) * rden);
    }
  }
}

// Three 4-wave workgroups per CU (three waves per SIMD, each from another workgroup), as Piper
// Attention's attention_w3_kernel: a 2-stage LDS ring per workgroup and no score look-ahead, to
// fit 168 VGPRs.  Iteration t: wait for this wave's copies of tile t, barrier (every copy of
// tile t landed, every read of tile t - 1 done), start the copy of tile t + 1 into the stage
// tile t - 1 used, then the scores, head and tail of tile t.  Same per-block arithmetic as
// sage_attention_kernel, in the same order, so the output is bit-identical to the other plans.
template <int D, bool kCausal, int kOut, bool kPerThread, bool kFp16Partials>
__global__ void __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(3, 3)))
sage_attention_w3_kernel(const SageParams p) {
  constexpr int NW = 4;
  using L = SageLayout<D, NW>;
  constexpr int kChunksD = D / 32;
  __shared__ __attribute__((aligned(16))) char smem[2 * L::kStageBytes];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5;
  const int n = lane & 31;
  const TileCoord tc = workgroup_tile<kCausal>(p);
  const int bh = __builtin_amdgcn_readfirstlane(tc.bh);
  const int qtile = __builtin_amdgcn_readfirstlane(tc.qtile);
  const int q0 = qtile * (NW * 32) + wave * 32;
  const bool wave_live = q0 < p.query_length;

  int tiles = p.nkb;
  int wave_tiles = wave_live ? p.nkb : 0;
  if constexpr (kCausal) {
    const int last_query = min(p.query_length, (qtile + 1) * NW * 32) - 1;
    tiles = last_query / kKeyBlock + 1;
    wave_tiles = wave_live ? (min(p.query_length, q0 + 32) - 1) / kKeyBlock + 1 : 0;
  }

  // query loads first (untracked), then the copies of tile 0, then a wait for the query only
  v4i raw[D / 16];
  if (wave_live) issue_query_loads<D>(p, bh, q0, n, h, raw);
  copy_block<L>(p, smem, bh, 0, wave, lane);
  v4i qf[kChunksD];
  float cq = 0.0f;
  if (wave_live) {
    if (wave < L::kFullWaves)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(L::kRounds) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(L::kRounds - 1) : "memory");
#pragma unroll
    for (int i = 0; i < D / 16; ++i) asm volatile("" : "+v"(raw[i]));
    cq = quantize_query_block<D, kPerThread>(p, q0, n, raw, qf) * (p.scale_log2e * kScoreUnit);
  } else {
#pragma unroll
    for (int c = 0; c < kChunksD; ++c) qf[c] = v4i{0, 0, 0, 0};
  }

  v16f acc[kChunksD];
#pragma unroll
  for (int j = 0; j < kChunksD; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
  float den = 0.0f;
  float mrun = -__builtin_inff();
  const int krow = 16 * ((n >> 2) & 1) + 4 * (n >> 3) + (n & 3);

  for (int t = 0; t < tiles; ++t) {
    if constexpr (!kCausal) progress_priority(t, 1, tiles);  // causal: workgroups differ in length
    stage_barrier<0>();
    if (t + 1 < tiles) copy_block<L>(p, smem + ((t + 1) & 1) * L::kStageBytes, bh, t + 1, wave, lane);
    if (t < wave_tiles) {
      const char* stage = smem + (t & 1) * L::kStageBytes;
      v16i sc[2];
      block_scores<D, L>(stage, qf, h, krow, sc);
      float ct[4];
      if constexpr (kPerThread) {
        const float4 ks = *reinterpret_cast<const float4*>(stage + D);
        ct[0] = cq * ks.x;
        ct[1] = cq * ks.y;
        ct[2] = cq * ks.z;
        ct[3] = cq * ks.w;
      } else {
        ct[0] = ct[1] = ct[2] = ct[3] = cq * *reinterpret_cast<const float*>(stage + D);
      }
      float x[32];
      sage_block_head<D, kCausal, kPerThread>(sc, ct, t, q0, n, h, p.key_length, x, acc, den, mrun);
      sage_block_tail<D, NW, kFp16Partials>(stage, x, ct, n, h, acc, den, mrun);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no copy may outlive the waves

  const float total = cross_half_sum(den);
  const int query = q0 + n;
  if (!wave_live || query >= p.query_length) return;
  const float rden = 1.0f / fmaxf(total, 1e-30f);
  const float* vscale = p.value_scale + static_cast<long>(bh) * D;
  const long out_row = (static_cast<long>(bh) * p.query_length + query) * D;
#pragma unroll
  for (int j = 0; j < kChunksD; ++j) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * j + 8 * g + 4 * h;
      const float4 vs = *reinterpret_cast<const float4*>(vscale + d0);
      store4<kOut>(p.output, out_row + d0, (acc[j][4 * g + 0] * vs.x) * rden, (acc[j][4 * g + 1] * vs.y) * rden,
                   (acc[j][4 * g + 2] * vs.z) * rden, (acc[j][4 * g + 3] * vs.w) * rden);
    }
  }
}

template <int D, int NW, bool kCausal, bool kPerThread, bool kFp16Partials>
static hipError_t sage_launch_out(int out_dtype, const SageParams& sp, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(sp.query_tiles * sp.batch_heads));
  if constexpr (NW == 3) {  // three 4-wave workgroups per CU
    const dim3 block(256);
    switch (out_dtype) {
      case 0:
        hipLaunchKernelGGL((sage_attention_w3_kernel<D, kCausal, 0, kPerThread, kFp16Partials>), grid, block, 0, stream, sp);
        break;
      case 1:
        hipLaunchKernelGGL((sage_attention_w3_kernel<D, kCausal, 1, kPerThread, kFp16Partials>), grid, block, 0, stream, sp);
        break;
      default:
        hipLaunchKernelGGL((sage_attention_w3_kernel<D, kCausal, 2, kPerThread, kFp16Partials>), grid, block, 0, stream, sp);
        break;
    }
    return hipGetLastError();
  } else {
    const dim3 block(NW * 64);
    switch (out_dtype) {
      case 0:
        hipLaunchKernelGGL((sage_attention_kernel<D, NW, kCausal, 0, kPerThread, kFp16Partials>), grid, block, 0, stream,
                           sp);
        break;
      case 1:
        hipLaunchKernelGGL((sage_attention_kernel<D, NW, kCausal, 1, kPerThread, kFp16Partials>), grid, block, 0, stream,
                           sp);
        break;
      default:
        hipLaunchKernelGGL((sage_attention_kernel<D, NW, kCausal, 2, kPerThread, kFp16Partials>), grid, block, 0, stream,
                           sp);
        break;
    }
    return hipGetLastError();
  }
}

template <int D, int NW, bool kCausal, bool kPerThread>
static hipError_t sage_launch_partials(int out_dtype, const SageParams& sp, hipStream_t stream) {
  return sp.fp16_partials ? sage_launch_out<D, NW, kCausal, kPerThread, true>(out_dtype, sp, stream)
                          : sage_launch_out<D, NW, kCausal, kPerThread, false>(out_dtype, sp, stream);
}

template <int D, int NW, bool kCausal>
static hipError_t sage_launch_granularity(int out_dtype, const SageParams& sp, hipStream_t stream) {
  return sp.per_thread ? sage_launch_partials<D, NW, kCausal, true>(out_dtype, sp, stream)
                       : sage_launch_partials<D, NW, kCausal, false>(out_dtype, sp, stream);
}

template <int D, int NW>
static hipError_t sage_launch_causal(bool causal, int out_dtype, const SageParams& sp, hipStream_t stream) {
  return causal ? sage_launch_granularity<D, NW, true>(out_dtype, sp, stream)
                : sage_launch_granularity<D, NW, false>(out_dtype, sp, stream);
}

hipError_t launch_sage_attention(int head_dim, bool causal, int out_dtype, int waves, const SageParams& sp,
                                 hipStream_t stream) {
  // waves: 8 or 4 query waves per workgroup with two waves per SIMD, or 3 for three 4-wave
  // workgroups per CU (sage_attention_w3_kernel)
  if (head_dim == 128) {
    return waves == 3   ? sage_launch_causal<128, 3>(causal, out_dtype, sp, stream)
           : waves == 4 ? sage_launch_causal<128, 4>(causal, out_dtype, sp, stream)
                        : sage_launch_causal<128, 8>(causal, out_dtype, sp, stream);
  }
  return waves == 3   ? sage_launch_causal<64, 3>(causal, out_dtype, sp, stream)
         : waves == 4 ? sage_launch_causal<64, 4>(causal, out_dtype, sp, stream)
                      : sage_launch_causal<64, 8>(causal, out_dtype, sp, stream);
}

}  // namespace piper
