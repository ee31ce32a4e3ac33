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
//   copied with direct global -> LDS loads into an LDS ring: two stages, one block ahead, with
//   three workgroups per CU (the default); four or six stages in the two-waves-per-SIMD plans.
#include "common.h"
#include "kernels.h"
#include "quant.h"
#include "stream.h"

namespace piper {

constexpr float kLazyRescale = 8.0f;               // log2 headroom before num/den are rescaled
constexpr float kLog2Of255 = 7.994353436858858f;   // log2(255)
constexpr float kDirectRange = 96.0f;              // |block max| of the subtraction-free exp2 path

template <int D, int NW>
struct TileLayout : StagePieces<kv_tile_bytes(D), NW> {  // the tile record is the stage image
  static constexpr int kKStride = kv_k_stride(D);  // bytes per K row in LDS
  static constexpr int kVStride = kv_v_stride();   // bytes per V^T row in LDS
  static constexpr int kKBytes = kv_v_offset(D);
  static constexpr int kLogOffset = kv_log_offset(D);  // 64 floats: log2 of V row scales
  static constexpr int kInvOffset = kv_inv_offset(D);  // 64 floats: 1 / (255 * scale)
  static constexpr int kCorrOffset = kv_corr_offset(D);  // D ints: biased 128 * colsum
};

// Online softmax and PV of one 64-key block (block index t, staged at `stage`) for one wave.
// ct[g]: the score multiplier q_scale * k_scale * softmax_scale * log2(e) of key thread group g
// (keys k with (k % 8) / 2 == g; all four equal for per-block K scales).  Output register r of
// lane half h holds key 16h + r (and 32 + 16h + r), so register 4q + i belongs to group
// 2 (q % 2) + i / 2.
template <int D, int NW, bool kCausal>
__device__ __forceinline__ void block_update(const char* stage, const v16i (&s)[2], const float (&ct)[4], int t,
                                             int q0, int n, int h, uint32_t sel, float (&num)[D / 32][16],
                                             float (&den)[4], float& mref, float& mlim, float& kref) {
  using L = TileLayout<D, NW>;
  constexpr int kChunksD = D / 32;

  // ---- shifted scores x = s * c + log2(vs), in-lane over 32 keys, and the block max ----
  const float4* lk4 = reinterpret_cast<const float4*>(stage + L::kLogOffset);
  float x[32];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 la = lk4[4 * h + q];
    const float4 lb = lk4[8 + 4 * h + q];
    const float c01 = ct[2 * (q & 1)], c23 = ct[2 * (q & 1) + 1];
    x[4 * q + 0] = fmaf(unbias_score(s[0][4 * q + 0]), c01, la.x);
    x[4 * q + 1] = fmaf(unbias_score(s[0][4 * q + 1]), c01, la.y);
    x[4 * q + 2] = fmaf(unbias_score(s[0][4 * q + 2]), c23, la.z);
    x[4 * q + 3] = fmaf(unbias_score(s[0][4 * q + 3]), c23, la.w);
    x[16 + 4 * q + 0] = fmaf(unbias_score(s[1][4 * q + 0]), c01, lb.x);
    x[16 + 4 * q + 1] = fmaf(unbias_score(s[1][4 * q + 1]), c01, lb.y);
    x[16 + 4 * q + 2] = fmaf(unbias_score(s[1][4 * q + 2]), c23, lb.z);
    x[16 + 4 * q + 3] = fmaf(unbias_score(s[1][4 * q + 3]), c23, lb.w);
  }
  if constexpr (kCausal) {
    if (t * kKeyBlock + kKeyBlock - 1 > q0) {  // block crosses this wave's diagonal
      // Register r holds key t * 64 + 16 h + r' (r' = r or r + 16) for query q0 + n: masked when
      // r' > lim.  The lane id is read here, inside the branch, so that nothing lane-dependent
      // is kept live across the loop for it (a hoisted value spills at 168 VGPRs, and the
      // reload's vmcnt wait would also drain the tile copies in flight).
      int lane_id;
      asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane_id));
      const int lim = q0 - t * kKeyBlock + (lane_id & 31) - 16 * (lane_id >> 5);
#pragma unroll
      for (int r = 0; r < 32; ++r)
        if ((r < 16 ? r : 16 + r) > lim) x[r] = -__builtin_inff();
    }
  }
  const float mx = cross_half_max(max32(x));

  // ---- lazy rescale of num/den when the block maximum outgrows the reference by 2^8 ----
  // (kept beside mref: mlim = mref + 2^8 and kref = 255 * 2^-mref)
  const bool grow = mx > mlim;
  if (__builtin_amdgcn_ballot_w64(grow) != 0) {
    const float alpha = grow ? __builtin_amdgcn_exp2f(mref - mx) : 1.0f;
    if (grow) {
      mref = mx;
      mlim = mx + kLazyRescale;
      kref = __builtin_amdgcn_exp2f(kLog2Of255 - mx);
    }
#pragma unroll
    for (int j = 0; j < kChunksD; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) num[j][r] *= alpha;
#pragma unroll
    for (int q = 0; q < 4; ++q) den[q] *= alpha;
  }

  // ---- e = 255 * vs * p = exp2(x - bm + log2 255), den += sum(p) * beta, UINT8 codes ----
  // den holds four partial sums per lane (the lane's keys k with k % 4 = q), added across the
  // slots and the two lane halves once, in the epilogue
  const float4* iv4 = reinterpret_cast<const float4*>(stage + L::kInvOffset);
  float ps[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  uint32_t pw[8];
  float beta;  // the block's weight beside the reference maximum, 2^(bm - mref)
  float dw;    // the denominator weight of sum(ps)
  if (__builtin_amdgcn_ballot_w64(!(fabsf(mx) <= kDirectRange)) == 0) {
    // every block maximum of the wave finite and within +-96: E = exp2(x) and e = E * C with
    // C = 2^(log2 255 - bm), no per-key subtraction; the code FMA multiplies by C
    // (pack_scaled_codes), and sum(p) * beta = sum(E / (255 vs)) * C * beta, where
    // C * beta = 255 * 2^-mref = kref (mref >= bm - 2^8 >= -104: finite)
    const float c = __builtin_amdgcn_exp2f(kLog2Of255 - mx);
    beta = __builtin_amdgcn_exp2f(mx - mref);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 ia = iv4[4 * h + q];
      const float4 ib = iv4[8 + 4 * h + q];
      const float e0 = __builtin_amdgcn_exp2f(x[4 * q + 0]);
      const float e1 = __builtin_amdgcn_exp2f(x[4 * q + 1]);
      const float e2 = __builtin_amdgcn_exp2f(x[4 * q + 2]);
      const float e3 = __builtin_amdgcn_exp2f(x[4 * q + 3]);
      const float f0 = __builtin_amdgcn_exp2f(x[16 + 4 * q + 0]);
      const float f1 = __builtin_amdgcn_exp2f(x[16 + 4 * q + 1]);
      const float f2 = __builtin_amdgcn_exp2f(x[16 + 4 * q + 2]);
      const float f3 = __builtin_amdgcn_exp2f(x[16 + 4 * q + 3]);
      ps[0] = fmaf(e0, ia.x, ps[0]);
      ps[1] = fmaf(e1, ia.y, ps[1]);
      ps[2] = fmaf(e2, ia.z, ps[2]);
      ps[3] = fmaf(e3, ia.w, ps[3]);
      ps[0] = fmaf(f0, ib.x, ps[0]);
      ps[1] = fmaf(f1, ib.y, ps[1]);
      ps[2] = fmaf(f2, ib.z, ps[2]);
      ps[3] = fmaf(f3, ib.w, ps[3]);
      pw[q] = pack_scaled_codes(e0, e1, e2, e3, c, sel);
      pw[4 + q] = pack_scaled_codes(f0, f1, f2, f3, c, sel);
    }
    dw = kref;
  } else {
    // extreme, empty (causal) or non-finite block maxima: subtract the shift first, as the
    // reference's exp(s - bm)
    const bool empty = mx == -__builtin_inff();
    beta = empty ? 0.0f : __builtin_amdgcn_exp2f(mx - mref);
    const float shift = empty ? 0.0f : mx - kLog2Of255;
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
    dw = beta;
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) den[q] = fmaf(ps[q], dw, den[q]);
  const float weight = beta;  // the reference's 1/255 is applied once, in the epilogue
  const v4i p0 = {static_cast<int>(pw[0]), static_cast<int>(pw[1]), static_cast<int>(pw[2]), static_cast<int>(pw[3])};
  const v4i p1 = {static_cast<int>(pw[4]), static_cast<int>(pw[5]), static_cast<int>(pw[6]), static_cast<int>(pw[7])};

  // ---- numerator: O^T += (V^T (u - 128) + 128 colsum) * beta (x 1/255 at the end), two D chunks' MFMA chains
  // in flight at a time (the score and probability registers are dead here) ----
  const v4i* corr4 = reinterpret_cast<const v4i*>(stage + L::kCorrOffset);
#pragma unroll
  for (int j0 = 0; j0 < kChunksD; j0 += 2) {
    v16i acc[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j = j0 + u;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const v4i c4 = corr4[8 * j + 2 * g + h];
        acc[u][4 * g + 0] = c4[0];
        acc[u][4 * g + 1] = c4[1];
        acc[u][4 * g + 2] = c4[2];
        acc[u][4 * g + 3] = c4[3];
      }
    }
    v4i a0[2], a1[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const char* vrow = stage + L::kKBytes + (32 * (j0 + u) + n) * L::kVStride + 16 * h;
      a0[u] = *reinterpret_cast<const v4i*>(vrow);
      a1[u] = *reinterpret_cast<const v4i*>(vrow + 32);
    }
    acc[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0[0], p0, acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0[1], p0, acc[1], 0, 0, 0);
    acc[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1[0], p1, acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1[1], p1, acc[1], 0, 0, 0);
    // acc started from the biased correction: its bits are 1.5 * 2^23 + (u @ v) exactly.
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int r = 0; r < 16; ++r) num[j0 + u][r] = fmaf(unbias(acc[u][r]), weight, num[j0 + u][r]);
  }
}

template <int D, int NW, bool kCausal, bool kPerThread, bool kBarrier>
__device__ __forceinline__ void pipeline_step(const AttnParams& p, char* smem, int t, int tiles, int wave_tiles, int bh,
                                              int wave, int lane, const v4i (&qf)[D / 32], float cq,
                                              int q0, int n, int h, int krow, uint32_t sel,
                                              const v16i (&s_cur)[2], v16i (&s_next)[2], float (&num)[D / 32][16],
                                              float (&den)[4], float& mref, float& mlim, float& kref) {
  using L = TileLayout<D, NW>;
  using R = Ring<NW>;
  // unconditional (clamped) so every iteration issues the same number of copies; a clamped
  // copy lands in a stage no iteration reads before it is written again
  copy_block<L>(p, smem + ((t + R::kLead) % R::kStages) * L::kStageBytes, bh, min(t + R::kLead, tiles - 1), wave,
                lane);
  if (t < wave_tiles) {
    block_scores<D, L>(smem + ((t + 1) % R::kStages) * L::kStageBytes, qf, h, krow, s_next);  // unused past the end
    const char* stage = smem + (t % R::kStages) * L::kStageBytes;
    // the K scales of the tile's four thread groups sit in the padding of K row 0
    float ct[4];
    if constexpr (kPerThread) {
      const float4 ks = *reinterpret_cast<const float4*>(stage + D);
      ct[0] = cq * ks.x;
      ct[1] = cq * ks.y;
      ct[2] = cq * ks.z;
      ct[3] = cq * ks.w;
    } else {  // per-block scales: the four slots hold the same value
      ct[0] = ct[1] = ct[2] = ct[3] = cq * *reinterpret_cast<const float*>(stage + D);
    }
    block_update<D, NW, kCausal>(stage, s_cur, ct, t, q0, n, h, sel, num, den, mref, mlim, kref);
  }
  if constexpr (kBarrier) stage_barrier_keep_last<L>(wave);
}

// Two waves per SIMD (at most 256 VGPRs): one 8-wave or two 4-wave workgroups per CU.
template <int D, int NW, bool kCausal, int kOut, bool kPerThread>
__global__ void __launch_bounds__(NW * 64, 8 / NW) attention_kernel(const AttnParams p) {
  using L = TileLayout<D, NW>;
  using R = Ring<NW>;
  constexpr int kChunksD = D / 32;
  constexpr int kLead = R::kLead;
  __shared__ __attribute__((aligned(16))) char smem[R::kStages * L::kStageBytes];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5;  // lane half
  const int n = lane & 31;  // query column within the wave
  // wave-uniform in SGPRs (the runtime division is VALU code): per-block key scales then come
  // from scalar loads, which do not share the vmcnt counter with the direct LDS copies
  const TileCoord tc = workgroup_tile<kCausal>(p);
  const int bh = __builtin_amdgcn_readfirstlane(tc.bh);
  const int qtile = __builtin_amdgcn_readfirstlane(tc.qtile);
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
    // the scale of this lane's query row: slot n % 8 of its block (every slot, per block)
    cq = p.query_scale[(static_cast<long>(bh) * p.nqb + (q0 >> 5)) * kQueryScaleSlots + (kPerThread ? (n & 7) : 0)] *
         (p.scale_log2e * kScoreUnit);
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
  for (int b = 0; b < kLead; ++b) copy_block<L>(p, smem + b * L::kStageBytes, bh, min(b, tiles - 1), wave, lane);

  if (fused_live) {
    // wait for the query loads only (issued before this wave's kLead * kRounds or
    // kLead * (kRounds - 1) copies), then quantise while the copies land
    if (wave < L::kFullWaves)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLead * L::kRounds) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLead * (L::kRounds - 1)) : "memory");
#pragma unroll
    for (int i = 0; i < D / 16; ++i) asm volatile("" : "+v"(raw[i]));
    cq = quantize_query_block<D, kPerThread>(p, q0, n, raw, qf) * (p.scale_log2e * kScoreUnit);
  }

  float num[kChunksD][16];
#pragma unroll
  for (int j = 0; j < kChunksD; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) num[j][r] = 0.0f;
  float den[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  float mref = -__builtin_inff();
  float mlim = -__builtin_inff();
  float kref = 0.0f;

  // MFMA row m of the K operand holds key 16*((m>>2)&1) + 4*(m>>3) + (m&3), so that output
  // register r of lane half h holds key 16h + r.
  const int krow = 16 * ((n >> 2) & 1) + 4 * (n >> 3) + (n & 3);
  const uint32_t sel = code_selector();

  stage_barrier<0>();  // all prologue copies landed

  v16i s_a[2], s_b[2];  // scores of the current and the next block, alternating
  if (wave_tiles > 0) block_scores<D, L>(smem, qf, h, krow, s_a);

  // unrolled by two so both score sets keep static names; one barrier per pair (8 waves) or
  // per iteration (4 waves)
  int t = 0;
  for (; t + 1 < tiles; t += 2) {
    pipeline_step<D, NW, kCausal, kPerThread, R::kEveryIteration>(p, smem, t, tiles, wave_tiles, bh, wave, lane, qf, cq,
                                                               q0, n, h, krow, sel, s_a, s_b, num, den, mref, mlim, kref);
    pipeline_step<D, NW, kCausal, kPerThread, true>(p, smem, t + 1, tiles, wave_tiles, bh, wave, lane, qf, cq, q0, n,
                                        h, krow, sel, s_b, s_a, num, den, mref, mlim, kref);
  }
  if (t < tiles)
    pipeline_step<D, NW, kCausal, kPerThread, false>(p, smem, t, tiles, wave_tiles, bh, wave, lane, qf, cq, q0, n, h,
                                         krow, sel, s_a, s_b, num, den, mref, mlim, kref);
  // no direct copy may still be writing this workgroup's LDS when its waves end
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- epilogue: num / max(den, 1e-30) + mean(V), one query per lane ----
  // the row's denominator: the four partial sums of both lane halves
  const float den_total = cross_half_sum((den[0] + den[1]) + (den[2] + den[3]));
  const int query = q0 + n;
  if (!wave_live || query >= p.query_length) return;
  const float rden = (1.0f / 255.0f) / fmaxf(den_total, 1e-30f);  // the numerator holds 255 x the reference's
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

// Three 4-wave workgroups per CU: three waves per SIMD (at most 168 VGPRs), each from another
// workgroup, so one wave's waits on its MFMA results, LDS reads and barriers are covered by the
// other two waves' VALU work.  That needs the register file of the two-wave kernels' look-ahead
// (the next block's scores, 32 VGPRs) and most of its LDS: each workgroup streams the tile
// records through two stages (2 x 20 KiB at D = 128, 120 KiB per CU).  Iteration t: wait for
// this wave's copies of tile t, barrier (every copy of tile t landed and published, every read
// of tile t - 1 done), start the copy of tile t + 1 into the stage tile t - 1 used, then the
// scores, softmax and PV of tile t.  The arithmetic is block_update's, so the output is
// bit-identical to the other plans.
// kOut: 0, 1, 2 = fp16, bf16, fp32 output; kPartials = the key-range split's partial sums
// (non-causal only): the workgroup covers key tiles [part * part_tiles, +part_tiles) of its query
// tile and writes its numerator, denominator and reference maximum for attention_merge_kernel.
constexpr int kPartials = 3;

// One query tile (and, for the key-range split, one key part) of attention_w3_kernel or of the
// work-queue kernel below: the whole prologue, key loop and epilogue of one workgroup.  The caller
// provides the LDS stages and the lane id; every wave of the workgroup calls it with the same tile.
template <int D, bool kCausal, int kOut, bool kPerThread, bool kFreshLane = false>
__device__ __forceinline__ void w3_tile(const AttnParams& p, char* smem, TileCoord tc, int part, int lane) {
  constexpr int NW = 4;
  using L = TileLayout<D, NW>;
  constexpr int kChunksD = D / 32;
  static_assert(kOut != kPartials || !kCausal, "the key-range split is non-causal");

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5;
  const int n = lane & 31;
  const int bh = __builtin_amdgcn_readfirstlane(tc.bh);
  const int qtile = __builtin_amdgcn_readfirstlane(tc.qtile);
  part = __builtin_amdgcn_readfirstlane(part);
  const int q0 = qtile * (NW * 32) + wave * 32;
  const bool wave_live = q0 < p.query_length;

  // key tiles [t0, t0 + tiles) of this workgroup, local index i = t - t0
  int t0 = 0;
  int tiles = p.nkb;
  if constexpr (kOut == kPartials) {
    t0 = part * p.part_tiles;
    tiles = max(0, min(p.part_tiles, p.nkb - t0));
  }
  int wave_tiles = wave_live ? tiles : 0;
  if constexpr (kCausal) {
    const int last_query = min(p.query_length, (qtile + 1) * NW * 32) - 1;
    tiles = last_query / kKeyBlock + 1;
    wave_tiles = wave_live ? (min(p.query_length, q0 + 32) - 1) / kKeyBlock + 1 : 0;
  }

  v4i qf[kChunksD];
  float cq = 0.0f;
  const bool fused_live = p.fused_query && wave_live;
  v4i raw[D / 16];
  if (fused_live) issue_query_loads<D>(p, bh, q0, n, h, raw);
  if (!p.fused_query && q0 < p.sq32) {
    if constexpr (kCausal) {
      // a wave-uniform base plus an unsigned 32-bit lane offset (the scalar-base load form): in
      // the causal kernels a 64-bit lane offset keeps its zero high half live across the key
      // loop, and it spills there (the non-causal kernels keep the 64-bit form: 0.3-0.6% faster)
      const int8_t* qblock = p.query_code + (static_cast<long>(bh) * p.sq32 + q0) * D;
      const uint32_t qoff = static_cast<uint32_t>(n * D + 16 * h);
#pragma unroll
      for (int c = 0; c < kChunksD; ++c) qf[c] = *reinterpret_cast<const v4i*>(qblock + qoff + 32 * c);
      const float* qscale = p.query_scale + (static_cast<long>(bh) * p.nqb + (q0 >> 5)) * kQueryScaleSlots;
      cq = qscale[kPerThread ? static_cast<uint32_t>(n & 7) : 0u] * p.score_multiplier;
    } else {
      const int8_t* qrow = p.query_code + (static_cast<long>(bh) * p.sq32 + q0 + n) * D + 16 * h;
#pragma unroll
      for (int c = 0; c < kChunksD; ++c) qf[c] = *reinterpret_cast<const v4i*>(qrow + 32 * c);
      cq = p.query_scale[(static_cast<long>(bh) * p.nqb + (q0 >> 5)) * kQueryScaleSlots + (kPerThread ? (n & 7) : 0)] *
           p.score_multiplier;
    }
#pragma unroll
    for (int c = 0; c < kChunksD; ++c) asm volatile("" ::"v"(qf[c]));
    asm volatile("" ::"v"(cq));
  } else {
#pragma unroll
    for (int c = 0; c < kChunksD; ++c) qf[c] = v4i{0, 0, 0, 0};
  }

  if (tiles > 0) copy_block<L>(p, smem, bh, t0, wave, lane);  // tile t0 into stage 0
  if (fused_live) {
    // wait for the query loads only (issued before this wave's copies of tile t0)
    if (tiles == 0)
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else if (wave < L::kFullWaves)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(L::kRounds) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(L::kRounds - 1) : "memory");
#pragma unroll
    for (int i = 0; i < D / 16; ++i) asm volatile("" : "+v"(raw[i]));
    cq = quantize_query_block<D, kPerThread>(p, q0, n, raw, qf) * p.score_multiplier;
  }

  float num[kChunksD][16];
#pragma unroll
  for (int j = 0; j < kChunksD; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) num[j][r] = 0.0f;
  float den[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  float mref = -__builtin_inff();
  float mlim = -__builtin_inff();
  float kref = 0.0f;
  const int krow = 16 * ((n >> 2) & 1) + 4 * (n >> 3) + (n & 3);
  const uint32_t sel = code_selector();

  for (int i = 0; i < tiles; ++i) {
    // this wave's copies of tile i landed; after the barrier every wave's have, and every read
    // of tile i - 1 (stage (i + 1) % 2) is done
    if constexpr (!kCausal) progress_priority(i, 1, tiles);  // causal: workgroups differ in length
    stage_barrier<0>();
    if (i + 1 < tiles) copy_block<L>(p, smem + ((i + 1) & 1) * L::kStageBytes, bh, t0 + i + 1, wave, lane);
    const int t = t0 + i;
    if (i < wave_tiles) {
      const char* stage = smem + (i & 1) * L::kStageBytes;
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
      block_update<D, NW, kCausal>(stage, sc, ct, t, q0, n, h, sel, num, den, mref, mlim, kref);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // the row's denominator: the four partial sums of both lane halves
  const float den_total = cross_half_sum((den[0] + den[1]) + (den[2] + den[3]));
  // kFreshLane (the work-queue kernel and the causal kernel): the lane's row and half read again
  // rather than kept through the key loop
  int epilogue_lane = lane;
  if constexpr (kFreshLane) asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(epilogue_lane));
  const int eh = epilogue_lane >> 5;
  const int en = epilogue_lane & 31;
  const int query = q0 + en;
  if (!wave_live || query >= p.query_length) return;
  if constexpr (kOut == kPartials) {
    const long rows = static_cast<long>(p.batch_heads) * p.query_length;
    const long row = static_cast<long>(part) * rows + static_cast<long>(bh) * p.query_length + query;
    float* dst = p.partials + row * D;
#pragma unroll
    for (int j = 0; j < kChunksD; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4*>(dst + 32 * j + 8 * g + 4 * eh) =
            make_float4(num[j][4 * g + 0], num[j][4 * g + 1], num[j][4 * g + 2], num[j][4 * g + 3]);
    // both lane halves hold the row's den_total and mref
    if (eh == 0) reinterpret_cast<float2*>(p.partials + p.key_parts * rows * D)[row] = make_float2(den_total, mref);
    return;
  } else {
    const float rden = (1.0f / 255.0f) / fmaxf(den_total, 1e-30f);  // the numerator holds 255 x the reference's
    const float* vmean = p.value_mean + static_cast<long>(bh) * D;
    const long out_row = (static_cast<long>(bh) * p.query_length + query) * D;
#pragma unroll
    for (int j = 0; j < kChunksD; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * j + 8 * g + 4 * eh;
        float4 m = make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (!kCausal) m = *reinterpret_cast<const float4*>(vmean + d0);
        store4<kOut>(p.output, out_row + d0, fmaf(num[j][4 * g + 0], rden, m.x), fmaf(num[j][4 * g + 1], rden, m.y),
                     fmaf(num[j][4 * g + 2], rden, m.z), fmaf(num[j][4 * g + 3], rden, m.w));
      }
    }
  }
}

template <int D, bool kCausal, int kOut, bool kPerThread>
__global__ void __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(3, 3)))
attention_w3_kernel(const AttnParams p) {
  __shared__ __attribute__((aligned(16))) char smem[2 * TileLayout<D, 4>::kStageBytes];
  int part = 0;
  TileCoord tc;
  if constexpr (kOut == kPartials) {
    // logical id -> (batch-head, key part, query tile): the workgroups of one key range of a
    // head are neighbours, so an XCD's workgroups stream the same tiles through its L2
    const int logical = p.xcd_remap ? xcd_remap(blockIdx.x, gridDim.x) : static_cast<int>(blockIdx.x);
    const int per_head = p.key_parts * p.query_tiles;
    tc.bh = logical / per_head;
    const int rem = logical - tc.bh * per_head;
    part = rem / p.query_tiles;
    tc.qtile = rem - part * p.query_tiles;
  } else {
    tc = workgroup_tile<kCausal>(p);
  }
  // causal: the lane id read again for the epilogue (kept through the key loop, its half bit
  // spills at 168 VGPRs)
  w3_tile<D, kCausal, kOut, kPerThread, kCausal>(p, smem, tc, part, threadIdx.x & 63);
}

// The work-queue plan: a persistent grid (at most three workgroups per CU) whose workgroups take
// query tiles from one queue per XCC instead of waiting for the hardware to dispatch them.  The
// hardware deals workgroups round-robin over the XCCs in id order, so a workgroup that cannot be
// placed on a full XCC holds back the next ones for every XCC: with causal tiles of unequal
// length, slots stayed empty 7-28 us after a short tile ended.  Here queue q holds the logical ids
// that XCC q runs under the XCD-aware order (the same tiles in the same longest-first order);
// workgroup b takes its tiles from queue b % queue_xccs with one relaxed atomic each, and once that
// queue is empty from the others in turn.  The tiles are computed exactly as by
// attention_w3_kernel, so the output is bit-identical.  Every claim increments a counter, so each
// workgroup ends after at most (tiles + queues) claims; no workgroup waits for another.
template <int D, bool kCausal, int kOut, bool kPerThread>
__global__ void __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(3, 3)))
attention_w3_queue_kernel(const AttnParams p) {
  static_assert(kOut != kPartials, "the work-queue plan has no key-range split");
  __shared__ __attribute__((aligned(16))) char smem[2 * TileLayout<D, 4>::kStageBytes];
  // The claim state lives in LDS (state[0]: the tile claimed, state[1]: the queue being taken
  // from).  Nothing of the claim may stay in registers across the tiles: at 168 VGPRs the key loop
  // has none to spare, so the lane id and a zero are read afresh in each iteration with inline
  // assembly the compiler cannot hoist, the LDS addresses are formed from them, and the divisors
  // are laundered the same way (hoisted, their reciprocals would hold registers too).
  __shared__ int state[4];
  for (bool first = true;; first = false) {
    int lane, zero;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane));
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
    int queues = p.queue_xccs, qt = p.query_tiles, heads = p.batch_heads;
    asm volatile("" : "+s"(queues), "+s"(qt), "+s"(heads));
    const int total = qt * heads;
    const int base = total / queues, rem = total - base * queues;
    volatile int* st = state + zero;
    if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) == 0) {
      // wave 0 claims: lane 0 takes the next tile of queue q; when q is empty, every lane reads
      // one queue's counter and the wave moves to the first queue with tiles left, or stops when
      // it has seen every queue empty.  Each attempt increments a counter, and a counter stops
      // being tried once it has passed its queue's length, so the loop ends.
      int q = __builtin_amdgcn_readfirstlane(first ? static_cast<int>(blockIdx.x) % queues : st[1]);
      int logical = -1;
      // the first tile needs no atomic: the workers of queue q start with its first tiles in
      // order (queue_init_kernel starts each counter past them), so the grid does not open with
      // every workgroup's atomic on the same few counters
      const int rank = static_cast<int>(blockIdx.x) / queues;
      if (first && rank < base + (q < rem ? 1 : 0)) logical = q * base + min(q, rem) + rank;
      while (logical < 0) {
        int i = 0;
        if (lane == 0)
          i = static_cast<int>(__hip_atomic_fetch_add(p.queue + q, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        i = __builtin_amdgcn_readfirstlane(i);
        if (i < base + (q < rem ? 1 : 0)) {
          logical = q * base + min(q, rem) + i;
          break;
        }
        const int other = q + lane < queues ? q + lane : q + lane - queues;
        bool left = false;
        if (lane < queues)
          left = static_cast<int>(__hip_atomic_load(p.queue + other, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) <
                 base + (other < rem ? 1 : 0);
        const uint64_t with_tiles = __builtin_amdgcn_ballot_w64(left);
        if (with_tiles == 0) break;
        const int step = __builtin_ctzll(with_tiles);
        q = q + step < queues ? q + step : q + step - queues;
      }
      if (lane == 0) {
        st[0] = logical;
        st[1] = q;
      }
    }
    // the claim is visible to every wave, and every wave is done with the previous tile's stages
    __syncthreads();
    const int logical = __builtin_amdgcn_readfirstlane(st[0]);
    __syncthreads();  // every wave has read the claim before thread 0 overwrites it
    if (logical < 0) return;
    // the key-tile and query counts laundered too: conditions derived from them were hoisted as
    // per-lane flags
    AttnParams pl = p;
    asm volatile("" : "+s"(pl.nkb), "+s"(pl.query_length));
    w3_tile<D, kCausal, kOut, kPerThread, true>(pl, smem, queue_tile<kCausal>(pl, logical, queues, qt, heads), 0, lane);
  }
}

// Sets the work-queue counters before the persistent grid (a fill kernel rather than
// hipMemsetAsync, so that a captured graph replays it correctly): queue q starts past the tiles
// its workers take first without an atomic, min(its tiles, its workers).
__global__ void __launch_bounds__(64) queue_init_kernel(uint32_t* counters, int queues, int total, int workers) {
  const int q = static_cast<int>(threadIdx.x);
  if (q >= queues) return;
  const int tiles = total / queues + (q < total % queues ? 1 : 0);
  const int starters = workers / queues + (q < workers % queues ? 1 : 0);
  counters[q] = static_cast<uint32_t>(min(tiles, starters));
}

// The key-range split's merge, one thread per four features of a query row: the parts' reference
// maxima m_p are aligned on their maximum M with weights 2^(m_p - M) (0 for a part that saw no
// key), then num = sum w_p num_p, den = sum w_p den_p, and the epilogue of the unsplit kernel:
// num / (255 max(den, 1e-30)) + mean(V).  The parts' sums enter in another order than one
// sequential pass, so split plans agree with the others to rounding, not bit for bit.
template <int D, int kOut>
__global__ void __launch_bounds__(256) attention_merge_kernel(const AttnParams p) {
  const long rows = static_cast<long>(p.batch_heads) * p.query_length;
  const long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= rows * (D / 4)) return;
  const long row = i / (D / 4);
  const int d0 = static_cast<int>(i - row * (D / 4)) * 4;
  const int bh = static_cast<int>(row / p.query_length);
  const float2* stats = reinterpret_cast<const float2*>(p.partials + p.key_parts * rows * D);
  float top = -__builtin_inff();
  for (int q = 0; q < p.key_parts; ++q) top = fmaxf(top, stats[q * rows + row].y);
  float den = 0.0f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int q = 0; q < p.key_parts; ++q) {
    const float2 st = stats[q * rows + row];
    const float w = st.y == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(st.y - top);
    den = fmaf(st.x, w, den);
    const float4 v = *reinterpret_cast<const float4*>(p.partials + (q * rows + row) * D + d0);
    acc.x = fmaf(v.x, w, acc.x);
    acc.y = fmaf(v.y, w, acc.y);
    acc.z = fmaf(v.z, w, acc.z);
    acc.w = fmaf(v.w, w, acc.w);
  }
  const float rden = (1.0f / 255.0f) / fmaxf(den, 1e-30f);
  const float4 m = *reinterpret_cast<const float4*>(p.value_mean + static_cast<long>(bh) * D + d0);
  store4<kOut>(p.output, row * D + d0, fmaf(acc.x, rden, m.x), fmaf(acc.y, rden, m.y), fmaf(acc.z, rden, m.z),
               fmaf(acc.w, rden, m.w));
}

template <int D, bool kCausal, bool kPerThread>
static hipError_t launch_w3(int out_dtype, const AttnParams& ap, hipStream_t stream) {
  const dim3 block(256);
  if (ap.queue_xccs > 0) {
    hipLaunchKernelGGL(queue_init_kernel, dim3(1), dim3(64), 0, stream, ap.queue, ap.queue_xccs,
                       ap.query_tiles * ap.batch_heads, ap.queue_workers);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    const dim3 grid(static_cast<unsigned>(ap.queue_workers));
    switch (out_dtype) {
      case 0: hipLaunchKernelGGL((attention_w3_queue_kernel<D, kCausal, 0, kPerThread>), grid, block, 0, stream, ap); break;
      case 1: hipLaunchKernelGGL((attention_w3_queue_kernel<D, kCausal, 1, kPerThread>), grid, block, 0, stream, ap); break;
      default: hipLaunchKernelGGL((attention_w3_queue_kernel<D, kCausal, 2, kPerThread>), grid, block, 0, stream, ap); break;
    }
    return hipGetLastError();
  }
  if constexpr (!kCausal) {
    if (ap.key_parts > 1) {
      const dim3 grid(static_cast<unsigned>(ap.query_tiles * ap.batch_heads * ap.key_parts));
      hipLaunchKernelGGL((attention_w3_kernel<D, false, kPartials, kPerThread>), grid, block, 0, stream, ap);
      hipError_t err = hipGetLastError();
      if (err != hipSuccess) return err;
      const long threads = static_cast<long>(ap.batch_heads) * ap.query_length * (D / 4);
      const dim3 merge_grid(static_cast<unsigned>((threads + 255) / 256));
      switch (out_dtype) {
        case 0: hipLaunchKernelGGL((attention_merge_kernel<D, 0>), merge_grid, block, 0, stream, ap); break;
        case 1: hipLaunchKernelGGL((attention_merge_kernel<D, 1>), merge_grid, block, 0, stream, ap); break;
        default: hipLaunchKernelGGL((attention_merge_kernel<D, 2>), merge_grid, block, 0, stream, ap); break;
      }
      return hipGetLastError();
    }
  }
  const dim3 grid(static_cast<unsigned>(ap.query_tiles * ap.batch_heads));
  switch (out_dtype) {
    case 0: hipLaunchKernelGGL((attention_w3_kernel<D, kCausal, 0, kPerThread>), grid, block, 0, stream, ap); break;
    case 1: hipLaunchKernelGGL((attention_w3_kernel<D, kCausal, 1, kPerThread>), grid, block, 0, stream, ap); break;
    default: hipLaunchKernelGGL((attention_w3_kernel<D, kCausal, 2, kPerThread>), grid, block, 0, stream, ap); break;
  }
  return hipGetLastError();
}

template <int D, int NW, bool kCausal, bool kPerThread>
static hipError_t launch_out(int out_dtype, const AttnParams& ap, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(ap.query_tiles * ap.batch_heads));
  const dim3 block(NW * 64);
  switch (out_dtype) {
    case 0: hipLaunchKernelGGL((attention_kernel<D, NW, kCausal, 0, kPerThread>), grid, block, 0, stream, ap); break;
    case 1: hipLaunchKernelGGL((attention_kernel<D, NW, kCausal, 1, kPerThread>), grid, block, 0, stream, ap); break;
    default: hipLaunchKernelGGL((attention_kernel<D, NW, kCausal, 2, kPerThread>), grid, block, 0, stream, ap); break;
  }
  return hipGetLastError();
}

template <int D, int NW, bool kCausal>
static hipError_t launch_granularity(int out_dtype, const AttnParams& ap, hipStream_t stream) {
  if constexpr (NW == 3)
    return ap.per_thread ? launch_w3<D, kCausal, true>(out_dtype, ap, stream)
                         : launch_w3<D, kCausal, false>(out_dtype, ap, stream);
  else
    return ap.per_thread ? launch_out<D, NW, kCausal, true>(out_dtype, ap, stream)
                         : launch_out<D, NW, kCausal, false>(out_dtype, ap, stream);
}

template <int D, int NW>
static hipError_t launch_causal(bool causal, int out_dtype, const AttnParams& ap, hipStream_t stream) {
  return causal ? launch_granularity<D, NW, true>(out_dtype, ap, stream)
                : launch_granularity<D, NW, false>(out_dtype, ap, stream);
}

hipError_t launch_attention(int head_dim, bool causal, int out_dtype, int waves, const AttnParams& ap,
                            hipStream_t stream) {
  // waves: 8 or 4 query waves per workgroup with two waves per SIMD, or 3 for three 4-wave
  // workgroups per CU (attention_w3_kernel)
  if (head_dim == 128) {
    return waves == 3   ? launch_causal<128, 3>(causal, out_dtype, ap, stream)
           : waves == 4 ? launch_causal<128, 4>(causal, out_dtype, ap, stream)
                        : launch_causal<128, 8>(causal, out_dtype, ap, stream);
  }
  return waves == 3   ? launch_causal<64, 3>(causal, out_dtype, ap, stream)
         : waves == 4 ? launch_causal<64, 4>(causal, out_dtype, ap, stream)
                      : launch_causal<64, 8>(causal, out_dtype, ap, stream);
}

}  // namespace piper
