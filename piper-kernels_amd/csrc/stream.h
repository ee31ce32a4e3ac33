// Streaming machinery shared by the gfx950 attention kernels (Piper Attention and
// SageAttention2++): tile records copied straight from HBM into a ring of LDS stages, the
// workgroup barriers that keep those copies in flight, the in-prologue query quantisation,
// the INT8 score MFMAs and the output stores.
//
// A tile layout type L provides kWaves (waves per workgroup), kKStride (bytes per K row in a
// stage), kStageBytes (one tile record = one stage, a KiB multiple), kPieces (1 KiB pieces per
// stage), kRounds (pieces per wave, rounded up) and kFullWaves (waves that copy kRounds
// pieces).  Parameter structs provide kv_tiles and nkb (tile records of a batch-head), and
// for the query quantisation query, heads, query_length and query_bf16.
#pragma once

#include "common.h"
#include "quant.h"

namespace piper {

// Pieces of a stage of kStageBytes copied by NW waves.
template <int kStageBytes_, int NW>
struct StagePieces {
  static constexpr int kWaves = NW;
  static constexpr int kStageBytes = kStageBytes_;
  static constexpr int kPieces = kStageBytes / 1024;  // 1 KiB per wave-wide 16-byte load
  static constexpr int kRounds = (kPieces + NW - 1) / NW;
  static constexpr int kFullWaves = kPieces % NW == 0 ? NW : kPieces % NW;  // waves with kRounds pieces
  static_assert(kStageBytes % 1024 == 0, "a stage is a whole number of KiB");
};

// LDS ring of kStages tile records, shared by both attention kernels.  Iteration t consumes block t (stage t % kStages), issues
// the QK MFMAs of block t + 1 first so they run under the softmax VALU work, and starts the
// direct copy of block t + kLead.  The barrier after iteration i waits for every copy issued
// before iteration i.
// 8-wave workgroups (one per CU): 6 stages, a lead of 4 and a barrier after every second
// iteration.  A copy issued at iteration t is complete and published by the barrier after
// iteration t + 1 or t + 2, before its first read (QK at iteration t + kLead - 1), and the
// stage it overwrites was last read at iteration t - 2, before the barrier after t - 2 or t - 1.
// 4-wave workgroups (two per CU: at D = 128 two 4-stage rings take 160 KiB (Piper Attention)
// or 152 KiB (SageAttention2++) of the CU's 160 KiB): 4 stages, a lead of 3 and a barrier
// after every iteration.  A copy issued at iteration t is published by the barrier after
// t + 1, before its first read at t + 2, and the stage it overwrites was last read at
// iteration t - 1, before the barrier after t - 1.
template <int NW>
struct Ring {
  static constexpr int kStages = NW == 4 ? 4 : 6;
  static constexpr int kLead = NW == 4 ? 3 : 4;
  static constexpr bool kEveryIteration = NW == 4;
  static_assert(kStages >= kLead + (kEveryIteration ? 1 : 2), "a copy must not overwrite a stage still being read");
  static_assert(kLead >= (kEveryIteration ? 3 : 4), "a copy must be published before its first read");
};

// Workgroup -> (batch-head, query tile) of both attention kernels.  With the XCD remap the
// logical ids of one XCD are contiguous (xcd_remap).  Non-causal grids and causal grids in
// forward order walk the query tiles of one head after another; causal grids in longest-first
// order (the work of a query tile grows with its index) walk each head's tiles longest first.
// With causal_interleave they instead go in longest-processing-time order across the heads
// that share an L2: when the batch-heads split evenly over the 8 XCDs, each XCD's range covers
// its own batch-heads and walks the query tiles longest first across all of them (without the
// remap the whole grid does).  That shortens the tail of short and medium sequences; for long
// sequences with many heads the head-by-head order keeps more of the K/V reuse in L2.
struct TileCoord {
  int bh;
  int qtile;
};

template <bool kCausal, class Params>
__device__ __forceinline__ TileCoord workgroup_tile(const Params& p) {
  const int logical = p.xcd_remap ? xcd_remap(blockIdx.x, gridDim.x) : static_cast<int>(blockIdx.x);
  const int qt = p.query_tiles;
  if (kCausal && !p.causal_forward && p.causal_interleave && !(p.xcd_remap && (p.batch_heads & 7) != 0)) {
    int heads = p.batch_heads;
    int base_bh = 0;
    int r = logical;
    if (p.xcd_remap) {  // batch_heads % 8 == 0: one group of heads per XCD
      heads = p.batch_heads >> 3;
      const int group = logical / (heads * qt);
      base_bh = group * heads;
      r = logical - group * heads * qt;
    }
    const int rank = r / heads;
    return {base_bh + (r - rank * heads), qt - 1 - rank};
  }
  const int bh = logical / qt;
  const int qtile = logical - bh * qt;
  return {bh, kCausal && !p.causal_forward ? qt - 1 - qtile : qtile};
}

// Logical id -> (batch-head, query tile) of the work-queue plan, whose `queues` queues hold
// consecutive logical ranges (queue q: what XCC q runs under the XCD-aware order); qt and
// batch_heads are p.query_tiles and p.batch_heads, passed in by the caller.  The same order
// as workgroup_tile with the XCD remap: with causal_interleave and batch-heads divisible by the
// queues, each queue walks its own batch-heads' query tiles longest first across them.
template <bool kCausal, class Params>
__device__ __forceinline__ TileCoord queue_tile(const Params& p, int logical, int queues, int qt, int batch_heads) {
  if (kCausal && !p.causal_forward && p.causal_interleave && batch_heads % queues == 0) {
    const int heads = batch_heads / queues;
    const int group = logical / (heads * qt);
    const int r = logical - group * heads * qt;
    const int rank = r / heads;
    return {group * heads + (r - rank * heads), qt - 1 - rank};
  }
  const int bh = logical / qt;
  const int qtile = logical - bh * qt;
  return {bh, kCausal && !p.causal_forward ? qt - 1 - qtile : qtile};
}

// One wave-wide global_load_lds_dwordx4: lane i copies 16 bytes from src + off (src
// wave-uniform, held in SGPRs; off the lane's 32-bit offset) to LDS byte lds + 16 * i.  The
// scalar-base form keeps the per-piece address arithmetic on the scalar unit.  Issued as inline
// assembly so that the compiler's wait insertion does not treat every later LDS read as
// dependent on it: the waits are explicit (stage_barrier, and a drain before the waves end).
__device__ __forceinline__ void copy_piece(const char* src, uint32_t off, uint32_t lds) {
  // s_nop: one wait state between the SALU write of M0 and the LDS DMA that reads it
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(src), "{m0}"(lds) : "memory");
}

__device__ __forceinline__ uint32_t lds_address(const char* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}

// Direct global -> LDS copy of the tile record of block t into one LDS stage: wave w copies
// 1 KiB pieces w, w + NW, ... (each lane 16 bytes), so the per-lane addresses are loop
// invariant and no VGPRs hold staged data.  Completion is tracked by this wave's vmcnt.
template <class L, class Params>
__device__ __forceinline__ void copy_block(const Params& p, char* stage, int bh, int t, int wave, int lane) {
  constexpr int NW = L::kWaves;
  const char* tile = reinterpret_cast<const char*>(p.kv_tiles) + (static_cast<long>(bh) * p.nkb + t) * L::kStageBytes;
  const uint32_t base = lds_address(stage);
#pragma unroll
  for (int r = 0; r < L::kRounds; ++r) {
    const int piece = wave + r * NW;  // wave-uniform: a scalar branch
    if (piece < L::kPieces) copy_piece(tile + piece * 1024, lane * 16, base + piece * 1024);
  }
}

// Workgroup barrier that lets this wave's newest kInFlight direct loads stay in flight.
// (__syncthreads would drain every outstanding load.)  LDS reads are waited for as well, so
// a stage is never overwritten under a pending read.
template <int kInFlight>
__device__ __forceinline__ void stage_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kInFlight) : "memory");
}

template <class L>
__device__ __forceinline__ void stage_barrier_keep_last(int wave) {
  if (wave < L::kFullWaves)
    stage_barrier<L::kRounds>();
  else
    stage_barrier<L::kRounds - 1>();
}

// Wave priority by the workgroup's progress through its tiles: 3 in the first quarter, then 2, 1
// and 0 in the last, each set at the iteration [t, t + step) that reaches its quarter mark.  The
// SIMD arbiter otherwise favours the oldest wave, so the workgroups sharing a CU drift apart and,
// at the end of the grid, slots idle while the youngest workgroups finish alone.  For grids of
// equal-length workgroups (non-causal); the level is the wave's issue priority (s_setprio), not a
// stream priority.
__device__ __forceinline__ void progress_priority(int t, int step, int tiles) {
  const int q1 = tiles / 4, q2 = tiles / 2, q3 = (3 * tiles) / 4;
  if (t == 0) __builtin_amdgcn_s_setprio(3);
  if (t <= q1 && q1 < t + step) __builtin_amdgcn_s_setprio(2);
  if (t <= q2 && q2 < t + step) __builtin_amdgcn_s_setprio(1);
  if (t <= q3 && q3 < t + step) __builtin_amdgcn_s_setprio(0);
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
    const uint2 v = make_uint2(pack_bf16x2(a, b), pack_bf16x2(c, d));
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + index) = v;
  } else {
    const uint2 v = make_uint2(pack_half2(a, b), pack_half2(c, d));
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + index) = v;
  }
}

// Value of an integer accumulator that started from kAccBias: one exact FP32 subtraction.
// (The element arrives as a scalar: this clang's __builtin_bit_cast of an ext_vector
// subscript reads element 0.)
__device__ __forceinline__ float unbias(int bits) { return __builtin_bit_cast(float, bits) - kAccBiasValue; }

// Score accumulators start from the bit pattern of 1/(2 pi), which the MFMA takes as an inline
// constant accumulator operand (no registers hold it).  Its mantissa field 0x22F983 = 2292099
// exceeds |Q K^T| <= 128 * 127^2 = 2064512, so every result's bits stay in the binade
// [2^-3, 2^-2), where they read as 1/(2 pi) + score * 2^-26 exactly; subtracting 1/(2 pi) is
// exact (the two are within a factor of 2) and leaves score * 2^-26.  The kernels' score
// multipliers carry the compensating 2^26 (kScoreUnit), so score * 2^-26 * (c * 2^26) is the
// same exact product as score * c: every logit is bit-identical to one from an unbiased score
// (for multipliers c below 2^101, where c * 2^26 stays finite).
constexpr int kScoreBias = 0x3E22F983;
constexpr float kScoreUnit = 67108864.0f;  // 2^26
static_assert(128 * 127 * 127 < (kScoreBias & 0x7fffff), "a score must not leave the bias's binade");

__device__ __forceinline__ float unbias_score(int bits) {
  return __builtin_bit_cast(float, bits) - __builtin_bit_cast(float, kScoreBias);
}

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
template <int D, class Params>
__device__ __forceinline__ void issue_query_loads(const Params& p, int bh, int q0, int n, int h,
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
// zero-padded 32 x D block, codes round-half-even(x / scale) clamped to +-127; with kPerThread,
// sage/reference.py:23-39: one scale per thread group of rows {t, t+8, t+16, t+24}).  The
// amax is a wave-wide max (per block) or a max over the 8 lanes holding the group's rows (lane
// (n, h) holds row q0 + n, so the lanes whose index agrees in its low three bits); the 16 codes
// of each chunk are packed in element order, the layout of the prepared code rows.  Returns the
// scale of this lane's query row.
template <int D, bool kPerThread = false, class Params>
__device__ __forceinline__ float quantize_query_block(const Params& p, int q0, int n, const v4i (&raw)[D / 16],
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
  if constexpr (kPerThread) {
    // max over lanes l ^ 8, l ^ 16, l ^ 32 (the lanes whose low three bits agree) without lane
    // addresses: a row rotation by 8 (within 16 lanes, that is l ^ 8), then the gfx950 row-pair
    // and half swaps
    amax = fmaxf(amax, dpp<0x128>(amax));  // row_ror:8
    const uint32_t u16 = __float_as_uint(amax);
    const auto r16 = __builtin_amdgcn_permlane16_swap(u16, u16, false, false);
    amax = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
    const uint32_t u32 = __float_as_uint(amax);
    const auto r32 = __builtin_amdgcn_permlane32_swap(u32, u32, false, false);
    amax = fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
  } else {
    amax = wave_max(amax);
  }
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

// First MFMA of a score chain, its accumulator operand the inline constant 1/(2 pi)
// (kScoreBias).  Written as assembly because the compiler does not fold a constant that more
// than one MFMA uses: it keeps the splat in 16 SGPRs and copies them to VGPRs in every block.
// The result feeds only the next MFMA of its chain, as that MFMA's full accumulator operand,
// which the hardware interlocks; the leading s_nop covers a VALU write of a source operand.
__device__ __forceinline__ v16i score_mfma_first(v4i a, v4i b) {
  static_assert(kScoreBias == 0x3E22F983, "0.15915494 is the inline constant 1/(2 pi)");
  v16i r;
  asm("s_nop 1\n\tv_mfma_i32_32x32x32_i8 %0, %1, %2, 0.15915494" : "=&v"(r) : "v"(a), "v"(b));
  return r;
}

// Integer scores S^T = K Q^T of one 64-key block: s[0] keys 0..31, s[1] keys 32..63 (each
// lane: its query column, keys 16h + r after the K-row permutation).
template <int D, class L>
__device__ __forceinline__ void block_scores(const char* stage, const v4i (&qf)[D / 32], int h, int krow,
                                             v16i (&s)[2]) {
  // accumulators start from kScoreBias: each result reads as FP32 1/(2 pi) + score * 2^-26
  // exactly (unbias_score)
#pragma unroll
  for (int c = 0; c < D / 32; ++c) {
    const char* kb = stage + 32 * c + 16 * h;
    const v4i a0 = *reinterpret_cast<const v4i*>(kb + krow * L::kKStride);
    const v4i a1 = *reinterpret_cast<const v4i*>(kb + (32 + krow) * L::kKStride);
    if (c == 0) {
      s[0] = score_mfma_first(a0, qf[c]);
      s[1] = score_mfma_first(a1, qf[c]);
    } else {
      s[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, qf[c], s[0], 0, 0, 0);
      s[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, qf[c], s[1], 0, 0, 0);
    }
  }
}

}  // namespace piper
