// Prep kernels: order-defined K/V sequence means, per-block INT8 Q/K and per-key INT8 V
// (Piper Attention); K means, per-channel V scales, INT8 K and FP8 V (SageAttention2++).
//
// Behaviour follows the reference's portable algorithm (jumbledpoophj/piper-kernels 0.2.1):
//   K smoothing and per-block ("per_warp") Q/K codes  sage/reference.py:61-108
//   V centring (non-causal only) and per-key V codes   piper_attention/reference.py:22-59
// Every code and scale is bit-exact with that arithmetic: scale = amax/127 + 1e-7 in FP32
// (IEEE division, FP32 add), code = clamp(round_half_even(x / scale), -127, 127) with an IEEE
// division per element.  The K/V means are the reference's FP32 torch.mean(dim=2) on CPU bit
// for bit: its cascade summation order (common.h) and one FP32 division.
#include "common.h"
#include "kernels.h"
#include "quant.h"

#include <type_traits>

namespace piper {

// ---------------------------------------------------------------------------------------
// Means, pass 1: one workgroup per chunk of L^2 rows of K (tensor 0) or V (tensor 1) of one
// batch-head.  Thread (slot, column group) sums L-row blocks slot, slot + kSlots, ... of eight
// columns, each block's rows in row order from +0.0 (cascade level 0), with 16-byte loads of
// all the block's rows in flight; the block sums meet in LDS, and one thread per column adds
// the chunk's complete blocks in block order (level 1).  A short last chunk's trailing
// length % L rows are its last, incomplete block: their sum goes to slot `chunks`.
// SageAttention2++'s V statistic is the per-column max |v| instead (exact in any order).
// ---------------------------------------------------------------------------------------
template <bool kBf16, bool kAbsMax, bool kGuard>
__device__ __forceinline__ void sum_block_rows(const uint16_t* rows, long stride, int n, float (&acc)[8]) {
  constexpr int kUnroll = 16;  // rows in flight (16 B each); L is a power of two >= 16
  for (int r = 0; r < (kGuard ? n : kUnroll); r += kUnroll) {
    uint4 raw[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      raw[u] = !kGuard || r + u < n ? *reinterpret_cast<const uint4*>(rows + static_cast<long>(r + u) * stride)
                                    : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (!kGuard || r + u < n) {
        float f[8];
        widen8<kBf16>(raw[u], f);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = kAbsMax ? fmaxf(acc[i], fabsf(f[i])) : acc[i] + f[i];
      }
    }
  }
}

template <bool kBf16, int D, bool kAbsMax>
__device__ __forceinline__ void chunk_block_sums(const uint16_t* base, long stride, int L, int full, int blocks,
                                                 int tail, int slot, int group, float* block_sums) {
  constexpr int kSlots = 256 / (D / 8);
  for (int blk = slot; blk < blocks; blk += kSlots) {
    const uint16_t* rows = base + static_cast<long>(blk) * L * stride;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (blk < full) {
      for (int r = 0; r < L; r += 16) sum_block_rows<kBf16, kAbsMax, false>(rows + r * stride, stride, 16, acc);
    } else {
      sum_block_rows<kBf16, kAbsMax, true>(rows, stride, tail, acc);
    }
    float4* dst = reinterpret_cast<float4*>(block_sums + blk * D + 8 * group);
    dst[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    dst[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
}

// One chunk's partial sums into p.partials; `block_sums` is LDS of L * D floats.  Every thread of
// the workgroup takes part (a barrier inside).
template <bool kBf16, int D>
__device__ __forceinline__ void mean_chunk(const MeanParams& p, int tensor, int bh, int chunk, float* block_sums) {
  constexpr int kGroups = D / 8;
  const int b = bh / p.heads;
  const int h = bh - b * p.heads;
  const InputTensor& t = tensor == 0 ? p.key : p.value;
  const bool absmax = tensor == 1 && p.value_absmax;
  const int L = p.block_rows;
  const long row0 = static_cast<long>(chunk) * L * L;
  const int rows = static_cast<int>(min(static_cast<long>(L) * L, p.length - row0));
  const int full = rows / L;
  const int tail = rows - full * L;
  const int blocks = full + (tail > 0 ? 1 : 0);
  const int group = threadIdx.x % kGroups;
  const uint16_t* base =
      static_cast<const uint16_t*>(t.data) + b * t.stride_batch + h * t.stride_head + row0 * t.stride_seq + 8 * group;
  if (absmax)
    chunk_block_sums<kBf16, D, true>(base, t.stride_seq, L, full, blocks, tail, threadIdx.x / kGroups, group,
                                     block_sums);
  else
    chunk_block_sums<kBf16, D, false>(base, t.stride_seq, L, full, blocks, tail, threadIdx.x / kGroups, group,
                                      block_sums);
  __syncthreads();
  if (threadIdx.x >= D) return;
  const int col = threadIdx.x;
  float s = 0.0f;  // level 1: the complete blocks, in order
  for (int blk = 0; blk < full; ++blk) {
    const float v = block_sums[blk * D + col];
    s = absmax ? fmaxf(s, v) : s + v;
  }
  float* out = p.partials + ((static_cast<long>(tensor) * p.batch_heads + bh) * (p.chunks + 1) + chunk) * D + col;
  out[0] = s;
  if (chunk == p.chunks - 1) out[D] = tail > 0 ? block_sums[full * D + col] : 0.0f;  // slot `chunks`
}

template <bool kBf16, int D>
__global__ void __launch_bounds__(256) mean_partial_kernel(const MeanParams p) {
  extern __shared__ float block_sums[];  // [L][D]
  const int chunk = static_cast<int>(blockIdx.x % static_cast<unsigned>(p.chunks));
  const int rest = static_cast<int>(blockIdx.x / static_cast<unsigned>(p.chunks));
  mean_chunk<kBf16, D>(p, rest / p.batch_heads, rest % p.batch_heads, chunk, block_sums);
}


// Means, pass 2, one thread per (tensor, batch-head, column): the complete chunks' level-1 sums
// are added in groups of L (level 2), the group sums in order (level 3); then
// ((trailing rows + short chunk's blocks) + unfinished level 2) + level 3, divided by the length
// in FP32.  Causal calls write a zero V mean.  SageAttention2++ (value_absmax): the V column's
// max |v| over the chunks gives its FP8 scale amax / 2.25 + 1e-7
// (sage_attention_2pp/reference.py:22-23: FP32 division, FP32 add).
__device__ __forceinline__ void finalize_column(const MeanParams& p, int tensor, int bh, int d, int head_dim) {
  const int rem = bh * head_dim + d;
  float* dst = tensor == 0 ? p.key_mean : p.value_mean;
  if (tensor >= p.tensors) {
    dst[rem] = 0.0f;
    return;
  }
  const float* src =
      p.partials + (static_cast<long>(tensor) * p.batch_heads + bh) * (p.chunks + 1) * head_dim + d;
  if (tensor == 1 && p.value_absmax) {
    float amax = 0.0f;
    for (int c = 0; c <= p.chunks; ++c) amax = fmaxf(amax, src[static_cast<long>(c) * head_dim]);
    p.value_scale[rem] = __fadd_rn(amax / 2.25f, 1e-7f);
    return;
  }
  const int block = p.block_rows;
  const int full = static_cast<int>(p.length / (static_cast<long>(block) * block));  // complete chunks
  float level2 = 0.0f, level3 = 0.0f;
  constexpr int kBatch = 16;  // loads in flight; the additions stay in chunk order
  int c = 0;
  for (; c + kBatch <= full; c += kBatch) {
    float part[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) part[i] = src[static_cast<long>(c + i) * head_dim];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      level2 += part[i];
      if ((c + i + 1) % block == 0) {
        level3 += level2;
        level2 = 0.0f;
      }
    }
  }
  for (; c < full; ++c) {
    level2 += src[static_cast<long>(c) * head_dim];
    if ((c + 1) % block == 0) {
      level3 += level2;
      level2 = 0.0f;
    }
  }
  const float level1 = full < p.chunks ? src[static_cast<long>(full) * head_dim] : 0.0f;
  const float level0 = src[static_cast<long>(p.chunks) * head_dim];
  const float total = ((level0 + level1) + level2) + level3;
  dst[rem] = total / static_cast<float>(p.length);
}

__global__ void __launch_bounds__(64) mean_finalize_kernel(const MeanParams p, int head_dim) {
  const int gid = blockIdx.x * 64 + threadIdx.x;
  if (gid == 0 && p.status != nullptr) *p.status = 0u;  // this path never waits
  const int per_tensor = p.batch_heads * head_dim;
  if (gid >= 2 * per_tensor) return;
  const int tensor = gid / per_tensor;
  const int rem = gid - tensor * per_tensor;
  finalize_column(p, tensor, rem / head_dim, rem % head_dim, head_dim);
}

// ---------------------------------------------------------------------------------------
// Quantisation.  Each wave owns one unit: a 32-row Q block, a 64-row K block or a 64-key V
// tile (a workgroup of 4 waves holds units of one kind only).  No LDS: V tiles are written
// transposed straight from registers.
// ---------------------------------------------------------------------------------------
// Q or K block of kRows rows.  Per block (the reference's "per_warp", sage/reference.py:61-77):
// one scale over kRows x D values.  Per thread group (its "per_thread", sage/reference.py:23-58):
// a 32-row Q block has 8 scales, row r in group r % 8 (rows {t, t+8, t+16, t+24}); a 64-row K
// block has 4, row r in group (r % 8) / 2 (rows {8a + 2t + c}).  The block's kSlots group scales
// go to scale_out (per block: the one scale repeated), and key tiles carry them in the padding
// of K row 0 as well (bytes [D, D + 4 * kSlots)).  Codes go to rows of kStride bytes (D for
// query codes, the padded tile stride for keys).
template <bool kBf16, int D, int kRows, bool kCenter, int kStride, int kSlots, bool kGuard>
__device__ __forceinline__ void quantize_block(const InputTensor& in, int b, int h, int row0, int length,
                                               const float* __restrict__ mean, int8_t* __restrict__ codes,
                                               float* __restrict__ scale_out, bool per_thread) {
  constexpr int kGroups = D / 8;
  constexpr int kRowsPerIter = kWave / kGroups;
  constexpr int kIters = kRows / kRowsPerIter;
  static_assert(kSlots == 1 || kSlots == (kRows == 32 ? 8 : 4), "one scale or one per thread group");
  const int lane = threadIdx.x & 63;
  const int group = lane % kGroups;
  const int sub = lane / kGroups;
  const uint16_t* base = static_cast<const uint16_t*>(in.data) + b * in.stride_batch + h * in.stride_head +
                         group * 8;
  float mu[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) mu[i] = kCenter ? mean[group * 8 + i] : 0.0f;

  uint4 raw[kIters];
  float amax[2] = {0.0f, 0.0f};  // by iteration parity: a lane's rows fall in at most two groups
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    const int row = row0 + it * kRowsPerIter + sub;
    raw[it] = !kGuard || row < length ? *reinterpret_cast<const uint4*>(base + static_cast<long>(row) * in.stride_seq)
                                      : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    const int row = row0 + it * kRowsPerIter + sub;
    float f[8];
    widen8<kBf16>(raw[it], f);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // padded rows are zero after centring (sage/reference.py:13-20 pads the centred K)
      const float x = !kGuard || row < length ? (kCenter ? f[i] - mu[i] : f[i]) : 0.0f;
      amax[it & 1] = fmaxf(amax[it & 1], fabsf(x));
    }
  }
  // group of row r = it * kRowsPerIter + sub within the block, for each iteration parity
  const auto group_of = [&](int parity) {
    const int r = (parity * kRowsPerIter + sub) & 7;
    return kRows == 32 ? r : r >> 1;
  };
  float scale[2];
  if (!per_thread) {
    scale[0] = scale[1] = scale_from_amax(wave_max(fmaxf(amax[0], amax[1])));
  } else {
    // lanes whose rows share a group: the kGroups column lanes of one sub-row (Q), or of the two
    // sub-rows 2j, 2j + 1 (K) -- aligned runs of lanes; at D = 64 both parities are one group
    constexpr int kShare = kGroups * (kRows == 32 ? 1 : 2);
    amax[0] = group_max<kShare>(amax[0]);
    amax[1] = group_max<kShare>(amax[1]);
    if (kRowsPerIter == 8) amax[0] = amax[1] = fmaxf(amax[0], amax[1]);
    scale[0] = scale_from_amax(amax[0]);
    scale[1] = scale_from_amax(amax[1]);
  }
  const Divisor divisor[2] = {Divisor(scale[0]), Divisor(scale[1])};
  // The second pass widens and centres again from the packed rows: an empty asm "redefines"
  // them, so the compiler cannot keep the first pass's 8 floats per row live instead (64 more
  // VGPRs, which would halve the waves per SIMD).
#pragma unroll
  for (int it = 0; it < kIters; ++it) asm volatile("" : "+v"(raw[it].x), "+v"(raw[it].y), "+v"(raw[it].z), "+v"(raw[it].w));
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    const int row = row0 + it * kRowsPerIter + sub;
    float f[8];
    widen8<kBf16>(raw[it], f);
    uint32_t c[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = !kGuard || row < length ? (kCenter ? f[i] - mu[i] : f[i]) : 0.0f;
      c[i] = code_word(x, divisor[it & 1]);
    }
    uint2 packed = make_uint2(pack_low_bytes(c[0], c[1], c[2], c[3]), pack_low_bytes(c[4], c[5], c[6], c[7]));
    *reinterpret_cast<uint2*>(codes + static_cast<long>(it * kRowsPerIter + sub) * kStride + group * 8) = packed;
  }
  // key tiles also carry their scales in the padding of K row 0 (bytes [D, D + 4 * kSlots))
  float* tile_scales = kStride != D ? reinterpret_cast<float*>(codes + D) : nullptr;
  if (!per_thread || kSlots == 1) {
    if (lane < kSlots) {
      scale_out[lane] = scale[0];
      if (tile_scales != nullptr) tile_scales[lane] = scale[0];
    }
  } else if (group == 0 && (kRows == 32 || (sub & 1) == 0)) {
    // one lane per (sub-row group, parity) writes its group's scale
#pragma unroll
    for (int parity = 0; parity < 2; ++parity) {
      scale_out[group_of(parity)] = scale[parity];
      if (tile_scales != nullptr) tile_scales[group_of(parity)] = scale[parity];
    }
  }
}

// V tile: per-key scales, codes written transposed from registers, tile column sums.  Lane
// (group, sub) owns columns [8 group, +8) of the kKeys consecutive keys [kKeys sub, +kKeys): its
// codes, packed four keys to a word, are the 16-byte (D = 128) or 8-byte (D = 64) pieces of its
// eight V^T rows -- no transpose through LDS.  A key's |v| maximum is reduced over the kGroups
// lanes of its row of lanes with DPP.  The code words fill the registers the raw rows free, so
// the kernel fits four waves per SIMD, which overlap one another's loads with their arithmetic.
template <int kLanes>
__device__ __forceinline__ float row_group_max(float v) {  // max over aligned groups of kLanes lanes (8 or 16)
  v = fmaxf(v, dpp<0xB1>(v));  // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp<0x4E>(v));  // quad_perm [2,3,0,1]
  if constexpr (kLanes == 8) {
    v = fmaxf(v, dpp<0x141>(v));  // row_half_mirror: lane i and 7 - i of each half row
  } else {
    static_assert(kLanes == 16, "8 or 16 lanes");
    v = fmaxf(v, dpp<0x124>(v));  // row_ror:4
    v = fmaxf(v, dpp<0x128>(v));  // row_ror:8
  }
  return v;
}

template <int kN, int kI = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {  // f(integral_constant<int, i>) for i = 0 .. kN - 1
  if constexpr (kI < kN) {
    f(std::integral_constant<int, kI>{});
    static_for<kN, kI + 1>(f);
  }
}

// `word`'s low byte placed at byte kByte of `packed` (v_perm_b32 selectors: 0-3 pick bytes of
// the second operand, 4 the first operand's byte 0)
template <int kByte>
__device__ __forceinline__ uint32_t insert_byte(uint32_t packed, uint32_t word) {
  constexpr uint32_t kSel = (0x03020100u & ~(0xffu << (8 * kByte))) | (0x04u << (8 * kByte));
  return __builtin_amdgcn_perm(word, packed, kSel);
}

// Rows [16 sub, +16) of a 64-row K block or V tile (8 rows at D = 64), columns [8 group, +8):
// lane (group, sub)'s share of the unit, every load in flight before any arithmetic.  Rows past
// the end read as zero.
template <int D, bool kGuard>
__device__ __forceinline__ void load_unit_rows(const InputTensor& in, int b, int h, int kb, int length, int lane,
                                               uint4 (&raw)[kKeyBlock / (kWave / (D / 8))]) {
  constexpr int kGroups = D / 8;
  constexpr int kKeys = kKeyBlock / (kWave / kGroups);
  const int group = lane % kGroups;
  const int key0 = (lane / kGroups) * kKeys;
  const uint16_t* base =
      static_cast<const uint16_t*>(in.data) + b * in.stride_batch + h * in.stride_head + group * 8;
#pragma unroll
  for (int j = 0; j < kKeys; ++j) {
    const int row = kb * kKeyBlock + key0 + j;
    raw[j] = !kGuard || row < length ? *reinterpret_cast<const uint4*>(base + static_cast<long>(row) * in.stride_seq)
                                     : make_uint4(0, 0, 0, 0);
  }
}

template <bool kBf16, int D, bool kGuard>
__device__ __forceinline__ void quantize_value_rows(const QuantParams& p, int unit, int lane,
                                                    uint4 (&raw)[kKeyBlock / (kWave / (D / 8))],
                                                    const float (&mu)[8]);

template <bool kBf16, int D, bool kGuard>
__device__ __forceinline__ void quantize_value_tile(const QuantParams& p, int unit, int lane) {
  constexpr int kGroups = D / 8;
  const int bh = unit / p.nkb;
  const int kb = unit - bh * p.nkb;
  const int b = bh / p.heads;
  const int h = bh - b * p.heads;
  const int group = lane % kGroups;
  uint4 raw[kKeyBlock / (kWave / kGroups)];
  load_unit_rows<D, kGuard>(p.value, b, h, kb, p.key_length, lane, raw);
  float mu[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) mu[i] = p.center_value ? p.value_mean[static_cast<long>(bh) * D + group * 8 + i] : 0.0f;
  quantize_value_rows<kBf16, D, kGuard>(p, unit, lane, raw, mu);
}

// The V tile `unit` from lane (group, sub)'s rows `raw` (load_unit_rows) centred by `mu` (its
// eight columns' means, zeros when uncentred).
template <bool kBf16, int D, bool kGuard>
__device__ __forceinline__ void quantize_value_rows(const QuantParams& p, int unit, int lane,
                                                    uint4 (&raw)[kKeyBlock / (kWave / (D / 8))],
                                                    const float (&mu)[8]) {
  constexpr int kGroups = D / 8;
  constexpr int kSubs = kWave / kGroups;
  constexpr int kKeys = kKeyBlock / kSubs;
  const int bh = unit / p.nkb;
  const int kb = unit - bh * p.nkb;
  const int group = lane % kGroups;
  const int sub = lane / kGroups;
  const int key0 = sub * kKeys;  // first key of this lane in the tile

  uint8_t* tile = p.kv_tiles + static_cast<long>(unit) * kv_tile_bytes(D);
  int colsum[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float own_scale = 0.0f;  // the scale of key key0 + group (lanes with group < kKeys), for the metadata
  uint32_t packed[8][kKeys / 4];  // [column][four keys]: filled as raw[] empties, so the two share registers
#pragma unroll
  for (int j4 = 0; j4 < kKeys / 4; ++j4) {
    static_for<4>([&](auto u) {
      const int j = 4 * j4 + u;
      const bool valid = !kGuard || kb * kKeyBlock + key0 + j < p.key_length;
      float x[8];
      widen8<kBf16>(raw[j], x);
      float m = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        x[i] = valid ? x[i] - mu[i] : 0.0f;
        m = fmaxf(m, fabsf(x[i]));
      }
      const float scale = scale_from_amax(row_group_max<kGroups>(m));
      const Divisor divisor(scale);
      if (group == j) own_scale = scale;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t word = code_word(x[i], divisor);
        if constexpr (u == 0)
          packed[i][j4] = word;  // bytes 1-3 are replaced by the next three keys
        else
          packed[i][j4] = insert_byte<u>(packed[i][j4], word);
      }
    });
#pragma unroll
    for (int i = 0; i < 8; ++i)
      colsum[i] = __builtin_amdgcn_sdot4(static_cast<int>(packed[i][j4]), 0x01010101, colsum[i], false);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint8_t* dst = tile + kv_v_offset(D) + (group * 8 + i) * kv_v_stride() + key0;
    if constexpr (kKeys == 16)
      *reinterpret_cast<uint4*>(dst) = make_uint4(packed[i][0], packed[i][1], packed[i][2], packed[i][3]);
    else
      *reinterpret_cast<uint2*>(dst) = make_uint2(packed[i][0], packed[i][1]);
  }
  // per-key metadata, one key per lane: lane (group, sub) with group < kKeys owns key key0 + group
  float* meta = reinterpret_cast<float*>(tile + kv_log_offset(D));
  if (group < kKeys) {
    const int row = kb * kKeyBlock + key0 + group;
    const bool valid = !kGuard || row < p.key_length;
    p.value_scale[static_cast<long>(bh) * p.sk64 + row] = valid ? own_scale : 0.0f;
    meta[key0 + group] = valid ? log2f(own_scale) : -__builtin_inff();
    meta[kKeyBlock + key0 + group] = valid ? 1.0f / (255.0f * own_scale) : 0.0f;
  }
  // column sums over the tile's 64 keys: the kSubs lanes sharing a group hold disjoint keys
#pragma unroll
  for (int m = kGroups; m < kWave; m <<= 1)
#pragma unroll
    for (int i = 0; i < 8; ++i) colsum[i] += __shfl_xor(colsum[i], m, kWave);
  if (sub == 0) {
    // |PV| <= 64 * 255 * 127 < 2^22, so the biased accumulator stays exact (common.h)
    int32_t* correction = reinterpret_cast<int32_t*>(tile + kv_corr_offset(D)) + group * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) correction[i] = 128 * colsum[i] + kAccBias;
  }
}

template <bool kBf16, int D>
__device__ __forceinline__ void quantize_query_unit(const QuantParams& p, int unit) {  // one 32-row Q block
  const int bh = unit / p.nqb;
  const int qb = unit - bh * p.nqb;
  const int b = bh / p.heads;
  const int h = bh - b * p.heads;
  int8_t* codes = p.query_code + (static_cast<long>(bh) * p.sq32 + qb * kQueryBlock) * D;
  float* scales = p.query_scale + static_cast<long>(unit) * kQueryScaleSlots;
  if ((qb + 1) * kQueryBlock <= p.query_length)
    quantize_block<kBf16, D, kQueryBlock, false, D, kQueryScaleSlots, false>(
        p.query, b, h, qb * kQueryBlock, p.query_length, nullptr, codes, scales, p.per_thread);
  else
    quantize_block<kBf16, D, kQueryBlock, false, D, kQueryScaleSlots, true>(
        p.query, b, h, qb * kQueryBlock, p.query_length, nullptr, codes, scales, p.per_thread);
}

template <bool kBf16, int D>
__device__ __forceinline__ void quantize_key_unit(const QuantParams& p, int unit) {  // one 64-row K block
  const int bh = unit / p.nkb;
  const int kb = unit - bh * p.nkb;
  const int b = bh / p.heads;
  const int h = bh - b * p.heads;
  int8_t* tile = reinterpret_cast<int8_t*>(p.kv_tiles) + static_cast<long>(unit) * kv_tile_bytes(D);
  const float* mean = p.key_mean + static_cast<long>(bh) * D;
  float* scales = p.key_scale + static_cast<long>(unit) * kKeyScaleSlots;
  if ((kb + 1) * kKeyBlock <= p.key_length)
    quantize_block<kBf16, D, kKeyBlock, true, kv_k_stride(D), kKeyScaleSlots, false>(
        p.key, b, h, kb * kKeyBlock, p.key_length, mean, tile, scales, p.per_thread);
  else
    quantize_block<kBf16, D, kKeyBlock, true, kv_k_stride(D), kKeyScaleSlots, true>(
        p.key, b, h, kb * kKeyBlock, p.key_length, mean, tile, scales, p.per_thread);
}

template <bool kBf16, int D>
__device__ __forceinline__ void quantize_value_unit(const QuantParams& p, int unit, int lane) {  // one 64-key V tile
  if ((unit % p.nkb + 1) * kKeyBlock <= p.key_length)
    quantize_value_tile<kBf16, D, false>(p, unit, lane);
  else
    quantize_value_tile<kBf16, D, true>(p, unit, lane);
}

// One wave per unit, four units of one kind per workgroup: Q blocks (two-step path), K blocks,
// V tiles.  Four waves per SIMD (at most 128 VGPRs) overlap one another's loads with their
// arithmetic.  Causal calls take the K blocks last-read-first: the mean pass has just read K (and
// only K), so the most recently read rows are still in the last-level cache.
template <bool kBf16, int D>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) quantize_kernel(const QuantParams p) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  int block = blockIdx.x;
  if (block < p.q_blocks_wg) {
    const int unit = block * 4 + wave;
    if (unit < p.batch_heads * p.nqb) quantize_query_unit<kBf16, D>(p, unit);
    return;
  }
  block -= p.q_blocks_wg;
  if (block < p.k_blocks_wg) {
    const int unit = (p.center_value ? block : p.k_blocks_wg - 1 - block) * 4 + wave;
    if (unit < p.batch_heads * p.nkb) quantize_key_unit<kBf16, D>(p, unit);
    return;
  }
  const int unit = (block - p.k_blocks_wg) * 4 + wave;
  if (unit < p.batch_heads * p.nkb) quantize_value_unit<kBf16, D>(p, unit, lane);
}

// ---------------------------------------------------------------------------------------
// Single-pass prep (D = 128, cascade blocks of L = 16 rows, at most kSinglePassChunks chunks per
// sequence): K and V are read from HBM once.  One workgroup per 256-row chunk of one batch-head's
// K or V: wave w holds rows [64 w, +64) of the chunk (the chunk's K block or V tile 4 c + w) in
// registers, lane (group, sub) the columns [8 group, +8) of rows [16 sub, +16) -- exactly one
// cascade level-0 block, which it sums in row order.  The chunk's level-1 sums are published
// (write-through stores) and counted on the batch-head tensor's arrival counter; the chunk that
// arrives last computes the mean (levels 2 and 3, the torch order of the mean pass above) and
// writes it over the pending marks the launch left in the mean buffer; the other chunks poll
// their columns until the marks are gone.  Every chunk then quantises its rows from registers.
// Causal V needs no mean and does not wait.
//
// Progress: a chunk waits only for chunks of its own batch-head tensor, whose workgroup ids are
// consecutive; ids are remapped with the device's XCC count so that each XCC runs a consecutive
// range (workgroups are dealt round-robin over the XCCs, and an XCC dispatches its share in
// order), so once the first chunk of a tensor runs, the rest are dispatched as soon as slots free
// up -- and the host takes this path only when a tensor's chunks fit in one XCC's slots (at least
// four workgroups per CU).  Other work holding an XCC's slots (a kernel on another stream, another
// process) can still keep a tensor's last chunk from being dispatched, so every wait is bounded:
// past the spin limit the chunk computes the mean itself from the rows in HBM in the same
// cascade order (column_mean_from_rows: exact, slow), and counts itself in the status word.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float load_coherent(const float* p) {  // agent-scope relaxed: bypasses L2
  return __builtin_bit_cast(float, __hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT));
}

__device__ __forceinline__ void store_coherent(float* p, float v) {  // agent-scope relaxed: written through
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// K block from registers (load_unit_rows at D = 128): centred by `mu`, per-thread-group scales
// (group of row r: (r % 8) / 2, i.e. (j % 8) / 2 for this lane's row 16 sub + j) or one per
// block, codes into the tile's K rows, scales to scale_out and to the padding of K row 0 --
// the same values as quantize_block, which takes the rows in another lane order.
template <bool kBf16, bool kGuard>
__device__ __forceinline__ void quantize_key_rows(uint4 (&raw)[16], const float (&mu)[8], int valid_rows,
                                                  int8_t* __restrict__ tile, float* __restrict__ scale_out,
                                                  bool per_thread, int lane) {
  constexpr int D = 128;
  constexpr int kStride = kv_k_stride(D);
  const int group = lane & 15;
  const int sub = lane >> 4;
  float am[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    float f[8];
    widen8<kBf16>(raw[j], f);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = !kGuard || j < valid_rows ? f[i] - mu[i] : 0.0f;
      am[(j & 7) >> 1] = fmaxf(am[(j & 7) >> 1], fabsf(x));
    }
  }
  float scale[4];
  if (per_thread) {
#pragma unroll
    for (int t = 0; t < 4; ++t) scale[t] = scale_from_amax(wave_max(am[t]));
  } else {
    scale[0] = scale_from_amax(wave_max(fmaxf(fmaxf(am[0], am[1]), fmaxf(am[2], am[3]))));
    scale[1] = scale[2] = scale[3] = scale[0];
  }
  const Divisor divisor[4] = {Divisor(scale[0]), Divisor(scale[1]), Divisor(scale[2]), Divisor(scale[3])};
  // widen and centre again from the packed rows (as quantize_block: keeps 128 floats out of VGPRs)
#pragma unroll
  for (int j = 0; j < 16; ++j) asm volatile("" : "+v"(raw[j].x), "+v"(raw[j].y), "+v"(raw[j].z), "+v"(raw[j].w));
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    float f[8];
    widen8<kBf16>(raw[j], f);
    uint32_t c[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = !kGuard || j < valid_rows ? f[i] - mu[i] : 0.0f;
      c[i] = code_word(x, divisor[(j & 7) >> 1]);
    }
    *reinterpret_cast<uint2*>(tile + (16 * sub + j) * kStride + 8 * group) =
        make_uint2(pack_low_bytes(c[0], c[1], c[2], c[3]), pack_low_bytes(c[4], c[5], c[6], c[7]));
  }
  if (lane == 0) {
    const float4 s4 = make_float4(scale[0], scale[1], scale[2], scale[3]);
    *reinterpret_cast<float4*>(scale_out) = s4;
    *reinterpret_cast<float4*>(tile + D) = s4;
  }
}

struct SinglePassParams {
  QuantParams q;
  MeanParams m;
  uint32_t* arrivals;  // [batch_heads][2] chunks arrived (zero before the launch)
  uint32_t* status;    // chunks whose wait gave up and computed the mean themselves (zero before the launch)
  int kv_workgroups;   // batch_heads * 2 * chunks; Q-block workgroups (4 blocks each) follow
  int xccs;            // XCCs the workgroups are dealt over (the remap's stride)
  int spin_limit;      // polls before a wait gives up (0: no wait, every waiter computes the mean)
};

constexpr int kSinglePassChunks = 128;  // 2^15 keys: at most 8 level-2 groups of 16 chunks

// The mean of column `col` of one batch-head's K or V straight from its rows in HBM, in the
// cascade order of the published partials and single_pass_mean (L = 16): rows summed in
// blocks of 16 from +0.0 (level 0), 16 blocks per chunk (level 1), 16 chunks per group (level
// 2), the groups in order (level 3), then ((trailing rows + the short chunk's complete blocks)
// + the unfinished group) + the complete groups, divided by the length in FP32.  Bit-identical
// to the published mean; the fallback of a wait that gives up (one thread per column).
template <bool kBf16>
__device__ float block_rows_sum(const uint16_t* rows, long stride, int n) {
  float v[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const uint32_t bits = r < n ? static_cast<uint32_t>(rows[static_cast<long>(r) * stride]) : 0u;
    v[r] = kBf16 ? __uint_as_float(bits << 16) : half_bits_to_float(bits);
  }
  float acc = 0.0f;
#pragma unroll
  for (int r = 0; r < 16; ++r)
    if (r < n) acc += v[r];
  return acc;
}

template <bool kBf16>
__device__ float column_mean_from_rows(const InputTensor& in, int b, int h, int col, int length) {
  constexpr int L = 16;
  const uint16_t* base = static_cast<const uint16_t*>(in.data) + b * in.stride_batch + h * in.stride_head + col;
  const long stride = in.stride_seq;
  const int full = length / (L * L);  // complete chunks
  float level3 = 0.0f, group = 0.0f;
  for (int c = 0; c < full; ++c) {
    float chunk_sum = 0.0f;
    for (int blk = 0; blk < L; ++blk)
      chunk_sum += block_rows_sum<kBf16>(base + static_cast<long>(c * L * L + blk * L) * stride, stride, L);
    group += chunk_sum;
    if ((c + 1) % L == 0) {
      level3 += group;
      group = 0.0f;
    }
  }
  const float level2 = full % L != 0 ? group : 0.0f;
  const int rows = length - full * L * L;  // the short chunk, if any
  const int blocks = rows / L;
  const int tail = rows - blocks * L;
  float level1 = 0.0f;
  for (int blk = 0; blk < blocks; ++blk)
    level1 += block_rows_sum<kBf16>(base + static_cast<long>(full * L * L + blk * L) * stride, stride, L);
  const float level0 =
      tail > 0 ? block_rows_sum<kBf16>(base + static_cast<long>(full * L * L + blocks * L) * stride, stride, tail)
               : 0.0f;
  const float total = ((level0 + level1) + level2) + level3;
  return total / static_cast<float>(length);
}
constexpr uint32_t kMeanPending = 0x7fa5a5a5u;  // a signalling NaN: the mean slot before it is published

// The mean of one column from the published partials, torch's cascade order (finalize_column),
// with two threads per column: thread `half` sums the level-2 groups half, half + 2, ... of L
// chunks each (one group's loads in flight together, the groups one after another to keep the
// chunk's rows in registers), the groups meet in LDS and thread 0 of the pair combines them in
// order.
__device__ __forceinline__ float single_pass_mean(const MeanParams& p, const float* src, int col, int half,
                                                  float (*group_sums)[128]) {
  constexpr int L = 16;
  const int full = p.length / (L * L);  // complete chunks
  const int groups = (full + L - 1) / L;  // level-2 groups (the last may be unfinished)
#pragma unroll 1
  for (int g = half; g < groups; g += 2) {
    const int c0 = g * L;
    const int n = min(L, full - c0);
    float part[L];
#pragma unroll
    for (int i = 0; i < L; ++i) part[i] = i < n ? load_coherent(src + static_cast<long>(c0 + i) * 128) : 0.0f;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < L; ++i)
      if (i < n) s += part[i];
    group_sums[g][col] = s;
  }
  __syncthreads();
  if (half != 0) return 0.0f;
  float level3 = 0.0f, level2 = 0.0f;
  for (int g = 0; g < groups; ++g) {
    if ((g + 1) * L <= full) level3 += group_sums[g][col];
    else level2 = group_sums[g][col];
  }
  const float level1 = full < p.chunks ? load_coherent(src + static_cast<long>(full) * 128) : 0.0f;
  const float level0 = load_coherent(src + static_cast<long>(p.chunks) * 128);
  const float total = ((level0 + level1) + level2) + level3;
  return total / static_cast<float>(p.length);
}

// LDS of a single-pass workgroup.
struct SinglePassShared {
  float block_sums[16][128];  // the chunk's level-0 sums
  float group_sums[kSinglePassChunks / 16][128];
  float mean[128];
  int last;
};

// One chunk of tensor kTensor (0: K, 1: V) of batch-head bh: load, cascade sums, mean, codes.
// The whole pipeline is inlined once per tensor so that each keeps its 64 VGPRs of rows in
// registers without the other's code in between; a unit that reaches past the end of the
// sequence (at most one per batch-head) loads its rows again, guarded, inside its own branch.
template <bool kBf16, int kTensor>
__device__ __forceinline__ void single_pass_chunk(const SinglePassParams& p, SinglePassShared& sh, int bh, int chunk,
                                                  int wave, int lane) {
  constexpr int D = 128;
  constexpr int L = 16;
  const int chunks = p.m.chunks;
  const int pair = 2 * bh + kTensor;
  const int b = bh / p.q.heads;
  const int h = bh - b * p.q.heads;
  const int length = p.q.key_length;
  const InputTensor& in = kTensor == 0 ? p.q.key : p.q.value;
  const int kb = chunk * 4 + wave;  // this wave's K block / V tile
  const int group = lane & 15;
  const int sub = lane >> 4;
  const int first_row = kb * kKeyBlock + sub * 16;  // this lane's rows [first_row, +16)
  const int valid_rows = max(0, min(16, length - first_row));
  const bool full_unit = (kb + 1) * kKeyBlock <= length;

  uint4 raw[16];
  if (full_unit) {
    load_unit_rows<D, false>(in, b, h, kb, length, lane, raw);
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) raw[j] = make_uint4(0, 0, 0, 0);
  }

  float* mean_out = (kTensor == 0 ? p.m.key_mean : p.m.value_mean) + static_cast<long>(bh) * D;
  const bool centred = kTensor == 0 || p.q.center_value;
  if (centred) {
    // level 0: this lane's block of L rows, in row order from +0.0 (a partial unit reads its
    // rows here with guards; they are read again for the codes)
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (full_unit) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float f[8];
        widen8<kBf16>(raw[j], f);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += f[i];
      }
    } else if (valid_rows > 0) {
      const uint16_t* rows = static_cast<const uint16_t*>(in.data) + b * in.stride_batch + h * in.stride_head +
                             static_cast<long>(first_row) * in.stride_seq + 8 * group;
      for (int j = 0; j < valid_rows; ++j) {
        float f[8];
        widen8<kBf16>(*reinterpret_cast<const uint4*>(rows + static_cast<long>(j) * in.stride_seq), f);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += f[i];
      }
    }
    float4* dst = reinterpret_cast<float4*>(&sh.block_sums[4 * wave + sub][8 * group]);
    dst[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    dst[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
    // the K codes widen the packed rows again: the 128 floats of this pass stay dead (the V
    // tile's register reuse needs no such hint)
    if constexpr (kTensor == 0) {
#pragma unroll
      for (int j = 0; j < 16; ++j) asm volatile("" : "+v"(raw[j].x), "+v"(raw[j].y), "+v"(raw[j].z), "+v"(raw[j].w));
    }
    __syncthreads();
    // level 1: the chunk's complete blocks in order; a short last chunk's trailing rows go to
    // slot `chunks` (mean_chunk's layout)
    const int rows = min(L * L, length - chunk * L * L);
    const int full = rows / L;
    const int tail = rows - full * L;
    float* src = p.m.partials + (static_cast<long>(pair) * (chunks + 1)) * D;
    if (threadIdx.x < D) {
      const int col = threadIdx.x;
      float s = 0.0f;
      for (int blk = 0; blk < full; ++blk) s += sh.block_sums[blk][col];
      store_coherent(src + static_cast<long>(chunk) * D + col, s);
      if (chunk == chunks - 1)
        store_coherent(src + static_cast<long>(chunks) * D + col, tail > 0 ? sh.block_sums[full][col] : 0.0f);
    }
    __builtin_amdgcn_s_waitcnt(0);  // the stores are complete before the arrival is counted
    __syncthreads();
    if (threadIdx.x == 0)
      sh.last = __hip_atomic_fetch_add(p.arrivals + pair, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                static_cast<uint32_t>(chunks - 1);
    __syncthreads();
    if (sh.last) {
      const int col = threadIdx.x & (D - 1);
      const float m = single_pass_mean(p.m, src + col, col, threadIdx.x >> 7, sh.group_sums);
      if (threadIdx.x < D) {
        sh.mean[col] = m;
        store_coherent(mean_out + col, m);  // replaces the pending mark: the other chunks go on
      }
    } else {
      // wait for this column's mean to replace the pending mark (kMeanPending, a signalling NaN
      // that no arithmetic produces), at most spin_limit polls
      bool waiting = false;
      if (threadIdx.x < D) {
        uint32_t bits = kMeanPending;
        for (int polls = 0; polls < p.spin_limit; ++polls) {
          bits = __hip_atomic_load(reinterpret_cast<const uint32_t*>(mean_out) + threadIdx.x, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
          if (bits != kMeanPending) break;
          __builtin_amdgcn_s_sleep(2);
        }
        waiting = bits == kMeanPending;
        sh.mean[threadIdx.x] = __builtin_bit_cast(float, bits);
      }
      // a column still pending: the chunk computes every column's mean from the rows itself
      if (__syncthreads_or(waiting)) {
        if (threadIdx.x < D) sh.mean[threadIdx.x] = column_mean_from_rows<kBf16>(in, b, h, threadIdx.x, length);
        if (threadIdx.x == 0) __hip_atomic_fetch_add(p.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __syncthreads();
  } else if (chunk == 0 && threadIdx.x < D) {
    mean_out[threadIdx.x] = 0.0f;  // causal: V is not centred, its mean slot reads zero
  }
  if (kb >= p.q.nkb) return;

  float mu[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) mu[i] = centred ? sh.mean[8 * group + i] : 0.0f;
  const int unit = bh * p.q.nkb + kb;
  if constexpr (kTensor == 0) {
    int8_t* tile = reinterpret_cast<int8_t*>(p.q.kv_tiles) + static_cast<long>(unit) * kv_tile_bytes(D);
    float* scales = p.q.key_scale + static_cast<long>(unit) * kKeyScaleSlots;
    if (full_unit) {
      quantize_key_rows<kBf16, false>(raw, mu, valid_rows, tile, scales, p.q.per_thread, lane);
    } else {
      uint4 rows[16];
      load_unit_rows<D, true>(in, b, h, kb, length, lane, rows);
      quantize_key_rows<kBf16, true>(rows, mu, valid_rows, tile, scales, p.q.per_thread, lane);
    }
  } else {
    if (full_unit) {
      quantize_value_rows<kBf16, D, false>(p.q, unit, lane, raw, mu);
    } else {
      uint4 rows[16];
      load_unit_rows<D, true>(in, b, h, kb, length, lane, rows);
      quantize_value_rows<kBf16, D, true>(p.q, unit, lane, rows, mu);
    }
  }
}

template <bool kBf16>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4)))
prep_single_pass_kernel(const SinglePassParams p) {
  __shared__ __attribute__((aligned(16))) SinglePassShared sh;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: index math stays scalar
  const int lane = threadIdx.x & 63;
  const int logical = xcc_remap(blockIdx.x, gridDim.x, p.xccs);
  if (logical >= p.kv_workgroups) {  // the two-step path's Q blocks: no mean, no wait
    const int unit = (logical - p.kv_workgroups) * 4 + wave;
    if (unit < p.q.batch_heads * p.q.nqb) quantize_query_unit<kBf16, 128>(p.q, unit);
    return;
  }
  const int pair = logical / p.m.chunks;  // (batch-head, tensor): K and V of a batch-head are neighbours
  const int chunk = logical - pair * p.m.chunks;
  if (pair & 1) single_pass_chunk<kBf16, 1>(p, sh, pair >> 1, chunk, wave, lane);
  else single_pass_chunk<kBf16, 0>(p, sh, pair >> 1, chunk, wave, lane);
}

// Before the single-pass prep: arrival counters and status word cleared, the means marked
// pending (the V mean only when V is centred).
__global__ void __launch_bounds__(256) prep_clear_kernel(uint32_t* words, int count, float* key_mean, float* value_mean,
                                                         int means, int centre_value) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < count) words[i] = 0u;
  if (i < means) {
    key_mean[i] = __builtin_bit_cast(float, kMeanPending);
    if (centre_value) value_mean[i] = __builtin_bit_cast(float, kMeanPending);
  }
}

// ---------------------------------------------------------------------------------------
// SageAttention2++ quantisation (sage_attention_2pp/reference.py:22-25, 44-49).  Each wave
// owns a 64-row K block (the Piper K path, into the SageAttention2++ tile record) or a
// 64-key V tile: FP8 E4M3 codes of v / scale[channel] (the correctly rounded FP32 quotient,
// then v_cvt_pk_fp8_f32: round to nearest even, bit-identical to torch's float8_e4m3fn
// cast), written transposed into the record's V^T rows.  Keys past the end get code 0.
// ---------------------------------------------------------------------------------------
template <bool kBf16, int D>
__global__ void __launch_bounds__(256) sage_quantize_kernel(const SageQuantParams p) {

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int block = blockIdx.x;

  if (block < p.k_blocks_wg) {
    const int unit = block * 4 + wave;
    if (unit >= p.batch_heads * p.nkb) return;
    const int bh = unit / p.nkb;
    const int kb = unit - bh * p.nkb;
    const int b = bh / p.heads;
    const int h = bh - b * p.heads;
    int8_t* tile = reinterpret_cast<int8_t*>(p.kv_tiles) + static_cast<long>(unit) * sage_tile_bytes(D);
    const float* mean = p.key_mean + static_cast<long>(bh) * D;
    float* scales = p.key_scale + static_cast<long>(unit) * kKeyScaleSlots;
    if ((kb + 1) * kKeyBlock <= p.key_length)
      quantize_block<kBf16, D, kKeyBlock, true, kv_k_stride(D), kKeyScaleSlots, false>(
          p.key, b, h, kb * kKeyBlock, p.key_length, mean, tile, scales, p.per_thread);
    else
      quantize_block<kBf16, D, kKeyBlock, true, kv_k_stride(D), kKeyScaleSlots, true>(
          p.key, b, h, kb * kKeyBlock, p.key_length, mean, tile, scales, p.per_thread);
    return;
  }

  // V tile: lane (group, sub) owns columns [8 group, +8) of the kKeys consecutive keys
  // [kKeys sub, +kKeys), converts them with the per-channel divisors and packs four keys of a
  // column per word: the 16-byte (D = 128) or 8-byte (D = 64) pieces of its eight V^T rows.
  const int unit = (block - p.k_blocks_wg) * 4 + wave;
  if (unit >= p.batch_heads * p.nkb) return;
  const int bh = unit / p.nkb;
  const int kb = unit - bh * p.nkb;
  const int b = bh / p.heads;
  const int h = bh - b * p.heads;
  constexpr int kGroups = D / 8;
  constexpr int kSubs = kWave / kGroups;
  constexpr int kKeys = kKeyBlock / kSubs;
  const int group = lane % kGroups;
  const int sub = lane / kGroups;
  const int key0 = sub * kKeys;
  const uint16_t* base = static_cast<const uint16_t*>(p.value.data) + b * p.value.stride_batch +
                         h * p.value.stride_head + group * 8;
  uint4 raw[kKeys];
#pragma unroll
  for (int j = 0; j < kKeys; ++j) {
    const int row = kb * kKeyBlock + key0 + j;
    raw[j] = row < p.key_length ? *reinterpret_cast<const uint4*>(base + static_cast<long>(row) * p.value.stride_seq)
                                : make_uint4(0, 0, 0, 0);
  }
  Divisor divisor[8];  // this lane's 8 channels
#pragma unroll
  for (int i = 0; i < 8; ++i) divisor[i] = Divisor(p.value_scale[static_cast<long>(bh) * D + group * 8 + i]);
  uint32_t packed[8][kKeys / 4];  // [column][four keys]
#pragma unroll
  for (int j4 = 0; j4 < kKeys / 4; ++j4) {
    float q[4][8];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float f[8];
      widen8<kBf16>(raw[4 * j4 + u], f);
#pragma unroll
      for (int i = 0; i < 8; ++i) q[u][i] = divisor[i].quotient(f[i]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[0][i], q[1][i], 0, false);
      packed[i][j4] = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(q[2][i], q[3][i], lo, true));
    }
  }
  uint8_t* tile = p.kv_tiles + static_cast<long>(unit) * sage_tile_bytes(D);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint8_t* dst = tile + sage_v_offset(D) + (group * 8 + i) * kv_v_stride() + key0;
    if constexpr (kKeys == 16)
      *reinterpret_cast<uint4*>(dst) = make_uint4(packed[i][0], packed[i][1], packed[i][2], packed[i][3]);
    else
      *reinterpret_cast<uint2*>(dst) = make_uint2(packed[i][0], packed[i][1]);
  }
}

// ---------------------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------------------
template <bool kBf16, int D>
static hipError_t launch_mean_partials(const MeanParams& mp, hipStream_t stream) {
  // one workgroup per (tensor, batch-head, chunk); LDS holds the chunk's L block sums of D columns
  const long workgroups = static_cast<long>(mp.tensors) * mp.batch_heads * mp.chunks;
  const size_t lds = static_cast<size_t>(mp.block_rows) * D * sizeof(float);
  hipLaunchKernelGGL((mean_partial_kernel<kBf16, D>), dim3(static_cast<unsigned>(workgroups)), dim3(256), lds, stream,
                     mp);
  return hipGetLastError();
}

template <bool kBf16, int D>
static hipError_t launch_prep_typed(const MeanParams& mp, const QuantParams& qp, const PrepDevice& dev,
                                    hipStream_t stream) {
  if (D == 128 && mp.block_rows == 16 && mp.chunks <= kSinglePassChunks && !mp.value_absmax &&
      single_pass_resident(mp.chunks, dev.cus, dev.xccs)) {
    SinglePassParams sp{};
    sp.q = qp;
    sp.m = mp;
    const int words = static_cast<int>(prep_sync_words(mp.batch_heads));
    uint32_t* sync = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(mp.partials) +
                                                 prep_partial_bytes(mp.batch_heads, mp.length, D));
    sp.arrivals = sync;
    sp.status = sync + prep_status_word(mp.batch_heads);
    sp.kv_workgroups = 2 * mp.batch_heads * mp.chunks;
    sp.xccs = dev.xccs;
    sp.spin_limit = dev.spin_limit;
    // a fill kernel, not hipMemsetAsync: safe to record in a captured graph
    const int means = mp.batch_heads * D;
    const int threads = words > means ? words : means;
    hipLaunchKernelGGL(prep_clear_kernel, dim3((threads + 255) / 256), dim3(256), 0, stream, sync, words, mp.key_mean,
                       mp.value_mean, means, qp.center_value);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    const long workgroups = static_cast<long>(sp.kv_workgroups) + qp.q_blocks_wg;
    hipLaunchKernelGGL((prep_single_pass_kernel<kBf16>), dim3(static_cast<unsigned>(workgroups)), dim3(256), 0, stream,
                       sp);
    return hipGetLastError();
  }
  hipError_t err = launch_mean_partials<kBf16, D>(mp, stream);
  if (err != hipSuccess) return err;
  const int fin_threads = 2 * mp.batch_heads * D;
  hipLaunchKernelGGL(mean_finalize_kernel, dim3((fin_threads + 63) / 64), dim3(64), 0, stream, mp, D);
  err = hipGetLastError();
  if (err != hipSuccess) return err;
  const int blocks = qp.q_blocks_wg + qp.k_blocks_wg + qp.v_blocks_wg;
  hipLaunchKernelGGL((quantize_kernel<kBf16, D>), dim3(blocks), dim3(256), 0, stream, qp);
  return hipGetLastError();
}

template <bool kBf16, int D>
static hipError_t launch_sage_prep_typed(const MeanParams& mp, const SageQuantParams& qp, hipStream_t stream) {
  hipError_t err = launch_mean_partials<kBf16, D>(mp, stream);
  if (err != hipSuccess) return err;
  const int fin_threads = 2 * mp.batch_heads * D;
  hipLaunchKernelGGL(mean_finalize_kernel, dim3((fin_threads + 63) / 64), dim3(64), 0, stream, mp, D);
  err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL((sage_quantize_kernel<kBf16, D>), dim3(qp.k_blocks_wg + qp.v_blocks_wg), dim3(256), 0, stream,
                     qp);
  return hipGetLastError();
}

hipError_t launch_sage_prep(bool bf16, int head_dim, const MeanParams& mp, const SageQuantParams& qp,
                            hipStream_t stream) {
  if (bf16) {
    return head_dim == 128 ? launch_sage_prep_typed<true, 128>(mp, qp, stream)
                           : launch_sage_prep_typed<true, 64>(mp, qp, stream);
  }
  return head_dim == 128 ? launch_sage_prep_typed<false, 128>(mp, qp, stream)
                         : launch_sage_prep_typed<false, 64>(mp, qp, stream);
}

hipError_t launch_prep(bool bf16, int head_dim, const MeanParams& mp, const QuantParams& qp, const PrepDevice& dev,
                       hipStream_t stream) {
  if (bf16) {
    return head_dim == 128 ? launch_prep_typed<true, 128>(mp, qp, dev, stream)
                           : launch_prep_typed<true, 64>(mp, qp, dev, stream);
  }
  return head_dim == 128 ? launch_prep_typed<false, 128>(mp, qp, dev, stream)
                         : launch_prep_typed<false, 64>(mp, qp, dev, stream);
}

}  // namespace piper
