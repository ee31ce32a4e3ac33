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

namespace piper {

// ---------------------------------------------------------------------------------------
// Means, pass 1: one thread owns a column pair of one chunk of L^2 rows of K (tensor 0) or V
// (tensor 1).  It sums each L-row block in row order and the chunk's complete blocks in block
// order (the first two cascade levels); the thread of the last chunk also sums the trailing
// length % L rows.  SageAttention2++'s V statistic is the per-column max |v| instead (exact in
// any order).
// ---------------------------------------------------------------------------------------
template <bool kBf16>
__device__ __forceinline__ float2 widen_pair(uint32_t bits) {
  if constexpr (kBf16) return make_float2(__uint_as_float(bits << 16), __uint_as_float(bits & 0xffff0000u));
  return make_float2(half_bits_to_float(bits & 0xffffu), half_bits_to_float(bits >> 16));
}

template <bool kBf16, int D>
__global__ void __launch_bounds__(256) mean_partial_kernel(const MeanParams p) {
  constexpr int kPairs = D / 2;
  constexpr int kUnroll = 16;  // loads in flight; L is a power of two >= 16
  const long gid = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  const long per_tensor = static_cast<long>(p.batch_heads) * p.chunks * kPairs;
  if (gid >= per_tensor * p.tensors) return;
  const int tensor = static_cast<int>(gid / per_tensor);
  const long rem = gid - tensor * per_tensor;
  const int pair = static_cast<int>(rem % kPairs);
  const int chunk = static_cast<int>((rem / kPairs) % p.chunks);
  const int bh = static_cast<int>(rem / (static_cast<long>(kPairs) * p.chunks));
  const int b = bh / p.heads;
  const int h = bh - b * p.heads;

  const InputTensor& t = tensor == 0 ? p.key : p.value;
  // two adjacent 16-bit elements per 4-byte load (rows are 16-byte aligned, so the pair is too)
  const uint16_t* base = static_cast<const uint16_t*>(t.data) + b * t.stride_batch + h * t.stride_head + 2 * pair;
  const int block = p.block_rows;
  const long chunk_rows = static_cast<long>(block) * block;
  const int row0 = static_cast<int>(chunk * chunk_rows);
  const int row1 = static_cast<int>(min(row0 + chunk_rows, static_cast<long>(p.length)));
  const int blocks = (row1 - row0) / block;
  const bool absmax = tensor == 1 && p.value_absmax;

  float s0 = 0.0f, s1 = 0.0f;  // level 1: complete blocks of this chunk, in order
  int row = row0;
  for (int blk = 0; blk < blocks; ++blk) {
    float b0 = 0.0f, b1 = 0.0f;  // level 0: the block's rows, in order
    for (int r = 0; r < block; r += kUnroll) {
      uint32_t raw[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
        raw[u] = *reinterpret_cast<const uint32_t*>(base + static_cast<long>(row + u) * t.stride_seq);
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const float2 f = widen_pair<kBf16>(raw[u]);
        if (absmax) {
          b0 = fmaxf(b0, fabsf(f.x));
          b1 = fmaxf(b1, fabsf(f.y));
        } else {
          b0 += f.x;
          b1 += f.y;
        }
      }
      row += kUnroll;
    }
    if (absmax) {
      s0 = fmaxf(s0, b0);
      s1 = fmaxf(s1, b1);
    } else {
      s0 += b0;
      s1 += b1;
    }
  }
  float* out = p.partials + ((static_cast<long>(tensor) * p.batch_heads + bh) * (p.chunks + 1) + chunk) * D + 2 * pair;
  out[0] = s0;
  out[1] = s1;
  if (chunk == p.chunks - 1) {  // the trailing rows, summed in order from +0.0 (slot `chunks`)
    float a0 = 0.0f, a1 = 0.0f;
    for (; row < row1; ++row) {
      const float2 f = widen_pair<kBf16>(*reinterpret_cast<const uint32_t*>(base + static_cast<long>(row) * t.stride_seq));
      if (absmax) {
        a0 = fmaxf(a0, fabsf(f.x));
        a1 = fmaxf(a1, fabsf(f.y));
      } else {
        a0 += f.x;
        a1 += f.y;
      }
    }
    out[D] = a0;
    out[D + 1] = a1;
  }
}

// Means, pass 2, one thread per (tensor, batch-head, column): the complete chunks' level-1 sums
// are added in groups of L (level 2), the group sums in order (level 3); then
// ((trailing rows + short chunk's blocks) + unfinished level 2) + level 3, divided by the length
// in FP32.  Causal calls write a zero V mean.  SageAttention2++ (value_absmax): the V column's
// max |v| over the chunks gives its FP8 scale amax / 2.25 + 1e-7
// (sage_attention_2pp/reference.py:22-23: FP32 division, FP32 add).
__global__ void __launch_bounds__(64) mean_finalize_kernel(const MeanParams p, int head_dim) {
  const int gid = blockIdx.x * 64 + threadIdx.x;
  const int per_tensor = p.batch_heads * head_dim;
  if (gid >= 2 * per_tensor) return;
  const int tensor = gid / per_tensor;
  const int rem = gid - tensor * per_tensor;
  float* dst = tensor == 0 ? p.key_mean : p.value_mean;
  if (tensor >= p.tensors) {
    dst[rem] = 0.0f;
    return;
  }
  const int bh = rem / head_dim;
  const int d = rem - bh * head_dim;
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
template <bool kBf16, int D, int kRows, bool kCenter, int kStride, int kSlots>
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
    raw[it] = row < length ? *reinterpret_cast<const uint4*>(base + static_cast<long>(row) * in.stride_seq)
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
      const float x = row < length ? (kCenter ? f[i] - mu[i] : f[i]) : 0.0f;
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
#pragma unroll
  for (int it = 0; it < kIters; ++it) {
    const int row = row0 + it * kRowsPerIter + sub;
    float f[8];
    widen8<kBf16>(raw[it], f);
    uint32_t c[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = row < length ? (kCenter ? f[i] - mu[i] : f[i]) : 0.0f;
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

template <bool kBf16, int D>
__global__ void __launch_bounds__(256) quantize_kernel(const QuantParams p) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int block = blockIdx.x;

  if (block < p.q_blocks_wg) {
    const int unit = block * 4 + wave;
    if (unit >= p.batch_heads * p.nqb) return;
    const int bh = unit / p.nqb;
    const int qb = unit - bh * p.nqb;
    const int b = bh / p.heads;
    const int h = bh - b * p.heads;
    quantize_block<kBf16, D, kQueryBlock, false, D, kQueryScaleSlots>(
        p.query, b, h, qb * kQueryBlock, p.query_length, nullptr,
        p.query_code + (static_cast<long>(bh) * p.sq32 + qb * kQueryBlock) * D,
        p.query_scale + static_cast<long>(unit) * kQueryScaleSlots, p.per_thread);
    return;
  }
  if (block < p.q_blocks_wg + p.k_blocks_wg) {
    const int unit = (block - p.q_blocks_wg) * 4 + wave;
    if (unit >= p.batch_heads * p.nkb) return;
    const int bh = unit / p.nkb;
    const int kb = unit - bh * p.nkb;
    const int b = bh / p.heads;
    const int h = bh - b * p.heads;
    int8_t* tile = reinterpret_cast<int8_t*>(p.kv_tiles) + static_cast<long>(unit) * kv_tile_bytes(D);
    quantize_block<kBf16, D, kKeyBlock, true, kv_k_stride(D), kKeyScaleSlots>(
        p.key, b, h, kb * kKeyBlock, p.key_length, p.key_mean + static_cast<long>(bh) * D, tile,
        p.key_scale + static_cast<long>(unit) * kKeyScaleSlots, p.per_thread);
    return;
  }

  // ---- V tile: per-key scales, codes written transposed from registers, tile column sums ----
  const int unit = (block - p.q_blocks_wg - p.k_blocks_wg) * 4 + wave;
  if (unit >= p.batch_heads * p.nkb) return;
  const int bh = unit / p.nkb;
  const int kb = unit - bh * p.nkb;
  const int b = bh / p.heads;
  const int h = bh - b * p.heads;
  // lane (group, sub) owns columns [8 group, +8) of the kKeys consecutive keys
  // [kKeys sub, +kKeys): its codes, packed four keys to a word, are the 16-byte (D = 128) or
  // 8-byte (D = 64) pieces of its eight V^T rows -- no transpose through LDS.
  constexpr int kGroups = D / 8;
  constexpr int kSubs = kWave / kGroups;
  constexpr int kKeys = kKeyBlock / kSubs;
  const int group = lane % kGroups;
  const int sub = lane / kGroups;
  const int key0 = sub * kKeys;  // first key of this lane in the tile
  const uint16_t* base = static_cast<const uint16_t*>(p.value.data) + b * p.value.stride_batch +
                         h * p.value.stride_head + group * 8;
  uint4 raw[kKeys];  // every row in flight before any arithmetic
#pragma unroll
  for (int j = 0; j < kKeys; ++j) {
    const int row = kb * kKeyBlock + key0 + j;
    raw[j] = row < p.key_length ? *reinterpret_cast<const uint4*>(base + static_cast<long>(row) * p.value.stride_seq)
                                : make_uint4(0, 0, 0, 0);
  }
  float mu[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) mu[i] = p.center_value ? p.value_mean[static_cast<long>(bh) * D + group * 8 + i] : 0.0f;
  uint8_t* tile = p.kv_tiles + static_cast<long>(unit) * kv_tile_bytes(D);
  float* meta = reinterpret_cast<float*>(tile + kv_log_offset(D));
  uint32_t packed[8][kKeys / 4];  // [column][four keys]
  int colsum[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float own_scale = 0.0f;  // the scale of key key0 + group (lane group < kKeys), for the metadata
#pragma unroll
  for (int j4 = 0; j4 < kKeys / 4; ++j4) {
    uint32_t word[4][8];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = 4 * j4 + u;
      const int row = kb * kKeyBlock + key0 + j;
      const bool valid = row < p.key_length;
      float f[8];
      widen8<kBf16>(raw[j], f);
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        f[i] = valid ? f[i] - mu[i] : 0.0f;
        amax = fmaxf(amax, fabsf(f[i]));
      }
      amax = group_max<kGroups>(amax);
      const float scale = scale_from_amax(amax);
      const Divisor divisor(scale);
#pragma unroll
      for (int i = 0; i < 8; ++i) word[u][i] = code_word(f[i], divisor);
      if (group == j) own_scale = scale;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      packed[i][j4] = pack_low_bytes(word[0][i], word[1][i], word[2][i], word[3][i]);
      colsum[i] = __builtin_amdgcn_sdot4(static_cast<int>(packed[i][j4]), 0x01010101, colsum[i], false);
    }
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
  if (group < kKeys) {
    const int row = kb * kKeyBlock + key0 + group;
    const bool valid = row < p.key_length;
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
    quantize_block<kBf16, D, kKeyBlock, true, kv_k_stride(D), kKeyScaleSlots>(
        p.key, b, h, kb * kKeyBlock, p.key_length, p.key_mean + static_cast<long>(bh) * D, tile,
        p.key_scale + static_cast<long>(unit) * kKeyScaleSlots, p.per_thread);
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
static hipError_t launch_prep_typed(const MeanParams& mp, const QuantParams& qp, hipStream_t stream) {
  const long mean_threads = static_cast<long>(mp.batch_heads) * mp.chunks * (D / 2) * mp.tensors;
  hipLaunchKernelGGL((mean_partial_kernel<kBf16, D>), dim3(static_cast<unsigned>((mean_threads + 255) / 256)),
                     dim3(256), 0, stream, mp);
  hipError_t err = hipGetLastError();
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
  const long stat_threads = static_cast<long>(mp.batch_heads) * mp.chunks * (D / 2) * mp.tensors;
  hipLaunchKernelGGL((mean_partial_kernel<kBf16, D>), dim3(static_cast<unsigned>((stat_threads + 255) / 256)),
                     dim3(256), 0, stream, mp);
  hipError_t err = hipGetLastError();
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

hipError_t launch_prep(bool bf16, int head_dim, const MeanParams& mp, const QuantParams& qp, hipStream_t stream) {
  if (bf16) {
    return head_dim == 128 ? launch_prep_typed<true, 128>(mp, qp, stream) : launch_prep_typed<true, 64>(mp, qp, stream);
  }
  return head_dim == 128 ? launch_prep_typed<false, 128>(mp, qp, stream) : launch_prep_typed<false, 64>(mp, qp, stream);
}

}  // namespace piper
