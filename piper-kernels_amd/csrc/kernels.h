// Kernel parameter blocks and launchers shared by the C ABI and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace piper {

constexpr int kMeanLevels = 4;  // accumulator levels of torch's CPU cascade sum

// The K/V sequence means follow torch's CPU FP32 reduction order (the reference's
// torch.mean(dim=2), piper_attention/reference.py:50, sage/reference.py:89): rows are summed in
// blocks of L = cascade_block_rows(S) rows, L consecutive blocks form a level-1 sum over a
// chunk of L^2 rows, L consecutive level-1 sums form a level-2 sum, and the level-2 sums are
// added in order; trailing rows and unfinished levels are combined at the end as
// ((rows + level 1) + level 2) + level 3.  Every partial starts from +0.0 and every addition
// is one FP32 rounding; the mean is that sum divided by S in FP32.
__host__ __device__ inline int cascade_block_rows(int length) {
  const int ceil_log2 = length > 1 ? 32 - __builtin_clz(static_cast<unsigned>(length - 1)) : 0;
  const int power = ceil_log2 / kMeanLevels > 4 ? ceil_log2 / kMeanLevels : 4;
  return 1 << power;
}

__host__ __device__ inline int cascade_chunks(int length) {  // chunks of L^2 rows, the last may be short
  const long rows = static_cast<long>(cascade_block_rows(length)) * cascade_block_rows(length);
  return static_cast<int>((length + rows - 1) / rows);
}

// Workspace of piper_prepare: the mean partials ([2][batch_heads][chunks + 1][D] floats), then
// the single-pass prep's sync words (an arrival counter per batch-head tensor, a status word;
// the rest is spare, padding to 16 bytes).
inline long prep_partial_bytes(long batch_heads, int length, int head_dim) {
  return 2 * batch_heads * (cascade_chunks(length) + 1) * head_dim * 4;
}
inline long prep_sync_words(long batch_heads) { return 4 * batch_heads + 4; }
// Index of the status word among the sync words (after the 2 * batch_heads arrival counters):
// the number of chunks of the last call that gave up waiting and computed their mean themselves.
inline long prep_status_word(long batch_heads) { return 2 * batch_heads; }

// One 64-key tile record is byte for byte the attention kernel's LDS stage, so it is copied
// with direct global -> LDS loads in 1 KiB pieces: K codes [64][D] in rows of D + 16 bytes,
// V^T codes [D][64] in rows of 80 bytes (the 16 spare bytes per row spread LDS banks), 64
// log2 scales, 64 inverse multipliers, D biased corrections, padded to a KiB multiple.
// Bytes [D, D + 4) (padding of K row 0) hold the tile's K scale; other padding is unspecified.
constexpr int kv_k_stride(int head_dim) { return head_dim + 16; }
constexpr int kv_v_stride() { return 64 + 16; }
constexpr int kv_v_offset(int head_dim) { return 64 * kv_k_stride(head_dim); }
constexpr int kv_log_offset(int head_dim) { return kv_v_offset(head_dim) + head_dim * kv_v_stride(); }
constexpr int kv_inv_offset(int head_dim) { return kv_log_offset(head_dim) + 256; }
constexpr int kv_corr_offset(int head_dim) { return kv_inv_offset(head_dim) + 256; }
constexpr int kv_tile_bytes(int head_dim) { return (kv_corr_offset(head_dim) + 4 * head_dim + 1023) / 1024 * 1024; }

// SageAttention2++ tile record: the same K rows (and K scale in the padding of row 0),
// then FP8 E4M3 V^T codes [D][64] in rows of 80 bytes; no softmax metadata (the V scale is
// per channel and applied in the epilogue).  A whole number of KiB for D = 64 and 128.
constexpr int sage_v_offset(int head_dim) { return 64 * kv_k_stride(head_dim); }
constexpr int sage_tile_bytes(int head_dim) {
  return (sage_v_offset(head_dim) + head_dim * kv_v_stride() + 1023) / 1024 * 1024;
}

struct InputTensor {
  const void* data;  // 16-bit floats; the head_dim axis is contiguous
  long stride_batch;  // element strides
  long stride_head;
  long stride_seq;
};

struct MeanParams {
  InputTensor key;
  InputTensor value;
  // [tensors][batch_heads][chunks + 1][D]: the level-1 sum of each chunk of L^2 rows (for a
  // short last chunk, the sum of its complete L-row blocks), then the sum of the trailing
  // length % L rows; SageAttention2++'s V slots hold per-chunk max |v| instead
  float* partials;
  float* key_mean;   // [batch_heads][D]
  float* value_mean; // [batch_heads][D]
  int batch_heads;
  int heads;
  int length;  // key length
  int block_rows;  // L = cascade_block_rows(length)
  int chunks;      // cascade_chunks(length)
  int tensors; // 1 = K only (causal), 2 = K and V
  // 1: the V statistic is the per-column max of |v| (SageAttention2++), finalised into
  // value_scale = amax / 2.25 + 1e-7; 0: the V sum, finalised into value_mean
  int value_absmax;
  float* value_scale;  // [batch_heads][D] (value_absmax only)
  uint32_t* status;    // the prep's give-up count, cleared by the finalisation (NULL: none)
};

// Scales stored per quantisation block: one per thread group of the reference's per_thread
// granularity (8 per 32-row Q block, 4 per 64-row K block); per-block quantisation repeats its
// one scale in every slot, so the attention kernel reads both the same way.
constexpr int kQueryScaleSlots = 8;
constexpr int kKeyScaleSlots = 4;

struct QuantParams {
  InputTensor query;
  InputTensor key;
  InputTensor value;
  int batch_heads;
  int heads;
  int query_length;
  int key_length;
  int sq32;
  int sk64;
  int nqb;
  int nkb;
  int q_blocks_wg;  // workgroups (4 units each) per unit kind
  int k_blocks_wg;
  int v_blocks_wg;
  int center_value;
  int per_thread;  // 1: Q/K scales per thread group (per_thread); 0: one per block (per_warp)
  const float* key_mean;
  const float* value_mean;
  int8_t* query_code;
  float* query_scale;
  float* key_scale;
  float* value_scale;
  uint8_t* kv_tiles;  // [batch_heads][nkb][kv_tile_bytes(D)] (layout in piper_mi355x.h)
};

struct AttnParams {
  const int8_t* query_code;
  const float* query_scale;
  const float* key_scale;
  const uint8_t* kv_tiles;
  const float* value_mean;
  void* output;
  int batch_heads;
  int query_length;
  int key_length;
  int sq32;
  int sk64;
  int nqb;
  int nkb;
  int query_tiles;  // workgroup query tiles per (batch, head)
  float scale_log2e;
  int causal_forward;  // causal grids: 1 = query tiles in forward order, 0 = longest first
  int xcd_remap;       // 1 = consecutive workgroups of a head share an XCD, 0 = hardware order
  int causal_interleave;  // causal, longest first: 1 = across the heads of an XCD, 0 = head by head
  // Fused query quantisation: each wave quantises its own 32-row query block from `query`
  // (query_code and query_scale are then unused).
  int fused_query;
  // Q/K scale granularity: 1 = per thread group (query scale slot n % 8 of the row's block, the
  // tile's four K group scales), 0 = per block (slot 0, one K scale)
  int per_thread;
  int query_bf16;
  int heads;
  InputTensor query;
  // Key-range split (non-causal, three workgroups per CU): each query tile's key tiles are cut
  // into key_parts ranges of part_tiles tiles, one workgroup per range, which writes its
  // unnormalised numerator (x 255), denominator and reference maximum to `partials`
  // ([key_parts][batch_heads][query_length][D] floats, then [key_parts][batch_heads][query_length]
  // float2 (den, mref)); attention_merge_kernel combines them.  key_parts = 1: no split.
  int key_parts;
  int part_tiles;
  float* partials;
  // Work-queue plan (three workgroups per CU, no key-range split): a persistent grid takes query
  // tiles from queue_xccs queues of consecutive logical ids, counters in `queue` (zero before the
  // launch).  queue_xccs = 0: the hardware dispatches one workgroup per query tile.
  int queue_xccs;
  int queue_workers;  // the persistent grid (at most three workgroups per CU)
  float score_multiplier;  // scale_log2e * 2^26 (kScoreUnit), exact: the logits' multiplier per query scale
  uint32_t* queue;
};

// The workspace bytes of a key-range split (0 without one).
inline long attention_partial_bytes(long batch_heads, long query_length, int head_dim, int key_parts) {
  return key_parts > 1 ? static_cast<long>(key_parts) * batch_heads * query_length * (head_dim + 2) * 4 : 0;
}

// The work-queue plan's counters: one per XCC, at most kQueueCounters.
constexpr int kQueueCounters = 64;
constexpr long kQueueBytes = kQueueCounters * 4;

// SageAttention2++: the prep quantises K (per 64-row block, after K smoothing) and V (FP8
// per channel) into tile records; the attention kernel quantises each query block itself.
struct SageQuantParams {
  InputTensor key;
  InputTensor value;
  int batch_heads;
  int heads;
  int key_length;
  int nkb;
  int k_blocks_wg;  // workgroups (4 units each) per unit kind
  int v_blocks_wg;
  const float* key_mean;
  const float* value_scale;
  float* key_scale;   // [batch_heads][nkb][kKeyScaleSlots]
  uint8_t* kv_tiles;  // [batch_heads][nkb][sage_tile_bytes(D)]
  int per_thread;     // 1: K scales per thread group; 0: one per block, repeated in every slot
};

struct SageParams {
  const uint8_t* kv_tiles;
  const float* value_scale;  // [batch_heads][D]
  void* output;
  InputTensor query;
  int query_bf16;
  int heads;
  int batch_heads;
  int query_length;
  int key_length;
  int nkb;
  int query_tiles;  // workgroup query tiles per (batch, head)
  float scale_log2e;
  int causal_forward;
  int xcd_remap;
  int causal_interleave;
  int per_thread;  // Q/K scales per thread group (the tile's four K slots, per-row-group Q scales)
  int fp16_partials;  // round each block's FP8 product to FP16 (the reference's arithmetic)
};

constexpr int kPrepSpinLimit = 1 << 20;  // polls of a waiting single-pass chunk (with s_sleep): about a second

// The GPU the prep runs on, and the single-pass prep's wait bound.
struct PrepDevice {
  int cus;         // compute units
  int xccs;        // XCCs (accelerator complex dies) the workgroups are dealt over, round-robin
  int spin_limit;  // polls of a waiting chunk before it computes the mean itself (0: at once)
};

// The single-pass prep keeps each chunk of a batch-head tensor resident until the tensor's last
// chunk has arrived, so all of a tensor's chunks must fit in one XCC at once: at least four
// workgroups per CU (the kernel's occupancy allows more) on cus / xccs CUs.
__host__ __device__ inline bool single_pass_resident(int chunks, int cus, int xccs) {
  return xccs > 0 && cus >= xccs && chunks <= 4 * (cus / xccs);
}

hipError_t launch_prep(bool bf16, int head_dim, const MeanParams& mp, const QuantParams& qp, const PrepDevice& dev,
                       hipStream_t stream);
hipError_t launch_sage_prep(bool bf16, int head_dim, const MeanParams& mp, const SageQuantParams& qp,
                            hipStream_t stream);
hipError_t launch_sage_attention(int head_dim, bool causal, int out_dtype, int waves, const SageParams& sp,
                                 hipStream_t stream);

// out_dtype: 0 = fp16, 1 = bf16, 2 = fp32.  waves: 8 or 4 query waves per workgroup (two waves per
// SIMD), or 3 for three 4-wave workgroups per CU.
hipError_t launch_attention(int head_dim, bool causal, int out_dtype, int waves, const AttnParams& ap,
                            hipStream_t stream);

}  // namespace piper
