// Kernel parameter blocks and launchers shared by the C ABI and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace piper {

struct InputTensor {
  const void* data;  // 16-bit floats; the head_dim axis is contiguous
  long stride_batch;  // element strides
  long stride_head;
  long stride_seq;
};

struct MeanParams {
  InputTensor key;
  InputTensor value;
  double* partials;  // [tensors][batch_heads][chunks][D]
  float* key_mean;   // [batch_heads][D]
  float* value_mean; // [batch_heads][D]
  int batch_heads;
  int heads;
  int length;  // key length
  int chunks;  // ceil(length / 64)
  int tensors; // 1 = K only (causal), 2 = K and V
};

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
  const float* key_mean;
  const float* value_mean;
  int8_t* query_code;
  float* query_scale;
  int8_t* key_code;
  float* key_scale;
  int8_t* value_code;
  float* value_scale;
  float* value_log2_scale;
  float* value_inv_multiplier;
  int32_t* value_correction;
};

struct AttnParams {
  const int8_t* query_code;
  const float* query_scale;
  const int8_t* key_code;
  const float* key_scale;
  const int8_t* value_code;
  const float* value_log2_scale;
  const float* value_inv_multiplier;
  const int32_t* value_correction;
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
};

hipError_t launch_prep(bool bf16, int head_dim, const MeanParams& mp, const QuantParams& qp, hipStream_t stream);

// out_dtype: 0 = fp16, 1 = bf16, 2 = fp32.  waves: 4 or 8 query waves per workgroup.
hipError_t launch_attention(int head_dim, bool causal, int out_dtype, int waves, const AttnParams& ap,
                            hipStream_t stream);

}  // namespace piper
