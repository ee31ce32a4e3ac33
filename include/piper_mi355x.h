/*
 * piper_mi355x.h -- C ABI of the MI355X (gfx950) Piper Attention forward backend.
 *
 * The library exports plain extern "C" functions over POD structs: raw device pointers,
 * element strides and sizes, a HIP stream handle passed as void*, and an int status.
 * It never allocates or frees device memory and never synchronises the stream: the caller
 * (the Python host layer on PyTorch-ROCm) owns every buffer for the stream-ordered
 * lifetime of the launches.
 *
 * Reference interfaces these entry points replace (jumbledpoophj/piper-kernels 0.2.1):
 *   piper_prepare            <- _prepare_piper_attention
 *                               src/piper_kernels/attention/piper_attention/triton.py:772-890
 *                               (K/V means triton.py:638-699, Q/K quantisation
 *                               attention/kernels/qk_quantization/int8/sage/triton.py:238-356,
 *                               per-key V quantisation triton.py:176-246 / :839-860)
 *   piper_prepare_static     <- no reference counterpart: piper_prepare with its workspace in a
 *                               static per-GPU scratch, for callers that cannot allocate
 *   piper_attention_forward  <- _launch_piper_attention
 *                               src/piper_kernels/attention/piper_attention/triton.py:893-951
 *                               (fused kernel _piper_attention_kernel triton.py:303-635)
 *   piper_attention_forward_fused
 *                            <- piper_prepare (Q pass) + piper_attention_forward in one launch;
 *                               no Piper counterpart.  Precedent: the fused query quantisation
 *                               flag of SageAttention2++
 *                               src/piper_kernels/attention/sage_attention_2pp/_policy.py:24,118
 *   piper_sage_prepare       <- the K/V part of _prepare_sage_attention_2pp
 *                               src/piper_kernels/attention/sage_attention_2pp/triton.py:1000-1063
 *                               (statistics :60-151, FP8 V :154-195, K codes through
 *                               qk_quantization.prepare_key, as reference.py:44-49)
 *   piper_sage_attention_forward <- _launch_sage_attention_2pp (triton.py:1066-1102) with the
 *                               fused query quantisation of _prepare_query (:983-997);
 *                               kernel _sage_attention_2pp_kernel (:513-788)
 *   piper_sage_prepared_layout <- the buffer allocations of _prepare_sage_attention_2pp
 *   piper_prepared_layout    <- the buffer allocations of _prepare_piper_attention
 *                               (triton.py:797-874); the sizes the caller must provide
 *   piper_prepare_status     <- no reference counterpart: how many chunks of the last prep gave
 *                               up waiting for their tensor's mean and computed it themselves
 *   piper_attention_workspace_bytes
 *                            <- no reference counterpart: the partial-sum workspace of the
 *                               key-range split plans (small grids)
 *   piper_abi_version,
 *   piper_last_error         <- no reference counterpart: version handshake and the error
 *                               text the Python layer raises as RuntimeError
 *
 * Status codes: 0 on success; otherwise one of piper_status and piper_last_error()
 * returns a thread-local, NUL-terminated description.
 */
#ifndef PIPER_MI355X_H
#define PIPER_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PIPER_ABI_VERSION 5

/* Rows per quantisation group (sage/reference.py:6-7) and keys per P block (reference.py:16). */
#define PIPER_QUERY_BLOCK 32
#define PIPER_KEY_BLOCK 64
/* Scales stored per quantisation block: one per thread group of the reference's "per_thread"
 * Q/K granularity (sage/reference.py:23-58) -- query rows {t, t+8, t+16, t+24} of a 32-row
 * block share slot t, key rows {8a + 2t + c} of a 64-row block share slot t.  With the default
 * per-block ("per_warp") granularity every slot holds the block's one scale. */
#define PIPER_QUERY_SCALE_SLOTS 8
#define PIPER_KEY_SCALE_SLOTS 4

typedef enum piper_dtype {
  PIPER_FLOAT16 = 0,
  PIPER_BFLOAT16 = 1,
  PIPER_FLOAT32 = 2 /* attention output only: the FP32 result before the cast */
} piper_dtype;

typedef enum piper_status {
  PIPER_OK = 0,
  PIPER_ERROR_INVALID_ARGUMENT = 1,
  PIPER_ERROR_UNSUPPORTED = 2,
  PIPER_ERROR_HIP = 3
} piper_status;

typedef struct piper_shape {
  int64_t batch;
  int64_t heads;
  int64_t query_length;
  int64_t key_length;
  int64_t head_dim; /* 64 or 128 */
} piper_shape;

/* A [batch, heads, sequence, head_dim] input: element strides of the first three axes;
 * the head_dim axis must be contiguous (stride 1), as _validation.py:34-35 requires. */
typedef struct piper_tensor {
  const void* data;
  int64_t stride_batch;
  int64_t stride_head;
  int64_t stride_seq;
} piper_tensor;

/*
 * The prepared (quantised) operands, produced by piper_prepare and consumed by
 * piper_attention_forward.  With Sq32 = ceil(Sq/32)*32, Sk64 = ceil(Sk/64)*64,
 * nqb = Sq32/32 and nkb = Sk64/64, all arrays are dense and row-major:
 *
 *   query_code     int8    [B, H, Sq32, D]   Q codes, padded rows zero
 *   query_scale    float   [B, H, nqb, 8]    amax/127 + 1e-7 per 32-row block, or per thread
 *                                            group of it (PIPER_QUERY_SCALE_SLOTS)
 *   key_scale      float   [B, H, nkb, 4]    same for K - mean(K), per 64-row block or thread
 *                                            group (PIPER_KEY_SCALE_SLOTS)
 *   value_scale    float   [B, H, Sk64]      amax_D/127 + 1e-7 per V row (padding 0)
 *   key_mean       float   [B, H, D]         sequence mean of K: FP32, torch's CPU summation order
 *   value_mean     float   [B, H, D]         same for V; zeros when causal
 *   kv_tiles       bytes   [B, H, nkb, PIPER_KV_TILE_BYTES(D)]: one self-contained record
 *                  per 64-key tile, byte for byte the LDS stage of the attention kernel (it is
 *                  copied with direct global -> LDS loads in 1 KiB pieces):
 *       [0, 64*(D+16))           int8  K codes of K - mean(K), [64 keys][D], rows of D + 16
 *                                      bytes (padding rows of short tiles are zero codes);
 *                                      bytes [D, D+16) of row 0 hold the tile's 4 K scale
 *                                      slots (FP32, as key_scale)
 *       [PIPER_KV_V_OFFSET(D), +80*D)
 *                                int8  V codes of V - mean(V), transposed: [D][64 keys], rows
 *                                      of 80 bytes
 *       [PIPER_KV_LOG2_OFFSET(D), +256)  float log2(value_scale) of the 64 keys (padding -inf)
 *       [.. + 256, +256)         float 1 / (255 * value_scale) (padding 0)
 *       [.. + 512, +4*D)         int32 0x4B400000 + 128 * (sum over the 64 keys of the V
 *                                      codes), per feature: the affine correction of the PV
 *                                      product plus the bias that makes the integer result
 *                                      readable as FP32 1.5 * 2^23 + PV
 *                  Any other byte (row padding, the tail up to the KiB multiple) is
 *                  unspecified.
 */
#define PIPER_KV_V_OFFSET(head_dim) (64 * ((head_dim) + 16))
#define PIPER_KV_LOG2_OFFSET(head_dim) (PIPER_KV_V_OFFSET(head_dim) + 80 * (head_dim))
#define PIPER_KV_TILE_BYTES(head_dim) \
  ((PIPER_KV_LOG2_OFFSET(head_dim) + 512 + 4 * (head_dim) + 1023) / 1024 * 1024)

typedef struct piper_prepared {
  int8_t* query_code;
  float* query_scale;
  float* key_scale;
  float* value_scale;
  float* key_mean;
  float* value_mean;
  void* kv_tiles;
} piper_prepared;

/* Byte sizes of every caller-allocated buffer for a shape. */
typedef struct piper_layout {
  int64_t query_code_bytes;
  int64_t query_scale_bytes;
  int64_t key_scale_bytes;
  int64_t value_scale_bytes;
  int64_t mean_bytes; /* each of key_mean, value_mean */
  int64_t kv_tile_bytes; /* one tile record */
  int64_t kv_tiles_bytes; /* all tile records */
  int64_t workspace_bytes; /* scratch for piper_prepare, 16-byte aligned: FP32 partial sums of
                              the K/V means (torch's CPU summation order, so the means and every
                              K/V code equal the reference's torch.mean(dim=2) path bit for
                              bit), 2 * B * H * (ceil(Sk / L^2) + 1) * D * 4 bytes (L = 16 up to
                              Sk = 2^19), then 4 * (4 * B * H + 4) bytes of sync words: arrival
                              counters and the status word; the library clears what it needs on
                              the stream */
  int64_t workspace_status_offset; /* byte offset of the status word in the workspace (a
                              uint32: see piper_prepare_status) */
} piper_layout;

/* piper_prepare_args.flags */
#define PIPER_PREPARE_SKIP_QUERY 1 /* leave query_code / query_scale alone (they may be NULL):
                                      for piper_attention_forward_fused, which quantises Q itself */
#define PIPER_PREPARE_QK_PER_THREAD 2 /* Q and K scales per thread group (the reference's
                                         "per_thread"); default: one per block ("per_warp") */
#define PIPER_PREPARE_SELF_MEAN 4 /* diagnostic, for tests: every single-pass chunk that would wait
                                     for its tensor's mean computes it itself at once (the bounded
                                     wait's fallback; same bits, slower) */

typedef struct piper_prepare_args {
  int32_t abi_version; /* PIPER_ABI_VERSION */
  int32_t dtype;       /* PIPER_FLOAT16 or PIPER_BFLOAT16: dtype of query, key and value */
  int32_t is_causal;   /* causal calls leave V uncentred (value_mean = 0) */
  int32_t flags;       /* OR of PIPER_PREPARE_* (0: quantise Q, K and V) */
  piper_shape shape;
  piper_tensor query;
  piper_tensor key;
  piper_tensor value;
  piper_prepared prepared; /* outputs */
  void* workspace;
  int64_t workspace_bytes;
} piper_prepare_args;

/* Launch-plan bits of piper_attention_args.plan (results are identical for every plan; only
 * the speed differs).  Default (0): 8 query waves of 32 queries per workgroup, causal query
 * tiles dispatched longest first, workgroups of one head kept on one XCD. */
#define PIPER_PLAN_FOUR_WAVES 1     /* 4 query waves per workgroup, two workgroups per CU (4-stage LDS
                                       rings); the default is 8 waves, one workgroup per CU */
#define PIPER_PLAN_CAUSAL_FORWARD 2 /* causal: query tiles in forward order */
#define PIPER_PLAN_NO_XCD_REMAP 4   /* hardware workgroup order */
#define PIPER_PLAN_CAUSAL_INTERLEAVE 8 /* causal, longest first: query tiles dispatched longest first
                                          across the heads of each XCD (across all heads with
                                          PIPER_PLAN_NO_XCD_REMAP) instead of head by head */
#define PIPER_PLAN_THREE_WORKGROUPS 16 /* three 4-wave workgroups per CU (three waves per SIMD, 2-stage LDS
                                          rings); overrides PIPER_PLAN_FOUR_WAVES.  Both operators */
/* Key-range split (Piper Attention, non-causal, with PIPER_PLAN_THREE_WORKGROUPS): the key tiles
 * of each query tile are cut into `parts` ranges (2..8), one workgroup each, which write their
 * FP32 partial numerator, denominator and reference maximum to the call's workspace; a merge
 * kernel combines them (piper_attention_workspace_bytes gives the size).  For grids too small to
 * give every SIMD three waves.  The merge adds the parts in another order than one sequential
 * pass, so split plans agree with the others to rounding, not bit for bit. */
#define PIPER_PLAN_KEY_PARTS(parts) (((parts) - 1) << 5)
#define PIPER_PLAN_KEY_PARTS_OF(plan) ((((plan) >> 5) & 7) + 1)
/* Work queues (Piper Attention, with PIPER_PLAN_THREE_WORKGROUPS, no key-range split): a
 * persistent grid of at most three workgroups per CU takes the query tiles, in the order the
 * other bits give, from one queue per XCC (relaxed atomic counters in the call's workspace,
 * piper_attention_workspace_bytes) instead of one workgroup per tile dispatched by the hardware,
 * whose in-order round-robin over the XCCs leaves slots idle when tiles differ in length (causal).
 * Bit-identical to the other plans. */
#define PIPER_PLAN_WORK_QUEUE 256
#define PIPER_PLAN_MASK 511

/* piper_attention_args.flags / piper_attention_fused_args.flags */
#define PIPER_ATTENTION_QK_PER_THREAD 1 /* Q/K scales per thread group: read slot (row % 8) of the
                                           query scales and the tile's four K group scales; the
                                           fused entry point quantises Q per thread group too */

typedef struct piper_attention_args {
  int32_t abi_version;  /* PIPER_ABI_VERSION */
  int32_t output_dtype; /* PIPER_FLOAT16, PIPER_BFLOAT16 or PIPER_FLOAT32 */
  int32_t is_causal;
  int32_t plan;         /* launch plan: OR of PIPER_PLAN_* bits; 0 = the default plan */
  piper_shape shape;
  float scale;          /* softmax scale, finite and > 0 */
  int32_t flags;        /* PIPER_ATTENTION_QK_PER_THREAD if the prep ran with PIPER_PREPARE_QK_PER_THREAD */
  piper_prepared prepared; /* inputs, as written by piper_prepare */
  void* output;            /* [B, H, Sq, D] dense row-major, output_dtype */
  void* workspace;         /* key-range split plans: piper_attention_workspace_bytes bytes, 16-byte
                              aligned; otherwise unused (NULL) */
  int64_t workspace_bytes;
} piper_attention_args;

/* The fused entry point: like piper_attention_forward, but each query wave quantises its own
 * 32-row query block from `query` in the kernel (the same arithmetic as piper_prepare, so the
 * result is bit-identical), after a piper_prepare with PIPER_PREPARE_SKIP_QUERY.  Saves the
 * query pass of the prep and the query-code round trip through HBM. */
typedef struct piper_attention_fused_args {
  int32_t abi_version;  /* PIPER_ABI_VERSION */
  int32_t dtype;        /* of query: PIPER_FLOAT16 or PIPER_BFLOAT16 */
  int32_t output_dtype; /* PIPER_FLOAT16, PIPER_BFLOAT16 or PIPER_FLOAT32 */
  int32_t is_causal;
  int32_t plan;         /* OR of PIPER_PLAN_* bits */
  float scale;          /* softmax scale, finite and > 0 */
  int32_t flags;        /* PIPER_ATTENTION_QK_PER_THREAD with a per-thread-group K prep */
  int32_t reserved;     /* 0 */
  piper_shape shape;
  piper_tensor query;      /* [B, H, Sq, D], the layout rules of piper_prepare_args.query */
  piper_prepared prepared; /* from piper_prepare; query_code and query_scale are not read */
  void* output;            /* [B, H, Sq, D] dense row-major, output_dtype */
  void* workspace;         /* as piper_attention_args.workspace */
  int64_t workspace_bytes;
} piper_attention_fused_args;

/* ---------------------------------------------------------------------------------------
 * SageAttention2++ (src/piper_kernels/attention/sage_attention_2pp/, reference.py:15-104):
 * INT8 Q/K with K smoothing (per 32 query rows / 64 key rows), per-channel FP8 E4M3 V
 * (scale = amax_S|v| / 2.25 + 1e-7), FP8 probabilities in a frame shifted by ln 448.
 * The prep quantises K and V; the attention kernel quantises each query block itself.
 *
 * Tile record (PIPER_SAGE_TILE_BYTES(D) bytes per 64 keys, the kernel's LDS stage image):
 *   [0, PIPER_SAGE_V_OFFSET(D))  int8 K codes [64][D] in rows of D + 16 bytes; bytes
 *                                [D, D + 16) of row 0 hold the tile's 4 K scale slots (float)
 *   [PIPER_SAGE_V_OFFSET(D), +80 * D)  FP8 E4M3 V^T codes [D][64] in rows of 80 bytes
 *   padding to a KiB multiple; padding bytes are unspecified.
 * ------------------------------------------------------------------------------------- */
#define PIPER_SAGE_V_OFFSET(head_dim) (64 * ((head_dim) + 16))
#define PIPER_SAGE_TILE_BYTES(head_dim) ((PIPER_SAGE_V_OFFSET(head_dim) + 80 * (head_dim) + 1023) / 1024 * 1024)

typedef struct piper_sage_prepared {
  float* key_scale;   /* [B, H, Sk64/64, 4] INT8 K scales (PIPER_KEY_SCALE_SLOTS, as piper_prepared) */
  float* key_mean;    /* [B, H, D] the K smoothing mean (torch's CPU order, as piper_prepared) */
  float* value_scale; /* [B, H, D] FP8 V scales, per channel */
  void* kv_tiles;     /* [B, H, Sk64/64] tile records, 16-byte aligned */
} piper_sage_prepared;

typedef struct piper_sage_layout {
  int64_t key_scale_bytes;
  int64_t mean_bytes;        /* key_mean and value_scale, each */
  int64_t kv_tile_bytes;     /* one tile record */
  int64_t kv_tiles_bytes;    /* all tile records */
  int64_t workspace_bytes;   /* scratch for piper_sage_prepare */
} piper_sage_layout;

typedef struct piper_sage_prepare_args {
  int32_t abi_version; /* PIPER_ABI_VERSION */
  int32_t dtype;       /* PIPER_FLOAT16 or PIPER_BFLOAT16: dtype of key and value */
  int32_t flags;       /* 0 or PIPER_PREPARE_QK_PER_THREAD (K scales per thread group) */
  int32_t reserved;    /* 0 */
  piper_shape shape;   /* query_length is not used by the prep */
  piper_tensor key;
  piper_tensor value;
  piper_sage_prepared prepared; /* outputs */
  void* workspace;
  int64_t workspace_bytes;
} piper_sage_prepare_args;

/* piper_sage_attention_args.flags: round each 64-key block's FP8 product to FP16 before it joins
 * the FP32 accumulator -- the reference's arithmetic (sage_attention_2pp/reference.py:95-98, its
 * model of an FP16-accumulating FP8 MMA); without it the products of every block accumulate in
 * the MFMA's FP32 registers (faster and closer to exact). */
#define PIPER_SAGE_FP16_PARTIALS 2

typedef struct piper_sage_attention_args {
  int32_t abi_version;  /* PIPER_ABI_VERSION */
  int32_t dtype;        /* of query: PIPER_FLOAT16 or PIPER_BFLOAT16 */
  int32_t output_dtype; /* PIPER_FLOAT16, PIPER_BFLOAT16 or PIPER_FLOAT32 */
  int32_t is_causal;
  int32_t plan;         /* OR of PIPER_PLAN_* bits (the same launch plans) */
  float scale;          /* softmax scale, finite and > 0 */
  int32_t flags;        /* PIPER_ATTENTION_QK_PER_THREAD after a per-thread-group K prep: the
                           query is quantised per thread group as well; PIPER_SAGE_FP16_PARTIALS */
  int32_t reserved;     /* 0 */
  piper_shape shape;
  piper_tensor query;   /* [B, H, Sq, D], the layout rules of piper_prepare_args.query */
  piper_sage_prepared prepared; /* from piper_sage_prepare */
  void* output;         /* [B, H, Sq, D] dense row-major, output_dtype */
} piper_sage_attention_args;

int piper_abi_version(void);

/* Fill *layout with the buffer sizes piper_prepare / piper_attention_forward expect. */
int piper_prepared_layout(const piper_shape* shape, piper_layout* layout);

/* Quantise Q, K, V into args->prepared on `stream` (a hipStream_t; NULL = default stream);
 * with PIPER_PREPARE_SKIP_QUERY only K and V.  key_mean must be 4-byte aligned, the workspace
 * and the other prepared buffers 16-byte aligned.
 *
 * Launches, at D = 128 with Sk <= 32768 when one XCC of the device holds a tensor's 256-row
 * chunks at once (4 * CUs / XCCs >= ceil(Sk / 256); every MI355X partition mode): a fill kernel
 * (sync words cleared, means marked pending) and the single pass, which reads K and V once: each
 * chunk publishes its partial sums, the last chunk of a batch-head tensor finalises the mean,
 * the others wait for it (bounded: a chunk whose wait ends computes the mean itself from K/V in
 * HBM, same bits, and is counted in the status word), then every chunk quantises its rows.
 * Otherwise: FP32 mean partials (torch's CPU order), mean finalisation, one quantisation kernel.
 * Work on other streams or in other processes that holds the GPU's workgroup slots can delay a
 * tensor's last chunk: the results stay exact, the prep gets slower (piper_prepare_status). */
int piper_prepare(const piper_prepare_args* args, void* stream);

/* The status word of the last prep that used `workspace` (NULL: the static scratch of
 * piper_prepare_static on the current device) for `shape`: the number of single-pass chunks
 * whose bounded wait for their tensor's mean ended, so that they computed it themselves (0 for
 * the three-kernel path).  Diagnostic: copies the word to *count and synchronises `stream`. */
int piper_prepare_status(const piper_shape* shape, const void* workspace, uint32_t* count, void* stream);

/* piper_prepare without a caller workspace.  No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  args->workspace must be NULL and args->workspace_bytes 0; the
 * workspace (FP32 mean partials, then the sync words) goes to a static scratch array inside the
 * library instead, of PIPER_STATIC_SCRATCH_BYTES bytes per GPU (each GPU the library runs on
 * holds its own copy until the process ends).  Shapes whose piper_layout.workspace_bytes exceeds
 * it are rejected with PIPER_ERROR_UNSUPPORTED before anything is launched (2 * B * H *
 * (ceil(Sk / 256) + 1) * D * 4 + 4 * (4 * B * H + 4) bytes up to Sk = 2^19: 10.1 MiB for 80
 * batch-heads at Sk = 32768, D = 128).  Call it with the stream's device current.  It calls no
 * allocator.  Every call on one GPU shares that GPU's scratch, which each call clears and fills
 * on its stream: calls on one stream are ordered; calls that overlap on one GPU (other streams
 * or threads) race on the partials and on the single pass's arrival counters, and their means
 * and codes are then undefined.  Outputs are identical to piper_prepare's. */
#define PIPER_STATIC_SCRATCH_BYTES (16ll << 20)
int piper_prepare_static(const piper_prepare_args* args, void* stream);

/* Fused INT8-QK / UINT8-P x INT8-V online-softmax attention on `stream`. */
int piper_attention_forward(const piper_attention_args* args, void* stream);

/* Workspace bytes the attention entry points need for `plan`: parts * B * H * Sq * (D + 2) * 4 for
 * a key-range split, 256 for the work-queue plan (its counters; the library zeroes them on the
 * stream before each call), 0 otherwise. */
int piper_attention_workspace_bytes(const piper_shape* shape, int32_t plan, int64_t* bytes);

/* The same with the query quantised inside the kernel (see piper_attention_fused_args). */
int piper_attention_forward_fused(const piper_attention_fused_args* args, void* stream);

/* SageAttention2++: buffer sizes, K/V prep (statistics, INT8 K, FP8 V^T tile records) and the
 * fused attention kernel (INT8 QK, FP8 PV on v_mfma_f32_32x32x64_f8f6f4, FP32 accumulation). */
int piper_sage_prepared_layout(const piper_shape* shape, piper_sage_layout* layout);
int piper_sage_prepare(const piper_sage_prepare_args* args, void* stream);
int piper_sage_attention_forward(const piper_sage_attention_args* args, void* stream);

/* Thread-local description of the last failure on this thread ("" if none). */
const char* piper_last_error(void);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* PIPER_MI355X_H */
