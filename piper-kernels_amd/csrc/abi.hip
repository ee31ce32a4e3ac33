// extern "C" entry points of libpiper_mi355x.so (declared in include/piper_mi355x.h).
//
// Validation, launch geometry and error reporting only: the library never allocates,
// frees or synchronises; every buffer belongs to the caller.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "kernels.h"
#include "piper_mi355x.h"

// The tile record documented in the header is the layout the kernels use.
static_assert(PIPER_KV_TILE_BYTES(64) == piper::kv_tile_bytes(64), "tile record size (D = 64)");
static_assert(PIPER_KV_TILE_BYTES(128) == piper::kv_tile_bytes(128), "tile record size (D = 128)");
static_assert(PIPER_KV_V_OFFSET(128) == piper::kv_v_offset(128), "V^T offset");
static_assert(PIPER_KV_LOG2_OFFSET(128) == piper::kv_log_offset(128), "log2 offset");
static_assert(PIPER_KV_LOG2_OFFSET(64) == piper::kv_log_offset(64), "log2 offset");
static_assert(PIPER_SAGE_TILE_BYTES(64) == piper::sage_tile_bytes(64), "SageAttention2++ record size (D = 64)");
static_assert(PIPER_SAGE_TILE_BYTES(128) == piper::sage_tile_bytes(128), "SageAttention2++ record size (D = 128)");
static_assert(PIPER_SAGE_V_OFFSET(128) == piper::sage_v_offset(128), "SageAttention2++ V^T offset");
static_assert(PIPER_QUERY_SCALE_SLOTS == piper::kQueryScaleSlots && PIPER_KEY_SCALE_SLOTS == piper::kKeyScaleSlots,
              "scale slots per block");

// Static scratch of piper_prepare_static (see device_scratch below).
static __device__ __align__(256) unsigned char scratch[PIPER_STATIC_SCRATCH_BYTES];

namespace {

thread_local char g_last_error[512] = "";

int fail(int status, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
  return status;
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

int check_shape(const piper_shape* s) {
  if (s == nullptr) return fail(PIPER_ERROR_INVALID_ARGUMENT, "shape is NULL");
  if (s->batch <= 0 || s->heads <= 0 || s->query_length <= 0 || s->key_length <= 0)
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "dimensions must be positive, got B=%lld H=%lld Sq=%lld Sk=%lld",
                (long long)s->batch, (long long)s->heads, (long long)s->query_length, (long long)s->key_length);
  if (s->head_dim != 64 && s->head_dim != 128)
    return fail(PIPER_ERROR_UNSUPPORTED, "head_dim must be 64 or 128, got %lld", (long long)s->head_dim);
  // 32-bit index arithmetic inside the kernels: keep every per-call count well inside int.
  const int64_t bh = s->batch * s->heads;
  const int64_t longest = s->query_length > s->key_length ? s->query_length : s->key_length;
  if (bh > (1 << 24) || longest > (1 << 26) || bh * ceil_div(longest, 32) > (int64_t(1) << 30))
    return fail(PIPER_ERROR_UNSUPPORTED, "shape too large for this build");
  return PIPER_OK;
}

int check_input(const char* name, const piper_tensor& t) {
  if (t.data == nullptr) return fail(PIPER_ERROR_INVALID_ARGUMENT, "%s pointer is NULL", name);
  if (!aligned16(t.data) || (t.stride_batch % 8) != 0 || (t.stride_head % 8) != 0 || (t.stride_seq % 8) != 0)
    return fail(PIPER_ERROR_INVALID_ARGUMENT,
                "%s must be 16-byte aligned with batch/head/sequence strides that are multiples of 8 elements",
                name);
  return PIPER_OK;
}

// Static scratch of piper_prepare_static: the prep's workspace (FP32 mean partials, then the
// single pass's sync words) for callers that cannot allocate.  Each GPU the library runs on holds
// its own copy until the process ends.  In host code `scratch` only names the symbol: its device
// address on the current GPU comes from hipGetSymbolAddress, looked up once per device
// (device_scratch) and used for every launch.  Each call clears the sync words it uses with its
// own fill kernel and writes every partial it reads; calls that overlap on one GPU share the
// array and race (on the arrival counters too, which then give wrong means).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_address[kMaxDevices] = {};

int device_scratch(void** address) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return fail(PIPER_ERROR_HIP, "hipGetDevice failed: %s", hipGetErrorString(err));
  if (device < 0 || device >= kMaxDevices)
    return fail(PIPER_ERROR_UNSUPPORTED, "device %d is beyond the %d this build tracks", device, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_address[device] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr)
      return fail(PIPER_ERROR_HIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", device,
                  hipGetErrorString(err));
    g_scratch_address[device] = ptr;
  }
  *address = g_scratch_address[device];
  return PIPER_OK;
}

// Compute units and XCCs of the current device, looked up once per device: the single-pass
// prep deals its workgroups over the XCCs and needs a tensor's chunks resident in one XCC.
std::mutex g_topology_mutex;
int g_topology[kMaxDevices][2] = {};

int device_topology(int* cus, int* xccs) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return fail(PIPER_ERROR_HIP, "hipGetDevice failed: %s", hipGetErrorString(err));
  if (device < 0 || device >= kMaxDevices)
    return fail(PIPER_ERROR_UNSUPPORTED, "device %d is beyond the %d this build tracks", device, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_topology_mutex);
  if (g_topology[device][0] == 0) {
    int c = 0, x = 0;
    err = hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, device);
    if (err != hipSuccess) return fail(PIPER_ERROR_HIP, "compute-unit count query failed: %s", hipGetErrorString(err));
    // no XCC count (an older runtime): 0, which keeps the prep on its three-kernel path
    if (hipDeviceGetAttribute(&x, hipDeviceAttributeNumberOfXccs, device) != hipSuccess || x < 0) x = 0;
    (void)hipGetLastError();
    g_topology[device][0] = c;
    g_topology[device][1] = x;
  }
  *cus = g_topology[device][0];
  *xccs = g_topology[device][1];
  return PIPER_OK;
}

piper::InputTensor to_input(const piper_tensor& t) {
  return piper::InputTensor{t.data, static_cast<long>(t.stride_batch), static_cast<long>(t.stride_head),
                            static_cast<long>(t.stride_seq)};
}

// Validation and launch shared by piper_attention_forward (prepared query codes) and
// piper_attention_forward_fused (query != NULL: the kernel quantises the query itself).
int launch_attention_call(int32_t abi_version, int32_t output_dtype, int32_t is_causal, int32_t plan, int32_t flags,
                          const piper_shape& s, float scale, const piper_prepared& o, void* output,
                          const piper_tensor* query, int32_t query_dtype, void* workspace, int64_t workspace_bytes,
                          void* stream) {
  if (abi_version != PIPER_ABI_VERSION)
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "ABI version mismatch: caller %d, library %d", abi_version,
                PIPER_ABI_VERSION);
  if (output_dtype != PIPER_FLOAT16 && output_dtype != PIPER_BFLOAT16 && output_dtype != PIPER_FLOAT32)
    return fail(PIPER_ERROR_UNSUPPORTED, "output dtype must be float16, bfloat16 or float32");
  if (int st = check_shape(&s)) return st;
  if (is_causal && s.query_length != s.key_length)
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "causal attention requires equal query and key lengths");
  if (!(std::isfinite(scale) && scale > 0.0f))
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "scale must be finite and positive");
  if (plan < 0 || plan > PIPER_PLAN_MASK) return fail(PIPER_ERROR_UNSUPPORTED, "unknown plan %d", plan);
  if ((flags & ~PIPER_ATTENTION_QK_PER_THREAD) != 0) return fail(PIPER_ERROR_UNSUPPORTED, "unknown flags %d", flags);
  const int key_parts = PIPER_PLAN_KEY_PARTS_OF(plan);
  const bool work_queue = (plan & PIPER_PLAN_WORK_QUEUE) != 0;
  if (key_parts > 1) {
    if (is_causal) return fail(PIPER_ERROR_UNSUPPORTED, "the key-range split plans are non-causal");
    if (!(plan & PIPER_PLAN_THREE_WORKGROUPS))
      return fail(PIPER_ERROR_UNSUPPORTED, "the key-range split needs PIPER_PLAN_THREE_WORKGROUPS");
    if (work_queue) return fail(PIPER_ERROR_UNSUPPORTED, "the work-queue plan has no key-range split");
  }
  if (work_queue && !(plan & PIPER_PLAN_THREE_WORKGROUPS))
    return fail(PIPER_ERROR_UNSUPPORTED, "the work-queue plan needs PIPER_PLAN_THREE_WORKGROUPS");
  if (key_parts > 1 || work_queue) {
    int64_t need = 0;
    if (int st = piper_attention_workspace_bytes(&s, plan, &need)) return st;
    if (workspace == nullptr || workspace_bytes < need)
      return fail(PIPER_ERROR_INVALID_ARGUMENT, "the %s needs a workspace of %lld bytes, got %lld",
                  work_queue ? "work-queue plan" : "key-range split", (long long)need, (long long)workspace_bytes);
    if (!aligned16(workspace)) return fail(PIPER_ERROR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  }
  if (query != nullptr) {
    if (query_dtype != PIPER_FLOAT16 && query_dtype != PIPER_BFLOAT16)
      return fail(PIPER_ERROR_UNSUPPORTED, "query dtype must be float16 or bfloat16");
    if (int st = check_input("query", *query)) return st;
  } else if (!o.query_code || !o.query_scale) {
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "a prepared query pointer is NULL");
  } else if (!aligned16(o.query_code)) {
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "prepared query codes must be 16-byte aligned");
  }
  if (!o.key_scale || !o.kv_tiles || !o.value_mean || !output)
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "a prepared input or the output pointer is NULL");
  if (!aligned16(o.kv_tiles) || !aligned16(o.value_mean) || (reinterpret_cast<uintptr_t>(output) & 7u) != 0)
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "prepared buffers must be 16-byte and the output 8-byte aligned");

  // 3: three 4-wave workgroups per CU (attention_w3_kernel)
  const int waves = (plan & PIPER_PLAN_THREE_WORKGROUPS) ? 3 : (plan & PIPER_PLAN_FOUR_WAVES) ? 4 : 8;
  const int block_m = 32 * (waves == 3 ? 4 : waves);
  piper::AttnParams ap{};
  ap.query_code = o.query_code;
  ap.query_scale = o.query_scale;
  ap.key_scale = o.key_scale;
  ap.kv_tiles = static_cast<const uint8_t*>(o.kv_tiles);
  ap.value_mean = o.value_mean;
  ap.output = output;
  ap.batch_heads = static_cast<int>(s.batch * s.heads);
  ap.query_length = static_cast<int>(s.query_length);
  ap.key_length = static_cast<int>(s.key_length);
  ap.sq32 = static_cast<int>(ceil_div(s.query_length, PIPER_QUERY_BLOCK) * PIPER_QUERY_BLOCK);
  ap.sk64 = static_cast<int>(ceil_div(s.key_length, PIPER_KEY_BLOCK) * PIPER_KEY_BLOCK);
  ap.nqb = ap.sq32 / PIPER_QUERY_BLOCK;
  ap.nkb = ap.sk64 / PIPER_KEY_BLOCK;
  ap.query_tiles = static_cast<int>(ceil_div(s.query_length, block_m));
  ap.scale_log2e = static_cast<float>(static_cast<double>(scale) * 1.4426950408889634);
  ap.score_multiplier = ap.scale_log2e * 67108864.0f;  // x 2^26: exact
  ap.causal_forward = (plan & PIPER_PLAN_CAUSAL_FORWARD) ? 1 : 0;
  ap.xcd_remap = (plan & PIPER_PLAN_NO_XCD_REMAP) ? 0 : 1;
  ap.causal_interleave = (plan & PIPER_PLAN_CAUSAL_INTERLEAVE) ? 1 : 0;
  ap.heads = static_cast<int>(s.heads);
  ap.per_thread = (flags & PIPER_ATTENTION_QK_PER_THREAD) ? 1 : 0;
  if (query != nullptr) {
    ap.fused_query = 1;
    ap.query_bf16 = query_dtype == PIPER_BFLOAT16 ? 1 : 0;
    ap.query = to_input(*query);
  }
  // key-range split: part_tiles tiles per part, and no empty part
  ap.key_parts = 1;
  if (key_parts > 1) {
    ap.part_tiles = static_cast<int>(ceil_div(ap.nkb, key_parts));
    ap.key_parts = static_cast<int>(ceil_div(ap.nkb, ap.part_tiles));
    ap.partials = static_cast<float*>(workspace);
  }
  if (static_cast<int64_t>(ap.query_tiles) * ap.batch_heads * ap.key_parts > 0x7fffffff)
    return fail(PIPER_ERROR_UNSUPPORTED, "too many workgroups");
  if (work_queue) {
    // one queue per XCC of the device (one queue if the runtime reports no XCC count), a
    // persistent grid of three workgroups per CU, or fewer when there are fewer tiles
    int cus = 0, xccs = 0;
    if (int st = device_topology(&cus, &xccs)) return st;
    const long tiles = static_cast<long>(ap.query_tiles) * ap.batch_heads;
    ap.queue_xccs = std::max(1, std::min(xccs, piper::kQueueCounters));
    ap.queue_workers = static_cast<int>(std::max(1L, std::min(tiles, 3L * std::max(cus, 1))));
    ap.queue = static_cast<uint32_t*>(workspace);
  }

  const hipError_t err = piper::launch_attention(static_cast<int>(s.head_dim), is_causal != 0, output_dtype, waves,
                                                 ap, static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(PIPER_ERROR_HIP, "attention launch failed: %s", hipGetErrorString(err));
  g_last_error[0] = '\0';
  return PIPER_OK;
}

}  // namespace

extern "C" {

int piper_abi_version(void) { return PIPER_ABI_VERSION; }

const char* piper_last_error(void) { return g_last_error; }

int piper_prepared_layout(const piper_shape* shape, piper_layout* layout) {
  if (int st = check_shape(shape)) return st;
  if (layout == nullptr) return fail(PIPER_ERROR_INVALID_ARGUMENT, "layout is NULL");
  const int64_t bh = shape->batch * shape->heads;
  const int64_t d = shape->head_dim;
  const int64_t sq32 = ceil_div(shape->query_length, PIPER_QUERY_BLOCK) * PIPER_QUERY_BLOCK;
  const int64_t sk64 = ceil_div(shape->key_length, PIPER_KEY_BLOCK) * PIPER_KEY_BLOCK;
  const int64_t chunks = piper::cascade_chunks(static_cast<int>(shape->key_length));
  layout->query_code_bytes = bh * sq32 * d;
  layout->query_scale_bytes = bh * (sq32 / PIPER_QUERY_BLOCK) * PIPER_QUERY_SCALE_SLOTS * 4;
  layout->key_scale_bytes = bh * (sk64 / PIPER_KEY_BLOCK) * PIPER_KEY_SCALE_SLOTS * 4;
  layout->value_scale_bytes = bh * sk64 * 4;
  layout->mean_bytes = bh * d * 4;
  layout->kv_tile_bytes = PIPER_KV_TILE_BYTES(d);
  layout->kv_tiles_bytes = bh * (sk64 / PIPER_KEY_BLOCK) * PIPER_KV_TILE_BYTES(d);
  layout->workspace_bytes = 2 * bh * (chunks + 1) * d * 4 + 4 * piper::prep_sync_words(bh);
  layout->workspace_status_offset = 2 * bh * (chunks + 1) * d * 4 + 4 * piper::prep_status_word(bh);
  g_last_error[0] = '\0';
  return PIPER_OK;
}

// Validation and launches of piper_prepare; with use_scratch, the mean partials go to this
// GPU's static scratch instead of the caller's workspace (piper_prepare_static).
static int prepare_call(const piper_prepare_args* a, bool use_scratch, void* stream) {
  if (a == nullptr) return fail(PIPER_ERROR_INVALID_ARGUMENT, "args is NULL");
  if (a->abi_version != PIPER_ABI_VERSION)
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "ABI version mismatch: caller %d, library %d", a->abi_version,
                PIPER_ABI_VERSION);
  if (a->dtype != PIPER_FLOAT16 && a->dtype != PIPER_BFLOAT16)
    return fail(PIPER_ERROR_UNSUPPORTED, "input dtype must be float16 or bfloat16");
  if (int st = check_shape(&a->shape)) return st;
  if (a->is_causal && a->shape.query_length != a->shape.key_length)
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "causal attention requires equal query and key lengths");
  if ((a->flags & ~(PIPER_PREPARE_SKIP_QUERY | PIPER_PREPARE_QK_PER_THREAD | PIPER_PREPARE_SELF_MEAN)) != 0)
    return fail(PIPER_ERROR_UNSUPPORTED, "unknown flags %d", a->flags);
  const bool with_query = (a->flags & PIPER_PREPARE_SKIP_QUERY) == 0;
  if (with_query)
    if (int st = check_input("query", a->query)) return st;
  if (int st = check_input("key", a->key)) return st;
  if (int st = check_input("value", a->value)) return st;
  const piper_prepared& o = a->prepared;
  if ((with_query && (!o.query_code || !o.query_scale)) || !o.key_scale || !o.value_scale || !o.key_mean ||
      !o.value_mean || !o.kv_tiles)
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "a prepared output pointer is NULL");
  if ((with_query && !aligned16(o.query_code)) || !aligned16(o.kv_tiles) || !aligned16(o.value_mean))
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "prepared buffers must be 16-byte aligned");
  // the prep reads and writes the means and the workspace's sync words with 32-bit atomics
  if ((reinterpret_cast<uintptr_t>(o.key_mean) & 3u) != 0)
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "key_mean must be 4-byte aligned");
  if (!use_scratch && !aligned16(a->workspace))
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  piper_layout layout;
  if (int st = piper_prepared_layout(&a->shape, &layout)) return st;
  void* workspace = a->workspace;
  if (use_scratch) {
    if (a->workspace != nullptr || a->workspace_bytes != 0)
      return fail(PIPER_ERROR_INVALID_ARGUMENT, "piper_prepare_static takes no workspace (pass NULL and 0)");
    if (layout.workspace_bytes > PIPER_STATIC_SCRATCH_BYTES)
      return fail(PIPER_ERROR_UNSUPPORTED,
                  "shape needs %lld bytes of prep scratch, more than the static %lld bytes of piper_prepare_static "
                  "(use piper_prepare with a workspace)",
                  (long long)layout.workspace_bytes, (long long)PIPER_STATIC_SCRATCH_BYTES);
    if (int st = device_scratch(&workspace)) return st;
  } else if (a->workspace == nullptr || a->workspace_bytes < layout.workspace_bytes) {
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "workspace needs %lld bytes, got %lld",
                (long long)layout.workspace_bytes, (long long)a->workspace_bytes);
  }

  const piper_shape& s = a->shape;
  const int bh = static_cast<int>(s.batch * s.heads);
  const int d = static_cast<int>(s.head_dim);
  const int sq32 = static_cast<int>(ceil_div(s.query_length, PIPER_QUERY_BLOCK) * PIPER_QUERY_BLOCK);
  const int sk64 = static_cast<int>(ceil_div(s.key_length, PIPER_KEY_BLOCK) * PIPER_KEY_BLOCK);

  piper::MeanParams mp{};
  mp.key = to_input(a->key);
  mp.value = to_input(a->value);
  mp.partials = static_cast<float*>(workspace);
  mp.key_mean = o.key_mean;
  mp.value_mean = o.value_mean;
  mp.batch_heads = bh;
  mp.heads = static_cast<int>(s.heads);
  mp.length = static_cast<int>(s.key_length);
  mp.block_rows = piper::cascade_block_rows(static_cast<int>(s.key_length));
  mp.chunks = piper::cascade_chunks(static_cast<int>(s.key_length));
  mp.tensors = a->is_causal ? 1 : 2;
  mp.status = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + layout.workspace_status_offset);

  piper::PrepDevice dev{};
  if (int st = device_topology(&dev.cus, &dev.xccs)) return st;
  dev.spin_limit = (a->flags & PIPER_PREPARE_SELF_MEAN) ? 0 : piper::kPrepSpinLimit;

  piper::QuantParams qp{};
  qp.query = to_input(a->query);
  qp.key = to_input(a->key);
  qp.value = to_input(a->value);
  qp.batch_heads = bh;
  qp.heads = static_cast<int>(s.heads);
  qp.query_length = static_cast<int>(s.query_length);
  qp.key_length = static_cast<int>(s.key_length);
  qp.sq32 = sq32;
  qp.sk64 = sk64;
  qp.nqb = sq32 / PIPER_QUERY_BLOCK;
  qp.nkb = sk64 / PIPER_KEY_BLOCK;
  qp.q_blocks_wg = with_query ? static_cast<int>(ceil_div(static_cast<int64_t>(bh) * qp.nqb, 4)) : 0;
  qp.k_blocks_wg = static_cast<int>(ceil_div(static_cast<int64_t>(bh) * qp.nkb, 4));
  qp.v_blocks_wg = qp.k_blocks_wg;
  qp.center_value = a->is_causal ? 0 : 1;
  qp.per_thread = (a->flags & PIPER_PREPARE_QK_PER_THREAD) ? 1 : 0;
  qp.key_mean = o.key_mean;
  qp.value_mean = o.value_mean;
  qp.query_code = o.query_code;
  qp.query_scale = o.query_scale;
  qp.key_scale = o.key_scale;
  qp.value_scale = o.value_scale;
  qp.kv_tiles = static_cast<uint8_t*>(o.kv_tiles);

  const hipError_t err =
      piper::launch_prep(a->dtype == PIPER_BFLOAT16, d, mp, qp, dev, static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(PIPER_ERROR_HIP, "prep launch failed: %s", hipGetErrorString(err));
  g_last_error[0] = '\0';
  return PIPER_OK;
}

int piper_prepare(const piper_prepare_args* a, void* stream) { return prepare_call(a, false, stream); }

int piper_prepare_static(const piper_prepare_args* a, void* stream) { return prepare_call(a, true, stream); }

int piper_prepare_status(const piper_shape* shape, const void* workspace, uint32_t* count, void* stream) {
  if (count == nullptr) return fail(PIPER_ERROR_INVALID_ARGUMENT, "count is NULL");
  piper_layout layout;
  if (int st = piper_prepared_layout(shape, &layout)) return st;
  const void* base = workspace;
  if (base == nullptr) {
    void* scratch_address = nullptr;
    if (layout.workspace_bytes > PIPER_STATIC_SCRATCH_BYTES)
      return fail(PIPER_ERROR_UNSUPPORTED, "shape does not fit the static scratch of piper_prepare_static");
    if (int st = device_scratch(&scratch_address)) return st;
    base = scratch_address;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t word = 0;
  hipError_t err = hipMemcpyAsync(&word, static_cast<const char*>(base) + layout.workspace_status_offset,
                                  sizeof(word), hipMemcpyDeviceToHost, s);
  if (err == hipSuccess) err = hipStreamSynchronize(s);
  if (err != hipSuccess) return fail(PIPER_ERROR_HIP, "status read failed: %s", hipGetErrorString(err));
  *count = word;
  g_last_error[0] = '\0';
  return PIPER_OK;
}

int piper_attention_forward(const piper_attention_args* a, void* stream) {
  if (a == nullptr) return fail(PIPER_ERROR_INVALID_ARGUMENT, "args is NULL");
  return launch_attention_call(a->abi_version, a->output_dtype, a->is_causal, a->plan, a->flags, a->shape,
                               a->scale, a->prepared, a->output, nullptr, 0, a->workspace, a->workspace_bytes, stream);
}

int piper_attention_workspace_bytes(const piper_shape* shape, int32_t plan, int64_t* bytes) {
  if (int st = check_shape(shape)) return st;
  if (bytes == nullptr) return fail(PIPER_ERROR_INVALID_ARGUMENT, "bytes is NULL");
  if (plan < 0 || plan > PIPER_PLAN_MASK) return fail(PIPER_ERROR_UNSUPPORTED, "unknown plan %d", plan);
  *bytes = (plan & PIPER_PLAN_WORK_QUEUE)
               ? piper::kQueueBytes
               : piper::attention_partial_bytes(shape->batch * shape->heads, shape->query_length,
                                                static_cast<int>(shape->head_dim), PIPER_PLAN_KEY_PARTS_OF(plan));
  g_last_error[0] = '\0';
  return PIPER_OK;
}

int piper_attention_forward_fused(const piper_attention_fused_args* a, void* stream) {
  if (a == nullptr) return fail(PIPER_ERROR_INVALID_ARGUMENT, "args is NULL");
  return launch_attention_call(a->abi_version, a->output_dtype, a->is_causal, a->plan, a->flags, a->shape,
                               a->scale, a->prepared, a->output, &a->query, a->dtype, a->workspace,
                               a->workspace_bytes, stream);
}

int piper_sage_prepared_layout(const piper_shape* shape, piper_sage_layout* layout) {
  if (int st = check_shape(shape)) return st;
  if (layout == nullptr) return fail(PIPER_ERROR_INVALID_ARGUMENT, "layout is NULL");
  const int64_t bh = shape->batch * shape->heads;
  const int64_t d = shape->head_dim;
  const int64_t nkb = ceil_div(shape->key_length, PIPER_KEY_BLOCK);
  const int64_t chunks = piper::cascade_chunks(static_cast<int>(shape->key_length));
  layout->key_scale_bytes = bh * nkb * PIPER_KEY_SCALE_SLOTS * 4;
  layout->mean_bytes = bh * d * 4;
  layout->kv_tile_bytes = PIPER_SAGE_TILE_BYTES(d);
  layout->kv_tiles_bytes = bh * nkb * PIPER_SAGE_TILE_BYTES(d);
  layout->workspace_bytes = 2 * bh * (chunks + 1) * d * 4;
  g_last_error[0] = '\0';
  return PIPER_OK;
}

int piper_sage_prepare(const piper_sage_prepare_args* a, void* stream) {
  if (a == nullptr) return fail(PIPER_ERROR_INVALID_ARGUMENT, "args is NULL");
  if (a->abi_version != PIPER_ABI_VERSION)
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "ABI version mismatch: caller %d, library %d", a->abi_version,
                PIPER_ABI_VERSION);
  if (a->dtype != PIPER_FLOAT16 && a->dtype != PIPER_BFLOAT16)
    return fail(PIPER_ERROR_UNSUPPORTED, "input dtype must be float16 or bfloat16");
  if (int st = check_shape(&a->shape)) return st;
  if ((a->flags & ~PIPER_PREPARE_QK_PER_THREAD) != 0) return fail(PIPER_ERROR_UNSUPPORTED, "unknown flags %d", a->flags);
  if (int st = check_input("key", a->key)) return st;
  if (int st = check_input("value", a->value)) return st;
  const piper_sage_prepared& o = a->prepared;
  if (!o.key_scale || !o.key_mean || !o.value_scale || !o.kv_tiles)
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "a prepared output pointer is NULL");
  if (!aligned16(o.kv_tiles) || !aligned16(o.value_scale))
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "prepared buffers must be 16-byte aligned");
  piper_sage_layout layout;
  if (int st = piper_sage_prepared_layout(&a->shape, &layout)) return st;
  if (a->workspace == nullptr || a->workspace_bytes < layout.workspace_bytes)
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "workspace needs %lld bytes, got %lld",
                (long long)layout.workspace_bytes, (long long)a->workspace_bytes);

  const piper_shape& s = a->shape;
  const int bh = static_cast<int>(s.batch * s.heads);
  const int nkb = static_cast<int>(ceil_div(s.key_length, PIPER_KEY_BLOCK));

  // statistics: the K sum (torch's CPU order) and the per-column max |v|
  piper::MeanParams mp{};
  mp.key = to_input(a->key);
  mp.value = to_input(a->value);
  mp.partials = static_cast<float*>(a->workspace);
  mp.key_mean = o.key_mean;
  mp.value_mean = nullptr;
  mp.batch_heads = bh;
  mp.heads = static_cast<int>(s.heads);
  mp.length = static_cast<int>(s.key_length);
  mp.block_rows = piper::cascade_block_rows(static_cast<int>(s.key_length));
  mp.chunks = piper::cascade_chunks(static_cast<int>(s.key_length));
  mp.tensors = 2;
  mp.value_absmax = 1;
  mp.value_scale = o.value_scale;

  piper::SageQuantParams qp{};
  qp.key = to_input(a->key);
  qp.value = to_input(a->value);
  qp.batch_heads = bh;
  qp.heads = static_cast<int>(s.heads);
  qp.key_length = static_cast<int>(s.key_length);
  qp.nkb = nkb;
  qp.k_blocks_wg = static_cast<int>(ceil_div(static_cast<int64_t>(bh) * nkb, 4));
  qp.v_blocks_wg = qp.k_blocks_wg;
  qp.key_mean = o.key_mean;
  qp.value_scale = o.value_scale;
  qp.key_scale = o.key_scale;
  qp.kv_tiles = static_cast<uint8_t*>(o.kv_tiles);
  qp.per_thread = (a->flags & PIPER_PREPARE_QK_PER_THREAD) ? 1 : 0;

  const hipError_t err =
      piper::launch_sage_prep(a->dtype == PIPER_BFLOAT16, static_cast<int>(s.head_dim), mp, qp, static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(PIPER_ERROR_HIP, "prep launch failed: %s", hipGetErrorString(err));
  g_last_error[0] = '\0';
  return PIPER_OK;
}

int piper_sage_attention_forward(const piper_sage_attention_args* a, void* stream) {
  if (a == nullptr) return fail(PIPER_ERROR_INVALID_ARGUMENT, "args is NULL");
  if (a->abi_version != PIPER_ABI_VERSION)
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "ABI version mismatch: caller %d, library %d", a->abi_version,
                PIPER_ABI_VERSION);
  if (a->dtype != PIPER_FLOAT16 && a->dtype != PIPER_BFLOAT16)
    return fail(PIPER_ERROR_UNSUPPORTED, "query dtype must be float16 or bfloat16");
  if (a->output_dtype != PIPER_FLOAT16 && a->output_dtype != PIPER_BFLOAT16 && a->output_dtype != PIPER_FLOAT32)
    return fail(PIPER_ERROR_UNSUPPORTED, "output dtype must be float16, bfloat16 or float32");
  const piper_shape& s = a->shape;
  if (int st = check_shape(&s)) return st;
  if (a->is_causal && s.query_length != s.key_length)
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "causal attention requires equal query and key lengths");
  if (!(std::isfinite(a->scale) && a->scale > 0.0f))
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "scale must be finite and positive");
  if (a->plan < 0 || a->plan > PIPER_PLAN_MASK) return fail(PIPER_ERROR_UNSUPPORTED, "unknown plan %d", a->plan);
  if (PIPER_PLAN_KEY_PARTS_OF(a->plan) > 1)
    return fail(PIPER_ERROR_UNSUPPORTED, "SageAttention2++ has no key-range split plans");
  if (a->plan & PIPER_PLAN_WORK_QUEUE) return fail(PIPER_ERROR_UNSUPPORTED, "SageAttention2++ has no work-queue plan");
  if ((a->flags & ~(PIPER_ATTENTION_QK_PER_THREAD | PIPER_SAGE_FP16_PARTIALS)) != 0)
    return fail(PIPER_ERROR_UNSUPPORTED, "unknown flags %d", a->flags);
  if (int st = check_input("query", a->query)) return st;
  const piper_sage_prepared& o = a->prepared;
  if (!o.value_scale || !o.kv_tiles || !a->output)
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "a prepared input or the output pointer is NULL");
  if (!aligned16(o.kv_tiles) || !aligned16(o.value_scale) || (reinterpret_cast<uintptr_t>(a->output) & 7u) != 0)
    return fail(PIPER_ERROR_INVALID_ARGUMENT, "prepared buffers must be 16-byte and the output 8-byte aligned");

  // 3: three 4-wave workgroups per CU (sage_attention_w3_kernel)
  const int waves = (a->plan & PIPER_PLAN_THREE_WORKGROUPS) ? 3 : (a->plan & PIPER_PLAN_FOUR_WAVES) ? 4 : 8;
  piper::SageParams sp{};
  sp.kv_tiles = static_cast<const uint8_t*>(o.kv_tiles);
  sp.value_scale = o.value_scale;
  sp.output = a->output;
  sp.query = to_input(a->query);
  sp.query_bf16 = a->dtype == PIPER_BFLOAT16 ? 1 : 0;
  sp.heads = static_cast<int>(s.heads);
  sp.batch_heads = static_cast<int>(s.batch * s.heads);
  sp.query_length = static_cast<int>(s.query_length);
  sp.key_length = static_cast<int>(s.key_length);
  sp.nkb = static_cast<int>(ceil_div(s.key_length, PIPER_KEY_BLOCK));
  sp.query_tiles = static_cast<int>(ceil_div(s.query_length, 32 * (waves == 3 ? 4 : waves)));
  sp.scale_log2e = static_cast<float>(static_cast<double>(a->scale) * 1.4426950408889634);
  sp.causal_forward = (a->plan & PIPER_PLAN_CAUSAL_FORWARD) ? 1 : 0;
  sp.xcd_remap = (a->plan & PIPER_PLAN_NO_XCD_REMAP) ? 0 : 1;
  sp.causal_interleave = (a->plan & PIPER_PLAN_CAUSAL_INTERLEAVE) ? 1 : 0;
  sp.per_thread = (a->flags & PIPER_ATTENTION_QK_PER_THREAD) ? 1 : 0;
  sp.fp16_partials = (a->flags & PIPER_SAGE_FP16_PARTIALS) ? 1 : 0;
  if (static_cast<int64_t>(sp.query_tiles) * sp.batch_heads > 0x7fffffff)
    return fail(PIPER_ERROR_UNSUPPORTED, "too many workgroups");

  const hipError_t err = piper::launch_sage_attention(static_cast<int>(s.head_dim), a->is_causal != 0,
                                                      a->output_dtype, waves, sp, static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(PIPER_ERROR_HIP, "attention launch failed: %s", hipGetErrorString(err));
  g_last_error[0] = '\0';
  return PIPER_OK;
}

}  // extern "C"
