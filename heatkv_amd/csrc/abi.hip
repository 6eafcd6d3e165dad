// C ABI of libheatkv.so (declared in include/heatkv.h): argument checks,
// error codes and messages, then the launches in pack.hip / seg_attn.hip.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/heatkv.h"
#include "hkv_internal.h"

namespace {

thread_local std::string g_last_error;

int32_t fail(int32_t code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int32_t fail(int32_t code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int32_t ok() {
  g_last_error.clear();
  return HKV_OK;
}

int32_t elem_bytes(int32_t dt) {
  switch (dt) {
    case HKV_DTYPE_F16:
    case HKV_DTYPE_BF16: return 2;
    case HKV_DTYPE_F32: return 4;
    default: return 0;
  }
}

// ------------------------------------------------ allocation-free attention
//
// Workspace of hkv_segmented_attention_noalloc: the round split's counters
// plus two partial records per resident workgroup slot, for up to
// kScratchSlots slots (a 256-CU device at 2 workgroups per CU): 69.3 MB in
// every GPU the library runs on, held until the process ends.  Host code
// never uses the array's name as an address: each device's copy is looked up
// once with hipGetSymbolAddress and that pointer is what the kernels get.
constexpr int32_t kScratchSlots = 512;
constexpr int64_t kScratchBytes =
    hkv::kCounterBytes + 2LL * kScratchSlots * hkv::kPartialFloats * static_cast<int64_t>(sizeof(float));
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

__global__ void clear_words(uint32_t* p, int32_t n) {
  for (int32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// This device's scratch (device current), its counters cleared on `stream`
// at the first call; null when the runtime cannot give its address.
void* device_scratch(int device, hipStream_t stream) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[device] != nullptr) return g_scratch[device];
  void* ptr = nullptr;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) return nullptr;
  // the kernels leave the counters zero after every call; they start zero here
  clear_words<<<16, 256, 0, stream>>>(static_cast<uint32_t*>(ptr), static_cast<int32_t>(hkv::kCounterBytes / 4));
  if (hipGetLastError() != hipSuccess) return nullptr;
  g_scratch[device] = ptr;
  return ptr;
}

}  // namespace

extern "C" {

// 0.2.0: hkv_segmented_attention's dot modes and work plan arguments, the
// split-row K dtype; a work plan with no units is refused.
// 0.3.0: hkv_segmented_attention_append2 / _bind2 (a second append destination).
int32_t hkv_version(void) { return HKV_VERSION; }

int32_t hkv_device_ok(int32_t device) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return 0;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return 0;
  return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

const char* hkv_last_error(void) { return g_last_error.c_str(); }

int32_t hkv_pack_segments(const void* src_k, const void* src_v, void* dst_k, void* dst_v,
                          int64_t src_batch_stride, int64_t dst_batch_stride, int64_t src_rows,
                          int64_t dst_rows, int32_t batch, int32_t head_dim,
                          int32_t k_elem_bytes, int32_t v_elem_bytes,
                          const int64_t* dst_starts, const int64_t* src_starts,
                          const int64_t* lengths, int32_t n_items, int32_t max_length,
                          void* stream) {
  if (n_items < 0) return fail(HKV_ERR_INVALID_ARG, "n_items must be >= 0 (got %d)", n_items);
  if (n_items == 0 || max_length <= 0) return ok();
  if (batch <= 0 || batch > 65535)
    return fail(HKV_ERR_INVALID_ARG, "batch must be in [1, 65535] (got %d)", batch);
  if (head_dim <= 0 || head_dim > 128)
    return fail(HKV_ERR_UNSUPPORTED, "pack_flat_segments_kv currently supports head_dim <= 128");
  if ((k_elem_bytes != 2 && k_elem_bytes != 4) || (v_elem_bytes != 2 && v_elem_bytes != 4))
    return fail(HKV_ERR_UNSUPPORTED, "element sizes must be 2 or 4 bytes (got %d, %d)",
                k_elem_bytes, v_elem_bytes);
  if (!src_k || !src_v || !dst_k || !dst_v || !dst_starts || !src_starts || !lengths)
    return fail(HKV_ERR_INVALID_ARG, "null pointer argument");
  if (src_rows < 0 || dst_rows < 0 || src_batch_stride < 0 || dst_batch_stride < 0)
    return fail(HKV_ERR_INVALID_ARG, "negative size or stride");
  if (batch > 1 && (src_batch_stride < src_rows * head_dim || dst_batch_stride < dst_rows * head_dim))
    return fail(HKV_ERR_INVALID_ARG, "batch stride smaller than rows * head_dim");
  int64_t limit = max_length;
  if (limit > dst_rows) limit = dst_rows;
  if (limit > src_rows) limit = src_rows;
  if (limit <= 0) return ok();
  hkv::PackArgs a{};
  a.src_k = src_k;
  a.src_v = src_v;
  a.dst_k = dst_k;
  a.dst_v = dst_v;
  a.src_batch_stride = src_batch_stride;
  a.dst_batch_stride = dst_batch_stride;
  a.src_rows = src_rows;
  a.dst_rows = dst_rows;
  a.dst_starts = dst_starts;
  a.src_starts = src_starts;
  a.lengths = lengths;
  a.batch = batch;
  a.head_dim = head_dim;
  a.k_elem_bytes = k_elem_bytes;
  a.v_elem_bytes = v_elem_bytes;
  a.n_items = n_items;
  a.row_limit = static_cast<int32_t>(limit > 0x7fffffffLL ? 0x7fffffffLL : limit);
  const hipError_t e = hkv::launch_pack(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(HKV_ERR_LAUNCH, "pack kernel launch failed: %s", hipGetErrorString(e));
  return ok();
}

int32_t hkv_concat_kv(const void* old_k, const void* new_k, const void* old_v, const void* new_v, void* out_k,
                      void* out_v, int64_t groups, int64_t t_old, int64_t t_new, int64_t k_row_bytes,
                      int64_t v_row_bytes, void* stream) {
  if (groups < 0 || t_old < 0 || t_new < 0 || k_row_bytes <= 0 || v_row_bytes <= 0 || k_row_bytes % 2 != 0 ||
      v_row_bytes % 2 != 0)
    return fail(HKV_ERR_INVALID_ARG, "groups and row counts must be >= 0 and row sizes positive and even");
  if (groups == 0 || t_old + t_new == 0) return ok();
  if (!out_k || !out_v || (t_old > 0 && (!old_k || !old_v)) || (t_new > 0 && (!new_k || !new_v)))
    return fail(HKV_ERR_INVALID_ARG, "null pointer argument");
  if ((t_old > t_new ? t_old : t_new) * (k_row_bytes > v_row_bytes ? k_row_bytes : v_row_bytes) >
      65535LL * 64 * 1024)
    return fail(HKV_ERR_UNSUPPORTED, "a (batch, head) group of more than 4 GiB");
  hkv::ConcatArgs a{old_k, new_k, old_v, new_v, out_k, out_v, groups, t_old, t_new, k_row_bytes, v_row_bytes};
  const hipError_t e = hkv::launch_concat(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(HKV_ERR_LAUNCH, "concat launch failed: %s", hipGetErrorString(e));
  return ok();
}

int32_t hkv_segmented_attention(const void* q, const void* slab_k, const void* slab_v,
                                const int32_t* seg_starts, const int32_t* seg_ends,
                                const int32_t* seg_counts, const void* cur_k, const void* cur_v,
                                void* out, float* lse, int32_t batch, int32_t heads,
                                int32_t cur_len, int64_t slab_capacity, int32_t max_segments,
                                int32_t head_dim, int32_t q_dtype, int32_t k_dtype,
                                int32_t v_dtype, int32_t out_dtype, float softmax_scale, int32_t use_exp2,
                                int32_t qk_dot_mode, int32_t value_dot_mode,
                                const int32_t* work_plan, int32_t plan_units,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  // without append offsets the slab is only read
  return hkv_segmented_attention_append(q, const_cast<void*>(slab_k), const_cast<void*>(slab_v), seg_starts,
                                        seg_ends, seg_counts, cur_k, cur_v, out, lse, batch, heads, cur_len,
                                        slab_capacity, max_segments, head_dim, q_dtype, k_dtype, v_dtype, out_dtype,
                                        softmax_scale, use_exp2, qk_dot_mode, value_dot_mode, work_plan, plan_units,
                                        workspace, workspace_bytes, nullptr, stream);
}

// Validates the arguments of hkv_segmented_attention_append and fills `a`
// (0 or a negative HKV_ERR_* code with the message set).  With
// `check_tensors` false the tensor pointers (q, slab, current K/V, out) are
// not looked at: hkv_segmented_attention_bind checks them at each call.
namespace {
int32_t build_attention_args(hkv::AttnArgs& a, bool check_tensors, const void* q, void* slab_k, void* slab_v,
                                      const int32_t* seg_starts, const int32_t* seg_ends,
                                      const int32_t* seg_counts, const void* cur_k, const void* cur_v,
                                      void* out, float* lse, int32_t batch, int32_t heads,
                                      int32_t cur_len, int64_t slab_capacity, int32_t max_segments,
                                      int32_t head_dim, int32_t q_dtype, int32_t k_dtype,
                                      int32_t v_dtype, int32_t out_dtype, float softmax_scale, int32_t use_exp2,
                                      int32_t qk_dot_mode, int32_t value_dot_mode,
                                      const int32_t* work_plan, int32_t plan_units,
                                      void* workspace, int64_t workspace_bytes, const int32_t* append_offsets,
                                      void* slab2_k = nullptr, void* slab2_v = nullptr, int64_t slab2_capacity = 0,
                                      const int32_t* append2_offsets = nullptr) {
  (void)use_exp2;  // exp and exp2 modes are the same function; the kernel folds log2(e)
  if (qk_dot_mode < 0 || qk_dot_mode > 2)
    return fail(HKV_ERR_INVALID_ARG, "qk_dot_mode must be 0 (bf16), 1 (tf32) or 2 (fp32) (got %d)", qk_dot_mode);
  if (value_dot_mode != 0 && value_dot_mode != 2)
    return fail(HKV_ERR_INVALID_ARG, "value_dot_mode must be 0 (bf16) or 2 (fp32) (got %d)", value_dot_mode);
  // every (batch, head, query tile) item has a unit in a plan built for the
  // call, so a plan without units cannot match it (its outputs would stay unwritten)
  if (work_plan != nullptr && plan_units <= 0)
    return fail(HKV_ERR_INVALID_ARG, "plan_units must be > 0 with a work plan (got %d)", plan_units);
  if (head_dim != 128)
    return fail(HKV_ERR_UNSUPPORTED, "real_scale_fused_segmented v1 only supports head_dim=128");
  if (cur_len <= 0)
    return fail(HKV_ERR_UNSUPPORTED, "real_scale_fused_segmented requires current_len > 0");
  if (batch <= 0 || heads <= 0)
    return fail(HKV_ERR_INVALID_ARG, "batch and heads must be positive (got %d, %d)", batch, heads);
  if (heads > 1024)
    return fail(HKV_ERR_UNSUPPORTED, "real_scale_fused_segmented supports at most 1024 heads (got %d)", heads);
  const bool split_k = k_dtype == HKV_DTYPE_SPLIT_ROWS;
  if (elem_bytes(q_dtype) == 0 || (elem_bytes(k_dtype) == 0 && !split_k) || elem_bytes(v_dtype) == 0)
    return fail(HKV_ERR_UNSUPPORTED,
                "real_scale_fused_segmented supports only float16, bfloat16, or float32 tensors");
  if (split_k) {
    if (q_dtype != HKV_DTYPE_F32 || elem_bytes(v_dtype) != 2 || qk_dot_mode == 2 || value_dot_mode == 2)
      return fail(HKV_ERR_UNSUPPORTED,
                  "split K rows take float32 q, 16-bit v and the default (or tf32) dot modes (got q %d, v %d, "
                  "modes %d/%d)", q_dtype, v_dtype, qk_dot_mode, value_dot_mode);
  } else if (q_dtype != k_dtype) {
    return fail(HKV_ERR_UNSUPPORTED, "q and k must share one dtype (got %d and %d)", q_dtype, k_dtype);
  }
  if (out_dtype == 0) out_dtype = q_dtype;
  if (elem_bytes(out_dtype) == 0)
    return fail(HKV_ERR_UNSUPPORTED, "out_dtype must be 0 (q's dtype), float16, bfloat16 or float32 (got %d)",
                out_dtype);
  if (max_segments < 0 || max_segments > hkv::kMaxSegments)
    return fail(HKV_ERR_UNSUPPORTED, "max_segments must be in [0, %d] (got %d)", hkv::kMaxSegments,
                max_segments);
  if (slab_capacity < 0) return fail(HKV_ERR_INVALID_ARG, "slab_capacity must be >= 0");
  // Retained prior rows plus current rows index an int32 key stream.
  if (slab_capacity * static_cast<int64_t>(max_segments > 0 ? max_segments : 1) + cur_len >
      0x7fffffffLL)
    return fail(HKV_ERR_UNSUPPORTED, "slab_capacity * max_segments + current_len exceeds 2^31");
  if (!seg_counts || (max_segments > 0 && (!seg_starts || !seg_ends)) ||
      (check_tensors && (!q || !cur_k || !cur_v || !out)))
    return fail(HKV_ERR_INVALID_ARG, "null pointer argument");
  if (check_tensors && slab_capacity > 0 && (!slab_k || !slab_v))
    return fail(HKV_ERR_INVALID_ARG, "null slab pointer with nonzero capacity");
  if (workspace != nullptr) {
    if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0)
      return fail(HKV_ERR_INVALID_ARG, "workspace must be 256-byte aligned");
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess)
      return fail(HKV_ERR_DEVICE, "hipGetDevice failed");
    const int64_t need = hkv::split_workspace_bytes(hkv::split_slots(device));
    if (need <= 0) return fail(HKV_ERR_DEVICE, "cannot query the CU count of device %d", device);
    if (workspace_bytes < need)
      return fail(HKV_ERR_INVALID_ARG, "workspace of %lld bytes is smaller than the %lld required",
                  static_cast<long long>(workspace_bytes), static_cast<long long>(need));
  }
  // The kernels address one batch row of the slab and one (batch, head) of
  // the current tensors through 32-bit buffer offsets.
  const int64_t row_bytes = static_cast<int64_t>(head_dim) * 4;
  if (slab_capacity * row_bytes >= 0x7fffffffLL || static_cast<int64_t>(cur_len) * row_bytes >= 0x7fffffffLL)
    return fail(HKV_ERR_UNSUPPORTED, "slab rows per batch row and current_len must stay below %lld",
                static_cast<long long>(0x7fffffffLL / row_bytes));
  if (append_offsets != nullptr) {
    // the copy moves whole rows 16 bytes per access
    const uintptr_t bits = reinterpret_cast<uintptr_t>(slab_k) | reinterpret_cast<uintptr_t>(slab_v) |
                           reinterpret_cast<uintptr_t>(cur_k) | reinterpret_cast<uintptr_t>(cur_v);
    if (slab_capacity < cur_len || (check_tensors && (bits & 15) != 0))
      return fail(HKV_ERR_INVALID_ARG,
                  "the append needs slab_capacity >= current_len and 16-byte aligned slab and current tensors");
  }
  if (append2_offsets != nullptr) {
    // the second destination of the append: always bound with its tensors
    if (append_offsets == nullptr)
      return fail(HKV_ERR_INVALID_ARG, "append2_offsets needs append_offsets (it repeats that append)");
    if (!slab2_k || !slab2_v || slab2_capacity < cur_len ||
        ((reinterpret_cast<uintptr_t>(slab2_k) | reinterpret_cast<uintptr_t>(slab2_v)) & 15) != 0)
      return fail(HKV_ERR_INVALID_ARG,
                  "the second append needs 16-byte aligned slab2 tensors and slab2_capacity >= current_len");
    if (slab2_capacity * row_bytes >= 0x7fffffffLL)
      return fail(HKV_ERR_UNSUPPORTED, "slab2 rows per batch row must stay below %lld",
                  static_cast<long long>(0x7fffffffLL / row_bytes));
  }
  a = hkv::AttnArgs{};
  a.q = q;
  a.slab_k = slab_k;
  a.slab_v = slab_v;
  a.seg_starts = seg_starts;
  a.seg_ends = seg_ends;
  a.seg_counts = seg_counts;
  a.cur_k = cur_k;
  a.cur_v = cur_v;
  a.out = out;
  a.lse = lse;
  a.slab_capacity = slab_capacity;
  a.batch = batch;
  a.heads = heads;
  a.cur_len = cur_len;
  a.max_segments = max_segments;
  a.softmax_scale = softmax_scale;
  a.q_dtype = q_dtype;
  a.k_dtype = k_dtype;
  a.v_dtype = v_dtype;
  a.out_dtype = out_dtype;
  a.qk_dot_mode = qk_dot_mode;
  a.value_dot_mode = value_dot_mode;
  a.workspace = workspace;
  a.workspace_bytes = workspace != nullptr ? workspace_bytes : 0;
  a.plan = work_plan;
  a.plan_units = work_plan != nullptr ? plan_units : 0;
  a.append_offsets = append_offsets;
  a.append2_offsets = append2_offsets;
  a.slab2_k = append2_offsets != nullptr ? slab2_k : nullptr;
  a.slab2_v = append2_offsets != nullptr ? slab2_v : nullptr;
  a.slab2_capacity = append2_offsets != nullptr ? slab2_capacity : 0;
  return 0;
}
}  // namespace

int32_t hkv_segmented_attention_append(const void* q, void* slab_k, void* slab_v,
                                      const int32_t* seg_starts, const int32_t* seg_ends,
                                      const int32_t* seg_counts, const void* cur_k, const void* cur_v,
                                      void* out, float* lse, int32_t batch, int32_t heads,
                                      int32_t cur_len, int64_t slab_capacity, int32_t max_segments,
                                      int32_t head_dim, int32_t q_dtype, int32_t k_dtype,
                                      int32_t v_dtype, int32_t out_dtype, float softmax_scale, int32_t use_exp2,
                                      int32_t qk_dot_mode, int32_t value_dot_mode,
                                      const int32_t* work_plan, int32_t plan_units,
                                      void* workspace, int64_t workspace_bytes, const int32_t* append_offsets,
                                       void* stream) {
  hkv::AttnArgs a{};
  const int32_t code = build_attention_args(
      a, true, q, slab_k, slab_v, seg_starts, seg_ends, seg_counts, cur_k, cur_v, out, lse, batch, heads, cur_len,
      slab_capacity, max_segments, head_dim, q_dtype, k_dtype, v_dtype, out_dtype, softmax_scale, use_exp2,
      qk_dot_mode, value_dot_mode, work_plan, plan_units, workspace, workspace_bytes, append_offsets);
  if (code != 0) return code;
  const hipError_t e = hkv::launch_segmented_attention(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess)
    return fail(HKV_ERR_LAUNCH, "segmented attention launch failed: %s", hipGetErrorString(e));
  return ok();
}

int32_t hkv_segmented_attention_append2(const void* q, void* slab_k, void* slab_v,
                                       const int32_t* seg_starts, const int32_t* seg_ends,
                                       const int32_t* seg_counts, const void* cur_k, const void* cur_v,
                                       void* out, float* lse, int32_t batch, int32_t heads,
                                       int32_t cur_len, int64_t slab_capacity, int32_t max_segments,
                                       int32_t head_dim, int32_t q_dtype, int32_t k_dtype,
                                       int32_t v_dtype, int32_t out_dtype, float softmax_scale, int32_t use_exp2,
                                       int32_t qk_dot_mode, int32_t value_dot_mode,
                                       const int32_t* work_plan, int32_t plan_units,
                                       void* workspace, int64_t workspace_bytes, const int32_t* append_offsets,
                                       void* slab2_k, void* slab2_v, int64_t slab2_capacity,
                                       const int32_t* append2_offsets, void* stream) {
  hkv::AttnArgs a{};
  const int32_t code = build_attention_args(
      a, true, q, slab_k, slab_v, seg_starts, seg_ends, seg_counts, cur_k, cur_v, out, lse, batch, heads, cur_len,
      slab_capacity, max_segments, head_dim, q_dtype, k_dtype, v_dtype, out_dtype, softmax_scale, use_exp2,
      qk_dot_mode, value_dot_mode, work_plan, plan_units, workspace, workspace_bytes, append_offsets, slab2_k,
      slab2_v, slab2_capacity, append2_offsets);
  if (code != 0) return code;
  const hipError_t e = hkv::launch_segmented_attention(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess)
    return fail(HKV_ERR_LAUNCH, "segmented attention launch failed: %s", hipGetErrorString(e));
  return ok();
}

// The argument block of hkv_segmented_attention_bind: the validated launch
// arguments, the device they were validated for and a tag.
namespace {
constexpr uint32_t kBoundTag = 0x484b5641u;
struct BoundAttention {
  uint32_t tag;
  int32_t device;
  hkv::AttnArgs a;
};
}  // namespace

int64_t hkv_segmented_attention_bound_bytes(void) { return static_cast<int64_t>(sizeof(BoundAttention)); }

int32_t hkv_segmented_attention_bind(void* bound, int64_t bound_bytes, const int32_t* seg_starts,
                                     const int32_t* seg_ends, const int32_t* seg_counts, int32_t batch,
                                     int32_t heads, int32_t cur_len, int64_t slab_capacity, int32_t max_segments,
                                     int32_t head_dim, int32_t q_dtype, int32_t k_dtype, int32_t v_dtype,
                                     int32_t out_dtype, float softmax_scale, int32_t use_exp2, int32_t qk_dot_mode,
                                     int32_t value_dot_mode, const int32_t* work_plan, int32_t plan_units,
                                     void* workspace, int64_t workspace_bytes, const int32_t* append_offsets) {
  if (bound == nullptr || bound_bytes < static_cast<int64_t>(sizeof(BoundAttention)) ||
      (reinterpret_cast<uintptr_t>(bound) & 7) != 0)
    return fail(HKV_ERR_INVALID_ARG, "bound must point to %d bytes, 8-byte aligned (hkv_segmented_attention_bound_bytes)",
                static_cast<int>(sizeof(BoundAttention)));
  BoundAttention* b = static_cast<BoundAttention*>(bound);
  b->tag = 0;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return fail(HKV_ERR_DEVICE, "hipGetDevice failed");
  const int32_t code = build_attention_args(
      b->a, false, nullptr, nullptr, nullptr, seg_starts, seg_ends, seg_counts, nullptr, nullptr, nullptr, nullptr,
      batch, heads, cur_len, slab_capacity, max_segments, head_dim, q_dtype, k_dtype, v_dtype, out_dtype,
      softmax_scale, use_exp2, qk_dot_mode, value_dot_mode, work_plan, plan_units, workspace, workspace_bytes,
      append_offsets);
  if (code != 0) return code;
  b->device = device;
  b->tag = kBoundTag;
  return ok();
}

int32_t hkv_segmented_attention_bind2(void* bound, int64_t bound_bytes, const int32_t* seg_starts,
                                      const int32_t* seg_ends, const int32_t* seg_counts, int32_t batch,
                                      int32_t heads, int32_t cur_len, int64_t slab_capacity, int32_t max_segments,
                                      int32_t head_dim, int32_t q_dtype, int32_t k_dtype, int32_t v_dtype,
                                      int32_t out_dtype, float softmax_scale, int32_t use_exp2,
                                      int32_t qk_dot_mode, int32_t value_dot_mode, const int32_t* work_plan,
                                      int32_t plan_units, void* workspace, int64_t workspace_bytes,
                                      const int32_t* append_offsets, void* slab2_k, void* slab2_v,
                                      int64_t slab2_capacity, const int32_t* append2_offsets) {
  if (bound == nullptr || bound_bytes < static_cast<int64_t>(sizeof(BoundAttention)) ||
      (reinterpret_cast<uintptr_t>(bound) & 7) != 0)
    return fail(HKV_ERR_INVALID_ARG, "bound must point to %d bytes, 8-byte aligned (hkv_segmented_attention_bound_bytes)",
                static_cast<int>(sizeof(BoundAttention)));
  BoundAttention* b = static_cast<BoundAttention*>(bound);
  b->tag = 0;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return fail(HKV_ERR_DEVICE, "hipGetDevice failed");
  const int32_t code = build_attention_args(
      b->a, false, nullptr, nullptr, nullptr, seg_starts, seg_ends, seg_counts, nullptr, nullptr, nullptr, nullptr,
      batch, heads, cur_len, slab_capacity, max_segments, head_dim, q_dtype, k_dtype, v_dtype, out_dtype,
      softmax_scale, use_exp2, qk_dot_mode, value_dot_mode, work_plan, plan_units, workspace, workspace_bytes,
      append_offsets, slab2_k, slab2_v, slab2_capacity, append2_offsets);
  if (code != 0) return code;
  b->device = device;
  b->tag = kBoundTag;
  return ok();
}

int32_t hkv_segmented_attention_call(const void* bound, const void* q, void* slab_k, void* slab_v,
                                     const void* cur_k, const void* cur_v, void* out, void* stream) {
  const BoundAttention* b = static_cast<const BoundAttention*>(bound);
  if (b == nullptr || b->tag != kBoundTag) return fail(HKV_ERR_INVALID_ARG, "not a bound attention call");
  if (!q || !cur_k || !cur_v || !out || (b->a.slab_capacity > 0 && (!slab_k || !slab_v)))
    return fail(HKV_ERR_INVALID_ARG, "null pointer argument");
  if (b->a.append_offsets != nullptr &&
      ((reinterpret_cast<uintptr_t>(slab_k) | reinterpret_cast<uintptr_t>(slab_v) |
        reinterpret_cast<uintptr_t>(cur_k) | reinterpret_cast<uintptr_t>(cur_v)) & 15) != 0)
    return fail(HKV_ERR_INVALID_ARG, "the append needs 16-byte aligned slab and current tensors");
  hkv::AttnArgs a = b->a;
  a.q = q;
  a.slab_k = slab_k;
  a.slab_v = slab_v;
  a.cur_k = cur_k;
  a.cur_v = cur_v;
  a.out = out;
  const hipError_t e = hkv::launch_segmented_attention(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess)
    return fail(HKV_ERR_LAUNCH, "segmented attention launch failed: %s", hipGetErrorString(e));
  return ok();
}

int32_t hkv_qkv_produce(const void* qkv, int64_t token_stride, const float* q_bias,
                        const float* v_bias, const float* scale_mul, const float* rope,
                        int64_t rope_rows, int64_t rope_start, void* q_out, void* k_out,
                        void* v_out, void* slab_k, void* slab_v, const int32_t* append_offsets,
                        int64_t slab_capacity, int32_t batch, int32_t heads, int32_t len,
                        int32_t head_dim, int32_t qkv_dtype, int32_t q_dtype, int32_t k_dtype,
                        int32_t v_dtype, int32_t normalize, float eps, void* stream) {
  if (head_dim != 128) return fail(HKV_ERR_UNSUPPORTED, "qkv producer supports head_dim=128 only");
  if (elem_bytes(qkv_dtype) == 0 || v_dtype != qkv_dtype)
    return fail(HKV_ERR_UNSUPPORTED,
                "qkv producer takes a bfloat16, float16 or float32 projection and writes v in its dtype "
                "(got projection %d, v %d)", qkv_dtype, v_dtype);
  const bool split_k = k_dtype == HKV_DTYPE_SPLIT_ROWS;
  if (split_k ? q_dtype != HKV_DTYPE_F32 : (elem_bytes(q_dtype) == 0 || q_dtype != k_dtype))
    return fail(HKV_ERR_UNSUPPORTED,
                "q and k outputs must share one dtype: float32, float16 or bfloat16 (or float32 q with k as "
                "split rows)");
  if (batch < 0 || heads <= 0 || len < 0)
    return fail(HKV_ERR_INVALID_ARG, "batch, len must be >= 0 and heads > 0 (got %d, %d, %d)", batch,
                len, heads);
  if (batch == 0 || len == 0) return ok();
  if (!(eps >= 0.f)) return fail(HKV_ERR_INVALID_ARG, "eps must be >= 0");
  const int64_t hd = static_cast<int64_t>(heads) * head_dim;
  if (token_stride < 3 * hd || token_stride % 8 != 0)
    return fail(HKV_ERR_INVALID_ARG, "token_stride must be >= 3 * heads * head_dim and a multiple of 8");
  if (!qkv || !q_out || !k_out || !v_out) return fail(HKV_ERR_INVALID_ARG, "null pointer argument");
  if (rope != nullptr && (rope_start < 0 || rope_rows < rope_start + len))
    return fail(HKV_ERR_INVALID_ARG, "rope rows [%lld, %lld) outside the table of %lld rows",
                static_cast<long long>(rope_start), static_cast<long long>(rope_start + len),
                static_cast<long long>(rope_rows));
  if (append_offsets != nullptr && (!slab_k || !slab_v || slab_capacity <= 0))
    return fail(HKV_ERR_INVALID_ARG, "append needs slab_k, slab_v and slab_capacity > 0");
  // 16-byte vector accesses.
  const void* aligned[] = {qkv, q_bias, v_bias, rope, q_out, k_out, v_out, slab_k, slab_v};
  for (const void* p : aligned)
    if ((reinterpret_cast<uintptr_t>(p) & 15) != 0)
      return fail(HKV_ERR_INVALID_ARG, "tensor pointers must be 16-byte aligned");
  hkv::ProduceArgs a{};
  a.qkv = qkv;
  a.token_stride = token_stride;
  a.q_bias = q_bias;
  a.v_bias = v_bias;
  a.scale_mul = scale_mul;
  a.rope = rope;
  a.rope_rows = rope_rows;
  a.rope_start = rope_start;
  a.q_out = q_out;
  a.k_out = k_out;
  a.v_out = v_out;
  a.slab_k = append_offsets != nullptr ? slab_k : nullptr;
  a.slab_v = append_offsets != nullptr ? slab_v : nullptr;
  a.append_offsets = append_offsets;
  a.slab_capacity = slab_capacity;
  a.rows = static_cast<int64_t>(batch) * len * heads;
  a.heads = heads;
  a.len = len;
  a.qkv_dtype = qkv_dtype;
  a.q_dtype = q_dtype;
  a.k_dtype = k_dtype;
  a.normalize = normalize != 0;
  a.eps = eps;
  const hipError_t e = hkv::launch_produce(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(HKV_ERR_LAUNCH, "qkv producer launch failed: %s", hipGetErrorString(e));
  return ok();
}

int32_t hkv_segmented_attention_noalloc(const void* q, const void* slab_k, const void* slab_v,
                                        const int32_t* seg_starts, const int32_t* seg_ends,
                                        const int32_t* seg_counts, const void* cur_k, const void* cur_v,
                                        void* out, float* lse, int32_t batch, int32_t heads,
                                        int32_t cur_len, int64_t slab_capacity, int32_t max_segments,
                                        int32_t head_dim, int32_t q_dtype, int32_t k_dtype,
                                        int32_t v_dtype, int32_t out_dtype, float softmax_scale,
                                        int32_t use_exp2, int32_t qk_dot_mode, int32_t value_dot_mode,
                                        const int32_t* work_plan, int32_t plan_units, void* stream) {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return fail(HKV_ERR_DEVICE, "hipGetDevice failed");
  if (device < 0 || device >= kMaxDevices)
    return fail(HKV_ERR_UNSUPPORTED, "device %d: the allocation-free entry point serves devices 0..%d", device,
                kMaxDevices - 1);
  const int32_t slots = hkv::split_slots(device);
  if (slots <= 0) return fail(HKV_ERR_DEVICE, "cannot query the CU count of device %d", device);
  const int64_t need = hkv::split_workspace_bytes(slots);
  if (need > kScratchBytes)
    return fail(HKV_ERR_UNSUPPORTED,
                "device %d has %d resident workgroup slots; the allocation-free entry point's workspace "
                "(%lld bytes) serves at most %d",
                device, slots, static_cast<long long>(kScratchBytes), kScratchSlots);
  void* ws = device_scratch(device, static_cast<hipStream_t>(stream));
  if (ws == nullptr) return fail(HKV_ERR_DEVICE, "cannot resolve the attention scratch on device %d", device);
  return hkv_segmented_attention(q, slab_k, slab_v, seg_starts, seg_ends, seg_counts, cur_k, cur_v, out, lse,
                                 batch, heads, cur_len, slab_capacity, max_segments, head_dim, q_dtype, k_dtype,
                                 v_dtype, out_dtype, softmax_scale, use_exp2, qk_dot_mode, value_dot_mode,
                                 work_plan, plan_units, ws, kScratchBytes, stream);
}

int32_t hkv_segmented_attention_plan(const int32_t* seg_starts, const int32_t* seg_ends,
                                     const int32_t* seg_counts, int32_t heads, int32_t max_segments,
                                     int64_t slab_capacity, int32_t batch, int32_t cur_len,
                                     int32_t queries_per_item, int32_t slots, int32_t* units, int32_t max_units) {
  if (heads <= 0 || heads > 1024 || batch <= 0 || cur_len <= 0)
    return fail(HKV_ERR_INVALID_ARG, "heads in [1, 1024], batch and cur_len positive (got %d, %d, %d)", heads, batch,
                cur_len);
  if (queries_per_item != 128 && queries_per_item != 256)
    return fail(HKV_ERR_INVALID_ARG, "queries_per_item must be 128 or 256 (got %d)", queries_per_item);
  if (max_segments < 0 || max_segments > hkv::kMaxSegments)
    return fail(HKV_ERR_UNSUPPORTED, "max_segments must be in [0, %d] (got %d)", hkv::kMaxSegments, max_segments);
  if (slab_capacity < 0 || slots < 0 || max_units < 0)
    return fail(HKV_ERR_INVALID_ARG, "slab_capacity, slots and max_units must be >= 0");
  if (!seg_counts || (max_segments > 0 && (!seg_starts || !seg_ends)))
    return fail(HKV_ERR_INVALID_ARG, "null table pointer");
  const int64_t items = static_cast<int64_t>(batch) * heads * ((cur_len + 127) / 128);
  if (items > 0x3fffffffLL / 2) return fail(HKV_ERR_UNSUPPORTED, "too many work items (%lld)", static_cast<long long>(items));
  const int32_t n = hkv::build_attention_plan(seg_starts, seg_ends, seg_counts, heads, max_segments, slab_capacity,
                                              batch, cur_len, queries_per_item, slots, units, max_units);
  if (n < 0) return fail(HKV_ERR_INVALID_ARG, "the plan needs more than max_units = %d units", max_units);
  ok();
  return n;
}

int32_t hkv_segmented_attention_item_shape(int32_t q_dtype, int32_t k_dtype, int32_t v_dtype, int32_t heads,
                                           int32_t qk_dot_mode, int32_t value_dot_mode, int32_t device,
                                           int32_t* slots) {
  hkv::AttnArgs a{};
  a.q_dtype = q_dtype;
  a.k_dtype = k_dtype;
  a.v_dtype = v_dtype;
  a.heads = heads;
  a.qk_dot_mode = qk_dot_mode;
  a.value_dot_mode = value_dot_mode;
  const int32_t q = hkv::attention_item_queries(a);
  if (slots != nullptr) {
    const int32_t s = hkv::split_slots(device);
    if (s <= 0) return fail(HKV_ERR_DEVICE, "cannot query the CU count of device %d", device);
    // split_slots counts 2 workgroups per CU
    *slots = hkv::attention_workgroups_per_cu(a) == 2 ? s : s / 2;
  }
  ok();
  return q;
}

int32_t hkv_split_rows(const float* src, void* dst, int64_t rows, void* stream) {
  if (rows < 0) return fail(HKV_ERR_INVALID_ARG, "rows must be >= 0 (got %lld)", static_cast<long long>(rows));
  if (rows > 0 && (!src || !dst)) return fail(HKV_ERR_INVALID_ARG, "null pointer argument");
  if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) != 0)
    return fail(HKV_ERR_INVALID_ARG, "src and dst must be 16-byte aligned");
  const hipError_t e = hkv::launch_split_rows(src, dst, rows, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(HKV_ERR_LAUNCH, "split rows launch failed: %s", hipGetErrorString(e));
  return ok();
}

int32_t hkv_segmented_attention_slots(int32_t device) {
  const int32_t s = hkv::split_slots(device);
  if (s <= 0) return fail(HKV_ERR_DEVICE, "cannot query the CU count of device %d", device);
  ok();
  return s;
}

int64_t hkv_segmented_attention_workspace_bytes(int32_t device) {
  const int64_t need = hkv::split_workspace_bytes(hkv::split_slots(device));
  if (need <= 0) return fail(HKV_ERR_DEVICE, "cannot query the CU count of device %d", device);
  ok();
  return need;
}

}  // extern "C"
