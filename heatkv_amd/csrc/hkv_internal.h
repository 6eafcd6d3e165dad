// Internal launch interface shared by the kernel translation units and the
// C ABI in abi.hip.  Not installed; the public surface is include/heatkv.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hkv {

struct PackArgs {
  const void* src_k;
  const void* src_v;
  void* dst_k;
  void* dst_v;
  int64_t src_batch_stride;  // elements
  int64_t dst_batch_stride;  // elements
  int64_t src_rows;
  int64_t dst_rows;
  const int64_t* dst_starts;
  const int64_t* src_starts;
  const int64_t* lengths;
  int32_t batch;
  int32_t head_dim;
  int32_t k_elem_bytes;
  int32_t v_elem_bytes;
  int32_t n_items;
  int32_t row_limit;  // rows copied per item at most
};

hipError_t launch_pack(const PackArgs& a, hipStream_t stream);

// out_k[g] = (old_k[g], new_k[g]) rows, same for V, for `groups` (batch,
// head) groups of t_old and t_new rows (row sizes in bytes, even).
struct ConcatArgs {
  const void* old_k;
  const void* new_k;
  const void* old_v;
  const void* new_v;
  void* out_k;
  void* out_v;
  int64_t groups;
  int64_t t_old;
  int64_t t_new;
  int64_t k_row_bytes;
  int64_t v_row_bytes;
};

hipError_t launch_concat(const ConcatArgs& a, hipStream_t stream);

// kSplitRows: fp32 K rows stored as split rows (128 bf16 high parts, then
// 128 bf16 low parts; 512 bytes a row), the split kernel's K format.
enum Dtype : int32_t { kF16 = 1, kBF16 = 2, kF32 = 3, kSplitRows = 4 };

// Dot modes of the reference's REAL_PRUNING_FUSED_QK_DOT_MODE /
// REAL_PRUNING_FUSED_VALUE_DOT_MODE knobs (0 = default, 1 = TF32 (QK only),
// 2 = fp32 / IEEE).
enum DotMode : int32_t { kDotDefault = 0, kDotTf32 = 1, kDotFp32 = 2 };

struct AttnArgs {
  const void* q;
  const void* slab_k;
  const void* slab_v;
  const int32_t* seg_starts;
  const int32_t* seg_ends;
  const int32_t* seg_counts;
  const void* cur_k;
  const void* cur_v;
  void* out;
  float* lse;
  int64_t slab_capacity;
  int32_t batch;
  int32_t heads;
  int32_t cur_len;
  int32_t max_segments;
  float softmax_scale;
  int32_t q_dtype;
  int32_t k_dtype;
  int32_t v_dtype;
  int32_t out_dtype;        // element type of `out` (q_dtype by default)
  int32_t qk_dot_mode;      // DotMode of S = Q K^T
  int32_t value_dot_mode;   // DotMode of O = P V (kDotTf32 not used)
  void* workspace;          // round-split storage, or null
  int64_t workspace_bytes;
  const int32_t* plan;      // work plan (kPlanInts ints per unit), or null: planned in the kernel
  int32_t plan_units;
  int32_t ws_cuts;          // cut items the workspace holds (set by the launch)
  // Append of the current rows for the next scale, or null: current rows
  // [0, L) of (b, h) go to slab rows [off, off + L) of batch row b, off =
  // append_offsets[h] (-1: head h is not copied).
  const int32_t* append_offsets;
  int32_t append_first;     // first copy workgroup of a fused launch (set by the launch)
  // A second destination of the same rows, or null: slab2 rows
  // [off2, off2 + L) of batch row b, off2 = append2_offsets[h] (-1: none);
  // slab2 has the dtypes of the slab.
  const int32_t* append2_offsets;
  void* slab2_k;
  void* slab2_v;
  int64_t slab2_capacity;
};

// Work plan units (build_attention_plan): head, index in the head
// (b * n_qt + qt), key tiles [t0, t1), cut item (-1 = whole), part, 1
// when the launch's items differ in length (the 16-bit kernel then
// alternates its wave priority by tile) else 0, and 1 in cut units (the
// item's parts count in before publishing: attn::merge_parts) else 0.
constexpr int kPlanInts = 8;
int32_t build_attention_plan(const int32_t* seg_starts, const int32_t* seg_ends, const int32_t* seg_counts,
                             int32_t H, int32_t S, int64_t cap, int32_t B, int32_t L, int32_t bm, int32_t slots,
                             int32_t* out, int32_t max_units);

// The split-row kernel (seg_attn_split.hip): fp32 q, kSplitRows K, 16-bit V
// at the default dot modes; 256-query items, one workgroup per CU.
bool attention_split_supported(const AttnArgs& a);
int32_t attention_item_queries(const AttnArgs& a);
// Resident workgroups per CU of the attention kernel that runs for a (1 or 2).
int32_t attention_workgroups_per_cu(const AttnArgs& a);
hipError_t launch_split_rows(const float* src, void* dst, int64_t rows, hipStream_t stream);

constexpr int kMaxSegments = 256;

// Round split of the 16-bit attention kernel (workspace layout): kCounterBytes
// of int32 counters (one per cut item, at most one per resident workgroup
// slot, 2 slots per CU; each on a 64-byte line of its own, kCounterStride
// ints apart: the atomics of different items on one line serialize), then two
// partial records per slot of kPartialFloats floats (unnormalized O, running
// max and sum of 128 queries x 256 threads).
constexpr int kPartialFloats = 66 * 256;
constexpr int64_t kCounterBytes = 64 * 1024;
constexpr int32_t kCounterStride = 16;
constexpr int32_t kMaxCounters = static_cast<int32_t>(kCounterBytes / 4 / kCounterStride);  // 1024
int32_t split_slots(int device);  // 0 when the device cannot be queried
int64_t split_workspace_bytes(int32_t slots);

hipError_t launch_segmented_attention(const AttnArgs& a, hipStream_t stream);

struct ProduceArgs {
  const void* qkv;            // [B, L, 3, H, D] of qkv_dtype, token stride in elements
  int64_t token_stride;
  const float* q_bias;        // [H * D] or null
  const float* v_bias;        // [H * D] or null
  const float* scale_mul;     // [H] or null
  const float* rope;          // [2, rope_rows, D / 2] (cos, sin) or null
  int64_t rope_rows;
  int64_t rope_start;         // table row of token 0
  void* q_out;                // [B, H, L, D], q_dtype
  void* k_out;                // [B, H, L, D], k_dtype
  void* v_out;                // [B, H, L, D], qkv_dtype
  void* slab_k;               // [B, slab_capacity, D], k_dtype (append) or null
  void* slab_v;               // [B, slab_capacity, D], qkv_dtype
  const int32_t* append_offsets;  // [H], -1 = head not appended; null = no append
  int64_t slab_capacity;
  int64_t rows;               // B * L * H
  int32_t heads;
  int32_t len;
  int32_t qkv_dtype;          // the projection's element type, also v's
  int32_t q_dtype;
  int32_t k_dtype;
  int32_t normalize;
  float eps;
};

hipError_t launch_produce(const ProduceArgs& a, hipStream_t stream);

}  // namespace hkv
