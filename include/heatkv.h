/*
 * heatkv.h -- C ABI of libheatkv.so, the MI355X (gfx950) kernels behind the
 * HeatKV slab-compaction + segmented-attention path.
 *
 * Plain pointers and sizes only.  Every device pointer is a HIP device
 * address; `stream` is a hipStream_t passed as void* (NULL = null stream).
 * All calls are asynchronous on `stream`, allocate nothing, and return
 * HKV_OK (0) or a negative HKV_ERR_* code; hkv_last_error() then holds a
 * message for the calling thread.
 */
#ifndef HEATKV_H
#define HEATKV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HKV_OK 0
#define HKV_ERR_INVALID_ARG (-1)  /* maps to ValueError in the Python layer */
#define HKV_ERR_UNSUPPORTED (-2)  /* maps to RuntimeError (dtype / head_dim / sizes) */
#define HKV_ERR_LAUNCH (-3)       /* kernel launch failed (RuntimeError) */
#define HKV_ERR_DEVICE (-4)       /* no gfx950 device / runtime failure (RuntimeError) */

/* Element types (match torch.float16 / torch.bfloat16 / torch.float32). */
#define HKV_DTYPE_F16 1
#define HKV_DTYPE_BF16 2
#define HKV_DTYPE_F32 3
/* K only: fp32 rows stored as split rows, 128 bf16 high parts then 128 bf16
 * low parts per row (hi = x rounded to bf16, lo = (x - hi) rounded to bf16;
 * 512 bytes a row, written by hkv_split_rows).  With float32 q, 16-bit v and
 * the default (or tf32) dot modes the attention then runs its split-row
 * kernel.  No counterpart in the reference. */
#define HKV_DTYPE_SPLIT_ROWS 4

/*
 * Dense-prefix growth of the segmented cache in one launch: for each of
 * `groups` (batch, head) groups, out_k[g] = old_k[g] (t_old rows) followed by
 * new_k[g] (t_new rows), and the same for V; rows of k_row_bytes /
 * v_row_bytes bytes, every tensor contiguous ([groups, rows, ...]).  What
 * torch.cat((old_k, new_k), dim=2) and the same for V give, as one kernel.
 * Replaces the two concatenations of the reference's dense prefix
 * (enable_real_pruning_fast.py:1972-2038).
 */
int32_t hkv_concat_kv(const void* old_k, const void* new_k, const void* old_v, const void* new_v, void* out_k,
                      void* out_v, int64_t groups, int64_t t_old, int64_t t_new, int64_t k_row_bytes,
                      int64_t v_row_bytes, void* stream);

/* Library version, (major << 16) | (minor << 8) | patch: HKV_VERSION of the
 * header the library was built with.  A loader compares it with the version
 * of the header (or bindings) it was written against and refuses a mismatch. */
#define HKV_VERSION ((0 << 16) | (3 << 8) | 0)
int32_t hkv_version(void);

/* 1 when `device` is a gfx950 GPU this build can run on, else 0.
 * Loader check; the reference probes Triton/CUDA availability instead
 * (real_pruning_fused_attention.py:393-396, 522-525). */
int32_t hkv_device_ok(int32_t device);

/* Message for the last failing call on this thread ("" when none). */
const char* hkv_last_error(void);

/*
 * Slab pack / append: for every item i < n_items and batch row b < batch
 *   dst_k[b, dst_starts[i] + t, :] = src_k[b, src_starts[i] + t, :]
 *   dst_v[b, dst_starts[i] + t, :] = src_v[b, src_starts[i] + t, :]
 * for t < lengths[i]; rows outside the items are not written.
 *
 * Replaces pack_flat_segments_kv / _pack_flat_segments_kv_kernel
 * (real_pruning_fused_attention.py:365-441, 33-73).
 *   src_*  : [batch, *, head_dim] rows, batch stride src_batch_stride elements
 *   dst_*  : [batch, *, head_dim] rows, batch stride dst_batch_stride elements
 *   k_elem_bytes / v_elem_bytes : 2 or 4 (K and V may differ, e.g. fp32 K)
 *   dst_starts, src_starts, lengths : int64 device arrays of n_items
 *   src_rows / dst_rows : rows per batch of src / dst; a row outside
 *                [0, rows) is skipped (the reference's kernel does not check;
 *                this keeps bad descriptors from writing outside the slab)
 *   max_length : rows copied per item at most.  The reference's grid covers
 *                ceil(max_length / block_t) tiles of block_t rows, so its
 *                Python wrapper passes block_t * ceil(max_length / block_t).
 * head_dim <= 128 as in the reference (:415-416).
 */
int32_t hkv_pack_segments(const void* src_k, const void* src_v, void* dst_k, void* dst_v,
                          int64_t src_batch_stride, int64_t dst_batch_stride,
                          int64_t src_rows, int64_t dst_rows,
                          int32_t batch, int32_t head_dim,
                          int32_t k_elem_bytes, int32_t v_elem_bytes,
                          const int64_t* dst_starts, const int64_t* src_starts,
                          const int64_t* lengths, int32_t n_items, int32_t max_length,
                          void* stream);

/*
 * Segmented attention over a flat slab plus the current scale:
 *   out[b, l, h*D:(h+1)*D] = softmax(scale * q[b,h,l] . K_bh^T) V_bh
 * where K_bh = slab_k[b, starts[h,i]:ends[h,i]] for i < counts[h] (entries
 * with start >= end skipped), then cur_k[b, h]; V_bh likewise.
 *
 * Replaces fused_real_pruning_flat_segmented_attention /
 * _fused_real_pruning_segmented_attention_kernel
 * (real_pruning_fused_attention.py:445-591, 76-267).
 *   q, cur_k, cur_v : [batch, heads, cur_len, head_dim] contiguous
 *   slab_k, slab_v  : [batch, slab_capacity, head_dim] contiguous
 *   seg_starts, seg_ends : int32 [heads, max_segments]; seg_counts : int32 [heads]
 *   out  : [batch, cur_len, heads*head_dim] of out_dtype (0 = q_dtype, as in
 *          the reference; bf16 / fp16 store the fp32 result rounded to
 *          nearest even, what a later cast of an fp32 output would give)
 *   lse  : NULL, or float32 [batch, heads, cur_len] natural-log log-sum-exp
 *          of the scaled scores (not produced by the reference kernel)
 *   *_dtype : HKV_DTYPE_*; slab and current K share k_dtype, V share v_dtype;
 *              k_dtype HKV_DTYPE_SPLIT_ROWS needs q float32, v 16-bit and
 *              dot modes other than 2 (its rows are 512 bytes: slab_k is
 *              [batch, slab_capacity, 256] and cur_k [batch, heads, cur_len,
 *              256] of bf16); the work plan's items are then 256 queries
 *              (hkv_segmented_attention_item_shape)
 *   use_exp2 : the reference's softmax_mode ("exp" = 0, "exp2" = 1); both give
 *              the same mathematical result and this kernel always evaluates
 *              exp2 with scale*log2(e) folded in.
 *   qk_dot_mode : the reference's QK_DOT_MODE constexpr (:141-153, knob
 *              REAL_PRUNING_FUSED_QK_DOT_MODE, :298-308): 0 bf16, 1 tf32,
 *              2 fp32 (IEEE).  16-bit q/k products are exact in every mode;
 *              fp32 q/k are split into 2 bf16 pieces in modes 0 and 1 (~16
 *              significand bits, beyond TF32's 11) and 3 in mode 2 (fp32's 24).
 *   value_dot_mode : the reference's VALUE_DOT_MODE (:176-184, knob
 *              REAL_PRUNING_FUSED_VALUE_DOT_MODE, :286-295): 0 = P rounded to
 *              V's type (fp32 V: P and V in 2 bf16 pieces, beyond the
 *              reference's TF32 dot), 2 = an fp32 P V product (P in 3 pieces,
 *              V in as many as its type needs).
 *   work_plan, plan_units : NULL / 0 (the kernel orders its work from the
 *              tables itself), or a device copy of the plan that
 *              hkv_segmented_attention_plan built from host copies of these
 *              same tables, batch and cur_len: one workgroup per unit, no
 *              planning in the kernel (both kernels; a cut item's parts are
 *              merged through the workspace, so cuts need one).  A plan for
 *              other tables gives wrong results but stays inside the tensors.
 *   workspace, workspace_bytes : NULL / 0, or device memory of at least
 *              hkv_segmented_attention_workspace_bytes(device) bytes whose
 *              first 64 KiB (per-item counters) are zero before its first
 *              use (the calls leave them zero again; the rest is scratch).
 *              With it and no plan, for 16-bit inputs, a launch with fewer
 *              than two rounds of (batch, head, 128-query tile) items per resident
 *              workgroup slot (2 per CU) cuts some items into two halves of
 *              their key stream, merged through the workspace, so it fills
 *              whole rounds; without it every item is one workgroup.  Results
 *              agree to rounding; each mode is deterministic.  Calls that may
 *              run concurrently need separate workspaces.  No counterpart in
 *              the reference (its Triton grid is one program per item).
 * head_dim must be 128 and cur_len > 0 (:526-529).  Segment bounds are
 * clamped to [0, slab_capacity) and counts to [0, max_segments], so bad
 * tables cannot address outside the slab.  max_segments <= 256.
 */
int32_t hkv_segmented_attention(const void* q, const void* slab_k, const void* slab_v,
                                const int32_t* seg_starts, const int32_t* seg_ends,
                                const int32_t* seg_counts, const void* cur_k,
                                const void* cur_v, void* out, float* lse,
                                int32_t batch, int32_t heads, int32_t cur_len,
                                int64_t slab_capacity, int32_t max_segments, int32_t head_dim,
                                int32_t q_dtype, int32_t k_dtype, int32_t v_dtype,
                                int32_t out_dtype, float softmax_scale, int32_t use_exp2,
                                int32_t qk_dot_mode, int32_t value_dot_mode,
                                const int32_t* work_plan, int32_t plan_units,
                                void* workspace, int64_t workspace_bytes, void* stream);

/*
 * hkv_segmented_attention followed by the append of the current rows for
 * the next scale, in one launch with the 16-bit kernel (its copy workgroups
 * follow the attention workgroups) and in a second launch on `stream`
 * otherwise.  Replaces the attention call plus the static append of the
 * kept heads' current rows that follows it (enable_real_pruning_fast.py:
 * 1791-1807 -> 969-995) when every destination row lies outside the segments
 * this call reads.
 *   append_offsets : int32 [heads] on the device: current rows [0, cur_len)
 *                    of (b, h) are written to slab rows [off, off + cur_len)
 *                    of batch row b, off = append_offsets[h]; heads with
 *                    off < 0 or off + cur_len > slab_capacity are not
 *                    copied.  The rows written must not lie in any segment
 *                    of seg_starts / seg_ends (then the results are those of
 *                    the two calls in order; otherwise undefined).  NULL:
 *                    the call is hkv_segmented_attention.
 * The slab and current tensors must be 16-byte aligned and slab_capacity >=
 * cur_len.  Other arguments and results as hkv_segmented_attention.
 */
int32_t hkv_segmented_attention_append(const void* q, void* slab_k, void* slab_v,
                                       const int32_t* seg_starts, const int32_t* seg_ends,
                                       const int32_t* seg_counts, const void* cur_k,
                                       const void* cur_v, void* out, float* lse,
                                       int32_t batch, int32_t heads, int32_t cur_len,
                                       int64_t slab_capacity, int32_t max_segments, int32_t head_dim,
                                       int32_t q_dtype, int32_t k_dtype, int32_t v_dtype,
                                       int32_t out_dtype, float softmax_scale, int32_t use_exp2,
                                       int32_t qk_dot_mode, int32_t value_dot_mode,
                                       const int32_t* work_plan, int32_t plan_units,
                                       void* workspace, int64_t workspace_bytes,
                                       const int32_t* append_offsets, void* stream);

/*
 * hkv_segmented_attention_append whose copy also writes the same rows to a
 * second slab: current rows [0, cur_len) of (b, h) go to rows
 * [off, off + cur_len) of batch row b of slab2_k / slab2_v ([B,
 * slab2_capacity, D], the dtypes of slab_k / slab_v), off =
 * append2_offsets[h] (-1: not written), read once for both destinations.
 * Needs append_offsets; slab2 16-byte aligned, slab2_capacity >= cur_len, and
 * its written rows outside every row the launch reads.  No reference
 * counterpart: a dense-prefix step (enable_real_pruning_fast.py:1972-2038)
 * keeps its rows in the dense cache for the next dense step and puts them in
 * the slab of the first pruned target at once, so that target's activation
 * pack (:1639-1711) has nothing left to copy.
 */
int32_t hkv_segmented_attention_append2(const void* q, void* slab_k, void* slab_v,
                                        const int32_t* seg_starts, const int32_t* seg_ends,
                                        const int32_t* seg_counts, const void* cur_k,
                                        const void* cur_v, void* out, float* lse,
                                        int32_t batch, int32_t heads, int32_t cur_len,
                                        int64_t slab_capacity, int32_t max_segments, int32_t head_dim,
                                        int32_t q_dtype, int32_t k_dtype, int32_t v_dtype,
                                        int32_t out_dtype, float softmax_scale, int32_t use_exp2,
                                        int32_t qk_dot_mode, int32_t value_dot_mode,
                                        const int32_t* work_plan, int32_t plan_units,
                                        void* workspace, int64_t workspace_bytes,
                                        const int32_t* append_offsets, void* slab2_k, void* slab2_v,
                                        int64_t slab2_capacity, const int32_t* append2_offsets, void* stream);

/* A bound attention call: hkv_segmented_attention_append's arguments other
 * than the tensors (tables, shapes, dtypes, scale, dot modes, work plan,
 * workspace and append offsets) validated once into a caller-owned block of
 * hkv_segmented_attention_bound_bytes() bytes (8-byte aligned), on the
 * current device; hkv_segmented_attention_call then launches with new q,
 * slab K/V, current K/V and output pointers only (no LSE), on `stream`, with
 * that device current.  The tables, plan, workspace and offsets must stay
 * valid and unchanged while the block is used; the caller guarantees that the
 * new tensors have the bound shapes and dtypes (the kernels index them by
 * those).  No reference counterpart: for callers that repeat one call shape
 * many times, such as a cache's per-(layer, scale) steps, whose host cost per
 * launch then drops to the launch itself (the reference re-validates in
 * Python on every call, real_pruning_fused_attention.py:445-560). */
int64_t hkv_segmented_attention_bound_bytes(void);
int32_t hkv_segmented_attention_bind(void* bound, int64_t bound_bytes, const int32_t* seg_starts,
                                     const int32_t* seg_ends, const int32_t* seg_counts, int32_t batch,
                                     int32_t heads, int32_t cur_len, int64_t slab_capacity, int32_t max_segments,
                                     int32_t head_dim, int32_t q_dtype, int32_t k_dtype, int32_t v_dtype,
                                     int32_t out_dtype, float softmax_scale, int32_t use_exp2, int32_t qk_dot_mode,
                                     int32_t value_dot_mode, const int32_t* work_plan, int32_t plan_units,
                                     void* workspace, int64_t workspace_bytes, const int32_t* append_offsets);
/* hkv_segmented_attention_bind with hkv_segmented_attention_append2's second
 * destination, bound with the rest: slab2_k / slab2_v stay the same tensors
 * for every call of the block. */
int32_t hkv_segmented_attention_bind2(void* bound, int64_t bound_bytes, const int32_t* seg_starts,
                                      const int32_t* seg_ends, const int32_t* seg_counts, int32_t batch,
                                      int32_t heads, int32_t cur_len, int64_t slab_capacity, int32_t max_segments,
                                      int32_t head_dim, int32_t q_dtype, int32_t k_dtype, int32_t v_dtype,
                                      int32_t out_dtype, float softmax_scale, int32_t use_exp2,
                                      int32_t qk_dot_mode, int32_t value_dot_mode, const int32_t* work_plan,
                                      int32_t plan_units, void* workspace, int64_t workspace_bytes,
                                      const int32_t* append_offsets, void* slab2_k, void* slab2_v,
                                      int64_t slab2_capacity, const int32_t* append2_offsets);
int32_t hkv_segmented_attention_call(const void* bound, const void* q, void* slab_k, void* slab_v,
                                     const void* cur_k, const void* cur_v, void* out, void* stream);

/*
 * Work plan of hkv_segmented_attention for host copies of its offset tables
 * (int32 seg_starts / seg_ends [heads, max_segments], seg_counts [heads]),
 * batch and cur_len, for items of `queries_per_item` queries (128, or 256
 * for split K rows) and a device with `slots` resident attention workgroups
 * (hkv_segmented_attention_item_shape; 0 = cut nothing): writes plan units of 8
 * int32 each into `units` (host memory, room for max_units) and returns
 * their count, or only the count when `units` is NULL; a negative HKV_ERR_*
 * code on bad arguments.  Items (batch row, head, 128-query tile) are ordered
 * heaviest head first; when a launch has under four rounds of items per
 * slot, the heaviest items may be cut into two key-range parts chosen by
 * simulating the dispatch, and with at least two rounds the items are dealt
 * to the 8 XCDs (workgroup id % 8) in chunks of a (batch row, head)'s query
 * tiles, each XCD's list padded to equal length with empty units (head -1,
 * the workgroup leaves at once).  Unit: head, batch row * n_qt + query tile,
 * first and end key tile, cut index (-1 = whole item), part (0 or 1), a flag
 * (1 when the items' key tile counts differ by more than 5/4: the 16-bit
 * kernel then alternates its wave priority by tile so the two workgroups of a
 * CU share its SIMDs evenly; 0 otherwise and in empty units), and a flag (1
 * in every cut unit: the item's two parts count in before the first to
 * arrive publishes its partial result, and the second merges without
 * publishing its own; 0 in whole and empty units; a plan may also carry 0 in
 * cut units, whose parts then both publish and the last to count in merges).
 * Host-only: no device call.  No counterpart in the reference (its tables
 * are the whole plan: the Triton grid walks them).
 */
int32_t hkv_segmented_attention_plan(const int32_t* seg_starts, const int32_t* seg_ends,
                                     const int32_t* seg_counts, int32_t heads, int32_t max_segments,
                                     int64_t slab_capacity, int32_t batch, int32_t cur_len,
                                     int32_t queries_per_item, int32_t slots, int32_t* units, int32_t max_units);

/*
 * Item shape of hkv_segmented_attention for these dtypes and dot modes:
 * returns the queries per work item (128, or 256 for split K rows), and
 * writes the device's resident attention workgroups for the kernel that runs
 * (2 per CU for the 16-bit kernel and the staged kernel's plain modes, 1 per
 * CU for split K rows and for the staged kernel's fp32 QK dot mode on fp32 q,
 * fp32 value dot mode and fp32 V) to *slots when slots is not NULL (the
 * `queries_per_item` and `slots` of hkv_segmented_attention_plan); a negative
 * HKV_ERR_* code when the device cannot be queried.  No counterpart in the
 * reference.
 */
int32_t hkv_segmented_attention_item_shape(int32_t q_dtype, int32_t k_dtype, int32_t v_dtype, int32_t heads,
                                           int32_t qk_dot_mode, int32_t value_dot_mode, int32_t device,
                                           int32_t* slots);

/*
 * fp32 rows (`rows` x 128 contiguous, 16-byte aligned) to split rows at dst
 * (`rows` x 512 bytes, see HKV_DTYPE_SPLIT_ROWS), enqueued on `stream`.  No
 * counterpart in the reference: its Triton dot takes fp32 K as it is.
 */
int32_t hkv_split_rows(const float* src, void* dst, int64_t rows, void* stream);

/* Resident attention workgroups of `device` (2 per CU), the `slots` of
 * hkv_segmented_attention_plan; a negative HKV_ERR_* code when the device
 * cannot be queried.  No counterpart in the reference. */
int32_t hkv_segmented_attention_slots(int32_t device);

/*
 * Bytes of the hkv_segmented_attention workspace for `device` (64 KiB of
 * counters plus 2 partial records of 66 KiB per resident workgroup slot,
 * 2 slots per CU: about 69 MB on a 256-CU device); a negative HKV_ERR_*
 * code when the device cannot be queried.  No counterpart in the reference.
 */
int64_t hkv_segmented_attention_workspace_bytes(int32_t device);

/*
 * hkv_segmented_attention with its workspace taken from a static device
 * array of this library instead of the caller: the entry point allocates
 * nothing (no hipMalloc, hipFree or allocating library routine), for callers
 * that cannot allocate -- code under HIP graph capture, serving loops and
 * harnesses that forbid allocation.  No counterpart in the reference.
 * Arguments and results as hkv_segmented_attention (the workspace arguments
 * are absent).  The array holds the round split's counters and partial
 * records for up to 512 resident workgroup slots (a 256-CU device): 69.3 MB
 * per GPU the library runs on, held until the process ends; a device with
 * more slots is rejected (HKV_ERR_UNSUPPORTED).  Every call on one GPU shares
 * that GPU's array, so calls that may overlap on one GPU (other streams,
 * other host threads) race; calls in order on one stream do not.
 */
int32_t hkv_segmented_attention_noalloc(const void* q, const void* slab_k, const void* slab_v,
                                        const int32_t* seg_starts, const int32_t* seg_ends,
                                        const int32_t* seg_counts, const void* cur_k, const void* cur_v,
                                        void* out, float* lse, int32_t batch, int32_t heads,
                                        int32_t cur_len, int64_t slab_capacity, int32_t max_segments,
                                        int32_t head_dim, int32_t q_dtype, int32_t k_dtype,
                                        int32_t v_dtype, int32_t out_dtype, float softmax_scale,
                                        int32_t use_exp2, int32_t qk_dot_mode, int32_t value_dot_mode,
                                        const int32_t* work_plan, int32_t plan_units, void* stream);

/*
 * QKV producer epilogue of one scale: from the QKV projection output to the
 * attention-ready q, k, v, for every (b, l, h):
 *   x_q, x_k, x_v = qkv[b, l, 0|1|2, h, :] (+ q_bias / v_bias[h*D:(h+1)*D])
 *   if normalize: x_q /= max(||x_q||, eps); x_k /= max(||x_k||, eps)   (fp32)
 *   if scale_mul: x_q *= scale_mul[h]
 *   if rope: pairs (2i, 2i+1) of x_q and x_k rotated with
 *            c = rope[0, rope_start + l, i], s = rope[1, rope_start + l, i]:
 *            (c*x0 - s*x1, s*x0 + c*x1), each product and sum rounded
 *   q_out, k_out, v_out[b, h, l, :] = x_q, x_k, x_v
 *   if append_offsets and append_offsets[h] >= 0 (and the row fits):
 *     slab_k, slab_v[b, append_offsets[h] + l, :] = x_k, x_v
 *
 * Replaces the prologue of the reference layer forward under bf16 autocast
 * (enable_real_pruning_fast.py:2040-2072: qkv view/unbind/permute, cosine
 * attention normalize and scale_mul; apply_rotary_emb,
 * infinity/models/basic.py:97-117) and, with append_offsets, the append of
 * the kept heads' current rows into the slab that the reference runs after
 * attention (enable_real_pruning_fast.py:969-995, 1791-1807).  The append may
 * only be fused when no slab row it writes is read by this scale's attention.
 *   qkv : [batch, len, 3, heads, 128] of qkv_dtype (bf16 under the
 *         reference's bf16 autocast; fp16 under fp16 autocast; fp32 without
 *         autocast) with token stride token_stride elements (>= 3 * heads *
 *         128, multiple of 8)
 *   q_bias, v_bias : NULL or float32 [heads * 128]; added in fp32 to the
 *         projection output (the reference adds them before the GEMM output
 *         is rounded to the projection's type)
 *   scale_mul : NULL or float32 [heads] (the exp of the clamped learned scale)
 *   rope : NULL or float32 [2, rope_rows, 64] (cos table, then sin table);
 *          rows [rope_start, rope_start + len) are used
 *   q_out, k_out : [batch, heads, len, 128] of q_dtype == k_dtype: float32
 *          (the reference's values under autocast), float16 (the same
 *          11-bit significand as the TF32 products the reference's attention
 *          takes of fp32 q/k; elements beyond +-65504 become inf) or bfloat16;
 *          or float32 q with k_dtype HKV_DTYPE_SPLIT_ROWS: each k row as the
 *          split row hkv_split_rows writes of the float32 row (512 bytes), the
 *          K format of the split-row attention kernel, so attention calls on
 *          these rows need no split of their own
 *   v_out : [batch, heads, len, 128] of v_dtype == qkv_dtype (the
 *          projection's values; with v_bias, rounded once to that type)
 *   slab_k / slab_v : [batch, slab_capacity, 128] of k_dtype / v_dtype
 *          (split rows: 512-byte rows)
 *   append_offsets : NULL or int32 [heads] (-1 = head not appended)
 * All pointers 16-byte aligned.  Rows (b, l, h) with append_offsets[h] + l
 * outside [0, slab_capacity) are not appended.
 */
int32_t hkv_qkv_produce(const void* qkv, int64_t token_stride, const float* q_bias,
                        const float* v_bias, const float* scale_mul, const float* rope,
                        int64_t rope_rows, int64_t rope_start, void* q_out, void* k_out,
                        void* v_out, void* slab_k, void* slab_v, const int32_t* append_offsets,
                        int64_t slab_capacity, int32_t batch, int32_t heads, int32_t len,
                        int32_t head_dim, int32_t qkv_dtype, int32_t q_dtype, int32_t k_dtype,
                        int32_t v_dtype, int32_t normalize, float eps, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HEATKV_H */
