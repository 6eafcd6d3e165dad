// Slab pack / append kernel for gfx950.
//
// Semantics follow _pack_flat_segments_kv_kernel
// (real_pruning_fused_attention.py:33-73): item i copies lengths[i] rows of
// head_dim elements from src[b, src_starts[i]...] to dst[b, dst_starts[i]...]
// for K and V.  Rows of one item are consecutive in both tensors, so one
// (item, batch row) is a single contiguous byte range per tensor; the kernel
// is a batched memcpy that moves each range in 16-byte vectors when the
// pointers and row pitch allow it (128-bit loads and stores), else in 4- or
// 2-byte words.  The copy is bit-exact by construction.
//
// Work split: one workgroup of 256 threads per (item, 64-row chunk, batch
// row).  For bf16 D=128 a chunk is 16 KiB of K plus 16 KiB of V, four
// independent 16-byte loads in flight per thread per tensor.  Workgroups whose
// chunk lies beyond their item's length exit at once (append items all share
// one length, so none are idle there).
#include "hkv_internal.h"

namespace hkv {
namespace {

constexpr int kThreads = 256;
constexpr int kChunkRows = 64;
constexpr int kUnroll = 4;

struct alignas(16) U16B { uint32_t w[4]; };

template <typename U>
__device__ __forceinline__ void copy_range(char* __restrict__ dst, const char* __restrict__ src,
                                           int64_t bytes) {
  const int64_t n = bytes / static_cast<int64_t>(sizeof(U));
  U* d = reinterpret_cast<U*>(dst);
  const U* s = reinterpret_cast<const U*>(src);
  int64_t i = threadIdx.x;
  // Unrolled body: kUnroll loads issued before the stores.
  for (; i + (kUnroll - 1) * kThreads < n; i += kUnroll * kThreads) {
    U v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = s[i + u * kThreads];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) d[i + u * kThreads] = v[u];
  }
  for (; i < n; i += kThreads) d[i] = s[i];
}

template <typename UK, typename UV>
__global__ __launch_bounds__(kThreads) void pack_kernel(PackArgs a, int32_t chunks) {
  const int32_t item = blockIdx.x / chunks;
  const int32_t chunk = blockIdx.x - item * chunks;
  const int64_t b = blockIdx.y;
  // the three descriptors are read together, one memory round trip: the
  // empty asm takes all three at one point, so the compiler cannot sink two
  // of the reads past the early exit below (a second round trip)
  int64_t len = a.lengths[item];
  const int64_t src_start = a.src_starts[item];
  const int64_t dst_start = a.dst_starts[item];
  asm volatile("" : "+s"(len) : "s"(src_start), "s"(dst_start));
  if (len > a.row_limit) len = a.row_limit;
  const int64_t r0 = static_cast<int64_t>(chunk) * kChunkRows;
  if (r0 >= len) return;
  const int64_t r1 = (r0 + kChunkRows < len) ? r0 + kChunkRows : len;
  const int64_t s0 = src_start + r0;
  const int64_t d0 = dst_start + r0;
  // Clip the row range so that both the source and the destination row stay
  // inside their tensors.
  int64_t lo = 0;
  if (-s0 > lo) lo = -s0;
  if (-d0 > lo) lo = -d0;
  int64_t hi = r1 - r0;
  if (a.src_rows - s0 < hi) hi = a.src_rows - s0;
  if (a.dst_rows - d0 < hi) hi = a.dst_rows - d0;
  if (hi <= lo) return;
  const int64_t rows = hi - lo;
  const int64_t D = a.head_dim;
  const int64_t src_elem = b * a.src_batch_stride + (s0 + lo) * D;
  const int64_t dst_elem = b * a.dst_batch_stride + (d0 + lo) * D;
  copy_range<UK>(static_cast<char*>(a.dst_k) + dst_elem * a.k_elem_bytes,
                 static_cast<const char*>(a.src_k) + src_elem * a.k_elem_bytes,
                 rows * D * a.k_elem_bytes);
  copy_range<UV>(static_cast<char*>(a.dst_v) + dst_elem * a.v_elem_bytes,
                 static_cast<const char*>(a.src_v) + src_elem * a.v_elem_bytes,
                 rows * D * a.v_elem_bytes);
}

// Widest copy unit (16, 4 or 2 bytes) that keeps every access aligned.
int unit_bytes(const void* src, const void* dst, int64_t src_bs, int64_t dst_bs, int32_t D,
               int32_t esize) {
  const int cands[3] = {16, 4, 2};
  for (int u : cands) {
    if (u < esize && u != 16) continue;
    const bool ok = (reinterpret_cast<uintptr_t>(src) % u == 0) &&
                    (reinterpret_cast<uintptr_t>(dst) % u == 0) &&
                    ((static_cast<int64_t>(D) * esize) % u == 0) &&
                    ((src_bs * esize) % u == 0) && ((dst_bs * esize) % u == 0);
    if (ok) return u;
  }
  return esize;
}

template <typename UK>
hipError_t launch_v(const PackArgs& a, int uv, dim3 grid, int32_t chunks, hipStream_t st) {
  switch (uv) {
    case 16: pack_kernel<UK, U16B><<<grid, kThreads, 0, st>>>(a, chunks); break;
    case 4: pack_kernel<UK, uint32_t><<<grid, kThreads, 0, st>>>(a, chunks); break;
    default: pack_kernel<UK, uint16_t><<<grid, kThreads, 0, st>>>(a, chunks); break;
  }
  return hipGetLastError();
}

// Dense-prefix growth: out[g] = (old[g] rows, then new[g] rows) for every
// (batch, head) group g, for K and V in one launch.  blockIdx.y picks the
// range (old K, new K, old V, new V), blockIdx.z a 64 KiB chunk of it.
constexpr int64_t kConcatChunk = 64 * 1024;

template <typename U>
__global__ __launch_bounds__(kThreads) void concat_kernel(ConcatArgs a) {
  const int64_t g = blockIdx.x;
  const int part = static_cast<int>(blockIdx.y);
  const bool is_v = part >= 2;
  const bool is_new = (part & 1) != 0;
  const int64_t rb = is_v ? a.v_row_bytes : a.k_row_bytes;
  const int64_t rows = is_new ? a.t_new : a.t_old;
  const int64_t bytes = rows * rb;
  const int64_t c0 = static_cast<int64_t>(blockIdx.z) * kConcatChunk;
  if (c0 >= bytes) return;
  const int64_t n = bytes - c0 < kConcatChunk ? bytes - c0 : kConcatChunk;
  const char* src = static_cast<const char*>(is_v ? (is_new ? a.new_v : a.old_v) : (is_new ? a.new_k : a.old_k));
  char* dst = static_cast<char*>(is_v ? a.out_v : a.out_k);
  copy_range<U>(dst + g * (a.t_old + a.t_new) * rb + (is_new ? a.t_old * rb : 0) + c0, src + g * bytes + c0, n);
}

}  // namespace

hipError_t launch_concat(const ConcatArgs& a, hipStream_t stream) {
  if (a.groups <= 0 || (a.t_old + a.t_new) <= 0) return hipSuccess;
  const int64_t most = (a.t_old > a.t_new ? a.t_old : a.t_new) *
                       (a.k_row_bytes > a.v_row_bytes ? a.k_row_bytes : a.v_row_bytes);
  const int64_t chunks = (most + kConcatChunk - 1) / kConcatChunk;
  if (a.groups > 0x7fffffffLL || chunks > 65535) return hipErrorInvalidConfiguration;
  dim3 grid(static_cast<uint32_t>(a.groups), 4, static_cast<uint32_t>(chunks > 0 ? chunks : 1));
  // 16-byte units when every range start is 16-byte aligned
  const uintptr_t ptrs = reinterpret_cast<uintptr_t>(a.old_k) | reinterpret_cast<uintptr_t>(a.new_k) |
                         reinterpret_cast<uintptr_t>(a.old_v) | reinterpret_cast<uintptr_t>(a.new_v) |
                         reinterpret_cast<uintptr_t>(a.out_k) | reinterpret_cast<uintptr_t>(a.out_v);
  const bool wide = (ptrs % 16) == 0 && a.k_row_bytes % 16 == 0 && a.v_row_bytes % 16 == 0;
  if (wide) concat_kernel<U16B><<<grid, kThreads, 0, stream>>>(a);
  else concat_kernel<uint16_t><<<grid, kThreads, 0, stream>>>(a);
  return hipGetLastError();
}

hipError_t launch_pack(const PackArgs& a, hipStream_t stream) {
  if (a.n_items <= 0 || a.row_limit <= 0 || a.batch <= 0) return hipSuccess;
  const int64_t chunks64 = (static_cast<int64_t>(a.row_limit) + kChunkRows - 1) / kChunkRows;
  const int64_t blocks = chunks64 * a.n_items;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  const int32_t chunks = static_cast<int32_t>(chunks64);
  dim3 grid(static_cast<uint32_t>(blocks), static_cast<uint32_t>(a.batch), 1);
  const int uk = unit_bytes(a.src_k, a.dst_k, a.src_batch_stride, a.dst_batch_stride,
                            a.head_dim, a.k_elem_bytes);
  const int uv = unit_bytes(a.src_v, a.dst_v, a.src_batch_stride, a.dst_batch_stride,
                            a.head_dim, a.v_elem_bytes);
  switch (uk) {
    case 16: return launch_v<U16B>(a, uv, grid, chunks, stream);
    case 4: return launch_v<uint32_t>(a, uv, grid, chunks, stream);
    default: return launch_v<uint16_t>(a, uv, grid, chunks, stream);
  }
}

}  // namespace hkv
