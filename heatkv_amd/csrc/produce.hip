// Producer epilogue for gfx950: QKV projection output -> attention-ready
// q, k, v of one scale, with the optional append of the kept heads' K/V rows
// into the slab.
//
// Semantics follow the reference layer's prologue under bf16 autocast
// (enable_real_pruning_fast.py:2040-2072, infinity/models/basic.py:97-117):
//   qkv = linear(x) viewed [B, L, 3, H, D] (bf16)
//   q = normalize(q) * scale_mul[h];  k = normalize(k)     (fp32: the norm
//       runs in fp32 under autocast, so the quotient is fp32)
//   (q, k) = rotate pairs (2i, 2i+1) by the 2-D RoPE table row of each token:
//       x'[2i]   = cos * x[2i] - sin * x[2i+1]
//       x'[2i+1] = sin * x[2i] + cos * x[2i+1]   (each product and sum rounded
//       on its own, as the reference's elementwise tensor ops do)
//   q, k, v permuted to [B, H, L, D].
// normalize(x) = x / max(||x||_2, eps); the division is IEEE fp32.  The squared
// norm is summed in a different order than torch's reduction, so q and k
// agree with the reference to a few fp32 ulp, not bit for bit.
//
// Fused bias (optional): the reference adds q_bias / v_bias inside the GEMM,
// before the bf16 rounding of its output; here they are added in fp32 to the
// rounded GEMM output (a caller that needs the reference's rounding runs the
// GEMM with the bias and passes none here).
//
// Fused append (optional): rows (b, l, h) of heads with append_offsets[h] >= 0
// are also written to slab_k / slab_v[b, append_offsets[h] + l] -- the append
// of the current scale's kept heads that the reference runs after attention
// (:969-995, :2176-2253).  The caller may fuse it only when those slab rows
// are not read by the attention of this scale.
//
// Work split: 16 lanes per (b, l, h) row, 8 elements (16 bytes of bf16) per
// lane per tensor; rows in (b, l, h) order, so the 16 rows of a 256-thread
// workgroup read one token's contiguous q, k and v blocks and each row writes
// whole 512-byte (fp32) or 256-byte (bf16) output rows.  Pure streaming:
// 768 bytes read and 1280 bytes written per row with fp32 q/k (HBM bound).
#include "hkv_internal.h"

namespace hkv {
namespace {

constexpr int kThreads = 256;
constexpr int kLanes = 16;            // lanes per row
constexpr int kRowsPerBlock = kThreads / kLanes;
constexpr int kD = 128;
constexpr int kPer = kD / kLanes;     // elements per lane

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void unpack_bf16x8(u32x4_t w, float (&x)[kPer]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = __uint_as_float(w[i] << 16);
    x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

// Round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Round to nearest even; out-of-range values become +-inf.
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
}

template <int DT>
__device__ __forceinline__ void store_row8(void* base, int64_t elem, const float (&x)[kPer]) {
  if constexpr (DT == kSplitRows) {
    // split row (hkv_split_rows' format, 512 bytes like an fp32 row): the
    // 128 bf16 high parts hi = bf16(x), then the 128 low parts bf16(x - hi)
    u32x4_t hi, lo;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      hi[k] = pack_bf16x2(x[2 * k], x[2 * k + 1]);
      const float h0 = __builtin_bit_cast(float, hi[k] << 16);
      const float h1 = __builtin_bit_cast(float, hi[k] & 0xffff0000u);
      lo[k] = pack_bf16x2(x[2 * k] - h0, x[2 * k + 1] - h1);
    }
    uint8_t* const row = static_cast<uint8_t*>(base) + (elem / kD) * (kD * 4) + (elem % kD) * 2;
    *reinterpret_cast<u32x4_t*>(row) = hi;
    *reinterpret_cast<u32x4_t*>(row + kD * 2) = lo;
  } else if constexpr (DT == kF32) {
    f32x4_t* p = reinterpret_cast<f32x4_t*>(static_cast<float*>(base) + elem);
    p[0] = f32x4_t{x[0], x[1], x[2], x[3]};
    p[1] = f32x4_t{x[4], x[5], x[6], x[7]};
  } else if constexpr (DT == kF16) {
    u32x4_t w = {pack_f16x2(x[0], x[1]), pack_f16x2(x[2], x[3]), pack_f16x2(x[4], x[5]),
                 pack_f16x2(x[6], x[7])};
    *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(base) + elem) = w;
  } else {
    u32x4_t w = {pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]), pack_bf16x2(x[4], x[5]),
                 pack_bf16x2(x[6], x[7])};
    *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(base) + elem) = w;
  }
}

__device__ __forceinline__ void add_bias(float (&x)[kPer], const float* __restrict__ bias) {
  const f32x4_t b0 = reinterpret_cast<const f32x4_t*>(bias)[0];
  const f32x4_t b1 = reinterpret_cast<const f32x4_t*>(bias)[1];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[i] += b0[i];
    x[4 + i] += b1[i];
  }
}

// Sum over the 16 lanes of a row (lane groups are 16-aligned inside the wave).
__device__ __forceinline__ float row_sum(float v) {
#pragma unroll
  for (int m = kLanes / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kLanes);
  return v;
}

__device__ __forceinline__ void normalize(float (&x)[kPer], float eps) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) ss = fmaf(x[i], x[i], ss);
  float n = sqrtf(row_sum(ss));
  n = n < eps ? eps : n;  // clamp_min; a NaN norm stays NaN
#pragma unroll
  for (int i = 0; i < kPer; ++i) x[i] = x[i] / n;
}

// Pair rotation with separately rounded products and sums (no FMA).
__device__ __forceinline__ void rotate(float (&x)[kPer], f32x4_t c, f32x4_t s) {
#pragma clang fp contract(off)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float x0 = x[2 * i];
    const float x1 = x[2 * i + 1];
    const float a = c[i] * x0;
    const float b = s[i] * x1;
    const float d = s[i] * x0;
    const float e = c[i] * x1;
    x[2 * i] = a - b;
    x[2 * i + 1] = d + e;
  }
}

// 8 elements of the projection (element type IT) at `p` as floats; the raw
// bytes (16 for 16-bit types, 32 for fp32) in `raw` for a copy that keeps them.
template <int IT>
__device__ __forceinline__ void load_row8(const uint8_t* p, float (&x)[kPer], u32x4_t (&raw)[2]) {
  raw[0] = *reinterpret_cast<const u32x4_t*>(p);
  if constexpr (IT == kF32) {
    raw[1] = *reinterpret_cast<const u32x4_t*>(p + 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = __uint_as_float(raw[0][i]);
      x[4 + i] = __uint_as_float(raw[1][i]);
    }
  } else if constexpr (IT == kF16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(raw[0][i] & 0xffffu)));
      x[2 * i + 1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(raw[0][i] >> 16)));
    }
  } else {
    unpack_bf16x8(raw[0], x);
  }
}

template <int IT>
__device__ __forceinline__ void store_raw8(void* base, int64_t elem, const u32x4_t (&raw)[2]) {
  if constexpr (IT == kF32) {
    u32x4_t* p = reinterpret_cast<u32x4_t*>(static_cast<float*>(base) + elem);
    p[0] = raw[0];
    p[1] = raw[1];
  } else {
    *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(base) + elem) = raw[0];
  }
}

// IT: the projection's element type (bf16, fp16 or fp32), also v's; QT, KT:
// the q and k outputs' (KT kSplitRows: k as split rows).
template <int IT, int QT, int KT = QT>
__global__ __launch_bounds__(kThreads) void produce_kernel(ProduceArgs a) {
  constexpr int kElem = IT == kF32 ? 4 : 2;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / kLanes;
  const int j = threadIdx.x % kLanes;
  // Whole 16-lane rows leave together, so the row reductions stay complete.
  if (row >= a.rows) return;
  const int32_t h = static_cast<int32_t>(row % a.heads);
  const int64_t tok = row / a.heads;  // b * len + l
  const int32_t l = static_cast<int32_t>(tok % a.len);
  const int64_t b = tok / a.len;
  const int64_t hd = static_cast<int64_t>(a.heads) * kD;

  const uint8_t* src = static_cast<const uint8_t*>(a.qkv) +
                       (tok * a.token_stride + static_cast<int64_t>(h) * kD + j * kPer) * kElem;
  float q[kPer], k[kPer], v[kPer];
  u32x4_t rq[2], rk[2], rv[2];
  load_row8<IT>(src, q, rq);
  load_row8<IT>(src + hd * kElem, k, rk);
  load_row8<IT>(src + 2 * hd * kElem, v, rv);
  f32x4_t rc = {1.f, 1.f, 1.f, 1.f}, rs = {0.f, 0.f, 0.f, 0.f};
  if (a.rope != nullptr) {
    const int64_t pos = a.rope_start + l;
    rc = *reinterpret_cast<const f32x4_t*>(a.rope + pos * (kD / 2) + j * 4);
    rs = *reinterpret_cast<const f32x4_t*>(a.rope + (a.rope_rows + pos) * (kD / 2) + j * 4);
  }

  const int64_t bias_off = static_cast<int64_t>(h) * kD + j * kPer;
  if (a.q_bias != nullptr) add_bias(q, a.q_bias + bias_off);
  if (a.normalize) {
    normalize(q, a.eps);
    normalize(k, a.eps);
  }
  if (a.scale_mul != nullptr) {
    const float m = a.scale_mul[h];
#pragma unroll
    for (int i = 0; i < kPer; ++i) q[i] = q[i] * m;
  }
  if (a.rope != nullptr) {
    rotate(q, rc, rs);
    rotate(k, rc, rs);
  }

  const int64_t orow = ((b * a.heads + h) * a.len + l) * kD + j * kPer;
  store_row8<QT>(a.q_out, orow, q);
  store_row8<KT>(a.k_out, orow, k);
  // v keeps the projection's values and type (the bias, when given, added in
  // fp32 and rounded to that type once)
  if (a.v_bias != nullptr) {
    add_bias(v, a.v_bias + bias_off);
    store_row8<IT>(a.v_out, orow, v);
  } else {
    store_raw8<IT>(a.v_out, orow, rv);
  }

  if (a.append_offsets != nullptr) {
    const int32_t off = a.append_offsets[h];
    if (off >= 0 && static_cast<int64_t>(off) + l < a.slab_capacity) {
      const int64_t srow = (b * a.slab_capacity + off + l) * kD + j * kPer;
      store_row8<KT>(a.slab_k, srow, k);
      if (a.v_bias != nullptr) store_row8<IT>(a.slab_v, srow, v);
      else store_raw8<IT>(a.slab_v, srow, rv);
    }
  }
}

template <int IT>
hipError_t launch_for_input(const ProduceArgs& a, dim3 grid, hipStream_t stream) {
  if (a.k_dtype == kSplitRows) {
    if (a.q_dtype != kF32) return hipErrorInvalidValue;
    produce_kernel<IT, kF32, kSplitRows><<<grid, kThreads, 0, stream>>>(a);
    return hipGetLastError();
  }
  if (a.q_dtype != a.k_dtype) return hipErrorInvalidValue;
  switch (a.q_dtype) {
    case kF32: produce_kernel<IT, kF32><<<grid, kThreads, 0, stream>>>(a); break;
    case kF16: produce_kernel<IT, kF16><<<grid, kThreads, 0, stream>>>(a); break;
    case kBF16: produce_kernel<IT, kBF16><<<grid, kThreads, 0, stream>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_produce(const ProduceArgs& a, hipStream_t stream) {
  if (a.rows <= 0) return hipSuccess;
  const int64_t blocks = (a.rows + kRowsPerBlock - 1) / kRowsPerBlock;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  const dim3 grid(static_cast<uint32_t>(blocks));
  switch (a.qkv_dtype) {
    case kBF16: return launch_for_input<kBF16>(a, grid, stream);
    case kF16: return launch_for_input<kF16>(a, grid, stream);
    case kF32: return launch_for_input<kF32>(a, grid, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace hkv
