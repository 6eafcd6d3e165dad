// Segmented flash attention over a packed head-pruned KV slab, for gfx950.
//
// Semantics follow _fused_real_pruning_segmented_attention_kernel
// (real_pruning_fused_attention.py:76-267): query l of (b, h) attends to the
// slab rows of head h's segments in table order, then to the current scale's
// K/V rows of (b, h); online softmax with fp32 statistics, P rounded to the V
// operand type before the PV product, O / l at the end, output [B, L, H*D].
//
// Design (CDNA4, wave64):
//  * One workgroup = 4 waves = 128 queries of one (b, h).  A wave owns 32
//    query rows and keeps their Q fragments in registers for the whole call.
//  * Keys are walked as one virtual stream: retained prior rows (all segments
//    back to back, no per-segment tile restart) and then the current rows, in
//    tiles of 64 keys.  A 64-entry row table per tile (computed one tile ahead
//    by wave 0 from the segment prefix sums) maps stream position -> slab row
//    or current row, so short segments (1, 4, 16, 36 tokens) cost no padding.
//  * K and V tiles are fetched with 16-byte global loads into registers one
//    tile ahead (overlapping the MFMA work of the current tile), then stored
//    to LDS: K row-major (row pitch padded to 272 B, conflict-free 16-byte
//    reads), V transposed (V^T[d][key], XOR-swizzled 8-byte quads).
//  * S^T = K Q^T on v_mfma_f32_32x32x16_{bf16,f16}: with keys as the M index
//    each lane holds one query's 16 scores per 32-key block, so row max and
//    row sum need one cross-half exchange (lane l <-> l+32) per tile, and the
//    fp32 scores convert in place to the B operand of O^T = V^T P^T.
//  * exp2 with scale*log2(e) folded into one FMA per score.
//  * Workgroup ids are mapped so that consecutive work items (the query tiles
//    of one (b, h)) land on the same XCD (dispatch is round-robin over the 8
//    XCDs) and share that XCD's L2 for the head's K/V stream.
#include "hkv_internal.h"

namespace hkv {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kD = 128;
constexpr int kBM = 128;                 // queries per workgroup
constexpr int kBN = 64;                  // keys per tile
constexpr int kThreads = 256;
constexpr int kKPitch = kD * 2 + 16;     // bytes per K row in LDS
constexpr int kVtPitch = kBN * 2;        // bytes per V^T row in LDS
constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ uint32_t pack_bf16(float x, float y) {
  const uint16_t a = __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
  const uint16_t b = __builtin_bit_cast(uint16_t, static_cast<__bf16>(y));
  return static_cast<uint32_t>(a) | (static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ uint32_t pack_f16(float x, float y) {
  const uint16_t a = __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
  const uint16_t b = __builtin_bit_cast(uint16_t, static_cast<_Float16>(y));
  return static_cast<uint32_t>(a) | (static_cast<uint32_t>(b) << 16);
}
template <int MT>
__device__ __forceinline__ uint32_t pack2(float x, float y) {
  if constexpr (MT == kF16) return pack_f16(x, y);
  else return pack_bf16(x, y);
}
__device__ __forceinline__ float f16_to_f32(uint16_t v) {
  return static_cast<float>(__builtin_bit_cast(_Float16, v));
}

// Loads 8 consecutive elements of type DT at base + elem (elements) and
// returns them as 8 packed 16-bit values of the MFMA operand type MT.
// Invalid positions yield zeros (no memory access).
template <int DT, int MT>
__device__ __forceinline__ u32x4_t load8(const void* base, int64_t elem, bool valid) {
  u32x4_t r = {0u, 0u, 0u, 0u};
  if (!valid) return r;
  if constexpr (DT == kF32) {
    const f32x4_t* p = reinterpret_cast<const f32x4_t*>(static_cast<const float*>(base) + elem);
    const f32x4_t x = p[0];
    const f32x4_t y = p[1];
    r[0] = pack2<MT>(x[0], x[1]);
    r[1] = pack2<MT>(x[2], x[3]);
    r[2] = pack2<MT>(y[0], y[1]);
    r[3] = pack2<MT>(y[2], y[3]);
  } else {
    r = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(base) + elem);
    if constexpr (DT == kF16 && MT == kBF16) {
      // fp16 storage feeding a bf16 product (mixed q/k types): widen and round.
#pragma unroll
      for (int i = 0; i < 4; ++i)
        r[i] = pack_bf16(f16_to_f32(static_cast<uint16_t>(r[i] & 0xffffu)),
                         f16_to_f32(static_cast<uint16_t>(r[i] >> 16)));
    }
  }
  return r;
}

template <int MT>
__device__ __forceinline__ f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
  if constexpr (MT == kF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Physical 8-byte quad slot of key quad kq in V^T row d.  Distinct over any 16
// consecutive rows (conflict-free MFMA operand reads) and spread over all 16
// slots across the 16 d-chunks a wave writes (4-way = minimal write cost).
__device__ __forceinline__ int vt_slot(int d, int kq) {
  return kq ^ ((d & 15) ^ ((d >> 4) & 7));
}

template <int DT>
__device__ __forceinline__ void store4(void* out, int64_t elem, f32x4_t v) {
  if constexpr (DT == kF32) {
    *reinterpret_cast<f32x4_t*>(static_cast<float*>(out) + elem) = v;
  } else {
    u32x2_t w;
    w[0] = pack2<DT>(v[0], v[1]);
    w[1] = pack2<DT>(v[2], v[3]);
    *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(out) + elem) = w;
  }
}

template <int QDT, int KDT, int VDT>
__global__ __launch_bounds__(kThreads, 2) void seg_attn_kernel(AttnArgs a, float c, float scale_abs,
                                                               uint32_t q_sign, int32_t n_qt) {
  constexpr int MQK = (QDT == kF16 && KDT == kF16) ? kF16 : kBF16;
  constexpr int MV = (VDT == kF16) ? kF16 : kBF16;

  __shared__ __attribute__((aligned(16))) uint8_t k_lds[kBN * kKPitch];
  __shared__ __attribute__((aligned(16))) uint8_t vt_lds[kD * kVtPitch];
  __shared__ __attribute__((aligned(16))) int32_t rowtab[2][kBN];
  __shared__ int32_t seg_start[kMaxSegments];
  __shared__ int32_t seg_pref[kMaxSegments + 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;  // half of the wave: selects the k-slot group of MFMA operands
  const int H = a.heads;
  const int L = a.cur_len;

  // ---- work item (XCD-aware: equal shares of consecutive items per XCD)
  const int32_t n_items = a.batch * H * n_qt;
  int32_t item = blockIdx.x;
  if ((n_items & 7) == 0) item = (blockIdx.x & 7) * (n_items >> 3) + (blockIdx.x >> 3);
  const int32_t bh = item / n_qt;
  const int32_t qt = item - bh * n_qt;
  const int32_t b = bh / H;
  const int32_t h = bh - b * H;

  // ---- segment table of head h: clamped starts and exclusive length prefix
  int nseg = a.seg_counts[h];
  nseg = nseg < 0 ? 0 : (nseg > a.max_segments ? a.max_segments : nseg);
  for (int i = tid; i < nseg; i += kThreads) {
    int64_t st = a.seg_starts[static_cast<int64_t>(h) * a.max_segments + i];
    int64_t en = a.seg_ends[static_cast<int64_t>(h) * a.max_segments + i];
    st = st < 0 ? 0 : (st > a.slab_capacity ? a.slab_capacity : st);
    en = en < 0 ? 0 : (en > a.slab_capacity ? a.slab_capacity : en);
    seg_start[i] = static_cast<int32_t>(st);
    seg_pref[i + 1] = en > st ? static_cast<int32_t>(en - st) : 0;
  }
  __syncthreads();
  if (wave == 0) {
    int v[4];
    int local = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int idx = lane * 4 + k;
      v[k] = idx < nseg ? seg_pref[idx + 1] : 0;
      local += v[k];
    }
    int incl = local;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(incl, off, 64);
      if (lane >= off) incl += o;
    }
    int run = incl - local;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int idx = lane * 4 + k;
      run += v[k];
      if (idx < nseg) seg_pref[idx + 1] = run;
    }
    if (lane == 0) seg_pref[0] = 0;
  }
  __syncthreads();
  const int32_t R = seg_pref[nseg];  // retained prior rows of this head
  const int32_t T = R + L;           // keys in the stream
  const int32_t ntiles = (T + kBN - 1) / kBN;

  // ---- row table: stream position -> slab row (>= 0) or ~current row (< 0)
  int cur_seg = 0;
  auto fill_rowtab = [&](int tile, int buf) {
    const int j0 = tile * kBN;
    while (cur_seg < nseg && seg_pref[cur_seg + 1] <= j0) ++cur_seg;
    const int j = j0 + lane;
    int code;
    if (j < R) {
      int s = cur_seg;
      while (seg_pref[s + 1] <= j) ++s;
      code = seg_start[s] + (j - seg_pref[s]);
    } else if (j < T) {
      code = ~(j - R);
    } else {
      code = ~0;  // never dereferenced: loads of keys >= T are skipped
    }
    rowtab[buf][lane] = code;
  };

  // ---- loader role: key quad lq (keys 4lq..4lq+3), d-chunk lc (d 8lc..8lc+7)
  const int lq = tid >> 4;
  const int lc = tid & 15;
  u32x4_t kreg[4];
  u32x4_t vreg[4];
  const int64_t slab_row0 = static_cast<int64_t>(b) * a.slab_capacity;
  const int64_t cur_row0 = static_cast<int64_t>(bh) * L;
  auto issue_loads = [&](int tile, int buf) {
    const int4 codes = *reinterpret_cast<const int4*>(&rowtab[buf][lq * 4]);
    const int cc[4] = {codes.x, codes.y, codes.z, codes.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int code = cc[i];
      const bool valid = tile * kBN + lq * 4 + i < T;
      const bool in_slab = code >= 0;
      const int64_t row = in_slab ? slab_row0 + code : cur_row0 + (~code);
      const int64_t elem = row * kD + lc * 8;
      kreg[i] = load8<KDT, MQK>(in_slab ? a.slab_k : a.cur_k, elem, valid);
      vreg[i] = load8<VDT, MV>(in_slab ? a.slab_v : a.cur_v, elem, valid);
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<u32x4_t*>(k_lds + (lq * 4 + i) * kKPitch + lc * 16) = kreg[i];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      u32x2_t even, odd;
      even[0] = __builtin_amdgcn_perm(vreg[1][w], vreg[0][w], 0x05040100u);
      even[1] = __builtin_amdgcn_perm(vreg[3][w], vreg[2][w], 0x05040100u);
      odd[0] = __builtin_amdgcn_perm(vreg[1][w], vreg[0][w], 0x07060302u);
      odd[1] = __builtin_amdgcn_perm(vreg[3][w], vreg[2][w], 0x07060302u);
      const int d0 = lc * 8 + 2 * w;
      const int d1 = d0 + 1;
      *reinterpret_cast<u32x2_t*>(vt_lds + d0 * kVtPitch + 8 * vt_slot(d0, lq)) = even;
      *reinterpret_cast<u32x2_t*>(vt_lds + d1 * kVtPitch + 8 * vt_slot(d1, lq)) = odd;
    }
  };

  // ---- Q fragments (B operand of S^T = K Q^T): query row, d = 16ks + 8g .. +7
  const int32_t qrow = qt * kBM + wave * 32 + (lane & 31);
  const bool qvalid = qrow < L;
  u32x4_t qf[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    qf[ks] = load8<QDT, MQK>(a.q, (cur_row0 + qrow) * kD + ks * 16 + g * 8, qvalid);
    qf[ks] ^= q_sign;  // negative softmax scale: exact sign flip of q
  }

  f32x16_t oacc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) oacc[i] = f32x16_t{};
  float m_run = -1e30f;  // running max of raw scores (sign-adjusted)
  float l_run = 0.f;     // this lane's partial row sum

  if (wave == 0) fill_rowtab(0, 0);
  __syncthreads();
  issue_loads(0, 0);
  if (wave == 0 && ntiles > 1) fill_rowtab(1, 1);

  for (int t = 0; t < ntiles; ++t) {
    store_tile();
    __syncthreads();
    if (t + 1 < ntiles) issue_loads(t + 1, (t + 1) & 1);
    if (wave == 0 && t + 2 < ntiles) fill_rowtab(t + 2, t & 1);

    // S^T block kb: keys 32kb + (8(j>>2) + 4g + (j&3)), query lane&31
    f32x16_t s[2] = {f32x16_t{}, f32x16_t{}};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const u32x4_t kf = *reinterpret_cast<const u32x4_t*>(
            k_lds + (kb * 32 + (lane & 31)) * kKPitch + (ks * 16 + g * 8) * 2);
        s[kb] = mfma32<MQK>(kf, qf[ks], s[kb]);
      }
    }
    const bool tail = (t + 1) * kBN > T;
    if (tail) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int key = t * kBN + kb * 32 + 8 * (j >> 2) + 4 * g + (j & 3);
          if (key >= T) s[kb][j] = -__builtin_inff();
        }
    }
    float mx = s[0][0];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 16; ++j) mx = fmaxf(mx, s[kb][j]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = exp2f((m_run - m_new) * c);
    const float mc = m_new * c;
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float p = exp2f(__builtin_fmaf(s[kb][j], c, -mc));
        s[kb][j] = p;
      }
    if (tail) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int key = t * kBN + kb * 32 + 8 * (j >> 2) + 4 * g + (j & 3);
          if (key >= T) s[kb][j] = 0.f;
        }
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 16; ++j) psum += s[kb][j];
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < 4; ++db) oacc[db] *= alpha;

    // O^T += V^T P^T: k-step u covers keys 16u + {4g..4g+3, 8+4g..8+4g+3}
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const f32x16_t& sp = s[u >> 1];
      const int j0 = 8 * (u & 1);
      u32x4_t pf;
      pf[0] = pack2<MV>(sp[j0 + 0], sp[j0 + 1]);
      pf[1] = pack2<MV>(sp[j0 + 2], sp[j0 + 3]);
      pf[2] = pack2<MV>(sp[j0 + 4], sp[j0 + 5]);
      pf[3] = pack2<MV>(sp[j0 + 6], sp[j0 + 7]);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int d = db * 32 + (lane & 31);
        const uint8_t* row = vt_lds + d * kVtPitch;
        const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(row + 8 * vt_slot(d, 4 * u + g));
        const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(row + 8 * vt_slot(d, 4 * u + 2 + g));
        u32x4_t vf;
        vf[0] = lo[0];
        vf[1] = lo[1];
        vf[2] = hi[0];
        vf[3] = hi[1];
        oacc[db] = mfma32<MV>(vf, pf, oacc[db]);
      }
    }
    __syncthreads();
  }

  // ---- epilogue: O = acc / l, out[b, q, h*D + d]; lse = scale*m + ln(l)
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = 1.f / l_tot;
  if (qvalid) {
    const int64_t out_row = (static_cast<int64_t>(b) * L + qrow) * (static_cast<int64_t>(H) * kD) +
                            static_cast<int64_t>(h) * kD;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        f32x4_t v;
        v[0] = oacc[db][4 * jb + 0] * inv;
        v[1] = oacc[db][4 * jb + 1] * inv;
        v[2] = oacc[db][4 * jb + 2] * inv;
        v[3] = oacc[db][4 * jb + 3] * inv;
        store4<QDT>(a.out, out_row + db * 32 + 8 * jb + 4 * g, v);
      }
    if (a.lse != nullptr && g == 0)
      a.lse[cur_row0 + qrow] = m_run * scale_abs + __logf(l_tot);
  }
}

template <int QDT, int KDT>
hipError_t dispatch_v(const AttnArgs& a, dim3 grid, float c, float sabs, uint32_t qs, int32_t nqt,
                      hipStream_t st) {
  switch (a.v_dtype) {
    case kBF16: seg_attn_kernel<QDT, KDT, kBF16><<<grid, kThreads, 0, st>>>(a, c, sabs, qs, nqt); break;
    case kF16: seg_attn_kernel<QDT, KDT, kF16><<<grid, kThreads, 0, st>>>(a, c, sabs, qs, nqt); break;
    case kF32: seg_attn_kernel<QDT, KDT, kF32><<<grid, kThreads, 0, st>>>(a, c, sabs, qs, nqt); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_segmented_attention(const AttnArgs& a, hipStream_t stream) {
  const int32_t n_qt = (a.cur_len + kBM - 1) / kBM;
  const int64_t blocks = static_cast<int64_t>(a.batch) * a.heads * n_qt;
  if (blocks <= 0) return hipSuccess;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  dim3 grid(static_cast<uint32_t>(blocks));
  const float sabs = a.softmax_scale < 0.f ? -a.softmax_scale : a.softmax_scale;
  const float c = sabs * kLog2e;
  const uint32_t qs = a.softmax_scale < 0.f ? 0x80008000u : 0u;
  if (a.q_dtype != a.k_dtype) return hipErrorInvalidValue;
  switch (a.q_dtype) {
    case kBF16: return dispatch_v<kBF16, kBF16>(a, grid, c, sabs, qs, n_qt, stream);
    case kF16: return dispatch_v<kF16, kF16>(a, grid, c, sabs, qs, n_qt, stream);
    case kF32: return dispatch_v<kF32, kF32>(a, grid, c, sabs, qs, n_qt, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace hkv
