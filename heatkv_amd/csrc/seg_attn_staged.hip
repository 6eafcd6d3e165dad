// Segmented attention, register-staged variant: serves any mix of fp16 /
// bf16 / fp32 inputs (fp32 K or V are converted to bf16 MFMA operands while
// staging, which the direct-to-LDS variant cannot do).  fp32 q and k are
// split into bf16 high and low parts and S = K Q^T is taken as
// Kh Qh + Kl Qh + Kh Ql (three MFMAs per step, ~16 significand bits, beyond
// the TF32 products the reference's Triton dot uses for fp32 operands); fp32
// V and P are rounded to bf16 for O = P V.
//
// Each thread loads its share of the next 64-key tile into registers with
// 16-byte buffer loads (out-of-range rows read as zeros) while the current
// tile is computed, then stores it to LDS: K row-major with a 272-byte pitch
// (conflict-free 16-byte operand reads), V transposed to V^T[d][key] with a
// 136-byte pitch (conflict-free 8-byte operand reads) by a 4x8 register
// transpose of 16-bit values.
#include "attn_common.h"

namespace hkv {
namespace {

using namespace attn;

constexpr int kKPitch = kD * 2 + 16;   // bytes per K row in LDS
constexpr int kVtPitch = kBN * 2 + 8;  // bytes per V^T row in LDS

template <int QDT, int KDT, int VDT, int NW>
__global__ __launch_bounds__(NW * 64, 2) void seg_attn_staged_kernel(const AttnArgs a,
                                                                     const Scalars sc,
                                                                     const int32_t n_qt) {
  constexpr int MQK = (QDT == kF16 && KDT == kF16) ? kF16 : kBF16;
  constexpr int MV = (VDT == kF16) ? kF16 : kBF16;
  constexpr int kThreads = NW * 64;
  constexpr int kBM = NW * 32;
  constexpr int kQuadChunks = kBN / 4 * 16;  // (4-key quad, 16-byte d-chunk) pairs per tensor
  constexpr int kLoadsPerThread = 2 * kQuadChunks / kThreads;
  constexpr int kEK = KDT == kF32 ? 4 : 2;
  constexpr int kEV = VDT == kF32 ? 4 : 2;
  constexpr int kEQ = QDT == kF32 ? 4 : 2;
  constexpr bool kSplit = QDT == kF32 && KDT == kF32;
  static_assert(2 * kQuadChunks % kThreads == 0, "loader split");

  __shared__ __attribute__((aligned(16))) uint8_t k_lds[kBN * kKPitch];
  __shared__ __attribute__((aligned(16))) uint8_t k_lds_lo[kSplit ? kBN * kKPitch : 16];
  __shared__ __attribute__((aligned(16))) uint8_t vt_lds[kD * kVtPitch];
  __shared__ __attribute__((aligned(16))) int32_t rowtab[2][kBN];
  __shared__ int32_t seg_start[kMaxSegments];
  __shared__ int32_t seg_pref[kMaxSegments + 1];
  __shared__ __attribute__((aligned(16))) int32_t head_rows[kMaxHeads];
  __shared__ int32_t head_by_rank[kMaxHeads];

  const int64_t cap = a.slab_capacity;
  const int H = a.heads;
  const int L = a.cur_len;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;

  const WorkItem w = plan_work<kThreads>(a.seg_starts, a.seg_ends, a.seg_counts, cap, H,
                                         a.max_segments, a.batch, n_qt, head_rows, head_by_rank,
                                         seg_start, seg_pref, static_cast<int32_t>(blockIdx.x),
                                         reinterpret_cast<int32_t*>(k_lds), sizeof(k_lds) / 4);
  const int32_t R = w.R;
  const int32_t ntp = (R + kBN - 1) / kBN;
  const int32_t ntc = (L + kBN - 1) / kBN;
  const int32_t ntiles = ntp + ntc;

  const __amdgpu_buffer_rsrc_t rs_k = make_rsrc(
      static_cast<const uint8_t*>(a.slab_k) + static_cast<int64_t>(w.b) * cap * kD * kEK,
      static_cast<uint32_t>(cap * kD * kEK));
  const __amdgpu_buffer_rsrc_t rs_v = make_rsrc(
      static_cast<const uint8_t*>(a.slab_v) + static_cast<int64_t>(w.b) * cap * kD * kEV,
      static_cast<uint32_t>(cap * kD * kEV));
  const int64_t cur_row0 = static_cast<int64_t>(w.bh) * L;
  const __amdgpu_buffer_rsrc_t rc_k = make_rsrc(
      static_cast<const uint8_t*>(a.cur_k) + cur_row0 * kD * kEK, static_cast<uint32_t>(L * kD * kEK));
  const __amdgpu_buffer_rsrc_t rc_v = make_rsrc(
      static_cast<const uint8_t*>(a.cur_v) + cur_row0 * kD * kEV, static_cast<uint32_t>(L * kD * kEV));

  int cur_seg = 0;
  // quad-chunk i covers keys 4(i/16)..+3 at d 8(i%16)..+7 of K (i < kQuadChunks)
  // or of V; thread tid owns quad-chunks tid, tid + kThreads, ...
  u32x4_t lreg[kLoadsPerThread][4];
  u32x4_t lreg_lo[kSplit ? kLoadsPerThread : 1][4];  // low bf16 parts of fp32 K
  auto issue_loads = [&](int tile, int buf) {
    if (tile < ntp) {
#pragma unroll
      for (int it = 0; it < kLoadsPerThread; ++it) {
        const int item = tid + it * kThreads;
        const bool is_v = item >= kQuadChunks;
        const int qc = is_v ? item - kQuadChunks : item;
        const int lq = qc >> 4;
        const int lc = qc & 15;
        const int4 rows = *reinterpret_cast<const int4*>(&rowtab[buf][lq * 4]);
        const int rr[4] = {rows.x, rows.y, rows.z, rows.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (is_v)
            lreg[it][i] = load8<VDT, MV>(rs_v, rr[i] < 0 ? -1 : (rr[i] * kD + lc * 8) * kEV);
          else if constexpr (kSplit)
            load8_split(rs_k, rr[i] < 0 ? -1 : (rr[i] * kD + lc * 8) * kEK, lreg[it][i], lreg_lo[it][i]);
          else
            lreg[it][i] = load8<KDT, MQK>(rs_k, rr[i] < 0 ? -1 : (rr[i] * kD + lc * 8) * kEK);
        }
      }
    } else {
      const int row0 = (tile - ntp) * kBN;
#pragma unroll
      for (int it = 0; it < kLoadsPerThread; ++it) {
        const int item = tid + it * kThreads;
        const bool is_v = item >= kQuadChunks;
        const int qc = is_v ? item - kQuadChunks : item;
        const int lq = qc >> 4;
        const int lc = qc & 15;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = row0 + lq * 4 + i;
          if (is_v)
            lreg[it][i] = load8<VDT, MV>(rc_v, row < L ? (row * kD + lc * 8) * kEV : -1);
          else if constexpr (kSplit)
            load8_split(rc_k, row < L ? (row * kD + lc * 8) * kEK : -1, lreg[it][i], lreg_lo[it][i]);
          else
            lreg[it][i] = load8<KDT, MQK>(rc_k, row < L ? (row * kD + lc * 8) * kEK : -1);
        }
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int it = 0; it < kLoadsPerThread; ++it) {
      const int item = tid + it * kThreads;
      const bool is_v = item >= kQuadChunks;
      const int qc = is_v ? item - kQuadChunks : item;
      const int lq = qc >> 4;
      const int lc = qc & 15;
      const u32x4_t* r = lreg[it];
      if (!is_v) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          *reinterpret_cast<u32x4_t*>(k_lds + (lq * 4 + i) * kKPitch + lc * 16) = r[i];
          if constexpr (kSplit)
            *reinterpret_cast<u32x4_t*>(k_lds_lo + (lq * 4 + i) * kKPitch + lc * 16) = lreg_lo[it][i];
        }
      } else {
        // transpose 4 keys x 8 d into 8 rows of V^T (4 keys each)
#pragma unroll
        for (int wi = 0; wi < 4; ++wi) {
          u32x2_t even, odd;
          even[0] = __builtin_amdgcn_perm(r[1][wi], r[0][wi], 0x05040100u);
          even[1] = __builtin_amdgcn_perm(r[3][wi], r[2][wi], 0x05040100u);
          odd[0] = __builtin_amdgcn_perm(r[1][wi], r[0][wi], 0x07060302u);
          odd[1] = __builtin_amdgcn_perm(r[3][wi], r[2][wi], 0x07060302u);
          uint8_t* row = vt_lds + (lc * 8 + 2 * wi) * kVtPitch + lq * 8;
          *reinterpret_cast<u32x2_t*>(row) = even;
          *reinterpret_cast<u32x2_t*>(row + kVtPitch) = odd;
        }
      }
    }
  };

  // Q fragments (B operand of S^T = K Q^T): query row, d = 16ks + 8g .. +7
  const int32_t qrow = w.qt * kBM + wave * 32 + (lane & 31);
  u32x4_t qf[8];
  u32x4_t qf_lo[kSplit ? 8 : 1];
  {
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(
        static_cast<const uint8_t*>(a.q) + cur_row0 * kD * kEQ, static_cast<uint32_t>(L * kD * kEQ));
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const int32_t off = qrow < L ? (qrow * kD + ks * 16 + g * 8) * kEQ : -1;
      if constexpr (kSplit) {
        load8_split(rq, off, qf[ks], qf_lo[ks]);
        qf_lo[ks] ^= sc.q_sign;
      } else {
        qf[ks] = load8<QDT, MQK>(rq, off);
      }
      qf[ks] ^= sc.q_sign;
    }
  }

  f32x16_t oacc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) oacc[i] = f32x16_t{};
  float m_run = -1e30f;
  float l_run = 0.f;
  const uint8_t* k_lane = k_lds + (lane & 31) * kKPitch + g * 16;
  const uint8_t* v_lane = vt_lds + (lane & 31) * kVtPitch + g * 8;

  if (wave == 0 && ntp > 0) fill_rowtab(0, rowtab[0], cur_seg, w.nseg, R, seg_start, seg_pref);
  __syncthreads();
  issue_loads(0, 0);
  if (wave == 0 && 1 < ntp) fill_rowtab(1, rowtab[1], cur_seg, w.nseg, R, seg_start, seg_pref);

  for (int t = 0; t < ntiles; ++t) {
    store_tile();
    __syncthreads();
    if (t + 1 < ntiles) issue_loads(t + 1, (t + 1) & 1);
    if (wave == 0 && t + 2 < ntp)
      fill_rowtab(t + 2, rowtab[t & 1], cur_seg, w.nseg, R, seg_start, seg_pref);

    f32x16_t s[2] = {f32x16_t{}, f32x16_t{}};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const u32x4_t kf = *reinterpret_cast<const u32x4_t*>(k_lane + kb * 32 * kKPitch + ks * 32);
        s[kb] = mfma32<MQK>(kf, qf[ks], s[kb]);
        if constexpr (kSplit) {
          const u32x4_t kl = *reinterpret_cast<const u32x4_t*>(k_lane + (k_lds_lo - k_lds) + kb * 32 * kKPitch + ks * 32);
          s[kb] = mfma32<MQK>(kl, qf[ks], s[kb]);
          s[kb] = mfma32<MQK>(kf, qf_lo[ks], s[kb]);
        }
      }
    const int valid = t < ntp ? min(kBN, R - t * kBN) : min(kBN, L - (t - ntp) * kBN);
    softmax_tile(s, oacc, m_run, l_run, sc.c, sc.thresh, valid, g);
#pragma unroll
    for (int u = 0; u < kBN / 16; ++u) {
      const u32x4_t pf = p_operand<MV>(s, u);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const uint8_t* row = v_lane + db * 32 * kVtPitch + 32 * u;
        const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(row);
        const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(row + 16);
        const u32x4_t vf = {lo[0], lo[1], hi[0], hi[1]};
        oacc[db] = mfma32<MV>(vf, pf, oacc[db]);
      }
    }
    __syncthreads();
  }
  write_output(oacc, m_run, l_run, sc.c, a.out, a.lse, w.b, w.h, qrow, L, H, w.bh, g, a.out_dtype);
}

template <int QDT, int KDT, int VDT>
hipError_t launch(const AttnArgs& a, const Scalars& s, hipStream_t st) {
  constexpr int NW = 8;
  const int32_t n_qt = (a.cur_len + NW * 32 - 1) / (NW * 32);
  const int64_t blocks = static_cast<int64_t>(a.batch) * a.heads * n_qt;
  if (blocks <= 0) return hipSuccess;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  seg_attn_staged_kernel<QDT, KDT, VDT, NW><<<dim3(static_cast<uint32_t>(blocks)), NW * 64, 0, st>>>(
      a, s, n_qt);
  return hipGetLastError();
}

template <int QDT, int KDT>
hipError_t dispatch_v(const AttnArgs& a, const Scalars& s, hipStream_t st) {
  switch (a.v_dtype) {
    case kBF16: return launch<QDT, KDT, kBF16>(a, s, st);
    case kF16: return launch<QDT, KDT, kF16>(a, s, st);
    case kF32: return launch<QDT, KDT, kF32>(a, s, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_attention_staged(const AttnArgs& a, const attn::Scalars& s, hipStream_t stream) {
  if (a.q_dtype != a.k_dtype) return hipErrorInvalidValue;
  switch (a.q_dtype) {
    case kBF16: return dispatch_v<kBF16, kBF16>(a, s, stream);
    case kF16: return dispatch_v<kF16, kF16>(a, s, stream);
    case kF32: return dispatch_v<kF32, kF32>(a, s, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace hkv
