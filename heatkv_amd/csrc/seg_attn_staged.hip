// Segmented attention, register-staged variant: serves any mix of fp16 /
// bf16 / fp32 inputs and the reference's higher-precision dot modes, which
// the direct-to-LDS variant (16-bit operands straight from HBM) cannot.
//
// Precision by operand splitting.  A value x is written as NP bf16 pieces,
// x = x0 + x1 + ... with x0 = bf16(x), x1 = bf16(x - x0), ... (each
// subtraction is exact in fp32), so 2 pieces carry about 16 significand
// bits and 3 pieces all 24 of fp32.  A product of split operands is taken as
// the MFMA sum of the piece products a_i b_j with i + j < order (order = the
// larger piece count), which drops only terms below 2^-8(order) relative:
//  * QK: fp32 q/k are split in 2 pieces (3 products, ~16 bits; the
//    reference's default Triton dot of fp32 operands runs at TF32, 11 bits),
//    or 3 pieces under REAL_PRUNING_FUSED_QK_DOT_MODE=fp32/ieee (6 products,
//    fp32 accuracy).  16-bit q/k products are exact in every mode.
//  * PV: by default P is rounded to V's 16-bit type (the reference's
//    p.to(v.dtype)); with fp32 V the reference keeps P in fp32 and takes a
//    TF32 dot, here P and V are split in 2 pieces (3 products).  Under
//    REAL_PRUNING_FUSED_VALUE_DOT_MODE=fp32 (an fp32 P V product) P is split
//    in 3 pieces and V in as many as its type needs (bf16 1, fp16 2 -- both
//    exact -- and fp32 3).
//
// Each thread loads its share of the next 64-key tile into registers with
// 16-byte buffer loads (out-of-range rows read as zeros) while the current
// tile is computed, then stores it to LDS: K pieces row-major with a 272-byte
// pitch (conflict-free 16-byte operand reads), V pieces transposed to
// V^T[d][key] with a 136-byte pitch (conflict-free 8-byte operand reads) by
// a 4x8 register transpose of 16-bit values.
#include "attn_common.h"

namespace hkv {
namespace {

using namespace attn;

constexpr int kKPitch = kD * 2 + 16;   // bytes per K row in LDS
constexpr int kVtPitch = kBN * 2 + 8;  // bytes per V^T row in LDS

// Splits 8 fp32 values into NP packed operand pieces: bf16 pieces when
// NP > 1, else one piece of type MT (round to nearest even).
template <int MT, int NP>
__device__ __forceinline__ void split8(const float (&v)[8], u32x4_t (&out)[NP]) {
  if constexpr (NP == 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) out[0][i] = pack2<MT>(v[2 * i], v[2 * i + 1]);
  } else {
    float r[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = v[i];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t w = pack2<kBF16>(r[2 * i], r[2 * i + 1]);
        out[p][i] = w;
        if (p + 1 < NP) {
          r[2 * i] -= __builtin_bit_cast(float, w << 16);
          r[2 * i + 1] -= __builtin_bit_cast(float, w & 0xffff0000u);
        }
      }
    }
  }
}

// 8 consecutive elements of type DT, as loaded: 32 bytes for fp32, 16 for
// 16-bit types (w[1] unused).
struct Raw8 {
  u32x4_t w[2];
};

// Raw load of 8 elements of type DT at byte offset `off` of `r` (an offset of
// -1 yields zeros).
template <int DT>
__device__ __forceinline__ Raw8 load_raw8(__amdgpu_buffer_rsrc_t r, int32_t off) {
  Raw8 x;
  x.w[0] = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  if constexpr (DT == kF32) x.w[1] = __builtin_amdgcn_raw_buffer_load_b128(r, off < 0 ? -1 : off + 16, 0, 0);
  else x.w[1] = u32x4_t{};
  return x;
}

// The 8 raw elements as NP operand pieces (see split8); NP == 1 with a
// 16-bit DT equal to MT is the raw data itself.
template <int DT, int MT, int NP>
__device__ __forceinline__ void pieces8(const Raw8& x, u32x4_t (&out)[NP]) {
  if constexpr (NP == 1 && DT == MT) {
    out[0] = x.w[0];
  } else {
    // Whole-vector bit casts first: extracting single elements of a buffer
    // load's result and casting them miscompiles with this toolchain (the
    // vector load becomes one dword load, replicated).
    const f32x4_t x0 = __builtin_bit_cast(f32x4_t, x.w[0]);
    const f32x4_t x1 = __builtin_bit_cast(f32x4_t, x.w[1]);
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (DT == kF32) {
        v[i] = x0[i];
        v[4 + i] = x1[i];
      } else if constexpr (DT == kF16) {
        v[2 * i] = f16_to_f32(static_cast<uint16_t>(x.w[0][i] & 0xffffu));
        v[2 * i + 1] = f16_to_f32(static_cast<uint16_t>(x.w[0][i] >> 16));
      } else {
        v[2 * i] = __builtin_bit_cast(float, x.w[0][i] << 16);
        v[2 * i + 1] = __builtin_bit_cast(float, x.w[0][i] & 0xffff0000u);
      }
    }
    split8<MT, NP>(v, out);
  }
}

// Piece products of a split contraction step: (i, j) with i + j < ORDER.
template <int NA, int NB>
struct Products {
  static constexpr int kOrder = NA > NB ? NA : NB;
};

template <int MT, int NA, int NB>
__device__ __forceinline__ f32x16_t mfma_split(const u32x4_t (&a)[NA], const u32x4_t (&b)[NB], f32x16_t c) {
  constexpr int order = Products<NA, NB>::kOrder;
  // largest products first: pieces fall by 2^-8 each
#pragma unroll
  for (int s = 0; s < order; ++s)
#pragma unroll
    for (int i = 0; i <= s; ++i) {
      const int j = s - i;
      if (i < NA && j < NB) c = mfma32<MT>(a[i], b[j], c);
    }
  return c;
}

// NQS: q/k pieces; NPS / NVS: P / V pieces.  MQK / MV: operand types of
// one-piece products.
template <int QDT, int KDT, int VDT, int NQS, int NPS, int NVS, int NW, int MINB>
__global__ __launch_bounds__(NW * 64, MINB) void seg_attn_staged_kernel(const AttnArgs a,
                                                                        const Scalars sc,
                                                                        const int32_t n_qt) {
  constexpr int MQK = (NQS == 1 && QDT == kF16 && KDT == kF16) ? kF16 : kBF16;
  constexpr int MV = (NPS == 1 && NVS == 1 && VDT == kF16) ? kF16 : kBF16;
  constexpr int kThreads = NW * 64;
  constexpr int kBM = NW * 32;
  constexpr int kQuadChunks = kBN / 4 * 16;  // (4-key quad, 16-byte d-chunk) pairs per tensor
  constexpr int kLoadsPerThread = 2 * kQuadChunks / kThreads;
  constexpr int kEK = KDT == kF32 ? 4 : 2;
  constexpr int kEV = VDT == kF32 ? 4 : 2;
  constexpr int kEQ = QDT == kF32 ? 4 : 2;
  constexpr int kKBytes = kBN * kKPitch;
  constexpr int kVBytes = kD * kVtPitch;
  static_assert(2 * kQuadChunks % kThreads == 0, "loader split");
  static_assert(NQS >= 1 && NQS <= 3 && NPS >= 1 && NPS <= 3 && NVS >= 1 && NVS <= 3, "pieces");

  __shared__ __attribute__((aligned(16))) uint8_t k_lds[NQS * kKBytes];
  __shared__ __attribute__((aligned(16))) uint8_t vt_lds[NVS * kVBytes];
  __shared__ __attribute__((aligned(16))) int32_t rowtab[2][kBN];
  __shared__ int32_t seg_start[kMaxSegments];
  __shared__ int32_t seg_pref[kMaxSegments + 1];
  __shared__ __attribute__((aligned(16))) int32_t head_rows[kMaxHeads];
  __shared__ int32_t head_by_rank[kMaxHeads];
  __shared__ int32_t merge_turn;

  const int64_t cap = a.slab_capacity;
  const int H = a.heads;
  const int L = a.cur_len;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;

  // The workgroup's unit: from the caller's work plan (a whole item or one
  // key-range part of a cut item, merged through the workspace as in the
  // 16-bit kernel), else the workgroup's item in longest-first order.
  WorkItem w;
  Unit un{0, 0, 1, 0, 0, 0};
  int32_t p0 = 0, p1 = 0;
  if (a.plan != nullptr) {
    const int32_t* pu = a.plan + static_cast<int64_t>(blockIdx.x) * kPlanInts;
    const int32_t ph = pu[0], pj = pu[1], pcut = pu[4], ppart = pu[5];
    p0 = pu[2];
    p1 = pu[3];
    if (ph < 0 || ph >= H || pj < 0 || pj >= a.batch * n_qt) return;  // not a unit of this launch
    w.h = ph;
    w.b = pj / n_qt;
    w.qt = pj - w.b * n_qt;
    w.bh = w.b * H + w.h;
    const bool cut = pcut >= 0 && a.workspace != nullptr && pcut < a.ws_cuts && ppart >= 0 && ppart < 2;
    un.part = cut ? ppart : 0;
    un.parts = cut ? 2 : 1;
    un.record = cut ? 2 * pcut : 0;
    un.counter = cut ? pcut : 0;
    un.arrive = cut && pu[7] != 0 ? 1 : 0;
    load_head_segments<kThreads>(a.seg_starts, a.seg_ends, a.seg_counts, cap, a.max_segments, w, seg_start,
                                 seg_pref);
  } else {
    w = plan_work<kThreads>(a.seg_starts, a.seg_ends, a.seg_counts, cap, H, a.max_segments, a.batch, n_qt,
                            head_rows, head_by_rank, seg_start, seg_pref, static_cast<int32_t>(blockIdx.x),
                            reinterpret_cast<int32_t*>(k_lds), sizeof(k_lds) / 4);
  }
  const int32_t R = w.R;
  const int32_t ntp = (R + kBN - 1) / kBN;
  const int32_t ntc = (L + kBN - 1) / kBN;
  const int32_t ntiles = ntp + ntc;
  const int32_t parts = un.parts;
  int32_t t_begin = 0, t_end = ntiles;
  if (parts > 1) {
    t_begin = p0 < 0 ? 0 : (p0 > ntiles ? ntiles : p0);
    t_end = p1 < t_begin ? t_begin : (p1 > ntiles ? ntiles : p1);
  }
  // the output staging of a merge reuses the K buffers once the last tile is done
  constexpr bool kStageOut = NQS * kKBytes >= NW * 32 * kOutPitch;

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
  // raw elements in flight, split into operand pieces when stored to LDS
  Raw8 lreg[kLoadsPerThread][4];
  auto load_row = [&](bool is_v, __amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv, int32_t row, int lc,
                      Raw8& dst) {
    if (is_v) dst = load_raw8<VDT>(rv, row < 0 ? -1 : (row * kD + lc * 8) * kEV);
    else dst = load_raw8<KDT>(rk, row < 0 ? -1 : (row * kD + lc * 8) * kEK);
  };
  auto issue_loads = [&](int tile, int buf) {
#pragma unroll
    for (int it = 0; it < kLoadsPerThread; ++it) {
      const int item = tid + it * kThreads;
      const bool is_v = item >= kQuadChunks;
      const int qc = is_v ? item - kQuadChunks : item;
      const int lq = qc >> 4;
      const int lc = qc & 15;
      if (tile < ntp) {
        const int4 rows = *reinterpret_cast<const int4*>(&rowtab[buf][lq * 4]);
        const int rr[4] = {rows.x, rows.y, rows.z, rows.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) load_row(is_v, rs_k, rs_v, rr[i], lc, lreg[it][i]);
      } else {
        const int row0 = (tile - ntp) * kBN;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = row0 + lq * 4 + i;
          load_row(is_v, rc_k, rc_v, row < L ? row : -1, lc, lreg[it][i]);
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
      if (!is_v) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          u32x4_t pc[NQS];
          pieces8<KDT, MQK, NQS>(lreg[it][i], pc);
#pragma unroll
          for (int p = 0; p < NQS; ++p)
            *reinterpret_cast<u32x4_t*>(k_lds + p * kKBytes + (lq * 4 + i) * kKPitch + lc * 16) = pc[p];
        }
      } else {
        u32x4_t r[4][NVS];
#pragma unroll
        for (int i = 0; i < 4; ++i) pieces8<VDT, MV, NVS>(lreg[it][i], r[i]);
        // transpose 4 keys x 8 d into 8 rows of V^T (4 keys each), per piece
#pragma unroll
        for (int p = 0; p < NVS; ++p)
#pragma unroll
          for (int wi = 0; wi < 4; ++wi) {
            u32x2_t even, odd;
            even[0] = __builtin_amdgcn_perm(r[1][p][wi], r[0][p][wi], 0x05040100u);
            even[1] = __builtin_amdgcn_perm(r[3][p][wi], r[2][p][wi], 0x05040100u);
            odd[0] = __builtin_amdgcn_perm(r[1][p][wi], r[0][p][wi], 0x07060302u);
            odd[1] = __builtin_amdgcn_perm(r[3][p][wi], r[2][p][wi], 0x07060302u);
            uint8_t* row = vt_lds + p * kVBytes + (lc * 8 + 2 * wi) * kVtPitch + lq * 8;
            *reinterpret_cast<u32x2_t*>(row) = even;
            *reinterpret_cast<u32x2_t*>(row + kVtPitch) = odd;
          }
      }
    }
  };

  // Q fragments (B operand of S^T = K Q^T): query row, d = 16ks + 8g .. +7
  const int32_t qrow = w.qt * kBM + wave * 32 + (lane & 31);
  u32x4_t qf[8][NQS];
  {
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(
        static_cast<const uint8_t*>(a.q) + cur_row0 * kD * kEQ, static_cast<uint32_t>(L * kD * kEQ));
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const int32_t off = qrow < L ? (qrow * kD + ks * 16 + g * 8) * kEQ : -1;
      pieces8<QDT, MQK, NQS>(load_raw8<QDT>(rq, off), qf[ks]);
#pragma unroll
      for (int p = 0; p < NQS; ++p) qf[ks][p] ^= sc.q_sign;
    }
  }

  f32x16_t oacc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) oacc[i] = f32x16_t{};
  float m_run = -1e30f;
  float l_run = 0.f;
  const uint8_t* k_lane = k_lds + (lane & 31) * kKPitch + g * 16;
  const uint8_t* v_lane = vt_lds + (lane & 31) * kVtPitch + g * 8;

  if (t_begin >= t_end) {
    // a planned part with no key tiles (a plan that does not match these
    // tables): its record is empty -- zero weight in the merge
    f32x16_t none[4] = {};
    merge_parts<QDT, kThreads, kStageOut>(a, sc, un, parts, none, -1e30f, 0.f, w, qrow, L, H, g, merge_turn,
                                          k_lds + wave * 32 * kOutPitch);
    return;
  }
  if (wave == 0 && t_begin < ntp)
    fill_rowtab(t_begin, rowtab[t_begin & 1], cur_seg, w.nseg, R, seg_start, seg_pref);
  __syncthreads();
  issue_loads(t_begin, t_begin & 1);
  if (wave == 0 && t_begin + 1 < ntp && t_begin + 1 < t_end)
    fill_rowtab(t_begin + 1, rowtab[(t_begin + 1) & 1], cur_seg, w.nseg, R, seg_start, seg_pref);

  for (int t = t_begin; t < t_end; ++t) {
    store_tile();
    __syncthreads();
    if (t + 1 < t_end) issue_loads(t + 1, (t + 1) & 1);
    if (wave == 0 && t + 2 < ntp && t + 2 < t_end)
      fill_rowtab(t + 2, rowtab[t & 1], cur_seg, w.nseg, R, seg_start, seg_pref);

    f32x16_t s[2] = {f32x16_t{}, f32x16_t{}};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        u32x4_t kf[NQS];
#pragma unroll
        for (int p = 0; p < NQS; ++p)
          kf[p] = *reinterpret_cast<const u32x4_t*>(k_lane + p * kKBytes + kb * 32 * kKPitch + ks * 32);
        s[kb] = mfma_split<MQK, NQS, NQS>(kf, qf[ks], s[kb]);
      }
    const int valid = t < ntp ? min(kBN, R - t * kBN) : min(kBN, L - (t - ntp) * kBN);
    softmax_tile(s, oacc, m_run, l_run, sc.c, sc.thresh, valid, g);
#pragma unroll
    for (int u = 0; u < kBN / 16; ++u) {
      u32x4_t pf[NPS];
      {
        const f32x16_t& sp = s[u >> 1];
        const int j0 = 8 * (u & 1);
        const float pv8[8] = {sp[j0 + 0], sp[j0 + 1], sp[j0 + 2], sp[j0 + 3],
                              sp[j0 + 4], sp[j0 + 5], sp[j0 + 6], sp[j0 + 7]};
        split8<MV, NPS>(pv8, pf);
      }
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        u32x4_t vf[NVS];
#pragma unroll
        for (int p = 0; p < NVS; ++p) {
          const uint8_t* row = v_lane + p * kVBytes + db * 32 * kVtPitch + 32 * u;
          const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(row);
          const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(row + 16);
          vf[p] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
        }
        oacc[db] = mfma_split<MV, NVS, NPS>(vf, pf, oacc[db]);
      }
    }
    __syncthreads();
  }
  if (parts == 1) {
    write_output(oacc, m_run, l_run, sc.c, a.out, a.lse, w.b, w.h, qrow, L, H, w.bh, g, a.out_dtype);
    return;
  }
  merge_parts<QDT, kThreads, kStageOut>(a, sc, un, parts, oacc, m_run, l_run, w, qrow, L, H, g, merge_turn,
                                        k_lds + wave * 32 * kOutPitch);
}

template <int QDT, int KDT, int VDT, int NQS, int NPS, int NVS>
hipError_t launch(const AttnArgs& a, const Scalars& s, hipStream_t st) {
  // 4-wave workgroups of 128 queries (the work plan's items).  The plain
  // modes fit 256 registers per wave: two workgroups per CU.  The split modes
  // hold more pieces in LDS and registers: one workgroup per CU, so a wave may
  // hold 512 registers (no spills).
  constexpr bool kPlain = NQS <= 2 && NPS == 1 && NVS == 1;
  constexpr int NW = 4;
  constexpr int MINB = kPlain ? 2 : 1;
  const int32_t n_qt = (a.cur_len + NW * 32 - 1) / (NW * 32);
  const int64_t blocks = static_cast<int64_t>(a.batch) * a.heads * n_qt;
  if (blocks <= 0) return hipSuccess;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  AttnArgs b = a;
  b.ws_cuts = 0;
  if (a.workspace != nullptr && a.workspace_bytes > kCounterBytes) {
    const int64_t by_records = (a.workspace_bytes - kCounterBytes) / (2LL * 66 * NW * 64 * 4);
    b.ws_cuts = static_cast<int32_t>(by_records < kMaxCounters ? by_records : kMaxCounters);
  }
  const int64_t grid = a.plan != nullptr ? a.plan_units : blocks;
  if (grid <= 0) return hipSuccess;
  seg_attn_staged_kernel<QDT, KDT, VDT, NQS, NPS, NVS, NW, MINB>
      <<<dim3(static_cast<uint32_t>(grid)), NW * 64, 0, st>>>(b, s, n_qt);
  return hipGetLastError();
}

// Piece counts of the P V product for value type VDT.
template <int QDT, int KDT, int VDT, int NQS>
hipError_t dispatch_pv(const AttnArgs& a, const Scalars& s, hipStream_t st) {
  if (a.value_dot_mode == kDotFp32) {
    constexpr int nv = VDT == kBF16 ? 1 : (VDT == kF16 ? 2 : 3);
    return launch<QDT, KDT, VDT, NQS, 3, nv>(a, s, st);
  }
  if constexpr (VDT == kF32) return launch<QDT, KDT, VDT, NQS, 2, 2>(a, s, st);
  else return launch<QDT, KDT, VDT, NQS, 1, 1>(a, s, st);
}

template <int QDT, int KDT, int NQS>
hipError_t dispatch_v(const AttnArgs& a, const Scalars& s, hipStream_t st) {
  switch (a.v_dtype) {
    case kBF16: return dispatch_pv<QDT, KDT, kBF16, NQS>(a, s, st);
    case kF16: return dispatch_pv<QDT, KDT, kF16, NQS>(a, s, st);
    case kF32: return dispatch_pv<QDT, KDT, kF32, NQS>(a, s, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_attention_staged(const AttnArgs& a, const attn::Scalars& s, hipStream_t stream) {
  if (a.q_dtype != a.k_dtype) return hipErrorInvalidValue;
  switch (a.q_dtype) {
    case kBF16: return dispatch_v<kBF16, kBF16, 1>(a, s, stream);
    case kF16: return dispatch_v<kF16, kF16, 1>(a, s, stream);
    case kF32:
      return a.qk_dot_mode == kDotFp32 ? dispatch_v<kF32, kF32, 3>(a, s, stream)
                                       : dispatch_v<kF32, kF32, 2>(a, s, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace hkv
