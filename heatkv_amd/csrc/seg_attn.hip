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
#include <cstdio>
#include <cstdlib>

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
constexpr int kKPitch = kD * 2 + 16;     // bytes per K row in LDS (16-byte pad: conflict-free reads)
constexpr float kLog2e = 1.4426950408889634f;
// Lazy rescale: the running max used for exp2 is only moved when a row's max
// grows by more than this (log2 units); p <= 2^8 stays exact in fp32 and is
// rounded like any other value to the 16-bit PV operand.
constexpr float kRescaleLog2 = 8.0f;
constexpr int kMaxHeads = 1024;

// ---------------------------------------------------------------- conversions
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// Two fp32 values -> one dword of two 16-bit values (round to nearest even);
// the vector conversion lowers to a single v_cvt_pk_{bf16,f16}_f32.
template <int MT>
__device__ __forceinline__ uint32_t pack2(float x, float y) {
  const f32x2_t v = {x, y};
  if constexpr (MT == kF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
__device__ __forceinline__ float f16_to_f32(uint16_t v) {
  return static_cast<float>(__builtin_bit_cast(_Float16, v));
}

// Buffer resource over [base, base + bytes): raw loads outside it return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes),
                                           0x00020000);
}

// Loads 8 consecutive elements of type DT at byte offset `off` of `r` and
// returns them as 8 packed 16-bit values of the MFMA operand type MT.  An
// offset of -1 (outside every resource) yields zeros without a branch.
template <int DT, int MT>
__device__ __forceinline__ u32x4_t load8(__amdgpu_buffer_rsrc_t r, int32_t off) {
  if constexpr (DT == kF32) {
    // Whole-vector bit casts: casting single elements of a buffer-load result
    // miscompiles with this toolchain (one dword loaded and replicated).
    const f32x4_t x = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
    const f32x4_t y = __builtin_bit_cast(
        f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off < 0 ? -1 : off + 16, 0, 0));
    u32x4_t o;
    o[0] = pack2<MT>(x[0], x[1]);
    o[1] = pack2<MT>(x[2], x[3]);
    o[2] = pack2<MT>(y[0], y[1]);
    o[3] = pack2<MT>(y[2], y[3]);
    return o;
  } else {
    u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    if constexpr (DT == kF16 && MT == kBF16) {
      // fp16 storage feeding a bf16 product (mixed q/k types): widen and round.
#pragma unroll
      for (int i = 0; i < 4; ++i)
        v[i] = pack2<kBF16>(f16_to_f32(static_cast<uint16_t>(v[i] & 0xffffu)),
                            f16_to_f32(static_cast<uint16_t>(v[i] >> 16)));
    }
    return v;
  }
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

// NW waves per workgroup (32 query rows each), BN keys per tile.
template <int QDT, int KDT, int VDT, int NW, int BN>
__global__ __launch_bounds__(NW * 64, (NW == 4 && BN == 128) ? 1 : 2) void seg_attn_kernel(
    const AttnArgs a, const float c, const float scale_abs, const uint32_t q_sign,
    const int32_t n_qt) {
  constexpr int MQK = (QDT == kF16 && KDT == kF16) ? kF16 : kBF16;
  constexpr int MV = (VDT == kF16) ? kF16 : kBF16;
  constexpr int kThreads = NW * 64;
  constexpr int kBM = NW * 32;
  constexpr int kVtPitch = BN * 2 + 8;      // bytes per V^T row (8-byte pad: conflict-free reads)
  constexpr int kSB = BN / 32;              // 32-key score blocks per tile
  constexpr int kQuadChunks = BN / 4 * 16;  // (4-key quad, 16-byte d-chunk) pairs per tensor
  constexpr int kLoadsPerThread = 2 * kQuadChunks / kThreads;
  constexpr int kEK = KDT == kF32 ? 4 : 2;  // element bytes
  constexpr int kEV = VDT == kF32 ? 4 : 2;
  constexpr int kEQ = QDT == kF32 ? 4 : 2;
  static_assert(2 * kQuadChunks % kThreads == 0, "loader split");

  __shared__ __attribute__((aligned(16))) uint8_t k_lds[BN * kKPitch];
  __shared__ __attribute__((aligned(16))) uint8_t vt_lds[kD * kVtPitch];
  __shared__ __attribute__((aligned(16))) int32_t rowtab[2][BN];
  __shared__ int32_t seg_start[kMaxSegments];
  __shared__ int32_t seg_pref[kMaxSegments + 1];
  __shared__ int32_t head_rows[kMaxHeads];
  __shared__ int32_t head_by_rank[kMaxHeads];

  // Kernel arguments copied to locals once (keeps them in SGPRs).
  const int32_t* __restrict__ seg_starts = a.seg_starts;
  const int32_t* __restrict__ seg_ends = a.seg_ends;
  const int32_t* __restrict__ seg_counts = a.seg_counts;
  const int64_t cap = a.slab_capacity;
  const int H = a.heads;
  const int L = a.cur_len;
  const int S = a.max_segments;
  const int B = a.batch;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;  // half of the wave: selects the k-slot group of MFMA operands

  // ---- longest-first order of heads: every head's retained rows, then ranks
  for (int hh = tid; hh < H; hh += kThreads) {
    int n = seg_counts[hh];
    n = n < 0 ? 0 : (n > S ? S : n);
    int64_t rows = 0;
    for (int i = 0; i < n; ++i) {
      int64_t st = seg_starts[static_cast<int64_t>(hh) * S + i];
      int64_t en = seg_ends[static_cast<int64_t>(hh) * S + i];
      st = st < 0 ? 0 : (st > cap ? cap : st);
      en = en < 0 ? 0 : (en > cap ? cap : en);
      rows += en > st ? en - st : 0;
    }
    head_rows[hh] = static_cast<int32_t>(rows);
  }
  __syncthreads();
  for (int hh = tid; hh < H; hh += kThreads) {
    const int r = head_rows[hh];
    int rank = 0;
    for (int o = 0; o < H; ++o) {
      const int ro = head_rows[o];
      rank += (ro > r) || (ro == r && o < hh);
    }
    head_by_rank[rank] = hh;
  }
  __syncthreads();

  // ---- work item: heaviest heads first (workgroups start in id order, so the
  // dispatcher's greedy slot filling approximates longest-processing-time)
  const int32_t per_rank = B * n_qt;
  const int32_t rank = blockIdx.x / per_rank;
  const int32_t rem = blockIdx.x - rank * per_rank;
  const int32_t b = rem / n_qt;
  const int32_t qt = rem - b * n_qt;
  const int32_t h = head_by_rank[rank];
  const int32_t bh = b * H + h;

  // ---- segment table of head h: clamped starts and exclusive length prefix
  int nseg = seg_counts[h];
  nseg = nseg < 0 ? 0 : (nseg > S ? S : nseg);
  for (int i = tid; i < nseg; i += kThreads) {
    int64_t st = seg_starts[static_cast<int64_t>(h) * S + i];
    int64_t en = seg_ends[static_cast<int64_t>(h) * S + i];
    st = st < 0 ? 0 : (st > cap ? cap : st);
    en = en < 0 ? 0 : (en > cap ? cap : en);
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
  // Key stream: ntp tiles of retained prior rows (the last one padded), then
  // ntc tiles of current rows; every tile reads one tensor only.
  const int32_t R = seg_pref[nseg];
  const int32_t ntp = (R + BN - 1) / BN;
  const int32_t ntc = (L + BN - 1) / BN;
  const int32_t ntiles = ntp + ntc;

  // Buffer resources: batch b's slab rows and (b, h)'s current rows.
  const __amdgpu_buffer_rsrc_t rs_k = make_rsrc(
      static_cast<const uint8_t*>(a.slab_k) + static_cast<int64_t>(b) * cap * kD * kEK,
      static_cast<uint32_t>(cap * kD * kEK));
  const __amdgpu_buffer_rsrc_t rs_v = make_rsrc(
      static_cast<const uint8_t*>(a.slab_v) + static_cast<int64_t>(b) * cap * kD * kEV,
      static_cast<uint32_t>(cap * kD * kEV));
  const int64_t cur_row0 = static_cast<int64_t>(bh) * L;
  const __amdgpu_buffer_rsrc_t rc_k = make_rsrc(
      static_cast<const uint8_t*>(a.cur_k) + cur_row0 * kD * kEK, static_cast<uint32_t>(L * kD * kEK));
  const __amdgpu_buffer_rsrc_t rc_v = make_rsrc(
      static_cast<const uint8_t*>(a.cur_v) + cur_row0 * kD * kEV, static_cast<uint32_t>(L * kD * kEV));

  // ---- row table of a prior tile: stream position -> slab row, -1 past R
  int cur_seg = 0;
  auto fill_rowtab = [&](int tile, int buf) {
    const int j0 = tile * BN;
    while (cur_seg < nseg && seg_pref[cur_seg + 1] <= j0) ++cur_seg;
#pragma unroll
    for (int part = 0; part < BN / 64; ++part) {
      const int j = j0 + part * 64 + lane;
      int row = -1;
      if (j < R) {
        int s = cur_seg;
        while (seg_pref[s + 1] <= j) ++s;
        row = seg_start[s] + (j - seg_pref[s]);
      }
      rowtab[buf][part * 64 + lane] = row;
    }
  };

  // ---- loader: quad-chunk i covers keys 4(i/16)..+3 at d 8(i%16)..+7 of K (i <
  // kQuadChunks) or of V; thread tid owns quad-chunks tid, tid + kThreads, ...
  u32x4_t lreg[kLoadsPerThread][4];
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
          else
            lreg[it][i] = load8<KDT, MQK>(rs_k, rr[i] < 0 ? -1 : (rr[i] * kD + lc * 8) * kEK);
        }
      }
    } else {
      const int row0 = (tile - ntp) * BN;
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
        for (int i = 0; i < 4; ++i)
          *reinterpret_cast<u32x4_t*>(k_lds + (lq * 4 + i) * kKPitch + lc * 16) = r[i];
      } else {
        // transpose 4 keys x 8 d into 8 rows of V^T (4 keys each)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          u32x2_t even, odd;
          even[0] = __builtin_amdgcn_perm(r[1][w], r[0][w], 0x05040100u);
          even[1] = __builtin_amdgcn_perm(r[3][w], r[2][w], 0x05040100u);
          odd[0] = __builtin_amdgcn_perm(r[1][w], r[0][w], 0x07060302u);
          odd[1] = __builtin_amdgcn_perm(r[3][w], r[2][w], 0x07060302u);
          uint8_t* row = vt_lds + (lc * 8 + 2 * w) * kVtPitch + lq * 8;
          *reinterpret_cast<u32x2_t*>(row) = even;
          *reinterpret_cast<u32x2_t*>(row + kVtPitch) = odd;
        }
      }
    }
  };

  // ---- Q fragments (B operand of S^T = K Q^T): query row, d = 16ks + 8g .. +7
  const int32_t qrow = qt * kBM + wave * 32 + (lane & 31);
  const bool qvalid = qrow < L;
  u32x4_t qf[8];
  {
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(
        static_cast<const uint8_t*>(a.q) + cur_row0 * kD * kEQ, static_cast<uint32_t>(L * kD * kEQ));
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      qf[ks] = load8<QDT, MQK>(rq, qvalid ? (qrow * kD + ks * 16 + g * 8) * kEQ : -1);
      qf[ks] ^= q_sign;  // negative softmax scale: exact sign flip of q
    }
  }

  f32x16_t oacc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) oacc[i] = f32x16_t{};
  float m_run = -1e30f;  // reference max of raw scores (sign-adjusted) used by exp2
  float l_run = 0.f;     // this lane's partial row sum
  const float thresh = c > 0.f ? kRescaleLog2 / c : 0.f;

  // LDS operand addresses: lane part here, the rest are immediates.
  const uint8_t* k_lane = k_lds + (lane & 31) * kKPitch + g * 16;
  const uint8_t* v_lane = vt_lds + (lane & 31) * kVtPitch + g * 8;

  if (wave == 0 && ntp > 0) fill_rowtab(0, 0);
  __syncthreads();
  issue_loads(0, 0);
  if (wave == 0 && 1 < ntp) fill_rowtab(1, 1);

  for (int t = 0; t < ntiles; ++t) {
    store_tile();
    __syncthreads();
    if (t + 1 < ntiles) issue_loads(t + 1, (t + 1) & 1);
    if (wave == 0 && t + 2 < ntp) fill_rowtab(t + 2, t & 1);

    // S^T block kb: keys 32kb + (8(j>>2) + 4g + (j&3)), query lane&31
    f32x16_t s[kSB];
#pragma unroll
    for (int kb = 0; kb < kSB; ++kb) s[kb] = f32x16_t{};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
#pragma unroll
      for (int kb = 0; kb < kSB; ++kb) {
        const u32x4_t kf = *reinterpret_cast<const u32x4_t*>(k_lane + kb * 32 * kKPitch + ks * 32);
        s[kb] = mfma32<MQK>(kf, qf[ks], s[kb]);
      }
    }
    // keys of this tile that exist: prior tiles end at R, current tiles at L
    const int valid_keys = t < ntp ? min(BN, R - t * BN) : min(BN, L - (t - ntp) * BN);
    const bool partial = valid_keys < BN;
    if (partial) {
#pragma unroll
      for (int kb = 0; kb < kSB; ++kb)
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (kb * 32 + 8 * (j >> 2) + 4 * g + (j & 3) >= valid_keys) s[kb][j] = -__builtin_inff();
    }
    float mx = s[0][0];
#pragma unroll
    for (int kb = 0; kb < kSB; ++kb)
#pragma unroll
      for (int j = 0; j < 16; ++j) mx = fmaxf(mx, s[kb][j]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    // Move the reference max only when some row of the wave grew past the
    // threshold (always on the first tile, where m_run is -1e30).
    if (__any(mx - m_run > thresh)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) oacc[db] *= alpha;
      m_run = m_new;
    }
    const float mc = m_run * c;
#pragma unroll
    for (int kb = 0; kb < kSB; ++kb)
#pragma unroll
      for (int j = 0; j < 16; ++j) s[kb][j] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][j], c, -mc));
    if (partial) {
#pragma unroll
      for (int kb = 0; kb < kSB; ++kb)
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (kb * 32 + 8 * (j >> 2) + 4 * g + (j & 3) >= valid_keys) s[kb][j] = 0.f;
    }
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < kSB; ++kb)
#pragma unroll
      for (int j = 0; j < 16; ++j) psum += s[kb][j];
    l_run += psum;

    // O^T += V^T P^T: k-step u covers keys 16u + {4g..4g+3, 8+4g..8+4g+3}
#pragma unroll
    for (int u = 0; u < BN / 16; ++u) {
      const f32x16_t& sp = s[u >> 1];
      const int j0 = 8 * (u & 1);
      u32x4_t pf;
      pf[0] = pack2<MV>(sp[j0 + 0], sp[j0 + 1]);
      pf[1] = pack2<MV>(sp[j0 + 2], sp[j0 + 3]);
      pf[2] = pack2<MV>(sp[j0 + 4], sp[j0 + 5]);
      pf[3] = pack2<MV>(sp[j0 + 6], sp[j0 + 7]);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const uint8_t* row = v_lane + db * 32 * kVtPitch + 32 * u;
        const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(row);
        const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(row + 16);
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

struct Variant {
  int nw;
  int bn;
};

// Tile shape: waves per workgroup x keys per tile.  HKV_ATTN_VARIANT (read
// once) selects another compiled shape for tuning sweeps: "4x64", "8x64",
// "4x128" (one wave per SIMD, accumulators in AGPRs).
Variant variant() {
  static Variant v = [] {
    Variant r{4, 64};
    if (const char* e = std::getenv("HKV_ATTN_VARIANT")) {
      int nw = 0, bn = 0;
      if (std::sscanf(e, "%dx%d", &nw, &bn) == 2 &&
          ((nw == 4 && (bn == 64 || bn == 128)) || (nw == 8 && bn == 64)))
        r = Variant{nw, bn};
    }
    return r;
  }();
  return v;
}

template <int QDT, int KDT, int VDT>
hipError_t launch_shape(const AttnArgs& a, float c, float sabs, uint32_t qs, hipStream_t st) {
  const Variant v = variant();
  const int32_t bm = v.nw * 32;
  const int32_t n_qt = (a.cur_len + bm - 1) / bm;
  const int64_t blocks = static_cast<int64_t>(a.batch) * a.heads * n_qt;
  if (blocks <= 0) return hipSuccess;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  const dim3 grid(static_cast<uint32_t>(blocks));
  if (v.nw == 4 && v.bn == 64)
    seg_attn_kernel<QDT, KDT, VDT, 4, 64><<<grid, 256, 0, st>>>(a, c, sabs, qs, n_qt);
  else if (v.nw == 8 && v.bn == 64)
    seg_attn_kernel<QDT, KDT, VDT, 8, 64><<<grid, 512, 0, st>>>(a, c, sabs, qs, n_qt);
  else
    seg_attn_kernel<QDT, KDT, VDT, 4, 128><<<grid, 256, 0, st>>>(a, c, sabs, qs, n_qt);
  return hipGetLastError();
}

template <int QDT, int KDT>
hipError_t dispatch_v(const AttnArgs& a, float c, float sabs, uint32_t qs, hipStream_t st) {
  switch (a.v_dtype) {
    case kBF16: return launch_shape<QDT, KDT, kBF16>(a, c, sabs, qs, st);
    case kF16: return launch_shape<QDT, KDT, kF16>(a, c, sabs, qs, st);
    case kF32: return launch_shape<QDT, KDT, kF32>(a, c, sabs, qs, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_segmented_attention(const AttnArgs& a, hipStream_t stream) {
  if (a.heads > kMaxHeads) return hipErrorInvalidValue;
  const float sabs = a.softmax_scale < 0.f ? -a.softmax_scale : a.softmax_scale;
  const float c = sabs * kLog2e;
  const uint32_t qs = a.softmax_scale < 0.f ? 0x80008000u : 0u;
  if (a.q_dtype != a.k_dtype) return hipErrorInvalidValue;
  switch (a.q_dtype) {
    case kBF16: return dispatch_v<kBF16, kBF16>(a, c, sabs, qs, stream);
    case kF16: return dispatch_v<kF16, kF16>(a, c, sabs, qs, stream);
    case kF32: return dispatch_v<kF32, kF32>(a, c, sabs, qs, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace hkv
