// Segmented attention for fp32 q and k with 16-bit V at the default dot modes:
// split-bf16 products fed by DMA, software-pipelined.
//
// K arrives as split rows (dtype code kSplitRows): each row of 128 fp32
// values is stored as its 128 bf16 high parts, then its 128 bf16 low parts
// (hi = x rounded to bf16, lo = (x - hi) rounded to bf16; 512 bytes, the size
// of the fp32 row).  split_rows_kernel writes them from fp32 rows; q is split
// the same way when it is loaded.  S = Kh Qh + Kh Ql + Kl Qh then carries
// about 16 significand bits, as the register-staged kernel's 2-piece split
// (seg_attn_staged.hip) does, without re-splitting every K tile for every
// query tile.
//
// Layout and schedule (CDNA4, wave64), one workgroup of 8 waves x 32 queries
// (256 queries of one (b, h)) per CU:
//  * A 64-key tile moves global -> LDS with buffer_load_dwordx4 ... lds in
//    MFMA-operand order: the hi plane and the lo plane of K (16 KiB each, the
//    16-bit kernel's K block order) and V (16 KiB, the 16-bit kernel's V
//    order, read with ds_read_b64_tr_b16).  K has two stages, V three slots:
//    112 KiB.
//  * The software pipeline runs on 32-key halves: half j+1's 24 QK MFMAs
//    (8 k-steps x 3 products) are issued while the VALU turns half j's
//    scores into P, then half j's 8 PV MFMAs while the VALU takes half j+1's
//    row max.  Two S halves of 16 registers each, so both q pieces (64
//    registers) and O (64) fit 256 registers per wave.
//  * K of tile T is read by the half steps 2T - 1 and 2T, V of tile T by 2T
//    and 2T + 1.  Step 2T + 1 waits for tile T + 1 (issued two half steps
//    earlier), passes the tile's one barrier, which retires every read of
//    K(T) and V(T - 1), and issues K and V of tile T + 2 into their places:
//    each tile lands at least two half steps before its first use, and the
//    even half steps neither wait nor synchronize.
// Semantics as the other attention kernels (attn_common.h): online softmax in
// the exp2 domain with the lazy rescale, P rounded to V's type, current-scale
// tiles first, then the retained prior rows through the row tables.
#include "attn_common.h"

#include <type_traits>

namespace hkv {
namespace {

using namespace attn;

constexpr int kSW = 8;                           // waves per workgroup
constexpr int kSThreads = kSW * 64;
constexpr int kSBM = kSW * 32;                   // queries per item
constexpr int kSPlane = kBN * kD * 2;            // 16 KiB: one plane of a K tile
constexpr int kSKStage = 2 * kSPlane;            // K hi and lo planes of a tile
constexpr int kSVBase = 2 * kSKStage;            // V slots after the two K stages
constexpr int kSRing = kSVBase + 3 * kSPlane;    // 2 K stages + 3 V slots: 112 KiB
constexpr int kSRowBytes = 2 * kD * 2;           // a split K row
constexpr int kVRowBytes = kD * 2;               // a 16-bit V row
constexpr int32_t kPastEnd = static_cast<int32_t>(0x80000000u);

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t* lds_s16x4_ptr;
typedef __attribute__((address_space(3))) void* lds_void_ptr;

__device__ __forceinline__ u32x2_t ds_read_tr(const uint8_t* p) {
  return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(p)));
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_ptr)(p)));
}

// 16 bytes per lane from a buffer straight to LDS at `lds_addr` + 16 lane
// (see seg_attn_direct.hip: inline assembly so that LDS reads are not made
// to wait for every outstanding load; M0 is used by nothing else here).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const u32x4_t rsrc, uint32_t lds_addr, int32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voff), "s"(rsrc)
               : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ u32x4_t make_desc(const void* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  u32x4_t d;
  d[0] = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p));
  d[1] = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p >> 32) & 0xffffu);
  d[2] = __builtin_amdgcn_readfirstlane(bytes);
  d[3] = 0x00020000u;
  return d;
}

// Keys of half kb (32kb .. 32kb + 31) at or past `valid_keys` (of the tile) get -inf.
__device__ __forceinline__ void mask_half(f32x16_t& s, int kb, int valid_keys, int g) {
  const int lim = valid_keys - 32 * kb - 4 * g;
#pragma unroll
  for (int j = 0; j < 16; ++j)
    if (8 * (j >> 2) + (j & 3) >= lim) s[j] = -__builtin_inff();
}

__device__ __forceinline__ float half_max(const f32x16_t& s) {
  float mx = s[0];
#pragma unroll
  for (int j = 1; j < 16; ++j) mx = fmaxf(mx, s[j]);
  return pair_max(mx);
}

// p = exp2(c (s - m)) in place, l_run += sum of p (fp32, unrounded).
__device__ __forceinline__ void exp_half(f32x16_t& s, float m_run, float c, float& l_run) {
  const float mc = m_run * c;
#pragma unroll
  for (int j = 0; j < 16; ++j) s[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j], c, -mc));
  float p0 = s[0], p1 = s[8];
#pragma unroll
  for (int j = 1; j < 8; ++j) {
    p0 += s[j];
    p1 += s[8 + j];
  }
  l_run += p0 + p1;
}

// fp32 rows -> split rows: 16 threads per row, 8 values each.
__global__ __launch_bounds__(256) void split_rows_kernel(const float* __restrict__ src, uint8_t* __restrict__ dst,
                                                         int64_t rows) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t row = i >> 4;
  if (row >= rows) return;
  const int c = static_cast<int>(i & 15);
  const f32x4_t x = *reinterpret_cast<const f32x4_t*>(src + row * kD + c * 8);
  const f32x4_t y = *reinterpret_cast<const f32x4_t*>(src + row * kD + c * 8 + 4);
  const float v[8] = {x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
  u32x4_t hi, lo;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    hi[k] = pack2<kBF16>(v[2 * k], v[2 * k + 1]);
    const float h0 = __builtin_bit_cast(float, hi[k] << 16);
    const float h1 = __builtin_bit_cast(float, hi[k] & 0xffff0000u);
    lo[k] = pack2<kBF16>(v[2 * k] - h0, v[2 * k + 1] - h1);
  }
  uint8_t* const out = dst + row * kSRowBytes;
  *reinterpret_cast<u32x4_t*>(out + c * 16) = hi;
  *reinterpret_cast<u32x4_t*>(out + kD * 2 + c * 16) = lo;
}

template <int VDT>
__global__ __launch_bounds__(kSThreads, 1) void seg_attn_split_kernel(const int32_t* __restrict__ plan_p,
                                                                     const int32_t n_units, const AttnArgs a,
                                                                     const Scalars sc,
                                                                     const int32_t n_qt) {
  constexpr int kThreads = kSThreads;
  constexpr int kBM = kSBM;
  constexpr int MV = VDT;
  __shared__ __attribute__((aligned(1024))) uint8_t ring[kSRing];
  __shared__ __attribute__((aligned(16))) int32_t rowtab[3][kBN];
  __shared__ int32_t seg_start[kMaxSegments];
  __shared__ int32_t seg_pref[kMaxSegments + 1];
  __shared__ int32_t merge_turn;
  static_assert(kSRing >= kSW * 32 * kOutPitch, "output staging fits the ring");

  const int64_t cap = a.slab_capacity;
  const int H = a.heads;
  const int L = a.cur_len;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform by construction
  const int g = lane >> 5;
  // This workgroup's plan unit, loaded with the kernel arguments: the plan
  // pointer and unit count are preloaded into SGPRs (as in the 16-bit
  // kernel).
  int32_t pu[kPlanInts] = {};
  const bool planned = plan_p != nullptr && static_cast<int32_t>(blockIdx.x) < n_units;
  if (planned) {
    const int32_t* src = plan_p + static_cast<int64_t>(blockIdx.x) * kPlanInts;
#pragma unroll
    for (int i = 0; i < kPlanInts; ++i) pu[i] = src[i];
  }

  // The unit: from the caller's work plan (a whole item or one key-range
  // part of a cut item, merged through the workspace), else the workgroup's
  // item in longest-first order.
  WorkItem w;
  Unit un{0, 0, 1, 0, 0, 0};
  int32_t p0 = 0, p1 = 0;
  if (planned) {
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
    int32_t* head_rows = reinterpret_cast<int32_t*>(ring);
    w = plan_work<kThreads>(a.seg_starts, a.seg_ends, a.seg_counts, cap, H, a.max_segments, a.batch, n_qt,
                            head_rows, head_rows + kMaxHeads, seg_start, seg_pref,
                            static_cast<int32_t>(blockIdx.x), head_rows + 2 * kMaxHeads,
                            kSRing / 4 - 2 * kMaxHeads);
  }
  const int32_t R = w.R;
  const int32_t ntc = (L + kBN - 1) / kBN;
  const int32_t ntiles = (R + kBN - 1) / kBN + ntc;
  const int32_t parts = un.parts;
  int32_t tb = 0, te = ntiles;
  if (parts > 1) {
    tb = p0 < 0 ? 0 : (p0 > ntiles ? ntiles : p0);
    te = p1 < tb ? tb : (p1 > ntiles ? ntiles : p1);
  }
  const int32_t qrow = w.qt * kBM + wave * 32 + (lane & 31);
  if (tb >= te) {
    // a planned part with no key tiles (a plan that does not match these
    // tables): its record is empty -- zero weight in the merge
    f32x16_t none[4] = {};
    merge_parts<kF32, kThreads>(a, sc, un, parts, none, -1e30f, 0.f, w, qrow, L, H, g, merge_turn,
                                ring + wave * 32 * kOutPitch);
    return;
  }

  // Descriptors: K split rows and V rows of the slab (batch row b) and of
  // the current scale (b, h).
  const int64_t cur_row0 = static_cast<int64_t>(w.bh) * L;
  const u32x4_t dk_prior = make_desc(static_cast<const uint8_t*>(a.slab_k) + w.b * cap * kSRowBytes,
                                     static_cast<uint32_t>(cap * kSRowBytes));
  const u32x4_t dv_prior = make_desc(static_cast<const uint8_t*>(a.slab_v) + w.b * cap * kVRowBytes,
                                     static_cast<uint32_t>(cap * kVRowBytes));
  const uint8_t* const k_cur = static_cast<const uint8_t*>(a.cur_k) + cur_row0 * kSRowBytes;
  const uint8_t* const v_cur = static_cast<const uint8_t*>(a.cur_v) + cur_row0 * kVRowBytes;

  // This wave's DMA share of a tile: K blocks 4 wave .. + 3 (blocks 0..15 of
  // the hi plane, 16..31 of the lo plane) and V chunks 2 wave, 2 wave + 1.
  int k_key[4], k_col[4], v_key[2], v_col[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = 4 * wave + i;
    const int blk = q & 15;
    k_key[i] = (blk >> 3) * 32 + (lane & 31);
    k_col[i] = (q >> 4) * (kD * 2) + (blk & 7) * 32 + (lane >> 5) * 16;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int qv = 2 * wave + i;
    const int lp = lane & 31;
    const int db = 2 * (qv & 1) + (lane >> 5);
    v_key[i] = 16 * (qv >> 2) + 8 * ((qv >> 1) & 1) + 4 * (lp >> 4) + ((lp & 7) >> 1);
    v_col[i] = 2 * (db * 32 + 16 * ((lp >> 3) & 1) + 8 * (lp & 1));
  }
  const uint32_t ring_lds = lds_address(ring);

  auto issue_k = [&](int T) {
    const uint32_t dst = ring_lds + (T & 1) * kSKStage + wave * 4 * 1024;
    if (T < ntc) {
      const uint32_t skip = static_cast<uint32_t>(T) * (kBN * kSRowBytes);
      const u32x4_t d = make_desc(k_cur + skip, static_cast<uint32_t>(L) * kSRowBytes - skip);
#pragma unroll
      for (int i = 0; i < 4; ++i) dma16(d, dst + i * 1024, k_key[i] * kSRowBytes + k_col[i]);
    } else {
      const int32_t* rt = rowtab[(T - ntc) % 3];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int32_t row = rt[k_key[i]];
        dma16(dk_prior, dst + i * 1024, row < 0 ? kPastEnd : row * kSRowBytes + k_col[i]);
      }
    }
  };
  auto issue_v = [&](int T) {
    const uint32_t dst = ring_lds + kSVBase + (T % 3) * kSPlane + wave * 2 * 1024;
    if (T < ntc) {
      const uint32_t skip = static_cast<uint32_t>(T) * (kBN * kVRowBytes);
      const u32x4_t d = make_desc(v_cur + skip, static_cast<uint32_t>(L) * kVRowBytes - skip);
#pragma unroll
      for (int i = 0; i < 2; ++i) dma16(d, dst + i * 1024, v_key[i] * kVRowBytes + v_col[i]);
    } else {
      const int32_t* rt = rowtab[(T - ntc) % 3];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int32_t row = rt[v_key[i]];
        dma16(dv_prior, dst + i * 1024, row < 0 ? kPastEnd : row * kVRowBytes + v_col[i]);
      }
    }
  };
  auto valid_of = [&](int T) { return T < ntc ? min(kBN, L - T * kBN) : min(kBN, R - (T - ntc) * kBN); };
  int cur_seg = 0;
  auto fill = [&](int T) {  // wave 0: row table of tile T (a prior-row tile)
    if (T >= ntc && T < te)
      fill_rowtab<1>(T - ntc, rowtab[(T - ntc) % 3], cur_seg, w.nseg, R, seg_start, seg_pref, -1);
  };

  // Q in two bf16 pieces: B operands of S^T = K Q^T (query row, d = 16ks + 8g .. +7)
  u32x4_t qh[8], ql[8];
  {
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(static_cast<const uint8_t*>(a.q) + cur_row0 * kD * 4,
                                                static_cast<uint32_t>(L * kD * 4));
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
      load8_split(rq, qrow < L ? (qrow * kD + ks * 16 + g * 8) * 4 : -1, qh[ks], ql[ks]);
  }
  if (wave == 0) {
    fill(tb);
    fill(tb + 1);
  }
  __syncthreads();
  issue_k(tb);
  issue_v(tb);
  if (tb + 1 < te) {
    issue_k(tb + 1);
    issue_v(tb + 1);
  }
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    qh[ks] ^= sc.q_sign;
    ql[ks] ^= sc.q_sign;
  }

  f32x16_t oacc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) oacc[i] = f32x16_t{};
  float m_run = -1e30f;
  float l_run = 0.f;

  // S^T of half j (keys 32 (j & 1) .. of tile j >> 1) from its stage
  auto qk = [&](f32x16_t& s, int j) {
    const uint8_t* kst = ring + ((j >> 1) & 1) * kSKStage + (j & 1) * 8 * 1024 + lane * 16;
    s = f32x16_t{};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const u32x4_t kh = *reinterpret_cast<const u32x4_t*>(kst + ks * 1024);
      const u32x4_t kl = *reinterpret_cast<const u32x4_t*>(kst + kSPlane + ks * 1024);
      s = mfma32<kBF16>(kh, qh[ks], s);
      s = mfma32<kBF16>(kh, ql[ks], s);
      s = mfma32<kBF16>(kl, qh[ks], s);
    }
  };
  // O^T += V^T P^T over half j's keys (k-steps u = 2 (j & 1), + 1)
  auto pv = [&](const f32x16_t& s, int j) {
    const uint8_t* vst = ring + kSVBase + ((j >> 1) % 3) * kSPlane + lane * 8;
#pragma unroll
    for (int ul = 0; ul < 2; ++ul) {
      u32x4_t pf;
      pf[0] = pack2<MV>(s[8 * ul + 0], s[8 * ul + 1]);
      pf[1] = pack2<MV>(s[8 * ul + 2], s[8 * ul + 3]);
      pf[2] = pack2<MV>(s[8 * ul + 4], s[8 * ul + 5]);
      pf[3] = pack2<MV>(s[8 * ul + 6], s[8 * ul + 7]);
      const int u = 2 * (j & 1) + ul;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int blk = (db >> 1) * 1024 + (db & 1) * 512;
        const u32x2_t lo = ds_read_tr(vst + (u * 4 + 0) * 1024 + blk);
        const u32x2_t hi = ds_read_tr(vst + (u * 4 + 2) * 1024 + blk);
        const u32x4_t vf = {lo[0], lo[1], hi[0], hi[1]};
        oacc[db] = mfma32<MV>(vf, pf, oacc[db]);
      }
    }
  };
  auto masked_max = [&](f32x16_t& s, int j) {
    float mx = half_max(s);
    asm volatile("" : "+v"(mx));
    const int v = valid_of(j >> 1);
    if (v < 32 * ((j & 1) + 1)) {
      mask_half(s, j & 1, v, g);
      mx = half_max(s);
    }
    return mx;
  };

  // Prologue: tile tb landed (tile tb + 1 may be in flight: 6 DMAs per wave); S of half 2 tb and its max.
  if (tb + 1 < te) wait_vmcnt<6>();
  else wait_vmcnt<0>();
  __syncthreads();
  f32x16_t sa, sb;
  qk(sa, 2 * tb);
  move_max(oacc, m_run, l_run, masked_max(sa, 2 * tb), sc.c, sc.thresh);

  const int jend = 2 * te;
  // Half step j: scur = S(j) (max applied), snext receives S(j + 1) unless j
  // is the item's last half (kMore false: peeled, so that the steps of the
  // loop have no branch between their MFMAs and their softmax).
  auto step = [&](auto more_tag, f32x16_t& scur, f32x16_t& snext, int j) {
    constexpr bool kMore = decltype(more_tag)::value;
    const int T = j >> 1;
    // Waves w and w + 4 share a SIMD, whose issue favours the older wave:
    // left alone, waves 0-3 finish each tile ~1.1 us ahead and wait at its
    // barrier while waves 4-7 run one to a SIMD.  Raising waves 0-3 in the
    // even half steps and waves 4-7 in the odd ones (which start at the
    // barrier) keeps the pairs within ~0.3 us (-1.8 % on the 2B final step
    // at the model's precision).
    if (((j + (wave >> 2)) & 1) == 0)
      __builtin_amdgcn_s_setprio(1);
    else
      __builtin_amdgcn_s_setprio(0);
    if ((j & 1) == 0) {
      // tile T landed at step 2T - 1 (or in the prologue): no wait here
      if (wave == 0) fill(T + 2);
    } else {
      // tile T + 1 (the next half's K, the next step's V), issued two half
      // steps ago, is the only one in flight; after the barrier every read
      // of K(T) and V(T - 1) is done, so tile T + 2 takes their places
      wait_vmcnt<0>();
      __syncthreads();
      if (T + 2 < te) {
        issue_k(T + 2);
        issue_v(T + 2);
      }
    }
    if constexpr (kMore) qk(snext, j + 1);
    exp_half(scur, m_run, sc.c, l_run);
    pv(scur, j);
    if constexpr (kMore) {
      asm volatile("" : "+v"(l_run));
      move_max(oacc, m_run, l_run, masked_max(snext, j + 1), sc.c, sc.thresh);
    }
  };
  using More = std::integral_constant<bool, true>;
  using Last = std::integral_constant<bool, false>;
  int j = 2 * tb;
  for (; j + 2 < jend; j += 2) {
    step(More{}, sa, sb, j);
    step(More{}, sb, sa, j + 1);
  }
  step(More{}, sa, sb, j);
  step(Last{}, sb, sa, j + 1);
  __builtin_amdgcn_s_setprio(0);

  if (parts == 1) {
    if (a.out_dtype != kF32 && (reinterpret_cast<uintptr_t>(a.out) & 15) == 0) {
      __syncthreads();  // every wave is past its last tile: the ring is free
      uint8_t* const stage = ring + wave * 32 * kOutPitch;
      const int32_t qrow0 = w.qt * kBM + wave * 32;
      if (a.out_dtype == kF16)
        write_output_lds<kF16>(oacc, m_run, l_run, sc.c, a.out, a.lse, w.b, w.h, qrow0, L, H, w.bh, lane, stage);
      else
        write_output_lds<kBF16>(oacc, m_run, l_run, sc.c, a.out, a.lse, w.b, w.h, qrow0, L, H, w.bh, lane, stage);
    } else {
      write_output(oacc, m_run, l_run, sc.c, a.out, a.lse, w.b, w.h, qrow, L, H, w.bh, g, a.out_dtype);
    }
    return;
  }
  merge_parts<kF32, kThreads>(a, sc, un, parts, oacc, m_run, l_run, w, qrow, L, H, g, merge_turn,
                              ring + wave * 32 * kOutPitch);
}

template <int VDT>
hipError_t launch(const AttnArgs& a, const Scalars& s, hipStream_t st) {
  const int32_t n_qt = (a.cur_len + kSBM - 1) / kSBM;
  const int64_t items = static_cast<int64_t>(a.batch) * a.heads * n_qt;
  if (items <= 0) return hipSuccess;
  if (items > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  AttnArgs b = a;
  b.ws_cuts = 0;
  if (a.workspace != nullptr && a.workspace_bytes > kCounterBytes) {
    const int64_t by_records = (a.workspace_bytes - kCounterBytes) / (2LL * 66 * kSThreads * 4);
    b.ws_cuts = static_cast<int32_t>(by_records < kMaxCounters ? by_records : kMaxCounters);
  }
  const int64_t grid = a.plan != nullptr ? a.plan_units : items;
  if (grid <= 0) return hipSuccess;
  seg_attn_split_kernel<VDT><<<dim3(static_cast<uint32_t>(grid)), kSThreads, 0, st>>>(
      b.plan, b.plan != nullptr ? static_cast<int32_t>(grid) : 0, b, s, n_qt);
  return hipGetLastError();
}

}  // namespace

bool attention_split_supported(const AttnArgs& a) {
  const bool v16 = a.v_dtype == kBF16 || a.v_dtype == kF16;
  return a.q_dtype == kF32 && a.k_dtype == kSplitRows && v16 && a.heads <= kMaxHeads &&
         a.qk_dot_mode != kDotFp32 && a.value_dot_mode != kDotFp32;
}

hipError_t launch_attention_split(const AttnArgs& a, const attn::Scalars& s, hipStream_t stream) {
  if (!attention_split_supported(a)) return hipErrorInvalidValue;
  return a.v_dtype == kBF16 ? launch<kBF16>(a, s, stream) : launch<kF16>(a, s, stream);
}

hipError_t launch_split_rows(const float* src, void* dst, int64_t rows, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  const int64_t blocks = (rows * 16 + 255) / 256;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  split_rows_kernel<<<dim3(static_cast<uint32_t>(blocks)), 256, 0, stream>>>(src, static_cast<uint8_t*>(dst),
                                                                              rows);
  return hipGetLastError();
}

int32_t attention_item_queries(const AttnArgs& a) { return attention_split_supported(a) ? kSBM : 128; }

}  // namespace hkv
