// Device pieces shared by the two segmented-attention kernels
// (seg_attn_direct.hip for 16-bit K/V, seg_attn_staged.hip for fp32 K or V).
//
// Semantics follow _fused_real_pruning_segmented_attention_kernel
// (real_pruning_fused_attention.py:76-267): query l of (b, h) attends to the
// slab rows of head h's segments in table order, then to the current scale's
// K/V rows of (b, h); online softmax with fp32 statistics, P rounded to the V
// operand type before the PV product, O / l at the end, output [B, L, H*D].
//
// Common structure of both kernels (CDNA4, wave64):
//  * A workgroup handles 32 * NW queries of one (b, h); each wave owns 32
//    query rows and keeps their Q fragments in registers.
//  * Keys are walked as a stream of 64-key tiles: the retained prior rows of
//    head h (all segments back to back, no per-segment tile restart; a row
//    table maps stream position -> slab row) then, starting on a fresh tile,
//    the current rows.  Every tile therefore reads one tensor only.
//  * S^T = K Q^T on v_mfma_f32_32x32x16_{bf16,f16}: keys are the M index, so
//    each lane holds one query's scores (16 per 32-key block); row max and sum
//    need one exchange between lanes l and l + 32, and the fp32 scores convert
//    in place to the B operand of O^T = V^T P^T.
//  * exp2 with scale * log2(e) folded into one FMA per score; the running max
//    is moved lazily (only when a row grows by more than 2^8).
//  * Work items are ordered heaviest head first (longest-processing-time
//    order); the dispatcher fills free CU slots in workgroup-id order.  The
//    16-bit kernel can also cut some items into two parts of their key-tile
//    stream so a launch fills whole rounds of the CU slots (round split,
//    below).
#pragma once

#include "hkv_internal.h"

namespace hkv {
namespace attn {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kD = 128;
constexpr int kBN = 64;  // keys per tile
constexpr float kLog2e = 1.4426950408889634f;
// Lazy rescale: the reference max used by exp2 moves only when a row's max
// grows by more than this (log2 units); p <= 2^8 stays exact in fp32 and is
// rounded like any other value to the 16-bit PV operand.
constexpr float kRescaleLog2 = 8.0f;
constexpr int kMaxHeads = 1024;

// ---------------------------------------------------------------- conversions

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

// 8 fp32 values at byte offset `off` of `r` as two bf16 operands, x = hi +
// lo + O(2^-18 |x|): hi = x rounded to bf16, lo = (x - hi) rounded to bf16.
// A product taken as hi*hi + lo*hi + hi*lo then carries about 16 significand
// bits (TF32 carries 11).  An offset of -1 yields zeros.
__device__ __forceinline__ void load8_split(__amdgpu_buffer_rsrc_t r, int32_t off, u32x4_t& hi, u32x4_t& lo) {
  const f32x4_t x = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
  const f32x4_t y = __builtin_bit_cast(
      f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off < 0 ? -1 : off + 16, 0, 0));
  const float v[8] = {x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hi[i] = pack2<kBF16>(v[2 * i], v[2 * i + 1]);
    const float h0 = __builtin_bit_cast(float, hi[i] << 16);
    const float h1 = __builtin_bit_cast(float, hi[i] & 0xffff0000u);
    lo[i] = pack2<kBF16>(v[2 * i] - h0, v[2 * i + 1] - h1);
  }
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

// ---------------------------------------------------------------- work plan

struct WorkItem {
  int32_t b, h, qt, bh;
  int32_t nseg;  // live segment entries of head h
  int32_t R;     // retained prior rows of head h
};

// Retained prior rows of every head (clamped tables) into head_rows[H].
template <int kThreads>
__device__ __forceinline__ void compute_head_rows(const int32_t* __restrict__ seg_starts,
                                                  const int32_t* __restrict__ seg_ends,
                                                  const int32_t* __restrict__ seg_counts, int64_t cap,
                                                  int H, int S, int32_t* head_rows) {
  for (int hh = threadIdx.x; hh < H; hh += kThreads) {
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
}

// Exclusive prefix of segment lengths in place, by one wave: on entry
// seg_pref[i + 1] holds the length of entry i < nseg (nseg <= 256), on exit
// seg_pref[i] = sum of the lengths before entry i (seg_pref[nseg] = total).
__device__ __forceinline__ void length_prefix(int32_t* seg_pref, int nseg, int lane) {
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

// Head h's clamped segment starts and exclusive length prefix into LDS (ends
// with a workgroup barrier); returns the live entry count, w.R = its total.
// The count and the head's S table entries are loaded together (entries past
// the count are read and dropped), so the launch waits for one round trip,
// not two.
template <int kThreads>
__device__ __forceinline__ void load_head_segments(const int32_t* __restrict__ seg_starts,
                                                   const int32_t* __restrict__ seg_ends,
                                                   const int32_t* __restrict__ seg_counts,
                                                   int64_t cap, int S, WorkItem& w,
                                                   int32_t* seg_start, int32_t* seg_pref) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  int nseg = seg_counts[w.h];
  for (int i = tid; i < S; i += kThreads) {
    int64_t st = seg_starts[static_cast<int64_t>(w.h) * S + i];
    int64_t en = seg_ends[static_cast<int64_t>(w.h) * S + i];
    st = st < 0 ? 0 : (st > cap ? cap : st);
    en = en < 0 ? 0 : (en > cap ? cap : en);
    if (i < nseg) {
      seg_start[i] = static_cast<int32_t>(st);
      seg_pref[i + 1] = en > st ? static_cast<int32_t>(en - st) : 0;
    }
  }
  nseg = nseg < 0 ? 0 : (nseg > S ? S : nseg);
  __syncthreads();
  if (wave == 0) length_prefix(seg_pref, nseg, lane);
  __syncthreads();
  w.nseg = nseg;
  w.R = seg_pref[nseg];
}

// plan_work for H <= 64 heads and S <= 64 entries per head, by wave 0 alone
// with one workgroup barrier: each lane loads table entries (all in flight at
// once), LDS atomics sum every head's live lengths, lane h ranks head h
// against the others (read from LDS 16 at a time), a ballot finds the
// item's head, and a wave scan gives its length prefix.  Same result as the
// general path below (same clamping, same longest-first order, ties by head
// index).
// `bc` receives 3 ints for the other waves; head_rows is 16-byte aligned.
__device__ __forceinline__ WorkItem plan_work_small(const int32_t* __restrict__ seg_starts,
                                                    const int32_t* __restrict__ seg_ends,
                                                    const int32_t* __restrict__ seg_counts, int64_t cap,
                                                    int H, int S, int B, int32_t n_qt,
                                                    int32_t* head_rows, int32_t* bc, int32_t* seg_start,
                                                    int32_t* seg_pref, int32_t item, int32_t* tab) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int32_t HS = H * S;
  int32_t* const tab_start = tab;
  int32_t* const tab_len = tab + HS;
  int32_t* const tab_cnt = tab + 2 * HS;
  const int32_t per_rank = B * n_qt;
  const int32_t target = item / per_rank;
  if (tid < 64) {
    // the counts are clamped and go to LDS after the first batch of table
    // reads is issued, so that both arrive in one memory round trip
    const int n_raw = lane < H ? seg_counts[lane] : 0;
    int cnt = 0;
    auto publish_counts = [&]() {
      int n = n_raw;
      asm volatile("" : "+v"(n));  // not before the reads issued above it
      cnt = n < 0 ? 0 : (n > S ? S : n);
      if (lane < H) {
        tab_cnt[lane] = cnt;
        head_rows[lane] = 0;
      }
      __builtin_amdgcn_wave_barrier();
    };
    if (HS == 0) publish_counts();
    for (int p0 = 0; p0 < HS; p0 += 8 * 64) {
      int32_t st[8], en[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int p = p0 + k * 64 + lane;
        st[k] = p < HS ? seg_starts[p] : 0;
        en[k] = p < HS ? seg_ends[p] : 0;
      }
      if (p0 == 0) publish_counts();
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int p = p0 + k * 64 + lane;
        if (p < HS) {
          int64_t a = st[k], e = en[k];
          a = a < 0 ? 0 : (a > cap ? cap : a);
          e = e < 0 ? 0 : (e > cap ? cap : e);
          const int32_t len = e > a ? static_cast<int32_t>(e - a) : 0;
          tab_start[p] = static_cast<int32_t>(a);
          tab_len[p] = len;
          const int hh = p / S;
          if (p - hh * S < tab_cnt[hh]) atomicAdd(head_rows + hh, len);
        }
      }
    }
    // LDS operations of one wave complete in order: the sums are final here
    __builtin_amdgcn_wave_barrier();
    const int r = lane < H ? head_rows[lane] : -1;
    int rank = 0;
    const int4* const hr4 = reinterpret_cast<const int4*>(head_rows);
    for (int o0 = 0; o0 < H; o0 += 16) {  // 16 rows per LDS round trip
      int v[16];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int4 x = hr4[o0 / 4 + k];
        v[4 * k + 0] = x.x;
        v[4 * k + 1] = x.y;
        v[4 * k + 2] = x.z;
        v[4 * k + 3] = x.w;
      }
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int o = o0 + k;
        rank += o < H && ((v[k] > r) || (v[k] == r && o < lane));
      }
    }
    const uint64_t hit = __ballot(lane < H && rank == target);
    const int h = hit != 0 ? static_cast<int>(__builtin_ctzll(hit)) : 0;  // one lane matches
    const int nseg = __builtin_amdgcn_readlane(cnt, h);
    const int len = lane < nseg ? tab_len[h * S + lane] : 0;
    const int st0 = lane < nseg ? tab_start[h * S + lane] : 0;
    int incl = len;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(incl, off, 64);
      if (lane >= off) incl += o;
    }
    if (lane < nseg) {
      seg_start[lane] = st0;
      seg_pref[lane + 1] = incl;
    }
    if (lane == 0) {
      seg_pref[0] = 0;
      bc[0] = h;
      bc[1] = nseg;
      bc[2] = nseg > 0 ? __builtin_amdgcn_readlane(incl, nseg - 1) : 0;
    }
  }
  __syncthreads();
  WorkItem w;
  const int32_t rem = item - target * per_rank;
  w.b = rem / n_qt;
  w.qt = rem - w.b * n_qt;
  w.h = bc[0];
  w.bh = w.b * H + w.h;
  w.nseg = bc[1];
  w.R = bc[2];
  return w;
}

// Longest-first order of the heads, the (b, h, query tile) of item `item`
// in that order, and head h's clamped segment starts + exclusive length
// prefix in LDS.  Ends with a workgroup barrier.  head_rows / head_by_rank
// need `heads` entries.  `tab` (tab_ints ints of LDS, free until the
// return) holds every head's clamped table when 2 H S + H ints fit: then
// the tables are read from global memory once, all entries in parallel.
template <int kThreads>
__device__ __forceinline__ WorkItem plan_work(const int32_t* __restrict__ seg_starts,
                                              const int32_t* __restrict__ seg_ends,
                                              const int32_t* __restrict__ seg_counts, int64_t cap,
                                              int H, int S, int B, int32_t n_qt,
                                              int32_t* head_rows, int32_t* head_by_rank,
                                              int32_t* seg_start, int32_t* seg_pref,
                                              int32_t item, int32_t* tab, int32_t tab_ints) {
  const int tid = threadIdx.x;
  const int32_t HS = H * S;
  const bool in_lds = 2 * HS + H <= tab_ints;
  if (in_lds && H <= 64 && S <= 64)
    return plan_work_small(seg_starts, seg_ends, seg_counts, cap, H, S, B, n_qt, head_rows, head_by_rank,
                           seg_start, seg_pref, item, tab);
  int32_t* const tab_start = tab;
  int32_t* const tab_len = tab + HS;
  int32_t* const tab_cnt = tab + 2 * HS;
  if (in_lds) {
    for (int idx = tid; idx < HS; idx += kThreads) {
      int64_t st = seg_starts[idx];
      int64_t en = seg_ends[idx];
      st = st < 0 ? 0 : (st > cap ? cap : st);
      en = en < 0 ? 0 : (en > cap ? cap : en);
      tab_start[idx] = static_cast<int32_t>(st);
      tab_len[idx] = en > st ? static_cast<int32_t>(en - st) : 0;
    }
    for (int hh = tid; hh < H; hh += kThreads) {
      const int n = seg_counts[hh];
      tab_cnt[hh] = n < 0 ? 0 : (n > S ? S : n);
    }
    __syncthreads();
    for (int hh = tid; hh < H; hh += kThreads) {
      int32_t rows = 0;
      for (int i = 0; i < tab_cnt[hh]; ++i) rows += tab_len[hh * S + i];
      head_rows[hh] = rows;
    }
  } else {
    compute_head_rows<kThreads>(seg_starts, seg_ends, seg_counts, cap, H, S, head_rows);
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

  WorkItem w;
  const int32_t per_rank = B * n_qt;
  const int32_t rank = item / per_rank;
  const int32_t rem = item - rank * per_rank;
  w.b = rem / n_qt;
  w.qt = rem - w.b * n_qt;
  w.h = head_by_rank[rank];
  w.bh = w.b * H + w.h;
  if (!in_lds) {
    load_head_segments<kThreads>(seg_starts, seg_ends, seg_counts, cap, S, w, seg_start, seg_pref);
    return w;
  }
  // head h's entries from the LDS table, then the length prefix (wave 0)
  const int lane = tid & 63;
  const int nseg = tab_cnt[w.h];
  for (int i = tid; i < nseg; i += kThreads) {
    seg_start[i] = tab_start[w.h * S + i];
    seg_pref[i + 1] = tab_len[w.h * S + i];
  }
  __syncthreads();
  if (tid < 64) length_prefix(seg_pref, nseg, lane);
  __syncthreads();
  w.nseg = nseg;
  w.R = seg_pref[nseg];
  return w;
}

// ---------------------------------------------------------------- round split
//
// With a workspace, some items are cut into two parts of their key-tile
// stream so that the launch fills whole rounds of the device's resident
// workgroup slots G.  Items are numbered longest first.  With G < N < 2G
// items, the first (heaviest) 2G - N are cut, giving exactly 2G units, and
// the whole items run first: the second round is then made of halves, so
// it ends close to the first instead of waiting on heavy items that began
// in it whole (on the 2B sweep's scale 11, 576 items of 37 to 90 key tiles,
// a slot model gives 116 us against 133 us for cutting the lightest).  With
// N <= G, the first min(N, G - N) are cut, so the one round is not set by
// the heaviest item.  N >= 2G launches are not cut.  An item with fewer than
// 2 kMinPartTiles key tiles still runs whole: its second part finds too few
// tiles and leaves at once.  A part leaves its partial result (unnormalized
// O, running max and sum) in a workspace record; the part that completes an
// item last merges both records in part order.  Workgroup ids: with
// whole_first, items [two, N) whole, then the cut items' parts; otherwise
// the cut items' parts, then items [two, N) whole.  The parts of a cut item
// are adjacent when every item has at least 2 kMinPartTiles tiles;
// otherwise all first parts come before all second parts: workgroup ids are
// dealt to the 8 XCDs round robin, and adjacent second parts that leave at
// once would leave half of the XCDs idle.  (Measured on the 2B scales:
// adjacent parts run scale 9 in 36 us against 40 us grouped; grouped parts
// run scale 8 in 21 us against 30 us adjacent.)
// Key tiles a part of a cut item must have at least (measured on the 2B
// scales: parts of ~8.5 tiles gain 13 %, parts of ~5 tiles lose 20 %).
constexpr int32_t kMinPartTiles = 8;

struct RoundSplit {
  int32_t items;        // N
  int32_t two;          // cut items: [0, two) in longest-first order
  int32_t grouped;      // first parts, then second parts (else each item's two parts adjacent)
  int32_t whole_first;  // whole items before the cut items' parts
};

// `min_tiles`: key tiles every item has at least (its current-scale tiles).
__host__ __device__ __forceinline__ RoundSplit round_split(int32_t items, int32_t slots, int32_t min_tiles) {
  RoundSplit t{items, 0, min_tiles < 2 * kMinPartTiles ? 1 : 0, 0};
  if (slots <= 0 || items >= 2 * slots) return t;
  if (items > slots) {
    t.two = 2 * slots - items;
    t.whole_first = 1;
  } else {
    t.two = items < slots - items ? items : slots - items;
  }
  return t;
}

// Workgroups of a launch, and workspace records it needs (one counter per
// cut item, at most G).
__host__ __device__ __forceinline__ int64_t split_units(const RoundSplit& t) {
  return static_cast<int64_t>(t.items) + t.two;
}
__host__ __device__ __forceinline__ int64_t split_records(const RoundSplit& t) { return 2LL * t.two; }

struct Unit {
  int32_t item;     // in longest-first order
  int32_t part;     // 0 or 1
  int32_t parts;    // 1 or 2
  int32_t record;   // first record of the item (parts > 1)
  int32_t counter;  // counter of the item (parts > 1)
  int32_t arrive;   // 1: the two parts count in first, the second writes no record (merge_parts)
};

__host__ __device__ __forceinline__ Unit split_unit(const RoundSplit& t, int32_t j) {
  Unit u{j, 0, 1, 0, 0, 0};
  if (t.two == 0) return u;
  const int32_t lead = t.whole_first ? t.items - t.two : 0;  // whole items before the parts
  if (j < lead) {
    u.item = t.two + j;
    return u;
  }
  const int32_t k = j - lead;
  if (k < 2 * t.two) {
    const int32_t c = t.grouped ? (k < t.two ? k : k - t.two) : k / 2;  // cut item
    u.item = c;
    u.part = t.grouped ? (k < t.two ? 0 : 1) : k % 2;
    u.parts = 2;
    u.record = 2 * c;
    u.counter = c;
    u.arrive = 1;
    return u;
  }
  u.item = k - t.two;  // whole items after the parts: k - 2 two + two
  return u;
}

// Item of workgroup j when every item is whole, arranged so that all query
// tiles of one (head, batch row) run on one XCD: workgroup ids are dealt to
// the 8 XCDs round robin (j % 8), so the XCD's k-th workgroup (k = j / 8) takes
// query tile k % n_qt of its (k / n_qt)-th group, and groups (n_qt
// consecutive items in longest-first order) are dealt to XCDs in a snake
// order (0..7, 7..0, ...).  The K/V rows of a (head, batch row) are then
// fetched into one L2 instead of eight.  The XCDs' loads are only as even
// as the snake makes them, so this is used with at least 8 groups per XCD
// (fewer, and a few heavy groups would load some XCDs more than others;
// measured: 1.7 % faster at 256 groups, 2 % slower at 32).  Needs
// groups % 8 == 0; otherwise the identity.
constexpr int kXcds = 8;
__device__ __forceinline__ int32_t xcd_item(int32_t j, int32_t groups, int32_t n_qt) {
  if (groups % kXcds != 0 || groups < 8 * kXcds) return j;
  const int32_t x = j % kXcds;
  const int32_t k = j / kXcds;
  const int32_t lg = k / n_qt;
  const int32_t qt = k - lg * n_qt;
  const int32_t group = lg * kXcds + ((lg & 1) ? kXcds - 1 - x : x);
  return group * n_qt + qt;
}

// Row table of prior tile `tile` (wave 0, one entry per lane per 64 keys):
// stream position -> slab row * ROW_BYTES, or `past_end` past R.  With
// ROW_BYTES = 1 the entries are row indices.  `cur_seg` walks forward with
// the tiles (callers fill tiles in increasing order).
template <int ROW_BYTES = 1>
__device__ __forceinline__ void fill_rowtab(int tile, int32_t* rowtab, int& cur_seg, int nseg, int R,
                                            const int32_t* seg_start, const int32_t* seg_pref,
                                            int32_t past_end = -1) {
  const int lane = threadIdx.x & 63;
  const int j0 = tile * kBN;
  while (cur_seg < nseg && seg_pref[cur_seg + 1] <= j0) ++cur_seg;
  const int j = j0 + lane;
  int32_t row = past_end;
  if (j < R) {
    int s = cur_seg;
    while (seg_pref[s + 1] <= j) ++s;
    row = (seg_start[s] + (j - seg_pref[s])) * ROW_BYTES;
  }
  rowtab[lane] = row;
}

// ---------------------------------------------------------------- softmax

// Maximum / sum of v over lanes l and l ^ 32 (the two lanes that hold one
// query's scores) without an LDS round trip: v_permlane32_swap exchanges the
// lane halves of two registers.
__device__ __forceinline__ float pair_max(float v) {
  const uint32_t b = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
  return fmaxf(__builtin_bit_cast(float, static_cast<uint32_t>(r[0])),
               __builtin_bit_cast(float, static_cast<uint32_t>(r[1])));
}

__device__ __forceinline__ float pair_sum(float v) {
  const uint32_t b = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
  return __builtin_bit_cast(float, static_cast<uint32_t>(r[0])) +
         __builtin_bit_cast(float, static_cast<uint32_t>(r[1]));
}

// Online softmax of one 64-key tile held as S^T blocks (keys 32kb + 8(j>>2) +
// 4g + (j&3), query = lane & 31), in four steps that the pipelined kernel
// interleaves with matrix work: mask_tile, tile_max, move_max, exp_tile.
// Keys >= valid_keys get score -inf, hence p = exp2(-inf) = 0 (the launcher
// guarantees c > 0), so no second mask is needed after the exponentials.
__device__ __forceinline__ void mask_tile(f32x16_t (&s)[2], int valid_keys, int g) {
  // key index 32kb + 8(j>>2) + 4g + (j&3) >= valid  <=>  constant >= valid - 4g
  const int lim = valid_keys - 4 * g;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (kb * 32 + 8 * (j >> 2) + (j & 3) >= lim) s[kb][j] = -__builtin_inff();
}

// Row maximum of the tile for the lane's query (both lanes of the pair).
// A running chain: the compiler folds it into v_max3_f32 with few NaN
// canonicalizations of the MFMA results (a balanced tree needs one per leaf).
__device__ __forceinline__ float tile_max(const f32x16_t (&s)[2]) {
  float mx = s[0][0];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int j = 0; j < 16; ++j) mx = fmaxf(mx, s[kb][j]);
  return pair_max(mx);
}

// Moves the reference max (and rescales oacc / l_run) when a row's max grew
// by more than thresh; lazy, so it rarely runs after the first tiles.
__device__ __forceinline__ void move_max(f32x16_t (&oacc)[4], float& m_run, float& l_run, float mx,
                                         float c, float thresh) {
  if (__any(mx - m_run > thresh)) {
    const float m_new = fmaxf(m_run, mx);
    const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c);
    l_run *= alpha;
#pragma unroll
    for (int db = 0; db < 4; ++db) oacc[db] *= alpha;
    m_run = m_new;
  }
}

// p = exp2(c (s - m)) in place, l_run += sum of p (fp32, unrounded).
__device__ __forceinline__ void exp_tile(f32x16_t (&s)[2], float m_run, float c, float& l_run) {
  const float mc = m_run * c;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int j = 0; j < 16; ++j) s[kb][j] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][j], c, -mc));
  // four partial sums for ILP, each started from its first term (adding to
  // +0 is not an identity the compiler may drop)
  float psum[4];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      float& acc = psum[2 * kb + (j >> 3)];
      acc = (j & 7) == 0 ? s[kb][j] : acc + s[kb][j];
    }
  l_run += (psum[0] + psum[1]) + (psum[2] + psum[3]);
}

__device__ __forceinline__ void softmax_tile(f32x16_t (&s)[2], f32x16_t (&oacc)[4], float& m_run,
                                             float& l_run, float c, float thresh, int valid_keys,
                                             int g) {
  if (valid_keys < kBN) mask_tile(s, valid_keys, g);
  move_max(oacc, m_run, l_run, tile_max(s), c, thresh);
  exp_tile(s, m_run, c, l_run);
}

// P^T B-operand for PV k-step u (keys 16u + {4g..4g+3, 8+4g..8+4g+3}).
template <int MV>
__device__ __forceinline__ u32x4_t p_operand(const f32x16_t (&s)[2], int u) {
  const f32x16_t& sp = s[u >> 1];
  const int j0 = 8 * (u & 1);
  u32x4_t pf;
  pf[0] = pack2<MV>(sp[j0 + 0], sp[j0 + 1]);
  pf[1] = pack2<MV>(sp[j0 + 2], sp[j0 + 3]);
  pf[2] = pack2<MV>(sp[j0 + 4], sp[j0 + 5]);
  pf[3] = pack2<MV>(sp[j0 + 6], sp[j0 + 7]);
  return pf;
}

// O = acc / l to out[b, q, h*D + d] (d = 32db + 8(j>>2) + 4g + (j&3)) in
// `out_dtype` (fp32, or rounded to nearest even to bf16 / fp16), and
// lse = ln(2) (c m + log2(l)) for the lane's query (c = scale log2(e)).
template <int DT>
__device__ __forceinline__ void store_rows(const f32x16_t (&oacc)[4], float inv, void* out, int64_t out_row,
                                           int g) {
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      f32x4_t v;
      v[0] = oacc[db][4 * jb + 0] * inv;
      v[1] = oacc[db][4 * jb + 1] * inv;
      v[2] = oacc[db][4 * jb + 2] * inv;
      v[3] = oacc[db][4 * jb + 3] * inv;
      store4<DT>(out, out_row + db * 32 + 8 * jb + 4 * g, v);
    }
}

__device__ __forceinline__ void write_output(const f32x16_t (&oacc)[4], float m_run, float l_run,
                                             float c, void* out, float* lse, int64_t b, int64_t h,
                                             int32_t qrow, int L, int H, int64_t bh, int g,
                                             int32_t out_dtype) {
  const float l_tot = pair_sum(l_run);
  const float inv = 1.f / l_tot;
  if (qrow >= L) return;
  const int64_t out_row = (b * L + qrow) * (static_cast<int64_t>(H) * kD) + h * kD;
  if (out_dtype == kF32) store_rows<kF32>(oacc, inv, out, out_row, g);
  else if (out_dtype == kF16) store_rows<kF16>(oacc, inv, out, out_row, g);
  else store_rows<kBF16>(oacc, inv, out, out_row, g);
  if (lse != nullptr && g == 0) lse[bh * L + qrow] = (m_run * c + __log2f(l_tot)) * 0.6931471805599453f;
}

// write_output for 16-bit output types through LDS: each wave rounds its
// 32 x 128 tile into `stage` (32 rows of kOutPitch bytes, private to the
// wave; the pad spreads the rows over the banks), then stores whole 256-byte
// rows, 16 lanes per row and 4 rows per instruction (8 full-line stores
// instead of 16 that each touch 32 rows).  Same values as write_output.
// `qrow0` is the wave's first query; `out` must be 16-byte aligned.
constexpr int kOutPitch = kD * 2 + 16;
template <int DT>
__device__ __forceinline__ void write_output_lds(const f32x16_t (&oacc)[4], float m_run, float l_run,
                                                 float c, void* out, float* lse, int64_t b, int64_t h,
                                                 int32_t qrow0, int L, int H, int64_t bh, int lane,
                                                 uint8_t* stage) {
  const int g = lane >> 5;
  const int q = lane & 31;
  const float l_tot = pair_sum(l_run);
  const float inv = 1.f / l_tot;
  uint8_t* const mine = stage + q * kOutPitch;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      u32x2_t w;
      w[0] = pack2<DT>(oacc[db][4 * jb + 0] * inv, oacc[db][4 * jb + 1] * inv);
      w[1] = pack2<DT>(oacc[db][4 * jb + 2] * inv, oacc[db][4 * jb + 3] * inv);
      *reinterpret_cast<u32x2_t*>(mine + (db * 32 + 8 * jb + 4 * g) * 2) = w;
    }
  __builtin_amdgcn_wave_barrier();  // a wave's LDS operations run in order
  const int64_t row_stride = static_cast<int64_t>(H) * kD;
  uint16_t* const base = static_cast<uint16_t*>(out) + b * L * row_stride + h * kD + (lane & 15) * 8;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int row = 4 * k + (lane >> 4);
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(stage + row * kOutPitch + (lane & 15) * 16);
    if (qrow0 + row < L) *reinterpret_cast<u32x4_t*>(base + (qrow0 + row) * row_stride) = v;
  }
  if (lse != nullptr && g == 0 && qrow0 + q < L)
    lse[bh * L + qrow0 + q] = (m_run * c + __log2f(l_tot)) * 0.6931471805599453f;
}

// Launch plumbing shared by the two kernels.
struct Scalars {
  float c;          // max(|scale| * log2(e), kMinC): the exp2 multiplier, > 0
  float thresh;     // kRescaleLog2 / c: score growth (score units) that moves the max
  uint32_t q_sign;  // 0x80008000 when scale < 0: q's 16-bit operands are negated
};

// Smallest exp2 multiplier.  A softmax scale of 0 (uniform attention) runs
// with c = kMinC: every p is then exp2(~0) and the result is the uniform
// average, while -inf still masks the keys past a tile's end.
constexpr float kMinC = 1e-30f;

// s_waitcnt for "at most n vector-memory operations outstanding" (gfx9
// encoding; expcnt and lgkmcnt left at their maxima = not waited on).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Agent-scope relaxed loads and stores of the partial records and counters:
// coherent across the XCDs' L2 caches without writing back or invalidating
// them.
//
// Ordering of a record before its counter.  Every word of a record is written
// by an agent-scope atomic store (global_store ... sc1: written through to the
// device's coherence point) and read by an agent-scope atomic load (sc1: read
// from it).  The publishing workgroup waits for its stores to be acknowledged
// (s_waitcnt vmcnt(0), which on gfx9 counts stores) and for every wave
// (barrier) before its counter add (for two parts: the ready mark) is issued;
// the merging workgroup issues its record loads only after it has seen the
// counter's value (the returned value, or for two parts the ready mark read
// by its spin; then a barrier).
// So the hardware orders the record before the counter.  The memory model's
// way of saying it, an acq_rel counter add, adds a write-back and an
// invalidate of the whole XCD L2 (buffer_wbl2 / buffer_inv sc1) per part,
// which protects no data here (nothing in a record is written by a plain
// store) and costs 2.5% of the 2B final step (310 -> 317 us, 768 parts).
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Spins of the merging part's wait for the other part's record (each an
// agent-scope load and s_sleep 8, ~512 cycles): the other part has counted
// itself in and is resident, so its record lands within microseconds; the
// bound only keeps the wait finite.
constexpr int32_t kReadySpins = 1 << 20;

// Part of a cut item: publish the partial record, count it in, and if it is
// the item's last part to finish, merge every part and write the output.
// A record holds 66 * kThreads floats (each thread's 64 accumulators, its
// running max and its sum); item r's parts use records 2r and 2r + 1.  The
// output goes through `stage` (32 * kOutPitch bytes per wave) when
// kStageOut, else straight from registers.
//
// With un.arrive (every cut unit of the library's plans and round split)
// the two parts count themselves in first: the first to arrive writes its
// record and then adds a second time (ready); the second writes no record
// of its own -- it waits until the counter shows both arrivals and the
// ready mark (3), then merges from its registers and the other record
// (2B final step 298.9 vs 300.7 us, sweep scale 11 117.0 vs 120.2 us; with
// each counter on a line of its own also where the parts run side by side:
// sweep scale 9 33.1 vs 34.5 us, scale 8 20.1 vs 20.5 us).  Without it
// every part publishes its record before counting in, and the last to count
// merges.
template <int QDT, int kThreads, bool kStageOut = true>
__device__ __forceinline__ void merge_parts(const AttnArgs& a, const Scalars& sc, const Unit& un,
                                            int32_t parts, const f32x16_t (&oacc)[4], float m_run,
                                            float l_run, const WorkItem& w, int32_t qrow, int L, int H,
                                            int g, int32_t& merge_turn, uint8_t* stage) {
  const int tid = threadIdx.x;
  int32_t* const counters = static_cast<int32_t*>(a.workspace);
  float* const records = reinterpret_cast<float*>(static_cast<uint8_t*>(a.workspace) + kCounterBytes);
  float* const rec0 = records + static_cast<int64_t>(un.record) * (66 * kThreads);
  int32_t* const counter = counters + static_cast<int64_t>(un.counter) * kCounterStride;
  auto publish = [&]() {
    float* const mine = rec0 + static_cast<int64_t>(un.part) * (66 * kThreads);
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int j = 0; j < 16; ++j) st_agent(mine + (db * 16 + j) * kThreads + tid, oacc[db][j]);
    st_agent(mine + 64 * kThreads + tid, m_run);
    st_agent(mine + 65 * kThreads + tid, l_run);
    wait_vmcnt<0>();
    __syncthreads();
  };
  if (parts == 2 && un.arrive != 0) {
    if (tid == 0)
      merge_turn = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (merge_turn == 0) {
      // first to arrive: publish, then the ready mark
      publish();
      if (tid == 0)
        __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    if (tid == 0) {
      for (int32_t i = 0; i < kReadySpins; ++i) {
        if (__hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 3) break;
        __builtin_amdgcn_s_sleep(8);
      }
    }
    __syncthreads();
  } else {
    publish();
    if (tid == 0)
      merge_turn = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == parts - 1;
    __syncthreads();
    if (!merge_turn) return;
  }
  // Every part is published: combine the parts in part order (this part's
  // own values from registers, equal to its record), the same arithmetic
  // whichever part merges.
  float mp[4], lp[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const bool other = p < parts && p != un.part;
    const float* rec = rec0 + static_cast<int64_t>(p) * (66 * kThreads);
    mp[p] = other ? ld_agent(rec + 64 * kThreads + tid) : m_run;
    lp[p] = other ? ld_agent(rec + 65 * kThreads + tid) : l_run;
  }
  float m_new = mp[0];
#pragma unroll
  for (int p = 1; p < 4; ++p)
    if (p < parts) m_new = fmaxf(m_new, mp[p]);
  f32x16_t acc[4] = {};
  float l_acc = 0.f;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    if (p >= parts) break;
    const float al = __builtin_amdgcn_exp2f((mp[p] - m_new) * sc.c);
    const float* rec = rec0 + static_cast<int64_t>(p) * (66 * kThreads);
    if (p == un.part) {
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[db][j] = p == 0 ? oacc[db][j] * al : __builtin_fmaf(oacc[db][j], al, acc[db][j]);
    } else {
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const float o = ld_agent(rec + (db * 16 + j) * kThreads + tid);
          acc[db][j] = p == 0 ? o * al : __builtin_fmaf(o, al, acc[db][j]);
        }
    }
    l_acc = p == 0 ? lp[p] * al : __builtin_fmaf(lp[p], al, l_acc);
  }
  if (kStageOut && a.out_dtype != kF32 && (reinterpret_cast<uintptr_t>(a.out) & 15) == 0) {
    // the stage is free: every wave passed the barriers above after its last tile
    const int32_t qrow0 = qrow - (tid & 31);
    if (a.out_dtype == kF16)
      write_output_lds<kF16>(acc, m_new, l_acc, sc.c, a.out, a.lse, w.b, w.h, qrow0, L, H, w.bh, tid & 63, stage);
    else
      write_output_lds<kBF16>(acc, m_new, l_acc, sc.c, a.out, a.lse, w.b, w.h, qrow0, L, H, w.bh, tid & 63, stage);
  } else {
    write_output(acc, m_new, l_acc, sc.c, a.out, a.lse, w.b, w.h, qrow, L, H, w.bh, g, a.out_dtype);
  }
  if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The current rows' append (AttnArgs::append_offsets, and the second
// destination append2_offsets).  A copy block moves kAppendRows rows of K and
// of V of one (b, h), 16 bytes per lane per access (one access per lane and
// tensor for 16-bit rows), read once and written to each destination; a
// destination with off < 0 or off + L > its capacity is skipped.  The rows
// written lie outside every segment the launch reads (the caller's
// contract), so copy blocks and attention workgroups of one launch need no
// ordering.
constexpr int kAppendRows = 16;

__host__ __device__ inline int64_t append_blocks(int32_t batch, int32_t heads, int32_t L) {
  return static_cast<int64_t>(batch) * heads * ((L + kAppendRows - 1) / kAppendRows);
}

template <int kThreads>
__device__ __forceinline__ void append_block(const AttnArgs& a, uint32_t blk, int32_t k_row, int32_t v_row) {
  const int32_t L = a.cur_len;
  const uint32_t H = static_cast<uint32_t>(a.heads);
  const int64_t cap = a.slab_capacity;
  // 32-bit index arithmetic: blocks and (b, h) pairs fit a launch grid
  const uint32_t chunks = static_cast<uint32_t>((L + kAppendRows - 1) / kAppendRows);
  const uint32_t bh = blk / chunks;
  if (bh >= static_cast<uint32_t>(a.batch) * H) return;
  const int32_t h = static_cast<int32_t>(bh % H);
  const int64_t b = bh / H;
  const int32_t off = a.append_offsets[h];
  const bool w1 = off >= 0 && off <= cap - L;
  const int64_t cap2 = a.slab2_capacity;
  const int32_t off2 = a.append2_offsets != nullptr ? a.append2_offsets[h] : -1;
  const bool w2 = off2 >= 0 && off2 <= cap2 - L;
  if (!w1 && !w2) return;
  const int32_t r0 = static_cast<int32_t>(blk - bh * chunks) * kAppendRows;
  const int32_t rows = L - r0 < kAppendRows ? L - r0 : kAppendRows;
  const int64_t dst_row = b * cap + off + r0;
  const int64_t dst2_row = b * cap2 + off2 + r0;
  const int64_t src_row = static_cast<int64_t>(bh) * L + r0;
  const uint4* sk = reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(a.cur_k) + src_row * k_row);
  const uint4* sv = reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(a.cur_v) + src_row * v_row);
  uint4* dk = reinterpret_cast<uint4*>(static_cast<uint8_t*>(const_cast<void*>(a.slab_k)) + dst_row * k_row);
  uint4* dv = reinterpret_cast<uint4*>(static_cast<uint8_t*>(const_cast<void*>(a.slab_v)) + dst_row * v_row);
  uint4* dk2 = reinterpret_cast<uint4*>(static_cast<uint8_t*>(a.slab2_k) + dst2_row * k_row);
  uint4* dv2 = reinterpret_cast<uint4*>(static_cast<uint8_t*>(a.slab2_v) + dst2_row * v_row);
  const int32_t nk = rows * (k_row / 16);
  const int32_t nv = rows * (v_row / 16);
  // one access of each tensor in flight per lane: more (a deeper batch of
  // loads) makes the 16-bit kernel's register allocation spill
  const int32_t n = nk > nv ? nk : nv;
  for (int32_t u = static_cast<int32_t>(threadIdx.x); u < n; u += kThreads) {
    uint4 xk, xv;
    if (u < nk) xk = sk[u];
    if (u < nv) xv = sv[u];
    if (w1 && u < nk) dk[u] = xk;
    if (w1 && u < nv) dv[u] = xv;
    if (w2 && u < nk) dk2[u] = xk;
    if (w2 && u < nv) dv2[u] = xv;
  }
}

}  // namespace attn

hipError_t launch_attention_direct(const AttnArgs& a, const attn::Scalars& s, hipStream_t stream);
hipError_t launch_attention_staged(const AttnArgs& a, const attn::Scalars& s, hipStream_t stream);
hipError_t launch_attention_split(const AttnArgs& a, const attn::Scalars& s, hipStream_t stream);
bool attention_direct_supported(const AttnArgs& a);

}  // namespace hkv
