// Segmented attention, direct-to-LDS variant for 16-bit K and V (bf16/fp16).
//
// K/V tiles move global -> LDS with buffer_load_dwordx4 ... lds (asynchronous,
// no register staging; rows outside the tensors arrive as zeros) into a ring
// of 2 stages (the K half of stage t % 2 holds K(t), the V half V(t)), one
// tile ahead of their use, with one barrier per tile; K runs one tile ahead
// of V (software pipeline, see seg_attn_pipe_kernel).
//
// LDS holds each tile in MFMA-operand order, so every operand read is one
// contiguous 1 KiB (K) or 512 B (V) block per wave at a constant offset:
//  * K block (kb, ks), 1 KiB: lane l's 16 bytes are K[32kb + l%32][16ks +
//    8(l/32) .. +7], the A operand of S^T = K Q^T.  One DMA instruction fills
//    one block (32 key rows x 32 bytes).
//  * V block (db, u, h), 512 B: 64 chunks of 4 values; chunk 16G + j holds
//    V[16u + 4(G/2) + 8h + j/4][32db + 16(G%2) + 4(j%4) .. +3].  ds_read_b64_
//    tr_b16 of lane l at chunk l then yields V[16u + 4g + 8h + m][32db + l%32]
//    for m = 0..3 (lane i of a 16-lane group receives element i%4 of the
//    chunks of lanes 4m + i/4): four consecutive keys at the lane's d, i.e.
//    half of the A operand of O^T = V^T P^T for k-step u.  One DMA
//    instruction fills blocks (2p, u, h) and (2p+1, u, h): 8 key rows x 128
//    contiguous bytes.
#include "attn_common.h"

#include <type_traits>

namespace hkv {
namespace {

using namespace attn;

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t* lds_s16x4_ptr;
typedef __attribute__((address_space(3))) void* lds_void_ptr;

constexpr int kTileBytes = kBN * kD * 2;  // 16 KiB per tensor per tile
constexpr int kStageBytes = 2 * kTileBytes;
constexpr int kDmaPerTile = 2 * kTileBytes / 1024;  // wave-level 1 KiB DMA instructions

__device__ __forceinline__ u32x2_t ds_read_tr(const uint8_t* p) {
  return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(p)));
}

// 16-byte-per-lane buffer load of byte offset voff + IMM of `rsrc`, written
// straight to LDS at `lds_addr` (the wave-uniform LDS byte address; lane l
// lands at lds_addr + 16 l); the add rides in the same asm, so the compiler
// keeps one offset register per wave, not one per DMA instruction.  Issued as
// inline assembly so that the compiler, which cannot see the LDS write, does
// not make every later LDS read wait for all outstanding loads: ordering is
// explicit here (s_waitcnt vmcnt before each tile's barrier).
// M0 is written here and declared clobbered; nothing else in these kernels
// uses M0 (tests/test_build_isa.py checks the generated code), so the
// compiler's warning about clobbering a reserved register is silenced.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <int IMM>
__device__ __forceinline__ void dma16_at(const u32x4_t rsrc, uint32_t lds_addr, int32_t voff) {
  if constexpr (IMM == 0) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds_addr), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
  } else {
    int32_t tmp;
    asm volatile("v_add_u32_e32 %0, %4, %2\n\ts_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %3, 0 offen lds"
                 : "=&v"(tmp)
                 : "s"(lds_addr), "v"(voff), "s"(rsrc), "i"(IMM)
                 : "memory", "m0");
  }
}
#pragma clang diagnostic pop

// Raw buffer descriptor (gfx9 layout) over [base, base + bytes), uniform.
__device__ __forceinline__ u32x4_t make_desc(const void* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  u32x4_t d;
  d[0] = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p));
  d[1] = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p >> 32) & 0xffffu);
  d[2] = __builtin_amdgcn_readfirstlane(bytes);
  d[3] = 0x00020000u;
  return d;
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_ptr)(p)));
}

// Software-pipelined variant: K runs one tile ahead of V, so iteration t
// computes S(t+1) = K(t+1) Q^T on the matrix cores while the VALU turns S(t)
// into P(t) (exponentials, row sums, bf16 pack), then accumulates P(t) V(t)
// while the VALU takes the row max of S(t+1).  Each wave thus overlaps its
// own softmax with its own MFMAs instead of relying on the other wave of its
// SIMD being in the opposite phase.  Same ring (K half of stage t % 2 holds
// K(t), V half holds V(t)), same row tables (3 slots, filled 3 tiles ahead),
// one barrier per tile, one tile of DMA in flight per wave.
template <int QDT, int KDT, int VDT>
__global__ __launch_bounds__(256, 2) void seg_attn_pipe_kernel(
    const int32_t* __restrict__ plan_p, const int32_t n_units, const AttnArgs a, const Scalars sc,
    const int32_t n_qt, const RoundSplit split) {
  static_assert(KDT != kF32 && VDT != kF32 && QDT == KDT, "16-bit inputs only");
  constexpr int NW = 4;
  constexpr int NS = 2;
  constexpr int MQK = KDT;
  constexpr int MV = VDT;
  constexpr int kThreads = NW * 64;
  constexpr int kBM = NW * 32;
  constexpr int kDmaPerWave = kDmaPerTile / NW;
  static_assert(kPartialFloats == 66 * kThreads, "partial record layout");

  __shared__ __attribute__((aligned(1024))) uint8_t ring[NS * kStageBytes];
  __shared__ __attribute__((aligned(16))) int32_t rowtab[3][kBN];
  __shared__ int32_t seg_start[kMaxSegments];
  __shared__ int32_t seg_pref[kMaxSegments + 1];
  __shared__ int32_t merge_turn;
  static_assert(NS * kStageBytes >= 2 * kMaxHeads * 4, "head tables alias the ring");

  // This workgroup's plan unit.  The plan pointer and the unit count are the
  // first kernel arguments, preloaded into SGPRs (the build passes
  // -amdgpu-kernarg-preload-count=2 for this file), so the unit's load goes
  // out with the other kernel arguments' loads instead of after them (about
  // 0.5 us less per launch on the small scales).
  int32_t pu[kPlanInts] = {};
  const bool planned = plan_p != nullptr && static_cast<int32_t>(blockIdx.x) < n_units;
  if (planned) {
    const int32_t* src = plan_p + static_cast<int64_t>(blockIdx.x) * kPlanInts;
#pragma unroll
    for (int i = 0; i < kPlanInts; ++i) pu[i] = src[i];
  }
  if (a.append_offsets != nullptr && static_cast<int32_t>(blockIdx.x) >= a.append_first) {
    // a copy block of the fused append, after the attention workgroups
    append_block<256>(a, blockIdx.x - static_cast<uint32_t>(a.append_first), kD * 2, kD * 2);
    return;
  }
  const int64_t cap = a.slab_capacity;
  const int H = a.heads;
  const int L = a.cur_len;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform by construction
  const int g = lane >> 5;

  Unit un;
  WorkItem w;
  int32_t t_begin, t_end, parts;
  const int32_t ntc = (L + kBN - 1) / kBN;
  // An item's key stream: its ntc current-scale tiles first (addressed
  // without any table), then its R retained prior rows, ntp tiles through the
  // row tables.
  int32_t p0 = 0, p1 = 0;
  bool cut = false;
  bool shared = false;  // alternate the wave priority by tile (the plan says so)
  if (planned) {
    // the unit of this workgroup from the caller's work plan
    const int32_t ph = pu[0], pj = pu[1], pcut = pu[4], ppart = pu[5];
    p0 = pu[2];
    p1 = pu[3];
    shared = pu[6] != 0;
    if (ph < 0 || ph >= H || pj < 0 || pj >= a.batch * n_qt) return;  // not a unit of this launch
    w.h = ph;
    w.b = pj / n_qt;
    w.qt = pj - w.b * n_qt;
    w.bh = w.b * H + w.h;
    // a cut item's record and counter exist when the launch has a workspace
    cut = pcut >= 0 && a.workspace != nullptr && pcut < a.ws_cuts && ppart >= 0 && ppart < 2;
    parts = cut ? 2 : 1;
    un.item = 0;
    un.part = cut ? ppart : 0;
    un.parts = parts;
    un.record = cut ? 2 * pcut : 0;
    un.counter = cut ? pcut : 0;
    un.arrive = cut && pu[7] != 0 ? 1 : 0;
  } else {
    un = split_unit(split, static_cast<int32_t>(blockIdx.x));
    if (split.two == 0) un.item = xcd_item(un.item, a.batch * H, n_qt);
    int32_t* head_rows = reinterpret_cast<int32_t*>(ring);
    w = plan_work<kThreads>(a.seg_starts, a.seg_ends, a.seg_counts, cap, H, a.max_segments, a.batch, n_qt,
                            head_rows, head_rows + kMaxHeads, seg_start, seg_pref, un.item,
                            head_rows + 2 * kMaxHeads, NS * kStageBytes / 4 - 2 * kMaxHeads);
  }

  const bool k_wave = wave * kDmaPerWave < 16;
  const int64_t cur_row0 = static_cast<int64_t>(w.bh) * L;
  const u32x4_t d_prior = make_desc(
      static_cast<const uint8_t*>(k_wave ? a.slab_k : a.slab_v) + static_cast<int64_t>(w.b) * cap * kD * 2,
      static_cast<uint32_t>(cap * kD * 2));
  const uint8_t* const cur_base =
      static_cast<const uint8_t*>(k_wave ? a.cur_k : a.cur_v) + cur_row0 * kD * 2;
  const uint32_t cur_bytes = static_cast<uint32_t>(L * kD * 2);
  constexpr int32_t kPastEnd = static_cast<int32_t>(0x80000000u);

  // DMA i of a tile moves 32 key rows x 32 bytes (K waves: K block (wave, i))
  // or 8 key rows x 128 bytes (V waves); the lane's key row and byte column
  // follow from DMA 0's by constants: K key + 0, column + 32 i; V key +
  // 16 (i >> 2) + 8 ((i >> 1) & 1), column + 128 (i & 1).
  static_assert(kDmaPerWave == 8, "DMA pattern");
  int key0, col0;
  if (k_wave) {
    key0 = wave * 32 + (lane & 31);
    col0 = (lane >> 5) * 16;
  } else {
    const int lp = lane & 31;
    key0 = 32 * (wave - 2) + 4 * (lp >> 4) + ((lp & 7) >> 1);
    col0 = 2 * ((lane >> 5) * 32 + 16 * ((lp >> 3) & 1) + 8 * (lp & 1));
  }
  const int32_t off0 = key0 * (kD * 2) + col0;
  const uint32_t ring_lds = lds_address(ring) + wave * kDmaPerWave * 1024;

  // This wave's tensor (K or V) of current-scale tile c into stage c % 2.
  auto issue_cur = [&](int c) {
    const uint32_t dst = ring_lds + (c % NS) * kStageBytes;
    const uint32_t skip = static_cast<uint32_t>(c) * (kBN * kD * 2);
    const u32x4_t d_cur = make_desc(cur_base + skip, cur_bytes - skip);
    if (k_wave) {
      dma16_at<0>(d_cur, dst, off0);
      dma16_at<32>(d_cur, dst + 1024, off0);
      dma16_at<64>(d_cur, dst + 2048, off0);
      dma16_at<96>(d_cur, dst + 3072, off0);
      dma16_at<128>(d_cur, dst + 4096, off0);
      dma16_at<160>(d_cur, dst + 5120, off0);
      dma16_at<192>(d_cur, dst + 6144, off0);
      dma16_at<224>(d_cur, dst + 7168, off0);
    } else {
      dma16_at<0>(d_cur, dst, off0);
      dma16_at<128>(d_cur, dst + 1024, off0);
      dma16_at<2048>(d_cur, dst + 2048, off0);
      dma16_at<2176>(d_cur, dst + 3072, off0);
      dma16_at<4096>(d_cur, dst + 4096, off0);
      dma16_at<4224>(d_cur, dst + 5120, off0);
      dma16_at<6144>(d_cur, dst + 6144, off0);
      dma16_at<6272>(d_cur, dst + 7168, off0);
    }
  };
  // A planned unit whose first tile is a current-scale one (every whole item,
  // and a part that starts there) issues it before the head's segment tables
  // are loaded, and Q with it: the tables, the tile and Q arrive in one round
  // trip.
  const int32_t first = cut ? (p0 < 0 ? 0 : p0) : 0;
  const bool early = planned && first < ntc;
  if (early) issue_cur(first);

  // Q: its loads are in flight while the tables load and wave 0 fills the row tables
  const int32_t qrow = w.qt * kBM + wave * 32 + (lane & 31);
  u32x4_t qf[8];
  {
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(
        static_cast<const uint8_t*>(a.q) + cur_row0 * kD * 2, static_cast<uint32_t>(L * kD * 2));
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qf[ks] = load8<QDT, MQK>(rq, qrow < L ? (qrow * kD + ks * 16 + g * 8) * 2 : -1);
  }

  if (planned) {
    load_head_segments<kThreads>(a.seg_starts, a.seg_ends, a.seg_counts, cap, a.max_segments, w, seg_start,
                                 seg_pref);
    const int32_t ntiles = (w.R + kBN - 1) / kBN + ntc;
    t_begin = p0 < 0 ? 0 : (p0 > ntiles ? ntiles : p0);
    t_end = p1 < t_begin ? t_begin : (p1 > ntiles ? ntiles : p1);
    if (!cut) {  // a whole item, whatever the plan's range says
      t_begin = 0;
      t_end = ntiles;
    }
    if (t_begin >= t_end && !cut) {
      wait_vmcnt<0>();  // the early tile lands before the workgroup's LDS is released
      return;
    }
  } else {
    const int32_t ntiles = (w.R + kBN - 1) / kBN + ntc;
    // A part needs kMinPartTiles key tiles to pay for its record and the
    // merge, so a short item runs as fewer parts (one, below two such runs);
    // every part of the item sees the same tile count and agrees.  Parts past
    // the count leave at once.
    parts = ntiles / kMinPartTiles;
    parts = parts < 1 ? 1 : (parts < un.parts ? parts : un.parts);
    if (un.part >= parts) return;
    t_begin = un.part * ntiles / parts;
    t_end = (un.part + 1) * ntiles / parts;
  }
  const int32_t R = w.R;
  if (t_begin >= t_end) {
    // a planned part with no key tiles (a plan that does not match these
    // tables): its record is empty -- zero weight in the merge
    wait_vmcnt<0>();
    f32x16_t none[4] = {};
    merge_parts<QDT, kThreads>(a, sc, un, parts, none, -1e30f, 0.f, w, qrow, L, H, g, merge_turn,
                               ring + wave * 32 * kOutPitch);
    return;
  }

  // This wave's tensor (K or V) of tile `tile` into stage tile % 2.
  auto issue_tile = [&](int tile) {
    if (tile < ntc) {
      issue_cur(tile);
      return;
    }
    const int p = tile - ntc;
    const uint32_t dst = ring_lds + (tile % NS) * kStageBytes;
    const int32_t* rt = rowtab[p % 3];
    if (k_wave) {
      const int32_t r = rt[key0] + col0;
      dma16_at<0>(d_prior, dst, r);
      dma16_at<32>(d_prior, dst + 1024, r);
      dma16_at<64>(d_prior, dst + 2048, r);
      dma16_at<96>(d_prior, dst + 3072, r);
      dma16_at<128>(d_prior, dst + 4096, r);
      dma16_at<160>(d_prior, dst + 5120, r);
      dma16_at<192>(d_prior, dst + 6144, r);
      dma16_at<224>(d_prior, dst + 7168, r);
    } else {
      const int32_t r0 = rt[key0] + col0, r1 = rt[key0 + 8] + col0;
      const int32_t r2 = rt[key0 + 16] + col0, r3 = rt[key0 + 24] + col0;
      dma16_at<0>(d_prior, dst, r0);
      dma16_at<128>(d_prior, dst + 1024, r0);
      dma16_at<0>(d_prior, dst + 2048, r1);
      dma16_at<128>(d_prior, dst + 3072, r1);
      dma16_at<0>(d_prior, dst + 4096, r2);
      dma16_at<128>(d_prior, dst + 5120, r2);
      dma16_at<0>(d_prior, dst + 6144, r3);
      dma16_at<128>(d_prior, dst + 7168, r3);
    }
  };
  auto valid_of = [&](int t) { return t < ntc ? min(kBN, L - t * kBN) : min(kBN, R - (t - ntc) * kBN); };

  int cur_seg = 0;
  if (wave == 0) {
    for (int t = t_begin; t < t_begin + 3 && t < t_end; ++t)
      if (t >= ntc)
        fill_rowtab<kD * 2>(t - ntc, rowtab[(t - ntc) % 3], cur_seg, w.nseg, R, seg_start, seg_pref, kPastEnd);
  }
  __syncthreads();
  if (!early) issue_tile(t_begin);
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) qf[ks] ^= sc.q_sign;

  f32x16_t oacc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) oacc[i] = f32x16_t{};
  float m_run = -1e30f;
  float l_run = 0.f;

  // S(t) = K(t) Q^T from stage t % 2, one key block's 8 k-steps after the
  // other (each accumulator a chain of 8 MFMAs; 0.7-0.8 % faster on the 2B
  // and 8B final steps than alternating the two blocks, same sums)
  auto qk = [&](f32x16_t (&sx)[2], int t) {
    const uint8_t* kst = ring + (t % NS) * kStageBytes + lane * 16;
    sx[0] = f32x16_t{};
    sx[1] = f32x16_t{};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const u32x4_t kf = *reinterpret_cast<const u32x4_t*>(kst + (kb * 8 + ks) * 1024);
        sx[kb] = mfma32<MQK>(kf, qf[ks], sx[kb]);
      }
  };
  // O^T += V(t)^T P(t)^T from stage t % 2
  auto pv = [&](const u32x4_t (&pf)[4], int t) {
    const uint8_t* vst = ring + (t % NS) * kStageBytes + kTileBytes + lane * 8;
#pragma unroll
    for (int u = 0; u < kBN / 16; ++u)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int blk = (db >> 1) * 1024 + (db & 1) * 512;
        const u32x2_t lo = ds_read_tr(vst + (u * 4 + 0) * 1024 + blk);
        const u32x2_t hi = ds_read_tr(vst + (u * 4 + 2) * 1024 + blk);
        const u32x4_t vf = {lo[0], lo[1], hi[0], hi[1]};
        oacc[db] = mfma32<MV>(vf, pf[u], oacc[db]);
      }
  };
  auto pack = [&](const f32x16_t (&sx)[2], u32x4_t (&pf)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) pf[u] = p_operand<MV>(sx, u);
  };

  // Prologue: K(t0), V(t0) landed; K(t0 + 1) in flight; S(t0) and its max.
  wait_vmcnt<0>();
  __syncthreads();
  if (k_wave && t_begin + 1 < t_end) issue_tile(t_begin + 1);
  f32x16_t sa[2], sb[2];
  qk(sa, t_begin);
  if (valid_of(t_begin) < kBN) mask_tile(sa, valid_of(t_begin), g);
  move_max(oacc, m_run, l_run, tile_max(sa), sc.c, sc.thresh);

  // Iteration t: scur = S(t) (max applied), snext receives S(t + 1).
  auto step = [&](f32x16_t (&scur)[2], f32x16_t (&snext)[2], int t) {
    // The two workgroups of a CU share its SIMDs, whose issue favours the
    // older waves, so one item ran at a fraction of the other's rate until
    // it finished.  With items of unequal length (as the plan marks them)
    // the priority alternates by tile, with the workgroup id in the parity,
    // so the SIMDs are shared tile by tile and the items progress as the
    // plan assumes: -1.9 % on the 2B final step, -1 to -3 % on the sweep's
    // last scales; equal items (+3 % with it) keep the hardware's order.
    if (shared) {
      if (((t + static_cast<int>(blockIdx.x)) & 1) == 0)
        __builtin_amdgcn_s_setprio(1);
      else
        __builtin_amdgcn_s_setprio(0);
    }
    wait_vmcnt<0>();  // this wave's K(t + 1) or V(t)
    __syncthreads();
    if (k_wave) {
      if (t + 2 < t_end) issue_tile(t + 2);
    } else {
      if (t + 1 < t_end) issue_tile(t + 1);
    }
    if (wave == 0 && t + 3 < t_end && t + 3 >= ntc)
      fill_rowtab<kD * 2>(t + 3 - ntc, rowtab[(t + 3 - ntc) % 3], cur_seg, w.nseg, R, seg_start, seg_pref,
                          kPastEnd);
    u32x4_t pf[4];
    qk(snext, t + 1);
    exp_tile(scur, m_run, sc.c, l_run);
    pack(scur, pf);
    pv(pf, t);
    // The row sum and the max of a whole S(t + 1) are pinned to this block
    // (empty asm uses), so the scheduler interleaves them with the PV MFMAs
    // instead of sinking them past the branch of the rare partial-tile mask,
    // which then takes the max again (0.8-1 % faster on the 2B and 8B final
    // steps).
    asm volatile("" : "+v"(l_run));
    float mx = tile_max(snext);
    asm volatile("" : "+v"(mx));
    const int vn = valid_of(t + 1);
    if (vn < kBN) {
      mask_tile(snext, vn, g);
      mx = tile_max(snext);
    }
    move_max(oacc, m_run, l_run, mx, sc.c, sc.thresh);
  };
  int t = t_begin;
  for (; t + 2 < t_end; t += 2) {
    step(sa, sb, t);
    step(sb, sa, t + 1);
  }
  if (t + 1 < t_end) {
    step(sa, sb, t);
    ++t;
    // the last tile is in sb
    wait_vmcnt<0>();
    __syncthreads();
    u32x4_t pf[4];
    exp_tile(sb, m_run, sc.c, l_run);
    pack(sb, pf);
    pv(pf, t);
  } else {
    wait_vmcnt<0>();
    __syncthreads();
    u32x4_t pf[4];
    exp_tile(sa, m_run, sc.c, l_run);
    pack(sa, pf);
    pv(pf, t);
  }

  __builtin_amdgcn_s_setprio(0);
  if (parts == 1) {
    if (a.out_dtype != kF32 && (reinterpret_cast<uintptr_t>(a.out) & 15) == 0) {
      static_assert(NS * kStageBytes >= NW * 32 * kOutPitch, "output staging fits the ring");
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
  merge_parts<QDT, kThreads>(a, sc, un, parts, oacc, m_run, l_run, w, qrow, L, H, g, merge_turn,
                             ring + wave * 32 * kOutPitch);
}

// Resident workgroups of the kernel (2 per CU) on `device`, cached.
int32_t slots_of(int device) {
  static int32_t cache[64] = {};
  if (device < 0 || device >= 64) return 0;
  if (cache[device] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0)
      return 0;
    cache[device] = 2 * cus < kMaxCounters ? 2 * cus : kMaxCounters;  // a counter per slot
  }
  return cache[device];
}

template <int DT, int VDT>
hipError_t launch(const AttnArgs& a, const Scalars& s, hipStream_t st) {
  constexpr int kBM = 128;
  const int32_t n_qt = (a.cur_len + kBM - 1) / kBM;
  const int64_t items = static_cast<int64_t>(a.batch) * a.heads * n_qt;
  if (items <= 0) return hipSuccess;
  if (items > 0x3fffffffLL) return hipErrorInvalidConfiguration;
  // With a workspace, some items are cut in two so the launch fills whole rounds of slots.
  int device = 0;
  const int32_t slots = a.workspace != nullptr && hipGetDevice(&device) == hipSuccess ? slots_of(device) : 0;
  RoundSplit split{static_cast<int32_t>(items), 0, 0, 0};
  if (slots > 0 && a.workspace_bytes >= split_workspace_bytes(slots))
    split = round_split(static_cast<int32_t>(items), slots, (a.cur_len + kBN - 1) / kBN);
  AttnArgs b = a;
  b.ws_cuts = 0;
  if (a.workspace != nullptr && a.workspace_bytes > kCounterBytes) {
    const int64_t by_records = (a.workspace_bytes - kCounterBytes) / (2LL * kPartialFloats * 4);
    b.ws_cuts = static_cast<int32_t>(by_records < kMaxCounters ? by_records : kMaxCounters);
  }
  // the fused append's copy blocks follow the attention workgroups
  const int64_t copies = a.append_offsets != nullptr ? append_blocks(a.batch, a.heads, a.cur_len) : 0;
  const int64_t blocks = a.plan != nullptr ? (a.plan_units > 0 ? a.plan_units : 0) : split_units(split);
  if (blocks + copies <= 0) return hipSuccess;
  if (blocks + copies > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  b.append_first = static_cast<int32_t>(blocks);
  seg_attn_pipe_kernel<DT, DT, VDT><<<dim3(static_cast<uint32_t>(blocks + copies)), 256, 0, st>>>(
      b.plan, b.plan != nullptr ? static_cast<int32_t>(blocks) : 0, b, s, n_qt, split);
  return hipGetLastError();
}

}  // namespace

int32_t split_slots(int device) { return slots_of(device); }

int64_t split_workspace_bytes(int32_t slots) {
  if (slots <= 0) return 0;
  // at most one cut item per slot: counters and 2 records per slot
  return kCounterBytes + 2LL * slots * kPartialFloats * static_cast<int64_t>(sizeof(float));
}

bool attention_direct_supported(const AttnArgs& a) {
  const bool k16 = a.k_dtype == kBF16 || a.k_dtype == kF16;
  const bool v16 = a.v_dtype == kBF16 || a.v_dtype == kF16;
  // 16-bit q/k products are exact in every QK dot mode; an fp32 P V product
  // (value mode 2) needs the staged kernel's split P
  return k16 && v16 && a.q_dtype == a.k_dtype && a.heads <= attn::kMaxHeads && a.value_dot_mode != kDotFp32;
}

hipError_t launch_attention_direct(const AttnArgs& a, const attn::Scalars& s, hipStream_t stream) {
  if (!attention_direct_supported(a)) return hipErrorInvalidValue;
  if (a.k_dtype == kBF16)
    return a.v_dtype == kBF16 ? launch<kBF16, kBF16>(a, s, stream) : launch<kBF16, kF16>(a, s, stream);
  return a.v_dtype == kBF16 ? launch<kF16, kBF16>(a, s, stream) : launch<kF16, kF16>(a, s, stream);
}

}  // namespace hkv
