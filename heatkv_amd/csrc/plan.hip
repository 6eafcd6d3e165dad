// Host-side work plan of the 16-bit segmented-attention kernel.
//
// Without a plan every workgroup of the kernel computes the launch's work
// order from the device offset tables itself (heaviest head first, and the
// round split), a few microseconds per workgroup.  The tables of a (layer,
// target) do not change during a generation, so the caller can build the
// order once on the host from its copy of the tables and pass it with every
// call (as the reference uploads its offset tables once per layer and target,
// enable_real_pruning_fast.py:592-608).  A plan is a list of units, one per
// workgroup in dispatch order: a whole item (b, h, query tile of the
// kernel's bm queries) or one of the two key-range parts of a cut item,
// and whether the 16-bit kernel shares a CU's SIMDs tile by tile (items of
// unequal length).
//
// Choosing the cuts.  The hardware dispatches workgroups in id order to
// whatever slot frees first, i.e. list scheduling.  The plan simulates it
// over the device's resident slots (2 per CU) with a per-unit cost of its key
// tiles plus a fixed overhead (a part pays more: it publishes and merges a
// partial record), for cutting the k heaviest items at a fraction f of their
// tiles, whole items first (heaviest first), then the parts (longest first),
// and keeps the (k, f) with the shortest simulated makespan.  Launches with
// many rounds of items per slot balance without cuts and are not searched.
//
// Keeping a head's key/value rows in few L2s.  The 8 XCDs take workgroup ids
// round robin (id % 8), each with its own L2 and resident slots.  A launch
// whose query tiles of one (batch row, head) group are dealt over all XCDs
// reads that group's K/V into every L2.  A searched plan of at least two
// rounds of items therefore deals chunks of a group's query tiles to XCDs
// (heaviest first, each to the least loaded XCD), searches the cuts of each
// XCD's items over its own slots, and interleaves the 8 XCDs' unit lists
// (unit i of XCD x at id 8 i + x), padding the shorter lists with empty units
// that leave at once.  Whole groups per XCD read the least; half and quarter
// groups mix heavy and light items on an XCD, which its slots balance
// better: the chunk with the shortest simulated makespan is kept.  On the 2B
// final step (B = 2, 16 heads, L = 4096) quarters win: K/V is read into 4
// L2s instead of 8, and the simulated makespan equals the single-list plan's.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <functional>
#include <queue>
#include <vector>

#include "hkv_internal.h"

namespace hkv {
namespace {

constexpr int kPlanBN = 64;            // keys per tile
constexpr int kPlanMinPartTiles = 4;   // a part must have this many key tiles
constexpr double kUnitOverTiles = 1.5;  // start-up of a workgroup, in key-tile times
constexpr double kPartOverTiles = 4.0;  // record publish + merge of a part
constexpr int kNoSearchRounds = 4;     // items per slot above which nothing is cut
constexpr int kXcds = 8;               // L2 domains; workgroup id % 8 selects one

struct Item {
  int32_t h, j, n;
};

double simulate(const std::vector<std::pair<int32_t, bool>>& units, int slots) {
  std::priority_queue<double, std::vector<double>, std::greater<double>> free_at;
  for (int s = 0; s < slots; ++s) free_at.push(0.0);
  double end = 0.0;
  for (const auto& u : units) {
    const double t = free_at.top();
    free_at.pop();
    const double f = t + u.first + kUnitOverTiles + (u.second ? kPartOverTiles : 0.0);
    end = std::max(end, f);
    free_at.push(f);
  }
  return end;
}

struct Cut {
  int32_t k = 0;   // heaviest items cut
  double f = 0.5;  // fraction of an item's tiles in its first part
};

int32_t first_part(int32_t n, double f) {
  int32_t a = static_cast<int32_t>(n * f + 0.5);
  return std::min(std::max(a, kPlanMinPartTiles), n - kPlanMinPartTiles);
}

bool cuttable(int32_t n) { return n >= 2 * kPlanMinPartTiles; }

std::vector<std::pair<int32_t, bool>> units_for(const std::vector<Item>& items, const Cut& c) {
  std::vector<std::pair<int32_t, bool>> whole, parts;
  for (size_t i = 0; i < items.size(); ++i) {
    const int32_t n = items[i].n;
    if (static_cast<int32_t>(i) < c.k && cuttable(n)) {
      const int32_t a = first_part(n, c.f);
      parts.push_back({a, true});
      parts.push_back({n - a, true});
    } else {
      whole.push_back({n, false});
    }
  }
  std::stable_sort(parts.begin(), parts.end(), [](const auto& x, const auto& y) { return x.first > y.first; });
  whole.insert(whole.end(), parts.begin(), parts.end());
  return whole;
}

// The best cut of `items` (heaviest first) over `slots` resident slots, with
// at most `kmax` cut items (one counter and two records each), and its
// simulated makespan.
Cut search_cuts(const std::vector<Item>& items, int slots, int32_t kmax, double* makespan = nullptr) {
  Cut best;
  const int32_t N = static_cast<int32_t>(items.size());
  const bool any_cuttable = std::any_of(items.begin(), items.end(), [](const Item& it) { return cuttable(it.n); });
  double best_t = simulate(units_for(items, best), slots);
  if (makespan != nullptr) *makespan = best_t;
  if (slots <= 0 || N >= kNoSearchRounds * slots || !any_cuttable) return best;
  kmax = std::min(N, kmax);
  const int32_t step = std::max(1, slots / 32);
  for (int32_t k = step; k <= kmax; k += step) {
    for (double f : {0.3, 0.35, 0.4, 0.45, 0.5, 0.55, 0.6, 0.65, 0.7}) {
      const Cut c{k, f};
      const double t = simulate(units_for(items, c), slots);
      if (t < best_t * 0.995) {
        best_t = t;
        best = c;
      }
    }
  }
  if (makespan != nullptr) *makespan = best_t;
  return best;
}

// Deals chunks of `per_group` consecutive items (one group's query tiles:
// equal tile counts; heaviest group first) to the XCDs: each chunk goes whole
// to the least loaded XCD unless that would pass the XCD's share of the work
// by more than half an item; then the XCD is filled to its share and the rest
// of the chunk moves on to the next least loaded one.  Each XCD's list stays
// heaviest first.
std::vector<std::vector<Item>> deal_groups(const std::vector<Item>& items, int32_t per_group) {
  std::vector<std::vector<Item>> xi(kXcds);
  double load[kXcds] = {};
  double total = 0.0;
  for (const Item& it : items) total += it.n + kUnitOverTiles;
  const double share = total / kXcds;
  const int32_t N = static_cast<int32_t>(items.size());
  for (int32_t g0 = 0; g0 < N; g0 += per_group) {
    const double c = items[g0].n + kUnitOverTiles;
    int32_t q = 0;
    while (q < per_group) {
      const int x = static_cast<int>(std::min_element(load, load + kXcds) - load);
      int32_t take = per_group - q;
      if (load[x] + take * c > share + 0.5 * c) {
        const int32_t fit = static_cast<int32_t>(std::lround((share - load[x]) / c));
        take = std::min(std::max(fit, 1), per_group - q);
      }
      for (int32_t i = 0; i < take; ++i) xi[x].push_back(items[g0 + q + i]);
      load[x] += take * c;
      q += take;
    }
  }
  return xi;
}

// Workgroup j's item when every item is whole: the 8 XCDs take workgroup ids
// round robin (j % 8), so with at least 8 (head, batch row) groups per XCD the
// query tiles of one group are dealt to one XCD (groups snake over the XCDs),
// sharing its L2.  Identity otherwise.
int32_t xcd_order(int32_t j, int32_t groups, int32_t n_qt) {
  if (groups % kXcds != 0 || groups < 8 * kXcds) return j;
  const int32_t x = j % kXcds;
  const int32_t k = j / kXcds;
  const int32_t lg = k / n_qt;
  const int32_t qt = k - lg * n_qt;
  const int32_t group = lg * kXcds + ((lg & 1) ? kXcds - 1 - x : x);
  return group * n_qt + qt;
}

// HKV_PLAN_DEAL=0 turns the dealing to XCDs off (one list for all slots), to
// measure what it gains.
bool deal_enabled() {
  const char* e = std::getenv("HKV_PLAN_DEAL");
  return e == nullptr || e[0] != '0';
}

}  // namespace

int32_t build_attention_plan(const int32_t* seg_starts, const int32_t* seg_ends, const int32_t* seg_counts,
                             int32_t H, int32_t S, int64_t cap, int32_t B, int32_t L, int32_t bm, int32_t slots,
                             int32_t* out, int32_t max_units) {
  const int32_t n_qt = (L + bm - 1) / bm;
  const int32_t ntc = (L + kPlanBN - 1) / kPlanBN;
  std::vector<int64_t> rows(H, 0);
  for (int32_t h = 0; h < H; ++h) {
    int32_t n = seg_counts[h];
    n = n < 0 ? 0 : (n > S ? S : n);
    for (int32_t i = 0; i < n; ++i) {
      int64_t st = seg_starts[static_cast<int64_t>(h) * S + i];
      int64_t en = seg_ends[static_cast<int64_t>(h) * S + i];
      st = st < 0 ? 0 : (st > cap ? cap : st);
      en = en < 0 ? 0 : (en > cap ? cap : en);
      rows[h] += en > st ? en - st : 0;
    }
  }
  // heads heaviest first (ties by index); within a head its items in order
  std::vector<int32_t> heads(H);
  for (int32_t h = 0; h < H; ++h) heads[h] = h;
  std::stable_sort(heads.begin(), heads.end(), [&](int32_t x, int32_t y) { return rows[x] > rows[y]; });
  const int32_t per_h = B * n_qt;
  std::vector<Item> items;
  items.reserve(static_cast<size_t>(H) * per_h);
  for (int32_t h : heads) {
    const int32_t n = static_cast<int32_t>((rows[h] + kPlanBN - 1) / kPlanBN) + ntc;
    for (int32_t j = 0; j < per_h; ++j) items.push_back({h, j, n});
  }
  const int32_t N = static_cast<int32_t>(items.size());
  // Items of unequal length (more than 5/4 between the longest and the
  // shortest): the kernel shares a CU's SIMDs between its two workgroups
  // tile by tile (wave priority), so the items progress at the rates the
  // dispatch simulation assumes.  Equal items (every head keeping as many
  // rows) balance without it and run faster when the workgroups drift apart.
  int32_t n_min = 0, n_max = 0;
  for (const Item& it : items) {
    n_min = n_min == 0 || it.n < n_min ? it.n : n_min;
    n_max = it.n > n_max ? it.n : n_max;
  }
  const int32_t shared = 4LL * n_max > 5LL * n_min ? 1 : 0;

  // units in dispatch order, one list per XCD (a single list when not dealt)
  struct Unit {
    int32_t h, j, t0, t1, cut, part;
  };
  int32_t cuts = 0;
  auto make_units = [&](const std::vector<Item>& its, const Cut& c, std::vector<Unit>& dst) {
    std::vector<Unit> parts;
    for (int32_t i = 0; i < static_cast<int32_t>(its.size()); ++i) {
      const Item& it = its[i];
      if (i < c.k && cuttable(it.n)) {
        const int32_t a = first_part(it.n, c.f);
        parts.push_back({it.h, it.j, 0, a, cuts, 0});
        parts.push_back({it.h, it.j, a, it.n, cuts, 1});
        ++cuts;
      } else {
        dst.push_back({it.h, it.j, 0, it.n, -1, 0});
      }
    }
    std::stable_sort(parts.begin(), parts.end(),
                     [](const Unit& x, const Unit& y) { return x.t1 - x.t0 > y.t1 - y.t0; });
    const bool had_parts = !parts.empty();
    dst.insert(dst.end(), parts.begin(), parts.end());
    return had_parts;
  };

  const bool searched = slots > 0 && N < kNoSearchRounds * slots &&
                        std::any_of(items.begin(), items.end(), [](const Item& it) { return cuttable(it.n); });
  const bool dealt = searched && N >= 2 * slots && slots % kXcds == 0 && H * B >= kXcds && deal_enabled();
  std::vector<std::vector<Unit>> lists;
  bool grouped = false;  // whole items only, in XCD groups by xcd_order
  if (dealt) {
    // Whole groups per XCD first; halves and quarters of groups (a group's
    // K/V then read into two or four L2s) when they shorten the simulated
    // makespan by more than 1%: mixing heavy and light items on an XCD
    // balances its slots better.
    std::vector<std::vector<Item>> best_xi;
    std::vector<Cut> best_cuts;
    double best_t = 0.0;
    for (int32_t chunk = n_qt; chunk >= 1 && chunk * 4 >= n_qt; chunk /= 2) {
      if (n_qt % chunk != 0) break;
      std::vector<std::vector<Item>> xi = deal_groups(items, chunk);
      std::vector<Cut> cs(kXcds);
      double t = 0.0;
      for (int x = 0; x < kXcds; ++x) {
        double tx = 0.0;
        cs[x] = search_cuts(xi[x], slots / kXcds, slots / kXcds, &tx);
        t = std::max(t, tx);
      }
      if (best_xi.empty() || t < best_t * 0.99) {
        best_t = t;
        best_xi = std::move(xi);
        best_cuts = cs;
      }
    }
    lists.resize(kXcds);
    for (int x = 0; x < kXcds; ++x) make_units(best_xi[x], best_cuts[x], lists[x]);
  } else {
    lists.resize(1);
    const Cut c = searched ? search_cuts(items, slots, slots) : Cut{};
    grouped = !make_units(items, c, lists[0]);
  }
  size_t longest = 0;
  for (const auto& l : lists) longest = std::max(longest, l.size());
  const int32_t n_units = static_cast<int32_t>(longest * lists.size());
  if (out == nullptr) return n_units;
  if (n_units > max_units) return -1;
  auto emit = [&](int32_t u, const Unit* x) {
    int32_t* o = out + static_cast<int64_t>(u) * kPlanInts;
    if (x == nullptr) {  // an empty unit: the workgroup leaves at once
      o[0] = -1;
      o[1] = -1;
      o[2] = 0;
      o[3] = 0;
      o[4] = -1;
      o[5] = 0;
    } else {
      o[0] = x->h;
      o[1] = x->j;
      o[2] = x->t0;
      o[3] = x->t1;
      o[4] = x->cut;
      o[5] = x->part;
    }
    o[6] = x == nullptr ? 0 : shared;
    // a cut item's two parts count in first; the second writes no record
    o[7] = x != nullptr && x->cut >= 0 ? 1 : 0;
  };
  if (lists.size() == 1) {
    const std::vector<Unit>& l = lists[0];
    for (int32_t k = 0; k < n_units; ++k) emit(k, &l[grouped ? xcd_order(k, H * B, n_qt) : k]);
  } else {
    for (size_t i = 0; i < longest; ++i)
      for (int x = 0; x < kXcds; ++x)
        emit(static_cast<int32_t>(i * kXcds + x), i < lists[x].size() ? &lists[x][i] : nullptr);
  }
  return n_units;
}

}  // namespace hkv
