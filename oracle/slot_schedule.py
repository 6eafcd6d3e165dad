"""Restatement of the reference's static slab allocator (test infrastructure only).

Follows, step for step, enable_real_pruning_fast.py:

* ``capacity_bound``            -- ``_segmented_flat_cache_capacity_for_layer`` (:206-234)
* ``build_schedule``            -- ``_segmented_flat_build_static_slot_schedule`` (:260-558)
* ``merge_free_blocks``         -- ``_segmented_flat_merge_free_blocks`` (:1033-1047)
* ``flatten_copy_items``        -- ``_segmented_flat_static_copy_metadata_for_runs`` (:610-671)

and the policy lookup of ``ScaleSpecificPruningController``
(enable_pruning.py:380-401) with ``_scale_token_ranges`` (:182-189).

Pinning (tests/test_oracle_schedule.py):

* static keep policies (every (head, source) pair either kept for every target
  or never): offsets equal the exclusive prefix sum of token counts over kept
  pairs in (source asc, head asc) order -- a closed form independent of this
  code;
* hand-worked progressive-removal cases whose best-fit placements were derived
  on paper (reuse of a freed block, tie to the lowest offset, merge of adjacent
  free blocks, bump allocation);
* invariants at every target: live segments pairwise disjoint, inside
  ``[0, capacity)``, tables sorted by source scale, ``counts[h]`` equal to the
  number of live pairs of head h, and capacity >= the live row count.

* under the HeatKV policy's progressive removal (orders/2b.json at budgets
  0.1 and 0.35, all 32 layers), the product allocator is compared with the
  reference's own allocator function (tests/golden/slab_2b.json, written by
  tests/golden/make_slab_golden.py, which compiles and runs just that
  function from the reference module's text: the module imports ``timm`` /
  ``flash_attn`` through ``infinity.models.basic`` and cannot be imported
  here), and this restatement with the product on the same removal sets.
"""

from __future__ import annotations

import numpy as np

SIDES_13 = (1, 2, 4, 6, 8, 12, 16, 20, 24, 32, 40, 48, 64)


def scale_token_ranges(sides):
    """``{scale: (start, end)}`` token ranges for square scales (enable_pruning.py:182-189)."""
    ranges = {}
    cursor = 0
    for i, side in enumerate(sides):
        nxt = cursor + int(side) * int(side)
        ranges[i] = (cursor, nxt)
        cursor = nxt
    return ranges


class PolicyView:
    """Policy lookup of ScaleSpecificPruningController (enable_pruning.py:380-401).

    ``static_removed[target][source][layer] -> set(heads)``.  A target missing
    from the map falls back to the largest present target <= it; with none, every
    source in ``[source_start, source_end]`` maps to an empty set.
    """

    def __init__(self, static_removed, *, num_layers, source_start=4, source_end=11):
        self.static_removed = static_removed
        self.num_layers = int(num_layers)
        self.source_start = int(source_start)
        self.source_end = int(source_end)

    def _state(self, target):
        if target in self.static_removed:
            return self.static_removed[target]
        lower = [t for t in self.static_removed if t <= target]
        if not lower:
            return {
                s: {layer: set() for layer in range(self.num_layers)}
                for s in range(self.source_start, self.source_end + 1)
            }
        return self.static_removed[max(lower)]

    def removed_heads_by_source_for(self, layer, target):
        state = self._state(target)
        return {s: set(by_layer.get(layer, set())) for s, by_layer in state.items()}


def capacity_bound(policy, scale_ranges, num_scales, layer, num_heads):
    """Max over targets of live rows if nothing is freed (:206-234)."""
    best = 0
    for target in range(1, num_scales):
        removed = policy.removed_heads_by_source_for(layer, target)
        total = 0
        for source, (a, b) in scale_ranges.items():
            if int(source) >= target:
                continue
            n = int(b) - int(a)
            if n <= 0:
                continue
            total += (int(num_heads) - len(removed.get(int(source), set()))) * n
        best = max(best, total)
    return best


def merge_free_blocks(blocks):
    """Sort by offset and coalesce overlapping/adjacent blocks (:1033-1047)."""
    out = []
    for off, ln in sorted((int(o), int(l)) for o, l in blocks if int(l) > 0):
        if out and off <= out[-1][0] + out[-1][1]:
            end = max(out[-1][0] + out[-1][1], off + ln)
            out[-1][1] = end - out[-1][0]
        else:
            out.append([off, ln])
    return [(o, l) for o, l in out]


def _intervals(policy, scale_ranges, num_scales, layer, num_heads):
    """(:276-307) one interval per (source, head) alive for >= 1 target."""
    res = []
    for source in sorted(scale_ranges):
        a, b = scale_ranges[source]
        first = int(source) + 1
        if first >= num_scales:
            continue
        n = int(b) - int(a)
        if n <= 0:
            continue
        for head in range(int(num_heads)):
            stop = num_scales
            for target in range(first, num_scales):
                if head in policy.removed_heads_by_source_for(layer, target).get(int(source), set()):
                    stop = target
                    break
            if stop <= first:
                continue
            res.append(dict(source_scale=int(source), head=head, start_target=first,
                            end_target=int(stop), length=n, scale_start=int(a), scale_end=int(b)))
    return res


def _allocate(intervals):
    """Best-fit with lowest-offset tie break, frees before each placement (:309-363)."""
    free = []
    live = []
    high = 0
    placed = []
    order = sorted(intervals, key=lambda it: (it["start_target"], it["end_target"],
                                              -it["length"], it["source_scale"], it["head"]))
    for it in order:
        keep = []
        for other in live:
            if other["end_target"] <= it["start_target"]:
                free.append((other["offset"], other["length"]))
            else:
                keep.append(other)
        live = keep
        free = merge_free_blocks(free)
        need = it["length"]
        best = None  # (leftover, index, offset, length)
        for i, (off, ln) in enumerate(free):
            if ln < need:
                continue
            cand = (ln - need, i, off, ln)
            if best is None or (cand[0], cand[2]) < (best[0], best[2]):
                best = cand
        if best is not None:
            _, i, off, ln = best
            if ln == need:
                del free[i]
            else:
                free[i] = (off + need, ln - need)
            where = off
        else:
            where = high
            high += need
        seg = dict(it)
        seg["offset"] = int(where)
        placed.append(seg)
        live.append(seg)
    return placed, high


def _tables(placed, num_scales, num_heads):
    """Per-target (starts, ends, counts) int32 tables (:379-412)."""
    by_target = {}
    tables = {}
    for target in range(1, num_scales):
        alive = [s for s in placed if s["start_target"] <= target < s["end_target"]]
        by_target[target] = alive
        per_head = [[] for _ in range(num_heads)]
        for s in alive:
            per_head[s["head"]].append(s)
        width = max((len(x) for x in per_head), default=0)
        st = np.zeros((num_heads, width), dtype=np.int32)
        en = np.zeros((num_heads, width), dtype=np.int32)
        ct = np.zeros((num_heads,), dtype=np.int32)
        for h, items in enumerate(per_head):
            items = sorted(items, key=lambda s: s["source_scale"])
            ct[h] = len(items)
            for i, s in enumerate(items):
                st[h, i] = s["offset"]
                en[h, i] = s["offset"] + s["length"]
        tables[target] = (st, en, ct)
    return by_target, tables


def _copy_runs(items, sequence_len):
    """``build_copy_runs`` (:414-482): group by contiguous destination."""
    runs = []
    cur = None
    for it in sorted(items, key=lambda v: int(v["dst_offset"])):
        dst = int(it["dst_offset"])
        n = int(it["length"])
        if n <= 0:
            continue
        if cur is not None and dst != cur["dst_end"]:
            runs.append(cur)
            cur = None
        if cur is None:
            cur = dict(dst_start=dst, dst_end=dst, sequence_len=int(sequence_len), copy_items=[])
        cur["copy_items"].append(dict(dst_start=dst,
                                      src_start=int(it["head"]) * int(sequence_len) + int(it["src_start"]),
                                      length=n))
        cur["dst_end"] += n
    if cur is not None and cur["copy_items"]:
        runs.append(cur)
    return runs


def flatten_copy_items(runs):
    """(:610-645) concatenated copy items of a run list, or None when empty."""
    items = [c for r in runs for c in r["copy_items"]]
    if not items:
        return None
    lengths = [c["length"] for c in items]
    return dict(dst_starts=[c["dst_start"] for c in items],
                src_starts=[c["src_start"] for c in items],
                lengths=lengths, max_length=max(lengths), slots=sum(lengths),
                item_count=len(items))


def build_schedule(policy, scale_ranges, *, layer, num_heads, allow_overalloc=True):
    """Static slot schedule for one layer (:260-558)."""
    num_scales = len(scale_ranges)
    bound = capacity_bound(policy, scale_ranges, num_scales, layer, num_heads)
    placed, high = _allocate(_intervals(policy, scale_ranges, num_scales, layer, num_heads))
    if high > bound and not allow_overalloc:
        return dict(enabled=False, capacity=bound, capacity_bound=bound, allocated_capacity=high)
    by_key = {(s["source_scale"], s["head"]): s for s in placed}
    by_target, tables = _tables(placed, num_scales, num_heads)

    old_pack = {}
    old_lens = {}
    for target, alive in by_target.items():
        rng = scale_ranges.get(target)
        if rng is None:
            continue
        old_len = int(rng[0])
        old_lens[target] = old_len
        items = []
        for s in alive:
            hi = min(s["scale_end"], old_len)
            if s["scale_start"] < hi:
                items.append(dict(dst_offset=s["offset"], head=s["head"],
                                  src_start=s["scale_start"], length=hi - s["scale_start"]))
        old_pack[target] = _copy_runs(items, old_len)

    append = {}
    for cur, (a, b) in scale_ranges.items():
        nxt = int(cur) + 1
        if nxt >= num_scales:
            continue
        n = int(b) - int(a)
        if n <= 0:
            continue
        items = []
        for h in range(num_heads):
            s = by_key.get((int(cur), h))
            if s is None or not (s["start_target"] <= nxt < s["end_target"]):
                continue
            items.append(dict(dst_offset=s["offset"], head=h, src_start=0, length=n))
        append[(int(cur), nxt)] = _copy_runs(items, n)

    return dict(enabled=True, capacity=int(high), capacity_bound=int(bound),
                allocated_capacity=int(high), overalloc_slots=max(0, int(high) - int(bound)),
                segments=placed, segments_by_key=by_key, segments_by_target=by_target,
                metadata_cpu_by_target=tables, old_pack_runs_by_target=old_pack,
                old_pack_cache_lens_by_target=old_lens, append_runs_by_key=append)
