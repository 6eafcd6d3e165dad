"""Static slab layout of one layer: offsets, per-target offset tables, copy descriptors.

Host-side (Python) part of the path, computed once per layer when pruning is
enabled, exactly as the reference does in
``_segmented_flat_build_static_slot_schedule`` (enable_real_pruning_fast.py:260-558).
The layout is a contract (slab packing must be bit-exact), so the allocation
rules are the reference's:

1. every (source scale s, head h) pair that stays alive for at least one
   target becomes an interval ``[s + 1, end_target)`` of ``tokens(s)`` rows,
   ``end_target`` being the first target whose removed set for source s holds h
   (:276-307);
2. intervals are placed in ``(start_target, end_target, -length, s, h)`` order
   (:313-322);
3. before each placement every placed interval with ``end_target <=
   start_target`` returns its rows to the free list, which is kept sorted and
   coalesced (:323-335, :1033-1047);
4. best fit: the free block with the smallest ``(leftover, offset)`` is used
   from its front; with none large enough the high-water mark grows
   (:337-363); the slab capacity is the final high-water mark.

The implementation here is independent of the reference's code (heap of live
intervals ordered by end target, bisect-maintained free list) and is checked
against the restatement in ``oracle/slot_schedule.py`` and against the closed
form for static keep policies.
"""

from __future__ import annotations

import bisect
import heapq
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Mapping, Optional, Sequence, Set, Tuple

import torch

# Infinity's 1:1, 1M-pixel 13-scale schedule (infinity/utils/dynamic_resolution.py:7, 27-41).
SIDES_1M = (1, 2, 4, 6, 8, 12, 16, 20, 24, 32, 40, 48, 64)


def scale_token_ranges(sides: Sequence[int]) -> Dict[int, Tuple[int, int]]:
    """Token range ``[start, end)`` of each square scale in the flattened sequence."""
    out = {}
    start = 0
    for idx, side in enumerate(sides):
        out[idx] = (start, start + int(side) * int(side))
        start += int(side) * int(side)
    return out


RemovedLookup = Callable[[int], Mapping[int, Set[int]]]


@dataclass
class Segment:
    """One (source scale, head) run of rows in the slab."""

    source_scale: int
    head: int
    start_target: int
    end_target: int
    length: int
    scale_start: int
    scale_end: int
    offset: int = -1

    def live_at(self, target: int) -> bool:
        return self.start_target <= target < self.end_target


@dataclass
class CopyPlan:
    """Flattened copy items of one pack/append call (int64 descriptors)."""

    dst_starts: List[int]
    src_starts: List[int]
    lengths: List[int]
    sequence_len: int

    @property
    def max_length(self) -> int:
        return max(self.lengths) if self.lengths else 0

    @property
    def slots(self) -> int:
        return sum(self.lengths)

    def __len__(self) -> int:
        return len(self.lengths)


@dataclass
class SlabSchedule:
    """Result of ``build_slab_schedule`` for one layer."""

    num_heads: int
    num_scales: int
    scale_ranges: Dict[int, Tuple[int, int]]
    capacity: int
    capacity_bound: int
    segments: List[Segment]
    tables: Dict[int, Tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = field(default_factory=dict)
    append_plans: Dict[Tuple[int, int], CopyPlan] = field(default_factory=dict)
    activation_plans: Dict[int, CopyPlan] = field(default_factory=dict)
    _device_cache: Dict[tuple, object] = field(default_factory=dict, repr=False)

    @property
    def overalloc_slots(self) -> int:
        return max(0, self.capacity - self.capacity_bound)

    def segment(self, source_scale: int, head: int) -> Optional[Segment]:
        for seg in self.segments:
            if seg.source_scale == source_scale and seg.head == head:
                return seg
        return None

    def live_segments(self, target: int) -> List[Segment]:
        return [s for s in self.segments if s.live_at(target)]

    def retained_rows(self, target: int) -> List[int]:
        """Retained prior rows per head at ``target`` (R_h)."""
        rows = [0] * self.num_heads
        for s in self.live_segments(target):
            rows[s.head] += s.length
        return rows

    def device_tables(self, target: int, device) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """Offset tables for ``target`` on ``device``, moved once and cached."""
        key = ("tables", str(device), int(target))
        hit = self._device_cache.get(key)
        if hit is None:
            hit = tuple(t.to(device) for t in self.tables[int(target)])
            self._device_cache[key] = hit
        return hit

    def device_work_plan(self, target: int, device, batch: int, cur_len: int, *, build: bool = True,
                         item_shape: Tuple[int, Optional[int]] = (128, None)) -> Optional[torch.Tensor]:
        """Attention work plan of ``target``'s tables for ``batch`` rows of
        ``cur_len`` queries on ``device`` (segmented_attention_plan) for a
        kernel's ``item_shape`` (``(queries_per_item, slots)``, as
        attention_item_shape reports it; slots None: the device's default),
        built on the host and moved once, cached.  With ``build=False`` only
        a plan already made is returned (None otherwise)."""
        from .real_pruning_fused_attention import segmented_attention_plan

        qpi, slots = item_shape
        key = ("work_plan", str(device), int(target), int(batch), int(cur_len), int(qpi), slots)
        hit = self._device_cache.get(key)
        if hit is None and build:
            st, en, ct = self.tables[int(target)]
            hit = segmented_attention_plan(st, en, ct, batch_size=batch, current_len=cur_len,
                                           capacity=self.capacity, device=device,
                                           queries_per_item=qpi, slots=slots)
            self._device_cache[key] = hit
        return hit

    def fused_append(self, scale: int, device, *,
                     build: bool = True) -> Optional[Tuple[Optional[torch.Tensor], CopyPlan]]:
        """Split of the append of ``scale`` (plan ``(scale, scale + 1)``) for a
        producer that writes K/V rows before this scale's attention runs.

        Returns ``(offsets, residual)``: ``offsets`` is an int32 ``[H]`` device
        tensor with the slab offset of every head whose destination rows lie
        outside all segments live at ``scale`` (the rows the attention reads),
        -1 for the others (None when no head qualifies); ``residual`` is the
        plan of the heads left to the copy after attention.  Cached per
        (device, scale); with ``build=False`` only a split already made is
        returned (None otherwise)."""
        key = ("fused_append", str(device), int(scale))
        hit = self._device_cache.get(key)
        if hit is not None or not build:
            return hit
        plan = self.append_plans.get((int(scale), int(scale) + 1))
        if plan is None or len(plan) == 0:
            hit = (None, plan if plan is not None else CopyPlan([], [], [], 0))
            self._device_cache[key] = hit
            return hit
        n = plan.sequence_len
        live = sorted((s.offset, s.offset + s.length) for s in self.live_segments(int(scale)))
        starts = [a for a, _ in live]
        offsets = [-1] * self.num_heads
        rest = []
        for d, src, ln in zip(plan.dst_starts, plan.src_starts, plan.lengths):
            whole_head = ln == n and src % n == 0
            # live segments are disjoint, so the last one starting before
            # d + ln ends last among them
            i = bisect.bisect_left(starts, d + ln)
            clash = i > 0 and live[i - 1][1] > d
            if whole_head and not clash:
                offsets[src // n] = d
            else:
                rest.append((d, src, ln))
        residual = CopyPlan([r[0] for r in rest], [r[1] for r in rest], [r[2] for r in rest], n)
        dev_offsets = None
        if any(o >= 0 for o in offsets):
            dev_offsets = torch.tensor(offsets, dtype=torch.int32).to(device)
        hit = (dev_offsets, residual)
        self._device_cache[key] = hit
        return hit

    def device_plan(self, plan: CopyPlan, device, tag) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        key = ("plan", str(device), tag)
        hit = self._device_cache.get(key)
        if hit is None:
            hit = tuple(
                torch.tensor(v, dtype=torch.int64).to(device)
                for v in (plan.dst_starts, plan.src_starts, plan.lengths)
            )
            self._device_cache[key] = hit
        return hit


class _FreeList:
    """Sorted, coalesced list of free ``[offset, offset + length)`` blocks."""

    def __init__(self):
        self.offsets: List[int] = []
        self.lengths: List[int] = []

    def release(self, offset: int, length: int) -> None:
        if length <= 0:
            return
        i = bisect.bisect_left(self.offsets, offset)
        self.offsets.insert(i, offset)
        self.lengths.insert(i, length)
        # coalesce with the right neighbour(s), then with the left one
        while i + 1 < len(self.offsets) and self.offsets[i + 1] <= self.offsets[i] + self.lengths[i]:
            end = max(self.offsets[i] + self.lengths[i], self.offsets[i + 1] + self.lengths[i + 1])
            self.lengths[i] = end - self.offsets[i]
            del self.offsets[i + 1]
            del self.lengths[i + 1]
        if i > 0 and self.offsets[i] <= self.offsets[i - 1] + self.lengths[i - 1]:
            end = max(self.offsets[i - 1] + self.lengths[i - 1], self.offsets[i] + self.lengths[i])
            self.lengths[i - 1] = end - self.offsets[i - 1]
            del self.offsets[i]
            del self.lengths[i]

    def take_best_fit(self, length: int) -> Optional[int]:
        best = -1
        best_key = None
        for i, (off, ln) in enumerate(zip(self.offsets, self.lengths)):
            if ln >= length:
                key = (ln - length, off)
                if best_key is None or key < best_key:
                    best, best_key = i, key
        if best < 0:
            return None
        off = self.offsets[best]
        if self.lengths[best] == length:
            del self.offsets[best]
            del self.lengths[best]
        else:
            self.offsets[best] = off + length
            self.lengths[best] -= length
        return off


def _removed_lookup_from_controller(controller, layer_idx: int) -> RemovedLookup:
    cache: Dict[int, Mapping[int, Set[int]]] = {}

    def lookup(target: int):
        hit = cache.get(target)
        if hit is None:
            hit = controller.removed_heads_by_source_for(layer_idx, target)
            cache[target] = hit
        return hit

    return lookup


def build_slab_schedule(
    removed: RemovedLookup,
    *,
    num_heads: int,
    scale_ranges: Mapping[int, Tuple[int, int]],
    num_scales: Optional[int] = None,
) -> SlabSchedule:
    """Allocate slab offsets for one layer.

    ``removed(target)`` returns ``{source_scale: set(heads removed)}`` at that
    target (the reference's ``removed_heads_by_source_for(layer, target)``).
    """
    ranges = {int(k): (int(v[0]), int(v[1])) for k, v in scale_ranges.items()}
    n_scales = len(ranges) if num_scales is None else int(num_scales)
    H = int(num_heads)

    # capacity bound: live rows per target if nothing were freed (:206-234)
    bound = 0
    for target in range(1, n_scales):
        rem = removed(target)
        rows = 0
        for s, (a, b) in ranges.items():
            if s < target and b > a:
                rows += (H - len(rem.get(s, ()))) * (b - a)
        bound = max(bound, rows)

    # 1. intervals
    segs: List[Segment] = []
    for s in sorted(ranges):
        a, b = ranges[s]
        if s + 1 >= n_scales or b <= a:
            continue
        # first target at which each head is dropped for this source
        end_for_head = [n_scales] * H
        pending = set(range(H))
        for target in range(s + 1, n_scales):
            if not pending:
                break
            dropped = removed(target).get(s, set())
            for h in list(pending):
                if h in dropped:
                    end_for_head[h] = target
                    pending.discard(h)
        for h in range(H):
            if end_for_head[h] > s + 1:
                segs.append(Segment(s, h, s + 1, end_for_head[h], b - a, a, b))

    # 2-4. placement
    order = sorted(segs, key=lambda g: (g.start_target, g.end_target, -g.length, g.source_scale, g.head))
    free = _FreeList()
    live: List[Tuple[int, int, Segment]] = []  # heap by end_target
    high = 0
    for n, seg in enumerate(order):
        while live and live[0][0] <= seg.start_target:
            _, _, done = heapq.heappop(live)
            free.release(done.offset, done.length)
        off = free.take_best_fit(seg.length)
        if off is None:
            off = high
            high += seg.length
        seg.offset = off
        heapq.heappush(live, (seg.end_target, n, seg))

    sched = SlabSchedule(num_heads=H, num_scales=n_scales, scale_ranges=ranges, capacity=high,
                         capacity_bound=bound, segments=order)

    # per-target offset tables (:379-412)
    for target in range(1, n_scales):
        per_head: List[List[Segment]] = [[] for _ in range(H)]
        for seg in order:
            if seg.live_at(target):
                per_head[seg.head].append(seg)
        width = max((len(x) for x in per_head), default=0)
        starts = torch.zeros((H, width), dtype=torch.int32)
        ends = torch.zeros((H, width), dtype=torch.int32)
        counts = torch.zeros((H,), dtype=torch.int32)
        for h, items in enumerate(per_head):
            items.sort(key=lambda g: g.source_scale)
            counts[h] = len(items)
            for i, g in enumerate(items):
                starts[h, i] = g.offset
                ends[h, i] = g.offset + g.length
        sched.tables[target] = (starts, ends, counts)

    # copy descriptors, items ordered by destination offset (:414-542, :610-645)
    def plan(items, seq_len):
        items = sorted((it for it in items if it[2] > 0), key=lambda it: it[0])
        return CopyPlan(dst_starts=[it[0] for it in items],
                        src_starts=[it[1] for it in items],
                        lengths=[it[2] for it in items], sequence_len=int(seq_len))

    for target in range(1, n_scales):
        if target not in ranges:
            continue
        old_len = ranges[target][0]
        items = []
        for seg in order:
            if seg.live_at(target):
                hi = min(seg.scale_end, old_len)
                if seg.scale_start < hi:
                    items.append((seg.offset, seg.head * old_len + seg.scale_start, hi - seg.scale_start))
        sched.activation_plans[target] = plan(items, old_len)
    for s, (a, b) in ranges.items():
        if s + 1 >= n_scales or b <= a:
            continue
        n = b - a
        items = []
        for seg in order:
            if seg.source_scale == s and seg.live_at(s + 1):
                items.append((seg.offset, seg.head * n, n))
        sched.append_plans[(s, s + 1)] = plan(items, n)
    return sched


def build_static_slot_schedule(controller, *, layer_idx: int, num_heads: int) -> SlabSchedule:
    """Same entry as the reference's builder: takes a pruning controller.

    ``controller`` provides ``scale_ranges``, ``scale_schedule`` and
    ``removed_heads_by_source_for(layer_idx, target)``
    (enable_pruning.py:328-401).
    """
    return build_slab_schedule(
        _removed_lookup_from_controller(controller, layer_idx),
        num_heads=num_heads,
        scale_ranges=controller.scale_ranges,
        num_scales=len(controller.scale_schedule),
    )
