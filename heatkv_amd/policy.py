"""HeatKV scale-specific head-removal policy: which (source scale, head, layer)
KV segments are dropped at each target scale for a KV budget.

Host-side restatement of the policy the reference computes once when pruning
is enabled (tools/utils.py:63-305, 308-597; enable_pruning.py:48-50, 91-170,
182-189, 328-401), feeding the slab allocator
(:func:`heatkv_amd.slab_schedule.build_static_slot_schedule`):

* :func:`pruned_heads_for_budget` -- how many (layer, head) slots must be
  pruned after each scale so the peak incoming cache stays within the budget
  (tools/utils.py:235-305);
* :func:`strict_pruning_schedule_for_budget_scale_specific` -- the removed
  atoms per target scale (the first ``x`` entries of each source scale's
  removal order) and which of them must already be active inside the scale,
  layer by layer, so every layer-cache checkpoint stays under the budget
  (tools/utils.py:308-522);
* :func:`strict_removed_heads_by_scale_specific_for_budget` -- the removed
  heads seen at each target scale (tools/utils.py:525-597);
* :class:`ScaleSpecificPruningController` -- the lookup the allocator and the
  attention path use (enable_pruning.py:328-401).

Atoms are ``(source_scale, head, layer)`` triples, removal orders are lists of
``(head, layer)`` pairs, one per source scale ``source_scale_start ..
source_scale_end``.  Error types and messages follow the reference.

The layer-by-layer activation is computed here with running per-(source,
layer) removed counts and an incrementally maintained cache total, rather than
by recounting the active set for every candidate; the activation order (last
layer first, then larger source scale, then rank in that scale's order) and
every comparison are the reference's, so the results are identical (pinned by
tests/golden/policy_2b.json, written from the reference itself).
"""

from __future__ import annotations

import json
import math
from typing import Dict, Iterable, List, Mapping, Optional, Sequence, Set, Tuple

from .slab_schedule import SIDES_1M, scale_token_ranges

Atom = Tuple[int, int, int]  # (source_scale, head, layer)


def scale_schedule(sides: Sequence[int] = SIDES_1M) -> List[Tuple[int, int, int]]:
    """``[(1, h, w)]`` per scale: the 1:1, 1M-pixel schedule of
    ``get_scale_schedule`` (tools/utils.py:600-601, 63-65)."""
    return [(1, int(s), int(s)) for s in sides]


def _tokens(sides: Sequence[int]) -> List[int]:
    return [h * w for _, h, w in scale_schedule(sides)]


# ---------------------------------------------------------------- validation

def _check_order(order, *, num_layers: int, num_heads: int) -> Tuple[Tuple[int, int], ...]:
    """(head, layer) pairs, each slot exactly once (tools/utils.py:68-92)."""
    slots = int(num_layers) * int(num_heads)
    if len(order) != slots:
        raise ValueError(f"expected {slots} removal-order entries, got {len(order)}")
    out = []
    seen = set()
    for pos, pair in enumerate(order):
        if not isinstance(pair, (tuple, list)) or len(pair) != 2:
            raise ValueError(f"removal_order[{pos}] must be a (head, layer) tuple")
        head, layer = int(pair[0]), int(pair[1])
        if not 0 <= head < num_heads:
            raise ValueError(f"head index out of range at position {pos}: {head}")
        if not 0 <= layer < num_layers:
            raise ValueError(f"layer index out of range at position {pos}: {layer}")
        if (head, layer) in seen:
            raise ValueError(f"duplicate (head, layer) entry at position {pos}: {(head, layer)}")
        seen.add((head, layer))
        out.append((head, layer))
    return tuple(out)


def normalize_orders(orders, *, num_layers: int, num_heads: int, source_scale_start: int = 4,
                     source_scale_end: int = 11) -> Tuple[Tuple[Tuple[int, int], ...], ...]:
    """One validated order per source scale (tools/utils.py:95-121)."""
    want = int(source_scale_end) - int(source_scale_start) + 1
    if len(orders) != want:
        raise ValueError(
            "scale_specific_removal_orders must contain exactly "
            f"{want} orders for source scales {source_scale_start}-{source_scale_end}"
        )
    return tuple(_check_order(o, num_layers=num_layers, num_heads=num_heads) for o in orders)


def load_orders(path: str):
    """The removal orders of an ``orders/<model>.json`` file: a list (one per
    source scale) of lists of ``[head, layer]`` pairs."""
    with open(path) as fh:
        return json.load(fh)


# ---------------------------------------------------------------- budgets

def pruned_heads_for_budget(budget, *, retained_tokens: int = 51, num_layers: int = 32,
                            num_heads: int = 16, skip_last_scale: bool = True,
                            sides: Sequence[int] = SIDES_1M) -> Dict[int, int]:
    """Slots to prune after each scale so the incoming cache (all earlier
    scales; a pruned slot keeps ``retained_tokens``) stays within ``budget``
    times its peak (tools/utils.py:235-305).  Keyed by scale index."""
    budget = float(budget)
    if not 0.0 <= budget <= 1.0:
        raise ValueError(f"budget must be in [0, 1], got {budget}")
    tokens = _tokens(sides)
    if not tokens:
        return {}
    slots = int(num_layers) * int(num_heads)
    if slots <= 0:
        raise ValueError("num_layers * num_heads must be positive")
    if retained_tokens < 0:
        raise ValueError("retained_tokens must be non-negative")

    incoming = []
    cached = 0
    last = len(tokens) - 1
    for idx, n in enumerate(tokens):
        incoming.append(cached)
        if idx < last or not skip_last_scale:
            cached += n
    peak = max(incoming, default=0)
    if peak <= 0:
        return {idx: 0 for idx in range(len(tokens))}
    floor_ratio = min(retained_tokens, peak) / peak
    if budget + 1e-12 < floor_ratio:
        raise ValueError(f"budget {budget} is below the minimum feasible ratio {floor_ratio:.12f}")

    allowed = budget * peak
    out = {}
    for idx, inc in enumerate(incoming):
        kept = min(retained_tokens, inc)
        if inc <= allowed:
            need = 0
        elif inc == kept:
            raise ValueError(f"budget {budget} is infeasible at scale index {idx}")
        else:
            need = math.ceil(slots * (inc - allowed) / (inc - kept))
        out[idx] = max(0, min(slots, need))
    return out


# ---------------------------------------------------------------- strict schedule

def _by_source_and_layer(atoms: Iterable[Atom], *, num_layers: int,
                         source_scales: Sequence[int]) -> Dict[int, Dict[int, Tuple[int, ...]]]:
    """``{source: {layer: heads}}`` with heads sorted (tools/utils.py:165-178
    groups the same atoms; its tuples follow set iteration order)."""
    grouped: Dict[int, Dict[int, List[int]]] = {s: {l: [] for l in range(num_layers)} for s in source_scales}
    for s, h, l in atoms:
        grouped[s][l].append(h)
    return {s: {l: tuple(sorted(hs)) for l, hs in lm.items()} for s, lm in grouped.items()}


def strict_pruning_schedule_for_budget_scale_specific(
    budget,
    scale_specific_removal_orders,
    *,
    num_layers: int = 32,
    num_heads: int = 16,
    source_scale_start: int = 4,
    source_scale_end: int = 11,
    protected_prefix_scales: int = 4,
    skip_last_scale: bool = True,
    sides: Sequence[int] = SIDES_1M,
) -> dict:
    """Removed atoms per target scale and their early activation inside the
    scale (tools/utils.py:308-522).

    At target ``t`` the removed atoms are the first ``x`` entries of the order
    of every source scale ``start .. min(end, t)``, ``x`` = the prune count of
    scale ``t + 1``.  Walking the layers of scale ``t`` (the cache then holds
    the protected prefix, every source scale up to ``t - 1`` and scale ``t``
    for the layers written so far), the atoms of layers already passed are
    active; whenever the cache exceeds ``budget`` times its unpruned peak, not
    yet active atoms of later layers are activated (last layer first, then
    larger source scale, then order rank) until it fits.
    """
    budget = float(budget)
    if not 0.0 <= budget <= 1.0:
        raise ValueError(f"budget must be in [0, 1], got {budget}")
    L, H = int(num_layers), int(num_heads)
    if L <= 0 or H <= 0:
        raise ValueError("num_layers * num_heads must be positive")
    s0, s1 = int(source_scale_start), int(source_scale_end)
    orders = {s0 + i: o for i, o in enumerate(
        normalize_orders(scale_specific_removal_orders, num_layers=L, num_heads=H,
                         source_scale_start=s0, source_scale_end=s1))}
    rank = {s: {slot: r for r, slot in enumerate(o)} for s, o in orders.items()}

    tokens = _tokens(sides)
    if not tokens:
        return {"final_removed_counts": {}, "final_removed_by_scale": {}, "early_activation_by_scale": {}}
    S = len(tokens)
    budgeted = S - 1 if skip_last_scale else S
    sources = tuple(range(s0, min(s1, S - 1) + 1))
    if budgeted <= 0:
        empty = _by_source_and_layer((), num_layers=L, source_scales=sources)
        return {"final_removed_counts": {t: 0 for t in range(S)},
                "final_removed_by_scale": {t: {s: dict(m) for s, m in empty.items()} for t in range(S)},
                "early_activation_by_scale": {t: {} for t in range(S)}}

    peak = sum(tokens[:budgeted])
    protected_tokens = sum(tokens[:min(int(protected_prefix_scales), S)])
    floor_ratio = protected_tokens / peak if peak > 0 else 0.0
    if budget + 1e-12 < floor_ratio:
        raise ValueError(f"budget {budget} is below the minimum feasible ratio {floor_ratio:.12f}")
    limit = budget * L * H * peak
    counts_by_scale = pruned_heads_for_budget(budget, retained_tokens=protected_tokens, num_layers=L,
                                              num_heads=H, skip_last_scale=skip_last_scale, sides=sides)

    final_counts: Dict[int, int] = {}
    final_by_scale: Dict[int, dict] = {}
    early_by_scale: Dict[int, dict] = {}
    active: Set[Atom] = set()

    def cache_total(t: int, written: int, removed: Mapping[Tuple[int, int], int]) -> int:
        # protected prefix + every counted source scale, scale t only up to `written`
        total = L * H * sum(tokens[:min(int(protected_prefix_scales), t)])
        for s in range(s0, min(s1, t) + 1):
            for l in range(L):
                if s == t and l > written:
                    continue
                total += (H - removed.get((s, l), 0)) * tokens[s]
        return total

    for t in range(S):
        if t >= budgeted:
            final_counts[t] = len(active)
            final_by_scale[t] = _by_source_and_layer(active, num_layers=L, source_scales=sources)
            early_by_scale[t] = {}
            continue
        nxt = min(t + 1, S - 1)
        x = int(counts_by_scale.get(nxt, counts_by_scale.get(t, 0)))
        target: Set[Atom] = set()
        for s in range(s0, min(s1, t) + 1):
            for h, l in orders[s][:x]:
                target.add((s, h, l))
        # candidates in activation priority: last layer, larger source, order rank
        queue = sorted(target, key=lambda a: (-a[2], -a[0], rank[a[0]][(a[1], a[2])]))

        cur = set(active)
        removed: Dict[Tuple[int, int], int] = {}
        for s, _, l in cur:
            removed[(s, l)] = removed.get((s, l), 0) + 1
        by_layer: Dict[int, List[Atom]] = {}
        for a in target:
            by_layer.setdefault(a[2], []).append(a)

        early: Dict[int, List[Atom]] = {}
        for layer in range(L):
            for a in by_layer.get(layer, ()):
                if a not in cur:
                    cur.add(a)
                    removed[(a[0], a[2])] = removed.get((a[0], a[2]), 0) + 1
            total = cache_total(t, layer, removed)
            if total <= limit:
                continue
            fired: List[Atom] = []
            for a in queue:
                # only atoms of later layers; source scale t has not written them yet
                if a in cur or a[2] <= layer or a[0] == t:
                    continue
                cur.add(a)
                removed[(a[0], a[2])] = removed.get((a[0], a[2]), 0) + 1
                fired.append(a)
                # the atom's (source, layer) term is counted (source < t), so
                # the total drops by one head of that scale
                total -= tokens[a[0]]
                if total <= limit:
                    break
            if total > limit:
                raise ValueError(f"budget {budget} is infeasible at scale index {t}, layer {layer}")
            if fired:
                early[layer] = fired

        if cache_total(t, L - 1, removed) > limit:
            raise ValueError(f"budget {budget} is infeasible at end of scale index {t}")
        if cur != target:
            raise RuntimeError(
                "strict scale-specific schedule failed to activate "
                f"end-of-scale removals at scale index {t}"
            )
        active = set(target)
        final_counts[t] = len(active)
        final_by_scale[t] = _by_source_and_layer(active, num_layers=L, source_scales=sources)
        early_by_scale[t] = early

    return {"final_removed_counts": final_counts, "final_removed_by_scale": final_by_scale,
            "early_activation_by_scale": early_by_scale}


def strict_removed_heads_by_scale_specific_for_budget(
    budget,
    scale_specific_removal_orders,
    *,
    num_layers: int = 32,
    num_heads: int = 16,
    source_scale_start: int = 4,
    source_scale_end: int = 11,
    protected_prefix_scales: int = 4,
    skip_last_scale: bool = True,
    strict_schedule: Optional[dict] = None,
    sides: Sequence[int] = SIDES_1M,
) -> dict:
    """Removed heads seen at each target scale: the previous scale's final
    removals plus every atom activated early inside this scale
    (tools/utils.py:525-597).  ``removed_heads_by_scale[t][source][layer]`` is
    a sorted tuple of heads."""
    L, H = int(num_layers), int(num_heads)
    s0, s1 = int(source_scale_start), int(source_scale_end)
    orders = normalize_orders(scale_specific_removal_orders, num_layers=L, num_heads=H,
                              source_scale_start=s0, source_scale_end=s1)
    S = len(sides)
    sched = strict_schedule if strict_schedule is not None else strict_pruning_schedule_for_budget_scale_specific(
        budget, orders, num_layers=L, num_heads=H, source_scale_start=s0, source_scale_end=s1,
        protected_prefix_scales=protected_prefix_scales, skip_last_scale=skip_last_scale, sides=sides)
    sources = tuple(range(s0, min(s1, S - 1) + 1))

    removed_by_scale, removed_counts, remaining = {}, {}, {}
    prev: Set[Atom] = set()
    for t in range(S):
        top = min(s1, t, S - 1)
        n_src = top - s0 + 1 if top >= s0 else 0
        seen = set(prev)
        for atoms in sched["early_activation_by_scale"].get(t, {}).values():
            seen.update(tuple(int(v) for v in a) for a in atoms)
        removed_by_scale[t] = _by_source_and_layer(seen, num_layers=L, source_scales=sources)
        removed_counts[t] = len(seen)
        remaining[t] = n_src * L * H - len(seen)
        prev = {(int(s), int(h), int(l))
                for s, lm in sched["final_removed_by_scale"].get(t, {}).items()
                for l, hs in lm.items() for h in hs}
    return {"removed_heads_by_scale": removed_by_scale, "removed_counts_by_scale": removed_counts,
            "remaining_atoms_by_scale": remaining, "strict_schedule": sched}


# ---------------------------------------------------------------- controller

def _empty_removed(num_layers: int) -> Dict[int, Set[int]]:
    return {l: set() for l in range(num_layers)}


def normalize_removed_heads_by_scale(removed_heads_by_scale, *, num_layers: int, num_heads: int,
                                     source_scale_start: int = 4, source_scale_end: int = 11):
    """``{target: {source: {layer: set(heads)}}}`` with every source scale of
    the range present, checked like enable_pruning.py:115-179."""
    L = int(num_layers)
    out = {}
    for t, source_map in removed_heads_by_scale.items():
        t = int(t)
        if not isinstance(source_map, dict):
            raise ValueError(f"removed_heads_by_scale[{t}] must be a dict")
        norm = {s: _empty_removed(L) for s in range(int(source_scale_start), int(source_scale_end) + 1)}
        for s, layer_map in source_map.items():
            s = int(s)
            if not int(source_scale_start) <= s <= int(source_scale_end):
                raise ValueError(f"removed_heads_by_scale[{t}] source scale out of range: {s}")
            if not isinstance(layer_map, dict):
                raise ValueError(f"removed_heads_by_scale[{t}][{s}] must be a dict")
            layers = _empty_removed(L)
            for l, heads in layer_map.items():
                l = int(l)
                if not 0 <= l < L:
                    raise ValueError(f"removed_heads_by_scale[{t}][{s}] layer index out of range: {l}")
                for h in heads:
                    h = int(h)
                    if not 0 <= h < num_heads:
                        raise ValueError(
                            f"removed_heads_by_scale[{t}][{s}] head index out of range for layer {l}: {h}")
                    if h in layers[l]:
                        raise ValueError(f"removed_heads_by_scale[{t}][{s}] duplicate head {h} for layer {l}")
                    layers[l].add(h)
            norm[s] = layers
        out[t] = norm
    return out


class ScaleSpecificPruningController:
    """Removed-head lookup per (layer, target scale, source scale)
    (enable_pruning.py:328-401).

    Built either from a precomputed ``static_removed_heads_by_scale`` (what
    the fused segmented path uses) or from ``prune_counts`` and the removal
    orders (the first ``count`` entries of each source scale's order, for
    sources below the target).  A target without an entry falls back to the
    nearest lower one.
    """

    def __init__(self, *, num_layers, num_heads, static_removed_heads_by_scale=None, prune_counts=None,
                 scale_specific_removal_orders=None, source_scale_start=4, source_scale_end=11,
                 sides: Sequence[int] = SIDES_1M):
        self.num_layers = int(num_layers)
        self.num_heads = int(num_heads)
        self.source_scale_start = int(source_scale_start)
        self.source_scale_end = int(source_scale_end)
        self.scale_schedule = scale_schedule(sides)
        self.scale_ranges = scale_token_ranges(sides)
        if static_removed_heads_by_scale is not None:
            self._static_removed_heads_by_scale = static_removed_heads_by_scale
            return
        self.prune_counts = dict(prune_counts)
        slots = self.num_layers * self.num_heads
        table = {}
        for t in range(len(self.scale_schedule)):
            x = max(0, min(slots, int(self.prune_counts.get(t, 0))))
            by_source = {}
            for s in range(self.source_scale_start, min(self.source_scale_end, t - 1) + 1):
                removed = _empty_removed(self.num_layers)
                for h, l in scale_specific_removal_orders[s - self.source_scale_start][:x]:
                    removed[l].add(h)
                by_source[s] = removed
            table[t] = by_source
        self._static_removed_heads_by_scale = table

    def reset(self):
        return None

    def _removed_heads_state(self, target_scale_idx):
        table = self._static_removed_heads_by_scale
        if target_scale_idx in table:
            return table[target_scale_idx]
        lower = [t for t in table if t <= target_scale_idx]
        if not lower:
            return {s: _empty_removed(self.num_layers)
                    for s in range(self.source_scale_start, self.source_scale_end + 1)}
        return table[max(lower)]

    def removed_heads_for(self, layer_idx, target_scale_idx, source_scale_idx):
        source = self._removed_heads_state(target_scale_idx).get(source_scale_idx)
        if source is None:
            return set()
        return set(source.get(layer_idx, set()))

    def removed_heads_by_source_for(self, layer_idx, target_scale_idx):
        return {s: set(m.get(layer_idx, set()))
                for s, m in self._removed_heads_state(target_scale_idx).items()}


def controller_for_budget(budget, scale_specific_removal_orders, *, num_layers: int, num_heads: int,
                          protected_prefix_scales: int = 4, source_scale_start: Optional[int] = None,
                          skip_last_scale: bool = True, sides: Sequence[int] = SIDES_1M):
    """The controller ``enable_real_pruning_scale_specific_fast`` builds
    (enable_real_pruning_fast.py:2279-2340): strict removed heads for the
    budget, normalized, as a static table."""
    protected_prefix_scales = int(protected_prefix_scales)
    if protected_prefix_scales < 0:
        raise ValueError("protected_prefix_scales must be non-negative")
    start = protected_prefix_scales if source_scale_start is None else int(source_scale_start)
    if len(sides) <= protected_prefix_scales:
        raise ValueError("scale-specific real pruning fast requires at least one scale after the protected prefix")
    orders = normalize_orders(scale_specific_removal_orders, num_layers=num_layers, num_heads=num_heads,
                              source_scale_start=start)
    view = strict_removed_heads_by_scale_specific_for_budget(
        budget, orders, num_layers=num_layers, num_heads=num_heads, source_scale_start=start,
        protected_prefix_scales=protected_prefix_scales, skip_last_scale=skip_last_scale, sides=sides)
    table = normalize_removed_heads_by_scale(view["removed_heads_by_scale"], num_layers=num_layers,
                                             num_heads=num_heads, source_scale_start=start)
    return ScaleSpecificPruningController(num_layers=num_layers, num_heads=num_heads,
                                          static_removed_heads_by_scale=table, source_scale_start=start,
                                          sides=sides)
