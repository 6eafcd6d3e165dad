"""HeatKV removal policy (heatkv_amd/policy.py) against the reference's own
outputs, and the slab allocator under the real, progressive removal policy.

Golden vectors: tests/golden/policy_2b.json, written by
tests/golden/make_policy_golden.py from the reference's tools/utils.py and
enable_pruning.py on the reference's orders/2b.json (kept here as
tests/golden/orders_2b.json): prune counts for several budgets, the strict
schedule's end-of-scale counts and early activations (in activation order),
and the controller's removed heads for every (target, source, layer).

The allocator run on those removal sets (offsets change as heads are dropped
between targets) is checked against the allocator restatement in
oracle/slot_schedule.py, against its invariants, and against the
reference's own allocator: tests/golden/slab_2b.json, written by
tests/golden/make_slab_golden.py, holds the capacity and every segment's
offset and end target of all 32 layers at budgets 0.1 and 0.35, and
digests of their offset tables and copy descriptors, as
``_segmented_flat_build_static_slot_schedule``
(enable_real_pruning_fast.py:260-558) gives them.
"""

from __future__ import annotations

import hashlib
import json
import os

import numpy as np
import pytest

from heatkv_amd import policy as P
from heatkv_amd.slab_schedule import SIDES_1M, build_static_slot_schedule, scale_token_ranges
from oracle import slot_schedule as osched

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = json.load(open(os.path.join(HERE, "golden", "policy_2b.json")))
ORDERS = json.load(open(os.path.join(HERE, "golden", "orders_2b.json")))
L, H, START = GOLD["num_layers"], GOLD["num_heads"], GOLD["source_scale_start"]


def _mask(ctrl, t, s):
    bits = 0
    for layer in range(L):
        for h in ctrl.removed_heads_for(layer, t, s):
            bits |= 1 << (layer * H + int(h))
    return format(bits, "x")


@pytest.mark.parametrize("key", sorted(GOLD["pruned_heads"]))
def test_pruned_heads_for_budget_matches_reference(key):
    budget, retained, skip = key.split("/")
    want = GOLD["pruned_heads"][key]
    kw = dict(retained_tokens=int(retained), num_layers=L, num_heads=H, skip_last_scale=bool(int(skip)))
    if "error" in want:
        with pytest.raises(ValueError) as e:
            P.pruned_heads_for_budget(float(budget), **kw)
        assert str(e.value) == want["error"]
        return
    got = P.pruned_heads_for_budget(float(budget), **kw)
    assert {str(k): v for k, v in got.items()} == want


@pytest.mark.parametrize("budget", sorted(GOLD["strict"]))
def test_strict_schedule_matches_reference(budget):
    want = GOLD["strict"][budget]
    sched = P.strict_pruning_schedule_for_budget_scale_specific(
        float(budget), ORDERS, num_layers=L, num_heads=H, source_scale_start=START,
        protected_prefix_scales=START)
    assert {str(t): n for t, n in sched["final_removed_counts"].items()} == want["final_removed_counts"]
    early = {str(t): {str(l): [list(a) for a in atoms] for l, atoms in m.items()}
             for t, m in sched["early_activation_by_scale"].items()}
    assert early == want["early_activation"]  # same atoms, same activation order
    view = P.strict_removed_heads_by_scale_specific_for_budget(
        float(budget), ORDERS, num_layers=L, num_heads=H, source_scale_start=START,
        protected_prefix_scales=START, strict_schedule=sched)
    assert {str(t): n for t, n in view["removed_counts_by_scale"].items()} == want["removed_counts_by_scale"]
    assert {str(t): n for t, n in view["remaining_atoms_by_scale"].items()} == want["remaining_atoms_by_scale"]


@pytest.mark.parametrize("budget", sorted(GOLD["strict"]))
def test_controller_matches_reference(budget):
    want = GOLD["strict"][budget]["removed_mask"]
    ctrl = P.controller_for_budget(float(budget), ORDERS, num_layers=L, num_heads=H, protected_prefix_scales=START)
    for t in range(13):
        for s in range(START, 12):
            assert _mask(ctrl, t, s) == want[str(t)][str(s)], (budget, t, s)


def test_swapped_order_entries_change_the_result():
    """The golden vectors distinguish the order ranks: swapping two early
    entries of one source scale's order changes the removed sets."""
    orders = [list(map(list, o)) for o in ORDERS]
    orders[5][0], orders[5][300] = orders[5][300], orders[5][0]
    ctrl = P.controller_for_budget(0.1, orders, num_layers=L, num_heads=H, protected_prefix_scales=START)
    want = GOLD["strict"]["0.1"]["removed_mask"]
    assert any(_mask(ctrl, t, START + 5) != want[str(t)][str(START + 5)] for t in range(13))


def test_budget_is_respected_at_every_layer_checkpoint():
    """Independent of the reference's code: with the removed sets the schedule
    reports (end-of-scale sets plus early activations up to each layer), the
    cached tokens after every layer of every budgeted scale stay within
    budget x the unpruned peak (the definition of the strict schedule)."""
    budget = 0.1
    sched = P.strict_pruning_schedule_for_budget_scale_specific(
        budget, ORDERS, num_layers=L, num_heads=H, source_scale_start=START, protected_prefix_scales=START)
    tokens = [s * s for s in SIDES_1M]
    S = len(tokens)
    limit = budget * L * H * sum(tokens[:S - 1])
    prev = set()
    for t in range(S - 1):
        fin = {(int(s), int(h), int(l)) for s, lm in sched["final_removed_by_scale"][t].items()
               for l, hs in lm.items() for h in hs}
        early = sched["early_activation_by_scale"][t]
        for written in range(L):
            removed = set(prev) | {a for a in fin if a[2] <= written}
            for l, atoms in early.items():
                if l <= written:
                    removed.update(tuple(a) for a in atoms)
            rows = L * H * sum(tokens[:min(START, t)])
            for s in range(START, min(11, t) + 1):
                for l in range(L):
                    if s == t and l > written:
                        continue
                    rows += (H - sum(1 for a in removed if a[0] == s and a[2] == l)) * tokens[s]
            assert rows <= limit + 1e-6, (t, written, rows, limit)
        prev = fin


def test_policy_errors_follow_the_reference():
    with pytest.raises(ValueError, match="budget must be in"):
        P.pruned_heads_for_budget(1.5)
    with pytest.raises(ValueError, match="below the minimum feasible ratio"):
        P.strict_pruning_schedule_for_budget_scale_specific(0.0001, ORDERS, num_layers=L, num_heads=H,
                                                             source_scale_start=START, protected_prefix_scales=START)
    with pytest.raises(ValueError, match="must contain exactly 9 orders"):
        P.normalize_orders(ORDERS[:8], num_layers=L, num_heads=H, source_scale_start=START)
    bad = [list(map(list, o)) for o in ORDERS]
    bad[0][1] = list(bad[0][0])
    with pytest.raises(ValueError, match="duplicate"):
        P.normalize_orders(bad, num_layers=L, num_heads=H, source_scale_start=START)


SLAB_GOLD = json.load(open(os.path.join(HERE, "golden", "slab_2b.json")))


def _digest(*arrays) -> str:
    """SHA-256 (16 hex digits) of the arrays' shapes and int64 values, as the golden file's."""
    h = hashlib.sha256()
    for a in arrays:
        a = np.asarray(a, dtype=np.int64)
        h.update(np.asarray(a.shape, dtype=np.int64).tobytes())
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()[:16]


def _plan_digest(plan) -> str:
    items = np.asarray(list(zip(plan.dst_starts, plan.src_starts, plan.lengths)), dtype=np.int64).reshape(-1, 3)
    return _digest(items, [plan.sequence_len if plan.lengths else 0])


@pytest.mark.parametrize("budget", sorted(SLAB_GOLD["budgets"]))
def test_allocator_matches_reference_offsets(budget):
    """Progressive removal (heads dropped part-way, freed rows reused by best
    fit): capacity, capacity bound and every (source, head) segment's end
    target and slab offset of all 32 layers equal the reference allocator's,
    and so do the offset tables of every target and the copy descriptors of
    every activation and append (compared through digests of their values)."""
    ctrl = P.controller_for_budget(float(budget), ORDERS, num_layers=L, num_heads=H, protected_prefix_scales=START)
    reused = 0
    for layer, want in enumerate(SLAB_GOLD["budgets"][budget]):
        got = build_static_slot_schedule(ctrl, layer_idx=layer, num_heads=H)
        assert (got.capacity, got.capacity_bound) == (want["capacity"], want["capacity_bound"]), layer
        segs = sorted([g.source_scale, g.head, g.end_target, g.offset] for g in got.segments)
        assert segs == want["segments"], layer
        assert {str(t): _digest(*(x.numpy() for x in tab)) for t, tab in got.tables.items()} == want["tables"]
        assert {str(t): _plan_digest(p) for t, p in got.activation_plans.items()} == want["activation"], layer
        assert {str(s): _plan_digest(p) for (s, _), p in got.append_plans.items()} == want["append"], layer
        # rows freed by a dropped head are given to a later segment
        ends = {(s[3], s[2]) for s in want["segments"] if s[2] < 13}
        reused += any(s[3] == o and s[0] + 1 >= e for s in want["segments"] for o, e in ends)
    assert reused > 0


@pytest.mark.parametrize("budget", [0.1, 0.2])
def test_allocator_under_the_real_policy(budget):
    """Slab schedules of all 32 layers under the strict policy: equal to the
    oracle allocator's, and live segments disjoint, inside the capacity, one
    per live (source, head), tables sorted by source scale."""
    ctrl = P.controller_for_budget(budget, ORDERS, num_layers=L, num_heads=H, protected_prefix_scales=START)
    ranges = scale_token_ranges(SIDES_1M)
    table = {t: ctrl._removed_heads_state(t) for t in range(13)}
    view = osched.PolicyView(table, num_layers=L, source_start=START, source_end=11)
    progressive = 0
    for layer in range(L):
        got = build_static_slot_schedule(ctrl, layer_idx=layer, num_heads=H)
        ref = osched.build_schedule(view, {k: v for k, v in ranges.items()}, layer=layer, num_heads=H)
        assert got.capacity == ref["capacity"]
        for t in range(1, 13):
            src_of = {(g.head, g.offset): g.source_scale for g in got.segments if g.live_at(t)}
            st, en, ct = (x.numpy() for x in got.tables[t])
            ost, oen, oct_ = ref["metadata_cpu_by_target"][t]
            assert np.array_equal(ct, oct_) and np.array_equal(st, ost) and np.array_equal(en, oen), (layer, t)
            removed = ctrl.removed_heads_by_source_for(layer, t)
            live = []
            for h in range(H):
                n = int(ct[h])
                srcs = [g.source_scale for g in got.segments if g.head == h and g.live_at(t)]
                want = [s for s in range(t) if h not in removed.get(s, set())]
                assert sorted(srcs) == want == sorted(set(srcs)), (layer, t, h)
                assert n == len(want)
                assert [src_of[(h, int(st[h, i]))] for i in range(n)] == want  # sorted by source scale
                for i in range(n):
                    assert 0 <= st[h, i] < en[h, i] <= got.capacity
                    live.append((int(st[h, i]), int(en[h, i])))
            live.sort()
            assert all(a[1] <= b[0] for a, b in zip(live, live[1:])), (layer, t)
        ends = {g.end_target for g in got.segments}
        progressive += any(e < 13 for e in ends)
    assert progressive > 0  # some heads are dropped part-way: progressive removal is exercised


def test_enable_attaches_policy_schedule_and_cache():
    import torch

    from heatkv_amd import canonical_method, enable_real_pruning_scale_specific_fused_segmented

    class SelfAttention(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.num_heads = H

    model = torch.nn.Sequential(*[SelfAttention() for _ in range(L)])
    out = enable_real_pruning_scale_specific_fused_segmented(
        model, 0.1, ORDERS, protected_prefix_scales=START, source_scale_start=START,
        requested_generation_batch_size=1)
    assert out is model
    layers = list(model)
    assert [m.layer_idx for m in layers] == list(range(L))
    ctrl = layers[0].heatkv_controller
    want = GOLD["strict"]["0.1"]["removed_mask"]
    assert all(_mask(ctrl, t, s) == want[str(t)][str(s)] for t in range(13) for s in range(START, 12))
    for m in (layers[0], layers[-1]):
        ref = build_static_slot_schedule(ctrl, layer_idx=m.layer_idx, num_heads=H)
        assert m.heatkv_schedule.capacity == ref.capacity
        assert m.heatkv_cache.removed(12) == ctrl.removed_heads_by_source_for(m.layer_idx, 12)
    with pytest.raises(ValueError, match="merge_mode='exact'"):
        enable_real_pruning_scale_specific_fused_segmented(model, 0.1, ORDERS, merge_mode="approx")
    assert canonical_method("fused-segmented") == canonical_method("fused_segmented") == "real_scale_fused_segmented"
    with pytest.raises(ValueError):
        canonical_method("dense")


def test_general_enable_entry_checks_attention_impl():
    import torch

    from heatkv_amd import enable_real_pruning_scale_specific_fast

    class SelfAttention(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.num_heads = H

    model = torch.nn.Sequential(*[SelfAttention() for _ in range(L)])
    with pytest.raises(ValueError, match="unsupported real pruning fast attention_impl: 'dense'"):
        enable_real_pruning_scale_specific_fast(model, 0.1, ORDERS, attention_impl="dense")
    with pytest.raises(ValueError, match="merge_mode='exact'"):
        enable_real_pruning_scale_specific_fast(model, 0.1, ORDERS, merge_mode="approx")
    out = enable_real_pruning_scale_specific_fast(model, 0.1, ORDERS, protected_prefix_scales=START,
                                                  source_scale_start=START)
    assert out is model and [m.layer_idx for m in model] == list(range(L))
    want = GOLD["strict"]["0.1"]["removed_mask"]
    ctrl = model[0].heatkv_controller
    assert all(_mask(ctrl, t, s) == want[str(t)][str(s)] for t in range(13) for s in range(START, 12))
