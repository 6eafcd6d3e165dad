"""Pins the allocator oracle and checks the product schedule against it.

Oracle pins (independent of oracle/slot_schedule.py's own code):
* static keep policies -> offsets are the exclusive prefix sum of token counts
  over kept (source asc, head asc) pairs (closed form);
* a hand-worked progressive-removal case (offsets, capacity, capacity bound,
  per-target tables, append and activation descriptors derived on paper);
* a hand-worked interval sequence exercising best fit over a lower offset,
  the lowest-offset tie break, coalescing and bump allocation;
* invariants on random progressive policies.
Product check: heatkv_amd.slab_schedule equals the oracle on random policies.
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from heatkv_amd import slab_schedule as ps
from heatkv_amd import workloads as W
from oracle import slot_schedule as osched

# ------------------------------------------------------------------ helpers


def _policy_view(removed_by_target, num_scales):
    static = {t: {s: {0: set(hs)} for s, hs in by_src.items()} for t, by_src in removed_by_target.items()}
    return osched.PolicyView(static, num_layers=1, source_start=0, source_end=num_scales - 1)


def _product(removed_by_target, ranges, H):
    pol = _policy_view(removed_by_target, len(ranges))
    return ps.build_slab_schedule(lambda t: pol.removed_heads_by_source_for(0, t), num_heads=H,
                                  scale_ranges=ranges, num_scales=len(ranges))


def _oracle(removed_by_target, ranges, H):
    return osched.build_schedule(_policy_view(removed_by_target, len(ranges)), ranges, layer=0, num_heads=H)


def _flat(plan_runs):
    f = osched.flatten_copy_items(plan_runs)
    return ([], [], []) if f is None else (f["dst_starts"], f["src_starts"], f["lengths"])


def _assert_same(prod, orc):
    assert prod.capacity == orc["capacity"]
    assert prod.capacity_bound == orc["capacity_bound"]
    po = {(s.source_scale, s.head): (s.offset, s.start_target, s.end_target, s.length) for s in prod.segments}
    oo = {(s["source_scale"], s["head"]): (s["offset"], s["start_target"], s["end_target"], s["length"])
          for s in orc["segments"]}
    assert po == oo
    for t, (st, en, ct) in orc["metadata_cpu_by_target"].items():
        pst, pen, pct = prod.tables[t]
        assert np.array_equal(pst.numpy(), st) and np.array_equal(pen.numpy(), en)
        assert np.array_equal(pct.numpy(), ct)
    for key, runs in orc["append_runs_by_key"].items():
        plan = prod.append_plans[key]
        assert (plan.dst_starts, plan.src_starts, plan.lengths) == _flat(runs)
    for t, runs in orc["old_pack_runs_by_target"].items():
        plan = prod.activation_plans[t]
        assert (plan.dst_starts, plan.src_starts, plan.lengths) == _flat(runs)


def _check_invariants(sched_dict, num_heads):
    cap = sched_dict["capacity"]
    segs = sched_dict["segments"]
    for t, (st, en, ct) in sched_dict["metadata_cpu_by_target"].items():
        live = [s for s in segs if s["start_target"] <= t < s["end_target"]]
        spans = sorted((s["offset"], s["offset"] + s["length"]) for s in live)
        for (a0, a1), (b0, _) in zip(spans, spans[1:]):
            assert a1 <= b0, "live segments overlap"
        assert all(0 <= a and b <= cap for a, b in spans)
        assert cap >= sum(b - a for a, b in spans)
        for h in range(num_heads):
            mine = sorted((s for s in live if s["head"] == h), key=lambda s: s["source_scale"])
            assert int(ct[h]) == len(mine)
            for i, s in enumerate(mine):
                assert st[h, i] == s["offset"] and en[h, i] == s["offset"] + s["length"]


def _random_progressive(seed, num_scales=9, H=6):
    rnd = random.Random(seed)
    sides = [1, 2, 3, 4, 5, 6, 8, 9, 11, 12, 13][:num_scales]
    ranges = osched.scale_token_ranges(sides)
    removed = {}
    state = {}
    for t in range(1, num_scales):
        for s in range(t):
            cur = state.setdefault(s, set())
            if rnd.random() < 0.5:
                cur |= {rnd.randrange(H) for _ in range(rnd.randrange(1, 3))}
        if rnd.random() < 0.8:  # sometimes omit a target: lookup falls back to the lower one
            removed[t] = {s: set(v) for s, v in state.items()}
    return removed, ranges, H


# ------------------------------------------------------------------ oracle pins


@pytest.mark.parametrize("seed", range(5))
def test_static_policy_closed_form(seed):
    rng = np.random.default_rng(seed)
    sides = [1, 2, 4, 6, 8, 12, 16, 20]
    ranges = osched.scale_token_ranges(sides)
    H, S = 5, len(sides)
    keep = rng.random((H, S - 1)) < 0.5
    removed = {t: {s: {h for h in range(H) if not keep[h, s]} for s in range(t)} for t in range(1, S)}
    orc = _oracle(removed, ranges, H)
    expect = {}
    cursor = 0
    for s in range(S - 1):
        for h in range(H):
            if keep[h, s]:
                expect[(s, h)] = cursor
                cursor += ranges[s][1] - ranges[s][0]
    got = {(g["source_scale"], g["head"]): g["offset"] for g in orc["segments"]}
    assert got == expect
    assert orc["capacity"] == cursor
    prod = _product(removed, ranges, H)
    assert {(g.source_scale, g.head): g.offset for g in prod.segments} == expect


def test_hand_worked_progressive_case():
    # token counts 1, 4, 4, 9, 16; 2 heads; removals derived on paper
    ranges = {0: (0, 1), 1: (1, 5), 2: (5, 9), 3: (9, 18), 4: (18, 34)}
    removed = {1: {}, 2: {0: {0}}, 3: {0: {0}, 1: {1}}, 4: {0: {0}, 1: {1}, 2: {0}}}
    orc = _oracle(removed, ranges, 2)
    offsets = {(g["source_scale"], g["head"]): g["offset"] for g in orc["segments"]}
    assert offsets == {(0, 0): 0, (0, 1): 1, (1, 1): 2, (1, 0): 6, (2, 0): 2, (2, 1): 10,
                       (3, 0): 14, (3, 1): 23}
    assert orc["capacity"] == 32 and orc["capacity_bound"] == 27
    tables = orc["metadata_cpu_by_target"]
    assert tables[4][0].tolist() == [[6, 14, 0], [1, 10, 23]]
    assert tables[4][1].tolist() == [[10, 23, 0], [2, 14, 32]]
    assert tables[4][2].tolist() == [2, 3]
    assert tables[3][0].tolist() == [[6, 2], [1, 10]] and tables[3][1].tolist() == [[10, 6], [2, 14]]
    assert tables[2][0].tolist() == [[6, 0], [1, 2]] and tables[2][2].tolist() == [1, 2]
    assert tables[1][0].tolist() == [[0], [1]]
    app = orc["append_runs_by_key"]
    assert _flat(app[(0, 1)]) == ([0, 1], [0, 1], [1, 1])
    assert _flat(app[(1, 2)]) == ([2, 6], [4, 0], [4, 4])
    assert _flat(app[(2, 3)]) == ([2, 10], [0, 4], [4, 4])
    assert _flat(app[(3, 4)]) == ([14, 23], [0, 9], [9, 9])
    assert _flat(orc["old_pack_runs_by_target"][4]) == ([1, 6, 10, 14, 23], [18, 1, 23, 9, 27],
                                                        [1, 4, 4, 9, 9])
    _check_invariants(orc, 2)
    _assert_same(_product(removed, ranges, 2), orc)


def test_hand_worked_best_fit_sequence():
    def iv(start, end, n, s, h):
        return dict(source_scale=s, head=h, start_target=start, end_target=end, length=n,
                    scale_start=0, scale_end=n)

    intervals = [iv(1, 3, 9, 0, 0), iv(1, 9, 2, 0, 1), iv(2, 3, 4, 1, 0), iv(2, 9, 1, 1, 1),
                 iv(3, 9, 4, 2, 0), iv(3, 9, 4, 2, 1), iv(4, 5, 3, 3, 0), iv(4, 9, 1, 3, 1),
                 iv(4, 5, 3, 3, 2), iv(5, 9, 3, 4, 0)]
    placed, high = osched._allocate(intervals)
    got = {(p["source_scale"], p["head"]): p["offset"] for p in placed}
    # (2,0): best fit takes the exact 4-row hole at 11 over the 9-row hole at 0;
    # (4,0): two exact 3-row holes (4 and 16) -> lowest offset
    assert got == {(0, 0): 0, (0, 1): 9, (1, 0): 11, (1, 1): 15, (2, 0): 11, (2, 1): 0,
                   (3, 0): 4, (3, 2): 16, (3, 1): 7, (4, 0): 4}
    assert high == 19


def test_merge_free_blocks():
    assert osched.merge_free_blocks([(10, 5), (0, 4), (4, 2), (20, 0), (14, 3)]) == [(0, 6), (10, 7)]
    fl = ps._FreeList()
    for off, n in [(10, 5), (0, 4), (4, 2), (20, 0), (14, 3)]:
        fl.release(off, n)
    assert list(zip(fl.offsets, fl.lengths)) == [(0, 6), (10, 7)]
    assert fl.take_best_fit(7) == 10 and list(zip(fl.offsets, fl.lengths)) == [(0, 6)]
    assert fl.take_best_fit(7) is None


@pytest.mark.parametrize("seed", range(40))
def test_invariants_random_progressive(seed):
    removed, ranges, H = _random_progressive(seed)
    _check_invariants(_oracle(removed, ranges, H), H)


# ------------------------------------------------------------------ product vs oracle


@pytest.mark.parametrize("seed", range(60))
def test_product_matches_oracle_random(seed):
    removed, ranges, H = _random_progressive(seed, num_scales=6 + seed % 6, H=3 + seed % 5)
    _assert_same(_product(removed, ranges, H), _oracle(removed, ranges, H))


@pytest.mark.parametrize("cfg", [1, 2, 4, 5])
def test_product_matches_oracle_workloads(cfg):
    wl = W.config(cfg)
    H, n_prior = wl.keep.shape
    removed = {t: {s: {h for h in range(H) if not bool(wl.keep[h, s])} for s in range(min(t, n_prior))}
               for t in range(1, len(wl.sides))}
    orc = _oracle(removed, osched.scale_token_ranges(wl.sides), H)
    _assert_same(wl.schedule, orc)


def test_static_slot_schedule_controller_entry():
    class Controller:
        scale_schedule = [(1, s, s) for s in ps.SIDES_1M[:6]]
        scale_ranges = ps.scale_token_ranges(ps.SIDES_1M[:6])

        def removed_heads_by_source_for(self, layer, target):
            assert layer == 3
            return {s: ({1} if s >= 2 else set()) for s in range(target)}

    sched = ps.build_static_slot_schedule(Controller(), layer_idx=3, num_heads=2)
    assert sched.capacity == 1 * 2 + 4 * 2 + 16 + 36 + 64
    assert sched.tables[5][2].tolist() == [5, 2]
    assert torch.equal(sched.tables[5][0][1], torch.tensor([1, 6, 0, 0, 0], dtype=torch.int32))
