"""Host work plan of the attention kernel (hkv_segmented_attention_plan), on the CPU.

Checks, for the benchmark workloads and random tables: every (batch row,
head, 128-query tile) item's key tiles are covered exactly once by the plan's
units (empty units, head -1, leave at once), a cut item has exactly two parts
[0, a) and [a, n) with one counter index each, counters are dense and below
the slot count, on each XCD (unit id % 8) whole items come first heaviest
first and parts longest first, and the tile counts are those of the tables
(ceil(R_h / 64) + ceil(L / 64), with R_h the clamped retained rows).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from heatkv_amd import segmented_attention_plan
from heatkv_amd import workloads as W


def _rows(st, en, ct, cap):
    H, S = st.shape
    out = []
    for h in range(H):
        n = min(max(int(ct[h]), 0), S)
        r = 0
        for i in range(n):
            a = min(max(int(st[h, i]), 0), cap)
            b = min(max(int(en[h, i]), 0), cap)
            r += max(b - a, 0)
        out.append(r)
    return out


def _check(plan, st, en, ct, B, L, cap, slots):
    plan = plan.numpy()
    H = st.shape[0]
    n_qt = -(-L // 128)
    ntc = -(-L // 64)
    rows = _rows(st, en, ct, cap)
    tiles = {h: -(-rows[h] // 64) + ntc for h in range(H)}
    cover = {}
    cuts = {}
    # field 6: 1 in every unit when the items' tile counts differ by more
    # than 5/4 (the kernel then shares each CU tile by tile), else 0
    shared = int(4 * max(tiles.values()) > 5 * min(tiles.values())) if tiles else 0
    # field 7: 1 in every cut unit (its item's parts count in before
    # publishing: arrival-first merge), 0 in whole ones
    for h, j, t0, t1, cut, part, z0, z1 in plan.tolist():
        if h == -1:  # an empty unit
            assert (j, t0, t1, cut, part, z0, z1) == (-1, 0, 0, -1, 0, 0, 0)
            continue
        assert 0 <= h < H and 0 <= j < B * n_qt and z0 == shared and z1 == int(cut >= 0)
        assert 0 <= t0 < t1 <= tiles[h]
        cover.setdefault((h, j), []).append((t0, t1))
        if cut >= 0:
            cuts.setdefault(cut, []).append((h, j, part, t0, t1))
        else:
            assert (t0, t1) == (0, tiles[h])
    assert len(cover) == H * B * n_qt
    for (h, j), segs in cover.items():
        segs.sort()
        assert segs[0][0] == 0 and segs[-1][1] == tiles[h]
        assert all(a[1] == b[0] for a, b in zip(segs, segs[1:]))
    assert sorted(cuts) == list(range(len(cuts)))
    assert len(cuts) <= max(slots, 0)
    for c, ps in cuts.items():
        assert len(ps) == 2 and ps[0][:2] == ps[1][:2] and {p[2] for p in ps} == {0, 1}
        first = [p for p in ps if p[2] == 0][0]
        assert first[3] == 0 and first[4] - first[3] >= 4 and tiles[first[0]] - first[4] >= 4
    # on each XCD whole units come first, heaviest head first, then the parts
    # longest first (plans without cuts are permuted into XCD groups of equal
    # work instead)
    if cuts:
        units = plan.tolist()
        for x in range(8):
            mine = [u for u in units[x::8] if u[0] >= 0]
            whole = [u for u in mine if u[4] < 0]
            assert mine[:len(whole)] == whole
            sizes = [tiles[u[0]] for u in whole]
            assert sizes == sorted(sizes, reverse=True)
            lens = [u[3] - u[2] for u in mine[len(whole):]]
            assert lens == sorted(lens, reverse=True)
    # empty units only pad the XCD lists: fewer than 8 per unit index
    assert (plan[:, 0] < 0).sum() < 8 * max(1, -(-len(plan) // 8))
    return len(cuts)


@pytest.mark.parametrize("cfg", [1, 2, 5])
def test_plan_of_benchmark_workloads(cfg):
    wl = W.config(cfg)
    st, en, ct = (t.numpy() for t in wl.tables())
    cap = wl.schedule.capacity
    for slots in (0, 512):
        plan = segmented_attention_plan(st, en, ct, batch_size=wl.batch, current_len=wl.cur_len, capacity=cap,
                                        slots=slots)
        cuts = _check(plan, st, en, ct, wl.batch, wl.cur_len, cap, slots)
        if slots == 0:
            assert cuts == 0


def test_plan_cuts_the_2b_final_step():
    """The 2B final step (1024 items, two rounds of 512 slots, two heads with
    1.8x the others' key tiles) is cut; without cuts list scheduling ends at
    184 tile times against an average of 145.  Its items are dealt to XCDs in
    chunks of at least a quarter of a group: each (batch row, head) group's
    units land on at most 4 of the 8 XCDs, and every XCD list is padded to
    the same length."""
    wl = W.config(2)
    st, en, ct = (t.numpy() for t in wl.tables())
    plan = segmented_attention_plan(st, en, ct, batch_size=2, current_len=4096, capacity=wl.schedule.capacity,
                                    slots=512)
    assert _check(plan, st, en, ct, 2, 4096, wl.schedule.capacity, 512) > 0
    assert len(plan) % 8 == 0
    xcds = {}
    for i, (h, j) in enumerate(plan[:, :2].tolist()):
        if h >= 0:
            xcds.setdefault((h, j // 32), set()).add(i % 8)
    assert len(xcds) == 32 and max(len(v) for v in xcds.values()) <= 4


@pytest.mark.parametrize("seed", range(8))
def test_plan_random_tables(seed):
    g = torch.Generator().manual_seed(seed)
    H = int(torch.randint(1, 70, (1,), generator=g))
    S = int(torch.randint(0, 20, (1,), generator=g))
    B = int(torch.randint(1, 4, (1,), generator=g))
    L = int(torch.randint(1, 3000, (1,), generator=g))
    cap = int(torch.randint(0, 9000, (1,), generator=g))
    st = torch.randint(-10, cap + 10, (H, S), generator=g, dtype=torch.int32).numpy()
    en = (st + torch.randint(-5, 2000, (H, S), generator=g, dtype=torch.int32).numpy()).astype(np.int32)
    ct = torch.randint(-1, S + 2, (H,), generator=g, dtype=torch.int32).numpy()
    for slots in (0, 8, 512):
        plan = segmented_attention_plan(st, en, ct, batch_size=B, current_len=L, capacity=cap, slots=slots)
        _check(plan, st, en, ct, B, L, cap, slots)


def test_plan_argument_errors():
    z = np.zeros((2, 1), np.int32)
    c = np.zeros(2, np.int32)
    with pytest.raises(ValueError):
        segmented_attention_plan(z, z, c, batch_size=0, current_len=10, capacity=0, slots=4)
    with pytest.raises(ValueError):
        segmented_attention_plan(z, z[:1], c, batch_size=1, current_len=10, capacity=0, slots=4)
