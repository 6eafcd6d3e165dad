"""Host control flow of SegmentedLayerCache on the CPU (no GPU, no HIP).

The HIP operators are replaced, for this test only, by CPU restatements
from oracle/ (attention: oracle/segmented_attention.py; pack: oracle/pack.py;
the dense-prefix concatenation: torch.cat, what it computes)
so the dense prefix -> activation -> segmented -> append -> reset flow of
enable_real_pruning_fast.py:1951-2254 can be checked here: every step's
output must equal attention over the keys a static keep policy retains, the
phase profiler must see the reference's phases, and the slab must hold the
retained rows bit-exactly.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from heatkv_amd import phase_profile as prof
from heatkv_amd import segmented_cache as sc
from heatkv_amd import workloads as W
from oracle import pack as opack
from oracle import segmented_attention as oattn


def _cpu_attention(*, q, persisted_k, persisted_v, segment_starts, segment_ends, segment_counts,
                   current_k, current_v, softmax_scale, softmax_mode="exp", append_offsets=None, append_also=None,
                   **_):
    if append_offsets is not None:
        # the fused append (and its second destination), written before the
        # attention reads the slab: a row that a segment of this call covered
        # would change the result
        L = current_k.shape[2]
        dests = [(persisted_k, persisted_v, append_offsets)]
        if append_also is not None:
            dests.append(append_also)
        for dk, dv, offs in dests:
            for h, off in enumerate(offs.tolist()):
                if 0 <= off <= dk.shape[1] - L:
                    dk[:, off:off + L] = current_k[:, h]
                    dv[:, off:off + L] = current_v[:, h]
    f = lambda t: None if t is None else t.float().numpy()  # noqa: E731
    out, _ = oattn.flat_segmented_attention(
        f(q), f(persisted_k), f(persisted_v), segment_starts.numpy(), segment_ends.numpy(),
        segment_counts.numpy(), f(current_k), f(current_v), softmax_scale)
    return torch.from_numpy(out).to(q.dtype)


def _cpu_pack(*, dst_k, dst_v, src_k, src_v, dst_starts, src_starts, lengths, max_length=None, **_):
    for dst, src in ((dst_k, src_k), (dst_v, src_v)):
        d = dst.view(torch.int16).numpy() if dst.element_size() == 2 else dst.numpy()
        s = src.view(torch.int16).numpy() if src.element_size() == 2 else src.numpy()
        opack.pack_flat_segments(d, s, dst_starts.tolist(), src_starts.tolist(), lengths.tolist())
    return dst_k, dst_v


def _cpu_concat(old_k, new_k, old_v, new_v):
    return torch.cat((old_k, new_k), dim=2), torch.cat((old_v, new_v), dim=2)


@pytest.fixture
def cpu_ops(monkeypatch):
    monkeypatch.setattr(sc, "fused_real_pruning_flat_segmented_attention", _cpu_attention)
    monkeypatch.setattr(sc, "pack_flat_segments_kv", _cpu_pack)
    monkeypatch.setattr(sc, "concat_kv", _cpu_concat)


def _expected(inputs, keep, t, scale):
    """Attention of scale t over the retained prior scales + itself, per (b, h)."""
    q, k, v = inputs[t]
    B, H, L, D = q.shape
    out = np.zeros((B, L, H * D), np.float32)
    for h in range(H):
        ks = [inputs[s][1][:, h] for s in W.retained_scales(keep, t, h)] + [k[:, h]]
        vs = [inputs[s][2][:, h] for s in W.retained_scales(keep, t, h)] + [v[:, h]]
        kk = torch.cat(ks, dim=1).float().numpy()
        vv = torch.cat(vs, dim=1).float().numpy()
        for b in range(B):
            o, _ = oattn.flat_segmented_attention(
                q[b:b + 1, h:h + 1].float().numpy(), None, None, np.zeros((1, 0), np.int32),
                np.zeros((1, 0), np.int32), np.zeros(1, np.int32), kk[b][None, None], vv[b][None, None], scale)
            out[b, :, h * D:(h + 1) * D] = o[0]
    return out


@pytest.mark.parametrize("baseline_prefix", ["1", "0"])
def test_generation_flow_matches_retained_key_attention(cpu_ops, monkeypatch, baseline_prefix):
    monkeypatch.setenv("REAL_PRUNING_FUSED_SEGMENTED_BASELINE_PREFIX", baseline_prefix)
    sides = (1, 2, 4, 6, 8)
    H, B, D = 4, 2, 16
    g = torch.Generator().manual_seed(3)
    keep = torch.rand((H, len(sides) - 1), generator=g) < 0.5
    keep[:, :2] = True
    sched = W.schedule_from_keep(keep, sides)
    cache = sc.SegmentedLayerCache(sched, W.removed_from_keep(keep, len(sides)), num_heads=H)
    inputs = W.generation_inputs(batch=B, heads=H, sides=sides, seed=5, dtype=torch.float32, head_dim=D)
    scale = D ** -0.5
    prof.set_real_pruning_fast_phase_profile_enabled(True)
    try:
        for t, (q, k, v) in enumerate(inputs):
            out = cache.step(q, k, v, t, scale)
            np.testing.assert_allclose(out.numpy(), _expected(inputs, keep, t, scale), rtol=2e-5, atol=2e-5)
            if cache.active and t + 1 < len(sides):
                # the slab holds every segment live at t + 1, bit-exact
                for seg in sched.live_segments(t + 1):
                    src_k = inputs[seg.source_scale][1][:, seg.head]
                    got = cache.cached_k[:, seg.offset:seg.offset + seg.length]
                    assert torch.equal(got, src_k), (t, seg)
        snap = prof.snapshot_real_pruning_fast_phase_profile()
    finally:
        prof.set_real_pruning_fast_phase_profile_enabled(False)
    assert cache.logical_len == 0 and cache.cached_k is None  # reset at the final scale
    assert snap["calls"]["attention"] == len(sides)
    assert snap["calls"].get("compact", 0) >= 1
    assert snap["segmented_flat_stats"]["storage_allocations"] == 1


def test_unpruned_policy_stays_dense(cpu_ops):
    sides = (1, 2, 4)
    H = 2
    keep = torch.ones((H, len(sides) - 1), dtype=torch.bool)
    sched = W.schedule_from_keep(keep, sides)
    cache = sc.SegmentedLayerCache(sched, W.removed_from_keep(keep, len(sides)), num_heads=H)
    inputs = W.generation_inputs(batch=1, heads=H, sides=sides, seed=1, dtype=torch.float32, head_dim=8)
    for t, (q, k, v) in enumerate(inputs[:-1]):
        cache.step(q, k, v, t, 0.3)
        assert not cache.active
        dk, dv = cache.dense_kv()
        assert dk.shape[2] == sum(s * s for s in sides[:t + 1])
        # the dense prefix holds every row so far, in order
        assert torch.equal(dk, torch.cat([inputs[s][1] for s in range(t + 1)], dim=2))
        assert torch.equal(dv, torch.cat([inputs[s][2] for s in range(t + 1)], dim=2))


@pytest.mark.parametrize("fused_append", ["1", "0"])
def test_dense_prefix_in_place_or_concatenated(cpu_ops, monkeypatch, fused_append):
    """With the fused append on, the dense prefix lives in one buffer sized
    for every dense scale (each step's rows written by its attention call,
    which also writes them into the slab, so the activation packs nothing);
    with it off, the cache concatenates and packs as the reference does.
    Same outputs and the same slab rows either way."""
    monkeypatch.setenv("HKV_FUSED_APPEND", fused_append)
    sides = (1, 2, 4, 6, 8)
    H, B, D = 3, 2, 16
    keep = torch.ones((H, len(sides) - 1), dtype=torch.bool)
    keep[1, 0] = False  # the first removal is at target 4: scales 0-3 are the dense prefix
    keep[2, 1] = False
    keep[:, :3] = True
    keep[0, 3] = False
    sched = W.schedule_from_keep(keep, sides)
    cache = sc.SegmentedLayerCache(sched, W.removed_from_keep(keep, len(sides)), num_heads=H)
    inputs = W.generation_inputs(batch=B, heads=H, sides=sides, seed=9, dtype=torch.float32, head_dim=D)
    packs = []

    def counting_pack(**kw):
        packs.append(kw["lengths"].tolist())
        return _cpu_pack(**kw)

    monkeypatch.setattr(sc, "pack_flat_segments_kv", counting_pack)
    for t, (q, k, v) in enumerate(inputs):
        out = cache.step(q, k, v, t, D ** -0.5)
        np.testing.assert_allclose(out.numpy(), _expected(inputs, keep, t, D ** -0.5), rtol=2e-5, atol=2e-5)
        if t < 3:
            assert (cache.dense_buf is not None) == (fused_append == "1") and not cache.active
            if cache.dense_buf is not None:
                assert cache.dense_buf[0].shape[2] == sum(s * s for s in sides[:4])
        elif t == 3:
            assert cache.active and cache.dense_buf is None
            # in place, the dense steps' launches also wrote their rows into the
            # slab (append_also), so the activation packed nothing; concatenated,
            # the activation packs the dense cache
            assert (len(packs) == 0) == (fused_append == "1")
            for seg in sched.live_segments(4):
                src = inputs[seg.source_scale][1][:, seg.head]
                assert torch.equal(cache.cached_k[:, seg.offset:seg.offset + seg.length], src), seg


@pytest.mark.parametrize("layer", [7, 0])
@pytest.mark.parametrize("fused_append", ["1", "0"])
def test_generation_flow_under_reference_policy(cpu_ops, monkeypatch, fused_append, layer):
    """The 13-scale generation of one layer under the reference's HeatKV
    policy (orders/2b.json, budget 0.1, first source scale 3; pinned by
    tests/test_policy.py): heads are dropped part-way, freed slab rows are
    reused by later appends, and every step still equals attention over the
    keys the policy keeps (head_dim 16 to keep the CPU run short).  With
    HKV_FUSED_APPEND on, the appends ride on the attention calls (the host
    stand-in writes them before it reads the slab)."""
    import json
    import os

    monkeypatch.setenv("HKV_FUSED_APPEND", fused_append)
    fused_calls = []   # appends fused into segmented attention calls (heads written)
    dense_calls = []   # dense-prefix calls that write their rows into the in-place buffer

    def counting_attention(**kw):
        if kw.get("append_offsets") is not None:
            (fused_calls if cache.active else dense_calls).append(int((kw["append_offsets"] >= 0).sum()))
        return _cpu_attention(**kw)

    monkeypatch.setattr(sc, "fused_real_pruning_flat_segmented_attention", counting_attention)

    from heatkv_amd import policy as P
    from heatkv_amd.slab_schedule import SIDES_1M, build_static_slot_schedule

    here = os.path.dirname(os.path.abspath(__file__))
    orders = json.load(open(os.path.join(here, "golden", "orders_2b.json")))
    H = 16
    ctrl = P.controller_for_budget(0.1, orders, num_layers=32, num_heads=H, protected_prefix_scales=3)
    sched = build_static_slot_schedule(ctrl, layer_idx=layer, num_heads=H)
    assert any(g.end_target < len(SIDES_1M) for g in sched.segments)  # progressive removal
    removed = lambda t: ctrl.removed_heads_by_source_for(layer, t)  # noqa: E731
    cache = sc.SegmentedLayerCache(sched, removed, num_heads=H)
    inputs = W.generation_inputs(batch=1, heads=H, sides=SIDES_1M, seed=9, dtype=torch.float32, head_dim=16)
    scale = 0.25
    for t, (q, k, v) in enumerate(inputs):
        out = cache.step(q, k, v, t, scale).numpy()
        rem = removed(t)
        for h in range(H):
            srcs = [s for s in range(t) if h not in rem.get(s, set())]
            kk = torch.cat([inputs[s][1][:, h] for s in srcs] + [k[:, h]], dim=1).numpy()
            vv = torch.cat([inputs[s][2][:, h] for s in srcs] + [v[:, h]], dim=1).numpy()
            o, _ = oattn.flat_segmented_attention(
                q[:, h:h + 1].numpy(), None, None, np.zeros((1, 0), np.int32), np.zeros((1, 0), np.int32),
                np.zeros(1, np.int32), kk[:, None], vv[:, None], scale)
            np.testing.assert_allclose(out[:, :, h * 16:(h + 1) * 16], o, rtol=2e-5, atol=2e-5)
        if cache.active and t + 1 < len(SIDES_1M):
            for seg in sched.live_segments(t + 1):
                got = cache.cached_k[:, seg.offset:seg.offset + seg.length]
                assert torch.equal(got, inputs[seg.source_scale][1][:, seg.head]), (t, seg)
    assert cache.cached_k is None
    if fused_append == "1":
        # layer 7 fuses one head's append at scale 9; layer 0 fuses most heads
        # at scales 8-11 and copies the rest after the attention
        assert sum(fused_calls) > 0 and (layer != 0 or len(fused_calls) == 4), fused_calls
        # the dense prefix grows in place, every head at every step before the
        # first target with removed heads
        act = next(t for t in range(1, len(SIDES_1M)) if any(len(s) for s in removed(t).values()))
        assert act >= 3 and dense_calls == [H] * act, (act, dense_calls)
    else:
        assert not fused_calls and not dense_calls


def test_fused_append_split_under_reference_policy(cpu_ops):
    """The producer-side append (rows written before the scale's attention)
    under orders/2b.json at budget 0.1: the split covers the whole append plan,
    the offered heads never touch a row the attention reads, and a generation
    that writes them ahead of attention (emulated on the host) equals the
    retained-key attention and keeps the live slab rows intact."""
    import json
    import os

    from heatkv_amd import policy as P
    from heatkv_amd.slab_schedule import SIDES_1M, build_static_slot_schedule

    here = os.path.dirname(os.path.abspath(__file__))
    orders = json.load(open(os.path.join(here, "golden", "orders_2b.json")))
    H = 16
    ctrl = P.controller_for_budget(0.1, orders, num_layers=32, num_heads=H, protected_prefix_scales=3)
    offered = 0
    for layer in range(32):
        sched = build_static_slot_schedule(ctrl, layer_idx=layer, num_heads=H)
        for (s, _), plan in sched.append_plans.items():
            offs, rest = sched.fused_append(s, "cpu")
            n = plan.sequence_len
            fused = set()
            if offs is not None:
                fused = {(int(o), h * n, n) for h, o in enumerate(offs.tolist()) if o >= 0}
            items = set(zip(plan.dst_starts, plan.src_starts, plan.lengths))
            assert fused | set(zip(rest.dst_starts, rest.src_starts, rest.lengths)) == items
            assert not fused & set(zip(rest.dst_starts, rest.src_starts, rest.lengths))
            live = [(g.offset, g.offset + g.length) for g in sched.live_segments(s)]
            for d, _, ln in fused:
                assert all(d + ln <= a or b <= d for a, b in live), (layer, s, d)
            offered += len(fused)
    assert offered > 0

    layer = 29
    sched = build_static_slot_schedule(ctrl, layer_idx=layer, num_heads=H)
    removed = lambda t: ctrl.removed_heads_by_source_for(layer, t)  # noqa: E731
    cache = sc.SegmentedLayerCache(sched, removed, num_heads=H)
    inputs = W.generation_inputs(batch=1, heads=H, sides=SIDES_1M, seed=5, dtype=torch.float32, head_dim=16)
    used = 0
    for t, (q, k, v) in enumerate(inputs):
        app = cache.producer_append(t, torch.float32, "cpu")
        if app is not None:
            slab_k, slab_v, offs = app
            L = k.shape[2]
            for h, o in enumerate(offs.tolist()):
                if o >= 0:
                    slab_k[:, o:o + L] = k[:, h]
                    slab_v[:, o:o + L] = v[:, h]
            used += 1
        out = cache.step(q, k, v, t, 0.25, appended=app is not None).numpy()
        rem = removed(t)
        for h in range(H):
            srcs = [s for s in range(t) if h not in rem.get(s, set())]
            kk = torch.cat([inputs[s][1][:, h] for s in srcs] + [k[:, h]], dim=1).numpy()
            vv = torch.cat([inputs[s][2][:, h] for s in srcs] + [v[:, h]], dim=1).numpy()
            o, _ = oattn.flat_segmented_attention(
                q[:, h:h + 1].numpy(), None, None, np.zeros((1, 0), np.int32), np.zeros((1, 0), np.int32),
                np.zeros(1, np.int32), kk[:, None], vv[:, None], 0.25)
            np.testing.assert_allclose(out[:, :, h * 16:(h + 1) * 16], o, rtol=2e-5, atol=2e-5)
        if cache.active and t + 1 < len(SIDES_1M):
            for seg in sched.live_segments(t + 1):
                got = cache.cached_k[:, seg.offset:seg.offset + seg.length]
                assert torch.equal(got, inputs[seg.source_scale][1][:, seg.head]), (t, seg)
    assert used >= 3
    with pytest.raises(RuntimeError, match="active slab"):
        cache.step(*inputs[0], 0, 0.25, appended=True)
