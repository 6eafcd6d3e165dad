"""Replayed steps of SegmentedLayerCache give the same bits as the full step.

A cache records each eager GPU step of its first generation (the validated
attention launch and the state changes after it, heatkv_amd/segmented_cache.py
_StepReplay) and later generations repeat them without the step's host logic.
Three generations of the 2B sweep's layer 0 (13 scales, B=2, 16 heads, the
bench's static keep policy at budget 0.1, dense prefix -> activation ->
segmented steps with fused appends -> final reset) on one cache with the same
inputs: every output of generations 2 and 3 bit-identical to generation 1's
(whose outputs the sweep parity test checks against the oracle), and the
slab's live rows bit-exact after every step.  Changing a knob the launches
read (HKV_FUSED_APPEND) between generations drops the recorded steps (the
unfused path gives the same bits).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from heatkv_amd import workloads as W
from heatkv_amd.segmented_cache import SegmentedLayerCache
from support import bits

pytestmark = pytest.mark.gpu


def _generation(cache, inputs, device, scale):
    outs = []
    for t, (q, k, v) in enumerate(inputs):
        outs.append(cache.step(q, k, v, t, scale))
        torch.cuda.synchronize(device)
    return [bits(o) for o in outs]


def test_replayed_generations_bit_identical(device, monkeypatch):
    sides = W.SIDES_1M
    keep = W.sweep_keep_policies(layers=1, heads=16, sides=sides)[0]
    sched = W.schedule_from_keep(keep, sides)
    cache = SegmentedLayerCache(sched, W.removed_from_keep(keep, len(sides)), num_heads=16)
    inputs = [tuple(t.to(device) for t in x)
              for x in W.generation_inputs(batch=2, heads=16, sides=sides, seed=2000)]
    scale = 1.0 / math.sqrt(128)
    first = _generation(cache, inputs, device, scale)
    recorded = len(cache._replays)
    print(f"[replay] recorded steps {recorded}", flush=True)
    assert recorded == len(sides)
    for gen in (2, 3):
        again = _generation(cache, inputs, device, scale)
        for t, (a, b) in enumerate(zip(first, again)):
            assert np.array_equal(a, b), (gen, t)
    # a knob the launches read changes: the recorded steps are dropped and re-recorded
    monkeypatch.setenv("HKV_FUSED_APPEND", "0")
    off = _generation(cache, inputs, device, scale)
    assert 0 < len(cache._replays) < recorded  # the dense prefix now concatenates (a step not recorded)
    for t, (a, b) in enumerate(zip(first, off)):
        # the same attention with the append after the launch instead of in it
        assert np.array_equal(a, b), ("fused append off", t)


def test_replay_keeps_slab_rows(device):
    """Every live slab row bit-exact after each replayed step (as the full
    steps leave it)."""
    sides = W.SIDES_1M
    keep = W.sweep_keep_policies(layers=2, heads=16, sides=sides)[1]
    sched = W.schedule_from_keep(keep, sides)
    cache = SegmentedLayerCache(sched, W.removed_from_keep(keep, len(sides)), num_heads=16)
    inputs = [tuple(t.to(device) for t in x)
              for x in W.generation_inputs(batch=2, heads=16, sides=sides, seed=2001)]
    scale = 1.0 / math.sqrt(128)
    _generation(cache, inputs, device, scale)
    checked = 0
    for t, (q, k, v) in enumerate(inputs):
        cache.step(q, k, v, t, scale)
        torch.cuda.synchronize(device)
        if cache.active and t + 1 < len(sides):
            slab_k, slab_v = bits(cache.cached_k), bits(cache.cached_v)
            for seg in sched.live_segments(t + 1):
                rows = slice(seg.offset, seg.offset + seg.length)
                assert np.array_equal(slab_k[:, rows], bits(inputs[seg.source_scale][1][:, seg.head])), (t, seg)
                assert np.array_equal(slab_v[:, rows], bits(inputs[seg.source_scale][2][:, seg.head])), (t, seg)
                checked += seg.length
    assert checked > 0


def test_abi_bound_call_bit_identical(device):
    """hkv_segmented_attention_bind + hkv_segmented_attention_call (the
    library side of the replay) against hkv_segmented_attention on the 2B
    final step with its work plan and workspace: NaN-prefilled outputs, same
    bits; a block that was never bound is refused."""
    import ctypes

    from heatkv_amd import _lib, segmented_attention_plan

    wl = W.config(2)
    slab_k, slab_v = W.build_slab(wl, device)
    st, en, ct = wl.schedule.device_tables(wl.target, device)
    q, ck, cv = (t.to(device) for t in (wl.q, wl.cur_k, wl.cur_v))
    B, H, L, D = q.shape
    hst, hen, hct = wl.tables()
    plan = segmented_attention_plan(hst, hen, hct, batch_size=B, current_len=L, capacity=wl.schedule.capacity,
                                    device=device)
    ws = _lib.attention_workspace(device)
    lib = _lib.load()
    stream = torch.cuda.current_stream(device).cuda_stream
    codes = [_lib.dtype_code(t.dtype) for t in (q, ck, cv)]
    fixed = (B, H, L, wl.schedule.capacity, int(st.shape[1]), D, *codes, 0, float(wl.softmax_scale), 0, 0, 0,
             plan.data_ptr(), int(plan.shape[0]), ws.data_ptr(), ws.numel())
    ref = torch.full((B, L, H * D), float("nan"), dtype=q.dtype, device=device)
    _lib.check(lib.hkv_segmented_attention(q.data_ptr(), slab_k.data_ptr(), slab_v.data_ptr(), st.data_ptr(),
                                           en.data_ptr(), ct.data_ptr(), ck.data_ptr(), cv.data_ptr(),
                                           ref.data_ptr(), None, *fixed, stream))
    size = int(lib.hkv_segmented_attention_bound_bytes())
    block = (ctypes.c_int64 * ((size + 7) // 8))()
    unbound = (ctypes.c_int64 * ((size + 7) // 8))()
    _lib.check(lib.hkv_segmented_attention_bind(ctypes.addressof(block), size, st.data_ptr(), en.data_ptr(),
                                                ct.data_ptr(), *fixed, None))
    for _ in range(2):
        out = torch.full((B, L, H * D), float("nan"), dtype=q.dtype, device=device)
        _lib.check(lib.hkv_segmented_attention_call(ctypes.addressof(block), q.data_ptr(), slab_k.data_ptr(),
                                                    slab_v.data_ptr(), ck.data_ptr(), cv.data_ptr(),
                                                    out.data_ptr(), stream))
        torch.cuda.synchronize(device)
        assert np.array_equal(bits(out), bits(ref))
    code = lib.hkv_segmented_attention_call(ctypes.addressof(unbound), q.data_ptr(), slab_k.data_ptr(),
                                            slab_v.data_ptr(), ck.data_ptr(), cv.data_ptr(), out.data_ptr(), stream)
    assert code == _lib.HKV_ERR_INVALID_ARG
