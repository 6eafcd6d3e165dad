"""GPU parity of the generation sweep the bench times: the bench's own
per-layer static keep policies (heatkv_amd.workloads.sweep_keep_policies,
budget 0.1, seed 1000 + layer, scales 0-2 forced kept) and per-layer inputs
(seed 2000 + layer), through SegmentedLayerCache for whole 13-scale 2B
generations (batch 2, 16 heads x 128, bf16): the dense prefix, the
activation pack at the first pruned target, the slab appends (fused into the
attention launch where their rows lie outside the step's segments) and the
attention of every step, with the work plans the cache builds.

Every (batch row, head) of every step against fp32 attention over exactly
the keys the policy keeps (oracle/segmented_attention.py), within the
contract tolerances, and after each append every live slab row bit-exact
against its source K/V.  The call site is the reference's per-layer-step
control flow (enable_real_pruning_fast.py:1951-2254).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from heatkv_amd import workloads as W
from heatkv_amd.segmented_cache import SegmentedLayerCache
from support import assert_attention_close, bits, kept_keys_reference, to_np

pytestmark = pytest.mark.gpu

LAYERS, HEADS, BATCH = 32, 16, 2


@pytest.mark.parametrize("layer", [0, 31])
def test_sweep_layer_generation(device, layer):
    sides = W.SIDES_1M
    keep = W.sweep_keep_policies(layers=LAYERS, heads=HEADS, sides=sides)[layer]
    sched = W.schedule_from_keep(keep, sides)
    print(f"[sweep] layer {layer} kept pairs {int(keep.sum())} capacity {sched.capacity}", flush=True)
    cache = SegmentedLayerCache(sched, W.removed_from_keep(keep, len(sides)), num_heads=HEADS)
    inputs = W.generation_inputs(batch=BATCH, heads=HEADS, sides=sides, seed=2000 + layer)
    scale = 1.0 / math.sqrt(128)
    checked_rows = 0
    for t, (q, k, v) in enumerate(inputs):
        out = cache.step(q.to(device), k.to(device), v.to(device), t, scale)
        torch.cuda.synchronize(device)
        ref, _ = kept_keys_reference(inputs, lambda h: W.retained_scales(keep, t, h), t, scale)
        o = to_np(out)
        for b in range(BATCH):
            for h in range(HEADS):
                sl = slice(h * 128, (h + 1) * 128)
                assert_attention_close(o[b, :, sl], None, ref[b, :, sl], None,
                                       what=f"layer {layer} step {t} b {b} h {h}")
        print(f"[sweep] layer {layer} step {t} ok (L={q.shape[2]})", flush=True)
        if cache.active and t + 1 < len(sides):
            slab_k, slab_v = bits(cache.cached_k), bits(cache.cached_v)
            live = list(sched.live_segments(t + 1))
            for seg in live:
                rows = slice(seg.offset, seg.offset + seg.length)
                assert np.array_equal(slab_k[:, rows], bits(inputs[seg.source_scale][1][:, seg.head])), (t, seg)
                assert np.array_equal(slab_v[:, rows], bits(inputs[seg.source_scale][2][:, seg.head])), (t, seg)
                checked_rows += seg.length
    # the slab held the pruned cache for the last steps (the cache resets after the final scale)
    assert checked_rows > 0
