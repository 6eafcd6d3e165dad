"""GPU parity of a whole 13-scale generation under the reference's HeatKV
policy (orders/2b.json at budget 0.1, protected prefix and first source
scale 3): heads are dropped part-way through the generation, so slab rows
freed by a dropped (source scale, head) are reused by later appends.

Per step, the attention output of SegmentedLayerCache (HIP pack + attention)
against fp32 attention over exactly the keys the policy keeps for each head
(oracle/segmented_attention.py), every (batch row, head) at every scale, and
after each append the live slab rows bit-exact against the source K/V.  The removed sets come from
heatkv_amd/policy.py, pinned to the reference by tests/test_policy.py.
"""

from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest
import torch

from heatkv_amd import policy as P
from heatkv_amd import segmented_cache as sc
from heatkv_amd import workloads as W
from heatkv_amd.slab_schedule import SIDES_1M, build_static_slot_schedule
from support import assert_attention_close, bits, kept_keys_reference, to_np

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
L_MODEL, H, START = 32, 16, 3


def _kept_sources(ctrl, layer, t, h):
    removed = ctrl.removed_heads_by_source_for(layer, t)
    return [s for s in range(t) if h not in removed.get(s, set())]


@pytest.mark.parametrize("layer,fused", [(0, "1"), (29, "1"), (0, "0")])
def test_generation_under_reference_policy(device, monkeypatch, layer, fused):
    # fused "1": appends whose rows lie outside the step's segments ride on its
    # attention launch (layer 0 has them at scales 8-11, next to copied heads)
    monkeypatch.setenv("HKV_FUSED_APPEND", fused)
    orders = json.load(open(os.path.join(HERE, "golden", "orders_2b.json")))
    ctrl = P.controller_for_budget(0.1, orders, num_layers=L_MODEL, num_heads=H, protected_prefix_scales=START)
    sched = build_static_slot_schedule(ctrl, layer_idx=layer, num_heads=H)
    dropped = sum(1 for g in sched.segments if g.end_target < len(SIDES_1M))
    print(f"[policy gen] layer {layer} fused {fused} capacity {sched.capacity} segments {len(sched.segments)} "
          f"dropped part-way {dropped}", flush=True)
    cache = sc.SegmentedLayerCache(sched, lambda t: ctrl.removed_heads_by_source_for(layer, t), num_heads=H)
    B = 2
    inputs = W.generation_inputs(batch=B, heads=H, sides=SIDES_1M, seed=100 + layer)
    scale = 1.0 / math.sqrt(128)
    for t, (q, k, v) in enumerate(inputs):
        out = cache.step(q.to(device), k.to(device), v.to(device), t, scale)
        torch.cuda.synchronize(device)
        ref, _ = kept_keys_reference(inputs, lambda h: _kept_sources(ctrl, layer, t, h), t, scale)
        o = to_np(out)
        for b in range(B):
            for h in range(H):
                sl = slice(h * 128, (h + 1) * 128)
                assert_attention_close(o[b, :, sl], None, ref[b, :, sl], None,
                                       what=f"layer {layer} step {t} b {b} h {h}")
        if cache.active and t + 1 < len(SIDES_1M):
            slab_k, slab_v = bits(cache.cached_k), bits(cache.cached_v)
            for seg in sched.live_segments(t + 1):
                rows = slice(seg.offset, seg.offset + seg.length)
                assert np.array_equal(slab_k[:, rows], bits(inputs[seg.source_scale][1][:, seg.head])), (t, seg)
                assert np.array_equal(slab_v[:, rows], bits(inputs[seg.source_scale][2][:, seg.head])), (t, seg)
    assert dropped > 0
