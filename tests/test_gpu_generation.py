"""GPU parity of a whole generation through SegmentedLayerCache (HIP pack + attention).

Config-1 shape (B=2, H=16, D=128, scales 1..16, bf16) with a static keep
policy: every step's output against fp32 attention over the keys the policy
retains (oracle/segmented_attention.py), within the contract tolerances, and
the slab's live rows bit-exact against the source K/V after each append.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from heatkv_amd import segmented_cache as sc
from heatkv_amd import workloads as W
from oracle import segmented_attention as oattn
from support import assert_attention_close, bits, to_np

pytestmark = pytest.mark.gpu


def _reference_step(inputs, keep, t, scale):
    q, k, v = inputs[t]
    B, H, L, D = q.shape
    out = np.zeros((B, L, H * D), np.float32)
    for h in range(H):
        scales = W.retained_scales(keep, t, h)
        kk = torch.cat([inputs[s][1][:, h] for s in scales] + [k[:, h]], dim=1)
        vv = torch.cat([inputs[s][2][:, h] for s in scales] + [v[:, h]], dim=1)
        z = np.zeros((1, 0), np.int32)
        o, _ = oattn.flat_segmented_attention(
            to_np(q[:, h:h + 1]), None, None, z, z, np.zeros(1, np.int32),
            to_np(kk[:, None]), to_np(vv[:, None]), scale)
        out[:, :, h * D:(h + 1) * D] = o
    return out


@pytest.mark.parametrize("baseline_prefix", ["1", "0"])
def test_generation_matches_oracle(device, monkeypatch, baseline_prefix):
    monkeypatch.setenv("REAL_PRUNING_FUSED_SEGMENTED_BASELINE_PREFIX", baseline_prefix)
    sides = W.SIDES_7
    B, H = 2, 16
    g = torch.Generator().manual_seed(11)
    keep = torch.rand((H, len(sides) - 1), generator=g, dtype=torch.float64) < 0.3
    keep[:, :3] = True
    print(f"[gen] prefix={baseline_prefix} kept pairs={int(keep.sum())}", flush=True)
    sched = W.schedule_from_keep(keep, sides)
    cache = sc.SegmentedLayerCache(sched, W.removed_from_keep(keep, len(sides)), num_heads=H)
    inputs = W.generation_inputs(batch=B, heads=H, sides=sides, seed=12)
    scale = 1.0 / math.sqrt(128)
    for t, (q, k, v) in enumerate(inputs):
        out = cache.step(q.to(device), k.to(device), v.to(device), t, scale)
        torch.cuda.synchronize(device)
        ref = _reference_step(inputs, keep, t, scale)
        assert_attention_close(to_np(out), None, ref, None, what=f"step {t}")
        if cache.active and t + 1 < len(sides):
            slab = bits(cache.cached_k)
            slab_v = bits(cache.cached_v)
            for seg in sched.live_segments(t + 1):
                rows = slice(seg.offset, seg.offset + seg.length)
                assert np.array_equal(slab[:, rows], bits(inputs[seg.source_scale][1][:, seg.head])), (t, seg)
                assert np.array_equal(slab_v[:, rows], bits(inputs[seg.source_scale][2][:, seg.head])), (t, seg)
    assert cache.cached_k is None
