"""GPU: a whole generation (every layer-step: dense prefix, activation pack,
segmented attention, appends) captured in a HIP graph and replayed gives the
eager results bit for bit, on every replay, with eager work between replays
(the harness's --graph mode, heatkv_amd/harness.py)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from heatkv_amd import _lib
from heatkv_amd import harness as Hn
from heatkv_amd.slab_schedule import SIDES_1M
from heatkv_amd.workloads import generation_inputs
from support import bits

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("method", ["real_scale_fused_segmented", "baseline"])
def test_graph_replays_match_eager(device, method):
    L, H = 3, 16
    orders = Hn.seeded_orders(L, H, 9, seed=2)
    layers = Hn.build_layers(method, num_layers=L, num_heads=H, budget=0.1, initial_scales=3, orders=orders)
    inputs = [generation_inputs(batch=2, heads=H, sides=SIDES_1M, seed=300 + l, device=device) for l in range(L)]
    scale = 1.0 / math.sqrt(128)
    sink = []

    def generation():
        sink.clear()
        for t in range(len(SIDES_1M)):
            for l in range(L):
                q, k, v = inputs[l][t]
                sink.append(layers[l].step(q, k, v, t, scale))

    print(f"[graph] {method}: eager reference", flush=True)
    generation()
    torch.cuda.synchronize(device)
    want = [bits(o) for o in sink]
    g = torch.cuda.CUDAGraph()
    before = dict(_lib._capture_workspaces)
    with torch.cuda.graph(g):
        generation()
    # one workspace for the whole capture (the calls run in order on its stream)
    new = [v for k, v in _lib._capture_workspaces.items() if before.get(k) is not v]
    assert len(new) == 1 and new[0][0] != 0
    outs = list(sink)
    for rep in range(3):
        print(f"[graph] {method}: replay {rep}", flush=True)
        g.replay()
        torch.cuda.synchronize(device)
        for i, (o, w) in enumerate(zip(outs, want)):
            assert np.array_equal(bits(o), w), (rep, i)
        generation()  # eager work between replays
        torch.cuda.synchronize(device)
        assert all(np.array_equal(bits(o), w) for o, w in zip(sink, want))


@pytest.mark.parametrize("method", ["real_scale_fused_segmented", "baseline"])
def test_layer_forward_graph_replays_match_eager(device, method):
    """Whole attention layers (QKV projection, HIP producer with the fused
    append, cache step, output projection) of a 13-scale generation, two
    chained 2B-shaped layers, captured in one HIP graph."""
    L, H = 2, 16
    orders = Hn.seeded_orders(L, H, 9, seed=4)
    sink = []
    generation = Hn._layer_generation(method, 2, sink, device=device, num_layers=L, num_heads=H,
                                      embed_dim=2048, budget=0.1, initial_scales=3, orders=orders, seed=5)
    print(f"[layer graph] {method}: eager reference", flush=True)
    generation()
    torch.cuda.synchronize(device)
    want = [bits(o) for o in sink]
    assert all(np.isfinite(o.float().cpu().numpy()).all() for o in sink)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        generation()
    outs = list(sink)
    for rep in range(3):
        print(f"[layer graph] {method}: replay {rep}", flush=True)
        g.replay()
        torch.cuda.synchronize(device)
        for i, (o, w) in enumerate(zip(outs, want)):
            assert np.array_equal(bits(o), w), (rep, i)
        generation()
        torch.cuda.synchronize(device)
        assert all(np.array_equal(bits(o), w) for o, w in zip(sink, want))
