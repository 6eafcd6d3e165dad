"""GPU: calls on two streams at once.

Attention launches that cut items (round split) keep per-item counters and
partial records in a workspace, one per (device, stream) in the Python layer.
Two such workloads issued alternately on two streams (default priority) must
give bit-for-bit the results they give one after the other on the current
stream, and each stream must hold its own workspace.  The producer runs on a
side stream too.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from heatkv_amd import _lib
from heatkv_amd import fused_real_pruning_flat_segmented_attention as attn
from heatkv_amd import produce as P
from heatkv_amd import workloads as W
from heatkv_amd.slab_schedule import SIDES_1M
from support import bits

pytestmark = pytest.mark.gpu


def _call(wl, device):
    slab_k, slab_v = W.build_slab(wl, device)
    st, en, ct = wl.schedule.device_tables(wl.target, device)
    return dict(q=wl.q.to(device), persisted_k=slab_k, persisted_v=slab_v, segment_starts=st,
                segment_ends=en, segment_counts=ct, current_k=wl.cur_k.to(device),
                current_v=wl.cur_v.to(device), softmax_scale=wl.softmax_scale)


def test_two_streams_match_sequential(device):
    # 7-scale shapes: 64 and 128 items, fewer than the CU slots, so items are cut
    wa = W.final_step(name="a", batch=2, heads=16, sides=W.SIDES_7, budget=0.1, seed=11)
    wb = W.final_step(name="b", batch=4, heads=16, sides=W.SIDES_7, budget=0.3, seed=12)
    ka, kb = _call(wa, device), _call(wb, device)
    torch.cuda.synchronize(device)
    want_a, want_b = bits(attn(**ka)), bits(attn(**kb))
    torch.cuda.synchronize(device)
    s1, s2 = torch.cuda.Stream(device), torch.cuda.Stream(device)
    s1.wait_stream(torch.cuda.current_stream(device))
    s2.wait_stream(torch.cuda.current_stream(device))
    outs_a, outs_b = [], []
    print("[streams] 8 alternating launches per stream", flush=True)
    for _ in range(8):
        with torch.cuda.stream(s1):
            outs_a.append(attn(**ka))
        with torch.cuda.stream(s2):
            outs_b.append(attn(**kb))
    torch.cuda.synchronize(device)
    for o in outs_a:
        assert np.array_equal(bits(o), want_a)
    for o in outs_b:
        assert np.array_equal(bits(o), want_b)
    idx = device.index if device.index is not None else torch.cuda.current_device()
    keys = {k for k in _lib._workspaces if k[0] == idx}
    assert {(idx, s1.cuda_stream), (idx, s2.cuda_stream)} <= keys


def test_producer_on_side_stream(device):
    sched = [(1, s, s) for s in SIDES_1M]
    table = P.rope2d_freqs_table(128, sched, 2, 128).to(device)
    gen = torch.Generator().manual_seed(3)
    qkv = torch.randn((2, 1024, 3 * 16 * 128), generator=gen).to(torch.bfloat16).to(device)
    sm = torch.linspace(4.0, 100.0, 16).to(device)
    start = P.rope_start(sched, 9)
    want = [bits(t) for t in P.qkv_produce(qkv, 16, scale_mul=sm, rope_table=table, rope_start_row=start)]
    torch.cuda.synchronize(device)
    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        got = P.qkv_produce(qkv, 16, scale_mul=sm, rope_table=table, rope_start_row=start)
    torch.cuda.synchronize(device)
    for g, w in zip(got, want):
        assert np.array_equal(bits(g), w)
