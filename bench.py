"""Benchmark: segmented attention of the 2B 1024^2 final scale on one MI355X.

One step = one ``fused_real_pruning_flat_segmented_attention`` call of the
final 64x64 scale (B=2, H=16, D=128, 4096 queries, budget-0.1 slab over the
6425-token prior, seed 1) with its inputs resident in HBM.  The slab is packed
once before timing (the final scale appends nothing).  ``--warmup`` untimed
steps, after an untimed clock ramp of ``--ramp-ms`` GPU milliseconds of the
same step, then ``--steps`` back-to-back
steps between two HIP events recorded on the stream the kernel runs on;
prints one JSON line.

* ``value``: attention TFLOP/s over the timed steps, FLOPs counted as
  sum_(b,h) 4 L (R_h + L) D with R_h the retained prior rows (no padding, no
  masked lanes).
* ``roofline``: the attention kernel against the bf16 dense MFMA peak; its
  average duration is the timed region / steps (the step is that one kernel).
  ``traffic`` is the HBM bytes per launch from the committed rocprofv3
  FETCH_SIZE / WRITE_SIZE summary in profiles/ (copy-calibrated).
* ``compaction``: the slab fill (one append launch per kept prior scale)
  against HBM bandwidth, issued eagerly and as graph replays (device time);
  these launches move 0.02-2 MB each and are latency-bound.
  ``compaction_8b_dense`` (with the budget leg): the same fill for the
  8B-class workload at budget 1.0 (12 launches, 1.7 GB), where the pack
  kernel meets the HBM bound.
* ``sweep``: the 2B generation sweep (32 layers x 13 scale steps, B=2,
  H=16, per-layer static keep policies at budget 0.1): every layer-step runs
  SegmentedLayerCache.step (dense-prefix attention, activation pack,
  segmented attention, append), timed per image, eagerly and as replays of
  the whole image captured in one HIP graph; ``per_scale_step``: the image
  captured as one graph per scale (all layers), replayed in order with HIP
  events between the replays: ms for all 32 layers, us per layer-step,
  attention TFLOP/s and the fraction of the step's roofline (max of its
  attention FLOPs at the bf16 peak and its algorithmic HBM bytes at 8 TB/s;
  bytes = q, current K/V, output, retained prior K/V and every copied row
  read + written once); ``graph_kernel_floor_us``: device time per kernel
  node of a replayed graph of one-element kernels, the latency floor of the
  small scales; plus a phase split from a separately profiled image (the
  profiler synchronizes each phase).
* ``budgets_8b_class``: the 8B-class final step (B=8, H=32) at keep budgets
  0.05 / 0.1 / 0.2 / 1.0 (1.0 = every prior token kept, the dense-equivalent
  case), ms per step and TFLOP/s.
* ``producer``: the QKV producer epilogue (normalize, scale_mul, 2-D RoPE,
  permute; fp32 q/k, bf16 v) of the same final scale against HBM bandwidth:
  algorithmic bytes = the bf16 projection read + q/k/v written + the scale's
  RoPE table rows.
* ``real_model``: the same final step as the cosine-attention model runs it
  under bf16 autocast: fp32 unit-norm k (slab and current), fp32 q scaled
  by 30, bf16 v, softmax scale 1 (split-bf16 q/k products on the split-row
  kernel), with the nominal FLOP count.  K is held as split rows, as the
  producer writes it and the cache keeps it (``k_split_rows=True``);
  ``ms_per_step_k_split_per_call``: the same call on fp32 K, which the
  operator splits first (two more launches); ``tf32_mode``: the same step with
  q and k in fp16 (TF32's significand, REAL_PRUNING_FUSED_QK_DOT_MODE=tf32).
* ``measured_peaks``: what this device reaches on plain library work in the
  same run: a bf16 8192^3 GEMM (torch.matmul, hipBLASLt) in TFLOP/s and a
  1 GiB device copy in GB/s (read + write), beside the nominal 2.5 PF / 8 TB/s;
  ``attention_frac_of_gemm`` relates the attention to the former.
* ``skewed_ragged``: the skewed-ragged final step (B=16, H=16, seed 3,
  retained lengths log-uniform in [0, 6425]) as its own leg.
* The secondary legs' ms per step (``real_model``, ``budgets_8b_class``,
  ``skewed_ragged``) is the median of three back-to-back timing windows.
* ``cpu_baseline``: the reference CPU path restated in torch (gather +
  scaled_dot_product_attention, fp32) on the host cores over whole steps
  (median of 5 after a warm-up), rank 0 only; ``cores`` = the threads used
  (the per-GPU CPU share), ``host_cpu_count`` = what the OS reports.
* ``host_us_per_call``: host microseconds to enqueue one headline step
  through the public operator (every check);
  ``host_us_per_bound_call``: the same step through its pre-validated launch
  (BoundSegmentedAttention, what SegmentedLayerCache replays after the first
  generation); ``sweep.host_us_per_layer_step``: host time per layer-step
  of the eager sweep images (SegmentedLayerCache.step, replayed).
* ``clock_ramp_ms``: untimed GPU time of the headline step run before its
  ``--warmup`` (default 300 ms: a cold GPU ramps its clock during the first
  few hundred milliseconds of load).
"""

from __future__ import annotations

import argparse
import gc
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_FLOPS = 2.5e15  # MI355X dense bf16 MFMA
PEAK_HBM_BPS = 8.0e12     # MI355X HBM3E
PROFILES = os.path.join(ROOT, "profiles")
ATTN_KERNEL = "seg_attn_pipe_kernel"


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 4, 5],
                    help="final-step workload (2 = the 2B 1024^2 final scale)")
    ap.add_argument("--budget", type=float, default=None, help="keep budget (configs 1, 2, 4)")
    ap.add_argument("--ramp-ms", type=float, default=300.0,
                    help="untimed GPU milliseconds of the headline step before its warmup (clock ramp)")
    ap.add_argument("--no-skewed", action="store_true", help="skip the skewed-ragged final step (B=16)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-repeats", type=int, default=5)
    ap.add_argument("--no-sweep", action="store_true", help="skip the 32-layer generation sweep")
    ap.add_argument("--no-budgets", action="store_true",
                    help="skip the 8B-class budget sweep (B=8, H=32, budgets 0.05/0.1/0.2/1.0)")
    ap.add_argument("--no-producer", action="store_true", help="skip the QKV producer leg")
    ap.add_argument("--no-real-model", action="store_true", help="skip the fp32 q/k (model precision) leg")
    ap.add_argument("--no-peaks", action="store_true", help="skip the measured GEMM / copy peaks")
    ap.add_argument("--sweep-images", type=int, default=3)
    ap.add_argument("--pack-only", action="store_true",
                    help="profiling mode: only the 8B-class budget-1.0 slab fill (12 pack launches per "
                         "fill); prints its compaction record")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="also run a plain device copy of this many MiB (3 launches) so that a "
                         "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE pass can scale its counters")
    return ap.parse_args()


def attention_call(wl, device):
    """Inputs of one final-step call on ``device`` (slab packed by the HIP pack
    kernel), with the work plan of its tables (built on the host once, as the
    segmented cache does per layer and target; HKV_ATTN_PLAN=0 leaves it out)."""
    from heatkv_amd import workloads as W
    from heatkv_amd.segmented_cache import work_plans_enabled

    slab_k, slab_v = W.build_slab(wl, device)
    st, en, ct = wl.schedule.device_tables(wl.target, device)
    from heatkv_amd import attention_item_shape

    q, ck, cv = (t.to(device) for t in (wl.q, wl.cur_k, wl.cur_v))
    plan = (wl.schedule.device_work_plan(wl.target, device, wl.batch, wl.cur_len,
                                         item_shape=attention_item_shape(q.dtype, ck.dtype, cv.dtype, device=device))
            if work_plans_enabled(device) else None)
    return dict(q=q, persisted_k=slab_k, persisted_v=slab_v, segment_starts=st, segment_ends=en,
                segment_counts=ct, current_k=ck, current_v=cv, softmax_scale=wl.softmax_scale,
                work_plan=plan)


def clock_ramp(fn, device, min_ms=300.0, max_wall_s=5.0, chunk=50):
    """Untimed launches of ``fn`` until at least ``min_ms`` of GPU time has run
    (bounded by ``max_wall_s`` of wall time): the GPU leaves its idle clocks
    during the first few hundred milliseconds of load, so a short timed region
    that starts cold measures the ramp rather than the kernel.  Returns the
    GPU milliseconds spent and the launches made."""
    import torch

    stream = torch.cuda.current_stream(device)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    spent, launches = 0.0, 0
    wall0 = time.perf_counter()
    while spent < min_ms and time.perf_counter() - wall0 < max_wall_s:
        e0.record(stream)
        for _ in range(chunk):
            fn()
        e1.record(stream)
        torch.cuda.synchronize(device)
        spent += e0.elapsed_time(e1)
        launches += chunk
    return spent, launches


def time_attention(kw, device, steps, warmup):
    """Milliseconds per step over ``steps`` back-to-back calls (HIP events on
    the kernel's stream) after ``warmup`` untimed calls."""
    import torch

    from heatkv_amd import fused_real_pruning_flat_segmented_attention as attn

    for _ in range(warmup):
        attn(**kw)
    stream = torch.cuda.current_stream(device)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(device)
    # no garbage-collector pause while the host enqueues the timed steps (a
    # pause then would leave the GPU idle inside the timed region)
    gc_was_on = gc.isenabled()
    gc.disable()
    try:
        host0 = time.perf_counter()
        t0.record(stream)
        for _ in range(steps):
            attn(**kw)
        t1.record(stream)
        host_us = (time.perf_counter() - host0) / steps * 1e6
    finally:
        if gc_was_on:
            gc.enable()
    torch.cuda.synchronize(device)
    return t0.elapsed_time(t1) / steps, host_us


def time_bound_host(kw, device, steps):
    """Host microseconds to enqueue one call of the same step through a
    pre-validated launch (BoundSegmentedAttention: what SegmentedLayerCache
    replays), the inputs resident on the GPU."""
    import torch

    from heatkv_amd.real_pruning_fused_attention import BoundSegmentedAttention

    _, bound = BoundSegmentedAttention.bind(**kw)
    if bound is None:
        return float("nan")
    args = (kw["q"], kw["current_k"], kw["current_v"], kw["persisted_k"], kw["persisted_v"])
    torch.cuda.synchronize(device)
    gc_was_on = gc.isenabled()
    gc.disable()
    try:
        host0 = time.perf_counter()
        for _ in range(steps):
            bound(*args)
        host_us = (time.perf_counter() - host0) / steps * 1e6
    finally:
        if gc_was_on:
            gc.enable()
    torch.cuda.synchronize(device)
    return host_us


def time_attention_median(kw, device, steps, warmup, windows=3):
    """Median over ``windows`` back-to-back timing windows of ``steps`` calls
    each (one warm-up of ``warmup`` calls first): the secondary legs report
    the median, so one window stretched by a host-side stall (the host
    descheduled while the GPU queue drains) does not stand for the kernel."""
    ms = []
    for i in range(windows):
        ms.append(time_attention(kw, device, steps, warmup if i == 0 else 0)[0])
    return sorted(ms)[len(ms) // 2]


def time_pack(wl, device, reps=20):
    """The slab fill of ``wl`` (one append launch per kept prior scale):
    average duration issued eagerly (host work per launch included) and as
    replays of the launches captured in one HIP graph (device time only),
    algorithmic bytes (read + write of every packed row), launch count and
    the bytes of the largest launch."""
    import torch

    from heatkv_amd import pack_flat_segments_kv

    sched = wl.schedule
    B, H, _, D = wl.prior_k.shape
    slab_k = torch.empty((B, sched.capacity, D), dtype=wl.prior_k.dtype, device=device)
    slab_v = torch.empty_like(slab_k)
    calls = []
    nbytes = 0
    largest = 0
    esz = wl.prior_k.element_size() + wl.prior_v.element_size()
    for s, plan in wl.prior_append_plans():
        a, b = sched.scale_ranges[s]
        sk = wl.prior_k[:, :, a:b].to(device).reshape(B, H * (b - a), D)
        sv = wl.prior_v[:, :, a:b].to(device).reshape(B, H * (b - a), D)
        meta = sched.device_plan(plan, device, ("append", s))
        calls.append(dict(dst_k=slab_k, dst_v=slab_v, src_k=sk, src_v=sv, dst_starts=meta[0],
                          src_starts=meta[1], lengths=meta[2], max_length=plan.max_length))
        nbytes += B * plan.slots * D * esz * 2
        largest = max(largest, B * plan.slots * D * esz * 2)

    def fill():
        for c in calls:
            pack_flat_segments_kv(**c)

    ms = _events_ms(fill, device, reps, 3)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fill()
    ms_graph = _events_ms(graph.replay, device, reps, 3)
    launches = len(calls)
    del graph, calls, slab_k, slab_v
    torch.cuda.empty_cache()
    return {"ms": round(ms, 5), "ms_graph": round(ms_graph, 5), "bytes": nbytes, "launches": launches,
            "largest_launch_bytes": largest,
            "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "GB/s_graph": round(nbytes / (ms_graph * 1e-3) / 1e9, 1),
            "frac_hbm_graph": round(nbytes / (ms_graph * 1e-3) / PEAK_HBM_BPS, 4)}


def time_sweep(device, images, layers=32, heads=16, batch=2):
    """ms per image of the 2B generation sweep and its algorithmic attention FLOPs."""
    import math

    import torch

    from heatkv_amd import phase_profile as prof
    from heatkv_amd import workloads as W
    from heatkv_amd.segmented_cache import SegmentedLayerCache

    sides = W.SIDES_1M
    keeps = W.sweep_keep_policies(layers=layers, heads=heads, sides=sides)
    caches = [SegmentedLayerCache(W.schedule_from_keep(k, sides), W.removed_from_keep(k, len(sides)),
                                  num_heads=heads) for k in keeps]
    inputs = [W.generation_inputs(batch=batch, heads=heads, sides=sides, seed=2000 + l, device=device)
              for l in range(layers)]
    scale = 1.0 / math.sqrt(128)
    step_flops = [0] * len(sides)
    for keep in keeps:
        for t, side in enumerate(sides):
            n = side * side
            for h in range(heads):
                r = sum(sides[s] ** 2 for s in W.retained_scales(keep, t, h))
                step_flops[t] += batch * 4 * n * (r + n) * 128
    flops = sum(step_flops)
    # algorithmic HBM bytes per scale step: q, current K/V and the output
    # (bf16), every retained prior row of K/V read once, and each copied row
    # (append / activation pack) read and written once
    step_bytes = [0] * len(sides)
    for keep, cache in zip(keeps, caches):
        for t, side in enumerate(sides):
            n = side * side
            r = sum(sides[s] ** 2 for h in range(heads) for s in W.retained_scales(keep, t, h))
            copied = 0
            plan = cache.schedule.append_plans.get((t, t + 1))
            if plan is not None:
                copied += plan.slots
            act = cache.schedule.activation_plans.get(t + 1)  # packed at the end of step t
            if act is not None:
                copied += act.slots
            step_bytes[t] += batch * 128 * 2 * (4 * heads * n + 2 * r + 4 * copied)

    def image(marks=None):
        for t in range(len(sides)):
            if marks is not None:
                marks[t].record(torch.cuda.current_stream(device))
            for l in range(layers):
                q, k, v = inputs[l][t]
                caches[l].step(q, k, v, t, scale)
        if marks is not None:
            marks[-1].record(torch.cuda.current_stream(device))

    image()
    stream = torch.cuda.current_stream(device)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(device)
    gc_was_on = gc.isenabled()
    gc.disable()
    try:
        host0 = time.perf_counter()
        t0.record(stream)
        for _ in range(images):
            image()
        t1.record(stream)
        # host time to enqueue one layer-step (SegmentedLayerCache.step:
        # replayed steps after the first image)
        host_us_step = (time.perf_counter() - host0) / (images * layers * len(sides)) * 1e6
    finally:
        if gc_was_on:
            gc.enable()
    torch.cuda.synchronize(device)
    ms = t0.elapsed_time(t1) / images
    # the same image captured in one HIP graph (all 416 layer-steps): replays
    # without the host's per-call work
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        image()
    graph.replay()
    torch.cuda.synchronize(device)
    t0.record(stream)
    for _ in range(images):
        graph.replay()
    t1.record(stream)
    torch.cuda.synchronize(device)
    ms_graph = t0.elapsed_time(t1) / images
    del graph
    # per-scale graphs: the image captured as 13 graphs (one per scale, all
    # layers; one shared memory pool, replayed in capture order), with events
    # between the replays: device time of each scale step without host work
    pool = None
    scale_graphs = []
    for t in range(len(sides)):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=pool):
            for l in range(layers):
                q, k, v = inputs[l][t]
                caches[l].step(q, k, v, t, scale)
        pool = g.pool()
        scale_graphs.append(g)
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(len(sides) + 1)]
    step_ms = [0.0] * len(sides)
    reps = max(1, images)
    for g in scale_graphs:
        g.replay()
    torch.cuda.synchronize(device)
    for _ in range(reps):
        marks[0].record(stream)
        for t, g in enumerate(scale_graphs):
            g.replay()
            marks[t + 1].record(stream)
        torch.cuda.synchronize(device)
        for t in range(len(sides)):
            step_ms[t] += marks[t].elapsed_time(marks[t + 1]) / reps
    del scale_graphs
    floor_us = graph_launch_floor_us(device)
    per_step = []
    for t in range(len(sides)):
        roof_ms = max(step_flops[t] / PEAK_BF16_FLOPS, step_bytes[t] / PEAK_HBM_BPS) * 1e3
        per_step.append({"scale": t, "side": sides[t], "ms_all_layers": round(step_ms[t], 4),
                         "us_per_layer_step": round(step_ms[t] / layers * 1e3, 2),
                         "attention_tflops": round(step_flops[t] / (step_ms[t] * 1e-3) / 1e12, 1),
                         "roofline_us_per_layer_step": round(roof_ms / layers * 1e3, 3),
                         "roofline_bound": "mfma" if step_flops[t] / PEAK_BF16_FLOPS
                         >= step_bytes[t] / PEAK_HBM_BPS else "hbm",
                         "frac_roofline": round(roof_ms / step_ms[t], 4)})
    prof.set_real_pruning_fast_phase_profile_enabled(True)
    try:
        image()
        snap = prof.snapshot_real_pruning_fast_phase_profile()
    finally:
        prof.set_real_pruning_fast_phase_profile_enabled(False)
    return dict(what=f"{layers} layers x {len(sides)} scale steps, B={batch}, H={heads}, budget 0.1, "
                     "static per-layer keep policies (seed 1000 + layer)",
                ms_per_image=round(ms, 3), ms_per_image_graph=round(ms_graph, 3),
                host_us_per_layer_step=round(host_us_step, 2), attention_flops=flops,
                tflops=round(flops / (ms * 1e-3) / 1e12, 1),
                per_scale_step=per_step, graph_kernel_floor_us=round(floor_us, 2),
                phase_gpu_ms_profiled={k: round(v, 3) for k, v in snap["cuda_ms"].items()},
                phase_calls=snap["calls"],
                copy_bytes_per_image=int(snap["segmented_flat_stats"].get("static_copy_bytes", 0)))


def time_producer(device, batch=2, heads=16, reps=100, warmup=20):
    """QKV producer of the final 64x64 scale (L=4096) from a bf16 projection:
    average duration, algorithmic bytes and bandwidth."""
    import torch

    from heatkv_amd import produce as P
    from heatkv_amd.slab_schedule import SIDES_1M

    sched = [(1, s, s) for s in SIDES_1M]
    L, D = SIDES_1M[-1] ** 2, 128
    g = torch.Generator().manual_seed(0)
    qkv = torch.randn((batch, L, 3 * heads * D), generator=g).to(torch.bfloat16).to(device)
    sm = (torch.rand(heads, generator=g) * 4.6).exp().to(device)
    table = P.rope2d_freqs_table(D, sched, 2, 128).to(device)
    start = P.rope_start(sched, len(sched) - 1)

    def run():
        return P.qkv_produce(qkv, heads, scale_mul=sm, rope_table=table, rope_start_row=start)

    for _ in range(warmup):
        run()
    stream = torch.cuda.current_stream(device)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(device)
    t0.record(stream)
    for _ in range(reps):
        run()
    t1.record(stream)
    torch.cuda.synchronize(device)
    ms = t0.elapsed_time(t1) / reps
    elems = batch * L * heads * D
    nbytes = elems * 2 * 3 + elems * (4 + 4 + 2) + 2 * L * (D // 2) * 4
    # practical HBM ceiling for comparison: a plain device copy of the same size
    src = torch.empty(nbytes // 2, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize(device)
    c0 = torch.cuda.Event(enable_timing=True)
    c1 = torch.cuda.Event(enable_timing=True)
    c0.record(stream)
    for _ in range(20):
        dst.copy_(src)
    c1.record(stream)
    torch.cuda.synchronize(device)
    copy_gbs = 2 * src.numel() / (c0.elapsed_time(c1) / 20 * 1e-3) / 1e9
    del src, dst
    return {"what": f"QKV producer, final scale (B={batch}, L={L}, H={heads}), fp32 q/k, bf16 v",
            "kernel": "produce_kernel", "us": round(ms * 1e3, 2), "bytes": nbytes,
            "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac_hbm": round(nbytes / (ms * 1e-3) / PEAK_HBM_BPS, 4),
            "traffic": measured_traffic("produce_kernel", "2b_final_1024"),
            "copy_GB/s_same_bytes": round(copy_gbs, 1)}


def time_real_model(device, steps=50, warmup=20):
    """Final 2B step at the model's precision: fp32 q/k, bf16 v, scale 1."""
    import torch
    import torch.nn.functional as F

    from heatkv_amd import workloads as W

    from heatkv_amd import attention_item_shape
    from heatkv_amd.segmented_cache import work_plans_enabled

    wl = W.config(2)
    kw = attention_call(wl, device)
    plan16 = kw["work_plan"]
    kw["q"] = F.normalize(kw["q"].float(), dim=-1) * 30.0
    kw["current_k"] = F.normalize(kw["current_k"].float(), dim=-1)
    kw["persisted_k"] = F.normalize(kw["persisted_k"].float().nan_to_num(0.0), dim=-1)
    kw["softmax_scale"] = 1.0
    shape = attention_item_shape(torch.float32, torch.float32, kw["current_v"].dtype, device=device)
    kw["work_plan"] = (wl.schedule.device_work_plan(wl.target, device, wl.batch, wl.cur_len, item_shape=shape)
                       if work_plans_enabled(device) else None)
    # fp32 K split on every call (the operator's own split, two extra launches)
    ms_split = time_attention_median(kw, device, steps, warmup)
    # K as split rows, the form the producer writes and the cache keeps
    # (qkv_produce(k_split_rows=True)): the model path
    from heatkv_amd.real_pruning_fused_attention import _split_rows

    fp32_k = {name: kw[name] for name in ("current_k", "persisted_k")}
    stream = torch.cuda.current_stream(device)
    for name, t in fp32_k.items():
        kw[name] = _split_rows(t, stream).view(torch.float32)
    kw["k_split_rows"] = True
    ms = time_attention_median(kw, device, steps, warmup)
    del kw["k_split_rows"]
    kw.update(fp32_k)
    for name in ("q", "current_k", "persisted_k"):
        kw[name] = kw[name].half()
    kw["work_plan"] = plan16
    ms16 = time_attention_median(kw, device, steps, warmup)
    flops = wl.attention_flops()
    kernel = f"split-row kernel ({shape[0]}-query items), K held as split rows as the producer writes it"
    return {"what": f"2b_final_1024 with fp32 q (x30) / k (unit), bf16 v, scale 1 ({kernel})",
            "ms_per_step": round(ms, 4), "tflops_nominal": round(flops / (ms * 1e-3) / 1e12, 1),
            "pct_of_bf16_peak_nominal": round(100.0 * flops / (ms * 1e-3) / PEAK_BF16_FLOPS, 2),
            "ms_per_step_k_split_per_call": round(ms_split, 4),
            "tf32_mode": {"what": "same step, q/k in fp16 (16-bit kernel)", "ms_per_step": round(ms16, 4),
                          "tflops": round(flops / (ms16 * 1e-3) / 1e12, 1)}}


def _events_ms(fn, device, reps, warmup):
    import torch

    for _ in range(warmup):
        fn()
    stream = torch.cuda.current_stream(device)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(device)
    t0.record(stream)
    for _ in range(reps):
        fn()
    t1.record(stream)
    torch.cuda.synchronize(device)
    return t0.elapsed_time(t1) / reps


def graph_launch_floor_us(device, nodes=64):
    """Device time per kernel node of a replayed HIP graph of ``nodes`` one-element kernels."""
    import torch

    x = torch.zeros(1, device=device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(nodes):
            x.add_(1.0)
    ms = _events_ms(graph.replay, device, 20, 3)
    del graph
    return ms * 1e3 / nodes


def measured_peaks(device):
    """bf16 GEMM TFLOP/s and device-copy GB/s reached on this device."""
    import torch

    n = 8192
    a = torch.randn((n, n), device=device, dtype=torch.bfloat16)
    b = torch.randn((n, n), device=device, dtype=torch.bfloat16)
    ms_mm = _events_ms(lambda: torch.matmul(a, b), device, 20, 10)
    del a, b
    src = torch.empty(1 << 30, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    ms_cp = _events_ms(lambda: dst.copy_(src), device, 20, 5)
    del src, dst
    torch.cuda.empty_cache()
    return {"bf16_gemm_8192_tflops": round(2 * n ** 3 / (ms_mm * 1e-3) / 1e12, 1),
            "copy_1gib_GBps": round(2 * (1 << 30) / (ms_cp * 1e-3) / 1e9, 1),
            "nominal_bf16_tflops": PEAK_BF16_FLOPS / 1e12, "nominal_hbm_GBps": PEAK_HBM_BPS / 1e9}


def time_final_step(config, device, steps=20, warmup=10):
    """One final-step workload (by config number) as its own leg: ms per step,
    TFLOP/s and the fraction of the bf16 peak."""
    import torch

    from heatkv_amd import workloads as W

    wl = W.config(config)
    kw = attention_call(wl, device)
    ms = time_attention_median(kw, device, steps, warmup)
    flops = wl.attention_flops()
    rows = wl.retained_rows()
    del kw
    torch.cuda.empty_cache()
    return {"workload": wl.name, "batch": wl.batch, "heads": wl.heads, "seed": wl.seed,
            "retained_rows_min_max": [min(rows), max(rows)], "ms_per_step": round(ms, 4),
            "flops_per_step": flops, "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
            "frac_bf16_peak": round(flops / (ms * 1e-3) / PEAK_BF16_FLOPS, 4)}


def time_budgets(device, steps=20, warmup=10):
    """The 8B-class final step (B=8, H=32, seed 2) at keep budgets 0.05, 0.1,
    0.2 and 1.0 (the unpruned, dense-equivalent case): ms per step and TFLOP/s."""
    import torch

    from heatkv_amd import workloads as W

    base = W.config(4, budget=1.0)
    out = {}
    for budget in (0.05, 0.1, 0.2, 1.0):
        wl = W.with_budget(base, budget)
        kw = attention_call(wl, device)
        ms = time_attention_median(kw, device, steps, warmup)
        flops = wl.attention_flops()
        out[str(budget)] = {"ms_per_step": round(ms, 4), "flops_per_step": flops,
                            "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
                            "pct_of_bf16_peak": round(100.0 * flops / (ms * 1e-3) / PEAK_BF16_FLOPS, 2),
                            "slab_capacity": wl.schedule.capacity}
        del kw
        torch.cuda.empty_cache()
    return {"workload": base.name, "batch": base.batch, "heads": base.heads, "budgets": out}


def copy_calibration(device, mib):
    """Plain copy of ``mib`` MiB, three launches: reads and writes exactly that many bytes each."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize(device)


def _host_slab(wl):
    """The slab as the host sees it: each live segment's rows at its offset (fp32)."""
    import torch

    B, H, _, D = wl.prior_k.shape
    slab_k = torch.zeros((B, wl.schedule.capacity, D), dtype=torch.float32)
    slab_v = torch.zeros_like(slab_k)
    for seg in wl.schedule.live_segments(wl.target):
        slab_k[:, seg.offset:seg.offset + seg.length] = wl.prior_k[:, seg.head, seg.scale_start:seg.scale_end].float()
        slab_v[:, seg.offset:seg.offset + seg.length] = wl.prior_v[:, seg.head, seg.scale_start:seg.scale_end].float()
    return slab_k, slab_v


def _cpu_model():
    """The host CPU as lscpu names it, with its family / model / stepping (a
    virtual machine may report a short model name such as "AMD EPYC")."""
    import subprocess

    fields = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            fields[key.strip()] = val.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    if "Model name" not in fields:
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        fields["Model name"] = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
    name = fields.get("Model name", "unknown")
    ids = [f"{k.lower()} {fields[k]}" for k in ("CPU family", "Model", "Stepping") if fields.get(k)]
    return f"{name} ({', '.join(ids)})" if ids else name


def cpu_baseline(wl, repeats):
    """The reference CPU path restated in torch (per (b, h): gather the head's
    slab segments, append the current K/V, scaled_dot_product_attention, in
    fp32) on the host cores: 1 warm-up, then the median of ``repeats`` whole
    steps, for the headline workload and the 7-scale CPU-plumbing workload."""
    import torch

    from heatkv_amd import workloads as W
    from oracle import segmented_attention as oattn

    host_cpus = os.cpu_count() or 1
    # the pool's CPU share per GPU is 16 threads (OMP_NUM_THREADS there)
    threads = max(1, min(host_cpus, int(os.environ.get("OMP_NUM_THREADS", host_cpus))))
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)

    def median_ms(w, reps):
        st, en, ct = (t.numpy() for t in w.tables())
        sk, sv = _host_slab(w)
        args = (w.q, sk, sv, st, en, ct, w.cur_k, w.cur_v, w.softmax_scale)
        oattn.flat_segmented_attention_sdpa(*args)  # warm-up
        times = []
        for _ in range(reps):
            t = time.perf_counter()
            oattn.flat_segmented_attention_sdpa(*args)
            times.append(time.perf_counter() - t)
        return statistics.median(times) * 1e3

    try:
        ms = median_ms(wl, repeats)
        ms1 = median_ms(W.config(1), max(repeats, 5))
    finally:
        torch.set_num_threads(prev)
    return dict(value=round(wl.attention_flops() / (ms * 1e-3) / 1e12, 4), unit="TFLOP/s", cores=threads,
                host_cpu_count=host_cpus, cpu_model=_cpu_model(), kind="port",
                sample=f"{repeats} whole steps of {wl.name} (B={wl.batch}, H={wl.heads}, L={wl.cur_len}) "
                       "after 1 warm-up, median; torch gather + scaled_dot_product_attention in fp32 "
                       "(the reference CPU path restated)",
                ms_per_step=round(ms, 2), config1_ms_per_step=round(ms1, 3))


def measured_traffic(kernel: str, workload: str):
    """HBM bytes per dispatch of ``kernel`` on ``workload`` from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (copy-calibrated), or None."""
    path = os.path.join(PROFILES, f"{kernel}__{workload}.traffic.json")
    try:
        with open(path) as fh:
            rec = json.load(fh)
        return int(rec["bytes_per_dispatch"])
    except (OSError, KeyError, ValueError):
        return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this path has no collective); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from heatkv_amd import workloads as W

    device = torch.device("cuda:0")
    if args.pack_only:
        dense = W.config(4, budget=1.0)
        rec = {"compaction_8b_dense": dict(
            what=f"slab fill of {dense.name} at budget 1.0 (every prior row kept)", **time_pack(dense, device))}
        if args.copy_calib_mib > 0:
            copy_calibration(device, args.copy_calib_mib)
        print(json.dumps(rec), flush=True)
        return
    wl = W.config(args.config, budget=args.budget)
    flops = wl.attention_flops()
    kw = attention_call(wl, device)
    from heatkv_amd import fused_real_pruning_flat_segmented_attention as attn

    ramp_ms, ramp_launches = clock_ramp(lambda: attn(**kw), device, args.ramp_ms)
    ms_step, host_us = time_attention(kw, device, args.steps, args.warmup)
    host_us_bound = time_bound_host(kw, device, args.steps)
    achieved = flops / (ms_step * 1e-3)
    pack = time_pack(wl, device)
    if args.copy_calib_mib > 0:
        copy_calibration(device, args.copy_calib_mib)
    rec = {
        "metric": "segmented-attn TFLOP/s & % bf16 MFMA peak; ms per scale step (2B, 1024^2)",
        "value": round(achieved / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": wl.name, "batch": wl.batch, "heads": wl.heads, "head_dim": 128,
            "cur_len": wl.cur_len, "prior_tokens": wl.prefix, "budget": wl.budget, "seed": wl.seed,
            "retained_rows_per_head": wl.retained_rows(), "slab_capacity": wl.schedule.capacity,
            "flops_per_step": flops,
        },
        "pct_of_bf16_peak": round(100.0 * achieved / PEAK_BF16_FLOPS, 2),
        "roofline": {
            "bound": "mfma", "achieved": round(achieved / 1e12, 3), "peak": PEAK_BF16_FLOPS / 1e12,
            "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_FLOPS, 4),
            "traffic": measured_traffic(ATTN_KERNEL, wl.name),
            "kernel": ATTN_KERNEL, "kernel_ms_mean": round(ms_step, 5),
        },
        "clock_ramp_ms": round(ramp_ms, 1),
        "clock_ramp_launches": ramp_launches,
        "host_us_per_call": round(host_us, 1),
        "host_us_per_bound_call": round(host_us_bound, 2),
        "compaction": dict(what=f"slab fill of {wl.name}: one append launch per kept prior scale",
                           **pack),
    }
    if not args.no_skewed:
        rec["skewed_ragged"] = time_final_step(5, device)
    if not args.no_producer:
        rec["producer"] = time_producer(device)
    if not args.no_real_model:
        rec["real_model"] = time_real_model(device)
    if not args.no_sweep:
        rec["sweep"] = time_sweep(device, args.sweep_images)
    if not args.no_budgets:
        rec["budgets_8b_class"] = time_budgets(device)
        dense = W.config(4, budget=1.0)
        rec["compaction_8b_dense"] = dict(
            what=f"slab fill of {dense.name} at budget 1.0 (every prior row kept)", **time_pack(dense, device))
        del dense
    if not args.no_peaks:
        rec["measured_peaks"] = measured_peaks(device)
        rec["attention_frac_of_gemm"] = round(achieved / 1e12 / rec["measured_peaks"]["bf16_gemm_8192_tflops"], 4)
    if not args.no_cpu:
        rec["cpu_baseline"] = cpu_baseline(wl, args.cpu_repeats)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
