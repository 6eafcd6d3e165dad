"""Cache-method profiling harness for the attention path, with the reference
harness's result fields (profile_cache_methods.py:194-266).

The reference times whole Infinity generations (weights, text encoder, VAE),
which are not available here; this harness times the part of a generation
that the cache method changes: for every scale step and every layer, the
attention over the layer's KV cache and the cache update, on synthetic
per-layer q/k/v of the 2B shape (13-scale 1024^2 schedule, 16 heads x 128,
CFG pair per image).  Methods:

* ``baseline`` -- the unpruned dense cache: K/V of every scale appended to a
  ``[B, H, T, D]`` cache and attended in full (through the same HIP kernel,
  one segment per head over the dense cache, as the segmented cache's dense
  prefix does; the reference's baseline is the model's own attention);
* ``real_scale_fused_segmented`` (aliases ``fused-segmented``,
  ``fused_segmented``) -- the HeatKV policy for ``--head-specific-budget``
  and ``--head-specific-initial-scales``, one SegmentedLayerCache per layer
  (HIP pack + segmented attention), as
  ``enable_real_pruning_scale_specific_fused_segmented`` sets it up.

``--layer-forward`` times whole attention layers instead: per layer a
cosine-attention module with Infinity ``SelfAttention``'s parameters (random
bf16 weights, ``--embed-dim`` 2048 for the 2B model) whose forward the enable
entry replaces (QKV projection, HIP producer, segmented cache step, output
projection), the layers chained within each scale step, one random input per
scale.  ``baseline`` is then the same forward with nothing pruned (budget 1,
the dense cache of every scale).

``--graph`` captures one whole generation (all layer-steps) in a HIP graph
after an eager warm-up run and times replays.  Usage::

    python -m heatkv_amd.harness --methods baseline real_scale_fused_segmented \\
        --orders orders/2b.json --json-out out.json
"""

from __future__ import annotations

import argparse
import json
import math
import random
import statistics
from pathlib import Path
from typing import Iterable, List, Optional

import torch

from . import phase_profile as prof
from .enable import METHOD_ALIASES, METHOD_NAME, enable_real_pruning_scale_specific_fused_segmented
from .policy import controller_for_budget, load_orders
from .produce import precompute_rope2d_freqs_grid
from .segmented_cache import SegmentedLayerCache
from .slab_schedule import SIDES_1M, build_slab_schedule, build_static_slot_schedule, scale_token_ranges
from .workloads import generation_inputs

BASELINE = "baseline"


def normalize_method(name: str) -> str:
    key = str(name).strip()
    if key == BASELINE:
        return BASELINE
    if key == METHOD_NAME or key in METHOD_ALIASES:
        return METHOD_NAME
    raise ValueError(f"unsupported method: {name}")


def seeded_orders(num_layers: int, num_heads: int, num_orders: int, seed: int):
    """Removal orders in the orders/<model>.json format (one permutation of the
    (head, layer) slots per source scale), drawn from ``seed``; stands in for
    a model's calibrated orders when none are given."""
    rng = random.Random(seed)
    slots = [[h, l] for l in range(num_layers) for h in range(num_heads)]
    out = []
    for _ in range(num_orders):
        order = list(slots)
        rng.shuffle(order)
        out.append(order)
    return out


def build_layers(method: str, *, num_layers: int, num_heads: int, budget: float, initial_scales: int,
                 orders) -> List:
    if method == BASELINE:
        none = build_slab_schedule(lambda t: {}, num_heads=num_heads, scale_ranges=scale_token_ranges(SIDES_1M))
        return [SegmentedLayerCache(none, lambda t: {}, num_heads=num_heads) for _ in range(num_layers)]
    ctrl = controller_for_budget(budget, orders, num_layers=num_layers, num_heads=num_heads,
                                 protected_prefix_scales=initial_scales, source_scale_start=initial_scales)
    layers = []
    for layer in range(num_layers):
        sched = build_static_slot_schedule(ctrl, layer_idx=layer, num_heads=num_heads)
        layers.append(SegmentedLayerCache(
            sched, lambda t, layer=layer: ctrl.removed_heads_by_source_for(layer, t), num_heads=num_heads))
    return layers


class SyntheticSelfAttention(torch.nn.Module):
    """Cosine-attention layer with the parameters and attributes of Infinity's
    ``SelfAttention`` (infinity/models/basic.py:196-246), randomly initialized
    from ``seed``; learned scales spread over [log 4, log 100].  Its own
    forward is never used: the enable entry replaces it."""

    def __init__(self, embed_dim: int, num_heads: int, seed: int):
        super().__init__()
        gen = torch.Generator().manual_seed(int(seed))
        self.num_heads, self.head_dim = int(num_heads), int(embed_dim) // int(num_heads)
        self.cos_attn, self.scale, self.caching = True, 1, False
        self.max_scale_mul = math.log(100)
        self.scale_mul_1H11 = torch.nn.Parameter(
            torch.linspace(math.log(4.0), math.log(100.0), num_heads).reshape(1, num_heads, 1, 1))
        bound = 1.0 / math.sqrt(embed_dim)
        self.mat_qkv = torch.nn.Linear(embed_dim, 3 * embed_dim, bias=False)
        self.proj = torch.nn.Linear(embed_dim, embed_dim)
        with torch.no_grad():
            self.mat_qkv.weight.uniform_(-bound, bound, generator=gen)
            self.proj.weight.uniform_(-bound, bound, generator=gen)
            self.proj.bias.uniform_(-bound, bound, generator=gen)
        self.q_bias = torch.nn.Parameter(torch.randn(embed_dim, generator=gen) * 0.02)
        self.v_bias = torch.nn.Parameter(torch.randn(embed_dim, generator=gen) * 0.02)
        self.register_buffer("zero_k_bias", torch.zeros(embed_dim))
        self.proj_drop = torch.nn.Identity()
        self.cached_k = self.cached_v = None

    def kv_caching(self, enable: bool):
        self.caching = bool(enable)
        self.cached_k = self.cached_v = None

    def forward(self, *args, **kwargs):
        raise NotImplementedError("enable_real_pruning_scale_specific_fused_segmented replaces this forward")


def build_model(method: str, *, device, num_layers: int, num_heads: int, embed_dim: int, budget: float,
                initial_scales: int, orders, seed: int = 0) -> torch.nn.ModuleList:
    """Chained synthetic attention layers (bf16) with the fused segmented path
    enabled; ``baseline`` enables it at budget 1 (nothing pruned)."""
    model = torch.nn.ModuleList([SyntheticSelfAttention(embed_dim, num_heads, seed * 1000 + l)
                                 for l in range(num_layers)])
    model = model.to(device=device, dtype=torch.bfloat16)
    return enable_real_pruning_scale_specific_fused_segmented(
        model, 1.0 if method == BASELINE else budget, orders, protected_prefix_scales=initial_scales,
        source_scale_start=initial_scales,
        module_filter=lambda m: isinstance(m, SyntheticSelfAttention))


def profile_one(method: str, batch_size: int, *, device, num_layers: int = 32, num_heads: int = 16,
                budget: float = 0.1, initial_scales: int = 3, orders=None, seed: int = 0, warmup: int = 1,
                repeats: int = 2, phase_profile: bool = True, graph: bool = False,
                layer_forward: bool = False, embed_dim: int = 2048) -> dict:
    """One (method, batch size) result with the reference harness's fields."""
    method = normalize_method(method)
    if orders is None:
        orders = seeded_orders(num_layers, num_heads, 12 - initial_scales, seed)
    B = 2 * int(batch_size)  # CFG pair per image
    sink: List[torch.Tensor] = []
    if layer_forward:
        generation = _layer_generation(method, B, sink, device=device, num_layers=num_layers,
                                       num_heads=num_heads, embed_dim=embed_dim, budget=budget,
                                       initial_scales=initial_scales, orders=orders, seed=seed)
    else:
        layers = build_layers(method, num_layers=num_layers, num_heads=num_heads, budget=budget,
                              initial_scales=initial_scales, orders=orders)
        inputs = [generation_inputs(batch=B, heads=num_heads, sides=SIDES_1M, seed=seed * 1000 + l,
                                    device=device) for l in range(num_layers)]
        scale = 1.0 / math.sqrt(128)

        def generation():
            sink.clear()
            for t in range(len(SIDES_1M)):
                for l in range(num_layers):
                    q, k, v = inputs[l][t]
                    sink.append(layers[l].step(q, k, v, t, scale))

    use_prof = phase_profile and method == METHOD_NAME and not graph
    g = None
    if graph:
        generation()  # eager run: builds every cached device table and copy plan
        torch.cuda.synchronize(device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            generation()
    timings, phases, peak_alloc, peak_res = [], [], [], []
    if use_prof:
        prof.set_real_pruning_fast_phase_profile_enabled(True)
    try:
        for run in range(warmup + repeats):
            torch.cuda.synchronize(device)
            torch.cuda.reset_peak_memory_stats(device)
            if use_prof:
                prof.reset_real_pruning_fast_phase_profile()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            if g is not None:
                g.replay()
            else:
                generation()
            end.record()
            end.synchronize()
            if run >= warmup:
                timings.append(float(start.elapsed_time(end)))
                peak_alloc.append(int(torch.cuda.max_memory_allocated(device)))
                peak_res.append(int(torch.cuda.max_memory_reserved(device)))
                if use_prof:
                    phases.append(prof.snapshot_real_pruning_fast_phase_profile(reset=True))
    finally:
        if use_prof:
            prof.set_real_pruning_fast_phase_profile_enabled(False)
    return {
        "method": method,
        "batch_size": int(batch_size),
        "decode": False,
        "warmup": int(warmup),
        "repeats": int(repeats),
        "latency_ms": timings,
        "median_ms": statistics.median(timings),
        "mean_ms": statistics.fmean(timings),
        "per_image_median_ms": statistics.median(timings) / float(batch_size),
        "peak_allocated_bytes": max(peak_alloc) if peak_alloc else 0,
        "peak_reserved_bytes": max(peak_res) if peak_res else 0,
        "phase_profiles": phases,
        "graph": bool(graph),
        "layer_forward": bool(layer_forward),
    }


def _layer_generation(method, B, sink, *, device, num_layers, num_heads, embed_dim, budget, initial_scales,
                      orders, seed):
    """A generation of chained synthetic attention layers (patched forward
    under bf16 autocast): returns the callable that runs one image."""
    model = build_model(method, device=device, num_layers=num_layers, num_heads=num_heads,
                        embed_dim=embed_dim, budget=budget, initial_scales=initial_scales, orders=orders,
                        seed=seed)
    sched = [(1, s, s) for s in SIDES_1M]
    grid = precompute_rope2d_freqs_grid(embed_dim // num_heads, {1.0: {"1M": {"scales": sched}}}, 2,
                                        pad_to_multiplier=128, device=device)
    gen = torch.Generator().manual_seed(int(seed))
    xs = [torch.randn((B, s * s, embed_dim), generator=gen).to(device=device, dtype=torch.bfloat16)
          for s in SIDES_1M]

    @torch.no_grad()
    def generation():
        sink.clear()
        for layer in model:
            layer.kv_caching(True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            for t in range(len(SIDES_1M)):
                x = xs[t]
                for layer in model:
                    x = layer(x, None, None, sched, grid, t)
                sink.append(x)

    return generation


def main(argv: Optional[Iterable[str]] = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--methods", nargs="+", default=[BASELINE, METHOD_NAME])
    ap.add_argument("--batch-sizes", type=lambda s: [int(x) for x in s.split(",")], default=[1])
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--repeats", type=int, default=2)
    ap.add_argument("--disable-phase-profile", action="store_true")
    ap.add_argument("--head-specific-budget", type=float, default=0.1)
    ap.add_argument("--head-specific-initial-scales", type=int, default=3)
    ap.add_argument("--orders", type=str, default=None,
                    help="removal orders file (orders/<model>.json format); default: seeded orders")
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--heads", type=int, default=16)
    ap.add_argument("--graph", action="store_true", help="time HIP-graph replays of a whole generation")
    ap.add_argument("--layer-forward", action="store_true",
                    help="time whole attention layers (QKV projection, producer, cache step, projection)")
    ap.add_argument("--embed-dim", type=int, default=2048)
    ap.add_argument("--json-out", type=str, default=None)
    args = ap.parse_args(argv)
    if args.warmup < 0 or args.repeats <= 0:
        ap.error("--warmup must be >= 0 and --repeats must be > 0")
    device = torch.device("cuda:0")
    orders = load_orders(args.orders) if args.orders else None
    results = []
    for batch_size in args.batch_sizes:
        for method in args.methods:
            res = profile_one(method, batch_size, device=device, num_layers=args.layers, num_heads=args.heads,
                              budget=args.head_specific_budget, initial_scales=args.head_specific_initial_scales,
                              orders=orders, seed=args.seed, warmup=args.warmup, repeats=args.repeats,
                              phase_profile=not args.disable_phase_profile, graph=args.graph,
                              layer_forward=args.layer_forward, embed_dim=args.embed_dim)
            results.append(res)
            print(f"{res['method']} b{batch_size}: median={res['median_ms']:.1f} ms "
                  f"per_image={res['per_image_median_ms']:.1f} ms "
                  f"peak_alloc={res['peak_allocated_bytes'] / 2**30:.2f} GiB "
                  f"peak_reserved={res['peak_reserved_bytes'] / 2**30:.2f} GiB", flush=True)
    payload = {
        "config": {
            "methods": [normalize_method(m) for m in args.methods],
            "batch_sizes": args.batch_sizes,
            "seed": args.seed,
            "decode": False,
            "warmup": args.warmup,
            "repeats": args.repeats,
            "head_specific_budget": args.head_specific_budget,
            "head_specific_initial_scales": args.head_specific_initial_scales,
            "graph": args.graph,
            "layer_forward": args.layer_forward,
            "data": ("synthetic inputs, random bf16 weights; attention layers (projections, producer, "
                     "attention, cache update)" if args.layer_forward else
                     "synthetic per-layer q/k/v (2B shape); attention + cache update only"),
        },
        "results": results,
    }
    if args.json_out:
        Path(args.json_out).write_text(json.dumps(payload, indent=2))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
