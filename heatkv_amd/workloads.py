"""Seeded synthetic workloads of the segmented path (the five benchmark shapes).

Shapes follow Infinity's 13-scale 1:1 1M schedule (sides 1..64, 10521 tokens;
the prior before the 64x64 scale is 6425 tokens).  Inputs are N(0, 1) drawn in
fp32 from ``torch.Generator().manual_seed(seed)`` and rounded to the compute
dtype; keep policies are static per (head, source scale): a kept pair stays in
the slab for every later target, a dropped pair is never stored.

Draw order for a final-step workload (fixed, so goldens are reproducible):
policy uniforms, then q, then K of every scale, then V of every scale.

* ``final_step(...)``        -- configs 1, 2, 4: attention of the last scale
  over the slab (kept prior scales) plus itself.  Scales 0-2 are always kept;
  each other prior (head, scale) pair is kept with probability
  ``p = (budget * prefix - 21) / (prefix - 21)`` so that E[R_h] = budget * prefix.
* ``skewed_final_step(...)`` -- config 5: per head a target retained length
  ``floor(exp(U(0, ln(prefix + 1)))) - 1`` realised greedily as a subset of the
  prior scales (largest first), no forced scales.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Set

import torch

from .slab_schedule import SIDES_1M, SlabSchedule, build_slab_schedule, scale_token_ranges

SIDES_7 = SIDES_1M[:7]
HEAD_DIM = 128
FORCED_SCALES = 3


@dataclass
class FinalStepWorkload:
    """One final-scale attention step: inputs, policy, schedule and packed slab plan."""

    name: str
    batch: int
    heads: int
    sides: tuple
    seed: int
    budget: Optional[float]
    keep: torch.Tensor              # bool [H, n_prior_scales]
    q: torch.Tensor                 # [B, H, L, D] (dtype)
    prior_k: torch.Tensor           # [B, H, prefix, D] dense K of every prior scale
    prior_v: torch.Tensor
    cur_k: torch.Tensor             # [B, H, L, D]
    cur_v: torch.Tensor
    schedule: SlabSchedule
    softmax_scale: float

    @property
    def target(self) -> int:
        return len(self.sides) - 1

    @property
    def cur_len(self) -> int:
        return self.q.shape[2]

    @property
    def prefix(self) -> int:
        return self.prior_k.shape[2]

    def tables(self):
        return self.schedule.tables[self.target]

    def retained_rows(self) -> List[int]:
        return self.schedule.retained_rows(self.target)

    def attention_flops(self) -> int:
        L, D = self.cur_len, self.q.shape[3]
        return self.batch * sum(4 * L * (r + L) * D for r in self.retained_rows())

    def prior_append_plans(self):
        """``[(scale, plan)]`` that fill the slab from the prior scales, in order."""
        out = []
        for s in range(self.target):
            plan = self.schedule.append_plans.get((s, s + 1))
            if plan is not None and len(plan):
                out.append((s, plan))
        return out


def keep_probability(budget: float, prefix: int, forced_tokens: int) -> float:
    if prefix <= forced_tokens:
        return 1.0
    p = (budget * prefix - forced_tokens) / (prefix - forced_tokens)
    return min(1.0, max(0.0, p))


def removed_from_keep(keep: torch.Tensor, num_scales: int):
    """Static keep mask -> ``removed(target) -> {source: set(heads)}``."""
    H, n_prior = keep.shape
    dropped: Dict[int, Set[int]] = {
        s: {h for h in range(H) if not bool(keep[h, s])} for s in range(n_prior)
    }

    def lookup(target: int):
        return {s: set(dropped[s]) for s in range(min(target, n_prior))}

    return lookup


def schedule_from_keep(keep: torch.Tensor, sides: Sequence[int]) -> SlabSchedule:
    ranges = scale_token_ranges(sides)
    return build_slab_schedule(removed_from_keep(keep, len(sides)), num_heads=keep.shape[0],
                               scale_ranges=ranges, num_scales=len(sides))


def _draw_inputs(gen, B, H, sides, dtype):
    ranges = scale_token_ranges(sides)
    total = ranges[len(sides) - 1][1]
    prefix = ranges[len(sides) - 1][0]
    L = total - prefix
    q = torch.randn((B, H, L, HEAD_DIM), generator=gen, dtype=torch.float32).to(dtype)
    k = torch.randn((B, H, total, HEAD_DIM), generator=gen, dtype=torch.float32).to(dtype)
    v = torch.randn((B, H, total, HEAD_DIM), generator=gen, dtype=torch.float32).to(dtype)
    return q, k[:, :, :prefix].contiguous(), v[:, :, :prefix].contiguous(), \
        k[:, :, prefix:].contiguous(), v[:, :, prefix:].contiguous()


def final_step(*, name: str, batch: int, heads: int, sides=SIDES_1M, budget: float = 0.1,
               seed: int = 1, dtype=torch.bfloat16, softmax_scale: Optional[float] = None,
               forced_scales: int = FORCED_SCALES) -> FinalStepWorkload:
    ranges = scale_token_ranges(sides)
    n_prior = len(sides) - 1
    prefix = ranges[n_prior][0]
    forced_tokens = ranges[min(forced_scales, n_prior) - 1][1] if forced_scales > 0 else 0
    p = keep_probability(budget, prefix, forced_tokens)
    gen = torch.Generator().manual_seed(int(seed))
    u = torch.rand((heads, n_prior), generator=gen, dtype=torch.float64)
    keep = u < p
    keep[:, :forced_scales] = True
    q, pk, pv, ck, cv = _draw_inputs(gen, batch, heads, sides, dtype)
    sched = schedule_from_keep(keep, sides)
    scale = 1.0 / math.sqrt(HEAD_DIM) if softmax_scale is None else float(softmax_scale)
    return FinalStepWorkload(name, batch, heads, tuple(sides), int(seed), float(budget), keep,
                             q, pk, pv, ck, cv, sched, scale)


def with_budget(wl: FinalStepWorkload, budget: float,
                forced_scales: int = FORCED_SCALES) -> FinalStepWorkload:
    """``wl`` (made by :func:`final_step`) at another keep budget: the same
    inputs and the same per-(head, scale) uniforms, thresholded at the new
    keep probability, so the kept sets of increasing budgets are nested."""
    ranges = scale_token_ranges(wl.sides)
    n_prior = len(wl.sides) - 1
    prefix = ranges[n_prior][0]
    forced_tokens = ranges[min(forced_scales, n_prior) - 1][1] if forced_scales > 0 else 0
    p = keep_probability(budget, prefix, forced_tokens)
    gen = torch.Generator().manual_seed(int(wl.seed))
    u = torch.rand((wl.heads, n_prior), generator=gen, dtype=torch.float64)
    keep = u < p
    keep[:, :forced_scales] = True
    return FinalStepWorkload(wl.name, wl.batch, wl.heads, wl.sides, wl.seed, float(budget), keep,
                             wl.q, wl.prior_k, wl.prior_v, wl.cur_k, wl.cur_v,
                             schedule_from_keep(keep, wl.sides), wl.softmax_scale)


def skewed_final_step(*, name: str = "skewed_ragged", batch: int = 16, heads: int = 16,
                      sides=SIDES_1M, seed: int = 3, dtype=torch.bfloat16) -> FinalStepWorkload:
    ranges = scale_token_ranges(sides)
    n_prior = len(sides) - 1
    prefix = ranges[n_prior][0]
    gen = torch.Generator().manual_seed(int(seed))
    u = torch.rand((heads,), generator=gen, dtype=torch.float64)
    keep = torch.zeros((heads, n_prior), dtype=torch.bool)
    sizes = [(ranges[s][1] - ranges[s][0], s) for s in range(n_prior)]
    for h in range(heads):
        want = int(math.floor(math.exp(float(u[h]) * math.log(prefix + 1)))) - 1
        for n, s in sorted(sizes, reverse=True):
            if n <= want:
                keep[h, s] = True
                want -= n
    q, pk, pv, ck, cv = _draw_inputs(gen, batch, heads, sides, dtype)
    sched = schedule_from_keep(keep, sides)
    return FinalStepWorkload(name, batch, heads, tuple(sides), int(seed), None, keep,
                             q, pk, pv, ck, cv, sched, 1.0 / math.sqrt(HEAD_DIM))


def config(n: int, *, dtype=torch.bfloat16, budget: Optional[float] = None) -> FinalStepWorkload:
    """The benchmark shapes by number (1, 2, 4, 5); 3 is the sweep (see ``sweep_layers``)."""
    if n == 1:
        return final_step(name="cpu_plumbing_7scale", batch=2, heads=16, sides=SIDES_7,
                          budget=0.1 if budget is None else budget, seed=0, dtype=dtype)
    if n == 2:
        return final_step(name="2b_final_1024", batch=2, heads=16, sides=SIDES_1M,
                          budget=0.1 if budget is None else budget, seed=1, dtype=dtype)
    if n == 4:
        return final_step(name="8b_class_final_1024", batch=8, heads=32, sides=SIDES_1M,
                          budget=0.1 if budget is None else budget, seed=2, dtype=dtype)
    if n == 5:
        return skewed_final_step(dtype=dtype)
    raise ValueError(f"no final-step workload numbered {n}")


def sweep_keep_policies(layers: int = 32, heads: int = 16, sides=SIDES_1M, budget: float = 0.1,
                        seed0: int = 1000) -> List[torch.Tensor]:
    """Per-layer static keep masks of the 2B generation sweep (seed ``seed0 + layer``)."""
    ranges = scale_token_ranges(sides)
    n_prior = len(sides) - 1
    prefix = ranges[n_prior][0]
    p = keep_probability(budget, prefix, ranges[FORCED_SCALES - 1][1])
    out = []
    for layer in range(layers):
        gen = torch.Generator().manual_seed(seed0 + layer)
        keep = torch.rand((heads, n_prior), generator=gen, dtype=torch.float64) < p
        keep[:, :FORCED_SCALES] = True
        out.append(keep)
    return out


def sweep_step(layer: int, target: int, *, layers: int = 32, batch: int = 2, heads: int = 16,
               sides=SIDES_1M, seed: Optional[int] = None, dtype=torch.bfloat16) -> FinalStepWorkload:
    """Step ``target`` of layer ``layer`` of the generation sweep as a
    workload: the sweep's keep policy and slab schedule (built for the whole
    generation, so its tables and capacity are the ones the sweep's cache
    uses at that step) with fresh N(0, 1) inputs of the scales up to
    ``target`` (seed 3000 + 16 layer + target by default)."""
    keep = sweep_keep_policies(layers=layers, heads=heads, sides=sides)[layer]
    sched = schedule_from_keep(keep, sides)
    seed = 3000 + 16 * layer + target if seed is None else int(seed)
    gen = torch.Generator().manual_seed(seed)
    q, pk, pv, ck, cv = _draw_inputs(gen, batch, heads, tuple(sides[:target + 1]), dtype)
    return FinalStepWorkload(f"sweep_layer{layer}_step{target}", batch, heads, tuple(sides[:target + 1]), seed,
                             0.1, keep, q, pk, pv, ck, cv, sched, 1.0 / math.sqrt(HEAD_DIM))


def build_slab(wl: FinalStepWorkload, device, *, fill: float = float("nan")):
    """Slab K/V of a final-step workload, filled by the HIP pack kernel.

    Appends every prior scale's kept heads in scale order with
    ``pack_flat_segments_kv`` (what the generation loop does step by step).
    Rows no segment owns hold ``fill`` (NaN by default, so a kernel that read
    a dead row would produce NaN).  Returns ``(slab_k, slab_v)`` on ``device``.
    """
    from .real_pruning_fused_attention import pack_flat_segments_kv

    sched = wl.schedule
    B, H, _, D = wl.prior_k.shape
    slab_k = torch.full((B, sched.capacity, D), fill, dtype=wl.prior_k.dtype, device=device)
    slab_v = torch.full((B, sched.capacity, D), fill, dtype=wl.prior_v.dtype, device=device)
    for s, plan in wl.prior_append_plans():
        a, b = sched.scale_ranges[s]
        src_k = wl.prior_k[:, :, a:b].to(device).reshape(B, H * (b - a), D)
        src_v = wl.prior_v[:, :, a:b].to(device).reshape(B, H * (b - a), D)
        dst_starts, src_starts, lengths = sched.device_plan(plan, device, ("append", s))
        pack_flat_segments_kv(dst_k=slab_k, dst_v=slab_v, src_k=src_k, src_v=src_v,
                              dst_starts=dst_starts, src_starts=src_starts, lengths=lengths,
                              max_length=plan.max_length)
    return slab_k, slab_v


def generation_inputs(*, batch: int, heads: int, sides=SIDES_1M, seed: int = 0, dtype=torch.bfloat16,
                      device="cpu", head_dim: int = HEAD_DIM):
    """Per-scale ``(q, k, v)`` ``[B, H, n_s, D]`` of one layer over a whole generation.

    N(0, 1) in fp32 from a seeded generator on ``device``, rounded to ``dtype``.
    """
    gen = torch.Generator(device=device).manual_seed(int(seed))
    out = []
    for side in sides:
        n = int(side) * int(side)
        shape = (batch, heads, n, head_dim)
        q, k, v = (torch.randn(shape, generator=gen, device=device, dtype=torch.float32).to(dtype)
                   for _ in range(3))
        out.append((q, k, v))
    return out


def retained_scales(keep: torch.Tensor, target: int, head: int) -> List[int]:
    """Prior scales whose tokens head ``head`` attends to at ``target`` under a static keep mask."""
    n_prior = keep.shape[1]
    return [s for s in range(min(target, n_prior)) if bool(keep[head, s])]
