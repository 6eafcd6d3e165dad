"""Phase profiler of the fused segmented path (materialize / attention / compact).

Same API and record layout as the reference's module-level profiler
(enable_real_pruning_fast.py:30-164): host time with ``perf_counter_ns``,
device time with a pair of HIP events per phase whose end event is
synchronized (so a profiled run serializes each phase, as the reference's
does), call counts, and byte / slot counters of the slab copies.
"""

from __future__ import annotations

import time
from typing import Optional

import torch

PHASES = frozenset({"materialize", "attention", "compact"})

_enabled = False
_cpu_ns: dict = {}
_gpu_ms: dict = {}
_calls: dict = {}
_stats: dict = {}


def reset_real_pruning_fast_phase_profile() -> None:
    """Clear every record (enable_real_pruning_fast.py:38-42)."""
    _cpu_ns.clear()
    _gpu_ms.clear()
    _calls.clear()
    _stats.clear()


def set_real_pruning_fast_phase_profile_enabled(enabled: bool = True) -> None:
    """Turn profiling on or off and clear the records (:45-48)."""
    global _enabled
    _enabled = bool(enabled)
    reset_real_pruning_fast_phase_profile()


def phase_profile_enabled() -> bool:
    return _enabled


def snapshot_real_pruning_fast_phase_profile(*, reset: bool = False) -> dict:
    """``{"cpu_ms", "cuda_ms", "calls", "segmented_flat_stats"}`` (:51-60)."""
    out = {
        "cpu_ms": {k: v / 1e6 for k, v in _cpu_ns.items()},
        "cuda_ms": dict(_gpu_ms),
        "calls": dict(_calls),
        "segmented_flat_stats": dict(_stats),
    }
    if reset:
        reset_real_pruning_fast_phase_profile()
    return out


class phase:
    """``with phase("attention"): ...`` records one call of a phase when profiling is on."""

    __slots__ = ("name", "t0", "e0", "e1")

    def __init__(self, name: str):
        self.name = name
        self.t0 = 0
        self.e0: Optional[torch.cuda.Event] = None
        self.e1: Optional[torch.cuda.Event] = None

    def __enter__(self):
        if not _enabled or self.name not in PHASES:
            return self
        if torch.cuda.is_available():
            self.e0 = torch.cuda.Event(enable_timing=True)
            self.e1 = torch.cuda.Event(enable_timing=True)
            self.e0.record()
        self.t0 = time.perf_counter_ns()
        return self

    def __exit__(self, *exc):
        if not _enabled or self.name not in PHASES or self.t0 == 0:
            return False
        _cpu_ns[self.name] = _cpu_ns.get(self.name, 0) + (time.perf_counter_ns() - self.t0)
        _calls[self.name] = _calls.get(self.name, 0) + 1
        if self.e0 is not None:
            self.e1.record()
            self.e1.synchronize()
            _gpu_ms[self.name] = _gpu_ms.get(self.name, 0.0) + float(self.e0.elapsed_time(self.e1))
        return False


def stat_add(name: str, value=1) -> None:
    """Add to a counter (:102-106)."""
    if _enabled:
        _stats[name] = _stats.get(name, 0) + value


def record_kv_copy(prefix: str, *, slots: int, k_tensor: torch.Tensor, v_tensor: torch.Tensor) -> None:
    """``<prefix>_slots`` and ``<prefix>_bytes`` of a K/V row copy (:117-164)."""
    if not _enabled:
        return
    slots = int(slots)
    stat_add(f"{prefix}_slots", slots)
    per_row = int(k_tensor.shape[0]) * int(k_tensor.shape[-1]) * (k_tensor.element_size() + v_tensor.element_size())
    stat_add(f"{prefix}_bytes", slots * per_row if slots > 0 else 0)
