"""Writes tests/golden/slab_2b.json: the reference's static slot schedule
(slab offsets and capacity, and digests of its offset tables and copy
descriptors) under the HeatKV policy's progressive removal, for the parity
test of heatkv_amd/slab_schedule.py.

Run in the build container only (it reads the reference from
/root/reference; nothing here runs on the GPU host):

    python tests/golden/make_slab_golden.py

The allocator is ``_segmented_flat_build_static_slot_schedule``
(enable_real_pruning_fast.py:260-558) with its helpers
``_segmented_flat_cache_capacity_for_layer`` (:206-234),
``_segmented_flat_static_schedule_allow_overalloc`` (:242-250) and
``_segmented_flat_merge_free_blocks`` (:1033-1047).  Its module imports the
Infinity model code (infinity.models.basic, which needs timm and flash_attn,
absent here), so only these four functions are compiled from the module's
text and run, with the names they use (os, torch, typing); nothing else of
the module runs.  The policy is the reference's own: tools/utils.py
(strict_pruning_schedule_for_budget_scale_specific,
strict_removed_heads_by_scale_specific_for_budget) and enable_pruning.py
(ScaleSpecificPruningController, which carries the 1M scale schedule and its
token ranges), on the reference's orders/2b.json (orders_2b.json here).
"""

from __future__ import annotations

import ast
import hashlib
import json
import os
import sys
import typing

import numpy as np
import torch

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))
FUNCTIONS = (
    "_segmented_flat_cache_capacity_for_layer",
    "_segmented_flat_static_schedule_allow_overalloc",
    "_segmented_flat_merge_free_blocks",
    "_segmented_flat_build_static_slot_schedule",
)


class _Layer:
    """An attention layer as the reference's validators see it (num_heads)."""

    def __init__(self, num_heads):
        self.num_heads = num_heads


def digest(*arrays) -> str:
    """First 16 hex digits of the SHA-256 of the arrays' shapes and int64 values."""
    h = hashlib.sha256()
    for a in arrays:
        a = np.asarray(a, dtype=np.int64)
        h.update(np.asarray(a.shape, dtype=np.int64).tobytes())
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()[:16]


def runs_digest(runs, sequence_len) -> str:
    """Digest of a copy-run list flattened to (dst_start, src_start, length) items in order."""
    items = [(it["dst_start"], it["src_start"], it["length"]) for r in runs for it in r["copy_items"]]
    return digest(np.asarray(items, dtype=np.int64).reshape(-1, 3), [sequence_len])


def reference_allocator():
    path = os.path.join(REF, "enable_real_pruning_fast.py")
    tree = ast.parse(open(path).read(), filename=path)
    defs = [n for n in tree.body if isinstance(n, ast.FunctionDef) and n.name in FUNCTIONS]
    if sorted(n.name for n in defs) != sorted(FUNCTIONS):
        raise RuntimeError(f"expected {FUNCTIONS} in {path}")
    code = compile(ast.Module(body=defs, type_ignores=[]), path, "exec",
                   flags=__import__("__future__").annotations.compiler_flag, dont_inherit=True)
    ns = {"os": os, "torch": torch, "Mapping": typing.Mapping, "Optional": typing.Optional}
    exec(code, ns)
    return ns["_segmented_flat_build_static_slot_schedule"]


def main():
    sys.path.insert(0, REF)
    from tools import utils as U  # noqa: E402
    import enable_pruning as P  # noqa: E402

    build = reference_allocator()
    orders = json.load(open(os.path.join(HERE, "orders_2b.json")))
    L, H, start = 32, 16, 3
    out = {"num_layers": L, "num_heads": H, "source_scale_start": start, "budgets": {}}
    layers = [_Layer(H) for _ in range(L)]
    for budget in (0.1, 0.35):
        sched = U.strict_pruning_schedule_for_budget_scale_specific(
            budget, orders, num_layers=L, num_heads=H, source_scale_start=start, protected_prefix_scales=start)
        view = U.strict_removed_heads_by_scale_specific_for_budget(
            budget, orders, num_layers=L, num_heads=H, source_scale_start=start, protected_prefix_scales=start,
            strict_schedule=sched)
        table = P._validate_and_normalize_removed_heads_by_scale_specific(
            view["removed_heads_by_scale"], layers, source_scale_start=start)
        ctrl = P.ScaleSpecificPruningController(num_layers=L, num_heads=H, static_removed_heads_by_scale=table,
                                                source_scale_start=start)
        per_layer = []
        for layer in range(L):
            res = build(ctrl, layer_idx=layer, num_heads=H)
            assert res["enabled"]
            # one row per (source scale, head) segment: source, head, end target, offset
            segs = sorted((int(s["source_scale"]), int(s["head"]), int(s["end_target"]), int(s["offset"]))
                          for s in res["segments"])
            # per-target offset tables (starts, ends, counts) and copy runs
            # (activation from the dense prefix of each target, append of
            # each scale for the next), as digests of their exact values
            tables = {str(t): digest(*(x.numpy() for x in res["metadata_cpu_by_target"][t]))
                      for t in sorted(res["metadata_cpu_by_target"])}
            activation = {str(t): runs_digest(runs, res["old_pack_cache_lens_by_target"][t])
                          for t, runs in sorted(res["old_pack_runs_by_target"].items())}
            append = {str(s): runs_digest(runs, runs[0]["sequence_len"] if runs else 0)
                      for (s, _), runs in sorted(res["append_runs_by_key"].items())}
            per_layer.append({"capacity": int(res["capacity"]), "capacity_bound": int(res["capacity_bound"]),
                              "segments": [list(s) for s in segs], "tables": tables, "activation": activation,
                              "append": append})
        out["budgets"][str(budget)] = per_layer
    with open(os.path.join(HERE, "slab_2b.json"), "w") as fh:
        json.dump(out, fh, separators=(",", ":"), sort_keys=True)
    print("wrote", os.path.join(HERE, "slab_2b.json"))


if __name__ == "__main__":
    main()
