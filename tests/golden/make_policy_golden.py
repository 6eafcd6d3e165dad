"""Writes tests/golden/policy_2b.json: input/output vectors of the reference's
HeatKV policy functions, for the parity tests of heatkv_amd/policy.py.

Run in the build container only (it imports the reference from
/root/reference; nothing here runs on the GPU host):

    python tests/golden/make_policy_golden.py

Imports tools/utils.py (pruned_heads_for_budget :235-305,
strict_pruning_schedule_for_budget_scale_specific :308-522,
strict_removed_heads_by_scale_specific_for_budget :525-597) and
enable_pruning.py (ScaleSpecificPruningController :328-401,
_validate_and_normalize_removed_heads_by_scale_specific :115-179).  The
removal orders are the reference's data file orders/2b.json (source scales
3..11, 16 heads x 32 layers), copied next to this script as orders_2b.json.
"""

from __future__ import annotations

import json
import os
import sys

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))


class _Layer:
    """An attention layer as the reference's validators see it (num_heads)."""

    def __init__(self, num_heads):
        self.num_heads = num_heads


def _mask(heads_by_layer, num_layers, num_heads):
    """Removed heads of every layer as one hex bit mask (bit layer * H + head)."""
    bits = 0
    for layer in range(num_layers):
        for h in heads_by_layer.get(layer, ()):
            bits |= 1 << (layer * num_heads + int(h))
    return format(bits, "x")


def main():
    sys.path.insert(0, REF)
    from tools import utils as U  # noqa: E402
    import enable_pruning as P  # noqa: E402

    with open(os.path.join(REF, "orders", "2b.json")) as fh:
        orders = json.load(fh)
    with open(os.path.join(HERE, "orders_2b.json"), "w") as fh:
        json.dump(orders, fh, separators=(",", ":"))

    L, H, start = 32, 16, 3
    out = {"num_layers": L, "num_heads": H, "source_scale_start": start, "pruned_heads": {}, "strict": {}}

    for budget in (0.05, 0.1, 0.2, 0.5, 1.0):
        for retained in (21, 51):
            for skip in (True, False):
                try:
                    res = U.pruned_heads_for_budget(budget, retained_tokens=retained, num_layers=L,
                                                    num_heads=H, skip_last_scale=skip)
                    val = {str(k): int(v) for k, v in res.items()}
                except ValueError as e:
                    val = {"error": str(e)}
                out["pruned_heads"][f"{budget}/{retained}/{int(skip)}"] = val

    layers = [_Layer(H) for _ in range(L)]
    for budget in (0.1, 0.2, 0.35):
        sched = U.strict_pruning_schedule_for_budget_scale_specific(
            budget, orders, num_layers=L, num_heads=H, source_scale_start=start, protected_prefix_scales=start)
        view = U.strict_removed_heads_by_scale_specific_for_budget(
            budget, orders, num_layers=L, num_heads=H, source_scale_start=start, protected_prefix_scales=start,
            strict_schedule=sched)
        table = P._validate_and_normalize_removed_heads_by_scale_specific(
            view["removed_heads_by_scale"], layers, source_scale_start=start)
        ctrl = P.ScaleSpecificPruningController(num_layers=L, num_heads=H, static_removed_heads_by_scale=table,
                                                source_scale_start=start)
        rec = {
            "final_removed_counts": {str(t): int(n) for t, n in sched["final_removed_counts"].items()},
            "early_activation": {
                str(t): {str(l): [[int(v) for v in a] for a in atoms] for l, atoms in m.items()}
                for t, m in sched["early_activation_by_scale"].items()},
            "removed_counts_by_scale": {str(t): int(n) for t, n in view["removed_counts_by_scale"].items()},
            "remaining_atoms_by_scale": {str(t): int(n) for t, n in view["remaining_atoms_by_scale"].items()},
            # controller lookup: removed heads per (target, source) as masks over (layer, head)
            "removed_mask": {
                str(t): {str(s): _mask({l: ctrl.removed_heads_for(l, t, s) for l in range(L)}, L, H)
                         for s in range(start, 12)}
                for t in range(13)},
        }
        out["strict"][str(budget)] = rec

    with open(os.path.join(HERE, "policy_2b.json"), "w") as fh:
        json.dump(out, fh, separators=(",", ":"), sort_keys=True)
    print("wrote", os.path.join(HERE, "policy_2b.json"))


if __name__ == "__main__":
    main()
