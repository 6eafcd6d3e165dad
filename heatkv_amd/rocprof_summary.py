"""Summaries of rocprofv3 CSV output for the kernels of this package.

Three reports, each written as a short text/JSON file under ``profiles/``:

* ``stats``   -- the ``*_kernel_stats.csv`` of a ``--kernel-trace --stats`` run
  as a markdown table (calls, average / min / max duration per kernel).
* ``traffic`` -- HBM bytes per dispatch of one kernel from two ``--pmc`` runs
  (``FETCH_SIZE``, then ``WRITE_SIZE``; both in KiB per dispatch).  Each
  counter is scaled by what it reads for a plain device copy of known size
  in the same run (``bench.py --copy-calib-mib N`` launches it): the copy
  moves N MiB each way, so ``factor = N MiB / counter(copy)``.
* ``counters`` -- mean per-dispatch values of any other ``--pmc`` counters.
* ``group``   -- a kernel launched as a fixed group of dispatches (e.g. the
  12 append launches of one slab fill): summed duration (``--kernel-trace``
  CSV) and calibrated HBM bytes (as in ``traffic``) per group, against the
  group's algorithmic bytes.

Usage::

    python -m heatkv_amd.rocprof_summary stats KT_DIR --out profiles/x.md --cmd "..."
    python -m heatkv_amd.rocprof_summary traffic --fetch F.csv --write W.csv \\
        --kernel seg_attn_direct --calib-mib 512 --out profiles/x.json --cmd "..."
    python -m heatkv_amd.rocprof_summary counters C.csv [C2.csv ...] --kernel seg_attn_direct \\
        --out profiles/x.md --cmd "..."
    python -m heatkv_amd.rocprof_summary group --trace KT_DIR --fetch F.csv --write W.csv \\
        --kernel pack_kernel --group 12 --algo-bytes N --calib-mib 512 --out profiles/x.json --cmd "..."
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import statistics
from collections import defaultdict
from typing import Dict, List

COPY_KERNEL = "__amd_rocclr_copyBuffer"


def _rows(path: str) -> List[dict]:
    with open(path, newline="") as fh:
        return list(csv.DictReader(fh))


def per_dispatch(path: str, kernel_substr: str) -> Dict[str, List[float]]:
    """``{counter: [value per dispatch]}`` of the dispatches whose name contains ``kernel_substr``."""
    out: Dict[str, List[float]] = defaultdict(list)
    for r in _rows(path):
        if kernel_substr in r["Kernel_Name"]:
            out[r["Counter_Name"]].append(float(r["Counter_Value"]))
    return dict(out)


def window_durations(kt_dir: str, kernel_substr: str) -> List[float]:
    """Durations (us) of every dispatch of ``kernel_substr`` in dispatch order
    (the ``*kernel_trace.csv`` of a ``--kernel-trace`` run)."""
    paths = glob.glob(os.path.join(kt_dir, "**", "*kernel_trace.csv"), recursive=True)
    if not paths:
        raise FileNotFoundError(f"no *kernel_trace.csv under {kt_dir}")
    rows = [r for r in _rows(paths[0]) if kernel_substr in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    return [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in rows]


def stats_markdown(kt_dir: str, cmd: str, window_kernel: str = "", window: int = 0) -> str:
    paths = glob.glob(os.path.join(kt_dir, "**", "*kernel_stats.csv"), recursive=True)
    if not paths:
        raise FileNotFoundError(f"no *kernel_stats.csv under {kt_dir}")
    lines = [
        "# rocprofv3 kernel-trace statistics",
        "",
        f"Command: `{cmd}`",
        "",
    ]
    if window_kernel and window > 0:
        d = window_durations(kt_dir, window_kernel)
        lines += [
            f"`{window_kernel}` dispatches (all of the run, and its last {window}):",
            "",
            "| dispatches | mean us | median us | min us | max us |",
            "|---|---:|---:|---:|---:|",
        ]
        for label, xs in ((f"all {len(d)}", d), (f"last {window}", d[-window:])):
            lines.append(f"| {label} | {statistics.mean(xs):.2f} | {statistics.median(xs):.2f} | "
                         f"{min(xs):.2f} | {max(xs):.2f} |")
        lines.append("")
    lines += [
        "| kernel | calls | avg us | min us | max us | share % |",
        "|---|---:|---:|---:|---:|---:|",
    ]
    for r in _rows(paths[0]):
        name = r["Name"]
        if len(name) > 110:
            name = name[:107] + "..."
        lines.append(
            f"| `{name}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
            f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.2f} |"
        )
    return "\n".join(lines) + "\n"


def traffic(fetch_csv: str, write_csv: str, kernel_substr: str, calib_mib: int, cmd: str) -> dict:
    """Calibrated HBM read / write bytes per dispatch of ``kernel_substr``."""
    calib_kib = calib_mib * 1024.0
    res = {"kernel": kernel_substr, "calibration_copy_mib": calib_mib, "command": cmd}
    for label, path, counter in (("read", fetch_csv, "FETCH_SIZE"), ("write", write_csv, "WRITE_SIZE")):
        kern = per_dispatch(path, kernel_substr).get(counter, [])
        copy = per_dispatch(path, COPY_KERNEL).get(counter, [])
        if not kern or not copy:
            raise ValueError(f"{path}: no {counter} values for {kernel_substr!r} or the copy kernel")
        copy_kib = max(copy)  # the calibration copies are the largest copyBuffer dispatches
        factor = calib_kib / copy_kib
        mean_kib = statistics.mean(kern)
        res[f"{counter}_kib_per_dispatch"] = round(mean_kib, 3)
        res[f"{counter}_copy_kib"] = round(copy_kib, 3)
        res[f"{label}_factor"] = round(factor, 4)
        res[f"{label}_bytes"] = int(round(mean_kib * factor * 1024.0))
        res[f"{label}_dispatches"] = len(kern)
    res["bytes_per_dispatch"] = res["read_bytes"] + res["write_bytes"]
    return res


def group_summary(trace_dir: str, fetch_csv: str, write_csv: str, kernel_substr: str, group: int,
                  algo_bytes: int, calib_mib: int, cmd: str) -> dict:
    """Per group of ``group`` dispatches of ``kernel_substr``: summed kernel
    time, calibrated HBM bytes, and the bandwidth of the algorithmic bytes."""
    paths = glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True)
    if not paths:
        raise FileNotFoundError(f"no *kernel_trace.csv under {trace_dir}")
    durs = [int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
            for r in _rows(paths[0]) if kernel_substr in r["Kernel_Name"]]
    if len(durs) < group or len(durs) % group:
        raise ValueError(f"{len(durs)} dispatches of {kernel_substr!r} do not form groups of {group}")
    groups = len(durs) // group
    ns = sum(durs) / groups
    t = traffic(fetch_csv, write_csv, kernel_substr, calib_mib, cmd)
    hbm = t["bytes_per_dispatch"] * group
    return {"kernel": kernel_substr, "command": cmd, "dispatches_per_group": group, "groups": groups,
            "kernel_us_per_group": round(ns / 1e3, 2), "algorithmic_bytes_per_group": int(algo_bytes),
            "achieved_GBps": round(algo_bytes / ns, 1), "hbm_bytes_per_group": int(hbm),
            "hbm_over_algorithmic": round(hbm / algo_bytes, 4), "read_factor": t["read_factor"],
            "write_factor": t["write_factor"]}


def counters_markdown(paths: List[str], kernel_substr: str, cmd: str, mean_us: float = 0.0) -> str:
    vals: Dict[str, List[float]] = {}
    for p in paths:
        vals.update(per_dispatch(p, kernel_substr))
    lines = [
        f"# rocprofv3 counters: `{kernel_substr}` (mean per dispatch)",
        "",
        f"Command: `{cmd}`",
        "",
        "| counter | value | dispatches |",
        "|---|---:|---:|",
    ]
    for k in sorted(vals):
        lines.append(f"| {k} | {statistics.mean(vals[k]):.0f} | {len(vals[k])} |")
    m = {k: statistics.mean(v) for k, v in vals.items()}
    derived = []
    if "GRBM_GUI_ACTIVE" in m:
        # GRBM_GUI_ACTIVE counts the 8 XCDs; SQ cycle counters sum the 1024 SIMDs
        cycles = m["GRBM_GUI_ACTIVE"] / 8.0
        derived.append(f"cycles per dispatch {cycles:.0f}")
        if mean_us:
            derived.append(f"clock under load {cycles / (mean_us * 1e3):.2f} GHz over a {mean_us:.2f} us mean dispatch")
        if "SQ_VALU_MFMA_BUSY_CYCLES" in m:
            derived.append(f"MFMA busy per SIMD {m['SQ_VALU_MFMA_BUSY_CYCLES'] / 1024.0 / cycles:.3f}")
    if "SQ_VALU_MFMA_BUSY_CYCLES" in m and "SQ_VALU_MFMA_COEXEC_CYCLES" in m:
        derived.append("VALU co-executing with MFMA: "
                       f"{m['SQ_VALU_MFMA_COEXEC_CYCLES'] / m['SQ_VALU_MFMA_BUSY_CYCLES']:.3f} of MFMA busy cycles")
    if "SQ_INSTS_MFMA" in m and m["SQ_INSTS_MFMA"] > 0:
        n = m["SQ_INSTS_MFMA"]
        if "SQ_INSTS_VALU" in m:
            trans = m.get("SQ_INSTS_VALU_TRANS_F32", 0.0)
            derived.append(f"non-MFMA VALU instructions per MFMA {(m['SQ_INSTS_VALU'] - n) / n:.2f} "
                           f"(of them transcendental {trans / n:.2f})")
        for key, label in (("SQ_INSTS_LDS", "LDS"), ("SQ_INSTS_SALU", "SALU")):
            if key in m:
                derived.append(f"{label} instructions per MFMA {m[key] / n:.2f}")
    if "SQ_WAIT_ANY" in m and "SQ_WAVE_CYCLES" in m:
        derived.append(f"SQ_WAIT_ANY / SQ_WAVE_CYCLES {m['SQ_WAIT_ANY'] / m['SQ_WAVE_CYCLES']:.3f}")
    if derived:
        lines += ["", "Derived:", ""] + [f"* {x}" for x in derived]
    return "\n".join(lines) + "\n"


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="what", required=True)
    a = sub.add_parser("stats")
    a.add_argument("kt_dir")
    a.add_argument("--out", required=True)
    a.add_argument("--cmd", required=True)
    a.add_argument("--window-kernel", default="", help="also the last --window dispatches of this kernel")
    a.add_argument("--window", type=int, default=0)
    b = sub.add_parser("traffic")
    b.add_argument("--fetch", required=True)
    b.add_argument("--write", required=True)
    b.add_argument("--kernel", required=True)
    b.add_argument("--calib-mib", type=int, required=True)
    b.add_argument("--out", required=True)
    b.add_argument("--cmd", required=True)
    c = sub.add_parser("counters")
    c.add_argument("csv", nargs="+")
    c.add_argument("--kernel", required=True)
    c.add_argument("--out", required=True)
    c.add_argument("--cmd", required=True)
    c.add_argument("--mean-us", type=float, default=0.0, help="the kernel's mean dispatch time (for the clock)")
    d = sub.add_parser("group")
    d.add_argument("--trace", required=True)
    d.add_argument("--fetch", required=True)
    d.add_argument("--write", required=True)
    d.add_argument("--kernel", required=True)
    d.add_argument("--group", type=int, required=True)
    d.add_argument("--algo-bytes", type=int, required=True)
    d.add_argument("--calib-mib", type=int, required=True)
    d.add_argument("--out", required=True)
    d.add_argument("--cmd", required=True)
    args = ap.parse_args(argv)
    if args.what == "stats":
        text = stats_markdown(args.kt_dir, args.cmd, args.window_kernel, args.window)
    elif args.what == "group":
        text = json.dumps(group_summary(args.trace, args.fetch, args.write, args.kernel, args.group,
                                        args.algo_bytes, args.calib_mib, args.cmd), indent=1) + "\n"
    elif args.what == "traffic":
        text = json.dumps(traffic(args.fetch, args.write, args.kernel, args.calib_mib, args.cmd), indent=1) + "\n"
    else:
        text = counters_markdown(args.csv, args.kernel, args.cmd, args.mean_us)
    os.makedirs(os.path.dirname(os.path.abspath(args.out)), exist_ok=True)
    with open(args.out, "w") as fh:
        fh.write(text)
    print(text)


if __name__ == "__main__":
    main()
