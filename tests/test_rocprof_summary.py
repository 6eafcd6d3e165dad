"""rocprofv3 CSV summaries (heatkv_amd.rocprof_summary) on small synthetic files."""

from __future__ import annotations

import csv
import json
import os

import pytest

from heatkv_amd import rocprof_summary as rs


def _write(path, header, rows):
    with open(path, "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(header)
        w.writerows(rows)


def _pmc(path, counter, values):
    """Counter rows: the kernel's dispatches, then one 512 MiB calibration copy."""
    rows = [["pack_kernel<U16B>", counter, v] for v in values]
    rows.append([rs.COPY_KERNEL, counter, {"FETCH_SIZE": 262144.0, "WRITE_SIZE": 524288.0}[counter]])
    _write(path, ["Kernel_Name", "Counter_Name", "Counter_Value"], rows)


def test_traffic_scales_by_the_copy(tmp_path):
    f, w = tmp_path / "f.csv", tmp_path / "w.csv"
    _pmc(f, "FETCH_SIZE", [100.0, 300.0])  # copy reads 262144 KiB for 512 MiB: factor 2
    _pmc(w, "WRITE_SIZE", [50.0, 50.0])    # factor 1
    t = rs.traffic(str(f), str(w), "pack_kernel", 512, "cmd")
    assert t["read_factor"] == 2.0 and t["write_factor"] == 1.0
    assert t["read_bytes"] == 200 * 2 * 1024 and t["write_bytes"] == 50 * 1024
    assert t["bytes_per_dispatch"] == 200 * 2 * 1024 + 50 * 1024


def test_group_summary(tmp_path):
    kt = tmp_path / "kt"
    os.makedirs(kt / "host")
    rows = []
    t0 = 1000
    for g in range(2):          # two groups of three dispatches: 1 + 2 + 3 us each
        for d in (1000, 2000, 3000):
            rows.append(["pack_kernel<U16B>", t0, t0 + d])
            t0 += d + 500
        rows.append(["other_kernel", t0, t0 + 7777])
        t0 += 8000
    _write(kt / "host" / "x_kernel_trace.csv", ["Kernel_Name", "Start_Timestamp", "End_Timestamp"], rows)
    f, w = tmp_path / "f.csv", tmp_path / "w.csv"
    _pmc(f, "FETCH_SIZE", [10.0] * 6)
    _pmc(w, "WRITE_SIZE", [20.0] * 6)
    out = rs.group_summary(str(kt), str(f), str(w), "pack_kernel", 3, 60000, 512, "cmd")
    assert out["groups"] == 2 and out["kernel_us_per_group"] == 6.0
    assert out["achieved_GBps"] == 10.0  # 60000 B in 6000 ns
    assert out["hbm_bytes_per_group"] == 3 * (10 * 2 + 20) * 1024
    with pytest.raises(ValueError):
        rs.group_summary(str(kt), str(f), str(w), "pack_kernel", 4, 1, 512, "cmd")
    out_path = tmp_path / "g.json"
    rs.main(["group", "--trace", str(kt), "--fetch", str(f), "--write", str(w), "--kernel", "pack_kernel",
             "--group", "3", "--algo-bytes", "60000", "--calib-mib", "512", "--out", str(out_path),
             "--cmd", "c"])
    assert json.loads(out_path.read_text())["groups"] == 2
