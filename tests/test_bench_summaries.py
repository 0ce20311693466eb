"""bench.py's traffic summary (host logic, no GPU): HBM bytes per launch come
from FETCH_SIZE / WRITE_SIZE readings scaled by what a plain 2^24-element
fp32 copy reads.  The same copy kernel also runs at 2^26 elements (the
cold-copy reference) in the profiled command, so the calibration must take
only the 2^24 dispatches, told apart by their grid size."""

from __future__ import annotations

import csv
import json
import os

import bench

COPY = "void nt::ew_flat_kernel<float, float, 1, 1, 4, 2, true, nt::CastOp<float, float> >(...)"
MUL_T = ("void nt::ew_tile4_kernel<float, float, 5, 2, true, "
         "nt::BinaryBwd<2, float, true, true, true, true> >(...)")


def _write(path, counter, rows):
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Grid_Size", "Kernel_Name",
                                          "Counter_Name", "Counter_Value"])
        w.writeheader()
        for i, (name, grid, value) in enumerate(rows):
            w.writerow({"Dispatch_Id": i, "Grid_Size": grid, "Kernel_Name": name,
                        "Counter_Name": counter, "Counter_Value": value})


def test_traffic_calibrates_on_the_small_copies(tmp_path, monkeypatch):
    # Readings shaped like MI355X's: FETCH_SIZE counts half of a stream's
    # reads, WRITE_SIZE all of its writes.  The 2^26 copies read 4x more.
    small, big = (1 << 24) // 8, (1 << 26) // 8
    mib = 1024.0  # one MiB in the counters' KiB
    fetch = [(COPY, small, 32 * mib)] * 3 + [(COPY, big, 128 * mib)] * 9 \
        + [(MUL_T, 4096 * 256, 5 * 32 * mib)]
    write = [(COPY, small, 64 * mib)] * 3 + [(COPY, big, 256 * mib)] * 9 \
        + [(MUL_T, 4096 * 256, 2 * 64 * mib)]
    _write(tmp_path / "fetch", "FETCH_SIZE", fetch)
    _write(tmp_path / "write", "WRITE_SIZE", write)
    (tmp_path / "profiles").mkdir()
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    bench.summarize("traffic", [str(tmp_path / "fetch"), str(tmp_path / "write")])
    t = json.load(open(tmp_path / "profiles" / "traffic.json"))
    assert t["fetch_scale"] == 2.0 and t["write_scale"] == 1.0
    # 5 operands read and 2 written, 64 MiB each: the algorithmic 28 B/element
    assert t["per_launch_bytes"] == {"mul|transposed|bwd": bench.ew_bytes("mul", "bwd")}
    assert bench.ew_bytes("mul", "bwd") == 7 * 64 * 1024 * 1024
