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


def _write_pmc(path, rows):
    """rows: (dispatch, kernel, grid, counter, value, duration_ns)."""
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Grid_Size", "Kernel_Name", "Counter_Name",
                                          "Counter_Value", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        for d, name, grid, counter, value, dur in rows:
            w.writerow({"Dispatch_Id": d, "Grid_Size": grid, "Kernel_Name": name,
                        "Counter_Name": counter, "Counter_Value": value,
                        "Start_Timestamp": 1000 * d, "End_Timestamp": 1000 * d + dur})


RED = "void nt::reduce_row_kernel<float, float, nt::SumAcc<float>, 4, 0, true>(...)"


def test_counter_summary_ratios(tmp_path, monkeypatch):
    # one 10-us dispatch at 2.4 GHz: 24,000 cycles; 8 resident waves per CU
    # over the whole kernel = 8 * 256 * 24000 / 4 quad-cycles of SQ_WAVE_CYCLES
    cyc = 10_000 * 2.4
    wc = 8 * 256 * cyc / 4
    s1 = [(1, RED, 131072, "SQ_WAVE_CYCLES", wc, 10_000), (1, RED, 131072, "SQ_WAIT_ANY", 0.5 * wc, 10_000),
          (1, RED, 131072, "SQ_WAIT_INST_ANY", 0.25 * wc, 10_000), (1, RED, 131072, "SQ_WAVES", 2048, 10_000)]
    # VALU busy half the time on every SIMD
    s2 = [(1, RED, 131072, "SQ_ACTIVE_INST_VALU", 0.5 * 1024 * cyc / 4, 10_000),
          (1, RED, 131072, "SQ_INSTS_VALU", 2048 * 100, 10_000)]
    _write_pmc(tmp_path / "p1", s1)
    _write_pmc(tmp_path / "p2", s2)
    (tmp_path / "profiles").mkdir()
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    bench.summarize("red_pmc", [str(tmp_path / "p1"), str(tmp_path / "p2")])
    row = [l for l in open(tmp_path / "profiles" / "reduce_config3_counters.md") if l.startswith("| `reduce")][0]
    cells = [c.strip() for c in row.split("|")]
    # kernel, grid, dispatches, us, waves/CU, wait, issue-wait, LDS-wait, VALU busy, VALU/wave
    assert cells[4:11] == ["10.0", "8.0", "0.50", "0.25", "0.000", "0.50", "100"]


def test_byte_summary_scales_by_the_copy(tmp_path, monkeypatch):
    mib = 1024.0
    f = [(1, COPY, (1 << 24) // 4, "FETCH_SIZE", 32 * mib, 1000), (2, RED, 131072, "FETCH_SIZE", 128 * mib, 1000)]
    w = [(1, COPY, (1 << 24) // 4, "WRITE_SIZE", 64 * mib, 1000), (2, RED, 131072, "WRITE_SIZE", 0.0, 1000)]
    _write_pmc(tmp_path / "f", f)
    _write_pmc(tmp_path / "w", w)
    (tmp_path / "profiles").mkdir()
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    bench.summarize("red_bytes", [str(tmp_path / "f"), str(tmp_path / "w")])
    rows = [l for l in open(tmp_path / "profiles" / "reduce_config3_hbm_traffic.md") if l.startswith("| `")]
    assert len(rows) == 1  # the calibration copy itself is not listed
    cells = [c.strip() for c in rows[0].split("|")]
    assert cells[4:6] == ["256.0", "0.0"]  # a 256 MiB read-only reduction


def test_next_rows_summary_assigns_dispatches_to_cases(tmp_path, monkeypatch):
    # Several next-row cases share one kernel and grid size (the transposed
    # copies), so the summary walks the trace in queue order: set-up copies
    # first, barrier and runtime copy kernels interleaved, then each case's
    # 1 + NEXT_ITERS calls (the uniform draw four kernels per call), the
    # first call of each untimed.
    path = tmp_path / "prof_next"
    path.mkdir()
    rows, t = [], 0

    def emit(name, us):
        nonlocal t
        rows.append({"Dispatch_Id": len(rows), "Kernel_Name": name,
                     "Start_Timestamp": t, "End_Timestamp": t + int(us * 1000)})
        t += int(us * 1000) + 500

    emit("void nt::ew_flat_kernel<float, float, 1, 1, 4, 1, true, nt::CastOp<float, float> >(...)", 5)
    want = {}
    for ci, (name, pat, per_call, _, _) in enumerate(bench.NEXT_ROWS):
        for c in range(1 + bench.NEXT_ITERS):
            if c == 3:
                emit("void nt::stream_fence_kernel()", 2)
            if ci == len(bench.NEXT_ROWS) - 1 and c == 0:
                emit("__amd_rocclr_copyBuffer", 4)
            for k in range(per_call):
                # the untimed first call is slow; timed calls take 10 + case index us
                emit(f"void nt::{pat}kernel_{k}(...)", 99.0 if c == 0 else 10.0 + ci)
        want[name] = per_call * (10.0 + ci)
    with open(path / "run_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    (tmp_path / "profiles").mkdir()
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    bench.summarize("next", [str(path)])
    text = open(tmp_path / "profiles" / "next_rows_trace.md").read()
    got = {}
    for line in text.splitlines():
        if line.startswith("| ") and "`" in line:
            cells = [c.strip() for c in line.replace("\\|", "/").split(" | ")]
            got[cells[0].lstrip("| ").replace("/", "|")] = (int(cells[2]), float(cells[3]))
    assert got == {n: (bench.NEXT_ITERS, us) for n, us in want.items()}
    # a trace whose dispatches do not follow the cases is refused
    rows[5]["Kernel_Name"] = "void nt::something_else(...)"
    with open(path / "run_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    try:
        bench.summarize("next", [str(path)])
    except SystemExit as e:
        assert "not" in str(e)
    else:
        raise AssertionError("a mismatched trace was summarised")
