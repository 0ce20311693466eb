"""The launch window that lets independent elementwise kernels skip the
stream's barrier (nanotorch_amd/csrc/launch_window.h), on the CPU:
tests/cpp/launch_window_test.cpp feeds it random kernels with random byte
ranges and closes, models the command processor's ordering (a barrier launch
waits for everything before it; a launch without the barrier may run
alongside every kernel back to the last barrier launch) and checks that no
two kernels that may run together touch the same bytes unless both only
read them, and that every barrier the window asks for has a reason."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_launch_window_orders_every_hazard(tmp_path):
    exe = tmp_path / "launch_window_test"
    subprocess.run(["g++", "-std=c++20", "-O1", "-g", "-fsanitize=address,undefined",
                    "-I", os.path.join(ROOT, "nanotorch_amd", "csrc"),
                    os.path.join(ROOT, "tests", "cpp", "launch_window_test.cpp"), "-o", str(exe)],
                   check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "errors=0" in res.stdout, res.stdout
