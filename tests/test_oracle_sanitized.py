"""The oracle's C++ under AddressSanitizer and UndefinedBehaviorSanitizer
(host code only, no GPU).

oracle/nt_oracle.cpp is compiled with the committed Makefile's flags plus
-fsanitize=address,undefined into a temporary library, and the oracle's own
pinning tests (tests/test_oracle_pinning.py: known answers, closed forms,
planted mistakes, the OpenMP matmul) run against it in a child process with
the sanitizer runtimes preloaded.  An out-of-bounds access, use after free or
undefined arithmetic in the oracle fails the test instead of silently
corrupting the values every GPU parity test is checked against."""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _runtime(name: str) -> str:
    path = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True,
                          text=True, check=True).stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else ""


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_oracle_under_asan_ubsan(tmp_path):
    asan, ubsan = _runtime("libasan.so"), _runtime("libubsan.so")
    if not asan or not ubsan:
        pytest.skip("sanitizer runtimes not installed")
    so = tmp_path / "libnt_oracle_san.so"
    subprocess.run(["g++", "-O1", "-g", "-std=c++20", "-fPIC", "-march=x86-64", "-ffp-contract=off",
                    "-fno-fast-math", "-fopenmp", "-fsanitize=address,undefined",
                    "-fno-sanitize-recover=undefined", "-shared", "-o", str(so),
                    os.path.join(ROOT, "oracle", "nt_oracle.cpp")], check=True)
    env = dict(os.environ, NT_ORACLE_LIB=str(so), LD_PRELOAD=f"{asan}:{ubsan}",
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:exitcode=66",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1:exitcode=67",
               OMP_NUM_THREADS="4")
    res = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-m", "not gpu",
                          "-p", "no:cacheprovider", os.path.join(ROOT, "tests", "test_oracle_pinning.py")],
                         capture_output=True, text=True, env=env, cwd=ROOT, timeout=900)
    out = res.stdout + res.stderr
    assert res.returncode == 0, out[-4000:]
    assert "passed" in res.stdout and "ERROR: AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
