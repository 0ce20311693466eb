"""The caching allocator under concurrent callers (host code only, no GPU).

libnt is bound with ctypes, which releases the GIL around every call, so
Python threads and a garbage collector freeing tensors on another thread
can enter the allocator at once.  tests/cpp/alloc_threads.cpp builds the
allocator class of the library (nanotorch_amd/csrc/caching_allocator.h)
over malloc, with ThreadSanitizer, and runs 8 threads of allocate / stamp /
check / free plus a thread that keeps releasing the cache."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_allocator_threads_tsan(tmp_path):
    exe = tmp_path / "alloc_threads"
    subprocess.run(["g++", "-std=c++20", "-O1", "-g", "-fsanitize=thread", "-pthread",
                    "-I", os.path.join(ROOT, "nanotorch_amd", "csrc"),
                    os.path.join(ROOT, "tests", "cpp", "alloc_threads.cpp"), "-o", str(exe)],
                   check=True)
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1 exitcode=66")
    res = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "errors=0 in_use=0 raw_live=0 rejected=1" in res.stdout, res.stdout
