"""Several host threads driving the device library at once.

The ctypes binding releases the GIL around every call, so these threads
really enter libnt concurrently; the library serialises them with its lock
(and the allocator with its own).  Each thread allocates, computes, checks
and frees in a loop, while the main thread forces garbage collection, so
storages are also freed from other threads.  Every result must be exact and
the allocator's byte count must return to where it started."""

from __future__ import annotations

import ctypes
import gc
import threading

import numpy as np
import pytest

from helpers import assert_bitexact, dev, rng

import nanotorch_amd as nt
from nanotorch_amd import _lib

pytestmark = pytest.mark.gpu


def _in_use() -> int:
    a, b = ctypes.c_size_t(0), ctypes.c_size_t(0)
    _lib.call("nt_memory_stats", ctypes.byref(a), ctypes.byref(b))
    return a.value


def test_threads_share_the_library(gpu):
    nt.sync()
    gc.collect()
    start = _in_use()
    errors: list = []

    def work(tid: int) -> None:
        try:
            r = rng(100 + tid)
            for it in range(40):
                shape = (int(r.integers(1, 300)), int(r.integers(1, 300)))
                a = r.standard_normal(shape).astype(np.float32)
                b = r.standard_normal(shape).astype(np.float32)
                x, y = dev(a), dev(b)
                z = (x * y + x).T  # a view of a fresh result
                s = nt.sum(x, axis=1)
                got = z.numpy()
                want = ((a * b) + a).T
                assert_bitexact(np.ascontiguousarray(got), np.ascontiguousarray(want), f"t{tid} it{it}")
                ref = a.astype(np.float64).sum(axis=1)
                assert np.allclose(s.numpy(), ref, rtol=1e-5, atol=1e-4)
                del x, y, z, s
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append((tid, repr(e)))

    ts = [threading.Thread(target=work, args=(i,)) for i in range(6)]
    for t in ts:
        t.start()
    while any(t.is_alive() for t in ts):
        gc.collect()
        for t in ts:
            t.join(timeout=0.01)
    assert not errors, errors
    nt.sync()
    gc.collect()
    assert _in_use() == start
