"""The library's host generator (nt_manual_seed / nt_host_uniform, its own
MT19937-64 and uniform conversion) against the oracle's std::mt19937_64 +
std::uniform_real_distribution -- the reference's generator
(src/cpp/random.h:5-13, src/cpp/factory.cu:73-83) -- bit for bit: chunked
draws continue one stream, float32 and float64 draws each consume one engine
output, and the bounds are applied as (r * (b - a)) + a.  No GPU needed."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from nanotorch_amd import _lib
import oracle as O

F32, F64 = 3, 4


def host_draws(n, code=F32, low=0.0, high=1.0):
    dt = np.float32 if code == F32 else np.float64
    out = np.empty(n, dtype=dt)
    rc = _lib.load().nt_host_uniform(ctypes.c_void_p(out.ctypes.data), code,
                                     ctypes.c_int64(n), ctypes.c_double(low),
                                     ctypes.c_double(high))
    assert rc == 0
    return out


def seed(s):
    assert _lib.load().nt_manual_seed(ctypes.c_uint64(s)) == 0


@pytest.mark.parametrize("s", [0, 1, 42, 5489, 2**63 + 12345, 2**64 - 1])
def test_host_stream_matches_reference(s):
    seed(s)
    chunks = [1, 310, 1, 1, 312, 313, 5000, 624, 7]
    got = np.concatenate([host_draws(n) for n in chunks])
    assert got.tobytes() == O.uniform(s, sum(chunks)).tobytes()


def test_host_float64_and_bounds():
    seed(77)
    plan = [(F32, 100, 0.0, 1.0), (F64, 333, 0.0, 1.0), (F32, 700, -3.0, 5.0),
            (F64, 50, 2.0, 2.5), (F32, 1, 1e-3, 1e3)]
    skip = 0
    for code, n, lo, hi in plan:
        got = host_draws(n, code, lo, hi)
        want = O.uniform(77, n, dtype=got.dtype, skip=skip, low=lo, high=hi)
        assert got.tobytes() == want.tobytes(), (code, n, lo, hi)
        skip += n


def test_host_reseed_restarts_stream():
    seed(3)
    a = host_draws(1000)
    seed(3)
    b = host_draws(1000)
    assert a.tobytes() == b.tobytes()
    assert host_draws(0).size == 0


def test_host_rejects_integer_dtype():
    buf = (ctypes.c_int64 * 2)()
    assert _lib.load().nt_host_uniform(ctypes.addressof(buf), 2, 2, 0.0, 1.0) == _lib.NT_ERR_VALUE


def test_jump_tables_build_and_self_check():
    """The device generator's host-side tables: the characteristic
    polynomial (Berlekamp-Massey must find degree 19937) and x^(w L) mod P
    for every substream, with the built-in check that a table jump lands on
    the window reached by stepping the generator directly.  No device."""
    import time

    t0 = time.perf_counter()
    assert _lib.load().nt_rng_prepare() == 0
    assert time.perf_counter() - t0 < 30
    assert _lib.load().nt_rng_prepare() == 0  # built once, then a no-op
