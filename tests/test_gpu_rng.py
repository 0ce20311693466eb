"""Device uniform draws (nt_device_uniform: MT19937-64 jumped ahead into
parallel substreams) against the reference's generator -- the oracle's
std::mt19937_64 through std::uniform_real_distribution
(src/cpp/random.h:5-13, src/cpp/factory.cu:73-83) -- bit for bit.

Sizes cover the head of a partly used block, whole and partial substreams
(79872 words each), several substreams, and more than one launch round
(512 substreams); interleaved host and device draws must continue one
stream; manual_seed restarts it; float64 and bounds follow the same
conversion.  The Python factories rand / randint on "cuda" draw on the
device and must equal their host results."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import nanotorch_amd as nt
from nanotorch_amd import _lib
from nanotorch_amd._storage import Storage
from nanotorch_amd.cuda import Device

import oracle as O

pytestmark = pytest.mark.gpu

SUB = 312 * 256          # raw words per substream
ROUND = 512 * SUB        # words per launch round
F32, F64 = 3, 4


def seed(s):
    nt.manual_seed(s)


def dev_draws(n, dtype=np.float32, low=0.0, high=1.0):
    ntd = nt.float32 if dtype == np.float32 else nt.float64
    st = Storage.allocate(n, ntd, Device.Cuda)
    if n:
        _lib.call("nt_device_uniform", st.data_ptr(), int(ntd), n, low, high)
    return nt.Tensor._new_contiguous(st, (n,)).numpy()


def host_draws(n, dtype=np.float32, low=0.0, high=1.0):
    out = np.empty(n, dtype=dtype)
    code = F32 if dtype == np.float32 else F64
    if n:
        _lib.call("nt_host_uniform", out.ctypes.data, code, n, low, high)
    return out


def same(a, b):
    return a.dtype == b.dtype and a.shape == b.shape and a.tobytes() == b.tobytes()


@pytest.mark.parametrize("n", [1, 7, 311, 312, 313, 1000, SUB - 1, SUB, SUB + 1,
                               3 * SUB + 5, 17 * SUB])
def test_device_draws_match_reference(gpu, n):
    for s in (42, 2**64 - 1):
        seed(s)
        got = dev_draws(n)
        assert same(got, O.uniform(s, n)), (s, n)


def test_device_draws_continue_a_partly_used_block(gpu):
    # every head length 0..311 of the current block, then a substream edge
    seed(11)
    lengths = [5, 300, 7, 312, 1, SUB + 200, 2 * SUB - 3, 311, 2]
    got = np.concatenate([dev_draws(k) for k in lengths])
    assert same(got, O.uniform(11, sum(lengths)))


def test_more_than_one_round(gpu):
    n = ROUND + 2 * SUB + 1234  # two launch rounds, the second partial
    seed(5)
    got = dev_draws(n)
    assert same(got, O.uniform(5, n))
    # the state after two rounds continues on the host
    assert same(host_draws(1000), O.uniform(5, 1000, skip=n))


def test_host_and_device_draws_share_one_stream(gpu):
    seed(123)
    plan = [("h", 5), ("d", 400), ("d", 1), ("h", 700), ("d", 2 * SUB + 3),
            ("h", 10), ("d", 312), ("h", 1), ("d", SUB)]
    parts = [host_draws(k) if where == "h" else dev_draws(k) for where, k in plan]
    assert same(np.concatenate(parts), O.uniform(123, sum(k for _, k in plan)))


def test_float64_and_bounds(gpu):
    seed(77)
    plan = [(np.float32, 100, 0.0, 1.0), (np.float64, 3 * SUB + 7, 0.0, 1.0),
            (np.float32, SUB + 9, -3.0, 5.0), (np.float64, 500, 2.0, 2.5),
            (np.float32, 1, 1e-3, 1e3)]
    skip = 0
    for dt, n, lo, hi in plan:
        got = dev_draws(n, dt, lo, hi)
        assert same(got, O.uniform(77, n, dtype=dt, skip=skip, low=lo, high=hi)), (dt, n)
        skip += n


def test_manual_seed_restarts_after_device_draws(gpu):
    seed(1)
    dev_draws(5 * SUB)  # queued work that the reseed supersedes
    seed(2)
    assert same(dev_draws(50), O.uniform(2, 50))
    seed(3)
    dev_draws(100)
    assert same(host_draws(10), O.uniform(3, 10, skip=100))
    seed(4)
    assert dev_draws(0).size == 0  # draws nothing, keeps the state
    assert same(host_draws(3), O.uniform(4, 3))


def test_config_size_draw(gpu):
    n = 2**26  # a [8192, 8192] float32 tensor
    seed(2024)
    got = dev_draws(n)
    want = O.uniform(2024, n)
    assert same(got, want)
    assert got.min() >= 0.0 and got.max() < 1.0


def test_device_uniform_errors(gpu):
    with pytest.raises(ValueError):
        _lib.call("nt_device_uniform", 0, 2, 4, 0.0, 1.0)  # int64: not a float dtype
    with pytest.raises(ValueError):
        _lib.call("nt_device_uniform", 0, F32, 4, 0.0, 1.0)  # no buffer


def test_rand_randint_on_device_equal_host(gpu):
    seed(9)
    a = nt.rand(64, 130, device="cuda")
    seed(9)
    b = nt.rand(64, 130)
    assert a.device == nt.Device.Cuda and same(a.numpy(), b.numpy())
    seed(9)
    c = nt.rand(3, 5, dtype=nt.float64, device="cuda")
    assert same(c.numpy(), O.uniform(9, 15, dtype=np.float64).reshape(3, 5))
    seed(10)
    r = nt.randint(-5, 17, (40, 50), device="cuda")
    seed(10)
    h = nt.randint(-5, 17, (40, 50))
    assert r.dtype == nt.int64 and same(r.numpy(), h.numpy())
    seed(10)
    r32 = nt.randint(0, 3, (7,), dtype=nt.int32, device="cuda")
    u = O.uniform(10, 7)
    # (u * f32(3)) + f32(0) in float32, truncated: factories.py:241-253
    assert r32.dtype == nt.int32
    assert r32.numpy().tolist() == [int(np.float32(v) * np.float32(3)) for v in u]
