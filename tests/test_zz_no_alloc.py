"""nt_reduce_noalloc, the allocation-free variant of nt_reduce, through the
C ABI: its results must equal nt_reduce's bit for bit (values, first
indices, tie counts; sums too, since both run the same kernels in the same
order), it must leave the caching allocator untouched (no block taken, none
cached), and a second call right after, on a smaller input, must not see the
first call's partial results in the shared static scratch array."""

from __future__ import annotations

import ctypes
import gc

import numpy as np
import pytest

from helpers import assert_bitexact, dev, rng, seed_of

import nanotorch_amd as nt
from nanotorch_amd import _kernels as K
from nanotorch_amd import _lib

pytestmark = pytest.mark.gpu


def _stats():
    a, b = ctypes.c_size_t(0), ctypes.c_size_t(0)
    _lib.call("nt_memory_stats", ctypes.byref(a), ctypes.byref(b))
    return a.value, b.value


def _outputs(op, kshape):
    k = int(np.prod(kshape))
    val = nt.Tensor(np.zeros(k, np.int64 if op in (_lib.R_ARGMAX, _lib.R_ARGMIN) else np.float32),
                    device="cuda")
    idx = nt.Tensor(np.zeros(k, np.int64), device="cuda")
    cnt = nt.Tensor(np.zeros(k, np.int32), device="cuda")
    return val, idx, cnt


def _call(fn, op, x, axes, outs, aux):
    val, idx, cnt = outs
    arr = _lib.axes_array(axes)
    vx = K.view_of(x)
    vv = K.view_of(val)
    vi = K.view_of(idx) if aux else None
    vc = K.view_of(cnt) if aux else None
    _lib.call(fn, op, ctypes.byref(vx), arr, len(axes), ctypes.byref(vv),
              ctypes.byref(vi) if aux else None, ctypes.byref(vc) if aux else None)


CASES = [
    # (shape, axes): column walk with partials (max/min: 8 MiB of them),
    # the row kernel split into segments, a full reduction, the generic path
    ((8192, 8192), (0,)),
    ((8192, 8192), (0, 1)),
    ((64, 1 << 20), (1,)),
    ((6, 50, 7000), (0, 2)),
]
OPS = [(_lib.R_SUM, False), (_lib.R_MAX, True), (_lib.R_MIN, True), (_lib.R_ARGMAX, False),
       (_lib.R_ARGMIN, False)]


@pytest.mark.parametrize("shape,axes", CASES)
def test_noalloc_reduce_matches_nt_reduce(gpu, shape, axes):
    r = rng(seed_of("noalloc", shape, axes))
    a = r.integers(-50, 50, shape).astype(np.float32)  # ties: counts and first indices
    x = dev(a)
    # the smaller second input: a different plan over part of the scratch
    small = (300, 2000) if len(shape) == 2 else (3, 40, 900)
    sx = dev(r.standard_normal(small).astype(np.float32))
    kshape = tuple(s for i, s in enumerate(shape) if i not in axes)
    skshape = tuple(s for i, s in enumerate(small) if i not in axes)
    nt.sync()
    for op, aux in OPS:
        want = _outputs(op, kshape)
        _call("nt_reduce", op, x, axes, want, aux)
        swant = _outputs(op, skshape)
        _call("nt_reduce", op, sx, axes, swant, aux)
        got = _outputs(op, kshape)
        sgot = _outputs(op, skshape)
        nt.sync()
        # Return every cached block to HIP first: nt_reduce above has just
        # cached partial blocks of exactly the sizes a fallback to the
        # allocator would ask for, and such an allocation would take one
        # and give it back, leaving both figures as they were.  With the
        # cache empty, any block taken inside the calls ends up cached.
        gc.collect()
        _lib.call("nt_empty_cache")
        before = _stats()
        assert before[1] == 0, before
        _call("nt_reduce_noalloc", op, x, axes, got, aux)
        _call("nt_reduce_noalloc", op, sx, axes, sgot, aux)
        nt.sync()
        after = _stats()
        assert after == before, (op, before, after)
        for w, g in zip(want + swant, got + sgot):
            assert_bitexact(g.numpy(), w.numpy(), f"op {op} {shape} {axes}")


def test_noalloc_reduce_errors_like_nt_reduce(gpu):
    x = dev(np.ones((4, 5), np.float32))
    out = nt.Tensor(np.zeros(3, np.float32), device="cuda")
    arr = _lib.axes_array((1,))
    vx, vo = K.view_of(x), K.view_of(out)
    rc = _lib.load().nt_reduce_noalloc(_lib.R_SUM, ctypes.byref(vx), arr, 1, ctypes.byref(vo),
                                       None, None)
    assert rc == _lib.load().nt_reduce(_lib.R_SUM, ctypes.byref(vx), arr, 1, ctypes.byref(vo),
                                       None, None) != 0
    arr = _lib.axes_array((2,))
    with pytest.raises(IndexError):
        _lib.call("nt_reduce_noalloc", _lib.R_SUM, ctypes.byref(vx), arr, 1, ctypes.byref(vo),
                  None, None)
