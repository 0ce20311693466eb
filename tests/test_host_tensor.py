"""Host-side tensor construction from numpy arrays (no GPU): the shape, dtype
and values match what the reference's constructor produces from
``data.tolist()`` (src/nanotorch/core.py:79-84), including 0-d arrays,
non-contiguous arrays and a dtype override."""

from __future__ import annotations

import numpy as np
import pytest

import nanotorch_amd as nt


@pytest.mark.parametrize("arr", [
    np.float32(2.5),
    np.full((), 7, np.int64),
    np.arange(5, dtype=np.float64),
    np.arange(12, dtype=np.int32).reshape(3, 4),
    np.arange(24, dtype=np.float32).reshape(2, 3, 4)[:, ::2, 1:].transpose(2, 0, 1),
    np.array([[True, False], [False, True]]),
])
def test_from_numpy_matches_tolist(arr):
    a = np.asarray(arr)
    t = nt.Tensor(a)
    ref = nt.tensor(a.tolist())
    assert t.shape == a.shape == ref.shape
    assert t.numpy().dtype == a.dtype
    assert t.cpu().tolist() == a.tolist()


def test_from_numpy_with_dtype_override():
    a = np.arange(6, dtype=np.int32).reshape(2, 3)
    t = nt.Tensor(a, dtype=nt.float32)
    assert t.dtype == nt.float32 and t.shape == (2, 3)
    assert t.cpu().tolist() == [[0.0, 1.0, 2.0], [3.0, 4.0, 5.0]]
