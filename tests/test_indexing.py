"""Advanced (sequence / mask) indexing on host tensors: the index plan and
its numpy execution, against the reference test-suite's known answers
(tests/golden/known_answers.json, "indexing") and against numpy where the
two index semantics coincide.  The device path is checked against the same
answers in test_gpu_indexing.py."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

import nanotorch_amd as nt

HERE = os.path.dirname(os.path.abspath(__file__))
CASES = json.load(open(os.path.join(HERE, "golden", "known_answers.json")))["indexing"]


def decode(sel, device="cpu"):
    if "list" in sel:
        return sel["list"]
    if "tensor" in sel:
        return nt.tensor(sel["tensor"]).to(device)
    if "int" in sel:
        return sel["int"]
    if "slice" in sel:
        return slice(*sel["slice"])
    if "ellipsis" in sel:
        return Ellipsis
    return None


def make_x(case, device="cpu"):
    if "arange" in case:
        return nt.arange(case["arange"]).reshape(*case["shape"]).to(device)
    return nt.tensor(case["x"]).to(device)


def run_case(case, device="cpu"):
    x = make_x(case, device)
    idx = tuple(decode(s, device) for s in case["index"])
    if case["kind"] == "get":
        if "error" in case:
            with pytest.raises({"IndexError": IndexError, "RuntimeError": RuntimeError}[case["error"]]):
                x[idx]
            return
        got = x[idx]
        assert got.cpu().tolist() == case["expected"], case["src"]
        if "shape" in case:
            assert got.shape == tuple(case["shape"]), case["src"]
    else:
        if "error" in case:
            with pytest.raises(IndexError):
                x[idx] = case["value"]
            return
        x[idx] = case["value"]
        assert x.cpu().tolist() == case["expected"], case["src"]


@pytest.mark.parametrize("case", CASES, ids=[c["src"].split(":")[-1] + c["kind"] for c in CASES])
def test_known_answers_host(case):
    run_case(case, "cpu")


def test_cast_view_index_host():
    """tests/test_ops/test_tensor_core.py:518-537: x[:, x[0].to(int)] == x."""
    x = nt.tensor([[0.0, 1.0, 2.0, 3.0], [1.0, 2.7182817459106445, 7.389056205749512,
                   20.08553695678711], [8.0, 9.0, 10.0, 11.0]])
    for dt in (nt.int32, nt.int64):
        assert x[:, x[0].to(dt)].tolist() == x.tolist()


# numpy agrees with the reference's plan when the fancy selectors sit on
# adjacent view axes or when every selector is fancy
NP_CASES = [
    ((5, 6, 7), lambda r: (r.integers(-5, 5, (3,)),)),
    ((5, 6, 7), lambda r: (slice(None), r.integers(0, 6, (2, 3)))),
    ((5, 6, 7), lambda r: (slice(1, 4), r.integers(0, 6, (4,)), r.integers(-7, 7, (4,)))),
    ((5, 6, 7), lambda r: (r.integers(0, 5, (3, 1)), slice(None), r.integers(0, 7, (1, 2)))),
    ((5, 6, 7), lambda r: (slice(None, None, 2), slice(None), r.random(7) > 0.5)),
    ((4, 3), lambda r: (r.integers(0, 4, (0,)),)),
    ((9,), lambda r: (r.integers(-9, 9, (4, 5)),)),
]


@pytest.mark.parametrize("k", range(len(NP_CASES)))
def test_getitem_matches_numpy(k):
    shape, mk = NP_CASES[k]
    r = np.random.default_rng(k)
    a = r.standard_normal(shape).astype(np.float32)
    idx = mk(r)
    tidx = tuple(i.tolist() if isinstance(i, np.ndarray) and i.dtype == np.bool_ else
                 (nt.tensor(i.tolist(), dtype=nt.int64) if isinstance(i, np.ndarray) else i)
                 for i in idx)
    got = nt.Tensor(a)[tidx]
    want = a[idx]
    assert got.shape == want.shape
    np.testing.assert_array_equal(got.numpy(), want)


def test_setitem_matches_numpy_and_last_wins():
    r = np.random.default_rng(5)
    a = r.standard_normal((6, 5)).astype(np.float32)
    rows = np.array([0, 2, 2, 5, 0])
    vals = r.standard_normal((5, 5)).astype(np.float32)
    x = nt.Tensor(a.copy())
    x[rows.tolist()] = nt.Tensor(vals)
    want = a.copy()
    for i, rr in enumerate(rows):  # sequential: the last write wins
        want[rr] = vals[i]
    np.testing.assert_array_equal(x.numpy(), want)


def test_setitem_after_basic_offset():
    """x[1:, [0, 2]] = v writes rows 1.. (numpy semantics); the reference
    scatters into the whole tensor from row 0 (its scatter_to_axes receives
    `self`, core.py:246-253) -- a deliberate deviation."""
    a = np.arange(20, dtype=np.float32).reshape(4, 5)
    x = nt.Tensor(a.copy())
    x[1:, [0, 2]] = -1.0
    want = a.copy()
    want[1:, [0, 2]] = -1.0
    np.testing.assert_array_equal(x.numpy(), want)


def test_plan_errors():
    x = nt.arange(12).reshape(3, 4)
    with pytest.raises(NotImplementedError):
        x[[[True, False], [False, True]]]
    with pytest.raises(IndexError):
        x[["a"]]
    with pytest.raises(IndexError):
        x[{1: 2}]
