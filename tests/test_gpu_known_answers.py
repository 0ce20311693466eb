"""The reference test-suite's known-answer tables (tests/golden/
known_answers.json, transcribed by tests/golden/make_golden.py with the
reference file:line of each entry) run on the device through the public
API -- `nt.tensor(...).to("cuda")`, Python operators, methods and `nt.*`
functions -- the way the reference's own tests call it.  test_oracle_pinning
checks the same tables against the oracle on the CPU."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

import nanotorch_amd as nt

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
KA = json.load(open(os.path.join(HERE, "golden", "known_answers.json")))
DT = {"bool": nt.bool_, "int32": nt.int32, "int64": nt.int64,
      "float32": nt.float32, "float64": nt.float64}


def cu(v, dtype=None):
    return nt.tensor(v, dtype=dtype).to("cuda") if dtype else nt.tensor(v).to("cuda")


def host(t):
    return t.cpu().tolist()


@pytest.mark.parametrize("case", KA["unary"], ids=lambda c: f"{c['op']}-{c['input']}")
def test_unary_known_answers_device(gpu, case):
    x = cu(case["input"])
    op = case["op"]
    if op == "pow":
        y = x ** case["exponent"]
    elif op == "relu":
        y = nt.relu(x)
    else:
        y = getattr(x, op)()
    got = np.array(host(y), dtype=np.float64)
    want = np.array(case["expected"], dtype=np.float64)
    assert got.shape == want.shape
    assert np.all(np.abs(got - want) <= case["tol"] + 1e-7 * np.abs(want)), (case, got)


_BIN = {"add": lambda a, b: a + b, "sub": lambda a, b: a - b, "mul": lambda a, b: a * b,
        "div": lambda a, b: a / b, "eq": lambda a, b: a == b, "gt": lambda a, b: a > b,
        "ge": lambda a, b: a >= b, "lt": lambda a, b: a < b, "le": lambda a, b: a <= b}


@pytest.mark.parametrize("case", KA["binary"], ids=lambda c: f"{c['op']}-{c['src'][-7:]}")
def test_binary_known_answers_device(gpu, case):
    got = _BIN[case["op"]](cu(case["a"]), cu(case["b"])).numpy()
    # the table's decimal values as the result dtype holds them
    want = np.array(case["expected"]).astype(got.dtype)
    assert np.array_equal(got, np.broadcast_to(want, got.shape)), (case, got)


def test_matmul_known_answers_device(gpu):
    a23 = cu(KA["matmul_a23"], nt.float32)
    named = {"a23.T": a23.T,
             "arange12[:, ::2]": nt.arange(12, dtype=nt.float32).reshape(3, 4).to("cuda")[:, ::2]}
    for case in KA["matmul"]:
        a = named[case["a"]] if isinstance(case["a"], str) else cu(case["a"], nt.float32)
        b = named[case["b"]] if isinstance(case["b"], str) else cu(case["b"], nt.float32)
        got = a @ b
        assert host(got) == case["expected"], case


@pytest.mark.parametrize("case", KA["reduction"], ids=lambda c: c["op"])
def test_reduction_known_answers_device(gpu, case):
    op = case["op"]
    if op == "sum":
        x = cu(case["input"])
        axis = tuple(case["axis"]) if isinstance(case["axis"], list) else case["axis"]
        got = x.sum(axis=axis, keepdim=case["keepdim"])
        assert list(got.shape) == case["shape"]
        assert host(got) == case["expected"]
    elif op == "select":
        x = cu(case["input"], nt.float32)
        assert x.max().cpu().item() == case["max"]
        assert x.min().cpu().item() == case["min"]
        assert nt.argmax(x).cpu().item() == case["argmax"]
        assert nt.argmin(x).cpu().item() == case["argmin"]
    elif op == "sum_default_dtype":
        x = cu(case["input"], DT[case["dtype"]])
        assert x.sum().dtype == DT[case["out_dtype"]]
    elif op == "sum_dtype_kwarg":
        x = cu(case["input"], DT[case["dtype"]])
        got = x.sum(dtype=DT[case["kwarg"]])
        assert got.dtype == DT[case["kwarg"]]
        assert got.cpu().item() == case["expected"]
    elif op == "mean_dtype_kwarg":
        x = cu(case["input"], DT[case["dtype"]])
        got = x.mean(dtype=DT[case["kwarg"]])
        assert got.cpu().item() == case["expected"]
    else:
        raise AssertionError(f"unknown case {op}")
