"""Writes known_answers.json: the known-answer tables of the reference's own
test-suite, transcribed as data (inputs and expected outputs), each entry
tagged with the reference file:line it comes from.  No reference code is
imported or run; re-running this script regenerates the same file.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import math
import os

E = math.e
HERE = os.path.dirname(os.path.abspath(__file__))


def unary_tables():
    t = []
    # tests/test_ops/test_tensor_unary_ops.py:10-26 (exp)
    for inp, exp in [(0.0, 1.0), (1.0, E), ([0, 1], [1.0, E]),
                     ([[0, 1], [2, 3]], [[1.0, E], [E**2, E**3]])]:
        t.append({"src": "tests/test_ops/test_tensor_unary_ops.py:10-26", "op": "exp",
                  "input": inp, "expected": exp, "tol": 1e-6})
    # :29-44 (log)
    for inp, exp in [(1.0, 0.0), (E, 1.0), ([1.0, E], [0.0, 1.0]),
                     ([[1.0, E], [E**2, E**3]], [[0.0, 1.0], [2.0, 3.0]])]:
        t.append({"src": "tests/test_ops/test_tensor_unary_ops.py:29-44", "op": "log",
                  "input": inp, "expected": exp, "tol": 1e-6})
    # :47-71 (pow, tol 1e-4)
    for inp, e, exp in [(1, 1, 1), (1, 0, 1), (0, 1, 0), (0, 0, 1), (1.0, 1, 1.0),
                        (1, 1.0, 1.0), (2, 2, 4), (3, 4.0, 81.0), (9.0, -2, 0.0123),
                        (2.5, 3.7, 29.6741), ([1, 2, 3], 2, [1, 4, 9]),
                        ([[1, 2], [3, 4]], 2.0, [[1.0, 4.0], [9.0, 16.0]]),
                        ([[1.0, 2.0], [3.0, 4.0]], 2, [[1.0, 4.0], [9.0, 16.0]])]:
        t.append({"src": "tests/test_ops/test_tensor_unary_ops.py:47-71", "op": "pow",
                  "input": inp, "exponent": e, "expected": exp, "tol": 1e-4})
    # :79-87 (relu)
    for inp, exp in [(1.0, 1.0), (-1.0, 0.0), ([1.0, -1.0, 0.0], [1.0, 0.0, 0.0])]:
        t.append({"src": "tests/test_ops/test_tensor_unary_ops.py:79-87", "op": "relu",
                  "input": inp, "expected": exp, "tol": 0.0})
    return t


def binary_tables():
    """tests/test_ops/test_tensor_binary_ops.py:8-196 (add/sub/mul/div with
    scalars, bools and broadcasting; comparisons against 3)."""
    t = []
    z57 = [[0.0] * 7 for _ in range(5)]
    f = lambda v: [[v] * 7 for _ in range(5)]  # noqa: E731
    rows = [
        ("add", 0.0, 3.14, 3.14), ("add", 0.0, -3.14, -3.14), ("add", 0.0, True, 1.0),
        ("add", False, 3.14, 3.14), ("sub", 0.0, 3.14, -3.14), ("sub", 3.14, 0.0, 3.14),
        ("sub", 0.0, -3.14, 3.14), ("sub", 0.0, True, -1.0), ("sub", False, 3.14, -3.14),
        ("mul", 1.0, 3.14, 3.14), ("mul", 1.0, -3.14, -3.14), ("mul", 1.0, True, 1.0),
        ("mul", True, 3.14, 3.14), ("div", 6.28, 2.0, 3.14), ("div", 6.28, -2.0, -3.14),
        ("div", 3.14, True, 3.14), ("div", False, 2.0, 0.0),
    ]
    for op, a, b, exp in rows:
        t.append({"src": "tests/test_ops/test_tensor_binary_ops.py:8-160", "op": op,
                  "a": a, "b": b, "expected": exp})
    t.append({"src": "tests/test_ops/test_tensor_binary_ops.py:15-16", "op": "add",
              "a": z57, "b": [[3.14] for _ in range(5)], "expected": f(3.14)})
    t.append({"src": "tests/test_ops/test_tensor_binary_ops.py:17-19", "op": "add",
              "a": z57, "b": [3.14] * 7, "expected": f(3.14)})
    t.append({"src": "tests/test_ops/test_tensor_binary_ops.py:148-152", "op": "div",
              "a": f(6.28), "b": [2.0] * 7, "expected": f(3.14)})
    ar = [[4 * i + j for j in range(4)] for i in range(3)]
    for op, fn in (("eq", lambda i: i == 3), ("gt", lambda i: i > 3), ("ge", lambda i: i >= 3),
                   ("lt", lambda i: i < 3), ("le", lambda i: i <= 3)):
        t.append({"src": "tests/test_ops/test_tensor_binary_ops.py:161-196", "op": op,
                  "a": ar, "b": 3, "expected": [[fn(4 * i + j) for j in range(4)] for i in range(3)]})
    return t


def matmul_tables():
    """tests/test_ops/test_tensor_binary_ops.py:197-270, 315-316."""
    a23 = [[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]]
    t = [
        {"a": [[1.0, 2.0], [3.0, 4.0]], "b": [[5.0, 6.0], [7.0, 8.0]],
         "expected": [[19.0, 22.0], [43.0, 50.0]]},
        {"a": [[0.0, 1.0, 2.0], [3.0, 4.0, 5.0]],
         "b": [[float(4 * i + j) for j in range(4)] for i in range(3)],
         "expected": [[20.0, 23.0, 26.0, 29.0], [56.0, 68.0, 80.0, 92.0]]},
        {"a": [[1.0, 2.0, 3.0]], "b": [[4.0], [5.0], [6.0]], "expected": [[32.0]]},
        {"a": a23, "b": "a23.T", "expected": [[14.0, 32.0], [32.0, 77.0]]},
        {"a": "a23.T", "b": a23,
         "expected": [[17.0, 22.0, 27.0], [22.0, 29.0, 36.0], [27.0, 36.0, 45.0]]},
        {"a": "arange12[:, ::2]", "b": [[1.0, 1.0], [1.0, 1.0]],
         "expected": [[2.0, 2.0], [10.0, 10.0], [18.0, 18.0]]},
        {"a": [0.0, 1.0, 2.0, 3.0, 4.0], "b": [0.0, 1.0, 2.0, 3.0, 4.0], "expected": 30.0},
    ]
    for x in t:
        x["src"] = "tests/test_ops/test_tensor_binary_ops.py:197-316"
    return t, a23


def reduction_tables():
    t = []
    # tests/test_ops/test_tensor_reduction_ops.py:177-220 (SUM_AXIS_KEEPDIM_SPEC)
    spec = [
        ([1.0, 2.0, 3.0], 0, False, [], 6.0), ([1.0, 2.0, 3.0], 0, True, [1], [6.0]),
        ([1.0, 2.0, 3.0], None, False, [], 6.0), ([1.0, 2.0, 3.0], None, True, [1], [6.0]),
        ([[1, 2, 3], [4, 5, 6]], 0, False, [3], [5, 7, 9]),
        ([[1, 2, 3], [4, 5, 6]], 0, True, [1, 3], [[5, 7, 9]]),
        ([[1, 2, 3], [4, 5, 6]], 1, False, [2], [6, 15]),
        ([[1, 2, 3], [4, 5, 6]], 1, True, [2, 1], [[6], [15]]),
        ([[1, 2, 3], [4, 5, 6]], -1, False, [2], [6, 15]),
        ([[1, 2, 3], [4, 5, 6]], -2, False, [3], [5, 7, 9]),
        ([[1, 2, 3], [4, 5, 6]], None, False, [], 21.0),
        ([[1, 2, 3], [4, 5, 6]], None, True, [1, 1], [[21.0]]),
        ([[1, 2, 3], [4, 5, 6]], [0, 1], False, [], 21.0),
        ([[[1, 2], [3, 4]], [[5, 6], [7, 8]]], 0, False, [2, 2], [[6, 8], [10, 12]]),
        ([[[1, 2], [3, 4]], [[5, 6], [7, 8]]], 1, False, [2, 2], [[4, 6], [12, 14]]),
        ([[[1, 2], [3, 4]], [[5, 6], [7, 8]]], 2, False, [2, 2], [[3, 7], [11, 15]]),
        ([[[1, 2], [3, 4]], [[5, 6], [7, 8]]], [0, 2], False, [2], [14, 22]),
        ([[[1, 2], [3, 4]], [[5, 6], [7, 8]]], [0, 2], True, [1, 2, 1], [[[14], [22]]]),
        ([[[1, 2], [3, 4]], [[5, 6], [7, 8]]], None, False, [], 36.0),
    ]
    for x, axis, kd, shape, exp in spec:
        t.append({"src": "tests/test_ops/test_tensor_reduction_ops.py:177-220", "op": "sum",
                  "input": x, "axis": axis, "keepdim": kd, "shape": shape, "expected": exp})
    # inputs "1d" and "1d-ties" (:52-53): first extremum on ties
    for x, mx, imx, mn, imn in [([0.0, 2.5, -1.5, 8, 7, 3], 8.0, 3, -1.5, 2),
                                ([0.0, -1.5, -1.5, 8, 8, 3], 8.0, 3, -1.5, 1)]:
        t.append({"src": "tests/test_ops/test_tensor_reduction_ops.py:52-53", "op": "select",
                  "input": x, "max": mx, "argmax": imx, "min": mn, "argmin": imn})
    # dtype contracts (:222-281)
    for inp, dt, out_dt in [([True, False, True], "bool", "int64"), ([1, 2, 3], "int32", "int64"),
                            ([1, 2, 3], "int64", "int64"), ([1.0, 2.0, 3.0], "float32", "float32"),
                            ([1.0, 2.0, 3.0], "float64", "float64")]:
        t.append({"src": "tests/test_ops/test_tensor_reduction_ops.py:224-238",
                  "op": "sum_default_dtype", "input": inp, "dtype": dt, "out_dtype": out_dt})
    for inp, dt, kw, exp in [([1, 2, 3], "int32", "float32", 6.0), ([1, 2, 3], "int32", "float64", 6.0),
                             ([1.5, 2.5], "float32", "float64", 4.0),
                             ([True, True, False], "bool", "int32", 2),
                             ([True, True, False], "bool", "float32", 2.0)]:
        t.append({"src": "tests/test_ops/test_tensor_reduction_ops.py:241-256",
                  "op": "sum_dtype_kwarg", "input": inp, "dtype": dt, "kwarg": kw, "expected": exp})
    for dt, kw in [("int32", "float32"), ("int64", "float64"), ("float32", "float64")]:
        t.append({"src": "tests/test_ops/test_tensor_reduction_ops.py:267-276",
                  "op": "mean_dtype_kwarg", "input": [1, 2, 3], "dtype": dt, "kwarg": kw,
                  "expected": 2.0})
    return t


def autograd_tables():
    """tests/test_autograd.py:34-144 closed forms."""
    return [
        {"src": "tests/test_autograd.py:34-40", "case": "3x", "x": 1.0, "grad": 3.0, "tol": 1e-6},
        {"src": "tests/test_autograd.py:43-51", "case": "exp(3x)", "x": 1.0, "grad": 60.2566,
         "tol": 1e-3},
        {"src": "tests/test_autograd.py:54-65", "case": "log(x1*x2)", "x1": 1.0, "x2": 5.0,
         "g1": 1.0, "g2": 0.2, "tol": 1e-6},
        {"src": "tests/test_autograd.py:68-81", "case": "sum(log(x1*x2))", "x1": [1.0, 5.0],
         "x2": [5.0, 1.0], "g1": [1.0, 0.2], "g2": [0.2, 1.0], "tol": 1e-6},
        {"src": "tests/test_autograd.py:84-104", "case": "sum(sum(x,0))",
         "x": [[1.0, 2.0], [2.0, 1.0]], "grad": [[1.0, 1.0], [1.0, 1.0]], "tol": 0.0},
        {"src": "tests/test_autograd.py:107-115", "case": "sum(x.T*g)",
         "x": [[0.0] * 3] * 2, "g": [[0, 1], [2, 3], [4, 5]], "grad": [[0, 2, 4], [1, 3, 5]],
         "tol": 0.0},
        {"src": "tests/test_autograd.py:132-144", "case": "sum(2*exp(x)+3*exp(x))",
         "x": [1.0, 2.0], "grad": [5 * E, 5 * E**2], "tol": 1e-5},
    ]


def indexing_tables():
    """Advanced indexing known answers, tests/test_ops/test_tensor_core.py.
    Selectors are encoded as {"list": v} (a Python sequence), {"tensor": v}
    (nt.tensor(v)), {"int": n}, {"slice": [start, stop, step]}, {"ellipsis": 1}
    or {"none": 1}; "x" is nt.tensor(x) unless "arange" gives
    nt.arange(n).reshape(shape)."""
    M = [[1, 2, 3, 4], [5, 6, 7, 8], [9, 10, 11, 12]]
    M3 = [[[1, 2], [3, 4]], [[5, 6], [7, 8]], [[9, 10], [11, 12]]]
    L = lambda v: {"list": v}  # noqa: E731
    T = lambda v: {"tensor": v}  # noqa: E731
    S = lambda a=None, b=None, c=None: {"slice": [a, b, c]}  # noqa: E731
    R12 = [[1, 2, 3, 4], [5, 6, 7, 8], [9, 10, 11, 12]][1:]
    get = [
        (":400-402", M, [L([1, 2])], R12),
        (":405-407", M, [T([1, 2])], R12),
        (":410-412", M, [L([False, True, True])], R12),
        (":415-417", M, [T([False, True, True])], R12),
        (":426-428", M, [L([-2, -1])], R12),
        (":431-433", M, [T([-2, -1])], R12),
        (":436-438", M, [S(), L([1, 2])], [[2, 3], [6, 7], [10, 11]]),
        (":441-443", M, [S(), T([1, 2])], [[2, 3], [6, 7], [10, 11]]),
        (":458-460", M, [L([1, 2, 1]), L([1, 1, 0])], [6, 10, 5]),
        (":463-465", M, [T([1, 2, 1]), T([1, 1, 0])], [6, 10, 5]),
        (":474-476", M, [L([1, 2, 1]), L([1])], [6, 10, 6]),
        (":479-481", M, [L([1]), L([1, 2, 1])], [6, 7, 6]),
        (":484-489", M, [L([[0, 1], [1, 2]])],
         [[[1, 2, 3, 4], [5, 6, 7, 8]], [[5, 6, 7, 8], [9, 10, 11, 12]]]),
        (":492-497", M, [T([[0, 1], [1, 2]])],
         [[[1, 2, 3, 4], [5, 6, 7, 8]], [[5, 6, 7, 8], [9, 10, 11, 12]]]),
        (":500-502", M3, [L([1, 1]), S(), L([1, 0])], [[6, 8], [5, 7]]),
        (":505-507", M3, [T([1, 1]), S(), T([1, 0])], [[6, 8], [5, 7]]),
    ]
    out = []
    for src, x, idx, exp in get:
        out.append({"src": "tests/test_ops/test_tensor_core.py" + src, "kind": "get",
                    "x": x, "index": idx, "expected": exp})
    out.append({"src": "tests/test_ops/test_tensor_core.py:446-449", "kind": "get",
                "x": M, "index": [L([])], "expected": [], "shape": [0, 4]})
    for src, idx, err in [(":420-423", [L([False, True])], "IndexError"),
                          (":468-471", [L([1, 2, 1]), L([1, 1, 0, 1])], "RuntimeError")]:
        out.append({"src": "tests/test_ops/test_tensor_core.py" + src, "kind": "get",
                    "x": M, "index": idx, "error": err})
    for idx in ([L([1, 4]), {"int": 2}, L([2, 3])], [L([1, -5])]):  # :509-514
        out.append({"src": "tests/test_ops/test_tensor_core.py:510-515", "kind": "get",
                    "arange": 60, "shape": [4, 3, 5], "index": idx, "error": "IndexError"})
    sets = [
        (":655-658", 6, [6], [L([True, False, False, True, False, True])], 12,
         [12, 1, 2, 12, 4, 12]),
        (":667-670", 6, [6], [L([1, 3, 5])], 12, [0, 12, 2, 12, 4, 12]),
        (":673-676", 6, [6], [T([1, 3, 5])], 12, [0, 12, 2, 12, 4, 12]),
        (":679-682", 6, [6], [L([1, 3, -1])], 12, [0, 12, 2, 12, 4, 12]),
        (":685-688", 6, [6], [L([0, 0, 0])], [12, 13, 14], [14, 1, 2, 3, 4, 5]),
        (":798-801", 12, [4, 3], [L([True, False, False, True])], 12,
         [[12, 12, 12], [3, 4, 5], [6, 7, 8], [12, 12, 12]]),
        (":810-813", 12, [4, 3], [L([0, 3])], 12,
         [[12, 12, 12], [3, 4, 5], [6, 7, 8], [12, 12, 12]]),
        (":816-819", 12, [4, 3], [L([0, -1])], 12,
         [[12, 12, 12], [3, 4, 5], [6, 7, 8], [12, 12, 12]]),
        (":828-831", 12, [3, 4], [S(), L([1, 2])], [[10, 20], [30, 40], [50, 60]],
         [[0, 10, 20, 3], [4, 30, 40, 7], [8, 50, 60, 11]]),
        (":834-837", 12, [3, 4], [L([[0, 1], [1, 2]])], 33,
         [[33, 33, 33, 33], [33, 33, 33, 33], [33, 33, 33, 33]]),
        (":840-843", 12, [3, 4], [L([0, 1]), L([1, 2])], 33,
         [[0, 33, 2, 3], [4, 5, 33, 7], [8, 9, 10, 11]]),
    ]
    for src, n, shape, idx, val, exp in sets:
        out.append({"src": "tests/test_ops/test_tensor_core.py" + src, "kind": "set",
                    "arange": n, "shape": shape, "index": idx, "value": val,
                    "expected": exp})
    for src, n, shape, idx in [(":661-664", 6, [6], [L([True, False, False, True, False])]),
                               (":691-694", 6, [6], [L([1, 3, 5, 12])]),
                               (":804-807", 12, [4, 3], [L([True, False, False])]),
                               (":822-825", 12, [4, 3], [L([0, 4])])]:
        out.append({"src": "tests/test_ops/test_tensor_core.py" + src, "kind": "set",
                    "arange": n, "shape": shape, "index": idx, "value": 12,
                    "error": "IndexError"})
    return out


def main() -> None:
    mm, a23 = matmul_tables()
    data = {
        "unary": unary_tables(),
        "binary": binary_tables(),
        "matmul": mm,
        "matmul_a23": a23,
        "reduction": reduction_tables(),
        "autograd": autograd_tables(),
        "indexing": indexing_tables(),
        "rng": {"src": "tests/test_factories.py:239-242", "seed": 42,
                "first": 0.7551555037498474,
                "second_msvc": 0.6390313506126404,
                "note": "the second value was produced with MSVC's STL; libstdc++ "
                        "gives 1 ulp more"},
    }
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(data, f, indent=1)


if __name__ == "__main__":
    main()
