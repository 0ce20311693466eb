"""Elementwise family on the GPU against the oracle (reference CPU loops).

Bar:
  * bit-exact: +, -, *, /, neg, relu, sqrt forward, comparisons, casts, and
    the fused backward chains made of IEEE ops only (neg, exp, sigmoid,
    relu, add, sub, mul, the a-gradient of div), given the same saved
    tensors;
  * rel 1e-6: exp/log/tanh/sigmoid/pow forward (device vs host libm);
  * rel 1e-6 against a condition-aware scale: chains whose reference form
    calls powf (log: x**-1, sqrt: y**-1, tanh: y**2, div b-gradient: b**2,
    pow: x**(e-1)).  glibc's powf is off correct rounding by one ulp on a
    fraction of a percent of inputs (test_oracle_pinning.py), the GPU
    evaluates v*v and 1/v correctly rounded, so the chains can differ by
    that ulp times the chain's sensitivity: |g|*(1 + y*y) for tanh,
    |result| otherwise, plus |old| in accumulate mode.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from helpers import assert_bitexact, assert_rel, dev, dev_T, host, rng, seed_of

import nanotorch_amd as nt
from nanotorch_amd import _kernels as K
from nanotorch_amd import _lib

pytestmark = pytest.mark.gpu

UNARY = [
    ("exp", _lib.EXP, O.EXP, (-4, 4), False),
    ("log", _lib.LOG, O.LOG, (0.1, 4), False),
    ("neg", _lib.NEG, O.NEG, (-4, 4), True),
    ("relu", _lib.RELU, O.RELU, None, True),
    ("sqrt", _lib.SQRT, O.SQRT, (0.1, 4), True),
    ("tanh", _lib.TANH, O.TANH, None, False),
    ("sigmoid", _lib.SIGMOID, O.SIGMOID, None, False),
    ("pow", _lib.POW, O.POW, (0.1, 4), False),
]

BINARY = [("add", _lib.ADD, O.ADD), ("sub", _lib.SUB, O.SUB),
          ("mul", _lib.MUL, O.MUL), ("div", _lib.DIV, O.DIV)]


def _inputs(r, dom, shape, dtype=np.float32):
    if dom is None:
        return r.standard_normal(shape).astype(dtype)
    return r.uniform(dom[0], dom[1], shape).astype(dtype)


def _mk(a, layout):
    return dev(a) if layout == "contig" else dev_T(a)


@pytest.mark.parametrize("layout", ["contig", "transposed"])
@pytest.mark.parametrize("shape", [(1, 1), (7, 13), (64, 64), (129, 300), (256, 1024)])
@pytest.mark.parametrize("name,op,oop,dom,exact", UNARY)
def test_unary_forward(gpu, name, op, oop, dom, exact, shape, layout):
    r = rng(seed_of(name, shape))
    a = _inputs(r, dom, shape)
    e = 2.5 if name == "pow" else 0.0
    x = _mk(a, layout)
    got = host(nt.Tensor._new_contiguous(K.unary(op, x, e), x.shape))
    want = O.unary(oop, a, e)
    if exact:
        assert_bitexact(got, want, name)
    else:
        assert_rel(got, want, 1e-6, name)


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
def test_unary_integer(gpu, dtype):
    r = rng(3)
    a = r.integers(-50, 50, (33, 17)).astype(dtype)
    for op, oop, e in ((_lib.NEG, O.NEG, 0), (_lib.RELU, O.RELU, 0), (_lib.POW, O.POW, 3)):
        x = dev(a)
        got = host(nt.Tensor._new_contiguous(K.unary(op, x, e), x.shape))
        assert_bitexact(got, O.unary(oop, a, e), f"int op {op}")


def test_unary_float64(gpu):
    r = rng(4)
    a = r.uniform(0.1, 4, (40, 50))
    for op, oop in ((_lib.EXP, O.EXP), (_lib.LOG, O.LOG), (_lib.SQRT, O.SQRT),
                    (_lib.TANH, O.TANH), (_lib.SIGMOID, O.SIGMOID)):
        got = host(nt.Tensor._new_contiguous(K.unary(op, dev(a), 0.0), a.shape))
        assert_rel(got, O.unary(oop, a), 1e-14, f"f64 op {op}")


def test_unary_dtype_errors(gpu):
    with pytest.raises(ValueError):
        K.unary(_lib.EXP, dev(np.arange(4, dtype=np.int64)))
    with pytest.raises(ValueError):
        K.unary(_lib.NEG, dev(np.array([True, False])))


@pytest.mark.parametrize("layout", ["contig", "transposed", "mixed"])
@pytest.mark.parametrize("shape", [(1, 1), (5, 7), (64, 64), (130, 257), (512, 384)])
@pytest.mark.parametrize("name,op,oop", BINARY)
def test_binary_forward(gpu, name, op, oop, shape, layout):
    r = rng(seed_of(name, shape, layout))
    a = r.standard_normal(shape).astype(np.float32)
    b = (r.uniform(0.5, 2, shape) if name == "div" else r.standard_normal(shape)).astype(
        np.float32
    )
    xa = _mk(a, "contig" if layout == "mixed" else layout)
    xb = _mk(b, "transposed" if layout == "mixed" else layout)
    got = host(nt.Tensor._new_contiguous(K.binary(op, xa, xb), shape))
    assert_bitexact(got, O.binary(oop, a, b), name)


@pytest.mark.parametrize("dtype", [np.bool_, np.int32, np.int64, np.float64])
def test_binary_other_dtypes(gpu, dtype):
    r = rng(5)
    if dtype == np.bool_:
        a = r.integers(0, 2, (17, 19)).astype(bool)
        b = r.integers(0, 2, (17, 19)).astype(bool)
        ops = [(_lib.ADD, O.ADD), (_lib.SUB, O.SUB), (_lib.MUL, O.MUL)]
    else:
        a = r.integers(-100, 100, (17, 19)).astype(dtype)
        b = r.integers(1, 100, (17, 19)).astype(dtype)
        ops = [(_lib.ADD, O.ADD), (_lib.SUB, O.SUB), (_lib.MUL, O.MUL), (_lib.DIV, O.DIV)]
    for op, oop in ops:
        got = host(nt.Tensor._new_contiguous(K.binary(op, dev(a), dev(b)), a.shape))
        assert_bitexact(got, O.binary(oop, a, b), f"{dtype} {op}")
    if dtype == np.bool_:
        with pytest.raises(ValueError):
            K.binary(_lib.DIV, dev(a), dev(b))


@pytest.mark.parametrize("op,oop", [(_lib.EQ, O.EQ), (_lib.GT, O.GT), (_lib.GE, O.GE)])
def test_compare(gpu, op, oop):
    r = rng(6)
    a = r.integers(-3, 3, (65, 33)).astype(np.float32)
    b = r.integers(-3, 3, (65, 33)).astype(np.float32)
    got = host(nt.Tensor._new_contiguous(K.binary(op, dev(a), dev_T(b)), a.shape))
    assert_bitexact(got, O.binary(oop, a, b), "compare")


def test_broadcast_and_strided_views(gpu):
    r = rng(7)
    a = r.standard_normal((6, 40, 50)).astype(np.float32)
    bias = r.standard_normal((50,)).astype(np.float32)
    col = r.standard_normal((40, 1)).astype(np.float32)
    x = dev(a)
    # row broadcast (bias), column broadcast, strided slices, 3-D transpose
    for other, onp in (
        (dev(bias).expand(6, 40, 50), np.broadcast_to(bias, a.shape)),
        (dev(col).expand(6, 40, 50), np.broadcast_to(col, a.shape)),
    ):
        got = host(nt.Tensor._new_contiguous(K.binary(_lib.ADD, x, other), a.shape))
        assert_bitexact(got, O.binary(O.ADD, a, np.ascontiguousarray(onp)), "bcast")
    big = r.standard_normal((6, 40, 100)).astype(np.float32)
    xs = dev(big)[:, :, ::2]
    got = host(nt.Tensor._new_contiguous(K.unary(_lib.NEG, xs), xs.shape))
    assert_bitexact(got, -big[:, :, ::2], "strided")
    xt = dev(a).transpose(0, 2)
    got = host(nt.Tensor._new_contiguous(K.unary(_lib.RELU, xt), xt.shape))
    assert_bitexact(got, O.unary(O.RELU, np.ascontiguousarray(a.transpose(2, 1, 0))), "3d-T")


@pytest.mark.parametrize("shape", [(64, 1024), (3, 8), (129, 4096), (2, 3, 16)])
def test_broadcast_rows(gpu, shape):
    """Contiguous operands with a broadcast row (bias), a broadcast column,
    and a scalar, in every operand position; plus an unaligned variant."""
    r = rng(seed_of("rows", shape))
    a = r.standard_normal(shape).astype(np.float32)
    row = r.uniform(0.5, 2, shape[-1:]).astype(np.float32)
    colshape = shape[:-1] + (1,)
    col = r.uniform(0.5, 2, colshape).astype(np.float32)
    sc = np.array(1.75, dtype=np.float32)
    cases = [
        (dev(row).expand(*shape), np.broadcast_to(row, shape)),
        (dev(col).expand(*shape), np.broadcast_to(col, shape)),
        (dev(sc.reshape((1,) * len(shape))).expand(*shape), np.broadcast_to(sc, shape)),
    ]
    x = dev(a)
    for op, oop in ((_lib.ADD, O.ADD), (_lib.SUB, O.SUB), (_lib.MUL, O.MUL), (_lib.DIV, O.DIV)):
        for other, onp in cases:
            onp = np.ascontiguousarray(onp)
            got = host(nt.Tensor._new_contiguous(K.binary(op, x, other), shape))
            assert_bitexact(got, O.binary(oop, a, onp), f"op {op} bcast right")
            got = host(nt.Tensor._new_contiguous(K.binary(op, other, x), shape))
            assert_bitexact(got, O.binary(oop, onp, a), f"op {op} bcast left")
    # unaligned base pointer (one-element offset) takes another path
    big = r.standard_normal((int(np.prod(shape)) + 1,)).astype(np.float32)
    xu = dev(big)[1:].reshape(*shape)
    got = host(nt.Tensor._new_contiguous(K.binary(_lib.MUL, xu, cases[0][0]), shape))
    want = O.binary(O.MUL, big[1:].reshape(shape), np.ascontiguousarray(cases[0][1]))
    assert_bitexact(got, want, "unaligned")


@pytest.mark.parametrize("src,dst", [(np.float32, np.float64), (np.float64, np.float32),
                                     (np.float32, np.int64), (np.int64, np.float32),
                                     (np.float32, np.bool_), (np.bool_, np.float32),
                                     (np.int64, np.int32), (np.int32, np.bool_)])
def test_cast(gpu, src, dst):
    r = rng(8)
    a = (r.standard_normal((31, 29)) * 10).astype(src)
    if src == np.bool_:
        a = r.integers(0, 2, (31, 29)).astype(bool)
    st = K.cast(dev(a)._storage, nt.Tensor(np.zeros(1, dtype=dst)).dtype)
    got = host(nt.Tensor._new_contiguous(st, a.shape))
    assert_bitexact(got, O.cast(a, dst), f"cast {src}->{dst}")


def test_inplace_and_copy(gpu):
    r = rng(9)
    a = r.standard_normal((70, 90)).astype(np.float32)
    b = r.standard_normal((90, 70)).astype(np.float32)
    for op, oop in ((_lib.ADD, O.ADD), (_lib.SUB, O.SUB), (_lib.MUL, O.MUL), (_lib.DIV, O.DIV)):
        x = dev(a)
        y = dev(b).T  # transposed operand
        v0 = x.version
        K.inplace(op, x, y)
        want = a.copy()
        O.inplace(oop, want, b.T)
        assert_bitexact(host(x), want, f"inplace {op}")
        assert x.version == v0 + 1
    # in place through a transposed view of the output
    x = dev(np.ascontiguousarray(a.T))
    K.inplace(_lib.ADD, x.T, dev(a))
    assert_bitexact(host(x), np.ascontiguousarray((a + a).T), "inplace via view")


def test_equals(gpu):
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    assert dev(a).equals(dev(a.copy()))
    b = a.copy()
    b[2, 3] = -1
    assert not dev(a).equals(dev(b))
    assert dev(a).T.equals(dev(np.ascontiguousarray(a.T)))


# --------------------------------------------------------------- backward

UNARY_BWD = [
    ("neg", _lib.NEG, None, lambda g, s: O.bwd_neg(g), (-4, 4), "none"),
    ("exp", _lib.EXP, O.EXP, O.bwd_exp, (-4, 4), "out"),
    ("log", _lib.LOG, O.LOG, O.bwd_log, (0.1, 4), "in"),
    ("sqrt", _lib.SQRT, O.SQRT, O.bwd_sqrt, (0.1, 4), "out"),
    ("tanh", _lib.TANH, O.TANH, O.bwd_tanh, None, "out"),
    ("sigmoid", _lib.SIGMOID, O.SIGMOID, O.bwd_sigmoid, None, "out"),
    ("relu", _lib.RELU, O.RELU, O.bwd_relu, None, "out"),
    ("pow", _lib.POW, O.POW, lambda g, x: O.bwd_pow(g, x, 2.5), (0.1, 4), "in"),
]


@pytest.mark.parametrize("acc", [False, True])
@pytest.mark.parametrize("layout", ["contig", "transposed"])
@pytest.mark.parametrize("name,op,oop,chain,dom,saved", UNARY_BWD)
def test_unary_backward_kernel(gpu, name, op, oop, chain, dom, saved, layout, acc):
    """Kernel parity: feed the oracle's saved tensor to the fused kernel."""
    r = rng(seed_of(name, layout, acc))
    shape = (130, 200)
    x = _inputs(r, dom, shape)
    g = r.standard_normal(shape).astype(np.float32)
    e = 2.5 if name == "pow" else 0.0
    s = None if saved == "none" else (x if saved == "in" else O.unary(oop, x, e))
    want = chain(g, s)
    scale = np.abs(want).astype(np.float64)
    if name == "tanh":
        scale = np.abs(g).astype(np.float64) * (1 + s.astype(np.float64) ** 2)
    old = r.standard_normal(shape).astype(np.float32)
    if acc:
        want = O.accumulate(old, want)
        scale = scale + np.abs(old)
    sv = None if s is None else _mk(s, layout)
    if acc:
        tgt = _mk(old, layout)
        K.unary_bwd(op, dev(g), sv, e, tgt)
        got = host(tgt)
    else:
        st = K.unary_bwd(op, dev(g), sv, e, None)
        got = host(nt.Tensor._new_contiguous(st, shape))
    if name in ("pow", "log", "sqrt", "tanh"):
        assert_rel(got, want, 1e-6, name, scale=scale)
    else:
        assert_bitexact(got, want, name)


@pytest.mark.parametrize("acc", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("need", [(True, True), (True, False), (False, True)])
@pytest.mark.parametrize("name,op,oop", BINARY)
def test_binary_backward_kernel(gpu, name, op, oop, need, acc):
    r = rng(seed_of(name, need, acc))
    shape = (97, 131)
    a = r.standard_normal(shape).astype(np.float32)
    b = (r.uniform(0.5, 2, shape) if name == "div" else r.standard_normal(shape)).astype(np.float32)
    g = r.standard_normal(shape).astype(np.float32)
    ga_w, gb_w = O.bwd_binary(oop, g, a, b)
    olds = [r.standard_normal(shape).astype(np.float32) for _ in range(2)]
    tg = [dev(olds[0]) if acc[0] else None, dev_T(olds[1]) if acc[1] else None]
    sa, sb = K.binary_bwd(op, dev(g), dev_T(a), dev(b), need[0], tg[0], need[1], tg[1])
    for i, (n, s_, w) in enumerate(((need[0], sa, ga_w), (need[1], sb, gb_w))):
        if not n:
            continue
        scale = np.abs(w).astype(np.float64)
        if acc[i]:
            got = host(tg[i])
            w = O.accumulate(olds[i], w)
            scale = scale + np.abs(olds[i])
        else:
            got = host(nt.Tensor._new_contiguous(s_, shape))
        if name == "div" and i == 1:  # reference form: (-a) / b**2 * g
            assert_rel(got, w, 1e-6, f"{name} grad {i}", scale=scale)
        else:
            assert_bitexact(got, w, f"{name} grad {i}")


@pytest.mark.parametrize("name,op,oop,chain,dom,saved", UNARY_BWD)
def test_unary_backward_first_write_into_transposed_target(gpu, name, op, oop, chain, dom, saved):
    """The C ABI's first-write mode into an existing strided gradient (the
    accumulate flag 0 with a target): the `.T` target overwritten, a saved
    input read through `.T` and a saved output contiguous, as the sweep's
    transposed layout has them; full and partial tiles."""
    import ctypes
    r = rng(seed_of("fw-T", name))
    shape = (260, 388)
    x = _inputs(r, dom, shape)
    g = r.standard_normal(shape).astype(np.float32)
    e = 2.5 if name == "pow" else 0.0
    s = None if saved == "none" else (x if saved == "in" else O.unary(oop, x, e))
    want = chain(g, s)
    sv = None if s is None else (dev_T(s) if saved == "in" else dev(s))
    tgt = dev_T(r.standard_normal(shape).astype(np.float32))  # overwritten
    tg = dev(g)  # every operand held for the call
    _lib.call("nt_unary_bwd", op, ctypes.byref(K.view_of(tg)),
              _lib.ref(None if sv is None else K.view_of(sv)), float(e),
              ctypes.byref(K.view_of(tgt)), 0)
    got = host(tgt)
    if name in ("pow", "log", "sqrt", "tanh"):
        scale = np.abs(want).astype(np.float64)
        if name == "tanh":
            scale = np.abs(g).astype(np.float64) * (1 + s.astype(np.float64) ** 2)
        assert_rel(got, want, 1e-6, name, scale=scale)
    else:
        assert_bitexact(got, want, name)


@pytest.mark.parametrize("name,op,oop", BINARY)
def test_binary_backward_first_write_into_transposed_targets(gpu, name, op, oop):
    """First-write into two existing `.T` gradients (both outputs exchanged,
    the inputs `.T` views too), through the C ABI."""
    import ctypes
    r = rng(seed_of("fw-T-bin", name))
    shape = (260, 388)
    a = r.standard_normal(shape).astype(np.float32)
    b = (r.uniform(0.5, 2, shape) if name == "div" else r.standard_normal(shape)).astype(np.float32)
    g = r.standard_normal(shape).astype(np.float32)
    ga_w, gb_w = O.bwd_binary(oop, g, a, b)
    ta, tb = (dev_T(r.standard_normal(shape).astype(np.float32)) for _ in range(2))
    ops = (dev(g), dev_T(a), dev_T(b), ta, tb)  # every operand held for the call
    vs = [K.view_of(t) for t in ops]
    _lib.call("nt_binary_bwd", op, *(ctypes.byref(v) for v in vs[:4]), 0, ctypes.byref(vs[4]), 0)
    assert_bitexact(host(ta), ga_w, f"{name} grad a")
    if name == "div":  # reference form: (-a) / b**2 * g
        assert_rel(host(tb), gb_w, 1e-6, f"{name} grad b", scale=np.abs(gb_w).astype(np.float64))
    else:
        assert_bitexact(host(tb), gb_w, f"{name} grad b")


@pytest.mark.parametrize("shape", [(196, 452), (452, 196), (68, 132), (132, 68),
                                   (4, 260), (260, 4), (132, 132)])
def test_tile_shapes_partial_tiles(gpu, shape):
    """The 16-byte tile kernel's fp32 tile shapes (64 x 64, 128 x 64 and
    64 x 128, picked by how many streams go through the LDS exchange and how
    many are read or written straight) on 4-aligned shapes that are not
    multiples of the tiles, so every launch has partial tiles along both
    axes.  Cases by stream counts (exchanged / straight): unary forward of a
    `.T` view (1 / 1), binary forward of two `.T` views (2 / 1), mul
    backward of `.T` operands into `.T` gradients (1 / 6), neg backward into
    a `.T` gradient (1 / 2), exp backward with a contiguous saved output
    (2 / 2) and with a `.T` one (1 / 3), each accumulating, and binary ops of
    a `.T` view with broadcast rows, columns and scalars; bit-exact."""
    r = rng(seed_of("tile-shapes", shape))
    a = r.standard_normal(shape).astype(np.float32)
    b = r.standard_normal(shape).astype(np.float32)
    g = r.standard_normal(shape).astype(np.float32)
    old = [r.standard_normal(shape).astype(np.float32) for _ in range(2)]
    for op, oop in ((_lib.NEG, O.NEG), (_lib.RELU, O.RELU)):
        got = host(nt.Tensor._new_contiguous(K.unary(op, dev_T(a), 0.0), shape))
        assert_bitexact(got, O.unary(oop, a, 0.0), f"unary fwd {op}")
    got = host(nt.Tensor._new_contiguous(K.binary(_lib.ADD, dev_T(a), dev_T(b)), shape))
    assert_bitexact(got, O.binary(O.ADD, a, b), "add fwd")
    tg = [dev_T(old[0]), dev_T(old[1])]
    K.binary_bwd(_lib.MUL, dev(g), dev_T(a), dev_T(b), True, tg[0], True, tg[1])
    ga, gb = O.bwd_binary(O.MUL, g, a, b)
    assert_bitexact(host(tg[0]), O.accumulate(old[0], ga), "mul bwd a")
    assert_bitexact(host(tg[1]), O.accumulate(old[1], gb), "mul bwd b")
    t = dev_T(old[0])
    K.unary_bwd(_lib.NEG, dev(g), None, 0.0, t)
    assert_bitexact(host(t), O.accumulate(old[0], O.bwd_neg(g)), "neg bwd")
    y = O.unary(O.EXP, a, 0.0)
    for saved in (dev(y), dev_T(y)):
        t = dev_T(old[1])
        K.unary_bwd(_lib.EXP, dev(g), saved, 0.0, t)
        assert_bitexact(host(t), O.accumulate(old[1], O.bwd_exp(g, y)), "exp bwd")
    # a `.T` operand beside a broadcast row (bias), a broadcast column and a
    # scalar, in both operand positions (one exchanged stream)
    row = r.uniform(0.5, 2, shape[1:]).astype(np.float32)
    col = r.uniform(0.5, 2, (shape[0], 1)).astype(np.float32)
    sc = np.array([[1.75]], np.float32)
    for other, onp in ((dev(row).expand(*shape), np.broadcast_to(row, shape)),
                       (dev(col).expand(*shape), np.broadcast_to(col, shape)),
                       (dev(sc).expand(*shape), np.broadcast_to(sc, shape))):
        onp = np.ascontiguousarray(onp)
        for op, oop in ((_lib.ADD, O.ADD), (_lib.DIV, O.DIV)):
            got = host(nt.Tensor._new_contiguous(K.binary(op, dev_T(a), other), shape))
            assert_bitexact(got, O.binary(oop, a, onp), f"op {op} .T with broadcast")
            got = host(nt.Tensor._new_contiguous(K.binary(op, other, dev_T(a)), shape))
            assert_bitexact(got, O.binary(oop, onp, a), f"op {op} broadcast with .T")


@pytest.mark.parametrize("dtype", [np.float64, np.int32, np.int64])
def test_tile_kernel_other_dtypes(gpu, dtype):
    """The 16-byte tile kernel for non-fp32 element types (64 x 64 tiles,
    vectors of four 8- or 4-byte elements) on 4-aligned shapes with partial
    tiles: binary ops and negation of `.T` views, comparisons, and casts
    from a `.T` view to another type; bit-exact."""
    r = rng(seed_of("tile-dtypes", np.dtype(dtype).name))
    shape = (132, 196)
    if np.issubdtype(dtype, np.integer):
        a = r.integers(-1000, 1000, shape).astype(dtype)
        b = r.integers(-1000, 1000, shape).astype(dtype)
    else:
        a = r.standard_normal(shape).astype(dtype)
        b = r.standard_normal(shape).astype(dtype)
    for op, oop in ((_lib.ADD, O.ADD), (_lib.SUB, O.SUB), (_lib.MUL, O.MUL)):
        got = host(nt.Tensor._new_contiguous(K.binary(op, dev_T(a), dev_T(b)), shape))
        assert_bitexact(got, O.binary(oop, a, b), f"{op} .T .T")
        got = host(nt.Tensor._new_contiguous(K.binary(op, dev_T(a), dev(b)), shape))
        assert_bitexact(got, O.binary(oop, a, b), f"{op} .T contiguous")
    got = host(nt.Tensor._new_contiguous(K.unary(_lib.NEG, dev_T(a), 0.0), shape))
    assert_bitexact(got, O.unary(O.NEG, a, 0.0), "neg .T")
    got = host(nt.Tensor._new_contiguous(K.binary(_lib.GT, dev_T(a), dev(b)), shape))
    assert_bitexact(got, a > b, "gt .T")
    for dst in (np.float32, np.float64, np.int64):
        if np.dtype(dst) == np.dtype(dtype):
            continue
        out = dev(np.zeros(shape, dst))
        K.copy_view(dev_T(a), out)
        assert_bitexact(host(out), O.cast(a, dst), f"cast .T {np.dtype(dtype).name}->{np.dtype(dst).name}")


# ------------------------------------------------------------ config 2 size


C2_UNARY = {n: (op, oop, chain, dom, saved) for n, op, oop, chain, dom, saved in UNARY_BWD}
C2_OPS = ["add", "sub", "mul", "div", "neg", "exp", "log", "sqrt", "pow", "relu", "sigmoid", "tanh"]


@pytest.mark.parametrize("layout", ["contig", "transposed"])
@pytest.mark.parametrize("name", C2_OPS)
def test_config2_full_size(gpu, name, layout):
    """Config 2 at its size, [4096, 4096] (2^24 elements), laid out as the
    sweep runs it: every tensor input contiguous, or every tensor input a
    `.T` view (the accumulation targets too); upstream g contiguous.  Forward,
    then the fused backward in accumulate mode (old + new), against the
    oracle; the saved tensor is the oracle's (kernel parity), contiguous like
    a forward output, or the input view itself where the op saves its input."""
    r = rng(seed_of("c2", name, layout))
    shape = (4096, 4096)
    g = r.standard_normal(shape).astype(np.float32)
    tg = dev(g)
    if name in ("add", "sub", "mul", "div"):
        op, oop = {"add": (_lib.ADD, O.ADD), "sub": (_lib.SUB, O.SUB),
                   "mul": (_lib.MUL, O.MUL), "div": (_lib.DIV, O.DIV)}[name]
        a = r.standard_normal(shape).astype(np.float32)
        b = (r.uniform(0.5, 2, shape) if name == "div" else r.standard_normal(shape)).astype(np.float32)
        xa, xb = _mk(a, layout), _mk(b, layout)
        got = host(nt.Tensor._new_contiguous(K.binary(op, xa, xb), shape))
        assert_bitexact(got, O.binary(oop, a, b), f"{name} fwd 2^24 {layout}")
        olds = [r.standard_normal(shape).astype(np.float32) for _ in range(2)]
        tgts = [_mk(o, layout) for o in olds]
        K.binary_bwd(op, tg, xa, xb, True, tgts[0], True, tgts[1])
        for i, w in enumerate(O.bwd_binary(oop, g, a, b)):
            want = O.accumulate(olds[i], w)
            if name == "div" and i == 1:
                scale = np.abs(w).astype(np.float64) + np.abs(olds[i])
                assert_rel(host(tgts[i]), want, 1e-6, f"div grad 1 2^24 {layout}", scale=scale)
            else:
                assert_bitexact(host(tgts[i]), want, f"{name} grad {i} 2^24 {layout}")
        return
    op, oop, chain, dom, saved = C2_UNARY[name]
    e = 2.5 if name == "pow" else 0.0
    x = _inputs(r, dom, shape)
    xx = _mk(x, layout)
    got = host(nt.Tensor._new_contiguous(K.unary(op, xx, e), shape))
    want_y = O.unary(oop, x, e) if oop is not None else O.unary(O.NEG, x)
    if name in ("neg", "relu", "sqrt"):
        assert_bitexact(got, want_y, f"{name} fwd 2^24 {layout}")
    else:
        assert_rel(got, want_y, 1e-6, f"{name} fwd 2^24 {layout}")
    s = None if saved == "none" else (x if saved == "in" else want_y)
    sv = None if s is None else (xx if saved == "in" else dev(s))
    new = chain(g, s)
    old = r.standard_normal(shape).astype(np.float32)
    tgt = _mk(old, layout)
    K.unary_bwd(op, tg, sv, e, tgt)
    want = O.accumulate(old, new)
    if name in ("pow", "log", "sqrt", "tanh"):
        scale = np.abs(new).astype(np.float64)
        if name == "tanh":
            scale = np.abs(g).astype(np.float64) * (1 + s.astype(np.float64) ** 2)
        assert_rel(host(tgt), want, 1e-6, f"{name} bwd 2^24 {layout}", scale=scale + np.abs(old))
    else:
        assert_bitexact(host(tgt), want, f"{name} bwd 2^24 {layout}")


# ------------------------------------------------- pow exponent fast paths

POW_EXPONENTS = [0.0, -0.0, 1.0, 2.0, 3.0, 4.0, -1.0, -2.0, -3.0, -4.0, 0.5, 1.5,
                 2.5, 3.5, 4.5, -0.5, -1.5, -2.5, -4.5, 5.0, 6.5, 1.25, -7.3]


def _pow_inputs(dtype):
    """Normal values over a wide range of both signs, then every special
    class pow distinguishes: +-0, +-inf, NaN, subnormals, values whose
    small powers overflow or underflow, and +-1."""
    r = rng(seed_of("pow-special", np.dtype(dtype).name))
    fi = np.finfo(dtype)
    mags = np.exp(r.uniform(np.log(1e-6), np.log(1e6), 4000))
    vals = np.concatenate([mags, -mags[:1000], r.uniform(0.1, 4, 1000)])
    special = [0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, fi.tiny, -fi.tiny,
               fi.tiny / 8, -fi.tiny / 8, fi.max, -fi.max, fi.max ** 0.25,
               fi.max ** 0.3, fi.tiny ** 0.25, fi.tiny ** 0.2, 2.0, 0.5]
    return np.concatenate([vals, np.array(special)]).astype(dtype)


def _assert_pow_close(got, want, rel, what):
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"{what}: NaN positions differ at {np.nonzero(gn != wn)[0][:5]}"
    g, w = got[~gn].astype(np.float64), want[~wn].astype(np.float64)
    inf = np.isinf(w) | np.isinf(g)
    assert np.array_equal(g[inf], w[inf]), f"{what}: infinities differ"
    g, w = g[~inf], w[~inf]
    sub = float(np.finfo(got.dtype).smallest_subnormal)
    err = np.abs(g - w)
    bad = err > rel * np.abs(w) + 2 * sub
    if bad.any():
        i = int(np.argmax(np.where(bad, err / np.maximum(np.abs(w), 1e-300), 0)))
        raise AssertionError(f"{what}: {int(bad.sum())} outside rel {rel}; "
                             f"got {g[i]!r} want {w[i]!r}")
    assert np.array_equal(np.signbit(g), np.signbit(w)), f"{what}: signs differ"


@pytest.mark.parametrize("dtype,rel", [(np.float32, 1e-6), (np.float64, 1e-14)])
@pytest.mark.parametrize("e", POW_EXPONENTS)
def test_pow_exponent_classes(gpu, e, dtype, rel):
    """Integer and half-integer exponents with |e| <= 4.5 take the
    multiply/sqrt path, the rest the library pow; both must agree with the
    host pow (glibc) on normal values and reproduce its special values."""
    a = _pow_inputs(dtype)
    got = host(nt.Tensor._new_contiguous(K.unary(_lib.POW, dev(a), e), a.shape))
    with np.errstate(over="ignore", divide="ignore", invalid="ignore"):
        # the inputs include extreme and special values on purpose
        want = O.unary(O.POW, a, e) if dtype == np.float32 else np.power(a, dtype(e))
    _assert_pow_close(got, want, rel, f"pow e={e} {np.dtype(dtype).name}")


@pytest.mark.parametrize("e", [2.0, 3.0, 1.5, 0.5, -1.0, -0.5, 4.5, 1.0])
def test_pow_backward_exponent_classes(gpu, e):
    """Backward evaluates pow(x, e - 1): the exponents above land on each
    fast-path class (and e = 1 on x**0)."""
    a = _pow_inputs(np.float32)
    g = rng(seed_of("pow-bwd", e)).standard_normal(a.shape).astype(np.float32)
    want = O.bwd_pow(g, a, e)
    got = host(nt.Tensor._new_contiguous(K.unary_bwd(_lib.POW, dev(g), dev(a), e, None),
                                         a.shape))
    _assert_pow_close(got, want, 1e-6, f"pow bwd e={e}")


@pytest.mark.parametrize("R", [1, 2, 3, 7, 8, 255, 256])
@pytest.mark.parametrize("C", [4, 1024, 4100])
def test_broadcast_rows_kernel(gpu, R, C):
    """Contiguous [R, C] results with a broadcast row (bias: strides (0, 1)),
    a broadcast column (strides (s, 0)) and a scalar, even and odd row
    counts (the row-broadcast kernel takes two rows per work-item when R
    is even), forward and accumulate, against the oracle, bit-exact."""
    r = rng(seed_of("rows", R, C))
    a = r.standard_normal((R, C)).astype(np.float32)
    row = r.standard_normal(C).astype(np.float32)
    col = r.standard_normal(R).astype(np.float32)
    xa = dev(a)
    got = host(xa + dev(row))
    assert_bitexact(got, O.binary(O.ADD, a, np.broadcast_to(row, (R, C))), "bias")
    got = host(xa * dev(col.reshape(R, 1)).expand(R, C))
    assert_bitexact(got, O.binary(O.MUL, a, np.broadcast_to(col.reshape(R, 1), (R, C))), "column")
    old = r.standard_normal((R, C)).astype(np.float32)
    tgt = dev(old)
    K.inplace(_lib.ADD, tgt, dev(row).reshape(1, C).expand(R, C))
    assert_bitexact(host(tgt), O.accumulate(old, np.ascontiguousarray(np.broadcast_to(row, (R, C)))),
                    "accumulate row")
    tgt = dev(old)
    K.inplace(_lib.ADD, tgt, dev(col).reshape(R, 1).expand(R, C))
    assert_bitexact(host(tgt), O.accumulate(old, np.ascontiguousarray(np.broadcast_to(col.reshape(R, 1), (R, C)))),
                    "accumulate column")
