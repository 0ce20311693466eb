"""Seeded random cases through the elementwise engine, the reductions and
matmul: operand layouts drawn from contiguous, `.T`, broadcast row,
broadcast column, scalar, every-other-column slice and one-element-offset
views, on shapes with and without 4-aligned sides, so that every launch
path (flat, rows, the tile kernels in each tile shape and orientation,
generic; every matmul kernel and split-K) is crossed with the others and
with partial tiles.  Each result is compared with the oracle on the same
logical arrays: bit-exact for + - * / and the exact unary ops, the backward
kernels' accumulation and max/min/argmax; sums within 1e-5 * sum|x|;
products within 1e-4 * (|A|.|B|)_ij.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from helpers import assert_bitexact, assert_rel, dev, dev_T, host, rng

import nanotorch_amd as nt
from nanotorch_amd import _kernels as K
from nanotorch_amd import _lib

pytestmark = pytest.mark.gpu

KINDS = ["contig", "T", "row", "col", "scalar", "slice", "offset"]
SIDES = [1, 3, 4, 7, 16, 60, 64, 65, 100, 128, 132, 200, 257]


def _values(r, shape, positive=False):
    v = r.standard_normal(shape).astype(np.float32)
    if positive:
        v = (np.abs(v) + 0.5).astype(np.float32)
    return v


def _operand(r, shape, kind, positive=False):
    """(device view, logical numpy array) of `shape` laid out as `kind`."""
    R, C = shape
    if kind == "T":
        a = _values(r, shape, positive)
        return dev_T(a), a
    if kind == "row":
        row = _values(r, (C,), positive)
        return dev(row).expand(R, C), np.ascontiguousarray(np.broadcast_to(row, shape))
    if kind == "col":
        col = _values(r, (R, 1), positive)
        return dev(col).expand(R, C), np.ascontiguousarray(np.broadcast_to(col, shape))
    if kind == "scalar":
        s = _values(r, (1, 1), positive)
        return dev(s).expand(R, C), np.ascontiguousarray(np.broadcast_to(s, shape))
    if kind == "slice":
        big = _values(r, (R, 2 * C), positive)
        return dev(big)[:, ::2], np.ascontiguousarray(big[:, ::2])
    if kind == "offset":
        flat = _values(r, (R * C + 1,), positive)
        return dev(flat)[1:].reshape(R, C), flat[1:].reshape(R, C)
    a = _values(r, shape, positive)
    return dev(a), a


def _target(r, shape, kind):
    """A writable gradient target: contiguous or a `.T` view."""
    a = _values(r, shape)
    return (dev_T(a) if kind == "T" else dev(a)), a


@pytest.mark.parametrize("case", range(60))
def test_random_binary_and_unary(gpu, case):
    r = rng(1000 + case)
    shape = (int(r.choice(SIDES)), int(r.choice(SIDES)))
    ka, kb = str(r.choice(KINDS)), str(r.choice(KINDS))
    xa, a = _operand(r, shape, ka)
    for op, oop in ((_lib.ADD, O.ADD), (_lib.SUB, O.SUB), (_lib.MUL, O.MUL), (_lib.DIV, O.DIV)):
        xb, b = _operand(r, shape, kb, positive=(op == _lib.DIV))
        got = host(nt.Tensor._new_contiguous(K.binary(op, xa, xb), shape))
        assert_bitexact(got, O.binary(oop, a, b), f"case {case} op {op} {ka}/{kb} {shape}")
    for op, oop in ((_lib.NEG, O.NEG), (_lib.RELU, O.RELU)):
        got = host(nt.Tensor._new_contiguous(K.unary(op, xa, 0.0), shape))
        assert_bitexact(got, O.unary(oop, a, 0.0), f"case {case} unary {op} {ka} {shape}")


@pytest.mark.parametrize("case", range(40))
def test_random_fused_backward(gpu, case):
    """mul backward into two gradient targets (contiguous or `.T`), and the
    exp backward from a saved output, accumulating; operands of any
    layout."""
    r = rng(2000 + case)
    shape = (int(r.choice(SIDES)), int(r.choice(SIDES)))
    kg, ka, kb = (str(r.choice(KINDS)) for _ in range(3))
    ta_kind, tb_kind = str(r.choice(["contig", "T"])), str(r.choice(["contig", "T"]))
    xg, g = _operand(r, shape, kg)
    xa, a = _operand(r, shape, ka)
    xb, b = _operand(r, shape, kb)
    tga, olda = _target(r, shape, ta_kind)
    tgb, oldb = _target(r, shape, tb_kind)
    K.binary_bwd(_lib.MUL, xg, xa, xb, True, tga, True, tgb)
    wa, wb = O.bwd_binary(O.MUL, g, a, b)
    tag = f"case {case} g={kg} a={ka} b={kb} ta={ta_kind} tb={tb_kind} {shape}"
    assert_bitexact(host(tga), O.accumulate(olda, wa), "mul bwd a " + tag)
    assert_bitexact(host(tgb), O.accumulate(oldb, wb), "mul bwd b " + tag)
    y = O.unary(O.EXP, a, 0.0)
    ky = str(r.choice(["contig", "T"]))
    sy = dev_T(y) if ky == "T" else dev(y)
    t, old = _target(r, shape, str(r.choice(["contig", "T"])))
    K.unary_bwd(_lib.EXP, xg, sy, 0.0, t)
    assert_bitexact(host(t), O.accumulate(old, O.bwd_exp(g, y)), "exp bwd " + tag)


@pytest.mark.parametrize("case", range(40))
def test_random_reductions(gpu, case):
    """sum / max / argmax over random axis sets of 2-D and 3-D contiguous,
    transposed and sliced views."""
    r = rng(3000 + case)
    nd = int(r.choice([2, 3]))
    sizes = [1, 2, 5, 31, 64, 100, 257, 1030, 4100] if nd == 2 else [1, 2, 5, 31, 64, 100, 257]
    shape = tuple(int(r.choice(sizes)) for _ in range(nd))
    base = r.integers(-50, 51, shape).astype(np.float32)
    kind = str(r.choice(["contig", "T", "slice"]))
    if kind == "T":
        x = dev(np.ascontiguousarray(np.swapaxes(base, 0, -1))).transpose(0, nd - 1)
        a = base
    elif kind == "slice":
        big = np.repeat(base, 2, axis=-1)
        x, a = dev(big)[..., ::2], big[..., ::2]
    else:
        x, a = dev(base), base
    naxes = int(r.integers(1, nd + 1))
    axes = tuple(int(v) for v in r.permutation(nd)[:naxes])
    kshape = tuple(s for i, s in enumerate(shape) if i not in axes)
    tag = f"case {case} {shape} {kind} axes={axes}"
    got = host(nt.Tensor._new_contiguous(K.reduce(_lib.R_SUM, x, axes, nt.float32), kshape))
    want = O.reduce(O.R_SUM, a, axes, np.float32)
    scale = O.reduce(O.R_SUM, np.abs(a).astype(np.float64), axes, np.float64)
    assert_rel(got, want, 1e-5, "sum " + tag, scale=scale)
    v, idx, cnt = K.reduce(_lib.R_MAX, x, axes, nt.float32, want_aux=True)
    assert_bitexact(host(nt.Tensor._new_contiguous(v, kshape)), O.reduce(O.R_MAX, a, axes), "max " + tag)
    assert_bitexact(host(nt.Tensor._new_contiguous(idx, kshape)), O.reduce(O.R_ARGMAX, a, axes), "argmax " + tag)


@pytest.mark.parametrize("case", range(30))
def test_random_matmul(gpu, case):
    """Products of random sizes (ragged, multiples of 4, of 32 and of 256, so
    that every matmul kernel and split-K are chosen), each operand
    contiguous, transposed or a column slice, an optional batch, written
    fresh or accumulated into a contiguous or `.T` target; within
    1e-4 * (|A|.|B|)_ij of the oracle's sequential product."""
    r = rng(4000 + case)
    dims = [1, 3, 4, 32, 96, 100, 256, 260, 512, 1024]
    M, Kd, N = (int(r.choice(dims)) for _ in range(3))
    if M * N * Kd > 1024 * 1024 * 256:
        Kd = 64
    batch = int(r.choice([1, 1, 3]))
    a = r.standard_normal((batch, M, Kd)).astype(np.float32)
    b = (r.standard_normal((batch, Kd, N)) / np.sqrt(Kd)).astype(np.float32)

    def place(v, kind):
        if kind == "T":
            return dev(np.ascontiguousarray(np.swapaxes(v, 1, 2))).transpose(1, 2)
        if kind == "slice":
            big = np.repeat(v, 2, axis=2)
            return dev(big)[:, :, ::2]
        return dev(v)

    ka, kb = str(r.choice(["contig", "T", "slice"])), str(r.choice(["contig", "T", "slice"]))
    xa, xb = place(a, ka), place(b, kb)
    want = np.stack([O.matmul(a[i], b[i], parallel=True) for i in range(batch)])
    scale = np.stack([O.matmul(np.abs(a[i]).astype(np.float64), np.abs(b[i]).astype(np.float64),
                               parallel=True) for i in range(batch)])
    tag = f"case {case} {batch}x{M}x{Kd}x{N} a={ka} b={kb}"
    if r.random() < 0.5:
        out_shape = (batch, M, N)
        got = host(nt.Tensor._new_contiguous(K.matmul(xa, xb, out_shape), out_shape))
        assert_rel(got, want, 1e-4, "fresh " + tag, scale=scale)
    else:
        old = r.standard_normal((batch, M, N)).astype(np.float32)
        kt = str(r.choice(["contig", "T"]))
        tgt = place(old, kt) if kt == "T" else dev(old)
        K.matmul_into(xa, xb, tgt, accumulate=True)
        assert_rel(host(tgt), want + old, 1e-4, f"accumulate into {kt} " + tag,
                   scale=scale + np.abs(old))


PERMS = [(0, 2, 1), (2, 1, 0), (1, 0, 2), (1, 2, 0), (2, 0, 1)]


def _permute(t, perm):
    """The view of t whose axis i is t's axis perm[i], by transposes."""
    cur = list(range(len(perm)))
    for i, want in enumerate(perm):
        j = cur.index(want)
        if j != i:
            t = t.transpose(i, j)
            cur[i], cur[j] = cur[j], cur[i]
    return t


@pytest.mark.parametrize("case", range(40))
def test_random_3d_permutes(gpu, case):
    """Copies, binary ops and the mul backward on permuted 3-D views (a
    batch of 2-D planes for the tile kernel when the unit strides share a
    plane, the generic kernel otherwise), against numpy's transpose."""
    r = rng(5000 + case)
    sides = [1, 3, 4, 8, 12, 64, 65, 128, 132]
    base_shape = tuple(int(r.choice(sides)) for _ in range(3))
    pa, pb = PERMS[int(r.integers(len(PERMS)))], PERMS[int(r.integers(len(PERMS)))]
    a0 = r.standard_normal(base_shape).astype(np.float32)
    xa = _permute(dev(a0), pa)
    a = np.ascontiguousarray(a0.transpose(pa))
    shape = a.shape
    # b: stored so that its permutation pb gives the logical shape of a
    inv = np.argsort(pb)
    b0 = r.standard_normal(tuple(shape[i] for i in inv)).astype(np.float32)
    xb = _permute(dev(b0), pb)
    b = np.ascontiguousarray(b0.transpose(pb))
    assert b.shape == shape
    tag = f"case {case} base {base_shape} perms {pa} {pb}"
    out = dev(np.zeros(shape, np.float32))
    K.copy_view(xa, out)
    assert_bitexact(host(out), a, "copy " + tag)
    for op, oop in ((_lib.ADD, O.ADD), (_lib.MUL, O.MUL)):
        got = host(nt.Tensor._new_contiguous(K.binary(op, xa, xb), shape))
        assert_bitexact(got, O.binary(oop, a, b), f"op {op} " + tag)
    g = r.standard_normal(shape).astype(np.float32)
    olds = [r.standard_normal(shape).astype(np.float32) for _ in range(2)]
    # gradient targets laid out like the operands
    ta = _permute(dev(np.ascontiguousarray(olds[0].transpose(np.argsort(pa)))), pa)
    tb = dev(olds[1])
    K.binary_bwd(_lib.MUL, dev(g), xa, xb, True, ta, True, tb)
    wa, wb = O.bwd_binary(O.MUL, g, a, b)
    assert_bitexact(host(ta), O.accumulate(olds[0], wa), "mul bwd a " + tag)
    assert_bitexact(host(tb), O.accumulate(olds[1], wb), "mul bwd b " + tag)


@pytest.mark.parametrize("case", range(30))
def test_random_3d_permute_reductions(gpu, case):
    """sum / max / min / argmax / argmin, the counts and the max/min
    backward of permuted 3-D views over axis tuples in random order (the
    reduced index follows the tuple's order), small integers so that ties
    occur: the first index must win and a tied slice routes no gradient."""
    r = rng(6000 + case)
    sides = [1, 2, 3, 8, 17, 64, 65, 130]
    base_shape = tuple(int(r.choice(sides)) for _ in range(3))
    perm = PERMS[int(r.integers(len(PERMS)))]
    # |values| <= 3: every partial sum of at most 130^3 of them is an
    # integer below 2^24, exact in fp32 whatever the summation order
    a0 = r.integers(-3, 4, base_shape).astype(np.float32)
    x = _permute(dev(a0), perm)
    a = np.ascontiguousarray(a0.transpose(perm))
    naxes = int(r.integers(1, 4))
    axes = tuple(int(v) for v in r.permutation(3)[:naxes])
    kshape = tuple(s for i, s in enumerate(a.shape) if i not in axes)
    tag = f"case {case} base {base_shape} perm {perm} axes={axes}"
    got = host(nt.Tensor._new_contiguous(K.reduce(_lib.R_SUM, x, axes, nt.float32), kshape))
    assert_bitexact(got, O.reduce(O.R_SUM, a, axes, np.float32), "sum " + tag)
    shape = a.shape
    gshape = tuple(1 if i in axes else d for i, d in enumerate(shape))
    g = r.standard_normal(kshape).astype(np.float32)
    for op, oop, aop in ((_lib.R_MAX, O.R_MAX, O.R_ARGMAX), (_lib.R_MIN, O.R_MIN, O.R_ARGMIN)):
        v, idx, cnt = K.reduce(op, x, axes, nt.float32, want_aux=True)
        assert_bitexact(host(nt.Tensor._new_contiguous(v, kshape)), O.reduce(oop, a, axes),
                        f"{op} value " + tag)
        assert_bitexact(host(nt.Tensor._new_contiguous(idx, kshape)), O.reduce(aop, a, axes),
                        f"{op} index " + tag)
        ext = O.reduce(oop, a, axes).reshape(gshape)
        want_cnt = (a == ext).sum(axis=axes).astype(np.int32).reshape(kshape)
        assert_bitexact(host(nt.Tensor._new_contiguous(cnt, kshape)), want_cnt, f"{op} count " + tag)
        # backward: g routed to the single extremum of each slice, 0 for a
        # slice with ties; into a new buffer, then accumulated into a target
        # laid out like x (permuted)
        want = O.sel_bwd(oop, g, a, axes)
        st = K.reduce_bwd(op, dev(g), 1.0, idx, cnt, axes, shape, None)
        assert_bitexact(host(nt.Tensor._new_contiguous(st, shape)), want, f"{op} bwd " + tag)
        old0 = r.standard_normal(base_shape).astype(np.float32)
        tgt = _permute(dev(old0), perm)
        K.reduce_bwd(op, dev(g), 1.0, idx, cnt, axes, shape, tgt)
        old = np.ascontiguousarray(old0.transpose(perm))
        assert_bitexact(host(tgt), O.accumulate(old, want), f"{op} bwd acc " + tag)


_DTS = [np.int32, np.int64, np.float32, np.float64]  # the reference's order


@pytest.mark.parametrize("case", range(24))
def test_random_mixed_dtype_binary(gpu, case):
    """Binary ops and comparisons between tensors of different dtypes, in
    either layout: the Python layer promotes to max(dtype) (int32 < int64 <
    float32 < float64) and casts with the reference's static_cast (large
    int64 values round to float32), then the device kernel runs; against
    numpy's casts and the oracle in the promoted dtype."""
    r = rng(8800 + case)
    shape = (int(r.choice([1, 7, 64, 257])), int(r.choice([1, 5, 64, 130])))
    i, j = int(r.integers(4)), int(r.integers(4))
    name = str(r.choice(["add", "sub", "mul", "gt", "ge", "eq"]))
    big = 2**40 if name != "mul" else 2**15  # int64 sums past float32's 24 bits
    def draw(dt):
        if dt == np.int32:
            return r.integers(-2**15, 2**15, shape).astype(np.int32)
        if dt == np.int64:
            return r.integers(-big, big, shape).astype(np.int64)
        return (r.standard_normal(shape) * 100).astype(dt)
    a, b = draw(_DTS[i]), draw(_DTS[j])
    if name in ("gt", "ge", "eq"):
        b[::2] = a[::2].astype(b.dtype)  # some equal pairs (after the cast)
    xa = dev(a) if r.random() < 0.5 else dev_T(a)
    xb = dev(b) if r.random() < 0.5 else dev_T(b)
    pd = _DTS[max(i, j)]
    ops = {"add": (lambda p, q: p + q, O.ADD), "sub": (lambda p, q: p - q, O.SUB),
           "mul": (lambda p, q: p * q, O.MUL), "gt": (lambda p, q: p > q, O.GT),
           "ge": (lambda p, q: p >= q, O.GE), "eq": (lambda p, q: p == q, O.EQ)}
    fn, oop = ops[name]
    got = host(fn(xa, xb))
    want = O.binary(oop, a.astype(pd), b.astype(pd))
    assert_bitexact(got, want, f"case {case} {name} {a.dtype}/{b.dtype} {shape}")


_CAST_DTS = [(np.bool_, nt.bool_), (np.int32, nt.int32), (np.int64, nt.int64),
             (np.float32, nt.float32), (np.float64, nt.float64)]


@pytest.mark.parametrize("case", range(20))
def test_random_device_casts(gpu, case):
    """Tensor.to(dtype) on the device from contiguous, .T and sliced views,
    every pair of dtypes: the reference's Storage::cast (static_cast; to bool
    s != 0, so NaN and -0.0 map as C++ does), values kept inside the target
    range; against numpy's C casts."""
    r = rng(9100 + case)
    shape = (int(r.choice([1, 6, 64, 130])), int(r.choice([1, 3, 64, 257])))
    (snp, _), (dnp, dnt) = (_CAST_DTS[int(r.integers(5))], _CAST_DTS[int(r.integers(5))])
    if snp == np.bool_:
        a = r.random(shape) < 0.5
    elif np.issubdtype(snp, np.integer):
        a = r.integers(-3000, 3000, shape).astype(snp)
        a[0, 0] = 0
    else:
        a = (r.standard_normal(shape) * 1000).astype(snp)
        a.flat[0] = -0.0
        if dnp == np.bool_:
            a.flat[-1] = np.nan  # static_cast<bool>(NaN) is true
    kind = str(r.choice(["contig", "T", "slice"]))
    if kind == "T":
        x = dev_T(a)
    elif kind == "slice":
        big = np.repeat(a, 2, axis=1)
        x, a = dev(big)[:, ::2], big[:, ::2]
    else:
        x = dev(a)
    got = host(x.to(dnt))
    want = (a != 0) if dnp == np.bool_ else a.astype(dnp)
    assert_bitexact(got, np.asarray(want, dtype=dnp), f"case {case} {a.dtype}->{np.dtype(dnp)} {kind} {shape}")


def _writable(r, shape, kind):
    """(device view, numpy copy of it, device base, numpy copy of the base,
    the base elements the view does not cover) of a writable target laid
    out as `kind`."""
    R, C = shape
    if kind == "T":
        a = _values(r, shape)
        d = dev_T(a)
        return d, a.copy(), d, a.copy(), lambda full: full[:0]
    if kind == "slice":
        big = _values(r, (R, 2 * C))
        d = dev(big)
        return d[:, ::2], np.ascontiguousarray(big[:, ::2]), d, big.copy(), lambda full: full[:, 1::2]
    if kind == "offset":
        flat = _values(r, (R * C + 1,))
        d = dev(flat)
        return d[1:].reshape(R, C), flat[1:].reshape(R, C).copy(), d, flat.copy(), lambda full: full[:1]
    a = _values(r, shape)
    d = dev(a)
    return d, a.copy(), d, a.copy(), lambda full: full[:0]


@pytest.mark.parametrize("case", range(24))
def test_random_inplace_on_views(gpu, case):
    """out op= other with out a contiguous, .T, sliced or misaligned view and
    other in any of the seven layouts (broadcasts included): the in-place
    kernels write through strided targets (tile and flat kernels, one output
    that is also an input); the elements outside the view stay untouched."""
    r = rng(9400 + case)
    shape = (int(r.choice(SIDES)), int(r.choice(SIDES)))
    tk = str(r.choice(["contig", "T", "slice", "offset"]))
    ok = str(r.choice(KINDS))
    name = str(r.choice(["add", "sub", "mul", "div"]))
    out, want, base, base_np, untouched = _writable(r, shape, tk)
    other, b = _operand(r, shape, ok, positive=(name == "div"))
    oop = {"add": O.ADD, "sub": O.SUB, "mul": O.MUL, "div": O.DIV}[name]
    with nt.no_grad():
        if name == "add":
            out += other
        elif name == "sub":
            out -= other
        elif name == "mul":
            out *= other
        else:
            out /= other
    O.inplace(oop, want, b)
    tag = f"case {case} {name} out {tk} other {ok} {shape}"
    assert_bitexact(host(out), want, tag)
    assert_bitexact(np.ascontiguousarray(untouched(host(base))),
                    np.ascontiguousarray(untouched(base_np)), "outside the view " + tag)
