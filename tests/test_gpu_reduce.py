"""Reductions on the GPU against the oracle (reference CPU loops).

Bar: max/min values, argmax/argmin indices, tie counts and the max/min
backward routing are bit-exact; sums/means satisfy
|gpu - ref| <= 1e-5 * sum|x| per output (the reference sums sequentially in
fp32, the GPU in a tree; both are within that bound of the exact sum).
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

SHAPES_AXES = [
    ((6,), (0,)),
    ((1,), (0,)),
    ((3, 5), (0,)),
    ((3, 5), (1,)),
    ((3, 5), (0, 1)),
    ((3, 5), (1, 0)),
    ((257, 1000), (1,)),
    ((1000, 257), (0,)),
    ((64, 4096), (1,)),
    ((4096, 64), (0,)),
    ((300, 2050), (0,)),
    ((513, 4096), (0,)),
    ((33, 1030), (0,)),
    ((10, 2, 5, 1), (1, 3)),
    ((10, 2, 5, 1), (3, 1)),
    ((7, 9, 11), (0, 2)),
    ((7, 9, 11), (2,)),
    ((5, 300, 7), (1,)),
    ((100003,), (0,)),
]

VIEWS = ["contig", "transposed", "strided"]


def _view(a, kind):
    if kind == "contig" or a.ndim < 2:
        return dev(a), a
    if kind == "transposed":
        t = dev(np.ascontiguousarray(np.swapaxes(a, 0, -1)))
        return t.transpose(0, a.ndim - 1), a
    big = np.repeat(a, 2, axis=-1)
    return dev(big)[..., ::2], big[..., ::2]


def _sum_bound(a, axes):
    return O.reduce(O.R_SUM, np.abs(a).astype(np.float64), axes, np.float64)


@pytest.mark.parametrize("view", VIEWS)
@pytest.mark.parametrize("shape,axes", SHAPES_AXES)
def test_reduce_forward(gpu, shape, axes, view):
    r = rng(seed_of(shape, axes, view))
    a = r.standard_normal(shape).astype(np.float32)
    x, a_view = _view(a, view)
    kshape = tuple(s for i, s in enumerate(shape) if i not in axes)
    # sum
    got = host(nt.Tensor._new_contiguous(K.reduce(_lib.R_SUM, x, axes, nt.float32), kshape))
    want = O.reduce(O.R_SUM, a_view, axes, np.float32)
    assert_rel(got, want, 1e-5, "sum", scale=_sum_bound(a_view, axes))
    # max / min with idx + count
    for op, oop, aop in ((_lib.R_MAX, O.R_MAX, O.R_ARGMAX), (_lib.R_MIN, O.R_MIN, O.R_ARGMIN)):
        v, idx, cnt = K.reduce(op, x, axes, nt.float32, want_aux=True)
        assert_bitexact(host(nt.Tensor._new_contiguous(v, kshape)), O.reduce(oop, a_view, axes), "max/min")
        assert_bitexact(host(nt.Tensor._new_contiguous(idx, kshape)), O.reduce(aop, a_view, axes), "idx")
    for op, oop in ((_lib.R_ARGMAX, O.R_ARGMAX), (_lib.R_ARGMIN, O.R_ARGMIN)):
        got = host(nt.Tensor._new_contiguous(K.reduce(op, x, axes, nt.int64), kshape))
        assert_bitexact(got, O.reduce(oop, a_view, axes), "argmax/argmin")


def test_ties_first_index_and_count(gpu):
    a = np.array([0.0, -1.5, -1.5, 8, 8, 3], dtype=np.float32)
    v, idx, cnt = K.reduce(_lib.R_MAX, dev(a), (0,), nt.float32, want_aux=True)
    assert host(nt.Tensor._new_contiguous(idx, ())) == 3
    assert host(nt.Tensor._new_contiguous(cnt, ())) == 2
    v, idx, cnt = K.reduce(_lib.R_MIN, dev(a), (0,), nt.float32, want_aux=True)
    assert host(nt.Tensor._new_contiguous(idx, ())) == 1
    # many ties spread over workgroups and segments
    r = rng(1)
    b = r.integers(0, 4, (64, 100000)).astype(np.float32)
    for axes in ((1,), (0,)):
        kshape = (64,) if axes == (1,) else (100000,)
        _, idx, cnt = K.reduce(_lib.R_MAX, dev(b), axes, nt.float32, want_aux=True)
        assert_bitexact(host(nt.Tensor._new_contiguous(idx, kshape)), O.reduce(O.R_ARGMAX, b, axes), "tie idx")
        m = b.max(axis=axes[0], keepdims=True)
        want_cnt = (b == m).sum(axis=axes[0]).astype(np.int32)
        assert_bitexact(host(nt.Tensor._new_contiguous(cnt, kshape)), want_cnt, "tie count")


@pytest.mark.parametrize("dtype", [np.float64, np.int32, np.int64, np.bool_])
def test_reduce_other_dtypes(gpu, dtype):
    r = rng(2)
    a = (r.standard_normal((37, 53)) * 100).astype(dtype) if dtype != np.bool_ else (
        r.integers(0, 2, (37, 53)).astype(bool))
    for axes in ((0,), (1,), (0, 1)):
        kshape = tuple(s for i, s in enumerate(a.shape) if i not in axes)
        out_dt = np.int64 if dtype in (np.int32, np.int64, np.bool_) else dtype
        got = host(nt.Tensor._new_contiguous(
            K.reduce(_lib.R_SUM, dev(a), axes, nt.Tensor(np.zeros(1, out_dt)).dtype), kshape))
        want = O.reduce(O.R_SUM, a, axes, out_dt)
        if dtype == np.float64:
            assert_rel(got, want, 1e-12, "f64 sum", scale=_sum_bound(a, axes))
        else:
            assert_bitexact(got, want, "int sum")
        for op, oop in ((_lib.R_MAX, O.R_MAX), (_lib.R_MIN, O.R_MIN), (_lib.R_ARGMAX, O.R_ARGMAX)):
            odt = nt.int64 if op == _lib.R_ARGMAX else dev(a).dtype
            got = host(nt.Tensor._new_contiguous(K.reduce(op, dev(a), axes, odt), kshape))
            assert_bitexact(got, O.reduce(oop, a, axes), f"{dtype} op {op}")


def test_sum_into_wider_dtype(gpu):
    a = rng(3).standard_normal((300, 500)).astype(np.float32)
    got = host(nt.Tensor._new_contiguous(K.reduce(_lib.R_SUM, dev(a), (1,), nt.float64), (300,)))
    want = O.reduce(O.R_SUM, a, (1,), np.float64)
    assert_rel(got, want, 1e-12, "f32->f64 sum", scale=_sum_bound(a, (1,)))


# --------------------------------------------------------------- backward


@pytest.mark.parametrize("acc", [False, True])
@pytest.mark.parametrize("shape,axes", [((300, 200), (0,)), ((300, 200), (1,)),
                                        ((300, 200), (0, 1)), ((4, 6, 8), (2, 0))])
@pytest.mark.parametrize("op", ["max", "min"])
def test_select_backward(gpu, op, shape, axes, acc):
    r = rng(seed_of(op, shape, axes, acc))
    a = r.integers(-20, 20, shape).astype(np.float32)  # plenty of ties
    a[0] = r.standard_normal(shape[1:]) if len(shape) > 1 else a[0]
    kshape = tuple(s for i, s in enumerate(shape) if i not in axes)
    g = r.standard_normal(kshape).astype(np.float32)
    nop = _lib.R_MAX if op == "max" else _lib.R_MIN
    oop = O.R_MAX if op == "max" else O.R_MIN
    _, idx, cnt = K.reduce(nop, dev(a), axes, nt.float32, want_aux=True)
    want = O.sel_bwd(oop, g, a, axes)
    old = r.standard_normal(shape).astype(np.float32)
    if acc:
        tgt = dev(old)
        K.reduce_bwd(nop, dev(g), 1.0, idx, cnt, axes, shape, tgt)
        got = host(tgt)
        want = O.accumulate(old, want)
    else:
        st = K.reduce_bwd(nop, dev(g), 1.0, idx, cnt, axes, shape, None)
        got = host(nt.Tensor._new_contiguous(st, shape))
    assert_bitexact(got, want, f"{op} bwd")


@pytest.mark.parametrize("acc", [False, True])
def test_mean_backward(gpu, acc):
    r = rng(5)
    shape, axes = (123, 77), (1,)
    g = r.standard_normal((123,)).astype(np.float32)
    n = 77
    # ops_reduction.py:129-138: expand(g) / denom
    want = O.binary(O.DIV, np.broadcast_to(g.reshape(123, 1), shape),
                    np.broadcast_to(O.scalar(n, np.float32), shape))
    old = r.standard_normal(shape).astype(np.float32)
    if acc:
        tgt = dev_T(old)
        K.reduce_bwd(_lib.R_MEAN, dev(g), float(n), None, None, axes, shape, tgt)
        assert_bitexact(host(tgt), O.accumulate(old, want), "mean bwd acc")
    else:
        st = K.reduce_bwd(_lib.R_MEAN, dev(g), float(n), None, None, axes, shape, None)
        assert_bitexact(host(nt.Tensor._new_contiguous(st, shape)), want, "mean bwd")


@pytest.mark.parametrize("axes", [(0,), (1,), (0, 1)])
def test_config3_full_size(gpu, axes):
    """Config 3 at its size, [8192, 8192] fp32 ~ N(0,1), along axis 0, axis 1
    and the full tensor: sum and mean within the condition-aware bound; max
    and min values, argmax / argmin indices and tie counts bit-exact; the
    backward of sum and mean (accumulate: old + broadcast(g) and
    old + broadcast(g) / n) bit-exact; max and min backward routing (first
    write and accumulate) bit-exact."""
    r = rng(seed_of("c3", axes))
    shape = (8192, 8192)
    a = r.standard_normal(shape).astype(np.float32)
    x = dev(a)
    kshape = tuple(s for i, s in enumerate(shape) if i not in axes)
    k = int(np.prod(kshape))
    n = a.size // k
    bound = _sum_bound(a, axes)
    got = host(nt.Tensor._new_contiguous(K.reduce(_lib.R_SUM, x, axes, nt.float32), kshape))
    want = O.reduce(O.R_SUM, a, axes, np.float32)
    assert_rel(got, want, 1e-5, "sum 2^26", scale=bound)
    # mean (ops_reduction.py:119-127): sum / float32(n), through the API
    got = host(nt.mean(x, axis=axes))
    assert_rel(got, O.mean_fwd(a, axes), 1e-5, "mean 2^26", scale=bound / n)
    g = r.standard_normal(kshape).astype(np.float32)
    gshape = tuple(1 if i in axes else s for i, s in enumerate(shape))
    gb = np.broadcast_to(g.reshape(gshape), shape)
    for op, oop, aop, name in ((_lib.R_MAX, O.R_MAX, O.R_ARGMAX, "max"),
                               (_lib.R_MIN, O.R_MIN, O.R_ARGMIN, "min")):
        v, idx, cnt = K.reduce(op, x, axes, nt.float32, want_aux=True)
        assert_bitexact(host(nt.Tensor._new_contiguous(v, kshape)), O.reduce(oop, a, axes), f"{name} 2^26")
        assert_bitexact(host(nt.Tensor._new_contiguous(idx, kshape)), O.reduce(aop, a, axes),
                        f"arg{name} 2^26")
        ext = O.reduce(oop, a, axes).reshape(gshape)
        want_cnt = (a == ext).sum(axis=axes).astype(np.int32).reshape(kshape)
        assert_bitexact(host(nt.Tensor._new_contiguous(cnt, kshape)), want_cnt, f"{name} count 2^26")
        want = O.sel_bwd(oop, g, a, axes)
        st = K.reduce_bwd(op, dev(g), 1.0, idx, cnt, axes, shape, None)
        assert_bitexact(host(nt.Tensor._new_contiguous(st, shape)), want, f"{name} bwd 2^26")
        old = r.standard_normal(shape).astype(np.float32)
        tgt = dev(old)
        K.reduce_bwd(op, dev(g), 1.0, idx, cnt, axes, shape, tgt)
        assert_bitexact(host(tgt), O.accumulate(old, want), f"{name} bwd acc 2^26")
    # sum backward (ops_reduction.py:67-74): broadcast(g), accumulated
    old = r.standard_normal(shape).astype(np.float32)
    tgt = dev(old)
    K.inplace(_lib.ADD, tgt, dev(g).reshape(*gshape).expand(*shape))
    assert_bitexact(host(tgt), O.accumulate(old, np.ascontiguousarray(gb)), "sum bwd acc 2^26")
    # mean backward (:129-138): broadcast(g) / float32(n), accumulated
    old = r.standard_normal(shape).astype(np.float32)
    tgt = dev(old)
    K.reduce_bwd(_lib.R_MEAN, dev(g), float(n), None, None, axes, shape, tgt)
    want = O.binary(O.DIV, gb, np.broadcast_to(O.scalar(n, np.float32), shape))
    assert_bitexact(host(tgt), O.accumulate(old, want), "mean bwd acc 2^26")


@pytest.mark.parametrize("D", [1, 2, 3, 4, 5, 7, 8, 9, 15, 16, 17, 31, 33, 64, 100, 257])
@pytest.mark.parametrize("K_", [2048, 1028])
def test_column_walk_row_counts(gpu, D, K_):
    """Max / min / sum along axis 0 of [D, K] for every small row count: the
    column walk's pipelined groups of rows (none, one, an odd or even
    number, a tail), its segment split and the wide (K >= 1024) and
    unaligned-width (K % 1024 != 0) column blocks; values, first indices
    and tie counts bit-exact (small integers: many ties)."""
    r = rng(seed_of("colwalk", D, K_))
    a = r.integers(-3, 4, (D, K_)).astype(np.float32)
    x = dev(a)
    for op, oop, aop in ((_lib.R_MAX, O.R_MAX, O.R_ARGMAX), (_lib.R_MIN, O.R_MIN, O.R_ARGMIN)):
        v, idx, cnt = K.reduce(op, x, (0,), nt.float32, want_aux=True)
        assert_bitexact(host(nt.Tensor._new_contiguous(v, (K_,))), O.reduce(oop, a, (0,)), f"{op} D={D}")
        assert_bitexact(host(nt.Tensor._new_contiguous(idx, (K_,))), O.reduce(aop, a, (0,)), f"arg {op} D={D}")
        want_cnt = (a == O.reduce(oop, a, (0,))[None, :]).sum(axis=0).astype(np.int32)
        assert_bitexact(host(nt.Tensor._new_contiguous(cnt, (K_,))), want_cnt, f"count {op} D={D}")
    got = host(nt.Tensor._new_contiguous(K.reduce(_lib.R_SUM, x, (0,), nt.float32), (K_,)))
    assert_bitexact(got, a.sum(axis=0).astype(np.float32), f"sum D={D}")  # small integers: exact


def test_split_slices_back_to_back(gpu):
    """Reductions whose slices are split over several workgroups (row and
    generic kernels), queued back to back with no host wait between them,
    so each launch's partials reuse memory that earlier launches with other
    slice and segment counts wrote.  Every result must be exact: small
    integers make fp32 sums exact and give max/min many ties."""
    r = rng(seed_of("split-slices"))
    cases = [
        ((1, 1 << 20), (1,)),       # row kernel, one slice in 256 segments
        ((3, 300001), (1,)),        # row kernel, unaligned rows (scalar loads)
        ((1 << 21,), (0,)),         # full reduction
        ((17, 65536), (1,)),
        ((255, 8192), (1,)),        # two segments per slice
        ((64, 9, 4000), (0, 2)),    # generic kernel, 9 slices
        ((1000, 3, 700), (0, 2)),   # generic kernel, 3 slices
    ]
    pending = []
    for shape, axes in cases * 2:
        a = r.integers(-3, 4, shape).astype(np.float32)
        x = dev(a)
        kshape = tuple(s for i, s in enumerate(shape) if i not in axes)
        s = K.reduce(_lib.R_SUM, x, axes, nt.float32)
        v, idx, cnt = K.reduce(_lib.R_MAX, x, axes, nt.float32, want_aux=True)
        am = K.reduce(_lib.R_ARGMIN, x, axes, nt.int64)
        pending.append((a, axes, kshape, s, v, idx, cnt, am, x))
    for a, axes, kshape, s, v, idx, cnt, am, _ in pending:
        tag = f"{a.shape} {axes}"
        want_sum = a.astype(np.int64).sum(axis=axes).astype(np.float32)
        assert_bitexact(host(nt.Tensor._new_contiguous(s, kshape)), want_sum, "sum " + tag)
        want_max = O.reduce(O.R_MAX, a, axes)
        assert_bitexact(host(nt.Tensor._new_contiguous(v, kshape)), want_max, "max " + tag)
        assert_bitexact(host(nt.Tensor._new_contiguous(idx, kshape)), O.reduce(O.R_ARGMAX, a, axes), "argmax " + tag)
        want_cnt = (a == np.expand_dims(want_max, axes)).sum(axis=axes).astype(np.int32)
        assert_bitexact(host(nt.Tensor._new_contiguous(cnt, kshape)), want_cnt, "count " + tag)
        assert_bitexact(host(nt.Tensor._new_contiguous(am, kshape)), O.reduce(O.R_ARGMIN, a, axes), "argmin " + tag)


@pytest.mark.parametrize("shape,axes", [
    ((5, 50000), (1,)),       # row kernel, slices split over segments
    ((64, 4096), (1,)),       # row kernel, one workgroup per slice
    ((1 << 20,), (0,)),       # full reduction
    ((4096, 1030), (0,)),     # column walk (wide blocks and a ragged edge)
    ((37, 9, 401), (0, 2)),   # generic kernel
])
def test_select_special_values(gpu, shape, axes):
    """Max / min / argmax / argmin and tie counts over +-inf, the neutral
    values -FLT_MAX / FLT_MAX themselves, signed zeros (the value of the
    first extremum is returned, bit for bit) and NaN.  Slices made only of
    -inf (max) or +inf (min) give the neutral value and index INT64_MAX, as
    the reference's loop does.  NaN never wins and is never counted (a
    documented deviation: the reference's result depends on where NaNs
    sit), which is the reference's result with each NaN replaced by -inf
    (max) or +inf (min), so the oracle runs on that array."""
    r = rng(seed_of("special", shape, axes))
    fmax = np.finfo(np.float32).max
    palette = np.array([np.nan, np.inf, -np.inf, -fmax, fmax, 0.0, -0.0, 1.0, -1.0], np.float32)
    a = r.standard_normal(shape).astype(np.float32)
    pick = r.random(shape) < 0.3
    a[pick] = palette[r.integers(0, len(palette), int(pick.sum()))]
    # whole slices of special values along the reduced axes (not for a full
    # reduction, whose one slice is the whole tensor)
    lead = [slice(None)] * a.ndim
    kept = [d for d in range(a.ndim) if d not in axes]
    specials = [[-np.inf], [np.inf], [np.nan], [0.0, -0.0], [-0.0, 0.0], [-np.inf, -fmax], [np.inf, fmax]]
    for i, vals in enumerate(specials if kept else []):
        idx = list(lead)
        for d in kept:
            idx[d] = i % a.shape[d]
        sub = a[tuple(idx)]
        sub[...] = np.asarray(vals, np.float32)[r.integers(0, len(vals), sub.shape)]
    x = dev(a)
    kshape = tuple(s for i, s in enumerate(shape) if i not in axes)
    for op, oop, aop, argop, fill in ((_lib.R_MAX, O.R_MAX, O.R_ARGMAX, _lib.R_ARGMAX, -np.inf),
                                      (_lib.R_MIN, O.R_MIN, O.R_ARGMIN, _lib.R_ARGMIN, np.inf)):
        ref_in = np.where(np.isnan(a), np.float32(fill), a)
        want = O.reduce(oop, ref_in, axes)
        v, idx, cnt = K.reduce(op, x, axes, nt.float32, want_aux=True)
        assert_bitexact(host(nt.Tensor._new_contiguous(v, kshape)), want, f"value {op}")
        want_idx = O.reduce(aop, ref_in, axes)
        assert_bitexact(host(nt.Tensor._new_contiguous(idx, kshape)), want_idx, f"index {op}")
        got_arg = host(nt.Tensor._new_contiguous(K.reduce(argop, x, axes, nt.int64), kshape))
        assert_bitexact(got_arg, want_idx, f"arg {op}")
        want_cnt = (ref_in == np.expand_dims(want, axes)).sum(axis=axes).astype(np.int32)
        assert_bitexact(host(nt.Tensor._new_contiguous(cnt, kshape)), want_cnt, f"count {op}")


@pytest.mark.parametrize("shape,axes", [((3000, 1030), (0,)), ((3, 200003), (1,)), ((1 << 19,), (0,))])
def test_float64_split_walks(gpu, shape, axes):
    """fp64 reductions long enough to be split over several workgroups: the
    column walk's round-robin rows and the row kernel's round-robin max/min
    chunks and contiguous sum ranges, with 32-byte vectors; sums within the
    fp64 bound, max/min values, indices and counts exact (integer-valued
    data: many ties)."""
    r = rng(seed_of("f64-split", shape, axes))
    a = r.integers(-20, 21, shape).astype(np.float64)
    x = dev(a)
    kshape = tuple(s for i, s in enumerate(shape) if i not in axes)
    got = host(nt.Tensor._new_contiguous(K.reduce(_lib.R_SUM, x, axes, nt.float64), kshape))
    assert_bitexact(got, a.sum(axis=axes), "f64 sum")  # integers: exact
    for op, oop, aop in ((_lib.R_MAX, O.R_MAX, O.R_ARGMAX), (_lib.R_MIN, O.R_MIN, O.R_ARGMIN)):
        v, idx, cnt = K.reduce(op, x, axes, nt.float64, want_aux=True)
        want = O.reduce(oop, a, axes)
        assert_bitexact(host(nt.Tensor._new_contiguous(v, kshape)), want, f"f64 {op}")
        assert_bitexact(host(nt.Tensor._new_contiguous(idx, kshape)), O.reduce(aop, a, axes), f"f64 arg {op}")
        want_cnt = (a == np.expand_dims(want, axes)).sum(axis=axes).astype(np.int32)
        assert_bitexact(host(nt.Tensor._new_contiguous(cnt, kshape)), want_cnt, f"f64 count {op}")
