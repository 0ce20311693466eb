"""Advanced indexing on the device (nt_gather_axes / nt_scatter_axes)
against the reference test-suite's known answers and against the host
path, which test_indexing.py pins to the same answers and to numpy.
Data movement only: bit-exact for every dtype."""

from __future__ import annotations

import numpy as np
import pytest

from test_indexing import CASES, run_case

import nanotorch_amd as nt
from nanotorch_amd import _fancy
from helpers import assert_bitexact, dev, dev_T, rng

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", CASES, ids=[c["src"].split(":")[-1] + c["kind"] for c in CASES])
def test_known_answers_device(gpu, case):
    run_case(case, "cuda")


def test_cast_view_index_device(gpu):
    """tests/test_ops/test_tensor_core.py:518-537 on the device."""
    x = nt.tensor([[0.0, 1.0, 2.0, 3.0], [1.0, 2.7182817459106445, 7.389056205749512,
                   20.08553695678711], [8.0, 9.0, 10.0, 11.0]]).to("cuda")
    for dt in (nt.int32, nt.int64):
        assert x[:, x[0].to(dt)].cpu().tolist() == x.cpu().tolist()


SELECTORS = [
    lambda r, s: (r.integers(-s[0], s[0], (7,)).tolist(),),
    lambda r, s: (slice(None), r.integers(0, s[1], (3, 4)).tolist()),
    lambda r, s: (slice(1, None, 2), r.integers(0, s[1], (5,)).tolist(), r.integers(0, s[2], (5,)).tolist()),
    lambda r, s: (r.integers(0, s[0], (4, 1)).tolist(), slice(None), r.integers(0, s[2], (1, 3)).tolist()),
    lambda r, s: (0, slice(None), r.integers(0, s[2], (6,)).tolist()),
    lambda r, s: (None, (r.random(s[0]) > 0.4).tolist(), Ellipsis, 2),
]


@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.int32, np.int64, np.bool_])
@pytest.mark.parametrize("k", range(len(SELECTORS)))
@pytest.mark.parametrize("layout", ["contig", "transposed"])
def test_getitem_device_vs_host(gpu, k, dtype, layout):
    r = rng(k * 10 + len(layout))
    shape = (6, 9, 5)
    a = (r.standard_normal(shape) * 10).astype(dtype)
    host = nt.Tensor(a)
    if layout == "contig":
        x = dev(a)
    else:  # same logical values, storage transposed on the last two axes
        x = dev(np.ascontiguousarray(np.swapaxes(a, 1, 2))).transpose(1, 2)
    idx = SELECTORS[k](r, shape)
    want = host[idx].numpy()
    got = x[idx]
    assert got.device == nt.Device.Cuda
    assert_bitexact(got.numpy(), want, f"selector {k}")


def test_index_tensors_on_device(gpu):
    r = rng(1)
    a = r.standard_normal((50, 8)).astype(np.float32)
    rows = r.integers(-50, 50, (20,))
    x = dev(a)
    got = x[nt.tensor(rows.tolist()).to("cuda")].numpy()
    assert_bitexact(got, a[rows], "device index tensor")


def test_gather_rows_large(gpu):
    """An embedding-style lookup: 8192 rows of a [50000, 1024] table."""
    r = rng(2)
    table = r.standard_normal((50000, 1024)).astype(np.float32)
    ids = r.integers(0, 50000, (8192,))
    got = dev(table)[ids.tolist()].numpy()
    assert_bitexact(got, table[ids], "row gather")


@pytest.mark.parametrize("dtype", [np.float32, np.int64, np.bool_])
def test_setitem_device_vs_host(gpu, dtype):
    r = rng(3)
    a = (r.standard_normal((8, 6, 5)) * 10).astype(dtype)
    cases = [
        ((r.integers(0, 8, (5,)).tolist(),), (5, 6, 5)),
        ((slice(None), [0, 3, 3, 5]), (8, 4, 5)),  # a repeated index
        ((slice(2, 7), [1, 4], [0, 2]), (5, 2)),  # basic offset + fancy
        (([1, 1, 1, 2], slice(None), [4, 4, 4, 0]), (4, 6)),  # repeated tuples
        (((r.random(8) > 0.5).tolist(),), None),
    ]
    for idx, vshape in cases:
        h = nt.Tensor(a.copy())
        d = dev(a)
        if vshape is None:
            vshape = h[idx].shape
        v = (r.standard_normal(vshape) * 10).astype(dtype)
        h[idx] = nt.Tensor(v)
        d[idx] = dev(v)
        assert_bitexact(d.numpy(), h.numpy(), f"setitem {idx}")
        # scalar and broadcast values
        h[idx] = 7
        d[idx] = 7
        assert_bitexact(d.numpy(), h.numpy(), f"setitem scalar {idx}")


def test_setitem_last_write_wins_device(gpu):
    r = rng(4)
    a = r.standard_normal((6, 300)).astype(np.float32)
    rows = [0, 2, 2, 5, 0, 2]
    vals = r.standard_normal((6, 300)).astype(np.float32)
    x = dev(a)
    x[rows] = dev(vals)
    want = a.copy()
    for i, rr in enumerate(rows):
        want[rr] = vals[i]
    assert_bitexact(x.numpy(), want, "last write wins")


def test_setitem_from_transposed_value(gpu):
    r = rng(5)
    a = r.standard_normal((10, 7)).astype(np.float32)
    w = r.standard_normal((10, 4)).astype(np.float32)
    x = dev(a)
    x[:, [0, 2, 4, 6]] = dev_T(w)  # logical w, transposed storage
    want = a.copy()
    want[:, [0, 2, 4, 6]] = w
    assert_bitexact(x.numpy(), want, "transposed value")


def test_out_of_range_index_through_abi(gpu):
    """A caller that skips the host checks gets IndexError from the kernel's
    own bounds test at the next synchronisation, once; no element outside
    the view is read (the gather writes zeros there) or written."""
    x = dev(np.arange(12, dtype=np.float32).reshape(3, 4))
    plan = _fancy.compute_plan((3, 4), ([0, 1],))
    plan.index_arrays = [np.array([0, 3], dtype=np.int64)]  # 3 >= axis length
    out = nt.Tensor(np.full((2, 4), 7.0, dtype=np.float32), device="cuda")
    _fancy._device_call("nt_gather_axes", plan, x, out)  # queues only
    with pytest.raises(IndexError):
        nt.sync()
    nt.sync()  # reported once
    assert out.cpu().tolist() == [[0.0, 1.0, 2.0, 3.0], [0.0] * 4]
    # scatter: the bad row is skipped, the good one written
    src = dev(np.full((2, 4), -1.0, dtype=np.float32))
    _fancy._device_call("nt_scatter_axes", plan, src, x)
    with pytest.raises(IndexError):
        x.cpu()  # the device-to-host copy reports it too
    assert x.cpu().tolist() == [[-1.0] * 4, [4.0, 5.0, 6.0, 7.0], [8.0, 9.0, 10.0, 11.0]]


@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.int64, np.bool_])
def test_row_gather_scatter_vector_path(gpu, dtype):
    """Row gathers / scatters take the 16-byte vector path when the rows are
    contiguous and aligned; offset views and odd widths take the scalar
    one.  Both against numpy, bit-exact."""
    r = rng(6)
    for rows_, width, off in ((300, 64, 0), (300, 64, 16), (300, 66, 0), (257, 48, 3)):
        base = (r.standard_normal(rows_ * width + off) * 10).astype(dtype)
        table = base[off:].reshape(rows_, width)
        t = dev(base)[off:].reshape(rows_, width)
        ids = r.integers(-rows_, rows_, (37,))
        assert_bitexact(t[ids.tolist()].numpy(), table[ids], f"gather {width} {off}")
        uniq = r.permutation(rows_)[:25]
        vals = (r.standard_normal((25, width)) * 10).astype(dtype)
        t[uniq.tolist()] = dev(vals)
        want = table.copy()
        want[uniq] = vals
        assert_bitexact(t.numpy(), want, f"scatter {width} {off}")


def _random_selector(r, shape):
    """A random index tuple: per axis an int, a slice (any step sign), an
    index list (negative entries and repeats allowed; all lists of one
    selector share a length so that they broadcast) or the whole axis."""
    nfancy_len = int(r.integers(1, 7))
    sel = []
    for d in shape[: int(r.integers(1, len(shape) + 1))]:
        u = r.random()
        if u < 0.2:
            sel.append(int(r.integers(-d, d)))
        elif u < 0.45:
            start, stop = (int(v) for v in r.integers(-d, d + 1, 2))
            step = int(r.choice([1, 2, 3, -1, -2]))
            sel.append(slice(start, stop, step))
        elif u < 0.8:
            sel.append([int(v) for v in r.integers(-d, d, nfancy_len)])
        else:
            sel.append(slice(None))
    return tuple(sel)


@pytest.mark.parametrize("case", range(20))
def test_random_selectors_device_vs_host(gpu, case):
    """Random basic + advanced index tuples on a device tensor (contiguous
    or with its last two axes stored transposed), __getitem__ and then
    __setitem__ of a scalar, against the host path of the same API."""
    r = rng(12000 + case)
    shape = tuple(int(v) for v in r.choice([3, 5, 8, 13], 3))
    a = (r.standard_normal(shape) * 10).astype(np.float32)
    if r.random() < 0.5:
        x = dev(a)
    else:
        x = dev(np.ascontiguousarray(np.swapaxes(a, 1, 2))).transpose(1, 2)
    h = nt.Tensor(a.copy())
    sel = _random_selector(r, shape)
    want = h[sel].numpy()
    got = x[sel]
    assert got.device == nt.Device.Cuda
    assert_bitexact(got.numpy(), want, f"case {case} getitem {sel}")
    h[sel] = 7.5
    x[sel] = 7.5
    assert_bitexact(x.numpy(), h.numpy(), f"case {case} setitem {sel}")
