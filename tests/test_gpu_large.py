"""Tensors past 2^31 (and 2^32) elements: the 64-bit index paths of every
kernel family.  Inputs are built on the device (fills plus a few scalar
writes at chosen positions beyond 2^31), and results are checked at those
positions and against closed forms, so nothing large crosses PCIe.  Every
expected value is exact in fp32 (small integers), so the checks are
bit-exact.  Each test returns its memory to HIP afterwards."""

from __future__ import annotations

import pytest

import nanotorch_amd as nt
from nanotorch_amd import _lib

pytestmark = pytest.mark.gpu

BIG = 2**31 + 4097  # past int32, with a tail that is not a multiple of 4


@pytest.fixture(autouse=True)
def _release(gpu):
    yield
    nt.sync()
    _lib.call("nt_empty_cache")


def at(t, *idx):
    return t[idx].cpu().item()


def test_flat_binary_and_unary_past_2_31():
    a = nt.full(BIG, value=1.5, device="cuda")
    b = nt.full(BIG, value=2.0, device="cuda")
    a[BIG - 1] = 3.0
    a[2**31] = -4.0
    c = a * b
    assert at(c, 0) == 3.0
    assert at(c, 2**31 - 1) == 3.0
    assert at(c, 2**31) == -8.0
    assert at(c, BIG - 1) == 6.0
    del b
    r = nt.relu(c)  # unary path, selection semantics
    assert at(r, 2**31) == 0.0 and at(r, BIG - 1) == 6.0


def test_full_reduction_past_2_31():
    x = nt.zeros(BIG, device="cuda")
    x[BIG - 5] = 7.0
    x[1000] = -3.0
    assert nt.sum(x).cpu().item() == 4.0
    assert x.max().cpu().item() == 7.0
    assert nt.argmax(x).cpu().item() == BIG - 5
    assert nt.argmin(x).cpu().item() == 1000


def test_max_backward_routes_past_2_31():
    x = nt.zeros(BIG, device="cuda")
    x[2**31 + 17] = 2.0
    x.enable_grad()
    x.max().backward()
    g = x.grad
    assert at(g, 2**31 + 17) == 1.0
    assert nt.sum(g).cpu().item() == 1.0


def test_axis0_reduction_past_2_31_rows():
    # [2^31 + 64, 2]: more rows than the column walk takes, the generic path
    rows = 2**31 + 64
    x = nt.zeros(rows, 2, device="cuda")
    x[rows - 3, 1] = 5.0
    x[2**31 + 1, 0] = -1.0
    m = x.max(axis=0)
    assert m.cpu().tolist() == [0.0, 5.0]
    assert nt.argmax(x, axis=0).cpu().tolist() == [0, rows - 3]
    assert nt.argmin(x, axis=0).cpu().tolist() == [2**31 + 1, 0]
    assert nt.sum(x, axis=0).cpu().tolist() == [-1.0, 5.0]


def test_broadcast_rows_past_2_32():
    # 2^32 + 2^16 elements: past the rows kernel's 32-bit range
    R, C = 2**16 + 1, 2**16
    x = nt.zeros(R, C, device="cuda")
    bias = nt.arange(C, dtype=nt.float32).to("cuda")
    x[R - 1, C - 1] = 1.0
    y = x + bias
    assert at(y, 0, 5) == 5.0
    assert at(y, R - 1, C - 1) == float(C - 1) + 1.0
    assert at(y, R - 1, 0) == 0.0


def test_matmul_operand_past_2_31():
    # A [65536, 32768] holds 2^31 elements: row offsets past int32
    M, K, N = 2**16, 2**15, 64
    a = nt.zeros(M, K, device="cuda")
    a[M - 1, :] = 1.0
    a[40000, K - 1] = 2.0
    b = nt.ones(K, N, device="cuda")
    c = a @ b
    assert at(c, M - 1, 0) == float(K)
    assert at(c, M - 1, N - 1) == float(K)
    assert at(c, 40000, 7) == 2.0
    assert at(c, 0, 0) == 0.0


def test_gather_scatter_past_2_31():
    x = nt.zeros(BIG, device="cuda")
    x[BIG - 2] = 9.0
    got = x[[BIG - 2, 0, 2**31 + 1]]
    assert got.cpu().tolist() == [9.0, 0.0, 0.0]
    x[[BIG - 1, 2**31]] = nt.tensor([4.0, 6.0]).to("cuda")
    assert at(x, BIG - 1) == 4.0 and at(x, 2**31) == 6.0
    assert nt.sum(x).cpu().item() == 19.0


def test_unaligned_flat_view_past_2_32():
    # x[1:] of 2^32 + 9 elements: a view whose start is not 16-byte aligned
    # takes the flat path one element per work-item, over more elements
    # than one dispatch can hold (launched in chunks)
    n = 2**32 + 9
    x = nt.full(n, value=1.0, device="cuda")
    x[2**32 + 3] = 5.0
    x[2**30 + 1] = -2.0
    y = -x[1:]
    assert y.shape == (n - 1,)
    assert at(y, 0) == -1.0
    assert at(y, 2**30) == 2.0
    assert at(y, 2**32 + 2) == -5.0
    assert at(y, n - 2) == -1.0
    assert at(y, 2**30 * 3 + 7) == -1.0


def test_fill_past_64_gib():
    # 2^34 + 12 fp32 (64 GiB + 48 B): more 16-byte words than one dispatch
    # of the fill kernel holds, so its grid-stride loop takes the rest
    n = 2**34 + 12
    x = nt.full(n, value=3.0, device="cuda")
    assert at(x, 0) == 3.0
    assert at(x, 2**32 * 4 - 1) == 3.0
    assert at(x, n - 1) == 3.0
    assert at(x, n - 13) == 3.0


@pytest.mark.parametrize("row_stride", [2**23, 2**24])
def test_tile_store_far_apart_rows(row_stride):
    # out[...] = x.T into the first 192 columns of a [256, row_stride] fp32
    # buffer: the transposed tile kernel (64 x 128 tiles) writes rows
    # row_stride elements apart.  With 2^23 a tile's rows span just under
    # 2^31 bytes, the byte offsets of its device-scope buffer stores reach
    # 2.11e9; with 2^24 they would pass 2^31, so the kernel takes the
    # streaming-store path instead.  Columns past 192 must stay untouched.
    import numpy as np
    R, C = 256, 192
    big = nt.zeros(R, row_stride, device="cuda")
    out = big[:, :C]
    xs = (np.arange(C * R, dtype=np.float32) % 1021.0).reshape(C, R)
    x = nt.tensor(xs.tolist()).to("cuda")
    out[...] = x.T
    got = np.array(out.cpu().tolist(), dtype=np.float32)
    assert np.array_equal(got, xs.T)
    edge = np.array(big[:, C:C + 8].cpu().tolist(), dtype=np.float32)
    assert not edge.any()
    assert at(big, R - 1, row_stride - 1) == 0.0
