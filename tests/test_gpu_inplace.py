"""In-place operators on the device, with the reference's contract
(tests/test_ops/test_tensor_inplace_ops.py:33-150 and :175-428): scalar,
bool and broadcasting right-hand sides; transposed left-hand sides that stay
on the device; storage identity, version bumps and the returned alias;
mutation of a base through slice, transpose and column-slice views;
self-aliased operands; ValueError for a right-hand side that does not
broadcast to the left; the strict primitive nt_inplace (same shape, dtype
and device, no broadcasting: RuntimeError, bool division: ValueError); and
the autograd guards.  Expected values come from numpy in fp32 on the same
inputs."""

from __future__ import annotations

import numpy as np
import pytest

import nanotorch_amd as nt
from nanotorch_amd import _kernels as K
from nanotorch_amd import _lib

pytestmark = pytest.mark.gpu


def _iadd(a, b):
    a += b
    return a


def _isub(a, b):
    a -= b
    return a


def _imul(a, b):
    a *= b
    return a


def _itruediv(a, b):
    a /= b
    return a


OPS = {"iadd": (_iadd, np.add), "isub": (_isub, np.subtract),
       "imul": (_imul, np.multiply), "itruediv": (_itruediv, np.divide)}
SEVEN = np.arange(7, dtype=np.float32)


def cu(a, dtype=np.float32):
    return nt.Tensor(np.asarray(a, dtype=dtype), device="cuda")


# (left shape, left fill, transposed left?, right-hand side)
CASES = [
    ((), 1.0, False, 3.14),
    ((), 1.0, False, -3.14),
    ((), 1.0, False, True),
    ((5,), 6.28, False, 2.0),
    ((5, 7), 6.28, False, 3.14),
    ((5, 7), 6.28, False, np.full((5, 7), 2.0, np.float32)),
    ((5, 7), 6.28, False, np.full((5, 1), 3.14, np.float32)),
    ((5, 7), 6.28, False, np.full(7, 2.0, np.float32)),
    ((7, 5), 0.0, True, SEVEN),
    ((7, 5), 24.0, True, np.array([1.0, 2.0, 3.0, 4.0, 6.0, 8.0, 12.0], np.float32)),
]


@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("k", range(len(CASES)))
def test_inplace_ops_device(gpu, op, k):
    shape, fill, transposed, rhs = CASES[k]
    fn, ref = OPS[op]
    left = np.full(shape, fill, np.float32)
    t = cu(left).T if transposed else cu(left)
    with np.errstate(invalid="ignore"):  # 0 / 0 is NaN on both sides
        want = ref(left.T if transposed else left,
                   rhs if isinstance(rhs, np.ndarray) else np.float32(rhs)).astype(np.float32)
    st, v0 = t.storage, t.version
    out = fn(t, cu(rhs) if isinstance(rhs, np.ndarray) else rhs)
    assert t.storage is st and out.storage is st and out.shape == t.shape
    assert t.version == v0 + 1
    assert t.device == nt.Device.Cuda
    np.testing.assert_array_equal(t.numpy(), want)
    fn(t, 1.0)
    assert t.version == v0 + 2


def test_mutation_through_views_device(gpu):
    a = nt.zeros(4, 4, device="cuda")
    a[1] += 1.0
    want = np.zeros((4, 4), np.float32)
    want[1] = 1.0
    np.testing.assert_array_equal(a.numpy(), want)

    b = nt.zeros(3, 4, device="cuda")
    bt = b.T
    bt += cu([0.0, 1.0, 2.0])
    np.testing.assert_array_equal(b.numpy(), np.repeat(np.arange(3, dtype=np.float32)[:, None], 4, 1))

    c = nt.zeros(3, 4, device="cuda")
    c[:, 1:3] += 1.0
    want = np.zeros((3, 4), np.float32)
    want[:, 1:3] = 1.0
    np.testing.assert_array_equal(c.numpy(), want)

    d = nt.ones(7, 5, device="cuda").T  # the reference's transposed-lhs cases
    d *= cu(SEVEN)
    np.testing.assert_array_equal(d.numpy(), np.tile(SEVEN, (5, 1)))


@pytest.mark.parametrize("op,start,want", [("iadd", 2.0, 4.0), ("isub", 3.0, 0.0),
                                           ("imul", 3.0, 9.0), ("itruediv", 3.0, 1.0)])
def test_self_aliased_device(gpu, op, start, want):
    t = nt.full(5, value=start, device="cuda")
    OPS[op][0](t, t)
    np.testing.assert_array_equal(t.numpy(), np.full(5, want, np.float32))


def test_broadcast_errors_device(gpu):
    t = nt.zeros(4, device="cuda")
    with pytest.raises(ValueError):
        t += nt.zeros(3, 4, device="cuda")
    u = nt.zeros(3, 4, device="cuda")
    with pytest.raises(ValueError):
        u += nt.zeros(5, device="cuda")


PRIMS = [_lib.ADD, _lib.SUB, _lib.MUL, _lib.DIV, _lib.COPY]


@pytest.mark.parametrize("op", PRIMS)
def test_primitive_errors_and_version(gpu, op):
    with pytest.raises(RuntimeError):  # shape: no broadcasting at this level
        K.inplace(op, nt.full(5, 7, value=2.0, device="cuda"), nt.full(5, value=2.0, device="cuda"))
    with pytest.raises(RuntimeError):  # dtype
        K.inplace(op, cu(np.zeros(5)), cu(np.zeros(5), np.float64))
    with pytest.raises(RuntimeError):  # device
        K.inplace(op, nt.zeros(5), nt.zeros(5, device="cuda"))
    a = nt.full(5, value=2.0, device="cuda")
    v0 = a.version
    K.inplace(op, a, nt.full(5, value=1.0, device="cuda"))
    assert a.version == v0 + 1


def test_primitive_bool_division_raises(gpu):
    a = nt.full(5, value=True, dtype=nt.bool_, device="cuda")
    b = nt.full(5, value=True, dtype=nt.bool_, device="cuda")
    with pytest.raises(ValueError):
        K.inplace(_lib.DIV, a, b)


@pytest.mark.parametrize("op,a,b,want", [
    (_lib.ADD, [1.0, 2.0, 3.0], [10.0, 20.0, 30.0], [11.0, 22.0, 33.0]),
    (_lib.SUB, [10.0, 20.0, 30.0], [1.0, 2.0, 3.0], [9.0, 18.0, 27.0]),
    (_lib.MUL, [1.0, 2.0, 3.0], [10.0, 20.0, 30.0], [10.0, 40.0, 90.0]),
    (_lib.DIV, [10.0, 20.0, 30.0], [2.0, 4.0, 6.0], [5.0, 5.0, 5.0]),
])
def test_primitive_values(gpu, op, a, b, want):
    x = cu(a)
    K.inplace(op, x, cu(b))
    assert x.cpu().tolist() == want


def test_primitive_copy(gpu):
    a = nt.zeros(3, 4, device="cuda")
    K.inplace(_lib.COPY, a, nt.full(3, 4, value=5.0, device="cuda"))
    assert a.cpu().tolist() == [[5.0] * 4] * 3
    z = nt.zeros(3, 4, device="cuda")
    K.inplace(_lib.COPY, z[1], cu([1.0, 2.0, 3.0, 4.0]))  # through a row view
    assert z.cpu().tolist() == [[0.0] * 4, [1.0, 2.0, 3.0, 4.0], [0.0] * 4]


@pytest.mark.parametrize("op", OPS)
def test_leaf_inplace_with_grad_raises_device(gpu, op):
    x = nt.tensor([1.0, 2.0, 3.0], requires_grad=True).to("cuda")
    assert x.is_leaf and x.requires_grad
    with pytest.raises(RuntimeError):
        OPS[op][0](x, 1.5)


def test_inplace_invalidates_saved_tensor_device(gpu):
    x = nt.tensor([1.0, 2.0, 3.0], requires_grad=True).to("cuda")
    y = x.exp()  # saves its output
    y += 1
    with pytest.raises(RuntimeError):
        y.sum().backward()


def test_inplace_without_saved_tensor_device(gpu):
    x = nt.tensor([1.0, 2.0, 3.0], requires_grad=True).to("cuda")
    y = x + 1  # saves nothing
    y += 2
    y.sum().backward()
    assert x.grad.cpu().tolist() == [1.0, 1.0, 1.0]
