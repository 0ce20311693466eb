"""Zero-size tensors on the device, with the reference's semantics for each
op family.  The reference's reduction ops return zeros of the reduced shape
for an empty input (ops_reduction.py:60-63); mean divides that by
numel // out_numel = 0, giving NaN; max/min/argmax/argmin raise IndexError
when an empty input would have to produce a value (ops_reduction.py:188-195,
ops.py:183-187, 222-226) and return an empty result otherwise.  The
reference's test-suite runs its "1d-empty" and "2d-empty" reduction inputs
on the device against torch (tests/test_ops/test_tensor_reduction_ops.py:56,61).
Elementwise, matmul, copy and indexing ops on empty operands return empty
results of the broadcast / product shape, and K = 0 products are zeros."""

from __future__ import annotations

import math

import numpy as np
import pytest

import nanotorch_amd as nt

pytestmark = pytest.mark.gpu


def empty(*shape, dtype=nt.float32):
    return nt.zeros(*shape, dtype=dtype, device="cuda")


@pytest.mark.parametrize("shape", [(0,), (3, 0), (0, 4), (2, 0, 3)])
def test_sum_mean_of_empty(gpu, shape):
    x = empty(*shape)
    s = x.sum()
    assert s.shape == () and s.cpu().item() == 0.0
    m = x.mean()
    assert math.isnan(m.cpu().item())
    for ax in range(len(shape)):
        out_shape = tuple(n for i, n in enumerate(shape) if i != ax)
        s = x.sum(axis=ax)
        assert s.shape == out_shape
        assert s.cpu().tolist() == np.zeros(out_shape).tolist()
        k = x.sum(axis=ax, keepdim=True)
        assert k.shape == tuple(1 if i == ax else n for i, n in enumerate(shape))


@pytest.mark.parametrize("op", ["max", "min"])
def test_max_min_of_empty(gpu, op):
    x = empty(3, 0)
    with pytest.raises(IndexError):
        getattr(x, op)()
    with pytest.raises(IndexError):
        getattr(x, op)(axis=1)  # three empty slices: no value to return
    r = getattr(x, op)(axis=0)  # zero slices: an empty result
    assert r.shape == (0,)
    argf = nt.argmax if op == "max" else nt.argmin
    with pytest.raises(IndexError):
        argf(x)
    assert argf(x, axis=0).shape == (0,)


def test_integer_sum_of_empty(gpu):
    x = empty(0, 5, dtype=nt.int32)
    s = x.sum()
    assert s.dtype == nt.int64 and s.cpu().item() == 0


@pytest.mark.parametrize("shape", [(0,), (4, 0), (0, 4)])
def test_elementwise_on_empty(gpu, shape):
    a = empty(*shape)
    b = empty(*shape)
    for y in (a + b, a - b, a * b, a / (b + 1.0), -a, a.exp(), nt.relu(a),
              nt.sigmoid(a), nt.tanh(a), a ** 2.5, a == b):
        assert y.shape == shape
        assert y.cpu().tolist() == np.zeros(shape).tolist() or y.numel == 0


def test_elementwise_broadcast_to_empty(gpu):
    a = empty(0, 4)
    b = nt.tensor([1.0, 2.0, 3.0, 4.0]).to("cuda")
    assert (a + b).shape == (0, 4)
    assert (a.T * b.reshape(4, 1)).shape == (4, 0)


@pytest.mark.parametrize("op", ["max", "min"])
def test_select_backward_of_empty(gpu, op):
    x = empty(3, 0)
    x.enable_grad()
    getattr(x, op)(axis=0).sum().backward()
    assert x.grad.shape == (3, 0)


def test_unary_backward_of_empty(gpu):
    for f in (lambda t: t.exp(), lambda t: t.log(), lambda t: nt.sqrt(t), nt.tanh,
              nt.sigmoid, lambda t: t ** 2.5, nt.relu, lambda t: -t):
        x = empty(2, 0)
        x.enable_grad()
        f(x).sum().backward()
        assert x.grad.shape == (2, 0)


def test_backward_through_empty(gpu):
    x = empty(0, 3)
    x.enable_grad()
    w = nt.tensor([1.0, 2.0, 3.0]).to("cuda")
    w.enable_grad()
    loss = ((x * w).exp() + x).sum()
    loss.backward()
    assert x.grad.shape == (0, 3)
    assert w.grad.shape == (3,) and w.grad.cpu().tolist() == [0.0, 0.0, 0.0]


@pytest.mark.parametrize("M,K,N", [(0, 5, 3), (3, 5, 0), (3, 0, 4), (0, 0, 0)])
def test_matmul_with_empty_dims(gpu, M, K, N):
    a = empty(M, K)
    b = empty(K, N)
    a.enable_grad()
    b.enable_grad()
    c = a @ b
    assert c.shape == (M, N)
    assert c.cpu().tolist() == np.zeros((M, N)).tolist()  # K = 0: zeros
    c.sum().backward()
    assert a.grad.shape == (M, K) and b.grad.shape == (K, N)
    assert a.grad.cpu().tolist() == np.zeros((M, K)).tolist()


def test_matmul_k0_accumulates_nothing(gpu):
    # a K = 0 product contributes zeros to an existing gradient
    a = nt.ones(3, 4, device="cuda")
    a.enable_grad()
    (a @ nt.ones(4, 2, device="cuda")).sum().backward()
    z = empty(3, 0)
    z.enable_grad()
    (z @ empty(0, 2)).sum().backward()
    assert z.grad.shape == (3, 0)
    assert a.grad.cpu().tolist() == [[2.0] * 4] * 3


def test_copy_cast_index_on_empty(gpu):
    x = empty(4, 0)
    assert x.T.clone().shape == (0, 4)
    assert x.to(nt.float64).dtype == nt.float64
    assert x.to(nt.int32).shape == (4, 0)
    y = nt.tensor([[1.0, 2.0], [3.0, 4.0]]).to("cuda")
    assert y[[]].shape == (0, 2)
    assert y[:, []].shape == (2, 0)
    assert y[[False, False]].shape == (0, 2)
    y[[]] = 5.0  # assigns nothing
    assert y.cpu().tolist() == [[1.0, 2.0], [3.0, 4.0]]
