"""Functional forms of the Tensor ops (reference: src/nanotorch/ops.py)."""

from __future__ import annotations

import math

from . import _kernels as K
from . import _lib
from . import autograd
from ._data_type import Dtype, promote_dtypes
from ._indexing import broadcast_shapes
from .core import Tensor


def clone(x: Tensor) -> Tensor:
    return x.clone()


def reshape(x: Tensor, *dims: int) -> Tensor:
    return x.reshape(*dims)


def transpose(x: Tensor, dim0: int, dim1: int) -> Tensor:
    return x.transpose(dim0, dim1)


def flatten(x: Tensor) -> Tensor:
    return x.flatten()


def equals(x: Tensor, y: Tensor) -> bool:
    return x.equals(y)


def add(x, y) -> Tensor:
    return x + y


def subtract(x, y) -> Tensor:
    return x - y


def multiply(x, y) -> Tensor:
    return x * y


def divide(x, y) -> Tensor:
    return x / y


def eq(x, y) -> Tensor:
    return x == y


def gt(x, y) -> Tensor:
    return x > y


def geq(x, y) -> Tensor:
    return x >= y


def lt(x, y) -> Tensor:
    return x < y


def leq(x, y) -> Tensor:
    return x <= y


def negate(x: Tensor) -> Tensor:
    return -x


def matmul(x: Tensor, y: Tensor) -> Tensor:
    return x @ y


def sum(x: Tensor, axis=None, keepdim: bool = False, *, dtype: Dtype | None = None) -> Tensor:
    return x.sum(axis, keepdim, dtype=dtype)


def mean(x: Tensor, axis=None, keepdim: bool = False, *, dtype: Dtype | None = None) -> Tensor:
    return x.mean(axis, keepdim, dtype=dtype)


def exp(x: Tensor) -> Tensor:
    return x.exp()


def log(x: Tensor) -> Tensor:
    return x.log()


def pow(x: Tensor, exponent) -> Tensor:
    return x.pow(exponent)


def relu(x: Tensor) -> Tensor:
    return autograd.ReluOp.apply(x)


def tanh(x: Tensor) -> Tensor:
    return autograd.TanhOp.apply(x)


def sqrt(x: Tensor) -> Tensor:
    return autograd.SqrtOp.apply(x)


def sigmoid(x: Tensor) -> Tensor:
    return autograd.SigmoidOp.apply(x)


def _arg_reduce(op: int, name: str, x: Tensor, axis, keepdim: bool) -> Tensor:
    if isinstance(axis, int):
        full_axis = (axis if axis >= 0 else axis + x.ndim,)
    elif axis is None:
        full_axis = tuple(range(x.ndim))
    else:
        raise ValueError(f"Axis must be int or None, found {type(axis)}")
    if keepdim:
        new_shape = tuple(1 if i in full_axis else s for i, s in enumerate(x.shape))
    else:
        new_shape = tuple(s for i, s in enumerate(x.shape) if i not in full_axis)
    if x.is_empty:
        if math.prod(new_shape) != 0:
            raise IndexError(f"{name}() expects reduction dim to be specified for numel=0.")
        return Tensor._new_contiguous(
            K.fill(math.prod(new_shape), 0, x.dtype, x.device), new_shape
        )
    return Tensor._new_contiguous(K.reduce(op, x, full_axis, Dtype.Int64), new_shape)


def argmin(x: Tensor, axis: int | None = None, keepdim: bool = False) -> Tensor:
    """Index of the first minimum along `axis` (flattened index if None)."""
    return _arg_reduce(_lib.R_ARGMIN, "argmin", x, axis, keepdim)


def argmax(x: Tensor, axis: int | None = None, keepdim: bool = False) -> Tensor:
    """Index of the first maximum along `axis` (flattened index if None)."""
    return _arg_reduce(_lib.R_ARGMAX, "argmax", x, axis, keepdim)


def _compare(op: int, x1: Tensor, x2: Tensor) -> Tensor:
    dtype = promote_dtypes(x1.dtype, x2.dtype)
    shape = broadcast_shapes(x1.shape, x2.shape)
    a = x1.to(dtype).expand(*shape)
    b = x2.to(dtype).expand(*shape)
    return Tensor._new_contiguous(K.binary(op, a, b), a.shape)


def equal_op_(x1: Tensor, x2: Tensor) -> Tensor:
    return _compare(_lib.EQ, x1, x2)


def greater_op_(x1: Tensor, x2: Tensor) -> Tensor:
    return _compare(_lib.GT, x1, x2)


def greater_eq_op_(x1: Tensor, x2: Tensor) -> Tensor:
    return _compare(_lib.GE, x1, x2)
