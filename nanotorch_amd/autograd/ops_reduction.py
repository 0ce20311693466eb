"""Reductions: sum, mean, max, min (differentiable).

Forward semantics restate src/nanotorch/autograd/ops_reduction.py: axis
normalisation (``broadcast_axis``), default sum dtype ``max(x.dtype,
Int64)``, mean as ``sum / float(numel_in // numel_out)`` (a division), empty
inputs giving zeros, keepdim shapes.

Backward:
 * sum  -- a broadcast *view* of the upstream gradient (no kernel), as the
           reference returns; accumulation adds it in place.
 * mean -- ``broadcast(g) / n`` in one kernel, fused with accumulation.
 * max/min -- the reference builds ``mask = x == max``, divides by
           ``mask.sum()`` in int64 (so tied slices get 0), and multiplies.  The
           forward kernel here also records, per slice, the first arg-extremum
           and how many elements equal the extremum; the backward kernel then
           writes ``g * (j == idx && count == 1 ? 1 : 0)`` without re-reading
           x (ops_reduction.py:201-212, 275-286).
"""

from __future__ import annotations

import math

from .. import _kernels as K
from .. import _lib
from .._data_type import Dtype, is_float, sizeof
from .._indexing import TensorShape
from ..core import Tensor
from ..cuda import Device
from .function import Function
from .ops_utils import broadcast_axis


def _out_shape(x: Tensor, axis: TensorShape, keepdim: bool) -> TensorShape:
    if keepdim:
        return tuple(1 if i in axis else s for i, s in enumerate(x.shape))
    return tuple(s for i, s in enumerate(x.shape) if i not in axis)


def _keepdim_shape(orig: TensorShape, axis: TensorShape) -> TensorShape:
    return tuple(1 if d in axis else orig[d] for d in range(len(orig)))


class SumOp(Function):
    """Sum over `axis` (int, tuple, or None for all); `dtype` sets the
    accumulation/output dtype (default max(x.dtype, int64))."""

    def forward(self, x: Tensor, axis=None, keepdim: bool = False, dtype: Dtype | None = None):
        self._axis = broadcast_axis(axis, x)
        if dtype is None:
            dtype = max(x.dtype, Dtype.Int64)
        dtype = Dtype(dtype)
        new_shape = _out_shape(x, self._axis, keepdim)
        self._x_dtype = x.dtype
        self._dtype = dtype
        # set before the empty case too (the reference sets it after, so its
        # backward through an empty sum fails, ops_reduction.py:60-64)
        self._orig_shape = x.shape
        if x.is_empty:
            return Tensor._new_contiguous(
                K.fill(math.prod(new_shape), 0, dtype, x.device), new_shape
            )
        st = K.reduce(_lib.R_SUM, x, self._axis, dtype)
        return Tensor._new_contiguous(st, new_shape)

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        if not self._orig_shape:
            return (grad_out,)
        kd = _keepdim_shape(self._orig_shape, self._axis)
        return (grad_out.reshape(*kd).expand(*self._orig_shape),)

    def fused_ok(self) -> bool:
        return is_float(self._dtype) and self._dtype == self._x_dtype

    def _backward_into(self, g: Tensor, needs, targets):
        if not needs[0]:
            return [None]
        (view,) = self.backward(g)
        if targets[0] is None:
            return [view]
        K.inplace(_lib.ADD, targets[0], view)
        return [targets[0]]

    @classmethod
    def flops(cls, x: Tensor, *args, **kwargs) -> int:
        return x.numel

    @classmethod
    def mem_bytes(cls, x: Tensor, *args, **kwargs) -> int:
        return x.numel * sizeof(x.dtype)


def _scalar_like(value, dtype: Dtype, device: Device) -> Tensor:
    return Tensor._new_contiguous(K.fill(1, value, dtype, device), ())


class MeanOp(Function):
    """Mean over `axis`: sum(x) / float(numel_in // numel_out)."""

    def forward(self, x: Tensor, axis=None, keepdim: bool = False, dtype: Dtype | None = None):
        if dtype is None:
            dtype = x.dtype
        dtype = Dtype(dtype)
        if dtype < Dtype.Float32:
            raise TypeError("Cannot take mean of integer tensor, cast to fp.")
        self._axis = broadcast_axis(axis, x)
        self._x_dtype = x.dtype
        self._dtype = dtype
        new_shape = _out_shape(x, self._axis, keepdim)
        if x.is_empty:
            s = Tensor._new_contiguous(
                K.fill(math.prod(new_shape), 0, dtype, x.device), new_shape
            )
        else:
            s = Tensor._new_contiguous(K.reduce(_lib.R_SUM, x, self._axis, dtype), new_shape)
        self._orig_shape = x.shape
        self._denom = x.numel // s.numel if s.numel else 0
        if s.device == Device.Cpu:
            K.require_device(s)
        denom = _scalar_like(float(self._denom), dtype, s.device).expand(*s.shape)
        return Tensor._new_contiguous(K.binary(_lib.DIV, s, denom), s.shape)

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        if not self._orig_shape:
            return (grad_out,)
        kd = _keepdim_shape(self._orig_shape, self._axis)
        return (grad_out.reshape(*kd).expand(*self._orig_shape) / self._denom,)

    def fused_ok(self) -> bool:
        return is_float(self._dtype) and self._dtype == self._x_dtype

    def _backward_into(self, g: Tensor, needs, targets):
        if not needs[0]:
            return [None]
        if not self._orig_shape:
            if targets[0] is None:
                return [g]
            K.inplace(_lib.ADD, targets[0], g)
            return [targets[0]]
        st = K.reduce_bwd(
            _lib.R_MEAN, g, float(self._denom), None, None, self._axis,
            self._orig_shape, targets[0],
        )
        if st is None:
            return [targets[0]]
        return [Tensor._new_contiguous(st, self._orig_shape)]

    @classmethod
    def flops(cls, x: Tensor, *args, **kwargs) -> int:
        return x.numel

    @classmethod
    def mem_bytes(cls, x: Tensor, *args, **kwargs) -> int:
        return x.numel * sizeof(x.dtype)


class _SelectOp(Function):
    """Shared max/min: forward keeps (value, first index, tie count)."""

    _op: int
    _empty_shape = None  # input shape when the input was empty

    def forward(self, x: Tensor, axis=None, keepdim: bool = False) -> Tensor:
        self._axis = broadcast_axis(axis, x)
        new_shape = _out_shape(x, self._axis, keepdim)
        self._x_dtype = x.dtype
        if x.is_empty:
            if math.prod(new_shape) != 0:
                raise IndexError(
                    "argmin() expects reduction dim to be specified for numel=0."
                )
            # backward returns an empty gradient (the reference's would read
            # the input shape it never recorded)
            self._empty_shape = x.shape
            return Tensor._new_contiguous(
                K.fill(math.prod(new_shape), 0, x.dtype, x.device), new_shape
            )
        self._orig_shape = x.shape
        val, idx, cnt = K.reduce(self._op, x, self._axis, x.dtype, want_aux=True)
        self._idx, self._cnt = idx, cnt
        out = Tensor._new_contiguous(val, new_shape)
        self.save_for_backward(x, out)
        return out

    def _grad(self, g: Tensor, target):
        self.saved_tensors  # raises if x or the result was modified in place
        return K.reduce_bwd(
            self._op, g, 1.0, self._idx, self._cnt, self._axis, self._orig_shape, target
        )

    def _empty_grad(self, g: Tensor) -> Tensor:
        return Tensor._new_contiguous(K.fill(0, 0, g.dtype, g.device), self._empty_shape)

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        if self._empty_shape is not None:
            return (self._empty_grad(grad_out),)
        if not self._orig_shape:
            return (grad_out,)
        return (Tensor._new_contiguous(self._grad(grad_out, None), self._orig_shape),)

    def fused_ok(self) -> bool:
        return is_float(self._x_dtype)

    def _backward_into(self, g: Tensor, needs, targets):
        if not needs[0]:
            return [None]
        if self._empty_shape is not None:
            return [targets[0] if targets[0] is not None else self._empty_grad(g)]
        if not self._orig_shape:
            if targets[0] is None:
                return [g]
            K.inplace(_lib.ADD, targets[0], g)
            return [targets[0]]
        st = self._grad(g, targets[0])
        if st is None:
            return [targets[0]]
        return [Tensor._new_contiguous(st, self._orig_shape)]

    @classmethod
    def flops(cls, x: Tensor, *args, **kwargs) -> int:
        return x.numel

    @classmethod
    def mem_bytes(cls, x: Tensor, *args, **kwargs) -> int:
        return x.numel * sizeof(x.dtype)


class MaxOp(_SelectOp):
    """Max over `axis`; the gradient goes to the unique arg-max of each slice
    (slices with tied maxima get a zero gradient, as in the reference)."""

    _op = _lib.R_MAX


class MinOp(_SelectOp):
    """Min over `axis`; gradient routing as MaxOp."""

    _op = _lib.R_MIN
