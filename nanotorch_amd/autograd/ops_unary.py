"""Unary differentiable ops: neg, exp, log, sqrt, tanh, sigmoid, pow, relu.

Forward semantics restate src/nanotorch/autograd/ops_unary.py (float-only
ops promote integer inputs to float32; exp/log/sqrt/tanh/sigmoid/pow return
empty inputs unchanged).  ``backward`` keeps the reference compositions;
``_backward_into`` evaluates the same rounding chain in one fused kernel
(nt_unary_bwd), accumulating into an existing gradient in the same pass.
"""

from __future__ import annotations

from .. import _kernels as K
from .. import _lib
from .._data_type import Dtype, is_float, promote_dtypes, sizeof
from ..core import Tensor
from .function import Function
from .ops_utils import unbroadcast


def _empty_passthrough(op: Function, x: Tensor) -> Tensor:
    """Forward of an empty input: the input itself, as the reference returns
    it.  The op saves nothing, so its backward passes the (empty) gradient
    through (the reference's backward would read saved tensors that were
    never saved)."""
    op._empty = True
    return x


def _empty_backward_into(g: Tensor, needs, targets) -> list:
    if not needs[0]:
        return [None] * len(needs)
    return [targets[0] if targets[0] is not None else g] + [None] * (len(needs) - 1)


class _UnaryOp(Function):
    _op: int
    _promote = True  # float-only op: integer inputs become float32
    _in_dtype = None
    _empty = False

    def _prepare(self, x: Tensor) -> Tensor:
        self._in_dtype = x.dtype
        if self._promote:
            x = x.to(promote_dtypes(x.dtype, Dtype.Float32))
        return x

    def fused_ok(self) -> bool:
        if self._empty:
            return True
        return is_float(self._in_dtype) and getattr(self, "_saved_ok", True)

    def _fused_saved(self):
        return self.saved_tensors[0]

    def _scalar(self) -> float:
        return 0.0

    def _backward_into(self, g: Tensor, needs, targets):
        if self._empty:
            return _empty_backward_into(g, needs, targets)
        if not needs[0]:
            return [None]
        saved = self._fused_saved()
        if g.shape != saved.shape and saved is not None:
            g = g.reshape(*saved.shape)
        st = K.unary_bwd(self._op, g, saved, self._scalar(), targets[0])
        if st is None:
            return [targets[0]]
        return [Tensor._new_contiguous(st, g.shape)]

    @classmethod
    def flops(cls, x: Tensor, *args) -> int:
        return x.numel

    @classmethod
    def mem_bytes(cls, x: Tensor, *args) -> int:
        return 2 * x.numel * sizeof(x.dtype)


class NegOp(_UnaryOp):
    """-x (integer dtypes allowed, bool raises ValueError)."""

    _op = _lib.NEG
    _promote = False

    def forward(self, x: Tensor) -> Tensor:
        self._shape = x.shape
        self._in_dtype = x.dtype
        return Tensor._new_contiguous(K.unary(_lib.NEG, x), x.shape)

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        return (unbroadcast(-1 * grad_out, self._shape),)

    def _backward_into(self, g: Tensor, needs, targets):
        if not needs[0]:
            return [None]
        if g.shape != self._shape:
            g = g.reshape(*self._shape)
        st = K.unary_bwd(_lib.NEG, g, None, 0.0, targets[0])
        if st is None:
            return [targets[0]]
        return [Tensor._new_contiguous(st, self._shape)]


class ExpOp(_UnaryOp):
    """exp(x); saves the output."""

    _op = _lib.EXP

    def forward(self, x: Tensor) -> Tensor:
        if x.is_empty:
            return _empty_passthrough(self, x)
        x = self._prepare(x)
        y = Tensor._new_contiguous(K.unary(_lib.EXP, x), x.shape)
        self.save_for_backward(y)
        return y

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        return (grad_out * self.saved_tensors[0],)


class LogOp(_UnaryOp):
    """log(x); saves the input."""

    _op = _lib.LOG

    def forward(self, x: Tensor) -> Tensor:
        if x.is_empty:
            return _empty_passthrough(self, x)
        x = self._prepare(x)
        self.save_for_backward(x)
        return Tensor._new_contiguous(K.unary(_lib.LOG, x), x.shape)

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        return (grad_out * self.saved_tensors[0] ** -1,)


class SqrtOp(_UnaryOp):
    """sqrt(x); saves the output."""

    _op = _lib.SQRT

    def forward(self, x: Tensor) -> Tensor:
        if x.is_empty:
            return _empty_passthrough(self, x)
        x = self._prepare(x)
        y = Tensor._new_contiguous(K.unary(_lib.SQRT, x), x.shape)
        self.save_for_backward(y)
        return y

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        y = self.saved_tensors[0]
        return (grad_out * 0.5 * y**-1,)


class TanhOp(_UnaryOp):
    """tanh(x); saves the output."""

    _op = _lib.TANH

    def forward(self, x: Tensor) -> Tensor:
        if x.is_empty:
            return _empty_passthrough(self, x)
        x = self._prepare(x)
        y = Tensor._new_contiguous(K.unary(_lib.TANH, x), x.shape)
        self.save_for_backward(y)
        return y

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        y = self.saved_tensors[0]
        return (grad_out * (1 - y**2),)


class SigmoidOp(_UnaryOp):
    """1 / (1 + exp(-x)); saves the output."""

    _op = _lib.SIGMOID

    def forward(self, x: Tensor) -> Tensor:
        if x.is_empty:
            return _empty_passthrough(self, x)
        x = self._prepare(x)
        y = Tensor._new_contiguous(K.unary(_lib.SIGMOID, x), x.shape)
        self.save_for_backward(y)
        return y

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        y = self.saved_tensors[0]
        return (grad_out * y * (1 - y),)


class PowOp(Function):
    """x ** exponent for a scalar-like exponent (a number or a 1-element
    tensor).  As in the reference, a Python float exponent becomes a float32
    tensor, so its value is float32-rounded even for float64 x."""

    _dtype = None
    _x_dtype = None
    _empty = False

    def forward(self, x: Tensor, exponent) -> Tensor:
        if x.is_empty:
            return _empty_passthrough(self, x)
        if not isinstance(exponent, Tensor):
            exponent = Tensor(exponent)
        dtype = promote_dtypes(x.dtype, exponent.dtype)
        e = float(exponent.cpu().item())
        if e < 0 and dtype <= Dtype.Int64:
            raise RuntimeError("Cannot use negative exponent with integer tensor.")
        self._x_dtype = x.dtype
        self._dtype = dtype
        self._e = e
        self.save_for_backward(x, exponent)
        return Tensor._new_contiguous(K.unary(_lib.POW, x.to(dtype), e), x.shape)

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        x, exponent = self.saved_tensors
        return (grad_out * exponent * x ** (exponent - 1),)

    def fused_ok(self) -> bool:
        if self._empty:
            return True
        return is_float(self._dtype) and self._x_dtype == self._dtype

    def _backward_into(self, g: Tensor, needs, targets):
        if self._empty:
            return _empty_backward_into(g, needs, targets)
        results = [None, None]
        if not needs[0]:
            return results
        x, _ = self.saved_tensors
        st = K.unary_bwd(_lib.POW, g, x, self._e, targets[0])
        results[0] = targets[0] if st is None else Tensor._new_contiguous(st, x.shape)
        return results

    @classmethod
    def flops(cls, x: Tensor, exponent) -> int:
        return x.numel

    @classmethod
    def mem_bytes(cls, x: Tensor, exponent) -> int:
        return 2 * x.numel * sizeof(x.dtype)


class ReluOp(_UnaryOp):
    """(x >= 0) ? x : 0 (any arithmetic dtype); saves the output."""

    _op = _lib.RELU
    _promote = False

    def forward(self, x: Tensor) -> Tensor:
        self._in_dtype = x.dtype
        y = Tensor._new_contiguous(K.unary(_lib.RELU, x), x.shape)
        self.save_for_backward(y)
        return y

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        y = self.saved_tensors[0]
        return (grad_out * (y > Tensor(0, device=y.device)),)
