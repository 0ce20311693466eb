"""nanotorch_amd: the nanotorch Tensor / autograd API on an MI355X backend.

Drop-in for the GPU path of nanotorch (az-fouche/nanotorch): the same
``Tensor``, ops, ``backward()`` and ``device="cuda"`` selection, computed by
hand-written HIP kernels for gfx950 in ``libnt.so`` (C ABI in include/nt.h),
called through ctypes.  Dunder methods are bound here, as in the reference's
package init (src/nanotorch/__init__.py:124-179).
"""

from . import _lib
from ._data_type import Dtype, bool_, float32, float64, int32, int64
from .autograd import (
    AddOp,
    ExpandOp,
    ExpOp,
    LogOp,
    MatmulOp,
    MaxOp,
    MeanOp,
    MinOp,
    MulOp,
    NegOp,
    PowOp,
    ReshapeOp,
    SubOp,
    SumOp,
    TransposeOp,
    TrueDivOp,
    no_grad,
)
from .core import Tensor, TensorLike
from .cuda import Device, is_available, sync
from .factories import arange, eye, full, manual_seed, ones, rand, randint, tensor, zeros
from .ops import (
    add,
    argmax,
    argmin,
    clone,
    divide,
    eq,
    equal_op_,
    equals,
    exp,
    flatten,
    geq,
    greater_eq_op_,
    greater_op_,
    gt,
    leq,
    log,
    lt,
    matmul,
    mean,
    multiply,
    negate,
    pow,
    relu,
    reshape,
    sigmoid,
    sqrt,
    subtract,
    sum,
    tanh,
    transpose,
)

__all__ = [
    "Device",
    "Dtype",
    "Tensor",
    "TensorLike",
    "add",
    "arange",
    "argmax",
    "argmin",
    "bool_",
    "clone",
    "divide",
    "eq",
    "equals",
    "exp",
    "eye",
    "flatten",
    "float32",
    "float64",
    "full",
    "geq",
    "gt",
    "int32",
    "int64",
    "is_available",
    "leq",
    "log",
    "lt",
    "manual_seed",
    "matmul",
    "mean",
    "multiply",
    "negate",
    "no_grad",
    "ones",
    "pow",
    "rand",
    "randint",
    "relu",
    "reshape",
    "sigmoid",
    "sqrt",
    "subtract",
    "sum",
    "sync",
    "tanh",
    "tensor",
    "transpose",
    "zeros",
]

_SCALAR_CACHE: dict = {}


def _totensor(x, *, anchor: Tensor) -> Tensor:
    """Wraps a Python scalar/list as a tensor on the anchor's device.

    Device scalars are cached by (type, value): building one costs a
    synchronous host-to-device copy, and the same constants (1, -1, lr)
    recur every step.  The cached tensors are internal and never written.
    """
    if isinstance(x, Tensor):
        return x
    if isinstance(x, (bool, int, float)) and anchor.device == Device.Cuda:
        key = (type(x), x)
        t = _SCALAR_CACHE.get(key)
        if t is None or t.version != 0:
            if len(_SCALAR_CACHE) > 1024:
                _SCALAR_CACHE.clear()
            t = Tensor(x, device=anchor.device)
            _SCALAR_CACHE[key] = t
        return t
    return Tensor(x, device=anchor.device)


Tensor.__add__ = lambda self, other: AddOp.apply(self, _totensor(other, anchor=self))
Tensor.__radd__ = lambda self, other: AddOp.apply(self, _totensor(other, anchor=self))
Tensor.__iadd__ = lambda self, other: AddOp.apply(self, _totensor(other, anchor=self), out=self)
Tensor.__mul__ = lambda self, other: MulOp.apply(self, _totensor(other, anchor=self))
Tensor.__rmul__ = lambda self, other: MulOp.apply(self, _totensor(other, anchor=self))
Tensor.__imul__ = lambda self, other: MulOp.apply(self, _totensor(other, anchor=self), out=self)
Tensor.__sub__ = lambda self, other: SubOp.apply(self, _totensor(other, anchor=self))
Tensor.__rsub__ = lambda self, other: SubOp.apply(_totensor(other, anchor=self), self)
Tensor.__isub__ = lambda self, other: SubOp.apply(self, _totensor(other, anchor=self), out=self)
Tensor.__truediv__ = lambda self, other: TrueDivOp.apply(self, _totensor(other, anchor=self))
Tensor.__rtruediv__ = lambda self, other: TrueDivOp.apply(_totensor(other, anchor=self), self)
Tensor.__itruediv__ = lambda self, other: TrueDivOp.apply(
    self, _totensor(other, anchor=self), out=self
)
Tensor.__neg__ = lambda self: NegOp.apply(self)
Tensor.__matmul__ = lambda self, other: MatmulOp.apply(self, _totensor(other, anchor=self))
Tensor.__pow__ = lambda self, exponent: PowOp.apply(self, _totensor(exponent, anchor=self))
Tensor.__rpow__ = lambda self, exponent: PowOp.apply(_totensor(exponent, anchor=self), self)
Tensor.__eq__ = lambda self, other: equal_op_(self, _totensor(other, anchor=self))
Tensor.__gt__ = lambda self, other: greater_op_(self, _totensor(other, anchor=self))
Tensor.__ge__ = lambda self, other: greater_eq_op_(self, _totensor(other, anchor=self))
Tensor.__lt__ = lambda self, other: _totensor(other, anchor=self) > self
Tensor.__le__ = lambda self, other: _totensor(other, anchor=self) >= self
Tensor.exp = lambda self: ExpOp.apply(self)
Tensor.log = lambda self: LogOp.apply(self)
Tensor.pow = lambda self, exponent: PowOp.apply(self, exponent)
Tensor.mean = lambda self, axis=None, keepdim=False, dtype=None: MeanOp.apply(
    self, axis, keepdim, dtype
)
Tensor.reshape = lambda self, *dims: ReshapeOp.apply(self, *dims)
Tensor.expand = lambda self, *dims: ExpandOp.apply(self, *dims)
Tensor.transpose = lambda self, dim0, dim1: TransposeOp.apply(self, dim0, dim1)
Tensor.sum = lambda self, axis=None, keepdim=False, dtype=None: SumOp.apply(
    self, axis, keepdim, dtype
)
Tensor.max = lambda self, axis=None, keepdim=False: MaxOp.apply(self, axis, keepdim)
Tensor.min = lambda self, axis=None, keepdim=False: MinOp.apply(self, axis, keepdim)
Tensor.__hash__ = None  # __eq__ is elementwise
