"""The strided Tensor and the autograd engine.

API and semantics follow the reference's ``nanotorch.Tensor``
(src/nanotorch/core.py:47-568): a tensor is a view (shape, element strides,
offset) of a typed 1-D storage; views alias; in-place ops bump the storage
version; ``backward()`` runs the engine of core.py:836-872.

Device model: tensors on ``"cuda"`` (the MI355X) are computed on by libnt's
HIP kernels.  Tensors on ``"cpu"`` hold host data: they can be created,
viewed, indexed, copied, cast, listed and moved to the device, but every
arithmetic op requires device tensors (there is no host compute path).
"""

from __future__ import annotations

import math
from typing import TYPE_CHECKING, Any, Sequence

from . import _fancy
from . import _kernels as K
from ._data_type import (
    Dtype,
    InputType,
    dtype_from_type,
    is_bool,
    is_float,
    is_int,
    promote_dtypes,
    sizeof,
)
from ._indexing import TensorShape, expand_ellipsis, is_contiguous_view
from ._storage import Storage
from .cuda import Device, DeviceLiteral, get_std_device

if TYPE_CHECKING:
    from .autograd import Function

MAX_TENSOR_LEVEL = 32

_NUMPY_DTYPES = {
    "bool": Dtype.Bool,
    "int32": Dtype.Int32,
    "int64": Dtype.Int64,
    "float32": Dtype.Float32,
    "float64": Dtype.Float64,
}


class Tensor:
    """Typed n-dimensional strided array with autograd.

    Parameters
    ----------
    data: list | float | int | bool | array-like
        Coefficients.  Objects with ``__array__`` (numpy arrays) of a
        supported dtype are copied through the buffer protocol; other
        array-likes go through ``tolist()``.
    dtype: Dtype | None
        Target dtype; inferred from the values (bool < int64 < float32) if
        omitted.
    requires_grad: bool
        Track gradients (float dtypes only).
    device: Device | "cpu" | "cuda"
        Where the storage lives.
    """

    def __init__(
        self,
        data: InputType,
        *,
        dtype: Dtype | None = None,
        requires_grad: bool = False,
        device: Device | DeviceLiteral = Device.Cpu,
    ):
        device = get_std_device(device)
        storage, shape, out_dtype = None, None, None
        if hasattr(data, "__array__") and hasattr(data, "tolist"):
            storage, shape, out_dtype = _from_array_like(data, dtype, device)
            if storage is None:
                data = data.tolist()
        if storage is None:
            out_dtype, shape, storage = _extract_tensor_data(data, device, dtype)
        self._storage = storage
        self._shape = tuple(shape)
        self._strides = _infer_strides(self._shape)
        self._offset = 0
        if out_dtype <= Dtype.Int64 and requires_grad:
            raise RuntimeError("Cannot enable grad on a non-float tensor.")
        self._requires_grad = requires_grad
        self._grad: Tensor | None = None
        self._grad_fn: Function | None = None

    # -- construction helpers ------------------------------------------------

    @classmethod
    def _new_contiguous(cls, storage: Storage, shape: TensorShape) -> Tensor:
        return cls._new_view(storage, tuple(shape), None, None)

    @classmethod
    def _new_view(
        cls,
        storage: Storage,
        shape: TensorShape,
        strides: TensorShape | None,
        offset: int | None,
    ) -> Tensor:
        shape = tuple(shape)
        strides = _infer_strides(shape) if strides is None else tuple(strides)
        offset = 0 if offset is None else offset
        if math.prod(shape) > 0:
            lo = offset + sum((s - 1) * st for s, st in zip(shape, strides) if st < 0)
            hi = offset + sum((s - 1) * st for s, st in zip(shape, strides) if st > 0)
            if lo < 0 or hi >= storage.size:
                raise IndexError(
                    f"View max index {hi} exceeds storage capacity {storage.size}."
                )
        new = cls.__new__(cls)
        new._storage = storage
        new._shape = shape
        new._strides = strides
        new._offset = offset
        new._requires_grad = False
        new._grad_fn = None
        new._grad = None
        return new

    # -- printing ------------------------------------------------------------

    def __repr__(self) -> str:
        c = self.cpu()
        if self.ndim == 0:
            return f"nt.Tensor({c.tolist()})"
        if self.ndim == 1:
            return f"nt.Tensor({_str_list_compact(c.tolist())})"
        if self.ndim == 2:
            rows = list(range(len(self))) if len(self) <= 5 else [0, 1, None, -2, -1]
            lines = []
            for i in rows:
                lines.append("..." if i is None else _str_list_compact(c[i].tolist()))
            return "nt.Tensor(" + "\n          ".join(lines) + ")"
        return (
            f"nt.Tensor(shape={self.shape}, {self.numel} x <{self.dtype.name}>, "
            f"d: {self.device.name})"
        )

    def __len__(self) -> int:
        return self._shape[0] if self._shape else 0

    # -- indexing --------------------------------------------------------------

    def __getitem__(self, index) -> Tensor:
        if not isinstance(index, tuple):
            index = (index,)
        if self.ndim == 0:
            raise IndexError("Cannot index a scalar value.")
        n_real = sum(1 for x in index if x is not None and x is not Ellipsis)
        if n_real > self.ndim:
            raise IndexError(f"Too many indices ({len(index)}) for {self.ndim}D array.")
        index = expand_ellipsis(index, self.shape)
        if not is_contiguous_view(index):
            # sequence / Tensor / mask selectors: a gathered copy
            # (reference: core.py:186-203)
            shape, strides, offset, new_index = _fancy.newview_indexing(self, index)
            view = Tensor._new_view(self._storage, shape, strides, offset)
            return _fancy.gather(view, _fancy.compute_plan(shape, new_index))
        view = _basic_index_view(self, index)
        return Tensor._new_view(self._storage, view[0], view[1], view[2])

    def __setitem__(self, index, value) -> None:
        if not isinstance(index, tuple):
            index = (index,)
        if self.ndim == 0:
            raise IndexError("Cannot index into a scalar tensor.")
        if len([x for x in index if x is not None]) > self.ndim:
            raise IndexError(f"Too many indices ({len(index)}) for {self.ndim}D array.")
        index = expand_ellipsis(index, self.shape)
        fancy = not is_contiguous_view(index)
        if fancy:
            shape, strides, offset, new_index = _fancy.newview_indexing(self, index)
        else:
            shape, strides, offset = _basic_index_view(self, index)
        if not isinstance(value, Tensor):
            value = Tensor(value, dtype=self.dtype, device=self.device)
        elif value.dtype != self.dtype:
            value = value.to(self.dtype)
        if value.device != self.device:
            value = value.to(self.device)
        target = Tensor._new_view(self._storage, shape, strides, offset)
        plan = _fancy.compute_plan(shape, new_index) if fancy else None
        try:
            value = value.expand(*(plan.new_shape if fancy else shape))
        except ValueError as e:
            raise IndexError(str(e)) from e
        if value._storage is self._storage:  # aliasing guard
            value = value._to_contiguous(force=True)
        if fancy:
            # scattered into the indexed view itself (the reference hands the
            # whole tensor to scatter_to_axes, core.py:246-253, which is only
            # right when no basic selector moved the view)
            _fancy.scatter(value, target, plan)
        else:
            K.copy_view(value, target)
        self._storage.bump_version()

    # -- properties --------------------------------------------------------------

    @property
    def dtype(self) -> Dtype:
        return self._storage.dtype

    @property
    def shape(self) -> TensorShape:
        return self._shape

    @property
    def ndim(self) -> int:
        return len(self._shape)

    @property
    def numel(self) -> int:
        return math.prod(self._shape)

    @property
    def is_empty(self) -> bool:
        return self.numel == 0

    @property
    def storage(self) -> Storage:
        return self._storage

    @property
    def strides(self) -> tuple[TensorShape, int]:
        """Returns (strides, offset)."""
        return self._strides, self._offset

    @property
    def device(self) -> Device:
        return self._storage.device

    @property
    def T(self) -> Tensor:
        from .autograd import TOp

        return TOp.apply(self)

    @property
    def version(self) -> int:
        return self._storage.version

    # -- conversion ----------------------------------------------------------------

    def to(self, target: Dtype | Device | str) -> Tensor:
        """Cast to a dtype or move to a device (no-op if already there)."""
        this = self
        if isinstance(target, Dtype):
            if target == self.dtype:
                return self
            if not this._is_contiguous(full_span=True):
                this = this._to_contiguous(force=True)
            new_buffer = K.cast(this._storage, target)
        else:
            device = get_std_device(target)
            if device == self.device:
                return self
            if not this._is_contiguous(full_span=True):
                this = this._to_contiguous(force=True)
            new_buffer = this._storage.to(device)
        out = Tensor._new_view(new_buffer, this._shape, this._strides, this._offset)
        if self.requires_grad and self.grad_fn is None:
            out.enable_grad()
        return out

    def cpu(self) -> Tensor:
        return self.to(Device.Cpu)

    def cuda(self) -> Tensor:
        return self.to(Device.Cuda)

    def numpy(self):
        """Host copy as a numpy array (needs numpy)."""
        import numpy as np

        c = self.cpu()._to_contiguous()
        names = {v: k for k, v in _NUMPY_DTYPES.items()}
        arr = np.frombuffer(c._storage.host_array(), dtype=names[c.dtype])
        return arr[c._offset : c._offset + c.numel].reshape(c._shape).copy()

    def clone(self) -> Tensor:
        if self._is_contiguous(full_span=True):
            return Tensor._new_contiguous(self._storage.clone(), self._shape)
        return self._to_contiguous(force=True)

    def flatten(self) -> Tensor:
        return self.reshape(self.numel)

    def equals(self, x2: Tensor) -> bool:
        """Same shape and equal values after dtype promotion."""
        if self.shape != x2.shape:
            return False
        if self.is_empty and x2.is_empty:
            return True
        promote = promote_dtypes(self.dtype, x2.dtype)
        first = self if promote == self.dtype else self.to(promote)
        if promote != x2.dtype:
            x2 = x2.to(promote)
        return K.equals(first, x2)

    def tolist(self) -> InputType:
        if self.device != Device.Cpu:
            raise RuntimeError("Tensor on device, call .cpu() first.")
        vals = K.host_values(self)
        if is_bool(self.dtype):
            vals = [bool(v) for v in vals]
        if self.ndim == 0:
            return vals[0]
        it = iter(vals)

        def rec(d: int):
            if d == self.ndim - 1:
                return [next(it) for _ in range(self._shape[d])]
            return [rec(d + 1) for _ in range(self._shape[d])]

        return rec(0)

    def item(self) -> bool | int | float:
        if self.numel != 1:
            raise RuntimeError(f"Cannot convert {self} to a scalar.")
        if self.device != Device.Cpu:
            raise RuntimeError("Tensor on device, call .cpu() first.")
        v = self._storage.host_array()[self._offset]
        return bool(v) if is_bool(self.dtype) else v

    def squeeze(self, *axes: int) -> Tensor:
        if len(axes) == 0:
            axes = tuple(range(self.ndim))
        axes = tuple(ax if ax >= 0 else ax + self.ndim for ax in axes)
        new_shape = [
            s for d, s in enumerate(self._shape) if not (d in axes and s == 1)
        ]
        return self.reshape(*new_shape)

    # -- ops bound in nanotorch_amd.__init__ -------------------------------------------

    def __add__(self, other): ...
    def __radd__(self, other): ...
    def __iadd__(self, other): ...
    def __sub__(self, other): ...
    def __rsub__(self, other): ...
    def __isub__(self, other): ...
    def __mul__(self, other): ...
    def __rmul__(self, other): ...
    def __imul__(self, other): ...
    def __truediv__(self, other): ...
    def __rtruediv__(self, other): ...
    def __itruediv__(self, other): ...
    def __neg__(self): ...
    def __matmul__(self, other): ...
    def __pow__(self, exponent): ...
    def __rpow__(self, exponent): ...
    def __eq__(self, other): ...  # type: ignore[override]
    def __gt__(self, other): ...
    def __ge__(self, other): ...
    def __lt__(self, other): ...
    def __le__(self, other): ...
    def exp(self) -> Tensor: ...
    def log(self) -> Tensor: ...
    def pow(self, exponent) -> Tensor: ...
    def sum(self, axis=None, keepdim=False, *, dtype=None) -> Tensor: ...
    def mean(self, axis=None, keepdim=False, *, dtype=None) -> Tensor: ...
    def max(self, axis=None, keepdim=False) -> Tensor: ...
    def min(self, axis=None, keepdim=False) -> Tensor: ...
    def reshape(self, *dims: int) -> Tensor: ...
    def transpose(self, dim0: int, dim1: int) -> Tensor: ...
    def expand(self, *dims: int) -> Tensor: ...

    # -- autograd ----------------------------------------------------------------------

    @property
    def requires_grad(self) -> bool:
        return self._requires_grad or self._grad_fn is not None

    @property
    def is_leaf(self) -> bool:
        return self._grad_fn is None

    @property
    def grad(self) -> Tensor | None:
        return self._grad

    @property
    def grad_fn(self) -> Function | None:
        return self._grad_fn

    def backward(self) -> None:
        """Backpropagate a scalar through the graph (core.py:511-526)."""
        if not self.requires_grad:
            raise RuntimeError(
                "Cannot call .backward() on a tensor that does not require grad "
                "and does not have a grad_fn."
            )
        if self.numel != 1:
            raise RuntimeError(
                f"Cannot call .backward() on a non-scalar tensor of shape {self.shape}"
            )
        seed = Tensor._new_contiguous(K.fill(1, 1.0, self.dtype, self.device), ())
        self._grad = seed if self._shape == () else seed.reshape(*self._shape)
        if not self.is_leaf:
            _backpropagate_grad(self)

    def attach_grad_fn(self, grad_fn: Function) -> None:
        self._grad_fn = grad_fn

    def zero_grad(self) -> None:
        self._grad = None

    def enable_grad(self) -> None:
        self._requires_grad = True

    # -- private -----------------------------------------------------------------------

    def _is_contiguous(self, full_span: bool = False) -> bool:
        if self._strides != _infer_strides(self._shape):
            return False
        if not full_span:
            return True
        return self._offset == 0 and self.numel == self._storage.size

    def _to_contiguous(self, force: bool = False) -> Tensor:
        if not force and self._is_contiguous():
            return self
        return Tensor._new_contiguous(K.clone_contiguous(self), self._shape)

    def _alias(self) -> Tensor:
        return Tensor._new_view(self._storage, self._shape, self._strides, self._offset)


# ------------------------------------------------------------------ helpers


def _extract_tensor_data(data, target_device: Device, user_dtype: Dtype | None):
    """Walks nested lists: shape, inferred dtype and flat values
    (reference: core.py:573-636)."""
    shape: list[int] = []
    flat: list = []
    auto_dtype: Dtype | None = None
    leaf_level: int | None = None

    def rec(node, level: int) -> None:
        nonlocal auto_dtype, leaf_level
        if level > MAX_TENSOR_LEVEL:
            raise ValueError(f"Maximum tensor depth reached: {MAX_TENSOR_LEVEL}")
        if isinstance(node, (bool, int, float)):
            if leaf_level is None:
                leaf_level = level
            elif level != leaf_level:
                raise ValueError("Leaf found at non-terminal level.")
            dt = dtype_from_type(node)
            if auto_dtype is None or dt > auto_dtype:
                auto_dtype = dt
            flat.append(node)
        elif isinstance(node, list):
            if level >= len(shape):
                shape.append(len(node))
            elif shape[level] != len(node):
                raise ValueError(
                    f"Unhomogeneous tensor shape detected ({shape[level]} != {len(node)})"
                )
            for child in node:
                rec(child, level + 1)
        else:
            raise TypeError(f"Unsupported tensor element type: {type(node)}")

    rec(data, 0)
    if auto_dtype is None:
        auto_dtype = Dtype.Float32
    final = Dtype(user_dtype) if user_dtype is not None else auto_dtype
    if is_bool(final):
        values = [bool(x) for x in flat]
    elif is_float(auto_dtype) and is_int(final):
        values = [int(x) for x in flat]
    else:
        values = flat
    return final, tuple(shape), Storage.from_iterable(values, final, target_device)


def _from_array_like(data, user_dtype, device):
    """Fast path for numpy-like arrays: copy the buffer directly."""
    name = str(getattr(data, "dtype", ""))
    dt = _NUMPY_DTYPES.get(name)
    if dt is None or (user_dtype is not None and Dtype(user_dtype) != dt):
        return None, None, None
    try:
        import numpy as np
    except ImportError:
        return None, None, None
    shape = tuple(np.shape(data))  # ascontiguousarray makes a 0-d array 1-d
    arr = np.ascontiguousarray(data)
    return Storage.from_buffer(arr, dt, device), shape, dt


def _infer_strides(shape: TensorShape) -> TensorShape:
    strides = []
    acc = 1
    for s in reversed(shape):
        strides.append(acc)
        acc *= s
    return tuple(reversed(strides))


def _str_list_compact(li: Any) -> str:
    if not isinstance(li, list) or len(li) < 8:
        return str(li)
    return (
        "["
        + ", ".join(str(x) for x in li[:3])
        + ", ..., "
        + ", ".join(str(x) for x in li[-3:])
        + "]"
    )


def _basic_index_view(x: Tensor, index: tuple):
    """int / slice / None indexing as (shape, strides, offset)
    (reference: core.py:777-830)."""
    offset = x._offset
    shape: list[int] = []
    strides: list[int] = []
    old = 0
    for sel in index:
        if sel is None:
            shape.append(1)
            strides.append(0)
            continue
        n = x._shape[old]
        if isinstance(sel, int):
            if sel < 0:
                sel += n
            if sel < 0 or sel >= n:
                raise IndexError(f"Cannot index at position {sel} in {n} elements.")
            offset += sel * x._strides[old]
        else:
            start, stop, step = sel.indices(n)
            shape.append(len(range(start, stop, step)))
            strides.append(x._strides[old] * step)
            offset += start * x._strides[old]
        old += 1
    while old < x.ndim:
        shape.append(x._shape[old])
        strides.append(x._strides[old])
        old += 1
    return tuple(shape), tuple(strides), offset


# ---------------------------------------------------------------- autograd


def _backpropagate_grad(seed: Tensor) -> None:
    """Backpropagation engine (reference: core.py:836-872).

    Nodes are gathered breadth-first while counting, for every tensor, how
    many graph edges consume it; a node's backward runs when its count drops
    to zero.  Gradients land in ``x._grad``: the first one is stored as is,
    later ones are added (``old + new``).  Functions that implement
    ``_backward_into`` compute and accumulate in one fused pass; others go
    through ``backward`` plus an in-place add.
    """
    to_visit = [seed]
    ncons = {id(seed): 0}
    order: list[tuple[Tensor, Any, tuple]] = []
    while to_visit:
        f_x = to_visit.pop(0)
        fn = f_x.grad_fn
        if fn is None:
            continue
        inputs = []
        for x in fn.inputs:
            if isinstance(x, Tensor):
                if x.requires_grad:
                    ncons[id(x)] = ncons.get(id(x), 0) + 1
                    to_visit.append(x)
                inputs.append(x)
        order.append((f_x, fn, tuple(inputs)))

    for f_x, fn, inputs in order:
        if f_x.grad is None:
            raise RuntimeError("f_x.grad is None.")
        ncons[id(f_x)] -= 1
        if ncons[id(f_x)] > 0:
            continue
        _run_backward(fn, f_x.grad, inputs)
        f_x._grad = None


def _has_overlap(t: Tensor) -> bool:
    return any(st == 0 and s > 1 for s, st in zip(t._shape, t._strides))


def _accumulation_target(x: Tensor) -> Tensor | None:
    """x's existing gradient, made safe to update in place.

    A gradient that shares storage with another tensor (the upstream
    gradient handed through by add/sub/views) or that is a broadcast view is
    first copied into a buffer of its own.  The reference adds in place into
    such tensors too, which also changes every tensor sharing the storage;
    here only x's gradient changes.
    """
    g = x._grad
    if g is None:
        return None
    if not getattr(x, "_grad_owned", False) or _has_overlap(g):
        g = g._to_contiguous(force=True)
        x._grad = g
        x._grad_owned = True
    return g


def _store_first(x: Tensor, r: Tensor, upstream: Tensor) -> None:
    x._grad = r
    x._grad_owned = r._storage is not upstream._storage


def _run_backward(fn, grad: Tensor, inputs: tuple) -> None:
    needs = [x.requires_grad for x in inputs]
    fused = getattr(fn, "_backward_into", None)
    distinct = len({id(x) for x in inputs}) == len(inputs)
    if fused is not None and fused.__self__.fused_ok():
        if distinct:
            groups = [list(range(len(inputs)))]
        else:
            # The same tensor feeds several inputs (e.g. x * x): hand out the
            # gradients one input at a time so each lands on the value the
            # previous one left, as `x._grad = g; x._grad += g2` does.
            groups = [[i] for i in range(len(inputs))]
        for grp in groups:
            sub_needs = [needs[i] and i in grp for i in range(len(inputs))]
            if not any(sub_needs):
                continue
            targets = [
                _accumulation_target(x) if n else None
                for x, n in zip(inputs, sub_needs)
            ]
            results = fused(grad, sub_needs, targets)
            for x, n, t, r in zip(inputs, sub_needs, targets, results):
                if n and t is None:
                    _store_first(x, r, grad)
        return
    grads = fn.backward(grad)
    for x, g in zip(inputs, grads):
        if not x.requires_grad:
            continue
        if x._grad is None:
            _store_first(x, g, grad)
        else:
            target = _accumulation_target(x)
            target += g


TensorLike = Tensor | float | int | bool | list
