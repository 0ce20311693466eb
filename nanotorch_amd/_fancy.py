"""Advanced (sequence / mask) indexing: the index plan and its execution.

The plan restates the reference's ``_newview_indexing`` and ``_FancyAxes``
(src/nanotorch/core.py:667-830): basic selectors (int, slice, None) first
make a view; the remaining sequence / Tensor / boolean-mask selectors sit on
that view's axes ("fancy" axes).  Index values are normalised (negative +=
axis length) and range-checked on the host, with the reference's error types;
masks (1-D only) become index lists; the index arrays are broadcast to one
shape.  The output shape puts the index shape in place of the fancy axes when
they are adjacent, and first otherwise.

Execution: on the device through ``nt_gather_axes`` / ``nt_scatter_axes``
(the reference's ``gather_from_axes`` / ``scatter_to_axes``,
src/cpp/ops/copy_ops.cu:7-160, which are host-only there); on host tensors
with numpy over the same plan.  A scatter whose index tuples repeat keeps the
last occurrence, as the reference's sequential loop does.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import TYPE_CHECKING, Sequence

import numpy as np

from . import _lib
from ._data_type import Dtype
from ._indexing import TensorShape, broadcast_shapes
from .cuda import Device

if TYPE_CHECKING:
    from .core import Tensor


def newview_indexing(x: "Tensor", index: tuple):
    """Applies the basic selectors: (shape, strides, offset, new_index),
    where new_index holds each remaining fancy selector at its view axis
    (reference: core.py:777-830)."""
    offset = x._offset
    shape: list[int] = []
    strides: list[int] = []
    new_index: list = []
    old = new = 0
    while old < x.ndim or new < len(index):
        if new >= len(index) or (
            not isinstance(index[new], (int, slice)) and index[new] is not None
        ):
            shape.append(x._shape[old])
            strides.append(x._strides[old])
            new_index.append(None if new >= len(index) else index[new])
            old += 1
            new += 1
            continue
        sel = index[new]
        if sel is None:
            shape.append(1)
            strides.append(0)
            new_index.append(None)
            new += 1
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
            new_index.append(None)
            offset += start * x._strides[old]
        old += 1
        new += 1
    return tuple(shape), tuple(strides), offset, tuple(new_index)


@dataclass
class FancyPlan:
    """The reference's _FancyAxes (core.py:667-774), with host index arrays."""

    new_shape: TensorShape
    fancy_dims_in_src: list[int]
    index_arrays: list[np.ndarray]  # int64, each of the broadcast index shape
    out_axis_is_fancy: list[bool]
    out_axis_target: list[int]

    @property
    def index_shape(self) -> TensorShape:
        return self.index_arrays[0].shape

    def keep_last(self) -> np.ndarray | None:
        """Bool array over the index shape marking the last occurrence of
        every index tuple, or None when no tuple repeats."""
        n = int(np.prod(self.index_shape, dtype=np.int64))
        if n <= 1:
            return None
        tuples = np.stack([a.reshape(-1) for a in self.index_arrays], axis=1)
        rev = tuples[::-1]
        _, first_in_rev = np.unique(rev, axis=0, return_index=True)
        if len(first_in_rev) == n:
            return None
        keep = np.zeros(n, dtype=np.bool_)
        keep[n - 1 - first_in_rev] = True
        return keep.reshape(self.index_shape)


def _selector_values(sel) -> np.ndarray:
    """Host array of an index selector, typed as the reference's
    ``Tensor(sel)`` would be (bool / int64 / float32 / ...)."""
    from .core import Tensor

    if isinstance(sel, Tensor):
        return sel.numpy()
    if isinstance(sel, Sequence) and not isinstance(sel, (str, bytes)):
        try:
            return Tensor(sel).numpy()
        except Exception as e:  # the reference's message and type
            raise IndexError(f"Could not interpret index as a Tensor: {e}")
    raise IndexError(f"Unexpected selector type {type(sel)}")


def compute_plan(shape: TensorShape, index: tuple) -> FancyPlan:
    fancy_dims: list[int] = []
    basic_axes: list[int] = []
    basic_shape: list[int] = []
    raw: list[np.ndarray] = []
    for dim in range(len(shape)):
        if dim >= len(index) or index[dim] is None or isinstance(index[dim], (int, slice)):
            basic_axes.append(dim)
            basic_shape.append(shape[dim])
            continue
        vals = np.array(_selector_values(index[dim]), copy=True)
        # negative -> += axis length, then range check, on the values as
        # stored (a mask's True compares as 1) -- reference core.py:705-712
        flat = vals.reshape(-1)
        if flat.dtype != np.bool_:
            neg = flat < 0
            if neg.any():
                flat[neg] = flat[neg] + shape[dim]
            bad = (flat < 0) | (flat >= shape[dim])
        else:
            bad = flat.astype(np.int64) >= shape[dim]
        if bad.any():
            v = flat[np.argmax(bad)]
            raise IndexError(f"Invalid index {v} in axis of len {shape[dim]}.")
        vals = flat.reshape(vals.shape)
        if vals.dtype == np.bool_:
            if vals.ndim > 1:
                raise NotImplementedError("nD boolean masks not here (yet).")
            if len(vals) != shape[dim]:
                raise IndexError(
                    f"Wrong boolean index shape: {len(vals)} (expected {shape[dim]})."
                )
            vals = np.nonzero(vals)[0]
        fancy_dims.append(dim)
        raw.append(vals.astype(np.int64))  # static_cast, as Tensor.to(Int64)

    ind_shape = broadcast_shapes(*(a.shape for a in raw))
    arrays = [np.ascontiguousarray(np.broadcast_to(a, ind_shape)) for a in raw]

    nfancy = len(fancy_dims)
    nidx = len(ind_shape)
    gaps = [fancy_dims[i + 1] - fancy_dims[i] for i in range(nfancy - 1)]
    is_fancy: list[bool] = []
    target: list[int] = []
    if nfancy > 0 and any(g != 1 for g in gaps):  # not adjacent: index dims first
        new_shape = tuple(list(ind_shape) + basic_shape)
        for i in range(len(new_shape)):
            if i < nidx:
                is_fancy.append(True)
                target.append(i)
            else:
                is_fancy.append(False)
                target.append(basic_axes[i - nidx])
    else:
        a0 = fancy_dims[0]
        new_shape = tuple(basic_shape[:a0] + list(ind_shape) + basic_shape[a0:])
        for i in range(len(new_shape)):
            if i < a0:
                is_fancy.append(False)
                target.append(basic_axes[i])
            elif i < a0 + nidx:
                is_fancy.append(True)
                target.append(i - a0)
            else:
                is_fancy.append(False)
                target.append(basic_axes[i - nidx])
    return FancyPlan(new_shape, fancy_dims, arrays, is_fancy, target)


# ------------------------------------------------------------------ execution


def _host_offsets(plan: FancyPlan, vshape, vstrides, voffset) -> np.ndarray:
    """Storage offsets, over the plan's output shape, of the indexed view's
    elements (the address computation of copy_ops.cu:120-139)."""
    nd = len(plan.new_shape)
    off = np.full((1,) * nd, voffset, dtype=np.int64)
    fancy_pos = [i for i in range(nd) if plan.out_axis_is_fancy[i]]
    a0 = fancy_pos[0] if fancy_pos else 0
    nidx = len(plan.index_shape)
    slot = {d: q for q, d in enumerate(plan.fancy_dims_in_src)}
    for i in range(nd):
        if plan.out_axis_is_fancy[i]:
            continue
        d = plan.out_axis_target[i]
        shp = [1] * nd
        shp[i] = plan.new_shape[i]
        off = off + (np.arange(plan.new_shape[i], dtype=np.int64) * vstrides[d]).reshape(shp)
    for d in range(len(vshape)):
        if d not in slot:
            continue
        contrib = plan.index_arrays[slot[d]] * vstrides[d]
        off = off + contrib.reshape([1] * a0 + list(plan.index_shape) + [1] * (nd - a0 - nidx))
    return np.broadcast_to(off, plan.new_shape)


def _device_call(fn: str, plan: FancyPlan, first, second, keep=None) -> None:
    from .core import Tensor
    from . import _kernels as K

    nf = len(plan.fancy_dims_in_src)
    idx_tensors = [Tensor(a, dtype=Dtype.Int64, device="cuda") for a in plan.index_arrays]
    views = (_lib.NtView * nf)(*[K.view_of(t) for t in idx_tensors])
    fd = (ctypes.c_int32 * nf)(*plan.fancy_dims_in_src)
    nd = len(plan.new_shape)
    isf = (ctypes.c_int32 * max(nd, 1))(*[1 if b else 0 for b in plan.out_axis_is_fancy])
    tgt = (ctypes.c_int32 * max(nd, 1))(*plan.out_axis_target)
    va, vb = K.view_of(first), K.view_of(second)
    args = [ctypes.byref(va), ctypes.byref(vb), nf, fd, views, isf, tgt]
    if fn == "nt_scatter_axes":
        if keep is not None:
            kt = Tensor(keep, dtype=Dtype.Bool, device="cuda")
            vk = K.view_of(kt)
            args.append(ctypes.byref(vk))
        else:
            args.append(None)
    _lib.call(fn, *args)


def gather(view: "Tensor", plan: FancyPlan) -> "Tensor":
    """Contiguous tensor of the plan's shape with the view's indexed values."""
    from .core import Tensor
    from ._storage import Storage

    n = int(np.prod(plan.new_shape, dtype=np.int64))
    store = Storage.allocate(n, view.dtype, view.device)
    out = Tensor._new_contiguous(store, plan.new_shape)
    if n == 0:
        return out
    if view.device == Device.Cpu:
        src = np.ctypeslib.as_array(view._storage.host_array())
        offs = _host_offsets(plan, view._shape, view._strides, view._offset)
        np.ctypeslib.as_array(store.host_array())[:n] = src[offs.reshape(-1)]
        return out
    _device_call("nt_gather_axes", plan, view, out)
    return out


def scatter(value: "Tensor", view: "Tensor", plan: FancyPlan) -> None:
    """view[indexed] = value, value already of the plan's shape (any strides)."""
    n = int(np.prod(plan.new_shape, dtype=np.int64))
    if n == 0:
        return
    keep = plan.keep_last()
    if view.device == Device.Cpu:
        dst = np.ctypeslib.as_array(view._storage.host_array())
        offs = _host_offsets(plan, view._shape, view._strides, view._offset)
        vals = np.broadcast_to(value.numpy(), plan.new_shape)
        if keep is not None:
            m = np.broadcast_to(
                keep.reshape(
                    [1] * (plan.out_axis_is_fancy.index(True))
                    + list(plan.index_shape)
                    + [1] * (len(plan.new_shape) - plan.out_axis_is_fancy.index(True)
                             - len(plan.index_shape))
                ),
                plan.new_shape,
            )
            offs, vals = offs[m], vals[m]
        dst[offs.reshape(-1)] = np.asarray(vals).reshape(-1)
        return
    _device_call("nt_scatter_axes", plan, value, view, keep)
