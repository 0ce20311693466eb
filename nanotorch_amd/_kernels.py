"""Device operations on tensor views: the call surface of the reference's
``_C`` kernels (src/nanotorch/_C.pyi:63-136), implemented over libnt.

Every function takes ``Tensor`` views, checks that they live on the device,
builds ``nt_view`` descriptors and calls one C ABI entry point.  Outputs are
fresh contiguous buffers in the view's logical row-major order, as in the
reference (src/cpp/ops/unary_ops.cu:9-16, binary_ops.cu:10-19).
"""

from __future__ import annotations

import ctypes
import math

from . import _lib
from ._data_type import Dtype
from ._storage import Storage
from .cuda import Device


def require_device(*tensors) -> None:
    """Device ops run on the GPU only; host tensors are staging buffers."""
    for t in tensors:
        if t.device != Device.Cuda:
            raise RuntimeError(
                "nanotorch_amd computes on the GPU: move tensors to "
                "device='cuda' (host tensors only hold and transfer data)."
            )


def _check_same_device(*tensors) -> None:
    devs = {t.device for t in tensors}
    if len(devs) > 1:
        raise RuntimeError("Expected all tensors on the same device.")


def view_of(t) -> _lib.NtView:
    s = t._storage
    return _lib.make_view(s.data_ptr(), t._offset, int(s.dtype), t._shape, t._strides)


def flat_view(storage: Storage, shape, offset: int = 0) -> _lib.NtView:
    strides = []
    acc = 1
    for d in reversed(shape):
        strides.append(acc)
        acc *= d
    return _lib.make_view(
        storage.data_ptr(), offset, int(storage.dtype), tuple(shape), tuple(reversed(strides))
    )


def _numel(shape) -> int:
    return math.prod(shape)


# ------------------------------------------------------------- factories


def fill(n: int, value, dtype: Dtype, device: Device) -> Storage:
    if Device(device) == Device.Cpu:
        return Storage.from_iterable([value] * n, dtype, Device.Cpu)
    out = Storage.allocate(n, dtype, Device.Cuda)
    if n:
        _lib.call("nt_fill", out.data_ptr(), int(dtype), n, float(value))
    return out


# ------------------------------------------------------------ elementwise


def unary(op: int, x, scalar: float = 0.0) -> Storage:
    require_device(x)
    out = Storage.allocate(_numel(x._shape), x.dtype, Device.Cuda)
    vx = view_of(x)
    vo = flat_view(out, x._shape)
    _lib.call("nt_unary", op, ctypes.byref(vx), float(scalar), ctypes.byref(vo))
    return out


def binary(op: int, x1, x2) -> Storage:
    require_device(x1, x2)
    if x1._shape != x2._shape:
        raise RuntimeError("_dispatch_binary: Expected two views of the same shape.")
    out_dtype = Dtype.Bool if op in (_lib.EQ, _lib.GT, _lib.GE) else x1.dtype
    out = Storage.allocate(_numel(x1._shape), out_dtype, Device.Cuda)
    v1, v2 = view_of(x1), view_of(x2)
    vo = flat_view(out, x1._shape)
    _lib.call("nt_binary", op, ctypes.byref(v1), ctypes.byref(v2), ctypes.byref(vo))
    return out


def sgd_step(p, g, lr32: float) -> None:
    """p = p - (g * lr32) in one pass, in place (the two roundings of the
    reference's `p -= p.grad * lr`, nn/optimizers.py:45-51); float32
    device tensors of one shape, lr32 already a float32 value."""
    require_device(p, g)
    vp, vg = view_of(p), view_of(g)
    _lib.call("nt_sgd_step", ctypes.byref(vp), ctypes.byref(vg), lr32)
    p._storage.bump_version()


def inplace(op: int, out, other) -> None:
    """out = out (op) other, in place (reference: inplace_ops.cu:39-79)."""
    require_device(out, other)
    vo, v2 = view_of(out), view_of(other)
    _lib.call("nt_inplace", op, ctypes.byref(vo), ctypes.byref(v2))
    out._storage.bump_version()


def copy_view(src, out) -> None:
    """out[...] = src, both strided views of one shape (copy_ops.cu:187-203)."""
    _check_same_device(src, out)
    if out.device == Device.Cpu:
        _host_copy(src, out)
        return
    vs, vo = view_of(src), view_of(out)
    _lib.call("nt_copy", ctypes.byref(vs), ctypes.byref(vo))


def clone_contiguous(x) -> Storage:
    """Contiguous copy of a view (copy_ops.cu:205-217)."""
    out = Storage.allocate(_numel(x._shape), x.dtype, x.device)
    if x.device == Device.Cpu:
        vals = host_values(x)
        if vals:
            out.host_array()[: len(vals)] = vals
        return out
    if _numel(x._shape):
        vs = view_of(x)
        vo = flat_view(out, x._shape)
        _lib.call("nt_copy", ctypes.byref(vs), ctypes.byref(vo))
    return out


def cast(storage: Storage, dtype: Dtype) -> Storage:
    """Whole-buffer dtype conversion; on the device, no host round trip
    (the reference's CUDA cast copies to the host and back,
    src/cpp/storage.cpp:50-51)."""
    if dtype == storage.dtype:
        return storage
    n = storage.size
    if storage.device == Device.Cpu:
        src = storage.host_array()[:n]
        return Storage.from_iterable(src, dtype, Device.Cpu)
    out = Storage.allocate(n, dtype, Device.Cuda)
    if n:
        vs = flat_view(storage, (n,))
        vo = flat_view(out, (n,))
        _lib.call("nt_copy", ctypes.byref(vs), ctypes.byref(vo))
    return out


def equals(x1, x2) -> bool:
    _check_same_device(x1, x2)
    if x1.device == Device.Cpu:
        return host_values(x1) == host_values(x2)
    v1, v2 = view_of(x1), view_of(x2)
    res = ctypes.c_int32(0)
    _lib.call("nt_equals", ctypes.byref(v1), ctypes.byref(v2), ctypes.byref(res))
    return bool(res.value)


# ---------------------------------------------------------------- backward


def unary_bwd(op: int, g, saved, scalar: float, gx_target) -> "Storage | None":
    """Fused unary backward.  gx_target is an existing gradient tensor to
    accumulate into (in place) or None; returns the new storage when None."""
    require_device(g)
    vg = view_of(g)
    vs = view_of(saved) if saved is not None else None
    if gx_target is None:
        out = Storage.allocate(_numel(g._shape), g.dtype, Device.Cuda)
        vo = flat_view(out, g._shape)
        _lib.call("nt_unary_bwd", op, ctypes.byref(vg), _lib.ref(vs), float(scalar), ctypes.byref(vo), 0)
        return out
    vo = view_of(gx_target)
    _lib.call("nt_unary_bwd", op, ctypes.byref(vg), _lib.ref(vs), float(scalar), ctypes.byref(vo), 1)
    gx_target._storage.bump_version()
    return None


def binary_bwd(op: int, g, a, b, need_a: bool, target_a, need_b: bool, target_b):
    """Fused binary backward; returns (new_storage_a | None, new_storage_b | None)."""
    require_device(g)
    vg = view_of(g)
    va = view_of(a) if a is not None else None
    vb = view_of(b) if b is not None else None
    outs = []
    views = []
    for need, target in ((need_a, target_a), (need_b, target_b)):
        if not need:
            outs.append(None)
            views.append((None, 0))
        elif target is None:
            st = Storage.allocate(_numel(g._shape), g.dtype, Device.Cuda)
            outs.append(st)
            views.append((flat_view(st, g._shape), 0))
        else:
            outs.append(None)
            views.append((view_of(target), 1))
    (vga, acc_a), (vgb, acc_b) = views
    _lib.call(
        "nt_binary_bwd",
        op,
        ctypes.byref(vg),
        _lib.ref(va),
        _lib.ref(vb),
        _lib.ref(vga),
        acc_a,
        _lib.ref(vgb),
        acc_b,
    )
    for need, target in ((need_a, target_a), (need_b, target_b)):
        if need and target is not None:
            target._storage.bump_version()
    return outs[0], outs[1]


# -------------------------------------------------------------- reductions


def reduce(op: int, x, axes, out_dtype: Dtype, want_aux: bool = False):
    """Reduction over `axes` (tuple order); returns Storage or
    (Storage, idx Storage, count Storage) when want_aux (max/min)."""
    require_device(x)
    keep = [s for i, s in enumerate(x._shape) if i not in axes]
    k = _numel(keep)
    out = Storage.allocate(k, out_dtype, Device.Cuda)
    vx = view_of(x)
    vo = flat_view(out, (k,))
    idx = cnt = None
    vi = vc = None
    if want_aux:
        idx = Storage.allocate(k, Dtype.Int64, Device.Cuda)
        cnt = Storage.allocate(k, Dtype.Int32, Device.Cuda)
        vi = flat_view(idx, (k,))
        vc = flat_view(cnt, (k,))
    arr = _lib.axes_array(axes)
    _lib.call(
        "nt_reduce", op, ctypes.byref(vx), arr, len(axes), ctypes.byref(vo), _lib.ref(vi), _lib.ref(vc)
    )
    if want_aux:
        return out, idx, cnt
    return out


def reduce_bwd(op: int, g, scale: float, idx, cnt, axes, shape, target):
    """Backward of a reduction into a tensor of `shape`.  g holds one value
    per kept index (any shape, made contiguous here); accumulates into
    `target` when given, else returns a new contiguous Storage."""
    require_device(g)
    g = g._to_contiguous()
    k = g.numel
    vg = _lib.make_view(g._storage.data_ptr(), g._offset, int(g.dtype), (k,), (1,))
    vi = flat_view(idx, (k,)) if idx is not None else None
    vc = flat_view(cnt, (k,)) if cnt is not None else None
    arr = _lib.axes_array(axes)
    if target is None:
        out = Storage.allocate(_numel(shape), g.dtype, Device.Cuda)
        vo = flat_view(out, shape)
        acc = 0
    else:
        out = None
        vo = view_of(target)
        acc = 1
    _lib.call(
        "nt_reduce_bwd",
        op,
        ctypes.byref(vg),
        float(scale),
        _lib.ref(vi),
        _lib.ref(vc),
        arr,
        len(axes),
        ctypes.byref(vo),
        acc,
    )
    if target is not None:
        target._storage.bump_version()
    return out


# ------------------------------------------------------------------ matmul


def matmul(x1, x2, out_shape) -> Storage:
    """Batched matmul of same-rank views (batch dims already expanded)."""
    require_device(x1, x2)
    if x1.dtype != x2.dtype:
        raise RuntimeError("matmul: dtype mismatch")
    out = Storage.allocate(_numel(out_shape), x1.dtype, Device.Cuda)
    v1, v2 = view_of(x1), view_of(x2)
    vo = flat_view(out, out_shape)
    _lib.call("nt_matmul", ctypes.byref(v1), ctypes.byref(v2), ctypes.byref(vo), 0)
    return out


def matmul_bias(x1, x2, bias, out_shape) -> Storage:
    """x1 @ x2 + bias (2-D float32 views, bias 1-D over the columns) in one
    product whose epilogue adds the bias: the same two fp32 roundings as the
    product followed by a broadcast add."""
    require_device(x1, x2, bias)
    out = Storage.allocate(_numel(out_shape), x1.dtype, Device.Cuda)
    v1, v2, vb = view_of(x1), view_of(x2), view_of(bias)
    vo = flat_view(out, out_shape)
    _lib.call("nt_matmul_bias", ctypes.byref(v1), ctypes.byref(v2), ctypes.byref(vb),
              ctypes.byref(vo))
    return out


def matmul_into(x1, x2, target, accumulate: bool) -> None:
    require_device(x1, x2, target)
    v1, v2, vo = view_of(x1), view_of(x2), view_of(target)
    _lib.call("nt_matmul", ctypes.byref(v1), ctypes.byref(v2), ctypes.byref(vo), int(accumulate))
    target._storage.bump_version()


# ------------------------------------------------------------- host helpers


def host_values(x) -> list:
    """Values of a host view in logical row-major order."""
    arr = x._storage.host_array()
    shape, strides, off = x._shape, x._strides, x._offset
    n = _numel(shape)
    if n == 0:
        return []
    out = []

    def rec(d: int, base: int) -> None:
        if d == len(shape):
            out.append(arr[base])
            return
        st = strides[d]
        for i in range(shape[d]):
            rec(d + 1, base + i * st)

    rec(0, off)
    return out


def _host_copy(src, out) -> None:
    vals = host_values(src)
    if src.dtype != out.dtype:
        from ._storage import _convert

        vals = [_convert(v, out.dtype) for v in vals]
    arr = out._storage.host_array()
    shape, strides = out._shape, out._strides
    it = iter(vals)

    def rec(d: int, base: int) -> None:
        if d == len(shape):
            arr[base] = next(it)
            return
        for i in range(shape[d]):
            rec(d + 1, base + i * strides[d])

    if _numel(shape):
        rec(0, out._offset)
