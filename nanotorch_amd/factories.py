"""Tensor factories (reference: src/nanotorch/factories.py)."""

from __future__ import annotations

import ctypes
import math

from . import _kernels as K
from . import _lib
from . import _data_type as dt
from ._data_type import Dtype
from ._storage import Storage
from .core import Tensor
from .cuda import Device, DeviceLiteral, get_std_device


def tensor(data, *, dtype: Dtype | None = None, requires_grad: bool = False,
           device: Device | DeviceLiteral = Device.Cpu) -> Tensor:
    return Tensor(data, dtype=dtype, requires_grad=requires_grad, device=device)


def _factory(shape, storage: Storage, requires_grad: bool) -> Tensor:
    x = Tensor._new_contiguous(storage, tuple(shape))
    if requires_grad:
        x.enable_grad()
    return x


def zeros(*shape: int, dtype: Dtype = dt.float32, requires_grad: bool = False,
          device: Device | DeviceLiteral = Device.Cpu) -> Tensor:
    return _factory(shape, K.fill(math.prod(shape), 0, dtype, get_std_device(device)),
                    requires_grad)


def ones(*shape: int, dtype: Dtype = dt.float32, requires_grad: bool = False,
         device: Device | DeviceLiteral = Device.Cpu) -> Tensor:
    return _factory(shape, K.fill(math.prod(shape), 1, dtype, get_std_device(device)),
                    requires_grad)


def full(*shape: int, value, dtype: Dtype = dt.float32, requires_grad: bool = False,
         device: Device | DeviceLiteral = Device.Cpu) -> Tensor:
    return _factory(shape, K.fill(math.prod(shape), value, dtype, get_std_device(device)),
                    requires_grad)


def eye(n: int, dtype: Dtype = dt.float32, requires_grad: bool = False,
        device: Device | DeviceLiteral = Device.Cpu) -> Tensor:
    vals = [1 if i % (n + 1) == 0 else 0 for i in range(n * n)]
    st = Storage.from_iterable(vals, dtype, get_std_device(device))
    return _factory((n, n), st, requires_grad)


def arange(n: int, start: int = 0, step: int = 1, dtype: Dtype = dt.int64,
           requires_grad: bool = False,
           device: Device | DeviceLiteral = Device.Cpu) -> Tensor:
    """x[i] = start + i * step, i < n."""
    st = Storage.from_iterable([start + i * step for i in range(n)], dtype,
                               get_std_device(device))
    return _factory((n,), st, requires_grad)


def manual_seed(seed: int) -> None:
    """Seeds the one generator behind rand / randint (host and device draws
    continue the same stream)."""
    _lib.call("nt_manual_seed", int(seed) & (2**64 - 1))


def _uniform(n: int, dtype: Dtype, device: Device) -> Storage:
    """n draws of U[0, 1) in the reference's stream (factory.cu:73-83): on the
    device they are generated there, on the host written to host memory."""
    if device == Device.Cuda:
        st = Storage.allocate(n, dtype, Device.Cuda)
        if n:
            _lib.call("nt_device_uniform", st.data_ptr(), int(dtype), n, 0.0, 1.0)
        return st
    host = Storage(n, dtype, Device.Cpu)
    if n:
        _lib.call("nt_host_uniform", ctypes.addressof(host.host_array()), int(dtype), n,
                  0.0, 1.0)
    return host


def rand(*shape: int, dtype: Dtype = dt.float32, requires_grad: bool = False,
         device: Device | DeviceLiteral = Device.Cpu) -> Tensor:
    """U[0, 1) from the reference's 64-bit Mersenne Twister stream."""
    if dtype <= dt.int64:
        raise ValueError("rand() cannot output non-float values.")
    st = _uniform(math.prod(shape), dtype, get_std_device(device))
    return _factory(shape, st, requires_grad)


def randint(low: int, high: int, shape: tuple[int, ...] | None = None,
            dtype: Dtype = dt.int64, requires_grad: bool = False,
            device: Device | DeviceLiteral = Device.Cpu) -> Tensor:
    """trunc(U[0,1) * (high - low) + low) in float32, then int64, then dtype:
    the reference's composition (factories.py:241-253)."""
    if dtype == dt.bool_:
        raise ValueError("randint() cannot output bool values.")
    shp = () if shape is None else tuple(shape)
    n = math.prod(shp)
    device = get_std_device(device)
    if device == Device.Cuda:
        u = _factory(shp, _uniform(n, dt.float32, device), False)
        x = (u * (high - low) + low).to(dt.int64).to(dtype)
        if requires_grad:
            x.enable_grad()
        return x
    u = _uniform(n, dt.float32, device)
    # float32 arithmetic as in the reference: (u * f32(high - low)) + f32(low)
    f = ctypes.c_float
    span, lo = f(float(high - low)).value, f(float(low)).value
    vals = []
    for v in u.host_array()[:n]:
        prod = f(v * span).value
        vals.append(int(f(prod + lo).value))
    st = Storage.from_iterable(vals, dtype, get_std_device(device))
    x = _factory(shp, st, False)
    if requires_grad:
        x.enable_grad()
    return x
