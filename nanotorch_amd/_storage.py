"""Typed 1-D buffers on the host or on the device.

Counterpart of the reference's ``Storage`` (src/cpp/storage.h:18-66,
src/cpp/storage.cpp): a refcounted typed buffer with a ``version`` counter
bumped by in-place ops.  Device buffers come from libnt's caching allocator
and go back to it when the Python object dies.  Host buffers are ctypes
arrays, which expose the buffer protocol like the reference's storage does.
"""

from __future__ import annotations

import ctypes

from . import _lib
from ._data_type import Dtype, ctype_of, sizeof
from .cuda import Device


class Storage:
    __slots__ = ("_dtype", "_device", "_size", "_ptr", "_host", "version", "__weakref__")

    def __init__(self, size: int, dtype: Dtype, device: Device, *, _zero: bool = True):
        self._dtype = Dtype(dtype)
        self._device = Device(device)
        self._size = int(size)
        self.version = 0
        self._ptr = None
        self._host = None
        if self._device == Device.Cpu:
            self._host = (ctype_of(self._dtype) * max(1, self._size))()
        else:
            p = ctypes.c_void_p()
            _lib.call("nt_malloc", ctypes.byref(p), max(1, self._size) * sizeof(self._dtype))
            self._ptr = p.value
            if _zero and self._size > 0:
                _lib.call("nt_fill", self._ptr, int(self._dtype), self._size, 0.0)

    # -- constructors -----------------------------------------------------

    @classmethod
    def allocate(cls, size: int, dtype: Dtype, device: Device) -> "Storage":
        """Uninitialised (device) or zeroed (host) buffer."""
        return cls(size, dtype, device, _zero=False)

    @classmethod
    def from_iterable(cls, values, dtype: Dtype, device: Device) -> "Storage":
        values = list(values)
        host = cls(len(values), dtype, Device.Cpu)
        if values:
            host._host[: len(values)] = [_convert(v, dtype) for v in values]
        return host if Device(device) == Device.Cpu else host.to(device)

    @classmethod
    def from_buffer(cls, buf, dtype: Dtype, device: Device) -> "Storage":
        """Copies a C-contiguous buffer (e.g. a numpy array) of matching dtype.

        Objects exposing ``__array_interface__`` are copied to the device
        straight from their memory; other buffers go through a host copy.
        """
        mv = memoryview(buf)
        if not mv.c_contiguous:
            raise ValueError("from_buffer needs a C-contiguous buffer")
        nbytes = mv.nbytes
        n = nbytes // sizeof(dtype)
        device = Device(device)
        iface = getattr(buf, "__array_interface__", None)
        if device == Device.Cuda and iface is not None and n:
            out = cls(n, dtype, Device.Cuda, _zero=False)
            _lib.call("nt_memcpy_h2d", out._ptr, iface["data"][0], nbytes)
            return out
        host = cls(n, dtype, Device.Cpu)
        if n:
            memoryview(host._host).cast("B")[:nbytes] = mv.cast("B")
        return host if device == Device.Cpu else host.to(device)

    # -- properties -------------------------------------------------------

    @property
    def dtype(self) -> Dtype:
        return self._dtype

    @property
    def device(self) -> Device:
        return self._device

    @property
    def size(self) -> int:
        return self._size

    @property
    def nbytes(self) -> int:
        return self._size * sizeof(self._dtype)

    def data_ptr(self) -> int:
        """Device address (device storage) or host address (host storage)."""
        if self._device == Device.Cpu:
            return ctypes.addressof(self._host)
        return self._ptr

    def host_array(self):
        if self._device != Device.Cpu:
            raise RuntimeError("Storage on device, call .cpu() first.")
        return self._host

    def __len__(self) -> int:
        return self._size

    def bump_version(self) -> None:
        self.version += 1

    # -- transfers --------------------------------------------------------

    def to(self, device: Device) -> "Storage":
        device = Device(device)
        if device == self._device:
            return self
        out = Storage(self._size, self._dtype, device, _zero=False)
        if self._size:
            if device == Device.Cuda:
                _lib.call("nt_memcpy_h2d", out._ptr, ctypes.addressof(self._host), self.nbytes)
            else:
                _lib.call("nt_memcpy_d2h", ctypes.addressof(out._host), self._ptr, self.nbytes)
        return out

    def clone(self) -> "Storage":
        out = Storage(self._size, self._dtype, self._device, _zero=False)
        if self._size:
            if self._device == Device.Cuda:
                _lib.call("nt_memcpy_d2d", out._ptr, self._ptr, self.nbytes)
            else:
                ctypes.memmove(out._host, self._host, self.nbytes)
        return out

    def __del__(self) -> None:
        ptr = getattr(self, "_ptr", None)
        if ptr is not None and _lib._lib is not None:
            _lib._lib.nt_free(ptr)
            self._ptr = None


def _convert(v, dtype: Dtype):
    """Python value -> value stored in a buffer of dtype (static_cast rules)."""
    if dtype == Dtype.Bool:
        return bool(v)
    if dtype in (Dtype.Int32, Dtype.Int64):
        return int(v)
    return float(v)
