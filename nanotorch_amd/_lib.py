"""ctypes binding of libnt.so, the HIP library behind every device op.

This module plays the role of the reference's pybind11 module
``nanotorch._C`` (src/cpp/_C.cpp:12-24): it loads the shared library that sits
next to this file, declares the C ABI of ``include/nt.h`` and converts status
codes into the exception types the reference raises (``RuntimeError`` for
shape/dtype/device mismatches and HIP errors, ``ValueError`` for unsupported
dtypes and bad matmul shapes).

There is no fallback: if ``libnt.so`` is missing or cannot be loaded, every
device operation raises.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_int64
from ctypes import c_size_t, c_uint64, c_void_p

NT_MAX_DIMS = 8

# nt_status
NT_OK = 0
NT_ERR_RUNTIME = 1
NT_ERR_VALUE = 2
NT_ERR_INDEX = 3
NT_ERR_OOM = 4

# nt_unary_op
EXP, LOG, NEG, RELU, SQRT, TANH, SIGMOID, POW = range(8)
# nt_binary_op
ADD, SUB, MUL, DIV, EQ, GT, GE, COPY = range(8)
# nt_reduce_op
R_SUM, R_MAX, R_MIN, R_ARGMAX, R_ARGMIN, R_MEAN = range(6)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libnt.so")


class NtView(ctypes.Structure):
    """Mirror of ``struct nt_view`` (include/nt.h)."""

    _fields_ = [
        ("data", c_void_p),
        ("offset", c_int64),
        ("dtype", c_int32),
        ("ndim", c_int32),
        ("shape", c_int64 * NT_MAX_DIMS),
        ("strides", c_int64 * NT_MAX_DIMS),
    ]


_VP = POINTER(NtView)

# name -> (restype, argtypes)
_SIGNATURES = {
    "nt_init": (c_int, []),
    "nt_is_available": (c_int, [POINTER(c_int)]),
    "nt_sync": (c_int, []),
    "nt_last_error": (c_char_p, []),
    "nt_malloc": (c_int, [POINTER(c_void_p), c_size_t]),
    "nt_free": (c_int, [c_void_p]),
    "nt_empty_cache": (c_int, []),
    "nt_memory_stats": (c_int, [POINTER(c_size_t), POINTER(c_size_t)]),
    "nt_memcpy_h2d": (c_int, [c_void_p, c_void_p, c_size_t]),
    "nt_memcpy_d2h": (c_int, [c_void_p, c_void_p, c_size_t]),
    "nt_memcpy_d2d": (c_int, [c_void_p, c_void_p, c_size_t]),
    "nt_fill": (c_int, [c_void_p, c_int32, c_int64, c_double]),
    "nt_copy": (c_int, [_VP, _VP]),
    "nt_unary": (c_int, [c_int32, _VP, c_double, _VP]),
    "nt_binary": (c_int, [c_int32, _VP, _VP, _VP]),
    "nt_inplace": (c_int, [c_int32, _VP, _VP]),
    "nt_equals": (c_int, [_VP, _VP, POINTER(c_int32)]),
    "nt_unary_bwd": (c_int, [c_int32, _VP, _VP, c_double, _VP, c_int32]),
    "nt_sgd_step": (c_int, [_VP, _VP, c_double]),
    "nt_binary_bwd": (c_int, [c_int32, _VP, _VP, _VP, _VP, c_int32, _VP, c_int32]),
    "nt_reduce": (c_int, [c_int32, _VP, POINTER(c_int64), c_int32, _VP, _VP, _VP]),
    "nt_reduce_noalloc": (c_int, [c_int32, _VP, POINTER(c_int64), c_int32, _VP, _VP, _VP]),
    "nt_reduce_bwd": (
        c_int,
        [c_int32, _VP, c_double, _VP, _VP, POINTER(c_int64), c_int32, _VP, c_int32],
    ),
    "nt_matmul": (c_int, [_VP, _VP, _VP, c_int32]),
    "nt_matmul_bias": (c_int, [_VP, _VP, _VP, _VP]),
    "nt_gather_axes": (
        c_int,
        [_VP, _VP, c_int32, POINTER(c_int32), _VP, POINTER(c_int32), POINTER(c_int32)],
    ),
    "nt_scatter_axes": (
        c_int,
        [_VP, _VP, c_int32, POINTER(c_int32), _VP, POINTER(c_int32), POINTER(c_int32), _VP],
    ),
    "nt_manual_seed": (c_int, [c_uint64]),
    "nt_host_uniform": (c_int, [c_void_p, c_int32, c_int64, c_double, c_double]),
    "nt_device_uniform": (c_int, [c_void_p, c_int32, c_int64, c_double, c_double]),
    "nt_rng_prepare": (c_int, []),
    "nt_event_create": (c_int, [POINTER(c_void_p)]),
    "nt_event_record": (c_int, [c_void_p]),
    "nt_event_elapsed_ms": (c_int, [c_void_p, c_void_p, POINTER(c_float)]),
    "nt_event_destroy": (c_int, [c_void_p]),
    "nt_launch_stats": (c_int, [POINTER(c_uint64), POINTER(c_uint64), POINTER(c_uint64)]),
}

_lib: ctypes.CDLL | None = None
_load_error: str | None = None


def load() -> ctypes.CDLL:
    """Returns the loaded library, raising ImportError if it is unavailable."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if _load_error is not None:
        raise ImportError(_load_error)
    if not os.path.exists(LIB_PATH):
        _load_error = (
            f"libnt.so not found at {LIB_PATH}; build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'` or "
            "`make -C nanotorch_amd/csrc`"
        )
        raise ImportError(_load_error)
    try:
        lib = ctypes.CDLL(LIB_PATH)
    except OSError as e:
        _load_error = f"cannot load {LIB_PATH}: {e}"
        raise ImportError(_load_error) from e
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def exported_symbols() -> list[str]:
    """Names of the C ABI entry points this binding expects."""
    return list(_SIGNATURES)


def check(rc: int) -> None:
    """Raises the exception matching a non-zero nt_status."""
    if rc == NT_OK:
        return
    msg = load().nt_last_error().decode(errors="replace")
    if rc == NT_ERR_VALUE:
        raise ValueError(msg)
    if rc == NT_ERR_INDEX:
        raise IndexError(msg)
    if rc == NT_ERR_OOM:
        raise MemoryError(msg)
    raise RuntimeError(msg)


def call(name: str, *args) -> None:
    """Calls a status-returning entry point and raises on failure."""
    check(getattr(load(), name)(*args))


def is_available() -> bool:
    try:
        lib = load()
    except ImportError:
        return False
    out = c_int(0)
    lib.nt_is_available(ctypes.byref(out))
    return bool(out.value)


def make_view(data: int | None, offset: int, dtype: int, shape, strides) -> NtView:
    v = NtView()
    v.data = data
    v.offset = offset
    v.dtype = int(dtype)
    nd = len(shape)
    if nd > NT_MAX_DIMS:
        raise RuntimeError(f"Tensors are limited to {NT_MAX_DIMS} dims on device.")
    v.ndim = nd
    for i in range(nd):
        v.shape[i] = shape[i]
        v.strides[i] = strides[i]
    return v


def ref(v: NtView | None):
    return None if v is None else ctypes.byref(v)


def axes_array(axes) -> ctypes.Array:
    arr = (c_int64 * max(1, len(axes)))()
    for i, a in enumerate(axes):
        arr[i] = a
    return arr


class Event:
    """HIP event recorded on the library stream."""

    def __init__(self) -> None:
        self._ev = c_void_p()
        call("nt_event_create", ctypes.byref(self._ev))

    def record(self) -> None:
        call("nt_event_record", self._ev)

    def elapsed_ms(self, end: "Event") -> float:
        ms = c_float(0.0)
        call("nt_event_elapsed_ms", self._ev, end._ev, ctypes.byref(ms))
        return float(ms.value)

    def __del__(self) -> None:
        if _lib is not None and self._ev:
            _lib.nt_event_destroy(self._ev)
