"""Tensor value types.

Restates src/nanotorch/_data_type.py: the dtype order Bool < Int32 < Int64 <
Float32 < Float64 is the promotion order (``promote_dtypes`` is ``max``), and
Python scalars map to Bool / Int64 / Float32.
"""

from __future__ import annotations

import ctypes
import enum

InputType = list | float | int | bool


class Dtype(enum.IntEnum):
    """Tensor dtype; values are the C ABI codes (``enum nt_dtype``)."""

    Bool = 0
    Int32 = 1
    Int64 = 2
    Float32 = 3
    Float64 = 4

    def __bool__(self) -> bool:  # every dtype is truthy, Bool (0) included
        return True


_CTYPES = {
    Dtype.Bool: ctypes.c_bool,
    Dtype.Int32: ctypes.c_int32,
    Dtype.Int64: ctypes.c_int64,
    Dtype.Float32: ctypes.c_float,
    Dtype.Float64: ctypes.c_double,
}


def ctype_of(dtype: Dtype):
    return _CTYPES[Dtype(dtype)]


def sizeof(dtype: Dtype) -> int:
    """Bytes per element (reference: core.py:35-44)."""
    return ctypes.sizeof(_CTYPES[Dtype(dtype)])


def dtype_from_type(data: InputType) -> Dtype:
    """Automatically initializes a Dtype from item."""
    if isinstance(data, bool):
        return Dtype.Bool
    if isinstance(data, int):
        return Dtype.Int64
    if isinstance(data, float):
        return Dtype.Float32
    raise TypeError(f"Unsupported Tensor value type: {type(data)}")


def is_bool(x: Dtype) -> bool:
    return x == Dtype.Bool


def is_int(x: Dtype) -> bool:
    return x in (Dtype.Int32, Dtype.Int64)


def is_float(x: Dtype) -> bool:
    return x in (Dtype.Float32, Dtype.Float64)


def promote_dtypes(*dtypes: Dtype) -> Dtype:
    """Compute the highest precision Dtype."""
    if not dtypes:
        return Dtype.Float32
    return Dtype(max(dtypes))


bool_ = Dtype.Bool
int32 = Dtype.Int32
int64 = Dtype.Int64
float32 = Dtype.Float32
float64 = Dtype.Float64
