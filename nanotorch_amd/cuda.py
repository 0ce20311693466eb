"""Device selection (reference: src/nanotorch/cuda.py:1-31).

``"cuda"`` names the MI355X; the name is kept so that code written for the
reference's GPU path runs unchanged.
"""

from __future__ import annotations

import enum
from typing import Literal

from . import _lib


class Device(enum.IntEnum):
    Cpu = 0
    Cuda = 1


DeviceLiteral = Literal["cpu", "cuda"]


def is_available() -> bool:
    """True if a HIP device and libnt.so are usable."""
    return _lib.is_available()


def sync() -> None:
    """Waits for all queued device work."""
    _lib.call("nt_sync")


def get_std_device(device: Device | str) -> Device:
    """Converts any device repr to standard Device."""
    if isinstance(device, Device):
        return device
    if device == "cpu":
        return Device.Cpu
    if device == "cuda":
        return Device.Cuda
    raise ValueError(f"Unknown device {device}.")
