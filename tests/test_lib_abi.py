"""The C ABI library loads without a GPU and exports every entry point that
include/nt.h declares (and the ctypes binding expects)."""

from __future__ import annotations

import ctypes
import os
import re

from conftest import ROOT

from nanotorch_amd import _lib


def _declared() -> list[str]:
    text = open(os.path.join(ROOT, "include", "nt.h")).read()
    return sorted(set(re.findall(r"^(?:int|const char \*)\s*(nt_\w+)\(", text, re.M)))


def test_header_declares_entry_points():
    names = _declared()
    assert "nt_matmul" in names and "nt_reduce" in names and len(names) >= 25


def test_library_exports_all_declared_symbols():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_matches_header():
    assert sorted(_lib.exported_symbols()) == _declared()


def test_load_and_status_without_device():
    lib = _lib.load()
    out = ctypes.c_int(-1)
    assert lib.nt_is_available(ctypes.byref(out)) == 0
    assert out.value in (0, 1)
    # the host generator needs no device
    buf = (ctypes.c_float * 2)()
    assert lib.nt_manual_seed(42) == 0
    assert lib.nt_host_uniform(ctypes.addressof(buf), 3, 2, 0.0, 1.0) == 0
    assert abs(buf[0] - 0.7551555037498474) < 1e-7


def test_view_struct_layout():
    # struct nt_view: void*, int64, int32, int32, int64[8], int64[8]
    assert ctypes.sizeof(_lib.NtView) == 8 + 8 + 4 + 4 + 64 + 64
    assert _lib.NtView.shape.offset == 24


def test_noalloc_entry_point_refuses_before_init():
    """nt_reduce_noalloc never initialises the library (initialisation
    allocates): before any other call it returns NT_ERR_RUNTIME."""
    lib = _lib.load()
    avail = ctypes.c_int(0)
    lib.nt_is_available(ctypes.byref(avail))
    if avail.value:
        return  # a GPU process may have initialised the library already
    rc = lib.nt_reduce_noalloc(0, None, None, 0, None, None, None)
    assert rc == _lib.NT_ERR_RUNTIME
    assert b"nt_init" in lib.nt_last_error()
