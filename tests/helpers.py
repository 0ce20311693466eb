"""Shared test helpers: numpy <-> device tensors, views, parity checks."""

from __future__ import annotations

import numpy as np

import nanotorch_amd as nt
from nanotorch_amd.core import Tensor

NP_DT = {
    np.dtype(np.bool_): nt.bool_,
    np.dtype(np.int32): nt.int32,
    np.dtype(np.int64): nt.int64,
    np.dtype(np.float32): nt.float32,
    np.dtype(np.float64): nt.float64,
}


def dev(a: np.ndarray, requires_grad: bool = False) -> Tensor:
    """Contiguous device tensor holding a copy of `a`."""
    a = np.ascontiguousarray(a)
    t = nt.Tensor(a, device="cuda")
    if requires_grad:
        t.enable_grad()
    return t


def dev_T(a: np.ndarray) -> Tensor:
    """Device tensor equal to `a` (2-D) but stored transposed: the `.T` view
    of a contiguous [C, R] storage, as config 2's strided variant."""
    return dev(np.ascontiguousarray(a.T)).T


def host(t: Tensor) -> np.ndarray:
    return t.numpy()


def bits(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype == np.float32:
        return a.view(np.uint32)
    if a.dtype == np.float64:
        return a.view(np.uint64)
    return a


def assert_bitexact(got: np.ndarray, want: np.ndarray, what: str = "") -> None:
    assert got.shape == want.shape, (what, got.shape, want.shape)
    assert got.dtype == want.dtype, (what, got.dtype, want.dtype)
    gb, wb = bits(got), bits(want)
    bad = np.nonzero(gb != wb)
    if bad[0].size:
        i = tuple(b[0] for b in bad)
        raise AssertionError(
            f"{what}: {bad[0].size} of {got.size} differ; first at {i}: "
            f"got {got[i]!r} want {want[i]!r}"
        )


def assert_rel(got: np.ndarray, want: np.ndarray, rel: float, what: str = "",
               scale: np.ndarray | None = None) -> None:
    """|got - want| <= rel * (|want| if scale is None else scale), elementwise."""
    assert got.shape == want.shape, (what, got.shape, want.shape)
    g = got.astype(np.float64)
    w = want.astype(np.float64)
    s = np.abs(w) if scale is None else scale
    err = np.abs(g - w)
    bad = err > rel * s
    # exact matches (incl. both zero / same inf) always pass
    bad &= ~(g == w)
    if bad.any():
        i = np.unravel_index(np.argmax(np.where(bad, err / np.maximum(s, 1e-300), 0)), g.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {g.size} outside rel {rel}; worst at {i}: "
            f"got {g[i]!r} want {w[i]!r} scale {s[i]!r}"
        )


def rng(seed: int = 0) -> np.random.Generator:
    return np.random.default_rng(seed)


def seed_of(*key) -> int:
    """Deterministic seed from a test's parameters (str hashes are salted)."""
    import zlib

    return zlib.crc32(repr(key).encode())
