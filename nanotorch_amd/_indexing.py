"""Shape helpers (restating src/nanotorch/_indexing.py:8-58)."""

from __future__ import annotations

from types import EllipsisType

TensorShape = tuple[int, ...]


def broadcast_shapes(*shapes: TensorShape) -> TensorShape:
    """Right-aligned broadcast of shapes; RuntimeError if incompatible."""
    if not shapes:
        return tuple()
    final = list(shapes[0])
    for s in shapes[1:]:
        s = list(s)
        if len(s) < len(final):
            s = [1] * (len(final) - len(s)) + s
        elif len(s) > len(final):
            final = [1] * (len(s) - len(final)) + final
        for i in range(len(final)):
            if final[i] == 1:
                final[i] = s[i]
            elif s[i] != 1 and final[i] != s[i]:
                raise RuntimeError(f"Cannot broadcast shapes {s} and {final}.")
    return tuple(final)


def expand_ellipsis(index: tuple, shape: TensorShape) -> tuple:
    """Expands an ellipsis into full slices: [..., 0] -> [:, :, :, 0]."""
    if len(index) == 0:
        return ()
    if sum(isinstance(i, EllipsisType) for i in index) > 1:
        raise IndexError("Multiple ellipses detected.")
    ndim = len(shape)
    nind = sum(i is not None for i in index)
    out: list = []
    for elem in index:
        if isinstance(elem, EllipsisType):
            out.extend([slice(None)] * (ndim - nind + 1))
        else:
            out.append(elem)
    return tuple(out)


def is_contiguous_view(index: tuple) -> bool:
    """True if the indexing is expressible as a strided view (no copy)."""
    return all(isinstance(i, (int, slice)) or i is None for i in index)
