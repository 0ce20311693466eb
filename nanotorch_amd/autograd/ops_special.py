"""View ops: reshape, expand, T, transpose (no copy unless a reshape needs a
contiguous input).  Restates src/nanotorch/autograd/ops_special.py:12-162."""

from __future__ import annotations

import math

from ..core import Tensor
from .function import Function
from .ops_utils import unbroadcast


class ReshapeOp(Function):
    """Reshaped view; copies first if the input is not contiguous."""

    def forward(self, x: Tensor, *dims: int) -> Tensor:
        if math.prod(dims) != x.numel:
            raise ValueError(f"Can't reshape {x.shape} into {dims}.")
        self._shape = x.shape
        if dims == x.shape:
            return x
        x = x._to_contiguous()
        return Tensor._new_view(x.storage, tuple(dims), None, x._offset)

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        return (grad_out.reshape(*self._shape),)


class ExpandOp(Function):
    """Broadcast view to `dims` (size-1 axes get stride 0; new leading axes
    are prepended)."""

    def forward(self, x: Tensor, *dims: int) -> Tensor:
        if len(dims) < x.ndim:
            raise ValueError(f"Cannot broadcast {x.shape} to {dims}.")
        self._orig_shape = x.shape
        if dims == x.shape:
            return x
        strides = list(x._strides)
        for i in range(len(dims)):
            if i >= x.ndim:
                strides = [0] + strides
            else:
                src, tgt = x.shape[-i - 1], dims[-i - 1]
                if src == tgt:
                    continue
                if src == 1:
                    strides[-i - 1] = 0
                else:
                    raise ValueError(f"Cannot broadcast {x.shape} to {dims} (mismatch).")
        return Tensor._new_view(x.storage, tuple(dims), tuple(strides), x._offset)

    def backward(self, grad_out: Tensor) -> tuple[Tensor]:
        return (unbroadcast(grad_out, self._orig_shape),)


class TOp(Function):
    """All axes reversed (x.T)."""

    def forward(self, x: Tensor) -> Tensor:
        if x.ndim < 2:
            return x
        strides, offset = x.strides
        return Tensor._new_view(
            x.storage, tuple(reversed(x.shape)), tuple(reversed(strides)), offset
        )

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        return (grad_out.T,)


class TransposeOp(Function):
    """Swaps two axes (view)."""

    def forward(self, x: Tensor, dim0: int, dim1: int) -> Tensor:
        self._dim0, self._dim1 = dim0, dim1
        if x.ndim < 2 or dim0 == dim1:
            return x
        strides, offset = x.strides
        shape, st = list(x.shape), list(strides)
        shape[dim0], shape[dim1] = shape[dim1], shape[dim0]
        st[dim0], st[dim1] = st[dim1], st[dim0]
        return Tensor._new_view(x.storage, tuple(shape), tuple(st), offset)

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        return (grad_out.transpose(self._dim0, self._dim1),)
