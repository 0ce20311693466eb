"""Base class of differentiable operations
(reference: src/nanotorch/autograd/function.py:11-93).

``apply`` runs ``forward``, records inputs, and attaches the node to the
output when any tensor input requires grad.  ``save_for_backward`` snapshots
storage versions so that an in-place change of a saved tensor is caught when
``saved_tensors`` is read.

Ops of this package may also define ``_backward_into(grad, needs, targets)``
with ``fused_ok()``: the engine then asks for all needed input gradients in
one call, passing each input's existing gradient (or None) as ``targets``;
the op accumulates into those in place and returns new tensors for the
others.  ``backward`` stays available with the reference's contract.
"""

from __future__ import annotations

from typing import Any

from ..core import Tensor
from .grad_mode import is_grad_enabled


class Function:
    def __init__(self) -> None:
        self._inputs: Any = None
        self._inputs_kw: Any = None
        self._saved_tensors: tuple[tuple[Tensor, int], ...] | None = None

    def __repr__(self) -> str:
        inner = (
            ""
            if self._saved_tensors is None
            else ", ".join("x" + str(i) for i in range(len(self._saved_tensors)))
        )
        return f"[{self.__class__.__name__}({inner})]"

    @property
    def inputs(self) -> tuple:
        if self._inputs is None:
            raise RuntimeError("No inputs saved during apply().")
        return self._inputs

    @property
    def saved_tensors(self) -> tuple[Tensor, ...]:
        if self._saved_tensors is None:
            raise RuntimeError("No tensor was saved during forward.")
        for x, v in self._saved_tensors:
            if x.version != v:
                raise RuntimeError(
                    "One of the tensors needed for grad computation was modified inplace."
                )
        return tuple(x for x, _ in self._saved_tensors)

    @classmethod
    def apply(cls, *args: Any, **kwargs: Any) -> Tensor:
        self = cls()
        self._inputs = args
        self._inputs_kw = kwargs
        output = self.forward(*args, **kwargs)
        if is_grad_enabled():
            if any(output is a for a in list(args) + list(kwargs.values())):
                output = output._alias()  # keeps the DAG structure
            if any(isinstance(t, Tensor) and t.requires_grad for t in args):
                output.attach_grad_fn(self)
        return output

    def save_for_backward(self, *tensors: Tensor) -> None:
        if is_grad_enabled():
            self._saved_tensors = tuple((x, x.version) for x in tensors)

    def fused_ok(self) -> bool:
        """Whether _backward_into handles this instance."""
        return False

    def forward(self, *inputs: Any) -> Tensor:
        raise NotImplementedError

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        raise NotImplementedError

    @classmethod
    def flops(cls, *args: Any, **kwargs: Any) -> int:
        return 0

    @classmethod
    def mem_bytes(cls, *args: Any, **kwargs: Any) -> int:
        return 0
