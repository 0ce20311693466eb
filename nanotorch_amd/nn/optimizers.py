"""Optimizers (reference: src/nanotorch/nn/optimizers.py)."""

from __future__ import annotations

from typing import Sequence

from .. import autograd as ag
from ..core import Tensor


class Optimizer:
    def __init__(self, parameters: Sequence[Tensor]) -> None:
        self._parameters = parameters

    @property
    def parameters(self) -> Sequence[Tensor]:
        return self._parameters

    def zero_grad(self) -> None:
        for p in self._parameters:
            p.zero_grad()

    def step(self) -> None:
        raise NotImplementedError


class GradientDescent(Optimizer):
    """p <- p - grad * float32(lr), two roundings, under no_grad."""

    def __init__(self, parameters: Sequence[Tensor], lr: float) -> None:
        super().__init__(parameters)
        self._lr = lr

    def step(self) -> None:
        for p in self.parameters:
            if p.requires_grad:
                if p.grad is None:
                    raise RuntimeError("Gradients not set, did you call backward?")
                with ag.no_grad():
                    p -= p.grad * self._lr
