"""Parametrised modules (reference: src/nanotorch/nn/module.py).

``Linear`` keeps the reference's He-uniform init ``2 * U[0,1) * z - z`` with
``z = sqrt(6 / fan_in)`` and zero bias; the arithmetic runs in float32 on the
device (same three roundings as the reference's host loop), so parameters
start on ``device`` (default "cuda").  ``Sigmoid`` is added next to ReLU and
Tanh (the reference exposes sigmoid only as a function).  ``Linear.forward``
on float32 device tensors runs the product and the bias add as one kernel
(``LinearOp``): same values and gradients as the reference's two ops.
"""

from __future__ import annotations

import math
from typing import Any, Sequence

from ..autograd import ReluOp, SigmoidOp, TanhOp
from ..autograd.ops_binary import LinearOp
from ..core import Tensor
from ..cuda import Device
from ..factories import rand, zeros


class Module:
    def __call__(self, *args: Any, **kwargs: Any) -> Any:
        return self.forward(*args, **kwargs)

    def parameters(self) -> Sequence[Tensor]:
        return []

    def to(self, device: Device | str) -> "Module":
        return self

    def forward(self, *args: Any, **kwargs: Any) -> Any:
        raise NotImplementedError


class Linear(Module):
    """y = x @ W + b with W [fan_in, fan_out]."""

    def __init__(self, fan_in: int, fan_out: int, bias: bool = True, *,
                 device: Device | str = "cuda") -> None:
        self._W = _kaiming_W(fan_in, fan_out, device)
        self._W.enable_grad()
        self._b = zeros(fan_out, requires_grad=True, device=device) if bias else None

    def parameters(self) -> Sequence[Tensor]:
        return [self._W] if self._b is None else [self._W, self._b]

    def to(self, device: Device | str) -> "Linear":
        self._W = self._W.to(device)
        if self._b is not None:
            self._b = self._b.to(device)
        return self

    def forward(self, x: Tensor) -> Tensor:
        if x.ndim != 2:
            raise NotImplementedError(f"Can only forward a 2D tensor for now, got {x.ndim}")
        if x.shape[1] != self._W.shape[0]:
            raise ValueError(f"Cannot align axes of size {x.shape[1]} and {self._W.shape[0]}.")
        if self._b is not None and LinearOp.usable(x, self._W, self._b):
            # the product and the bias add in one kernel, same roundings
            return LinearOp.apply(x, self._W, self._b)
        z = x @ self._W
        if self._b is not None:
            z = z + self._b
        return z


class ReLU(Module):
    def forward(self, x: Tensor) -> Tensor:
        return ReluOp.apply(x)


class Tanh(Module):
    def forward(self, x: Tensor) -> Tensor:
        return TanhOp.apply(x)


class Sigmoid(Module):
    def forward(self, x: Tensor) -> Tensor:
        return SigmoidOp.apply(x)


class Sequential(Module):
    def __init__(self, *modules: Module) -> None:
        self._modules = list(modules)

    def parameters(self) -> Sequence[Tensor]:
        params: list[Tensor] = []
        for m in self._modules:
            params.extend(m.parameters())
        return params

    def to(self, device: Device | str) -> "Sequential":
        self._modules = [m.to(device) for m in self._modules]
        return self

    def forward(self, *args: Any, **kwargs: Any) -> Any:
        x = None
        for i, m in enumerate(self._modules):
            x = m(*args, **kwargs) if i == 0 else m(x)
        return x


def _kaiming_W(fan_in: int, fan_out: int, device: Device | str = "cuda") -> Tensor:
    if fan_in <= 0 or fan_out <= 0:
        raise ValueError(
            f"Cannot initialize Linear with {fan_in=}, {fan_out=} (non-positive)."
        )
    z = math.sqrt(6 / fan_in)
    u = rand(fan_in, fan_out, device="cuda")  # drawn on the device, same stream
    w = 2 * u * z - z
    return w if str(device) in ("cuda", "Device.Cuda") or device == Device.Cuda else w.to(device)
