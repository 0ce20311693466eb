"""Optimizers (reference: src/nanotorch/nn/optimizers.py)."""

from __future__ import annotations

from typing import Sequence

import math
import struct

from .. import _kernels as K
from .. import autograd as ag
from .._data_type import Dtype
from ..core import Tensor
from ..cuda import Device


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
        # lr as the reference's 0-d scalar tensor holds it (float32).  A step
        # size beyond float32's range (an inf scalar), a NaN, or anything that
        # is not a plain real number (e.g. a Tensor) takes the composition,
        # which gives what `p -= g * lr` gives for it.
        try:
            lr32 = struct.unpack("f", struct.pack("f", self._lr))[0]
        except (OverflowError, struct.error, TypeError):
            lr32 = None
        if lr32 is not None and (math.isnan(lr32) or isinstance(self._lr, Tensor)):
            lr32 = None
        for p in self.parameters:
            if p.requires_grad:
                if p.grad is None:
                    raise RuntimeError("Gradients not set, did you call backward?")
                g = p.grad
                with ag.no_grad():
                    if (lr32 is not None and p.device == Device.Cuda and g.device == Device.Cuda
                            and p.dtype == Dtype.Float32 and g.dtype == Dtype.Float32
                            and p.shape == g.shape):
                        # one pass, same two roundings as the composition
                        K.sgd_step(p, g, lr32)
                    else:
                        p -= g * self._lr
