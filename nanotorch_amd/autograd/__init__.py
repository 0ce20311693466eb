"""Differentiable ops and the grad-mode switch
(reference: src/nanotorch/autograd/__init__.py)."""

from .function import Function
from .grad_mode import is_grad_enabled, no_grad
from .ops_binary import AddOp, MatmulOp, MulOp, SubOp, TrueDivOp
from .ops_reduction import MaxOp, MeanOp, MinOp, SumOp
from .ops_special import ExpandOp, ReshapeOp, TOp, TransposeOp
from .ops_unary import ExpOp, LogOp, NegOp, PowOp, ReluOp, SigmoidOp, SqrtOp, TanhOp

ALL_OPS_ = [
    AddOp,
    ExpOp,
    ExpandOp,
    LogOp,
    MatmulOp,
    MeanOp,
    MulOp,
    NegOp,
    PowOp,
    ReluOp,
    ReshapeOp,
    SigmoidOp,
    SqrtOp,
    SubOp,
    SumOp,
    TOp,
    TanhOp,
    TransposeOp,
    TrueDivOp,
    MinOp,
    MaxOp,
]

__all__ = [
    "AddOp",
    "ExpandOp",
    "ExpOp",
    "Function",
    "LogOp",
    "MatmulOp",
    "MaxOp",
    "MeanOp",
    "MinOp",
    "MulOp",
    "NegOp",
    "PowOp",
    "ReluOp",
    "ReshapeOp",
    "SigmoidOp",
    "SqrtOp",
    "SubOp",
    "SumOp",
    "TanhOp",
    "TOp",
    "TransposeOp",
    "TrueDivOp",
    "is_grad_enabled",
    "no_grad",
]
