"""Binary differentiable ops: add, sub, mul, truediv, matmul.

Forward semantics restate src/nanotorch/autograd/ops_binary.py: dtype
promotion to max(dtypes), right-aligned broadcasting through stride-0 views,
the ``out=`` in-place branch of ``_binary_kernel_op`` (:283-315) and the
matmul shape algebra of ``_matmul_broadcast`` (:318-343).

Backward: ``backward`` keeps the reference's compositions (:49-50, 95-100,
145-150, 197-202, 253-267).  ``_backward_into`` computes the same values with
one fused kernel per op (nt_binary_bwd) or, for matmul, one MFMA product per
gradient with the accumulation folded into its epilogue (nt_matmul with
accumulate), and only for the inputs that need a gradient.
"""

from __future__ import annotations

import math

from .. import _kernels as K
from .. import _lib
from .._data_type import is_float, promote_dtypes, sizeof
from .._indexing import broadcast_shapes
from ..core import Tensor, TensorShape
from .function import Function
from .grad_mode import is_grad_enabled
from .ops_utils import unbroadcast


class _ElementwiseBinary(Function):
    """Shared forward/backward plumbing of add/sub/mul/truediv."""

    _op: int
    _saves_inputs = False

    def forward(self, x1: Tensor, x2: Tensor, out: Tensor | None = None) -> Tensor:
        self._shapes = (x1.shape, x2.shape)
        self._in_dtypes = (x1.dtype, x2.dtype)
        if self._saves_inputs:
            self.save_for_backward(x1, x2)
        res = _binary_kernel_op(x1, x2, self._op, out=out)
        self._out_shape = res.shape
        self._out_dtype = res.dtype
        return res

    def fused_ok(self) -> bool:
        return (
            is_float(self._out_dtype)
            and self._in_dtypes[0] == self._out_dtype
            and self._in_dtypes[1] == self._out_dtype
        )

    def _backward_into(self, g: Tensor, needs, targets):
        op = self._op
        out_shape = self._out_shape
        if g.shape != out_shape:
            g = g.reshape(*out_shape)
        a = b = None
        if op in (_lib.MUL, _lib.DIV):
            x1, x2 = self.saved_tensors
            a = x1.expand(*out_shape)
            b = x2.expand(*out_shape)
        results = [None, None]
        # Gradients the kernel produces at full (output) shape.
        kneed = [False, False]
        ktarget = [None, None]
        for i in (0, 1):
            if not needs[i]:
                continue
            same = self._shapes[i] == out_shape
            passthrough = op == _lib.ADD or (op == _lib.SUB and i == 0)
            if passthrough and (targets[i] is None or not same):
                # d/dx = g: hand g itself on (the reference returns the same
                # tensor object), summed over broadcast axes if needed.
                r = unbroadcast(g, self._shapes[i])
                if targets[i] is None:
                    results[i] = r
                else:
                    K.inplace(_lib.ADD, targets[i], r)
                    results[i] = targets[i]
                continue
            kneed[i] = True
            ktarget[i] = targets[i] if same else None
        if any(kneed):
            sa, sb = K.binary_bwd(
                op, g, a, b, kneed[0], ktarget[0], kneed[1], ktarget[1]
            )
            for i, st in ((0, sa), (1, sb)):
                if not kneed[i]:
                    continue
                if st is None:  # accumulated in place
                    results[i] = targets[i]
                    continue
                full = Tensor._new_contiguous(st, out_shape)
                r = unbroadcast(full, self._shapes[i])
                if targets[i] is None:
                    results[i] = r
                else:
                    K.inplace(_lib.ADD, targets[i], r)
                    results[i] = targets[i]
        return results

    @classmethod
    def flops(cls, x1: Tensor, x2: Tensor, _=None) -> int:
        return math.prod(broadcast_shapes(x1.shape, x2.shape))

    @classmethod
    def mem_bytes(cls, x1: Tensor, x2: Tensor, _=None) -> int:
        shape = broadcast_shapes(x1.shape, x2.shape)
        return 3 * math.prod(shape) * sizeof(promote_dtypes(x1.dtype, x2.dtype))


class AddOp(_ElementwiseBinary):
    """x1 + x2 with promotion and broadcasting."""

    _op = _lib.ADD

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        return tuple(unbroadcast(grad_out, s) for s in self._shapes)


class SubOp(_ElementwiseBinary):
    """x1 - x2 with promotion and broadcasting."""

    _op = _lib.SUB

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        s1, s2 = self._shapes
        return unbroadcast(grad_out, s1), unbroadcast(-1 * grad_out, s2)


class MulOp(_ElementwiseBinary):
    """x1 * x2 with promotion and broadcasting."""

    _op = _lib.MUL
    _saves_inputs = True

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        x1, x2 = self.saved_tensors
        return (
            unbroadcast(x2 * grad_out, x1.shape),
            unbroadcast(x1 * grad_out, x2.shape),
        )


class TrueDivOp(_ElementwiseBinary):
    """x1 / x2 with promotion and broadcasting (1 / 0.0 gives inf)."""

    _op = _lib.DIV
    _saves_inputs = True

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        x1, x2 = self.saved_tensors
        return (
            unbroadcast(grad_out / x2, x1.shape),
            unbroadcast(-x1 / x2**2 * grad_out, x2.shape),
        )


class MatmulOp(Function):
    """Matrix product with numpy-style 1-D promotion and batch broadcasting:
    (k,)@(k,) -> (); (n,k)@(k,) -> (n,); (k,)@(k,m) -> (m,);
    (B1,n,k)@(B2,k,m) -> (B1::B2,n,m)."""

    def forward(self, x1: Tensor, x2: Tensor) -> Tensor:
        self.save_for_backward(x1, x2)
        self._shape1, self._shape2, shape_out = _matmul_broadcast(x1.shape, x2.shape)
        dtype = promote_dtypes(x1.dtype, x2.dtype)
        self._dtypes = (x1.dtype, x2.dtype, dtype)
        x1 = x1.to(dtype).expand(*self._shape1)
        if x2.ndim == 1 and self._shape2[-2:] == (x2.shape[0], 1):
            x2 = x2.reshape(x2.shape[0], 1)  # cannot expand to the right
        x2 = x2.to(dtype).expand(*self._shape2)
        full_out = tuple(self._shape1[:-2]) + (self._shape1[-2], self._shape2[-1])
        st = K.matmul(x1, x2, full_out)
        return Tensor._new_contiguous(st, shape_out)

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        x1, x2 = self.saved_tensors
        x2_shape = x2.shape
        x1_m = x1.expand(*self._shape1)
        if x2.ndim == 1 and self._shape2[-2:] == (x2.shape[0], 1):
            x2 = x2.reshape(x2.shape[0], 1)
        x2_m = x2.expand(*self._shape2)
        grad_out = grad_out.reshape(
            *broadcast_shapes(self._shape1[:-2], self._shape2[:-2]),
            self._shape1[-2],
            self._shape2[-1],
        )
        # The gradient of a 1-D right operand is reshaped back to (k,); the
        # reference keeps the (k, 1) column it multiplied with.
        return (
            unbroadcast(grad_out @ x2_m.transpose(-2, -1), x1.shape).reshape(*x1.shape),
            unbroadcast(x1_m.transpose(-2, -1) @ grad_out, x2.shape).reshape(*x2_shape),
        )

    def fused_ok(self) -> bool:
        d1, d2, d = self._dtypes
        return (
            is_float(d)
            and d1 == d
            and d2 == d
            and len(self._shape1) >= 2
            and len(self._saved_tensors[0][0].shape) == len(self._shape1)
            and self._saved_tensors[0][0].shape == self._shape1
            and self._saved_tensors[1][0].shape == self._shape2
        )

    def _backward_into(self, g: Tensor, needs, targets):
        """dA = G . B^T and dB = A^T . G, each one MFMA product reading the
        transposed operand in place; an existing gradient is accumulated in
        the product's epilogue."""
        x1, x2 = self.saved_tensors
        full_out = tuple(self._shape1[:-2]) + (self._shape1[-2], self._shape2[-1])
        if g.shape != full_out:
            g = g.reshape(*full_out)
        results = [None, None]
        if needs[0]:
            rhs = x2.transpose(-2, -1)
            if targets[0] is None:
                st = K.matmul(g, rhs, x1.shape)
                results[0] = Tensor._new_contiguous(st, x1.shape)
            else:
                K.matmul_into(g, rhs, targets[0], accumulate=True)
                results[0] = targets[0]
        if needs[1]:
            lhs = x1.transpose(-2, -1)
            if targets[1] is None:
                st = K.matmul(lhs, g, x2.shape)
                results[1] = Tensor._new_contiguous(st, x2.shape)
            else:
                K.matmul_into(lhs, g, targets[1], accumulate=True)
                results[1] = targets[1]
        return results

    @classmethod
    def flops(cls, x1: Tensor, x2: Tensor) -> int:
        s1, s2, _ = _matmul_broadcast(x1.shape, x2.shape)
        return 2 * math.prod(s1[:-2]) * s1[-2] * s2[-1] * s1[-1]

    @classmethod
    def mem_bytes(cls, x1: Tensor, x2: Tensor) -> int:
        s1, s2, _ = _matmul_broadcast(x1.shape, x2.shape)
        B, M, N, Kd = math.prod(s1[:-2]), s1[-2], s2[-1], s1[-1]
        return B * (M * Kd + Kd * N + M * N) * sizeof(promote_dtypes(x1.dtype, x2.dtype))


class LinearOp(Function):
    """x @ W + b for 2-D float32 device operands in one product whose
    epilogue adds b (nt_matmul_bias): the reference's Linear forward, a
    MatmulOp then an AddOp (src/nanotorch/nn/module.py:73-75), with the same
    two fp32 roundings (the product's, then the add's).  Its backward is
    those two ops' backward: dx = g . W^T and dW = x^T . g (MatmulOp,
    src/nanotorch/autograd/ops_binary.py:253-267, each one product reading
    the transposed operand in place), db = g summed over the rows (AddOp's
    unbroadcast, same file :49-50)."""

    def forward(self, x: Tensor, W: Tensor, b: Tensor) -> Tensor:
        self.save_for_backward(x, W)
        self._b_shape = b.shape
        shape = (x.shape[0], W.shape[1])
        return Tensor._new_contiguous(K.matmul_bias(x, W, b, shape), shape)

    def backward(self, grad_out: Tensor) -> tuple[Tensor, ...]:
        x, W = self.saved_tensors
        return (grad_out @ W.transpose(0, 1), x.transpose(0, 1) @ grad_out,
                unbroadcast(grad_out, self._b_shape))

    def fused_ok(self) -> bool:
        return True

    def _backward_into(self, g: Tensor, needs, targets):
        x, W = self.saved_tensors
        results = [None, None, None]
        for i, (lhs, rhs, shape) in enumerate(((g, W.transpose(0, 1), x.shape),
                                               (x.transpose(0, 1), g, W.shape))):
            if not needs[i]:
                continue
            if targets[i] is None:
                results[i] = Tensor._new_contiguous(K.matmul(lhs, rhs, shape), shape)
            else:
                K.matmul_into(lhs, rhs, targets[i], accumulate=True)
                results[i] = targets[i]
        if needs[2]:
            r = unbroadcast(g, self._b_shape)
            if targets[2] is None:
                results[2] = r
            else:
                K.inplace(_lib.ADD, targets[2], r)
                results[2] = targets[2]
        return results

    @classmethod
    def usable(cls, x: Tensor, W: Tensor, b: Tensor) -> bool:
        """Whether the fused form applies: 2-D float32 x and W and a 1-D
        float32 b over W's columns, all on the device."""
        from .._data_type import Dtype
        from ..cuda import Device
        return (x.ndim == 2 and W.ndim == 2 and b.ndim == 1 and b.shape[0] == W.shape[1]
                and x.shape[1] == W.shape[0]
                and all(t.device == Device.Cuda and t.dtype == Dtype.Float32 for t in (x, W, b)))


def _binary_kernel_op(x1: Tensor, x2: Tensor, op: int, out: Tensor | None = None) -> Tensor:
    """Promotion + broadcast + kernel call, with the reference's ``out=``
    semantics (ops_binary.py:283-315): ``out is x1`` runs in place, any other
    ``out`` receives a copy of the result (which is returned)."""
    if out is not None:
        if out.is_leaf and out.requires_grad and is_grad_enabled():
            raise RuntimeError(
                "A leaf variable that requires grad is being used in an in-place op."
            )
        dtype = out.dtype
        shape = out.shape
    else:
        dtype = promote_dtypes(x1.dtype, x2.dtype)
        shape = broadcast_shapes(x1.shape, x2.shape)
    out_is_x1 = out is x1
    x1 = x1.to(dtype).expand(*shape)
    x2 = x2.to(dtype).expand(*shape)
    if out is None:
        return Tensor._new_contiguous(K.binary(op, x1, x2), shape)
    if out_is_x1:
        K.inplace(op, x1, x2)
        return x1
    result = Tensor._new_contiguous(K.binary(op, x1, x2), shape)
    K.copy_view(result, out)
    out._storage.bump_version()
    return result


def _matmul_broadcast(
    x1: TensorShape, x2: TensorShape
) -> tuple[TensorShape, TensorShape, TensorShape]:
    """Shapes of the expanded operands and of the result."""
    if len(x1) == 0 or len(x2) == 0:
        raise RuntimeError("Scalar value encountered in matmul.")
    drop = []
    if len(x1) == 1:
        x1 = (1, *x1)
        drop.append(-2)
    if len(x2) == 1:
        x2 = (*x2, 1)
        drop.append(-1)
    if x1[-1] != x2[-2]:
        raise RuntimeError(f"Cannot multiply {x1} @ {x2}")
    bshape = broadcast_shapes(x1[:-2], x2[:-2])
    raw = list(bshape) + [x1[-2], x2[-1]]
    drop = [ax + len(raw) for ax in drop]
    shape_out = tuple(d for i, d in enumerate(raw) if i not in drop)
    return (
        tuple(list(bshape) + list(x1[-2:])),
        tuple(list(bshape) + list(x2[-2:])),
        shape_out,
    )

