"""Oracle: CPU restatement of the reference's CPU path, for checking only.

TEST INFRASTRUCTURE.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use this module; the nanotorch_amd package never imports it.

Primitives (unary / binary / in-place / cast / reduce / matmul) call
libnt_oracle.so (oracle/nt_oracle.cpp), which restates the reference's C++
CPU loops.  The backward functions below restate the reference's Python
compositions (src/nanotorch/autograd/ops_*.py) on those primitives, step by
step, including the dtype promotions and scalar tensors the reference
creates (a Python int scalar is an int64 tensor cast to the float dtype, a
Python float scalar is a float32 tensor), so every rounding happens where
the reference's does.  Inputs are numpy arrays (any non-negative strides;
numpy broadcasting views are the reference's stride-0 expand views).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# NT_ORACLE_LIB selects another build of the same source (the sanitizer
# build of tests/test_oracle_sanitized.py).
LIB = os.environ.get("NT_ORACLE_LIB") or os.path.join(HERE, "libnt_oracle.so")

EXP, LOG, NEG, RELU, SQRT, TANH, SIGMOID, POW = range(8)
ADD, SUB, MUL, DIV, EQ, GT, GE = range(7)
COPY = 7
R_SUM, R_MAX, R_MIN, R_ARGMAX, R_ARGMIN = range(5)

_CODES = {
    np.dtype(np.bool_): 0,
    np.dtype(np.int32): 1,
    np.dtype(np.int64): 2,
    np.dtype(np.float32): 3,
    np.dtype(np.float64): 4,
}
_NP = {v: k for k, v in _CODES.items()}


class OrView(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("offset", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int64 * 8),
        ("strides", ctypes.c_int64 * 8),
    ]


_lib = None


def build() -> None:
    """Compiles libnt_oracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        P = ctypes.POINTER(OrView)
        L.or_unary.argtypes = [ctypes.c_int32, P, ctypes.c_double, ctypes.c_void_p]
        L.or_binary.argtypes = [ctypes.c_int32, P, P, ctypes.c_void_p]
        L.or_inplace.argtypes = [ctypes.c_int32, P, P]
        L.or_cast.argtypes = [P, ctypes.c_int32, ctypes.c_void_p]
        L.or_reduce.argtypes = [
            ctypes.c_int32, P, ctypes.POINTER(ctypes.c_int64), ctypes.c_int32,
            ctypes.c_int32, ctypes.c_void_p,
        ]
        L.or_matmul.argtypes = [P, P, ctypes.c_void_p]
        L.or_matmul_omp.argtypes = [P, P, ctypes.c_void_p]
        L.or_uniform.argtypes = [ctypes.c_uint64, ctypes.c_int64, ctypes.c_int64,
                                 ctypes.c_int32, ctypes.c_double, ctypes.c_double,
                                 ctypes.c_void_p]
        L.or_mt64_output.argtypes = [ctypes.c_uint64, ctypes.c_int64]
        L.or_mt64_output.restype = ctypes.c_uint64
        L.or_last_error.restype = ctypes.c_char_p
        _lib = L
    return _lib


def _check(rc: int) -> None:
    if rc == 0:
        return
    msg = lib().or_last_error().decode()
    raise (ValueError if rc == 2 else RuntimeError)(msg)


def view(a: np.ndarray) -> OrView:
    v = OrView()
    v.data = a.__array_interface__["data"][0]
    v.offset = 0
    v.dtype = _CODES[a.dtype]
    v.ndim = a.ndim
    for i, (s, st) in enumerate(zip(a.shape, a.strides)):
        if st < 0:
            raise ValueError("negative strides not supported")
        v.shape[i] = s
        v.strides[i] = st // a.itemsize
    return v


def _out_ptr(o: np.ndarray) -> int:
    return o.__array_interface__["data"][0]


# ------------------------------------------------------------- primitives


def unary(op: int, x: np.ndarray, scalar: float = 0.0) -> np.ndarray:
    out = np.empty(x.shape, dtype=x.dtype)
    vx = view(x)
    _check(lib().or_unary(op, ctypes.byref(vx), float(scalar), _out_ptr(out)))
    return out


def binary(op: int, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    out = np.empty(a.shape, dtype=np.bool_ if op >= EQ else a.dtype)
    va, vb = view(a), view(b)
    _check(lib().or_binary(op, ctypes.byref(va), ctypes.byref(vb), _out_ptr(out)))
    return out


def inplace(op: int, out: np.ndarray, other: np.ndarray) -> None:
    vo, vx = view(out), view(other)
    _check(lib().or_inplace(op, ctypes.byref(vo), ctypes.byref(vx)))


def cast(x: np.ndarray, dtype) -> np.ndarray:
    dtype = np.dtype(dtype)
    if x.dtype == dtype:
        return x
    out = np.empty(x.shape, dtype=dtype)
    vx = view(x)
    _check(lib().or_cast(ctypes.byref(vx), _CODES[dtype], _out_ptr(out)))
    return out


def reduce(op: int, x: np.ndarray, axes, out_dtype=None) -> np.ndarray:
    axes = tuple(axes)
    keep = [s for i, s in enumerate(x.shape) if i not in axes]
    if op in (R_ARGMAX, R_ARGMIN):
        odt = np.dtype(np.int64)
    elif op in (R_MAX, R_MIN):
        odt = x.dtype
    else:
        odt = np.dtype(out_dtype if out_dtype is not None else x.dtype)
    out = np.empty(keep, dtype=odt)
    arr = (ctypes.c_int64 * max(1, len(axes)))(*axes)
    vx = view(x)
    _check(lib().or_reduce(op, ctypes.byref(vx), arr, len(axes), _CODES[odt], _out_ptr(out)))
    return out


def matmul(a: np.ndarray, b: np.ndarray, parallel: bool = False) -> np.ndarray:
    """Same-rank batched matmul, sequential k dot product per output."""
    shape = list(a.shape)
    shape[-1] = b.shape[-1]
    out = np.empty(shape, dtype=a.dtype)
    va, vb = view(a), view(b)
    fn = lib().or_matmul_omp if parallel else lib().or_matmul
    _check(fn(ctypes.byref(va), ctypes.byref(vb), _out_ptr(out)))
    return out


def uniform(seed: int, n: int, dtype=np.float32, skip: int = 0, low: float = 0.0,
            high: float = 1.0) -> np.ndarray:
    """Draws skip .. skip+n-1 of the reference's generator after
    manual_seed(seed): std::mt19937_64 through
    std::uniform_real_distribution<T>(low, high) (factory.cu:73-83)."""
    out = np.empty(n, dtype=dtype)
    code = _CODES[np.dtype(dtype)]
    _check(lib().or_uniform(seed, skip, n, code, low, high, _out_ptr(out)))
    return out


def mt64_output(seed: int, k: int) -> int:
    """The k-th (1-based) raw output of std::mt19937_64 seeded with seed."""
    return int(lib().or_mt64_output(seed, k))


# ------------------------------------------------- scalars as the reference


def scalar(value, like_dtype) -> np.ndarray:
    """A Python scalar as the reference wraps it: Tensor(value) has dtype
    bool / int64 / float32; binary ops then promote to max(dtypes) and cast
    the scalar with Storage::cast (static_cast)."""
    if isinstance(value, bool):
        src = np.array(value, dtype=np.bool_)
    elif isinstance(value, int):
        src = np.array(value, dtype=np.int64)
    else:
        src = np.array(value, dtype=np.float32)
    target = max(_CODES[src.dtype], _CODES[np.dtype(like_dtype)])
    return cast(src, _NP[target])


def bcast(x: np.ndarray, shape) -> np.ndarray:
    return np.broadcast_to(x, shape)


def mul_scalar(g: np.ndarray, value) -> np.ndarray:
    s = scalar(value, g.dtype)
    return binary(MUL, g, bcast(s, g.shape))


def rsub_scalar(value, y: np.ndarray) -> np.ndarray:
    s = scalar(value, y.dtype)
    return binary(SUB, bcast(s, y.shape), y)


def pow_scalar(x: np.ndarray, value) -> np.ndarray:
    """x ** value: PowOp with exponent Tensor(value); the exponent enters the
    kernel as float(item) converted to the promoted dtype
    (ops_unary.py:251-262)."""
    e = scalar(value, x.dtype)  # promote(x, exponent dtype)
    return unary(POW, cast(x, e.dtype), float(e))


# ------------------------------------------ backward compositions (fp)
# Each returns the new gradient term; accumulate() then applies the
# engine's `x._grad += grad` (core.py:868-871 -> inplace add).


def accumulate(old: np.ndarray, new: np.ndarray) -> np.ndarray:
    out = old.copy()
    inplace(ADD, out, new)
    return out


def bwd_neg(g):  # ops_unary.py:32-33: -1 * grad_out
    return mul_scalar(g, -1)


def bwd_exp(g, y):  # :69-70: grad_out * e_x
    return binary(MUL, g, y)


def bwd_log(g, x):  # :105-106: grad_out * x ** -1
    return binary(MUL, g, pow_scalar(x, -1))


def bwd_sqrt(g, y):  # :142-144: grad_out * 0.5 * sqrt_x ** -1
    return binary(MUL, mul_scalar(g, 0.5), pow_scalar(y, -1))


def bwd_tanh(g, y):  # :180-182: grad_out * (1 - tanh_x ** 2)
    return binary(MUL, g, rsub_scalar(1, pow_scalar(y, 2)))


def bwd_sigmoid(g, y):  # :218-220: grad_out * sig_x * (1 - sig_x)
    return binary(MUL, binary(MUL, g, y), rsub_scalar(1, y))


def bwd_relu(g, y):  # :287-289: grad_out * (result > Tensor(0))
    zero = scalar(0, y.dtype)
    mask = binary(GT, y, bcast(zero, y.shape))
    return binary(MUL, g, cast(mask, g.dtype))


def bwd_pow(g, x, e):
    """:264-266: grad_out * exponent * x ** (exponent - 1), exponent a
    Tensor(e) (float32 for a float e, int64 for an int e)."""
    et = np.array(e, dtype=np.int64 if isinstance(e, int) else np.float32)
    em1 = binary(SUB, et, cast(np.array(1, dtype=np.int64), et.dtype))
    t = binary(MUL, g, bcast(cast(et, g.dtype), g.shape))
    return binary(MUL, t, pow_scalar_tensor(x, em1))


def pow_scalar_tensor(x, et: np.ndarray):
    dt = _NP[max(_CODES[x.dtype], _CODES[et.dtype])]
    return unary(POW, cast(x, dt), float(et))


def bwd_binary(op: int, g, a, b):
    """(ga, gb) of add/sub/mul/div for equal shapes (ops_binary.py:49-50,
    95-100, 145-150, 197-202)."""
    if op == ADD:
        return g, g
    if op == SUB:
        return g, mul_scalar(g, -1)
    if op == MUL:
        return binary(MUL, b, g), binary(MUL, a, g)
    ga = binary(DIV, g, b)
    neg_a = unary(NEG, a)
    gb = binary(MUL, binary(DIV, neg_a, pow_scalar(b, 2)), g)
    return ga, gb


def sel_bwd(op: int, g_kept: np.ndarray, x: np.ndarray, axes) -> np.ndarray:
    """Max/min backward (ops_reduction.py:201-212): mask = x == expand(m);
    mask *= 1 / mask.sum(keepdim) (int64 division, then cast to bool);
    result = expand(g) * float(mask)."""
    axes = tuple(axes)
    m = reduce(R_MAX if op == R_MAX else R_MIN, x, axes)
    kd = tuple(1 if d in axes else s for d, s in enumerate(x.shape))
    mask = binary(EQ, x, bcast(m.reshape(kd), x.shape))
    cnt = reduce(R_SUM, mask, axes, np.int64).reshape(kd)
    one = np.array(1, dtype=np.int64)
    inv = binary(DIV, bcast(one, cnt.shape), cnt)  # int64 division
    inv_b = cast(inv, np.bool_)
    mask2 = mask.copy()
    inplace(MUL, mask2, bcast(inv_b, x.shape))
    gexp = bcast(g_kept.reshape(kd), x.shape)
    return binary(MUL, gexp, cast(mask2, g_kept.dtype))


def mean_fwd(x: np.ndarray, axes) -> np.ndarray:
    """ops_reduction.py:112-127: x.sum(dtype=x.dtype) / denom."""
    s = reduce(R_SUM, x, axes, x.dtype)
    denom = x.size // max(1, s.size)
    return binary(DIV, s, bcast(scalar(denom, s.dtype), s.shape))


# ------------------------------------------------------------ MLP step


def mlp_step(params, x, t, acts, lr: float, parallel: bool = True, stats: dict | None = None):
    """One training step of Sequential(Linear, act, ..., Linear) with loss
    mean((Y - T)**2) and GradientDescent, restating nn/module.py:64-76,
    train_mlp_basic.py:45-55, optimizers.py:45-51 and the backward chains of
    each op.  params: list of (W, b) float32 arrays, updated in place.
    acts: activation names between layers ('relu', 'tanh', 'sigmoid').
    Returns the loss (a numpy float32 scalar) before the update.

    With `stats` (a dict), also stores stats["sq_sum64"], the float64 sum of
    the squared-error tensor (Y - T)**2 the loss is the mean of, and
    stats["numel"]: the loss with the reference's sequential fp32
    summation error taken out (the backward does not depend on it); and,
    per layer i, stats["grads"][i] = (W.grad, b.grad) of this step,
    stats["layer_in"][i] = the layer's input A_i and stats["layer_dz"][i] =
    the gradient dZ_i of its output z = A_i @ W + b, so that W.grad =
    A_i^T @ dZ_i and b.grad = sum over rows of dZ_i."""
    mm = lambda a, b: matmul(a, b, parallel=parallel)  # noqa: E731
    hs = [x]  # layer inputs
    zs_saved = []  # saved activation outputs
    h = x
    n = len(params)
    for i, (W, b) in enumerate(params):
        z = binary(ADD, mm(h, W), bcast(b, (h.shape[0], W.shape[1])))
        if i < n - 1:
            a = acts[i]
            if a == "relu":
                y = unary(RELU, z)
            elif a == "tanh":
                y = unary(TANH, z)
            else:
                y = unary(SIGMOID, z)
            zs_saved.append(y)
            h = y
            hs.append(h)
        else:
            h = z
    Y = h
    d = binary(SUB, Y, t)
    sq = pow_scalar(d, 2)
    loss = mean_fwd(sq, tuple(range(sq.ndim)))
    if stats is not None:
        stats["sq_sum64"] = float(sq.astype(np.float64).sum())
        stats["numel"] = int(sq.size)
    # backward: loss grad 1.0 -> MeanOp: expand(g) / denom
    g0 = np.array(1.0, dtype=np.float32)
    gs = binary(DIV, bcast(g0, sq.shape), bcast(scalar(sq.size, np.float32), sq.shape))
    # PowOp(d, 2): grad * 2 * d ** 1
    gd = bwd_pow(gs, d, 2)
    gY = gd  # SubOp: grad for Y passes through
    grads = []
    dzs = []
    g = gY
    for i in range(n - 1, -1, -1):
        W, b = params[i]
        hin = hs[i]
        dzs.append(g)
        # z = (h @ W) + b: AddOp backward -> (g, unbroadcast(g, b.shape))
        gb = reduce(R_SUM, g, (0,), np.float32)
        gW = mm(hin.T, g)
        grads.append((gW, gb))
        if i > 0:
            gh = mm(g, W.T)
            y = zs_saved[i - 1]
            a = acts[i - 1]
            if a == "relu":
                g = bwd_relu(gh, y)
            elif a == "tanh":
                g = bwd_tanh(gh, y)
            else:
                g = bwd_sigmoid(gh, y)
    grads.reverse()
    dzs.reverse()
    if stats is not None:
        stats["grads"] = grads
        stats["layer_in"] = hs
        stats["layer_dz"] = dzs
    # SGD: p -= p.grad * lr  (two roundings)
    for (W, b), (gW, gb) in zip(params, grads):
        inplace(SUB, W, mul_scalar(gW, lr))
        inplace(SUB, b, mul_scalar(gb, lr))
    return loss


def threads() -> int:
    return int(lib().or_max_threads())


def has_openmp() -> bool:
    return bool(lib().or_has_openmp())

