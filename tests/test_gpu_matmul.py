"""MatMulOp forward and both gradients on the GPU (fp32 MFMA) against the
oracle's sequential dot products.

Bar: |gpu - ref| <= 1e-4 * (|A|.|B|)_ij per element (a different fp32
accumulation order), plus a normwise check, on every output element; the
config shapes against the oracle's OpenMP product (bit-identical to its
sequential k loop).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from helpers import assert_bitexact, assert_rel, dev, dev_T, host, rng, seed_of

import nanotorch_amd as nt
from nanotorch_amd import _kernels as K

pytestmark = pytest.mark.gpu


def _mm(x1, x2):
    out_shape = tuple(x1.shape[:-2]) + (x1.shape[-2], x2.shape[-1])
    return host(nt.Tensor._new_contiguous(K.matmul(x1, x2, out_shape), out_shape))


def _check(got, a, b, what):
    want = O.matmul(np.ascontiguousarray(a), np.ascontiguousarray(b), parallel=True)
    scale = O.matmul(np.abs(a).astype(np.float64), np.abs(b).astype(np.float64), parallel=True)
    assert_rel(got, want, 1e-4, what, scale=scale)
    nrm = np.linalg.norm(got.astype(np.float64) - want) / max(np.linalg.norm(want), 1e-30)
    assert nrm < 1e-5, (what, nrm)


SHAPES = [(1, 1, 1), (2, 3, 4), (5, 7, 3), (32, 32, 32), (128, 128, 128), (129, 33, 130),
          (257, 100, 63), (64, 1000, 96), (300, 257, 511), (1024, 512, 768),
          # K % 32 == 0 with ragged M / N (multiples of 4): the direct-to-LDS
          # kernel's clamped edge tiles, every layout pair
          (132, 96, 260), (36, 64, 100), (1000, 256, 1004), (4, 32, 4)]


@pytest.mark.parametrize("layout", ["NN", "TN", "NT", "TT"])
@pytest.mark.parametrize("M,K_,N", SHAPES)
def test_matmul_layouts(gpu, M, K_, N, layout):
    r = rng(seed_of(M, K_, N, layout))
    a = r.standard_normal((M, K_)).astype(np.float32)
    b = (r.standard_normal((K_, N)) / np.sqrt(K_)).astype(np.float32)
    xa = dev_T(a) if layout[0] == "T" else dev(a)
    xb = dev_T(b) if layout[1] == "T" else dev(b)
    _check(_mm(xa, xb), a, b, f"{layout} {M}x{K_}x{N}")


def test_matmul_generic_strides_and_batch(gpu):
    r = rng(1)
    a = r.standard_normal((3, 4 * 2)).astype(np.float32)
    b = np.ones((4, 2), dtype=np.float32)
    got = _mm(dev(np.arange(12, dtype=np.float32).reshape(3, 4))[:, ::2], dev(np.ones((2, 2), np.float32)))
    assert_bitexact(got, np.array([[2, 2], [10, 10], [18, 18]], np.float32), "strided ::2")
    # batched with a broadcast (stride-0) batch operand
    a = r.standard_normal((4, 3, 37, 19)).astype(np.float32)
    b = r.standard_normal((19, 23)).astype(np.float32)
    xb = dev(b).expand(4, 3, 19, 23)
    got = _mm(dev(a), xb)
    _check(got, a, np.broadcast_to(b, (4, 3, 19, 23)), "batched+bcast")
    # batched, vector layouts, K % 32 == 0 (direct-to-LDS kernel)
    a = r.standard_normal((2, 3, 68, 64)).astype(np.float32)
    b = r.standard_normal((2, 3, 64, 132)).astype(np.float32)
    _check(_mm(dev(a), dev(b)), a, b, "batched direct")
    del b


def test_matmul_other_dtypes_exact(gpu):
    """fp64 / int paths accumulate in k order like the reference: exact."""
    r = rng(2)
    for dt in (np.float64, np.int64, np.int32):
        a = (r.standard_normal((33, 45)) * 10).astype(dt)
        b = (r.standard_normal((45, 27)) * 10).astype(dt)
        got = _mm(dev(a), dev_T(b))
        assert_bitexact(got, O.matmul(a, b), f"{dt}")


def test_matmul_accumulate(gpu):
    r = rng(3)
    a = r.standard_normal((200, 150)).astype(np.float32)
    b = r.standard_normal((150, 170)).astype(np.float32)
    old = r.standard_normal((200, 170)).astype(np.float32)
    tgt = dev(old)
    K.matmul_into(dev(a), dev(b), tgt, accumulate=True)
    want = O.matmul(a, b) + old
    scale = O.matmul(np.abs(a).astype(np.float64), np.abs(b).astype(np.float64)) + np.abs(old)
    assert_rel(host(tgt), want, 1e-4, "accumulate", scale=scale)


def _full_check(got, want, scale, what):
    """Every output: |gpu - ref| <= 1e-4 * (|A|.|B|)_ij, and normwise."""
    assert_rel(got, want, 1e-4, what, scale=scale)
    nrm = np.linalg.norm(got.astype(np.float64) - want) / max(np.linalg.norm(want), 1e-30)
    assert nrm < 1e-5, (what, nrm)


@pytest.mark.parametrize("M,K_,N", [(4096, 4096, 4096), (8192, 1024, 4096)])
def test_config4_full_size(gpu, M, K_, N):
    """Config 4 at its shapes: forward, dA = dG.B^T and dB = A^T.dG through
    autograd (MatmulOp), with A contiguous and as a transposed view.  Every
    output element is compared with the oracle's sequential fp32 dot product
    (the reference's k loop) within 1e-4 * (|A|.|B|)_ij."""
    r = rng(seed_of("c4", M, K_, N))
    A = r.standard_normal((M, K_)).astype(np.float32)
    B = (r.standard_normal((K_, N)) / np.sqrt(K_)).astype(np.float32)
    G = r.standard_normal((M, N)).astype(np.float32)
    At, Bt = np.ascontiguousarray(A.T), np.ascontiguousarray(B.T)
    aA, aB, aG = (np.abs(v).astype(np.float64) for v in (A, B, G))
    ref = {"fwd": (O.matmul(A, B, parallel=True), aA @ aB),
           "dA": (O.matmul(G, Bt, parallel=True), aG @ aB.T),
           "dB": (O.matmul(At, G, parallel=True), aA.T @ aG)}
    del aA, aB, aG
    for a_layout in ("contig", "transposed"):
        xa = dev(A) if a_layout == "contig" else dev_T(A)
        xa.enable_grad()
        xb = dev(B, requires_grad=True)
        y = xa @ xb
        _full_check(host(y), *ref["fwd"], f"fwd {a_layout} {M}x{K_}x{N}")
        # backward with upstream G: loss = sum(y * G) has dL/dy = G
        loss = (y * dev(G)).sum()
        loss.backward()
        _full_check(host(xa.grad), *ref["dA"], f"dA {a_layout} {M}x{K_}x{N}")
        _full_check(host(xb.grad), *ref["dB"], f"dB {a_layout} {M}x{K_}x{N}")
        del xa, xb, y, loss


def _batched_T(a):
    """Batched device operand equal to `a`, stored with its last two axes
    swapped (a transposed view per batch)."""
    return dev(np.ascontiguousarray(np.swapaxes(a, -1, -2))).transpose(-2, -1)


@pytest.mark.parametrize("layout", ["NN", "TN", "NT", "TT"])
def test_wide_tile_kernel_full_check(gpu, layout):
    """16 x [1024, 128] @ [128, 1024]: M and N multiples of 256, K of 64,
    and 256 tiles of 256x256 -- the wide-tile kernel's conditions -- with
    every output compared, once written and once accumulated into C."""
    r = rng(seed_of("wide", layout))
    Bt, M, K_, N = 16, 1024, 128, 1024
    a = r.standard_normal((Bt, M, K_)).astype(np.float32)
    b = (r.standard_normal((Bt, K_, N)) / np.sqrt(K_)).astype(np.float32)
    xa = _batched_T(a) if layout[0] == "T" else dev(a)
    xb = _batched_T(b) if layout[1] == "T" else dev(b)
    _check(_mm(xa, xb), a, b, f"wide {layout}")
    old = r.standard_normal((Bt, M, N)).astype(np.float32)
    tgt = dev(old)
    K.matmul_into(xa, xb, tgt, accumulate=True)
    want = O.matmul(a, b, parallel=True) + old
    scale = O.matmul(np.abs(a).astype(np.float64), np.abs(b).astype(np.float64),
                     parallel=True) + np.abs(old)
    assert_rel(host(tgt), want, 1e-4, f"wide accumulate {layout}", scale=scale)


@pytest.mark.parametrize("layout", ["NN", "TN", "NT", "TT"])
@pytest.mark.parametrize("accumulate", [False, True])
def test_wide_tile_split_k_full_check(gpu, accumulate, layout):
    """[1024, 8192] @ [8192, 2048]: 32 tiles of 256x256, so the wide kernel
    splits K into 8 slices (one tile per CU) and sums them in slice order;
    every operand layout (TN is the dB = A^T.dG of autograd); every output
    compared with an fp64 product (the bound covers fp32 accumulation in any
    order)."""
    r = rng(seed_of("splitk", accumulate, layout))
    M, K_, N = 1024, 8192, 2048
    a = r.standard_normal((M, K_)).astype(np.float32)
    b = (r.standard_normal((K_, N)) / np.sqrt(K_)).astype(np.float32)
    old = r.standard_normal((M, N)).astype(np.float32)
    tgt = dev(old)
    xa = dev_T(a) if layout[0] == "T" else dev(a)
    xb = dev_T(b) if layout[1] == "T" else dev(b)
    K.matmul_into(xa, xb, tgt, accumulate=accumulate)
    want = a.astype(np.float64) @ b.astype(np.float64) + (old if accumulate else 0.0)
    scale = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64) + (
        np.abs(old) if accumulate else 0.0)
    assert_rel(host(tgt), want, 1e-4, f"split-K accumulate={accumulate}", scale=scale)


# ----------------------------------------------------- bias in the epilogue

BIAS_SHAPES = [(7, 5, 3), (129, 33, 130), (300, 257, 512),  # generic / edge tiles
               (1024, 512, 768),                            # 128x128 MFMA kernels
               (4096, 1024, 4096),                          # wide kernel, one pass
               (1024, 8192, 256),                           # wide kernel, split K
               (64, 0, 96)]                                  # K = 0: C = bias


@pytest.mark.parametrize("layout", ["NN", "TN"])
@pytest.mark.parametrize("M,K_,N", BIAS_SHAPES)
def test_matmul_bias_equals_product_then_add(gpu, M, K_, N, layout):
    """nt_matmul_bias (the bias added in the product's epilogue) against the
    same product from nt_matmul followed by the broadcast add kernel, bit for
    bit: the fused form keeps the two fp32 roundings of the reference's
    MatmulOp then AddOp."""
    r = rng(seed_of("mmbias", M, K_, N, layout))
    a = r.standard_normal((M, K_)).astype(np.float32)
    b = (r.standard_normal((K_, N)) / np.sqrt(max(K_, 1))).astype(np.float32)
    bias = r.standard_normal(N).astype(np.float32)
    ta = dev(a) if layout == "NN" else dev_T(a)
    tb, tbias = dev(b), dev(bias)
    fused = host(nt.Tensor._new_contiguous(K.matmul_bias(ta, tb, tbias, (M, N)), (M, N)))
    prod = nt.Tensor._new_contiguous(K.matmul(ta, tb, (M, N)), (M, N))
    want = host(prod + tbias)
    assert_bitexact(fused, want, f"bias {M}x{K_}x{N} {layout}")


def test_matmul_bias_rejects_bad_operands(gpu):
    a, b = dev(np.ones((4, 3), np.float32)), dev(np.ones((3, 5), np.float32))
    with pytest.raises(RuntimeError):
        K.matmul_bias(a, b, dev(np.ones(4, np.float32)), (4, 5))  # wrong length
    with pytest.raises(ValueError):
        K.matmul_bias(dev(np.ones((4, 3))), dev(np.ones((3, 5))), dev(np.ones(5)), (4, 5))


def test_linear_fused_forward_and_backward_match_the_composition(gpu):
    """nn.Linear on float32 device tensors (LinearOp: product + bias in one
    kernel) against the reference's composition x @ W + b through the
    Tensor API, bit for bit: output, dx, dW, db, first-write and
    accumulated."""
    from nanotorch_amd import nn
    r = rng(seed_of("linear-fused"))
    x = r.standard_normal((512, 256)).astype(np.float32)
    g = r.standard_normal((512, 384)).astype(np.float32)
    lin = nn.Linear(256, 384)
    W0 = host(lin._W)
    lin._b = dev(r.standard_normal(384).astype(np.float32), requires_grad=True)
    b0 = host(lin._b)
    results = []
    for fused in (True, False):
        W = dev(W0, requires_grad=True)
        b = dev(b0, requires_grad=True)
        X = dev(x, requires_grad=True)
        G = dev(g)
        for _ in range(2):  # the second pass accumulates into the grads
            if fused:
                lin._W, lin._b = W, b
                z = lin(X)
                assert type(z.grad_fn).__name__ == "LinearOp"
            else:
                z = X @ W + b
            (z * G).sum().backward()
        results.append([host(z), host(X.grad), host(W.grad), host(b.grad)])
    for name, f, c in zip(("z", "dx", "dW", "db"), *results):
        assert_bitexact(f, c, name)


@pytest.mark.parametrize("x_T", [False, True])
@pytest.mark.parametrize("x_grad,W_grad,b_grad", [(True, True, True), (False, True, True),
                                                  (True, False, False), (False, False, True)])
def test_linear_fused_grad_subsets_and_views(gpu, x_T, x_grad, W_grad, b_grad):
    """LinearOp against x @ W + b with the input read through a `.T` view
    and with each subset of x, W and b requiring a gradient (a frozen
    layer, the first layer's input): every gradient that exists matches
    the composition's bit for bit, the others stay None, and under no_grad
    neither form records a graph."""
    from nanotorch_amd import nn
    r = rng(seed_of("linear-subsets", x_T, x_grad, W_grad, b_grad))
    x = r.standard_normal((300, 130)).astype(np.float32)
    g = r.standard_normal((300, 96)).astype(np.float32)
    W0 = (r.standard_normal((130, 96)) / np.sqrt(130)).astype(np.float32)
    b0 = r.standard_normal(96).astype(np.float32)
    lin = nn.Linear(130, 96)
    results = []
    for fused in (True, False):
        W, b = dev(W0, requires_grad=W_grad), dev(b0, requires_grad=b_grad)
        leaf = dev(np.ascontiguousarray(x.T), requires_grad=x_grad) if x_T else dev(x, requires_grad=x_grad)
        X = leaf.T if x_T else leaf
        if fused:
            lin._W, lin._b = W, b
            z = lin(X)
            assert type(z.grad_fn).__name__ == "LinearOp"
        else:
            z = X @ W + b
        (z * dev(g)).sum().backward()
        results.append([host(z)] + [None if t.grad is None else host(t.grad) for t in (leaf, W, b)])
        with nt.no_grad():
            lin._W, lin._b = W, b
            assert (lin(X) if fused else X @ W + b).grad_fn is None
    for name, f, c, need in zip(("z", "dx", "dW", "db"), *results, (True, x_grad, W_grad, b_grad)):
        if not need:
            assert f is None and c is None, name
        else:
            assert_bitexact(f, c, name)


def test_linear_fused_saved_input_modified_in_place_raises(gpu):
    """LinearOp saves x and W for its backward: an in-place change to the
    input after the forward invalidates the saved version, and backward
    raises as it does for MatmulOp."""
    from nanotorch_amd import nn
    lin = nn.Linear(8, 4)
    h = dev(np.ones((5, 8), np.float32), requires_grad=True) * 2.0  # a non-leaf input
    z = lin(h)
    assert type(z.grad_fn).__name__ == "LinearOp"
    h += 1.0
    with pytest.raises(RuntimeError):
        z.sum().backward()


def test_matmul_bias_strided_operands(gpu):
    """nt_matmul_bias with a bias read through a stride-2 slice, an A whose
    rows repeat (a stride-0 expand) and a B read through `.T`, on the 128x128
    and the wide kernels: bit-identical to the product, then the add."""
    r = rng(seed_of("mmbias-strided"))
    for M, K_, N in ((200, 96, 136), (512, 512, 512)):
        row = r.standard_normal((1, K_)).astype(np.float32)
        ta = dev(row).expand(M, K_)                       # every row the same
        tb = dev_T((r.standard_normal((K_, N)) / np.sqrt(K_)).astype(np.float32))
        tbias = dev(r.standard_normal(2 * N).astype(np.float32))[::2]
        fused = host(nt.Tensor._new_contiguous(K.matmul_bias(ta, tb, tbias, (M, N)), (M, N)))
        prod = nt.Tensor._new_contiguous(K.matmul(ta, tb, (M, N)), (M, N))
        assert_bitexact(fused, host(prod + tbias), f"strided bias {M}x{K_}x{N}")
