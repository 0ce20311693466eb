"""Writes tests/golden/config5_trace.npz: the CPU reference's 20-step loss
trace for config 5 of BASELINE.json on bench.py's seeded inputs.

The network is Linear 1024->4096, tanh, Linear 4096->4096, sigmoid, Linear
4096->4096, ReLU, Linear 4096->1000 with zero biases; the loss is
mean((Y - T)**2) and the optimizer SGD with lr = float32(1e-3)
(scripts/train_mlp_basic.py:48-53, nn/optimizers.py:45-51,
autograd/ops_reduction.py:112-138).  Inputs come from bench.config5_inputs(5).

Each step is oracle.mlp_step, the reference's CPU kernels and Python
backward chains restated (oracle/), with its matmuls in the OpenMP order
(or_matmul_omp), which is bit-identical to the reference's sequential k loop.
It runs in a few minutes on 8 cores.

Stored (float32 unless noted):
  losses          [20]   the reference's loss of each step, before that
                         step's update: its MeanOp sums the 8,192,000 squared
                         errors sequentially in fp32, which at this length
                         under-reads the true mean by about 1.1%
  losses_exact64  [20]   float64: the same steps' squared-error tensors
                         summed in float64 and divided by their size, i.e.
                         the reference's loss without its summation error
  w{i}_idx        [4096] int64 flat positions of layer i's weight sampled
  w{i}_init       [4096] initial weight values at those positions
  w{i}_final      [4096] weights after 20 steps at those positions
  b{i}_final      [fan_out] biases after 20 steps (all of them)
  w{i}_sum64      ()     float64 sum of all final weights of layer i
  dw{i}_norm64    ()     float64 Frobenius norm of (final - initial) weights
  gw{i}_step0     [4096] W.grad of the first step at w{i}_idx
                         (A_i^T @ dZ_i, A_i the layer's input, dZ_i the
                         gradient of its output z = A_i @ W + b)
  gw{i}_scale     [4096] float64: (|A_i|^T @ |dZ_i|) at the same positions,
                         the size of the terms each gradient element sums
  gb{i}_step0     [fan_out] b.grad of the first step (dZ_i summed over rows)
  gb{i}_scale     [fan_out] float64: |dZ_i| summed over rows

Usage: python tests/golden/make_config5_trace.py [--steps 20]
"""

from __future__ import annotations

import argparse
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

import bench  # noqa: E402
import oracle as O  # noqa: E402

SAMPLES = 4096


def sample_idx(i: int, size: int) -> np.ndarray:
    """The SAMPLES flat positions of layer i's weight that are stored."""
    return np.random.default_rng(100 + i).integers(0, size, SAMPLES).astype(np.int64)


def step0_gradients(st: dict, params) -> dict:
    """W.grad and b.grad of the first step at the sampled positions, with the
    float64 size of the terms each element sums (|A|^T @ |dZ|)."""
    out = {}
    for i, (gw, gb) in enumerate(st["grads"]):
        a, dz = st["layer_in"][i], st["layer_dz"][i]
        w = params[i][0]
        idx = sample_idx(i, w.size)
        r, c = np.divmod(idx, w.shape[1])
        out[f"gw{i}_step0"] = gw.ravel()[idx].astype(np.float32)
        scale = np.empty(SAMPLES, np.float64)
        for j0 in range(0, SAMPLES, 512):  # 512 positions at a time: ~64 MB per operand
            sl = slice(j0, j0 + 512)
            scale[sl] = np.einsum("kj,kj->j", np.abs(a[:, r[sl]]).astype(np.float64),
                                  np.abs(dz[:, c[sl]]).astype(np.float64))
        out[f"gw{i}_scale"] = scale
        out[f"gb{i}_step0"] = np.asarray(gb, np.float32).copy()
        out[f"gb{i}_scale"] = np.abs(dz).astype(np.float64).sum(axis=0)
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--out", default=bench.C5_TRACE)
    args = ap.parse_args()
    x, t, params = bench.config5_inputs(5)
    init = [w.copy() for w, _ in params]
    print(f"oracle threads: {O.threads()}", flush=True)
    losses, exact = [], []
    first: dict = {}
    for s in range(args.steps):
        t0 = time.time()
        st: dict = {}
        losses.append(np.float32(O.mlp_step(params, x, t, bench.C5_ACTS, bench.C5_LR,
                                            parallel=True, stats=st)))
        exact.append(st["sq_sum64"] / st["numel"])
        if s == 0:
            first = step0_gradients(st, params)
        del st
        print(f"step {s}: loss {float(losses[-1]):.9g} exact-sum {exact[-1]:.9g} "
              f"({time.time() - t0:.1f} s)", flush=True)
    out = {"losses": np.array(losses, dtype=np.float32),
           "losses_exact64": np.array(exact, dtype=np.float64)}
    for i, ((w, b), w0) in enumerate(zip(params, init)):
        idx = sample_idx(i, w.size)
        out[f"w{i}_idx"] = idx
        out[f"w{i}_init"] = w0.ravel()[idx]
        out[f"w{i}_final"] = w.ravel()[idx]
        out[f"b{i}_final"] = b.copy()
        out[f"w{i}_sum64"] = np.float64(w.astype(np.float64).sum())
        out[f"dw{i}_norm64"] = np.float64(np.linalg.norm((w.astype(np.float64) - w0).ravel()))
    out.update(first)
    np.savez_compressed(args.out, **out)
    print(f"wrote {args.out}")


if __name__ == "__main__":
    main()
