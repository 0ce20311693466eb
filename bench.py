"""Benchmark of the MI355X hot path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--parts all|none|...]

Headline (`value`): config 2 of BASELINE.json -- the elementwise forward +
fused backward sweep at 2^24 fp32 elements ([4096, 4096]): each of add, sub,
mul, truediv, neg, exp, log, sqrt, pow(2.5), relu, sigmoid, tanh, forward and
backward in accumulate mode (the 12 forwards of a layout, then its 12
backwards), once on contiguous tensors and once on transposed (`.T`) views.
One step = one full sweep (48 kernels).  `value` is
the sweep's algorithmic HBM bytes / its time (GB/s); inputs are resident in
HBM before timing.  Timing uses HIP events on the library stream.

Parts reported beside it: config 3 reductions (GB/s), config 4 MatMulOp
forward + dA + dB (TFLOP/s), config 5 4-layer MLP training steps (step/s and
the loss trace), plus a single-threaded CPU baseline (the oracle, i.e. the
reference's CPU kernels restated) on a bounded sample of the headline
workload.

Data is synthetic (seeded normal / uniform per config); weights of the MLP
are random He-normal.

Profiles: `python bench.py --summarize KIND DIR [DIR2]` turns the csv output
of the rocprofv3 commands in PROFILE_CMDS into the summaries kept under
profiles/ (kernel statistics per part, and HBM bytes per launch from the
FETCH_SIZE / WRITE_SIZE passes, which the roofline's `traffic` reads).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import nanotorch_amd as nt  # noqa: E402
from nanotorch_amd import _kernels as K  # noqa: E402
from nanotorch_amd import _lib  # noqa: E402
from nanotorch_amd import nn  # noqa: E402
from nanotorch_amd._storage import Storage  # noqa: E402

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix, published

BASELINE_METRIC = "matmul fwd+bwd fp32 TFLOP/s; elementwise/reduce HBM GB/s; MLP step/s"


# ----------------------------------------------------------------- helpers


def dev(a: np.ndarray) -> nt.Tensor:
    return nt.Tensor(np.ascontiguousarray(a), device="cuda")


def dev_T(a: np.ndarray) -> nt.Tensor:
    return dev(np.ascontiguousarray(a.T)).T


def view(t) -> _lib.NtView:
    return K.view_of(t)


class Timer:
    """Brackets launches with HIP events on the library stream."""

    def __init__(self) -> None:
        self.marks: list[tuple[str, _lib.Event, _lib.Event]] = []

    def run(self, name: str, fn) -> None:
        a, b = _lib.Event(), _lib.Event()
        a.record()
        fn()
        b.record()
        self.marks.append((name, a, b))

    def durations(self) -> dict[str, list[float]]:
        out: dict[str, list[float]] = {}
        for name, a, b in self.marks:
            out.setdefault(name, []).append(a.elapsed_ms(b))
        return out


def _fresh(shape, dtype=nt.float32) -> nt.Tensor:
    return nt.Tensor._new_contiguous(Storage.allocate(math.prod(shape), dtype, nt.Device.Cuda), shape)


# --------------------------------------------------- config 2: elementwise

UNARY_OPS = [  # name, op, domain, saved ("in" | "out" | None), exponent
    ("neg", _lib.NEG, (-4, 4), None, 0.0),
    ("exp", _lib.EXP, (-4, 4), "out", 0.0),
    ("log", _lib.LOG, (0.1, 4), "in", 0.0),
    ("sqrt", _lib.SQRT, (0.1, 4), "out", 0.0),
    ("pow", _lib.POW, (0.1, 4), "in", 2.5),
    ("relu", _lib.RELU, None, "out", 0.0),
    ("sigmoid", _lib.SIGMOID, None, "out", 0.0),
    ("tanh", _lib.TANH, None, "out", 0.0),
]
BINARY_OPS = [("add", _lib.ADD), ("sub", _lib.SUB), ("mul", _lib.MUL), ("truediv", _lib.DIV)]

N_ELEM = 4096 * 4096


def ew_bytes(name: str, phase: str) -> int:
    """Algorithmic bytes per launch (fp32, 2^24 elements): each distinct
    tensor read once, each output written once.  `bwd` is accumulate mode:
    reads g (+ saved inputs) + old grads, writes the grads; `bwd_first` is
    first-write mode: reads g (+ saved inputs), writes the grads (add and
    sub write both, as the kernel does when handed both outputs)."""
    per = {
        ("fwd", "bin"): 12, ("fwd", "un"): 8,
        ("bwd", "add"): 20, ("bwd", "sub"): 20, ("bwd", "mul"): 28, ("bwd", "truediv"): 28,
        ("bwd", "neg"): 12,
        ("bwd_first", "add"): 12, ("bwd_first", "sub"): 12, ("bwd_first", "mul"): 20,
        ("bwd_first", "truediv"): 20, ("bwd_first", "neg"): 8,
    }
    binary = name in ("add", "sub", "mul", "truediv")
    if phase == "fwd":
        return per[("fwd", "bin" if binary else "un")] * N_ELEM
    return per.get((phase, name), 16 if phase == "bwd" else 12) * N_ELEM


class ElementwiseSweep:
    """Prepared tensors and C views for the config-2 sweep; `step()` queues
    the 48 kernels through the C ABI with no allocation in the loop.

    Order within a layout: the 12 forwards, then the 12 backwards in the
    same op order, as a training step runs every forward before any
    backward (the reference's engine, src/nanotorch/core.py:511-526 and
    836-872).  Between an op's forward and its backward the other 22
    kernels of the layout move ~5 GB, so the saved output `y` a backward
    reads (exp, sqrt, relu, sigmoid, tanh) has left the 256 MB Infinity
    Cache and comes from HBM, as every other operand of the sweep does.
    Queued forward-then-backward per op, those five backwards read a `y`
    written microseconds earlier and run above the rate HBM allows."""

    def __init__(self, seed: int = 0) -> None:
        r = np.random.default_rng(seed)
        shape = (4096, 4096)
        self.calls: list[tuple[str, str, str, object]] = []  # (op, layout, phase, fn)
        # the same backwards in first-write mode (not part of the step)
        self.first_write_calls: list[tuple[str, str, str, object]] = []
        lib = _lib.load()
        keep = []  # keep tensors alive
        for layout in ("contig", "transposed"):
            mk = dev if layout == "contig" else dev_T
            fwds: list = []
            bwds: list = []
            firsts: list = []
            for name, op in BINARY_OPS:
                a = r.standard_normal(shape).astype(np.float32)
                b = (r.uniform(0.5, 2, shape) if name == "truediv" else r.standard_normal(shape)).astype(np.float32)
                g = r.standard_normal(shape).astype(np.float32)
                ta, tb, tg = mk(a), mk(b), dev(g)
                out = _fresh(shape)
                # accumulation targets laid out like the inputs
                ga, gb = mk(r.standard_normal(shape).astype(np.float32)), mk(r.standard_normal(shape).astype(np.float32))
                va, vb, vg, vo, vga, vgb = view(ta), view(tb), view(tg), view(out), view(ga), view(gb)
                keep += [ta, tb, tg, out, ga, gb, va, vb, vg, vo, vga, vgb]
                fwds.append((name, layout, "fwd", (lib.nt_binary, (op, ctypes.byref(va), ctypes.byref(vb), ctypes.byref(vo)))))
                for acc, lst in ((1, bwds), (0, firsts)):
                    lst.append((name, layout, "bwd" if acc else "bwd_first", (lib.nt_binary_bwd, (
                        op, ctypes.byref(vg), ctypes.byref(va), ctypes.byref(vb),
                        ctypes.byref(vga), acc, ctypes.byref(vgb), acc))))
            for name, op, dom, saved, e in UNARY_OPS:
                x = (r.standard_normal(shape) if dom is None else r.uniform(dom[0], dom[1], shape)).astype(np.float32)
                g = r.standard_normal(shape).astype(np.float32)
                tx, tg = mk(x), dev(g)
                out = _fresh(shape)
                gx = mk(r.standard_normal(shape).astype(np.float32))
                vx, vg, vo, vgx = view(tx), view(tg), view(out), view(gx)
                # saved tensor: the forward output (contiguous) or the input view
                vs = vo if saved == "out" else (vx if saved == "in" else None)
                keep += [tx, tg, out, gx, vx, vg, vo, vgx]
                fwds.append((name, layout, "fwd", (lib.nt_unary, (op, ctypes.byref(vx), e, ctypes.byref(vo)))))
                for acc, lst in ((1, bwds), (0, firsts)):
                    lst.append((name, layout, "bwd" if acc else "bwd_first", (lib.nt_unary_bwd, (
                        op, ctypes.byref(vg), ctypes.byref(vs) if vs is not None else None, e,
                        ctypes.byref(vgx), acc))))
            self.calls += fwds + bwds
            self.first_write_calls += firsts
        self._keep = keep
        self.step_bytes = sum(ew_bytes(n, ph) for n, _, ph, _ in self.calls)

    def step(self, timer: Timer | None = None, first_write: bool = False) -> None:
        for name, layout, phase, (fn, args) in (self.first_write_calls if first_write
                                                 else self.calls):
            if timer is None:
                _lib.check(fn(*args))
            else:
                timer.run(f"{name}|{layout}|{phase}", lambda fn=fn, args=args: _lib.check(fn(*args)))


def launch_stats() -> dict:
    """nt_launch_stats: elementwise kernels queued without / with the stream
    barrier, and barrier kernels queued before other stream work."""
    u, o, f = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    _lib.call("nt_launch_stats", ctypes.byref(u), ctypes.byref(o), ctypes.byref(f))
    return {"unordered": u.value, "ordered": o.value, "fences": f.value}


def bench_elementwise(steps: int, warmup: int, first_write: bool = False) -> dict:
    """The sweep's whole-step time (events around the K steps; independent
    kernels overlap where the library's launch window admits them), then a
    per-kernel pass with events around each launch, which orders every
    kernel after the one before (no overlap): the per-kernel figures and the
    roofline come from that pass.  With `first_write`, the 24 backwards
    again in first-write mode (the grads overwritten, not accumulated),
    timed per launch the same way; not part of the step."""
    sw = ElementwiseSweep()
    for _ in range(warmup):
        sw.step()
    nt.sync()
    # whole-step timing: events around the K steps only
    t0, t1 = _lib.Event(), _lib.Event()
    nt.sync()
    l0 = launch_stats()
    t0.record()
    for _ in range(steps):
        sw.step()
    t1.record()
    nt.sync()
    l1 = launch_stats()
    total_ms = t0.elapsed_ms(t1)
    # per-kernel timing (separate pass, events around each launch)
    tm = Timer()
    for _ in range(max(2, steps // 2)):
        sw.step(tm)
    nt.sync()
    per = {}
    for key, ds in tm.durations().items():
        name, layout, phase = key.split("|")
        avg = sum(ds) / len(ds)
        gbs = ew_bytes(name, phase) / (avg * 1e-3) / 1e9
        per[key] = {"ms": round(avg, 5), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                    "bytes": ew_bytes(name, phase)}
    launches = {k: (l1[k] - l0[k]) / steps for k in l0}
    # the 24 backwards in first-write mode, timed the same way (per launch)
    tf = Timer()
    for _ in range(max(2, steps // 2) if first_write else 0):
        sw.step(tf, first_write=True)
    nt.sync()
    first = {}
    for key, ds in tf.durations().items():
        name, layout, phase = key.split("|")
        avg = sum(ds) / len(ds)
        gbs = ew_bytes(name, phase) / (avg * 1e-3) / 1e9
        first[key] = {"ms": round(avg, 5), "GB/s": round(gbs, 1),
                      "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": ew_bytes(name, phase)}
    return {"ms_per_step": total_ms / steps, "step_bytes": sw.step_bytes, "per_kernel": per,
            "launches_per_step": launches,
            "sum_of_kernel_ms": round(sum(v["ms"] for v in per.values()), 5),
            "first_write": first}


# ---------------------------------------------------- config 3: reductions


def bench_reductions(iters: int = 24) -> dict:
    """Config 3: sum / max / min forward and sum / mean / max backward over
    axis 0, axis 1 and the full [8192, 8192] fp32 tensor, through the C ABI
    with every output preallocated.  Each case runs `iters` launches back to
    back between two events on the library stream (host launch overhead
    overlaps the kernels), alternating two copies of the input and of each
    output so that a 268 MB operand is not re-read from the 256 MB Infinity
    Cache."""
    r = np.random.default_rng(3)
    shape = (8192, 8192)
    n = shape[0] * shape[1]
    lib = _lib.load()
    xs = [dev(r.standard_normal(shape).astype(np.float32)) for _ in range(2)]
    keep: list = []
    cases: dict[str, list] = {}

    def ref(obj):
        keep.append(obj)
        return ctypes.byref(obj)

    for axes, label in (((0,), "axis0"), ((1,), "axis1"), ((0, 1), "full")):
        kshape = tuple(s for i, s in enumerate(shape) if i not in axes)
        k = math.prod(kshape)
        arr = _lib.axes_array(axes)
        keep.append(arr)
        g = dev(r.standard_normal(k).astype(np.float32))
        vg = K.flat_view(g._storage, (k,))
        for op, name in ((_lib.R_SUM, "sum"), (_lib.R_MAX, "max"), (_lib.R_MIN, "min")):
            calls = []
            for c in range(2):
                o = _fresh((k,))
                aux = name != "sum"
                idx = _fresh((k,), nt.int64) if aux else None
                cnt = _fresh((k,), nt.int32) if aux else None
                keep += [o, idx, cnt]
                calls.append((lib.nt_reduce, (
                    op, ref(view(xs[c])), arr, len(axes), ref(K.flat_view(o._storage, (k,))),
                    ref(K.flat_view(idx._storage, (k,))) if aux else None,
                    ref(K.flat_view(cnt._storage, (k,))) if aux else None)))
                if name == "max" and c == 0:
                    vi = K.flat_view(idx._storage, (k,))
                    vc = K.flat_view(cnt._storage, (k,))
            cases[f"{name}|{label}|fwd"] = calls
        # the max forward's index and count, for the max backward
        lib.nt_reduce(_lib.R_MAX, ctypes.byref(view(xs[0])), arr, len(axes),
                      ctypes.byref(K.flat_view(_fresh((k,))._storage, (k,))),
                      ctypes.byref(vi), ctypes.byref(vc))
        olds = [dev(r.standard_normal(shape).astype(np.float32)) for _ in range(2)]
        gb = g.reshape(*[1 if i in axes else s for i, s in enumerate(shape)]).expand(*shape)
        outs = [_fresh(shape) for _ in range(2)]
        keep += [g, olds, outs, gb]
        # sum backward, accumulate: old += broadcast(g)
        cases[f"sum|{label}|bwd"] = [(lib.nt_inplace, (_lib.ADD, ref(view(olds[c])), ref(view(gb))))
                                     for c in range(2)]
        cases[f"mean|{label}|bwd"] = [(lib.nt_reduce_bwd, (
            _lib.R_MEAN, ref(vg), float(n // k), None, None, arr, len(axes),
            ref(view(outs[c])), 0)) for c in range(2)]
        cases[f"max|{label}|bwd"] = [(lib.nt_reduce_bwd, (
            _lib.R_MAX, ref(vg), 1.0, ref(vi), ref(vc), arr, len(axes),
            ref(view(outs[c])), 0)) for c in range(2)]
    fwd_bytes = n * 4
    bwd_bytes = {"sum": 2 * n * 4, "mean": n * 4, "max": n * 4}
    out = {}
    tot_b = tot_ms = 0.0
    order = [f"{o}|{l}|{p}" for l in ("axis0", "axis1", "full")
             for p, ops in (("fwd", ("sum", "max", "min")), ("bwd", ("sum", "mean", "max")))
             for o in ops]
    for key in order:
        calls = cases[key]
        for fn, args in calls:  # warm-up
            _lib.check(fn(*args))
        e0, e1 = _lib.Event(), _lib.Event()
        e0.record()
        for it in range(iters):
            fn, args = calls[it % 2]
            _lib.check(fn(*args))
        e1.record()
        nt.sync()
        avg = e0.elapsed_ms(e1) / iters
        op, _, phase = key.split("|")
        b = fwd_bytes if phase == "fwd" else bwd_bytes[op]
        gbs = b / (avg * 1e-3) / 1e9
        out[key] = {"ms": round(avg, 5), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
        tot_b += b
        tot_ms += avg
    return {"per_kernel": out, "aggregate_GB/s": round(tot_b / (tot_ms * 1e-3) / 1e9, 1)}


# ------------------------------------------------------- config 4: matmul


MM_SHAPES = ((4096, 4096, 4096), (8192, 1024, 4096))
MM_ITERS = 5


def bench_matmul(iters: int = MM_ITERS) -> dict:
    r = np.random.default_rng(4)
    res = {}
    for (M, Kd, N) in MM_SHAPES:
        A = r.standard_normal((M, Kd)).astype(np.float32)
        B = (r.standard_normal((Kd, N)) / np.sqrt(Kd)).astype(np.float32)
        G = r.standard_normal((M, N)).astype(np.float32)
        tb, tg = dev(B), dev(G)
        for a_layout in ("contig", "transposed"):
            ta = dev(A) if a_layout == "contig" else dev_T(A)
            c, da, db = _fresh((M, N)), _fresh((M, Kd)), _fresh((Kd, N))
            calls = [
                ("fwd", ta, tb, c), ("dA", tg, tb.T, da), ("dB", ta.T, tg, db),
            ]
            tm = Timer()
            for _ in range(iters + 1):
                for name, x1, x2, o in calls:
                    tm.run(name, lambda x1=x1, x2=x2, o=o: K.matmul_into(x1, x2, o, accumulate=False))
            nt.sync()
            flop = 2 * M * N * Kd
            key = f"{M}x{Kd}x{N}|{a_layout}"
            tot_ms = 0.0
            entry = {}
            for name, ds in tm.durations().items():
                avg = sum(ds[1:]) / len(ds[1:])
                tot_ms += avg
                tf = flop / (avg * 1e-3) / 1e12
                entry[name] = {"ms": round(avg, 4), "TFLOP/s": round(tf, 2),
                               "frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)}
            tf = 3 * flop / (tot_ms * 1e-3) / 1e12
            entry["fwd+dA+dB"] = {"ms": round(tot_ms, 4), "TFLOP/s": round(tf, 2),
                                  "frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)}
            res[key] = entry
    return res


# ---------------------------------------------------------- config 5: MLP


C5_DIMS = [1024, 4096, 4096, 4096, 1000]
C5_ACTS = ["tanh", "sigmoid", "relu"]
C5_BATCH = 8192
C5_LR = 1e-3
C5_TRACE = os.path.join(ROOT, "tests", "golden", "config5_trace.npz")


def config5_inputs(seed: int = 5):
    """Config 5's synthetic inputs, drawn in this order from
    numpy.random.default_rng(seed): X [8192, 1024] ~ N(0,1), T [8192, 1000]
    ~ N(0,1), then W_i [fan_in, fan_out] ~ N(0, 2/fan_in) (He-normal) for the
    four layers; biases are zero (nn.Linear's init, as the reference's
    Linear(bias=True)).  Returns float32 arrays (x, t, [(W, b), ...])."""
    r = np.random.default_rng(seed)
    x = r.standard_normal((C5_BATCH, C5_DIMS[0])).astype(np.float32)
    t = r.standard_normal((C5_BATCH, C5_DIMS[-1])).astype(np.float32)
    params = []
    for i in range(4):
        w = (r.standard_normal((C5_DIMS[i], C5_DIMS[i + 1])) * np.sqrt(2.0 / C5_DIMS[i])).astype(np.float32)
        params.append((w, np.zeros(C5_DIMS[i + 1], dtype=np.float32)))
    return x, t, params


def config5_model(params):
    """Sequential(Linear, Tanh, Linear, Sigmoid, Linear, ReLU, Linear) on the
    device with the given (W, b) arrays, and its Linear layers."""
    layers = []
    for w, b in params:
        lin = nn.Linear(w.shape[0], w.shape[1])
        lin._W = dev(w)
        lin._W.enable_grad()
        lin._b = dev(b)
        lin._b.enable_grad()
        layers.append(lin)
    model = nn.Sequential(layers[0], nn.Tanh(), layers[1], nn.Sigmoid(), layers[2],
                          nn.ReLU(), layers[3])
    return model, layers


def config5_reference_trace():
    """The CPU reference's 20-step loss trace for config5_inputs(5) (the
    committed fixture, written by tests/golden/make_config5_trace.py), as
    (losses, losses_exact64): the reference's literal losses, whose MeanOp
    sums 8,192,000 squared errors left to right in fp32 (~1.1% low here),
    and the mean of the same squared errors summed in fp64.  None when the
    fixture is absent."""
    if not os.path.exists(C5_TRACE):
        return None
    with np.load(C5_TRACE, allow_pickle=False) as z:
        return [float(v) for v in z["losses"]], [float(v) for v in z["losses_exact64"]]


def bench_mlp(steps: int = 20) -> dict:
    x, t, params = config5_inputs(5)
    X, T = dev(x), dev(t)
    model, _ = config5_model(params)
    del x, t, params
    opt = nn.GradientDescent(model.parameters(), lr=C5_LR)
    losses = []
    times = []
    for s in range(steps):
        e0, e1 = _lib.Event(), _lib.Event()
        e0.record()
        opt.zero_grad()
        y = model(X)
        loss = nt.mean((y - T) ** 2)
        loss.backward()
        opt.step()
        e1.record()
        losses.append(loss)
        times.append((e0, e1))
    nt.sync()
    ms = [a.elapsed_ms(b) for a, b in times]
    trace = [float(lo.cpu().item()) for lo in losses]
    steady = ms[2:] if len(ms) > 3 else ms
    avg = sum(steady) / len(steady)
    flop = 1_988_032_987_136  # per step; layer-1 dX is not computed (X needs no grad)
    out = {"step/s": round(1000.0 / avg, 3), "ms_per_step": round(avg, 3),
           "matmul_TFLOP/s": round(flop / (avg * 1e-3) / 1e12, 2),
           "loss_trace": [round(v, 7) for v in trace], "steps": steps}
    ref = config5_reference_trace()
    if ref is not None:
        # per-step relative deviation from the CPU reference's run of the
        # same 20 steps on the same seeded inputs: against the mean of its
        # squared errors (bar: 1e-4), and against its literal loss, which
        # carries its sequential fp32 summation error
        lit, exact = ref
        k = min(len(lit), len(trace))
        out["loss_max_rel_dev_vs_cpu_ref_exact_sum"] = float(
            max(abs(a - b) / abs(b) for a, b in zip(trace[:k], exact[:k])))
        out["loss_max_rel_dev_vs_cpu_ref_literal"] = float(
            max(abs(a - b) / abs(b) for a, b in zip(trace[:k], lit[:k])))
        out["cpu_ref_literal_vs_exact_sum"] = float(
            max(abs(a - b) / abs(b) for a, b in zip(lit[:k], exact[:k])))
        out["loss_steps_compared"] = k
    return out


# --------------------------------------------- next rows beside the path


def _index_args(fn: str, plan, first, second, keep_alive: list) -> list:
    """ctypes arguments of nt_gather_axes / nt_scatter_axes for a fixed plan,
    with the index arrays uploaded once (so the timed calls move no host
    data)."""
    import ctypes
    nf = len(plan.fancy_dims_in_src)
    idx = [nt.Tensor(a, dtype=nt.int64, device="cuda") for a in plan.index_arrays]
    views = (_lib.NtView * nf)(*[K.view_of(t) for t in idx])
    fd = (ctypes.c_int32 * nf)(*plan.fancy_dims_in_src)
    nd = len(plan.new_shape)
    isf = (ctypes.c_int32 * nd)(*[1 if b else 0 for b in plan.out_axis_is_fancy])
    tgt = (ctypes.c_int32 * nd)(*plan.out_axis_target)
    va, vb = K.view_of(first), K.view_of(second)
    keep_alive += [idx, views, fd, isf, tgt, va, vb]
    args = [ctypes.byref(va), ctypes.byref(vb), nf, fd, views, isf, tgt]
    if fn == "nt_scatter_axes":
        args.append(None)  # unique rows: no last-occurrence mask
    return args


_N8K = 8192 * 8192
_N4 = 64 * 512 * 512
# bench_next's cases in queue order: name, a substring of the kernel each
# call launches, kernels per call, algorithmic bytes (or None), FLOP (or
# None).  Every case runs 1 + NEXT_ITERS calls (an untimed first call).
NEXT_ROWS = [
    ("cast|f32->f64", "CastOp<float, double>", 1, 12 * _N8K, None),
    ("cast|f64->f32", "CastOp<double, float>", 1, 12 * _N8K, None),
    ("cast|i64->f32", "CastOp<long, float>", 1, 12 * _N8K, None),
    ("compare|gt", "CompareFwd", 1, 9 * _N8K, None),
    ("copy|transposed", "ew_tile4_kernel", 1, 8 * _N8K, None),
    # a batch of 64 planes: [64, 1024, 1024].transpose(1, 2) -> contiguous
    ("copy|3-D transpose(1,2)", "ew_tile4_kernel", 1, 8 * _N8K, None),
    # [64, 512, 512] transposed two ways: 64 planes of 512 x 512 (axes 1, 2),
    # and 512 planes of 512 x 64 (axes 0, 2)
    ("copy|[64,512,512].transpose(1,2)", "ew_tile4_kernel", 1, 8 * _N4, None),
    ("copy|[64,512,512].transpose(0,2)", "ew_tile4_kernel", 1, 8 * _N4, None),
    ("matmul|batched 16x1024^3", "mm_f32_mfma", 1, None, 2 * 16 * 1024**3),
    ("gather|8192 rows of [50000,1024]", "row_index_kernel", 1, 2 * 8192 * 1024 * 4 + 8 * 8192, None),
    ("scatter|8192 rows of [50000,1024]", "row_index_kernel", 1, 2 * 8192 * 1024 * 4 + 8 * 8192, None),
    # the reference's generator stream drawn on the device: bytes written
    ("uniform|f32 [8192,8192]", "rng_", 4, 4 * _N8K, None),
]
NEXT_ITERS = 12


def bench_next(iters: int = NEXT_ITERS) -> dict:
    """The rows next to the hot path, each timed over `iters` launches back
    to back between two HIP events on the library stream (elementwise
    launches on the rotating operand sets are independent and may overlap
    in the launch window): device casts and a comparison (no host round
    trip), strided copies of a transposed 2-D view and of batches of
    transposed planes, a batched matmul on the MFMA kernel, and
    advanced-index gather / scatter of rows.  Bytes are algorithmic (every
    operand once); GB/s against the HBM peak, TFLOP/s against the fp32 MFMA
    peak."""
    from nanotorch_amd import _fancy
    import ctypes
    r = np.random.default_rng(6)
    # [8192, 8192] operands in SETS copies used in turn: consecutive launches
    # touch different buffers, several GB apart, so nothing is served from
    # the 256 MB Infinity Cache (re-writing one output buffer back to back
    # was measured ~20% faster than HBM allows).
    SETS = 3
    shape = (8192, 8192)
    n = shape[0] * shape[1]

    def copies(t):
        out = [t]
        for _ in range(SETS - 1):
            c = _fresh(t.shape, t.dtype)
            K.copy_view(t, c)
            out.append(c)
        return out

    a = copies(dev(r.standard_normal(shape).astype(np.float32)))
    b = copies(dev(r.standard_normal(shape).astype(np.float32)))
    a64 = copies(dev(r.standard_normal(shape)))
    lab = copies(dev(r.integers(0, 1000, shape, dtype=np.int64)))
    o32 = [_fresh(shape) for _ in range(SETS)]
    o64 = [_fresh(shape, nt.float64) for _ in range(SETS)]
    ob = [_fresh(shape, nt.bool_) for _ in range(SETS)]
    B, Mb = 16, 1024
    xb = dev(r.standard_normal((B, Mb, Mb)).astype(np.float32))
    yb = dev((r.standard_normal((B, Mb, Mb)) / np.sqrt(Mb)).astype(np.float32))
    ob3 = _fresh((B, Mb, Mb))
    rows, width = 50000, 1024
    tables = copies(dev(r.standard_normal((rows, width)).astype(np.float32)))
    ids = r.permutation(rows)[:8192]
    gplan = _fancy.compute_plan(tables[0].shape, (ids.tolist(),))
    gouts = [_fresh(gplan.new_shape) for _ in range(SETS)]
    keep: list = []
    gargs = [_index_args("nt_gather_axes", gplan, tables[k], gouts[k], keep) for k in range(SETS)]
    sargs = [_index_args("nt_scatter_axes", gplan, gouts[k], tables[k], keep) for k in range(SETS)]
    vws = [(view(a[k]), view(b[k]), view(ob[k])) for k in range(SETS)]
    keep.append(vws)
    cmp_args = [(_lib.GT, ctypes.byref(x), ctypes.byref(y), ctypes.byref(z)) for x, y, z in vws]
    gbytes = 2 * gouts[0].numel * 4 + 8 * len(ids)
    a3 = [t.reshape(64, 1024, 1024) for t in a]
    o3 = [t.reshape(64, 1024, 1024) for t in o32]
    p3 = copies(dev(r.standard_normal((64, 512, 512)).astype(np.float32)))
    q3 = [_fresh((64, 512, 512)) for _ in range(SETS)]
    q3r = [_fresh((512, 512, 64)) for _ in range(SETS)]
    launch = {
        "cast|f32->f64": lambda k: K.copy_view(a[k], o64[k]),
        "cast|f64->f32": lambda k: K.copy_view(a64[k], o32[k]),
        "cast|i64->f32": lambda k: K.copy_view(lab[k], o32[k]),
        "compare|gt": lambda k: _lib.call("nt_binary", *cmp_args[k]),
        "copy|transposed": lambda k: K.copy_view(a[k].T, o32[k]),
        "copy|3-D transpose(1,2)": lambda k: K.copy_view(a3[k].transpose(1, 2), o3[k]),
        "copy|[64,512,512].transpose(1,2)": lambda k: K.copy_view(p3[k].transpose(1, 2), q3[k]),
        "copy|[64,512,512].transpose(0,2)": lambda k: K.copy_view(p3[k].transpose(0, 2), q3r[k]),
        "matmul|batched 16x1024^3": lambda k: K.matmul_into(xb, yb, ob3, accumulate=False),
        "gather|8192 rows of [50000,1024]": lambda k: _lib.call("nt_gather_axes", *gargs[k]),
        "scatter|8192 rows of [50000,1024]": lambda k: _lib.call("nt_scatter_axes", *sargs[k]),
        "uniform|f32 [8192,8192]": lambda k: _lib.call(
            "nt_device_uniform", o32[k]._storage.data_ptr(), int(nt.float32), n, 0.0, 1.0),
    }
    assert list(launch) == [c[0] for c in NEXT_ROWS] and gbytes == NEXT_ROWS[9][3]
    cases = {name: (launch[name], nbytes, flop) for name, _, _, nbytes, flop in NEXT_ROWS}
    out = {}
    for name, (fn, nbytes, flop) in cases.items():
        # back-to-back launches of one case between two events: the average
        # launch, with the stream kept busy
        fn(SETS - 1)
        e0, e1 = _lib.Event(), _lib.Event()
        e0.record()
        for it in range(iters):
            fn(it % SETS)
        e1.record()
        nt.sync()
        avg = e0.elapsed_ms(e1) / iters
        if flop is not None:
            tf = flop / (avg * 1e-3) / 1e12
            out[name] = {"ms": round(avg, 5), "TFLOP/s": round(tf, 2),
                         "frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)}
        else:
            gbs = nbytes / (avg * 1e-3) / 1e9
            out[name] = {"ms": round(avg, 5), "GB/s": round(gbs, 1),
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": nbytes}
    out["uniform|f32 [8192,8192]"]["Gdraws/s"] = round(n / (out["uniform|f32 [8192,8192]"]["ms"] * 1e-3) / 1e9, 2)
    # the same stream on one host core (the reference draws it there)
    hn = 1 << 24
    hbuf = np.empty(hn, np.float32)
    t0 = time.perf_counter()
    _lib.call("nt_host_uniform", hbuf.ctypes.data, int(nt.float32), hn, 0.0, 1.0)
    out["uniform|f32 host, 1 core"] = {"Gdraws/s": round(hn / (time.perf_counter() - t0) / 1e9, 3)}
    return out


def bench_copy_reference(iters: int = 8) -> dict:
    """The library's own contiguous copy (the elementwise engine's flat
    kernel, nt_copy) on cold buffers: 4 pairs of 2^26 fp32 arrays (2 GB in
    all, far beyond the 256 MB Infinity Cache) used in turn, launches back
    to back between two events (the four copies are independent, so the
    launch window lets them overlap, as it does the sweep's kernels).  The
    practical HBM rate of a read + write stream on this GPU, against which
    the sweep's fraction of the published peak reads."""
    n = 1 << 26
    pairs = [(_fresh((n,)), _fresh((n,))) for _ in range(4)]
    K.copy_view(*pairs[-1])
    e0, e1 = _lib.Event(), _lib.Event()
    e0.record()
    for it in range(iters):
        K.copy_view(*pairs[it % 4])
    e1.record()
    nt.sync()
    ms = e0.elapsed_ms(e1) / iters
    gbs = 8 * n / (ms * 1e-3) / 1e9
    return {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
            "bytes": 8 * n}


def bench_copy_sweep_size(iters: int = 16) -> dict:
    """The same copy at the sweep's size: 2^24 fp32 elements in, 2^24 out
    (the bytes of one contiguous unary forward), contiguous and from a `.T`
    view of a [4096, 4096] array (the bytes and layout of a transposed
    unary forward), over 8 rotating pairs (1 GB, not Infinity-Cache
    resident).  `ms` is timed as the sweep's per-kernel pass times its
    kernels, events around each launch (every copy ordered after the one
    before): the ceiling one launch of that length reaches, ramp-up and
    drain included, for the per-kernel figures.  `back_to_back_ms` is the
    same launches between two events only, where the independent copies
    overlap in the launch window."""
    n = 1 << 24
    side = 1 << 12
    pairs = [(_fresh((side, side)), _fresh((side, side))) for _ in range(8)]
    out = {}
    for name, src in (("contiguous", lambda a: a), ("transposed", lambda a: a.T)):
        for a, b in pairs:
            K.copy_view(src(a), b)
        tm = Timer()
        for it in range(iters):
            a, b = pairs[it % 8]
            tm.run(name, lambda a=a, b=b: K.copy_view(src(a), b))
        nt.sync()
        ds = tm.durations()[name]
        ms = sum(ds) / len(ds)
        e0, e1 = _lib.Event(), _lib.Event()
        e0.record()
        for it in range(iters):
            a, b = pairs[it % 8]
            K.copy_view(src(a), b)
        e1.record()
        nt.sync()
        b2b = e0.elapsed_ms(e1) / iters
        gbs = 8 * n / (ms * 1e-3) / 1e9
        out[name] = {"ms": round(ms, 5), "GB/s": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": 8 * n,
                     "back_to_back_ms": round(b2b, 5),
                     "back_to_back_frac": round(8 * n / (b2b * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    return out


# ------------------------------------------------------------ CPU baseline


def _host_cpu() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _timed(fn) -> float:
    t0 = time.perf_counter()
    fn()
    return time.perf_counter() - t0


def cpu_per_op(rows: int = 4096) -> dict:
    """ref-cpu-1t: the oracle (the reference's CPU kernels and Python
    backward compositions, restated; single thread, as the reference has no
    threads) timed per op on bounded samples of configs 2-5, with the GPU
    figures' byte / FLOP models, so that every GPU per-kernel figure has a
    CPU figure beside it.

    config 2: [rows, 4096] (by default the whole [4096, 4096] workload,
      10-40 s single-threaded depending on the host; a smaller sample would
      sit in the host caches and overstate the CPU rate), each op's forward and its backward
      composition plus the engine's accumulate, both layouts (the transposed
      operands are .T views of contiguous [4096, rows] arrays); the inputs
      of every op come from one pool per layout drawn from the op domains
      (arrays far larger than the host caches, so reuse warms nothing);
    config 3: [512, 8192] (1/16 of the rows), sum / max / min forward and
      sum (accumulate) / mean / max backward along axis 0, axis 1 and all;
    config 4: 2 output rows of each product (fwd, dA = dG.B^T, dB = A^T.dG,
      with A contiguous and as a .T view; dA does not read A), the
      reference's k loop per output, with the whole product's time
      extrapolated linearly in rows;
    config 5: one training step of the 4-layer network at batch 4, and the
      SGD update alone; the rest of the step is linear in the batch, so the
      step at batch 8192 is estimated as update + (step - update) * 2048."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    r = np.random.default_rng(7)
    out: dict = {"elementwise": {}, "reductions": {}, "matmul": {}, "mlp": {}}
    # ---- config 2
    shape = (rows, 4096)
    n = rows * 4096
    tot_b = tot_s = 0.0
    for layout in ("contig", "transposed"):
        mk = (lambda a: a) if layout == "contig" else (lambda a: np.ascontiguousarray(a.T).T)

        def draw(dom):
            v = r.standard_normal(shape) if dom is None else r.uniform(dom[0], dom[1], shape)
            return mk(v.astype(np.float32))
        pool = {dom: draw(dom) for dom in (None, (0.5, 2), (0.1, 4), (-4, 4))}
        pool["b"] = draw(None)
        g = r.standard_normal(shape).astype(np.float32)
        olds = [draw(None) for _ in range(2)]
        for name, op in (("add", O.ADD), ("sub", O.SUB), ("mul", O.MUL), ("truediv", O.DIV)):
            a = pool[None]
            b = pool[(0.5, 2)] if name == "truediv" else pool["b"]
            tf = _timed(lambda: O.binary(op, a, b))

            def bwd():
                ga, gb = O.bwd_binary(op, g, a, b)
                O.inplace(O.ADD, olds[0], ga)
                O.inplace(O.ADD, olds[1], gb)
            tb = _timed(bwd)
            for phase, t in (("fwd", tf), ("bwd", tb)):
                nb = ew_bytes(name, phase) * n // N_ELEM
                out["elementwise"][f"{name}|{layout}|{phase}"] = round(nb / t / 1e9, 3)
                tot_b += nb
                tot_s += t
        for name, op, dom, saved, e in UNARY_OPS:
            x = pool[dom]
            old = olds[0]
            oop = {"neg": O.NEG, "exp": O.EXP, "log": O.LOG, "sqrt": O.SQRT, "pow": O.POW,
                   "relu": O.RELU, "sigmoid": O.SIGMOID, "tanh": O.TANH}[name]
            y = None

            def fwd():
                nonlocal y
                y = O.unary(oop, x, e)
            tf = _timed(fwd)
            chain = {"neg": lambda: O.bwd_neg(g), "exp": lambda: O.bwd_exp(g, y),
                     "log": lambda: O.bwd_log(g, x), "sqrt": lambda: O.bwd_sqrt(g, y),
                     "pow": lambda: O.bwd_pow(g, x, 2.5), "relu": lambda: O.bwd_relu(g, y),
                     "sigmoid": lambda: O.bwd_sigmoid(g, y), "tanh": lambda: O.bwd_tanh(g, y)}[name]
            tb = _timed(lambda: O.inplace(O.ADD, old, chain()))
            for phase, t in (("fwd", tf), ("bwd", tb)):
                nb = ew_bytes(name, phase) * n // N_ELEM
                out["elementwise"][f"{name}|{layout}|{phase}"] = round(nb / t / 1e9, 3)
                tot_b += nb
                tot_s += t
    part = "the whole config-2 workload" if rows == 4096 else f"1/{4096 // rows} of config 2"
    out["elementwise_sample"] = f"[{rows}, 4096] ({part})"
    baseline = {"value": round(tot_b / tot_s / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"config-2 sweep on [{rows},4096] ({part}), "
                          f"forward + reference backward composition + accumulate, both layouts, "
                          f"single thread, {tot_s:.1f} s",
                "host_cpu": _host_cpu(), "host_nproc": os.cpu_count()}
    # ---- config 3
    x = r.standard_normal((512, 8192)).astype(np.float32)
    nx = x.size
    for label, axes in (("axis0", (0,)), ("axis1", (1,)), ("full", (0, 1))):
        kshape = tuple(s_ for i, s_ in enumerate(x.shape) if i not in axes)
        gshape = tuple(1 if i in axes else s_ for i, s_ in enumerate(x.shape))
        for name, op in (("sum", O.R_SUM), ("max", O.R_MAX), ("min", O.R_MIN)):
            t = _timed(lambda: O.reduce(op, x, axes, np.float32 if op == O.R_SUM else None))
            out["reductions"][f"{name}|{label}|fwd"] = round(nx * 4 / t / 1e9, 3)
        g = r.standard_normal(kshape).astype(np.float32)
        gb = np.broadcast_to(g.reshape(gshape), x.shape)
        old = r.standard_normal(x.shape).astype(np.float32)
        t = _timed(lambda: O.inplace(O.ADD, old, gb))  # engine: grad += expand(g)
        out["reductions"][f"sum|{label}|bwd"] = round(2 * nx * 4 / t / 1e9, 3)
        dn = nx // max(1, int(np.prod(kshape)))
        t = _timed(lambda: O.binary(O.DIV, gb, np.broadcast_to(O.scalar(dn, np.float32), x.shape)))
        out["reductions"][f"mean|{label}|bwd"] = round(nx * 4 / t / 1e9, 3)
        t = _timed(lambda: O.sel_bwd(O.R_MAX, g, x, axes))
        out["reductions"][f"max|{label}|bwd"] = round(nx * 4 / t / 1e9, 3)
    out["reductions_sample"] = "[512, 8192] fp32 (1/16 of config 3)"
    # ---- config 4
    rs = 2
    for (M, Kd, N) in ((4096, 4096, 4096), (8192, 1024, 4096)):
        A = r.standard_normal((M, Kd)).astype(np.float32)
        B = (r.standard_normal((Kd, N)) / np.sqrt(Kd)).astype(np.float32)
        G = r.standard_normal((M, N)).astype(np.float32)
        At = np.ascontiguousarray(A.T).T  # A as the .T view of a [K, M] storage
        for a_layout, AA in (("contig", A), ("transposed", At)):
            entry = {}
            for name, x1, x2, full_rows, (m_, k_, n_) in (
                    ("fwd", AA[:rs], B, M, (M, Kd, N)),
                    ("dA", G[:rs], B.T, M, (M, N, Kd)),
                    ("dB", AA[:, :rs].T, G, Kd, (Kd, M, N))):
                if name == "dA" and a_layout == "transposed":
                    entry[name] = out["matmul"][f"{M}x{Kd}x{N}|contig"][name]  # same operands
                    continue
                t = _timed(lambda: O.matmul(x1, x2))
                gf = 2.0 * rs * k_ * n_ / t / 1e9
                entry[name] = {"GFLOP/s": round(gf, 3),
                               "full_product_s_extrapolated": round(t * full_rows / rs, 1)}
            out["matmul"][f"{M}x{Kd}x{N}|{a_layout}"] = entry
    out["matmul_sample"] = f"{rs} output rows per product, extrapolated linearly"
    # ---- config 5: one step at batch 4, split into its batch-independent
    # part (the SGD update of all 41.9 M parameters, timed on its own) and a
    # per-sample part (everything else is linear in the batch)
    bsz = 4
    xb = r.standard_normal((bsz, C5_DIMS[0])).astype(np.float32)
    tb_ = r.standard_normal((bsz, C5_DIMS[-1])).astype(np.float32)
    params = [((r.standard_normal((C5_DIMS[i], C5_DIMS[i + 1])) * np.sqrt(2.0 / C5_DIMS[i])).astype(np.float32),
               np.zeros(C5_DIMS[i + 1], np.float32)) for i in range(4)]
    t_step = _timed(lambda: O.mlp_step(params, xb, tb_, C5_ACTS, C5_LR, parallel=False))

    def sgd():  # optimizers.py:51, p -= p.grad * lr, on gradient-sized arrays
        for W, b in params:
            O.inplace(O.SUB, W, O.mul_scalar(W, C5_LR))
            O.inplace(O.SUB, b, O.mul_scalar(b, C5_LR))
    t_sgd = min(t_step, _timed(sgd))
    full = t_sgd + (t_step - t_sgd) * C5_BATCH / bsz
    out["mlp"] = {"step_s_at_batch_4": round(t_step, 3), "sgd_update_s": round(t_sgd, 3),
                  "step_s_extrapolated_batch_8192": round(full, 1),
                  "step/s_extrapolated": round(1.0 / full, 6)}
    out["threads"] = 1
    out["host_cpu"] = _host_cpu()
    out["host_nproc"] = os.cpu_count()
    return {"baseline": baseline, "per_op": out}


def attach_cpu(parts: dict, cpu: dict) -> None:
    """Writes each CPU figure next to the matching GPU per-kernel figure
    (same key and byte / FLOP model) and the GPU/CPU ratio."""
    ew = parts.get("elementwise_per_kernel", {})
    for k, v in cpu["elementwise"].items():
        if k in ew:
            ew[k]["cpu_1t_GB/s"] = v
            ew[k]["gpu_over_cpu"] = round(ew[k]["GB/s"] / v, 1)
    red = parts.get("reductions", {}).get("per_kernel", {})
    for k, v in cpu["reductions"].items():
        if k in red:
            red[k]["cpu_1t_GB/s"] = v
            red[k]["gpu_over_cpu"] = round(red[k]["GB/s"] / v, 1)
    mm = parts.get("matmul", {})
    for k, ent in cpu["matmul"].items():
        for name, v in ent.items():
            if k in mm and name in mm[k]:
                mm[k][name]["cpu_1t_GFLOP/s"] = v["GFLOP/s"]
                mm[k][name]["cpu_1t_full_product_s"] = v["full_product_s_extrapolated"]
                mm[k][name]["gpu_over_cpu"] = round(mm[k][name]["TFLOP/s"] * 1e3 / v["GFLOP/s"], 0)
    if "mlp" in parts and cpu.get("mlp"):
        parts["mlp"]["cpu_1t_step_s_extrapolated"] = cpu["mlp"]["step_s_extrapolated_batch_8192"]
        parts["mlp"]["gpu_over_cpu"] = round(
            cpu["mlp"]["step_s_extrapolated_batch_8192"] / (parts["mlp"]["ms_per_step"] * 1e-3), 0)


def cpu_parts() -> dict:
    """The oracle (the reference's CPU kernels restated) on bounded samples
    of configs 1, 3 and 4, on this host's cores: single-threaded like the
    reference, plus the bit-identical OpenMP matmul on all cores."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    r = np.random.default_rng(9)
    out: dict = {"cores_available": os.cpu_count(), "threads_omp": O.threads()}
    # config 3 sample: [1024, 8192] (1/8 of the rows)
    x = r.standard_normal((1024, 8192)).astype(np.float32)
    red = {}
    for name, op, dt in (("sum", O.R_SUM, np.float32), ("max", O.R_MAX, None)):
        for label, axes in (("axis0", (0,)), ("axis1", (1,)), ("full", (0, 1))):
            t0 = time.perf_counter()
            O.reduce(op, x, axes, dt)
            dt_s = time.perf_counter() - t0
            red[f"{name}|{label}|fwd"] = round(x.nbytes / dt_s / 1e9, 3)
    out["reductions_GB/s_1thread"] = red
    out["reductions_sample"] = "[1024, 8192] fp32 (1/8 of config 3)"
    # config 4 sample: 512^3 single thread, 1024^3 on all cores
    mm = {}
    for n, par in ((512, False), (1024, True)):
        a = r.standard_normal((n, n)).astype(np.float32)
        b = (r.standard_normal((n, n)) / np.sqrt(n)).astype(np.float32)
        t0 = time.perf_counter()
        O.matmul(a, b, parallel=par)
        dt_s = time.perf_counter() - t0
        mm[f"{n}^3|{'omp' if par else '1thread'}"] = round(2 * n**3 / dt_s / 1e9, 3)
    out["matmul_GFLOP/s"] = mm
    # config 1: the 2-layer MLP step, single thread
    X = r.standard_normal((64, 784)).astype(np.float32)
    T = np.eye(10, dtype=np.float32)[r.integers(0, 10, 64)]
    params = [((r.standard_normal((784, 256)) * np.sqrt(2 / 784)).astype(np.float32),
               np.zeros(256, np.float32)),
              ((r.standard_normal((256, 10)) * np.sqrt(2 / 256)).astype(np.float32),
               np.zeros(10, np.float32))]
    t0 = time.perf_counter()
    steps = 5
    for _ in range(steps):
        O.mlp_step(params, X, T, ["relu"], 0.01, parallel=False)
    out["mlp_config1_step/s_1thread"] = round(steps / (time.perf_counter() - t0), 2)
    return out


# ---------------------------------------------------------------- profiles

PMC_SET1 = ("SQ_WAVES SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_WAIT_INST_LDS "
            "SQ_LDS_BANK_CONFLICT SQ_ACTIVE_INST_LDS GRBM_GUI_ACTIVE")
PMC_SET2 = ("SQ_INSTS_VALU SQ_ACTIVE_INST_VALU SQ_INSTS_LDS SQ_INSTS_VMEM_RD SQ_INSTS_VMEM_WR "
            "SQ_INST_LEVEL_VMEM SQ_ACTIVE_INST_VMEM SQ_LEVEL_WAVES GRBM_GUI_ACTIVE")
_PROF = "rocprofv3 --kernel-trace --stats --output-format csv -d gpurun_out/{d} -o run -- python -u bench.py {a}"
_PMC = "rocprofv3 --pmc {c} --output-format csv -d gpurun_out/{d} -o run -- python -u bench.py {a}"
PROFILE_CMDS = {
    "sweep": _PROF.format(d="prof_sweep", a="--steps 5 --warmup 2 --parts ew,first --calib"),
    "red": _PROF.format(d="prof_red", a="--parts red"),
    "mm": _PROF.format(d="prof_mm", a="--parts mm"),
    "mlp": _PROF.format(d="prof_mlp", a="--parts mlp --mlp-steps 5"),
    "next": _PROF.format(d="prof_next", a="--parts next"),
    "mm_pmc": _PMC.format(
        c="SQ_INSTS_MFMA SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES SQ_WAVE_CYCLES "
          "SQ_WAIT_INST_LDS SQ_LDS_BANK_CONFLICT",
        d="prof_mm_pmc", a="--parts mm"),
    "fetch": _PMC.format(c="FETCH_SIZE", d="prof_fetch", a="--steps 1 --warmup 0 --parts ew --calib"),
    "write": _PMC.format(c="WRITE_SIZE", d="prof_write", a="--steps 1 --warmup 0 --parts ew --calib"),
    # issue / wait / occupancy counters, two passes per part
    "ew_pmc1": _PMC.format(c=PMC_SET1, d="prof_ew_pmc1", a="--steps 1 --warmup 0 --parts ew"),
    "ew_pmc2": _PMC.format(c=PMC_SET2, d="prof_ew_pmc2", a="--steps 1 --warmup 0 --parts ew"),
    "mm_pmc1": _PMC.format(c=PMC_SET1, d="prof_mm_pmc1", a="--parts mm"),
    "mm_pmc2": _PMC.format(c=PMC_SET2, d="prof_mm_pmc2", a="--parts mm"),
    "red_pmc1": _PMC.format(c=PMC_SET1, d="prof_red_pmc1", a="--parts red"),
    "red_pmc2": _PMC.format(c=PMC_SET2, d="prof_red_pmc2", a="--parts red"),
    # HBM bytes of the reductions and of the MLP step (same calibration)
    "red_fetch": _PMC.format(c="FETCH_SIZE", d="prof_red_fetch", a="--parts red --calib"),
    "red_write": _PMC.format(c="WRITE_SIZE", d="prof_red_write", a="--parts red --calib"),
    "mlp_fetch": _PMC.format(c="FETCH_SIZE", d="prof_mlp_fetch", a="--parts mlp --mlp-steps 3 --calib"),
    "mlp_write": _PMC.format(c="WRITE_SIZE", d="prof_mlp_write", a="--parts mlp --mlp-steps 3 --calib"),
}
# Transposed-tile variants profiled inside the sweep (the library's
# NT_TILE_SHAPE / NT_TILE_ORIENT measurement knobs; results are identical):
# label -> environment prefix.
TILE_VARIANTS = {
    "rule": "",
    "64x64": "NT_TILE_SHAPE=64x64",
    "64x128": "NT_TILE_SHAPE=64x128",
    "128x128": "NT_TILE_SHAPE=128x128",
    "32x256": "NT_TILE_SHAPE=32x256",
    "keep": "NT_TILE_ORIENT=keep",
    "swap": "NT_TILE_ORIENT=swap",
}
for _lbl, _env in TILE_VARIANTS.items():
    for _i, _set in ((1, PMC_SET1), (2, PMC_SET2)):
        PROFILE_CMDS[f"tile_{_lbl}_pmc{_i}"] = ((_env + " ") if _env else "") + _PMC.format(
            c=_set, d=f"prof_tile_{_lbl}_{_i}", a="--steps 1 --warmup 0 --parts none")

PROFILE_FILES = {
    "sweep": ("elementwise_sweep_config2_trace.md", "Kernel statistics: config-2 elementwise sweep (the headline)"),
    "red": ("reduce_config3_trace.md", "Kernel statistics: config-3 reductions [8192, 8192] fp32"),
    "mm": ("matmul_config4_trace.md", "Kernel statistics: config-4 MatMulOp forward + dA + dB"),
    "mlp": ("mlp_config5_trace.md", "Kernel statistics: config-5 4-layer MLP training steps"),
    "next": ("next_rows_trace.md", "Kernel statistics: casts, comparison, strided copies (2-D and batched 3-D transposes, one tile kernel), device uniform draws, "
                                   "batched matmul, gather / scatter (the rows beside the path)"),
}
_UN = {0: "exp", 1: "log", 2: "neg", 3: "relu", 4: "sqrt", 5: "tanh", 6: "sigmoid", 7: "pow"}
_BI = {0: "add", 1: "sub", 2: "mul", 3: "truediv"}


def _short(name: str) -> str:
    import re
    n = name.replace("(anonymous namespace)::", "")
    n = re.sub(r"\(.*$", "", n)
    return n.replace("void nt::", "").replace("nt::", "")


def _mdc(v) -> str:
    """A markdown table cell: `|` inside a key (e.g. add|contig|fwd) escaped."""
    return str(v).replace("|", "\\|")


def _sweep_key(name: str):
    """Kernel name -> 'op|layout|phase' of the sweep (flat kernel: contiguous
    operands; tile kernel: transposed views).  A backward is `bwd` when it
    accumulates into its gradients (UnaryBwd's ACC, BinaryBwd's AA / AB for
    the gradients it produces), `bwd_first` when it overwrites them."""
    import re
    layout = "contig" if "ew_flat_kernel" in name else ("transposed" if "ew_tile4_kernel" in name else None)
    m = re.search(r"(UnaryFwd|UnaryBwd|BinaryFwd|BinaryBwd)<(\d+)((?:, [a-z0-9 ]+)*)>", name)
    if not layout or not m:
        return None
    kind, op = m.group(1), int(m.group(2))
    opn = (_UN if kind.startswith("Unary") else _BI)[op]
    if kind.endswith("Fwd"):
        return f"{opn}|{layout}|fwd"
    flags = [a.strip() == "true" for a in m.group(3).split(",")[2:]]  # after OP, T
    if kind == "UnaryBwd":
        acc = flags[:1]
    else:  # NA, NB, AA, AB: the accumulate flags of the produced gradients
        acc = [flags[2 + i] for i in range(2) if flags[i]]
    if all(acc):
        return f"{opn}|{layout}|bwd"
    return f"{opn}|{layout}|{'bwd_first' if not any(acc) else 'bwd_mixed'}"


def _mm_calls():
    """bench_matmul's calls in queue order: (M, K, N, A layout, product, is
    the untimed first round)."""
    out = []
    for (M, Kd, N) in MM_SHAPES:
        for lay in ("contig", "transposed"):
            for it in range(MM_ITERS + 1):
                for prod in ("fwd", "dA", "dB"):
                    out.append((M, Kd, N, lay, prod, it == 0))
    return out


def _mm_dispatches(rows):
    """Assigns matmul dispatches (dicts with Kernel_Name, in dispatch order)
    to bench_matmul's calls: each call is one product kernel, followed by
    the split-K sum kernel when K is split.  Yields (call, row, is_sum)."""
    calls = _mm_calls()
    ci = -1
    for r in rows:
        name = r["Kernel_Name"]
        if "mm_" not in name:
            continue
        is_sum = "splitk_sum" in name
        if not is_sum:
            ci += 1
        if 0 <= ci < len(calls):
            yield calls[ci], r, is_sum


SWEEP_TIMER_SWEEPS = 2  # bench_elementwise's per-kernel pass under PROFILE_CMDS["sweep"] (--steps 5)


def _summarize_sweep_trace(path: str, out_md: str) -> None:
    """Config-2 kernel times from the kernel trace: per sweep kernel, the
    average over every dispatch (warm-up, whole-step and per-kernel passes;
    in the whole-step passes independent kernels overlap, which stretches
    each one's start-to-end time) and over the per-kernel pass alone, whose
    launches are ordered one after another -- the durations bench.py's
    per-kernel figures and roofline come from."""
    import csv
    rows = sorted(csv.DictReader(open(os.path.join(path, "run_kernel_trace.csv"))),
                  key=lambda r: int(r["Dispatch_Id"]))
    per: dict = {}
    for r in rows:
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        key = (_short(r["Kernel_Name"]), _sweep_key(r["Kernel_Name"]) or "",
               f"{r['Grid_Size_X']}x{r['Grid_Size_Y']}")
        per.setdefault(key, []).append(us)
    total = sum(sum(v) for v in per.values())
    with open(out_md, "w") as o:
        o.write(f"# {PROFILE_FILES['sweep'][1]}\n\nCommand (repo root on the GPU box):\n\n"
                f"```\n{PROFILE_CMDS['sweep']}\n```\n\n"
                "Summarised with `python bench.py --summarize sweep gpurun_out/prof_sweep` from the "
                "kernel trace.  `all` averages every dispatch of the kernel (2 warm-up and 5 "
                "whole-step sweeps, where independent kernels are queued without the stream "
                "barrier and overlap their neighbours, then the per-kernel pass); `per-kernel "
                f"pass` averages the last {SWEEP_TIMER_SWEEPS} dispatches, bench.py's per-kernel "
                "pass, whose events order every launch after the one before: the durations the "
                "bench line's per-kernel figures and roofline are measured on.  "
                "`bwd_first` rows are bench.py's first-write pass (part `first`: the same "
                "backwards overwriting their gradients, events around each launch; every dispatch "
                "of theirs belongs to that pass).  "
                "`stream_fence_kernel` is the empty barrier kernel queued before an event or a "
                "copy while overlapped kernels may still run.\n\n"
                "| kernel | sweep key | grid | calls | all avg us | per-kernel pass avg us | "
                "min us | max us | share of kernel time % |\n|---|---|---|---|---|---|---|---|---|\n")
        for (name, sk, grid), v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
            tp = v[-SWEEP_TIMER_SWEEPS:] if sk else v
            o.write(f"| `{name[:150]}` | {_mdc(sk)} | {grid} | {len(v)} | {sum(v) / len(v):.2f} | "
                    f"{sum(tp) / len(tp):.2f} | {min(v):.2f} | {max(v):.2f} | "
                    f"{100 * sum(v) / total:.2f} |\n")


def _summarize_next_trace(path: str, out_md: str) -> None:
    """Next-row kernel times per bench_next case from the kernel trace: the
    dispatches from the first case's kernel on are assigned to the cases in
    queue order (NEXT_ROWS: 1 + NEXT_ITERS calls each, its kernels per call;
    the library's barrier kernels and the runtime's copy kernels left out),
    each case's first call untimed as in bench_next.  Several cases share a
    kernel (and a grid size), so a per-kernel table cannot tell them apart."""
    import csv
    rows = sorted(csv.DictReader(open(os.path.join(path, "run_kernel_trace.csv"))),
                  key=lambda r: int(r["Dispatch_Id"]))
    # neither the barrier kernels nor the runtime's copy kernels (the first
    # device draw uploads the generator's tables) belong to a case's calls
    rows = [r for r in rows if "stream_fence_kernel" not in r["Kernel_Name"]
            and "__amd_rocclr" not in r["Kernel_Name"]]
    i = next(j for j, r in enumerate(rows) if NEXT_ROWS[0][1] in r["Kernel_Name"])
    lines = []
    for name, pat, per_call, nbytes, flop in NEXT_ROWS:
        us, kname = [], ""
        for c in range(1 + NEXT_ITERS):
            ks = rows[i:i + per_call]
            i += per_call
            if len(ks) < per_call or not all(pat in r["Kernel_Name"] for r in ks):
                raise SystemExit(f"next-row trace: the dispatches at {i - per_call} are not {name}")
            kname = " + ".join(_short(r["Kernel_Name"])[:90] for r in ks)
            if c:
                us.append(sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in ks) / 1e3)
        avg = sum(us) / len(us)
        if flop is not None:
            rate = f"{flop / (avg * 1e-6) / 1e12:.1f} TFLOP/s | {flop / (avg * 1e-6) / 1e12 / FP32_MFMA_PEAK_TFLOPS:.3f}"
        else:
            rate = f"{nbytes / (avg * 1e-6) / 1e9:.1f} GB/s | {nbytes / (avg * 1e-6) / 1e9 / HBM_PEAK_GBS:.3f}"
        lines.append(f"| {_mdc(name)} | `{kname}` | {len(us)} | {avg:.2f} | {min(us):.2f} | {max(us):.2f} | {rate} |")
    with open(out_md, "w") as o:
        o.write(f"# {PROFILE_FILES['next'][1]}\n\nCommand (repo root on the GPU box):\n\n"
                f"```\n{PROFILE_CMDS['next']}\n```\n\n"
                "Summarised with `python bench.py --summarize next gpurun_out/prof_next` from the "
                "kernel trace: each case's dispatches, in queue order, its first call untimed as in "
                "bench.py.  `us` is the kernel time per call (the uniform draw: its four kernels "
                "summed); the rate is the case's algorithmic bytes (or FLOP) over it, against "
                f"{HBM_PEAK_GBS / 1000:.0f} TB/s (or {FP32_MFMA_PEAK_TFLOPS} TFLOP/s).  bench.py's own "
                "figures time the same calls back to back between two events, where independent "
                "elementwise launches over the rotating operand sets may overlap.\n\n"
                "| case | kernel(s) | timed calls | avg us | min us | max us | rate | frac |\n"
                "|---|---|---|---|---|---|---|---|\n")
        o.write("\n".join(lines) + "\n")


def _summarize_mm_trace(path: str, out_md: str) -> None:
    """Config-4 kernel times per product and shape from the kernel trace
    (one row per (shape, A layout, product): the product kernel and, with
    split K, the sum kernel), timed rounds only, as bench_matmul reports."""
    import csv
    rows = sorted(csv.DictReader(open(os.path.join(path, "run_kernel_trace.csv"))),
                  key=lambda r: int(r["Dispatch_Id"]))
    acc: dict = {}
    for (M, Kd, N, lay, prod, warm), r, is_sum in _mm_dispatches(rows):
        if warm:
            continue
        e = acc.setdefault((M, Kd, N, lay, prod), {"main": [], "sum": [], "name": "", "grid": ""})
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        if is_sum:
            e["sum"].append(us)
        else:
            e["main"].append(us)
            e["name"] = _short(r["Kernel_Name"])
            e["grid"] = f"{r['Grid_Size_X']}x{r['Grid_Size_Y']}"
    with open(out_md, "w") as o:
        o.write("# Kernel times: config-4 MatMulOp forward + dA + dB, per product and shape\n\n")
        o.write(f"Command (repo root on the GPU box):\n\n```\n{PROFILE_CMDS['mm']}\n```\n\n")
        o.write("Summarised with `python bench.py --summarize mm gpurun_out/prof_mm` from the "
                "kernel trace: each dispatch is matched to bench_matmul's call sequence (per shape, "
                "per A layout, rounds of fwd, dA = dG.B^T, dB = A^T.dG; the first round untimed), "
                "so the two config-4 shapes get rows of their own.  `sum us` is the split-K sum "
                "kernel where K is split; TFLOP/s = 2MNK / (product + sum).  Grid in work-items "
                "(x by split-K slices).\n\n")
        o.write("| shape MxKxN | A | product | kernel | grid | n | product us | sum us | TFLOP/s | frac of 157.3 |\n"
                "|---|---|---|---|---|---|---|---|---|---|\n")
        for (M, Kd, N, lay, prod), e in acc.items():
            mu = sum(e["main"]) / len(e["main"])
            su = sum(e["sum"]) / len(e["sum"]) if e["sum"] else 0.0
            m_, k_, n_ = {"fwd": (M, Kd, N), "dA": (M, N, Kd), "dB": (Kd, M, N)}[prod]
            tf = 2.0 * m_ * n_ * k_ / ((mu + su) * 1e-6) / 1e12
            o.write(f"| {M}x{Kd}x{N} | {lay} | {prod} | `{e['name'][:60]}` | {e['grid']} | {len(e['main'])} | "
                    f"{mu:.1f} | {su:.1f} | {tf:.1f} | {tf / FP32_MFMA_PEAK_TFLOPS:.3f} |\n")


def _summarize_mm_pmc(path: str, out_md: str) -> None:
    """MFMA-pipe utilisation per product and shape: busy cycles of the
    matrix pipe summed over the 1024 SIMDs, over SIMDs x duration x clock,
    each dispatch matched to bench_matmul's call sequence (_mm_dispatches)."""
    import csv
    simds, clock_ghz = 256 * 4, 2.4
    disp: dict[int, dict] = {}
    for r in csv.DictReader(open(os.path.join(path, "run_counter_collection.csv"))):
        d = disp.setdefault(int(r["Dispatch_Id"]), {
            "Kernel_Name": r["Kernel_Name"], "grid": r["Grid_Size"],
            "dur_ns": int(r["End_Timestamp"]) - int(r["Start_Timestamp"])})
        d[r["Counter_Name"]] = float(r["Counter_Value"])
    rows = [disp[k] for k in sorted(disp)]
    per: dict = {}
    for (M, Kd, N, lay, prod, warm), d, is_sum in _mm_dispatches(rows):
        if warm or is_sum:
            continue
        per.setdefault((M, Kd, N, lay, prod), []).append(d)
    with open(out_md, "w") as o:
        o.write("# MFMA-pipe utilisation: config-4 matmul kernels, per product and shape\n\n")
        o.write(f"Command (repo root on the GPU box):\n\n```\n{PROFILE_CMDS['mm_pmc']}\n```\n\n")
        o.write("Summarised with `python bench.py --summarize mm_pmc gpurun_out/prof_mm_pmc`; "
                "each dispatch is matched to bench_matmul's call sequence, timed rounds only, "
                "the product kernel alone (a split-K sum kernel has no MFMA). "
                "Utilisation = SQ_VALU_MFMA_BUSY_CYCLES (summed over the 1024 SIMDs) / "
                "(1024 x kernel duration x 2.4 GHz); each v_mfma_f32_32x32x2_f32 keeps the "
                "pipe busy 64 cycles, so this equals achieved / peak FLOP rate at 2.4 GHz. "
                "Durations are from this (counter-collecting) run.\n\n")
        o.write("| shape MxKxN | A | product | kernel | grid | n | avg us | MFMA instr | MFMA util | "
                "LDS-wait / wave cycles | LDS bank conflicts |\n"
                "|---|---|---|---|---|---|---|---|---|---|---|\n")
        for (M, Kd, N, lay, prod), ds in per.items():
            avg = lambda k: sum(x.get(k, 0.0) for x in ds) / len(ds)  # noqa: E731
            dur = avg("dur_ns")
            util = avg("SQ_VALU_MFMA_BUSY_CYCLES") / (simds * dur * clock_ghz) if dur else 0.0
            lw = avg("SQ_WAIT_INST_LDS") / max(avg("SQ_WAVE_CYCLES"), 1.0)
            o.write(f"| {M}x{Kd}x{N} | {lay} | {prod} | `{_short(ds[0]['Kernel_Name'])[:60]}` | "
                    f"{ds[0]['grid']} | {len(ds)} | {dur / 1e3:.1f} | {avg('SQ_INSTS_MFMA'):.0f} | "
                    f"{util:.3f} | {lw:.3f} | {avg('SQ_LDS_BANK_CONFLICT'):.0f} |\n")


def _load_pmc(path: str) -> dict:
    """{(kernel, grid): {counter or "dur_ns": per-dispatch average}}."""
    import csv
    acc: dict[tuple, dict] = {}
    for r in csv.DictReader(open(os.path.join(path, "run_counter_collection.csv"))):
        key = (_short(r["Kernel_Name"]), int(r["Grid_Size"]))
        d = acc.setdefault(key, {})
        disp = d.setdefault(r["Dispatch_Id"], {
            "dur_ns": int(r["End_Timestamp"]) - int(r["Start_Timestamp"])})
        disp[r["Counter_Name"]] = float(r["Counter_Value"])
    out = {}
    for key, d in acc.items():
        ds = list(d.values())
        names = set().union(*[x.keys() for x in ds])
        out[key] = {n: sum(x.get(n, 0.0) for x in ds) / len(ds) for n in names}
        out[key]["dispatches"] = len(ds)
    return out


def _summarize_pmc(part: str, dirs: list[str], out_md: str, title: str, keep) -> None:
    """Issue, wait, occupancy and LDS figures per kernel from the two counter
    passes (PMC_SET1, PMC_SET2) of one bench part."""
    cus, simds, clk = 256, 1024, 2.4
    a, b = _load_pmc(dirs[0]), _load_pmc(dirs[1])
    rows = []
    for key in sorted(a):
        name, grid = key
        if not keep(name):
            continue
        x, y = a[key], b.get(key, {})
        cyc = x["dur_ns"] * clk
        wc = max(x.get("SQ_WAVE_CYCLES", 0.0), 1.0)
        rows.append((name, grid, int(x["dispatches"]), x["dur_ns"] / 1e3,
                     wc * 4 / (cus * cyc),                       # resident waves per CU
                     x.get("SQ_WAIT_ANY", 0.0) / wc,              # waiting (s_waitcnt, barrier)
                     x.get("SQ_WAIT_INST_ANY", 0.0) / wc,         # ready, not issued
                     x.get("SQ_WAIT_INST_LDS", 0.0) / wc,
                     y.get("SQ_ACTIVE_INST_VALU", 0.0) * 4 / (simds * cyc) if y else float("nan"),
                     y.get("SQ_INSTS_VALU", 0.0) / max(x.get("SQ_WAVES", 1.0), 1.0) if y else float("nan"),
                     x.get("SQ_LDS_BANK_CONFLICT", 0.0) / (cus * cyc),
                     y.get("SQ_INST_LEVEL_VMEM", 0.0) / max(
                         y.get("SQ_INSTS_VMEM_RD", 0.0) + y.get("SQ_INSTS_VMEM_WR", 0.0), 1.0)
                     if y else float("nan")))
    with open(out_md, "w") as o:
        o.write(f"# {title}\n\nCommands (repo root on the GPU box):\n\n```\n"
                f"{PROFILE_CMDS[part + '_pmc1']}\n{PROFILE_CMDS[part + '_pmc2']}\n```\n\n"
                f"Summarised with `python bench.py --summarize {'mm_pmc12' if part == 'mm' else part + '_pmc'} "
                f"gpurun_out/prof_{part}_pmc1 "
                f"gpurun_out/prof_{part}_pmc2`.  Per dispatch, averaged; durations from the first "
                "(counter-collecting) pass.  SQ cycle counters are summed over the GPU's waves in "
                "units of 4 cycles (so resident waves per CU = 4 x SQ_WAVE_CYCLES / (256 CUs x "
                "cycles), at most 32):\n\n"
                "* waves/CU: average resident waves per CU;\n"
                "* wait: share of wave time in s_waitcnt / barrier waits (SQ_WAIT_ANY / SQ_WAVE_CYCLES);\n"
                "* issue-wait: share of wave time ready but not issued (SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES);\n"
                "* LDS-wait: SQ_WAIT_INST_LDS / SQ_WAVE_CYCLES;\n"
                "* VALU busy: SIMD cycles issuing VALU / (1024 SIMDs x cycles);\n"
                "* VALU/wave: VALU instructions per wave;\n"
                "* bank-conflict: LDS bank-conflict cycles per CU / cycles;\n"
                "* VMEM level/inst: SQ_INST_LEVEL_VMEM / VMEM instructions (a latency proxy, "
                "cycles x 4).\n\n"
                "| kernel | grid | dispatches | us | waves/CU | wait | issue-wait | LDS-wait | "
                "VALU busy | VALU/wave | bank-conflict | VMEM level/inst |\n"
                "|---|---|---|---|---|---|---|---|---|---|---|---|\n")
        for r in rows:
            o.write(f"| `{r[0][:110]}` | {_mdc(r[1])} | {r[2]} | {r[3]:.1f} | {r[4]:.1f} | {r[5]:.2f} | "
                    f"{r[6]:.2f} | {r[7]:.3f} | {r[8]:.2f} | {r[9]:.0f} | {r[10]:.3f} | {r[11]:.0f} |\n")


def _summarize_bytes(part: str, dirs: list[str], out_md: str, title: str, expect) -> None:
    """HBM bytes per dispatch of every kernel of one part from the
    FETCH_SIZE / WRITE_SIZE passes, scaled by the 2^24 copy of --calib."""
    f, w = _load_pmc(dirs[0]), _load_pmc(dirs[1])
    copy = [k for k in f if "CastOp<float, float>" in k[0] and k[1] == N_ELEM // 4]
    fs = 64 * 1024 / f[copy[0]]["FETCH_SIZE"]
    ws = 64 * 1024 / w[copy[0]]["WRITE_SIZE"]
    with open(out_md, "w") as o:
        o.write(f"# {title}\n\nCommands (repo root on the GPU box):\n\n```\n"
                f"{PROFILE_CMDS[part + '_fetch']}\n{PROFILE_CMDS[part + '_write']}\n```\n\n"
                f"Summarised with `python bench.py --summarize {part}_bytes gpurun_out/prof_{part}_fetch "
                f"gpurun_out/prof_{part}_write`.  Calibration: the 2^24-element copy of --calib "
                f"(64 MiB read, 64 MiB written) reads FETCH_SIZE {f[copy[0]]['FETCH_SIZE'] / 1024:.1f} MiB "
                f"and WRITE_SIZE {w[copy[0]]['WRITE_SIZE'] / 1024:.1f} MiB, so FETCH_SIZE is scaled by "
                f"{fs:.3f} and WRITE_SIZE by {ws:.3f}; `expected` is the algorithmic count "
                "(each operand read once, each output written once) where the kernel's role is "
                "known.\n\n"
                "| kernel | grid | dispatches | read MiB | written MiB | expected read / written MiB |\n"
                "|---|---|---|---|---|---|\n")
        for key in sorted(f):
            if key in copy or key[0].startswith("_rocclr") or key[0].startswith("__amd"):
                continue
            rd = f[key]["FETCH_SIZE"] * fs / 1024
            wr_ = w.get(key, {}).get("WRITE_SIZE", 0.0) * ws / 1024
            if rd + wr_ < 1.0:
                continue
            o.write(f"| `{key[0][:110]}` | {_mdc(key[1])} | {int(f[key]['dispatches'])} | {rd:.1f} | "
                    f"{wr_:.1f} | {expect(key[0], key[1]) or ''} |\n")


def _red_expect(name: str, grid: int) -> str:
    if name.startswith(("reduce_row_kernel", "reduce_col_kernel")):
        return "256 / partials"
    if name.startswith(("sel_bwd", "ew_rows_kernel<float, float, 1", "ew_flat_kernel<float, float, 1")):
        return "0 (g, index, count: 0.1) / 256"
    if name.startswith(("ew_rows_kernel<float, float, 2", "ew_flat_kernel<float, float, 2")):
        return "256 / 256"
    return ""


def _summarize_tile_variants(base: str, out_md: str) -> None:
    """Counter rows of every transposed sweep kernel under each tile variant
    (TILE_VARIANTS), from the two counter passes per variant under `base`
    (gpurun_out): which shape and orientation each kernel ran, its duration
    and what its waves did."""
    import re
    cus, simds, clk = 256, 1024, 2.4
    rows = []
    for lbl in TILE_VARIANTS:
        d1, d2 = (os.path.join(base, f"prof_tile_{lbl}_{i}") for i in (1, 2))
        if not (os.path.isdir(d1) and os.path.isdir(d2)):
            continue
        a, b = _load_pmc(d1), _load_pmc(d2)
        for (name, grid), x in a.items():
            key = _sweep_key(name)
            if not key or "|transposed|" not in key:
                continue
            y = b.get((name, grid), {})
            m = re.search(r"true, (\d+), (\d+),", name)
            cyc = x["dur_ns"] * clk
            wc = max(x.get("SQ_WAVE_CYCLES", 0.0), 1.0)
            rows.append((key, lbl, f"{m.group(1)}x{m.group(2)}" if m else "?", x["dur_ns"] / 1e3,
                         wc * 4 / (cus * cyc), x.get("SQ_WAIT_ANY", 0.0) / wc,
                         x.get("SQ_WAIT_INST_ANY", 0.0) / wc,
                         y.get("SQ_ACTIVE_INST_VALU", 0.0) * 4 / (simds * cyc) if y else float("nan"),
                         x.get("SQ_LDS_BANK_CONFLICT", 0.0) / (cus * cyc)))
    nb = {k: ew_bytes(k.split("|")[0], k.split("|")[2]) for k, *_ in rows}
    with open(out_md, "w") as o:
        o.write("# Transposed elementwise kernels under each tile variant (config-2 sweep)\n\n"
                "Commands (repo root on the GPU box), two counter passes per variant:\n\n```\n")
        for lbl in TILE_VARIANTS:
            o.write(PROFILE_CMDS[f"tile_{lbl}_pmc1"] + "\n" + PROFILE_CMDS[f"tile_{lbl}_pmc2"] + "\n")
        o.write("```\n\nSummarised with `python bench.py --summarize tile_variants gpurun_out`.  "
                "`rule` is the library's choice; the other variants force one compiled fp32 tile "
                "shape (the orientation still by the cost rule) or one orientation (the shape still "
                "by the rule) for every transposed kernel of the sweep (NT_TILE_SHAPE / "
                "NT_TILE_ORIENT; results are identical).  Durations are from the counter-collecting "
                "pass (kernels serialised); frac = algorithmic bytes / duration / 8 TB/s.  Columns as "
                "in elementwise_sweep_config2_counters.md: waves/CU resident, wait = s_waitcnt / "
                "barrier share of wave time, issue-wait = ready but not issued, VALU busy = SIMD "
                "cycles issuing VALU, bank-conflict = LDS bank-conflict cycles per CU / cycles.\n\n"
                "| kernel | variant | tile | us | frac | waves/CU | wait | issue-wait | VALU busy | "
                "bank-conflict |\n|---|---|---|---|---|---|---|---|---|---|\n")
        for key, lbl, tile, us, wv, w, iw, vb, bc in sorted(rows, key=lambda r: (r[0], r[3])):
            o.write(f"| {_mdc(key)} | {lbl} | {tile} | {us:.1f} | {nb[key] / (us * 1e-6) / 8e12:.3f} | "
                    f"{wv:.1f} | {w:.2f} | {iw:.2f} | {vb:.2f} | {bc:.3f} |\n")


def summarize(kind: str, dirs: list[str]) -> None:
    import csv
    prof = os.path.join(ROOT, "profiles")
    if kind == "tile_variants":
        _summarize_tile_variants(dirs[0], os.path.join(prof, "elementwise_transposed_tile_variants.md"))
        return
    if kind == "ew_pmc":
        _summarize_pmc("ew", dirs, os.path.join(prof, "elementwise_sweep_config2_counters.md"),
                       "Issue and wait counters: config-2 elementwise sweep kernels",
                       lambda n: n.startswith(("ew_flat_kernel", "ew_tile4_kernel")))
        return
    if kind == "red_pmc":
        _summarize_pmc("red", dirs, os.path.join(prof, "reduce_config3_counters.md"),
                       "Issue and wait counters: config-3 reduction kernels",
                       lambda n: not n.startswith(("_rocclr", "__amd")))
        return
    if kind == "mm_pmc12":
        _summarize_pmc("mm", dirs, os.path.join(prof, "matmul_config4_counters.md"),
                       "Issue and wait counters: config-4 matmul kernels",
                       lambda n: n.startswith("mm_"))
        return
    if kind == "red_bytes":
        _summarize_bytes("red", dirs, os.path.join(prof, "reduce_config3_hbm_traffic.md"),
                         "HBM traffic per launch: config-3 reductions", _red_expect)
        return
    if kind == "mlp_bytes":
        _summarize_bytes("mlp", dirs, os.path.join(prof, "mlp_config5_hbm_traffic.md"),
                         "HBM traffic per launch: config-5 MLP step kernels", lambda n, g: "")
        return
    if kind == "sweep":
        _summarize_sweep_trace(dirs[0], os.path.join(prof, PROFILE_FILES["sweep"][0]))
        return
    if kind == "mm":
        _summarize_mm_trace(dirs[0], os.path.join(prof, PROFILE_FILES["mm"][0]))
        return
    if kind == "next":
        _summarize_next_trace(dirs[0], os.path.join(prof, PROFILE_FILES["next"][0]))
        return
    if kind in PROFILE_FILES:
        fname, title = PROFILE_FILES[kind]
        rows = list(csv.DictReader(open(os.path.join(dirs[0], "run_kernel_stats.csv"))))
        o = [f"# {title}\n", "Command (repo root on the GPU box):\n",
             f"```\n{PROFILE_CMDS[kind]}\n```\n",
             f"Summarised with `python bench.py --summarize {kind} gpurun_out/prof_{kind}`.",
             "Durations are rocprofv3 kernel times in microseconds; a sweep row's",
             "`sweep key` names the bench.py entry it belongs to.\n",
             "| kernel | sweep key | calls | avg us | min us | max us | total % |",
             "|---|---|---|---|---|---|---|"]
        for r in rows:
            o.append(f"| `{_short(r['Name'])[:150]}` | {_mdc(_sweep_key(r['Name']) or '')} | {r['Calls']} | "
                     f"{float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
                     f"{float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.2f} |")
        with open(os.path.join(prof, fname), "w") as f:
            f.write("\n".join(o) + "\n")
        return
    if kind == "mm_pmc":
        _summarize_mm_pmc(dirs[0], os.path.join(prof, "matmul_config4_mfma_utilisation.md"))
        return
    if kind != "traffic":
        raise SystemExit(f"unknown profile kind {kind}")

    def load(path, counter):
        # per-kernel average, plus the copy kernel's readings by grid size:
        # the same copy kernel also runs at 2^26 elements (the cold-copy
        # reference), and only the 2^24 --calib copies calibrate
        d: dict[str, list[float]] = {}
        copies: dict[int, list[float]] = {}
        for r in csv.DictReader(open(os.path.join(path, "run_counter_collection.csv"))):
            if r.get("Counter_Name") == counter:
                d.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
                if "CastOp<float, float>" in r["Kernel_Name"]:
                    copies.setdefault(int(r["Grid_Size"]), []).append(float(r["Counter_Value"]))
        calib = copies[min(copies)]  # the smallest copies: 2^24 fp32
        return {k: sum(v) / len(v) for k, v in d.items()}, sum(calib) / len(calib)

    (fch, fcopy), (wr, wcopy) = load(dirs[0], "FETCH_SIZE"), load(dirs[1], "WRITE_SIZE")
    fs = 64 * 1024 / fcopy  # counters are KiB; the copy reads 64 MiB
    ws = 64 * 1024 / wcopy  # and writes 64 MiB
    per, rows = {}, []
    for k in fch:
        kk = _sweep_key(k)
        if kk is None:
            continue
        b = fch[k] * fs * 1024 + wr.get(k, 0) * ws * 1024
        per[kk] = int(round(b))
        rows.append((kk, fch[k] / 1024, wr.get(k, 0) / 1024, b / 2**20, ew_bytes(*kk.split("|")[::2]) / 2**20))
    with open(os.path.join(prof, "traffic.json"), "w") as f:
        json.dump({"source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE on bench.py --calib, "
                             "scaled by a plain copy's reading",
                   "commands": [PROFILE_CMDS["fetch"], PROFILE_CMDS["write"]],
                   "fetch_scale": fs, "write_scale": ws, "per_launch_bytes": per}, f, indent=1)
    with open(os.path.join(prof, "elementwise_sweep_config2_hbm_traffic.md"), "w") as o:
        o.write("# HBM traffic per launch: config-2 sweep kernels\n\n")
        o.write(f"Commands (repo root on the GPU box):\n\n```\n{PROFILE_CMDS['fetch']}\n"
                f"{PROFILE_CMDS['write']}\n```\n\n")
        o.write("Summarised with `python bench.py --summarize traffic gpurun_out/prof_fetch "
                "gpurun_out/prof_write` (also writes traffic.json, read by the roofline).\n\n")
        o.write(f"Calibration: a plain copy of 2^24 fp32 (64 MiB read, 64 MiB written) reads "
                f"FETCH_SIZE {fcopy / 1024:.1f} MiB and WRITE_SIZE {wcopy / 1024:.1f} MiB per "
                f"dispatch, so FETCH_SIZE is scaled by {fs:.3f} and WRITE_SIZE by {ws:.3f}.\n\n")
        o.write("| kernel | FETCH_SIZE MiB | WRITE_SIZE MiB | scaled traffic MiB | algorithmic MiB |\n"
                "|---|---|---|---|---|\n")
        for kk, fv, wv, t, alg in sorted(rows):
            o.write(f"| {_mdc(kk)} | {fv:.1f} | {wv:.1f} | {t:.1f} | {alg:.1f} |\n")


# -------------------------------------------------------------------- main


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--parts", default="all",
                    help="all | none (the headline sweep only) | comma list of "
                         "ew,first,red,mm,mlp,next,cpu (first: the sweep's backwards in "
                         "first-write mode)")
    ap.add_argument("--mlp-steps", type=int, default=20)
    ap.add_argument("--calib", action="store_true",
                    help="first run 3 plain copies of 2^24 fp32 (64 MiB read + 64 MiB "
                         "written each): the reference dispatch for HBM byte counters")
    ap.add_argument("--summarize", nargs="+", metavar=("KIND", "DIR"),
                    help="write a profiles/ summary from rocprofv3 csv output: "
                         "sweep|red|mm|mlp|next|mm_pmc DIR, traffic|red_bytes|mlp_bytes "
                         "FETCH_DIR WRITE_DIR, or ew_pmc|red_pmc PMC1_DIR PMC2_DIR")
    args = ap.parse_args()
    if args.summarize:
        summarize(args.summarize[0], args.summarize[1:])
        return 0
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for {max(args.gpus, world)}); "
              "this build has no multi-GPU path.", file=sys.stderr)
        return 2
    if not nt.is_available():
        print("no HIP device / libnt.so", file=sys.stderr)
        return 1
    parts = {"ew", "first", "red", "mm", "mlp", "next", "cpu"} if args.parts == "all" else (
        {"ew"} if args.parts == "none" else set(args.parts.split(",")))

    if args.calib:
        src = _fresh((N_ELEM,))
        dst = _fresh((N_ELEM,))
        for _ in range(3):
            K.copy_view(src, dst)
        nt.sync()

    if "ew" not in parts:
        # profiling runs of one part: print that part's results only
        line = {"parts": {}}
        if "red" in parts:
            line["parts"]["reductions"] = bench_reductions()
        if "mm" in parts:
            line["parts"]["matmul"] = bench_matmul()
        if "mlp" in parts:
            line["parts"]["mlp"] = bench_mlp(args.mlp_steps)
        if "next" in parts:
            line["parts"]["next_rows"] = bench_next()
        print(json.dumps(line), flush=True)
        return 0

    ew = bench_elementwise(args.steps, args.warmup, first_write="first" in parts)
    value = ew["step_bytes"] / (ew["ms_per_step"] * 1e-3) / 1e9
    # dominant kernel: the one with the largest share of the sweep's time
    dom_key, dom = max(ew["per_kernel"].items(), key=lambda kv: kv[1]["ms"])
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        # HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE
        # (scaled by a plain copy's reading); see profiles/traffic.json.
        with open(tpath) as f:
            traffic = json.load(f).get("per_launch_bytes", {}).get(dom_key)
    line = {
        "metric": "elementwise fwd+bwd HBM GB/s (config-2 sweep)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ew["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) / U[a,b] per config 2)",
        "config": {"workload": "config 2: 12 elementwise ops fwd + fused bwd (accumulate), "
                               "2^24 fp32 elements [4096,4096], contiguous and .T views",
                   "elements": N_ELEM, "kernels_per_step": len(ew["per_kernel"])},
        "baseline_metric": BASELINE_METRIC,
        "roofline": {"bound": "hbm", "kernel": dom_key, "achieved": dom["GB/s"],
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": dom["frac"],
                     "traffic": traffic, "bytes_per_launch": dom["bytes"]},
        "sweep_frac_of_peak": round(value / HBM_PEAK_GBS, 4),
        # kernels of a step queued without / with the stream barrier (the
        # launch window), and the per-kernel pass's sum of kernel times
        "launches_per_step": ew["launches_per_step"],
        "sum_of_kernel_ms": ew["sum_of_kernel_ms"],
        "parts": {"elementwise_per_kernel": ew["per_kernel"]},
    }
    if ew["first_write"]:
        fw = ew["first_write"]
        fb = sum(v["bytes"] for v in fw.values())
        fms = sum(v["ms"] for v in fw.values())
        line["parts"]["elementwise_first_write"] = {
            "per_kernel": fw,
            "aggregate_GB/s": round(fb / (fms * 1e-3) / 1e9, 1),
            "aggregate_frac": round(fb / (fms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    copy_ref = bench_copy_reference()
    copy_ref["sweep_vs_copy"] = round(value / copy_ref["GB/s"], 4)
    line["parts"]["copy_reference"] = copy_ref
    # the sweep's unary forwards against a copy of their own size and layout
    small = bench_copy_sweep_size()
    for lay, key in (("contig", "contiguous"), ("transposed", "transposed")):
        ks = [k for k in ew["per_kernel"] if k.endswith(f"|{lay}|fwd")
              and k.split("|")[0] not in ("add", "sub", "mul", "truediv")]
        mean = sum(ew["per_kernel"][k]["GB/s"] for k in ks) / len(ks)
        small[key]["unary_fwd_vs_copy"] = round(mean / small[key]["GB/s"], 4)
    line["parts"]["copy_reference_sweep_size"] = small
    if "red" in parts:
        line["parts"]["reductions"] = bench_reductions()
    if "mm" in parts:
        line["parts"]["matmul"] = bench_matmul()
    if "mlp" in parts:
        line["parts"]["mlp"] = bench_mlp(args.mlp_steps)
    if "next" in parts:
        line["parts"]["next_rows"] = bench_next()
    if "cpu" in parts:
        cpu = cpu_per_op()
        line["cpu_baseline"] = cpu["baseline"]
        attach_cpu(line["parts"], cpu["per_op"])
        line["parts"]["cpu_reference"] = cpu_parts()
        line["parts"]["cpu_reference"]["per_op_samples"] = {
            k: cpu["per_op"][k] for k in ("elementwise_sample", "reductions_sample", "matmul_sample",
                                          "threads", "host_cpu", "host_nproc")}
        line["parts"]["cpu_reference"]["mlp_config5"] = cpu["per_op"]["mlp"]
    else:
        line["cpu_baseline"] = None
    line["host"] = platform.node()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
