"""Elementwise kernels queued without the stream barrier (hipExtAnyOrderLaunch,
nanotorch_amd/csrc/launch_window.h): independent kernels may overlap, and
every kernel that shares bytes with one still in flight must wait for it.

Each test runs its sequence on 2^22-2^24-element tensors (long enough that
an unordered read-after-write, write-after-read or write-after-write would
corrupt many elements) and checks every result bit for bit against numpy,
and checks nt_launch_stats: independent sequences must have gone without the
barrier, dependent ones must not."""

from __future__ import annotations

import ctypes
import gc

import numpy as np
import pytest

from helpers import assert_bitexact, dev, host, rng, seed_of

import nanotorch_amd as nt
from nanotorch_amd import _kernels as K
from nanotorch_amd import _lib

pytestmark = pytest.mark.gpu

N = 1 << 22


def _stats():
    u, o, f = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    _lib.call("nt_launch_stats", ctypes.byref(u), ctypes.byref(o), ctypes.byref(f))
    return np.array([u.value, o.value, f.value], dtype=np.int64)


def _f32(r, n=N, lo=None, hi=None):
    if lo is None:
        return r.standard_normal(n).astype(np.float32)
    return r.uniform(lo, hi, n).astype(np.float32)


def test_independent_ops_overlap_and_match(gpu):
    r = rng(seed_of("overlap-indep"))
    a = [_f32(r) for _ in range(8)]
    b = [_f32(r, lo=0.5, hi=2) for _ in range(8)]
    ta, tb = [dev(x) for x in a], [dev(x) for x in b]
    nt.sync()  # closes the window: the first op below takes the barrier
    s0 = _stats()
    outs = [ta[0] + tb[0], ta[1] - tb[1], ta[2] * tb[2], ta[3] / tb[3],
            ta[4].exp(), nt.sqrt(tb[5]), nt.tanh(ta[6]), ta[7] * tb[7]]
    d = _stats() - s0
    want = [a[0] + b[0], a[1] - b[1], a[2] * b[2], a[3] / b[3], None, np.sqrt(b[5]), None,
            a[7] * b[7]]
    for i, (o, w) in enumerate(zip(outs, want)):
        if w is not None:
            assert_bitexact(host(o), w, f"op {i}")
    # exp / tanh: against the same kernels run one at a time
    nt.sync()
    assert_bitexact(host(outs[4]), host(ta[4].exp()), "exp")
    assert_bitexact(host(outs[6]), host(nt.tanh(ta[6])), "tanh")
    # 8 kernels, window of 6: the 1st and 7th take the barrier
    assert d[0] >= 5 and d[0] + d[1] == 8, d


def test_dependent_chain_keeps_order(gpu):
    r = rng(seed_of("overlap-chain"))
    n = 1 << 24
    a, b, c = _f32(r, n), _f32(r, n), _f32(r, n, 0.5, 2)
    ta, tb, tc = dev(a), dev(b), dev(c)
    nt.sync()
    s0 = _stats()
    y = ta + tb            # y = a + b
    z = y * tc             # reads y
    w = z - y              # reads z and y
    ta += w                # writes a, which the first kernel read
    v = ta / tc            # reads the new a
    d = _stats() - s0
    y_ = a + b
    z_ = y_ * c
    w_ = z_ - y_
    a_ = a + w_
    assert_bitexact(host(y), y_, "y")
    assert_bitexact(host(z), z_, "z")
    assert_bitexact(host(w), w_, "w")
    assert_bitexact(host(ta), a_, "a")
    assert_bitexact(host(v), a_ / c, "v")
    assert d[0] == 0, d  # every kernel depends on the one before


def test_write_after_read_and_write_after_write(gpu):
    r = rng(seed_of("overlap-war"))
    n = 1 << 24
    x, g, c, a, b = (_f32(r, n) for _ in range(5))
    tx, tg, tc, ta, tb = dev(x), dev(g), dev(c), dev(a), dev(b)
    unrelated = [dev(_f32(r)) for _ in range(2)]
    nt.sync()
    s0 = _stats()
    y = tx * tg            # reads x
    u = unrelated[0] + unrelated[1]   # independent: may overlap
    tx += tc               # writes x: must wait for the read above
    z = ta + tb            # writes z
    K.copy_view(tc, z)     # writes z again: must wait for the write above
    d = _stats() - s0
    assert_bitexact(host(y), x * g, "y read the old x")
    assert_bitexact(host(tx), x + c, "x += c")
    assert_bitexact(host(z), c, "z overwritten last")
    assert_bitexact(host(u), host(unrelated[0]) + host(unrelated[1]), "unrelated")
    assert d[0] >= 1, d


def test_transposed_and_overlapping_views(gpu):
    """Strided operands: the hazard check uses each view's byte span, so a
    write to a slice of a tensor that a `.T` view is still being read from
    must wait."""
    r = rng(seed_of("overlap-views"))
    m = np.ascontiguousarray(r.standard_normal((2048, 2048)).astype(np.float32))
    other = r.standard_normal((2048, 2048)).astype(np.float32)
    tm = dev(m)
    to = dev(other)
    nt.sync()
    y = tm.T + to              # tile kernel reading m through a .T view
    row = tm[100:200]          # a slice of the same storage
    row *= 3.0                 # writes bytes the kernel above reads
    want_m = m.copy()
    want_m[100:200] *= np.float32(3.0)
    assert_bitexact(host(y), m.T + other, "y")
    assert_bitexact(host(tm), want_m, "m")


def test_fences_order_other_stream_work(gpu):
    """After kernels that went without the barrier, a reduction, a
    device-to-host copy and an event all see their results complete."""
    r = rng(seed_of("overlap-fence"))
    a = [_f32(r) for _ in range(4)]
    ta = [dev(x) for x in a]
    ta[0] * 3.0  # the device scalar 3.0, built and cached before the timed part
    nt.sync()
    s0 = _stats()
    outs = [t * 3.0 for t in ta]     # independent: the 2nd-4th may skip the barrier
    total = outs[3].sum()            # a reduction of the last one
    back = host(outs[2])             # device-to-host copy
    d = _stats() - s0
    assert d[0] >= 2 and d[2] >= 1, d
    assert_bitexact(back, a[2] * np.float32(3.0), "copy")
    ref = float(np.sum((a[3] * np.float32(3.0)).astype(np.float64)))
    assert abs(float(host(total)) - ref) <= 1e-5 * float(np.sum(np.abs(a[3] * np.float32(3.0))))
    for o, x in zip(outs, a):
        assert_bitexact(host(o), x * np.float32(3.0), "outs")
    e0, e1 = _lib.Event(), _lib.Event()
    e0.record()
    more = [t + o for t, o in zip(ta, outs)]
    e1.record()
    assert e0.elapsed_ms(e1) > 0.0
    for m, x in zip(more, a):
        assert_bitexact(host(m), x + x * np.float32(3.0), "after the event")


def test_reused_allocations_wait_for_their_readers(gpu):
    """A tensor freed while a kernel that reads it may still run, its block
    handed straight to the next allocation: the new owner's first write must
    wait for that reader (the byte spans overlap), though nothing else ties
    the two kernels together."""
    r = rng(seed_of("overlap-reuse"))
    x0 = _f32(r)
    others = [_f32(r) for _ in range(12)]
    t_others = [dev(o) for o in others]
    t_others[0] + 1.0
    t_others[0] * 2.0  # the device scalars, built and cached first
    cur_t, cur = dev(x0), x0
    gc.collect()
    _lib.call("nt_empty_cache")  # the loop's freed block is then the only cached one
    nt.sync()
    results, reused = [], 0
    for i in range(12):
        y = cur_t * 2.0                    # reads cur
        old = cur_t._storage.data_ptr()
        del cur_t
        gc.collect()                       # cur's block goes back to the cache
        w = t_others[i] + 1.0              # allocates and writes a block
        reused += int(w._storage.data_ptr() == old)
        results.append((y, cur))
        cur_t, cur = w, others[i] + np.float32(1.0)
        del w  # cur_t is then the block's only owner
    for i, (y, prev) in enumerate(results):
        assert_bitexact(host(y), prev * np.float32(2.0), f"step {i}")
    assert_bitexact(host(cur_t), cur, "final")
    assert reused >= 6, reused  # the hazard this test is about did occur


@pytest.mark.parametrize("seed", range(4))
def test_random_op_streams_match_host(gpu, seed):
    """A random stream of elementwise ops over a pool of six 2^22-element
    tensors (each op reads one or two pool tensors, possibly its own
    destination, possibly through a `.T` view, and writes one), with a
    reduction or a device-to-host copy every few ops: every read-after-
    write, write-after-read and write-after-write between nearby ops is
    a hazard the launch window must order.  The same stream runs on the
    host in float32 (add, sub, neg, exact scalings and copies: every
    result exact), and every tensor must match bit for bit at each
    check and at the end."""
    r = rng(seed_of("overlap-random", seed))
    side = 2048
    pool_h = [r.integers(-8, 9, (side, side)).astype(np.float32) for _ in range(6)]
    pool_d = [dev(a) for a in pool_h]
    half, two = np.float32(0.5), np.float32(2.0)
    pool_d[0] * 0.5
    pool_d[0] * 2.0  # the device scalars, built and cached first
    nt.sync()
    s0 = _stats()
    for step in range(160):
        kind = int(r.integers(0, 10))
        dst, a, b = (int(v) for v in r.integers(0, 6, 3))
        tr_a = bool(r.integers(0, 4) == 0)  # read a through a .T view
        A_h = pool_h[a].T if tr_a else pool_h[a]
        A_d = pool_d[a].T if tr_a else pool_d[a]
        if kind == 9 and step % 3 == 0:
            # other stream work: a device-to-host copy or a reduction
            if r.integers(0, 2):
                assert_bitexact(host(pool_d[a]), pool_h[a], f"copy at step {step}")
            else:
                got = float(host(pool_d[a].sum()))
                want = float(np.sum(pool_h[a].astype(np.float64)))
                assert abs(got - want) <= 1e-5 * float(np.sum(np.abs(pool_h[a]))) + 1e-30
            continue
        if kind < 3:
            res_h = A_h + pool_h[b]
            K.copy_view(A_d + pool_d[b], pool_d[dst])
        elif kind < 5:
            res_h = A_h - pool_h[b]
            K.copy_view(A_d - pool_d[b], pool_d[dst])
        elif kind < 6:
            res_h = -A_h
            K.copy_view(-A_d, pool_d[dst])
        elif kind < 8:
            big = float(np.abs(A_h).max()) > 2.0**20
            res_h = A_h * (half if big else two)
            K.copy_view(A_d * (0.5 if big else 2.0), pool_d[dst])
        else:
            res_h = A_h.copy()
            K.copy_view(A_d, pool_d[dst])  # possibly a transposing copy onto itself's source
        pool_h[dst] = np.ascontiguousarray(res_h)
        if dst == a and tr_a:
            # an in-place transposing copy reads what it overwrites: keep the
            # pool well-defined by restoring the destination from the host
            pool_d[dst] = dev(pool_h[dst])
    d = _stats() - s0
    for i, (h_, d_) in enumerate(zip(pool_h, pool_d)):
        assert_bitexact(host(d_), h_, f"pool tensor {i}")
    assert d[0] >= 20, d  # the stream did overlap independent kernels
