"""The no-allocation dispatch (thvm_hip_dispatch_uop_kernel_noalloc) against
the allocating one, on the GPU, through the C ABI.

Programs that the allocating path ran only fused into another launch (an
elementwise consumer in a contraction's epilogue, a merged chain) are still
accepted: a training step of LeNet-5 at batch 256 and of the 2-layer MLP is
first replayed with no read between its dispatches (the bench's mode: held,
batched, fused), then every program of the step goes through the
no-allocation entry point first, and must match the allocating one.

Every lowered program of two traces, one after the other: the conv block at
its benchmark size [64,64,56,56] (matrix-core convolutions with packed
operands and a 128-way split-K weight gradient, split batchnorm reductions,
elementwise kernels), then the same block at [2,4,8,8], whose workspaces are
smaller. Each program runs first through thvm_hip_dispatch_uop_kernel (which
compiles it), then, from the same inputs, through the no-allocation entry
point with its output filled with a NaN sentinel: the two outputs must be
identical bit for bit (the same kernels in the same order; only the
workspace addresses differ), no hipMalloc may happen during the second call
and nothing may be compiled. Also: a program never compiled is refused with
THVM_HIP_ENOTREADY and leaves its output untouched; a split-K GEMM whose
partial sums exceed the static workspace (4096^3 with a forced 2-way split,
128 MiB) is refused with THVM_HIP_ESCRATCH.
"""
import ctypes as C
import os

import numpy as np
import pytest

from tests import tracetools as tt
from tests.test_gpu_parity import _reads_own_output
from tinyhvm_amd import _lib, trace

pytestmark = pytest.mark.gpu

WL = os.path.join(tt.ROOT, "tinyhvm_amd", "workloads")
SENTINEL = 0xFFFFFFFF
KNOBS = ("THVM_HIP_DENSE_FORCE", "THVM_HIP_DENSE_SPLITS")
OK, ENOTREADY, ESCRATCH = 0, -2, -3


def _fresh(env):
    L = _lib.lib()
    L.thvm_hip_shutdown()
    saved = {k: os.environ.pop(k, None) for k in KNOBS}
    os.environ.update(env)
    assert L.thvm_hip_init() == 0, "HIP backend failed to initialise"
    return L, saved


def _restore(L, saved):
    L.thvm_hip_shutdown()
    for k in KNOBS:
        os.environ.pop(k, None)
        if saved[k] is not None:
            os.environ[k] = saved[k]


def _counters(L):
    c = (C.c_uint64 * 10)()
    L.thvm_hip_counters(c, 10)
    return list(c)


def _read(L, live, n):
    buf = np.zeros((n + 3) // 4, dtype=np.uint32)
    L.thvm_hip_buf_read(live, buf.ctypes.data_as(C.c_void_p), n)
    return buf


def _compare_trace(L, path):
    """Replays `path`; every UOP record runs through both entry points."""
    recs = trace.read_trace(path)
    sizes = {}
    rp = tt.Replay(path, L.thvm_hip_backend())
    checked = 0
    try:
        for i, r in enumerate(recs):
            if r.tag == trace.ALLOC:
                sizes[r.f["id"]] = r.f["bytes"]
            if r.tag != trace.UOP:
                rp.run(i, i + 1)
                continue
            k = rp.kernel(i)
            out = rp.live(r.f["out"])
            n_out = sizes[r.f["out"]]
            leaves = (C.c_uint32 * max(len(r.f["leaf_bufs"]), 1))(*[rp.live(t) for t in r.f["leaf_bufs"]])
            nl = len(r.f["leaf_bufs"])
            before = _read(L, out, n_out)
            L.thvm_hip_dispatch_uop_kernel(out, leaves, nl, C.byref(k), 0)
            want = _read(L, out, n_out)
            own = _reads_own_output(k, r.f["out"], r.f["leaf_bufs"])
            fill = before if own else np.full_like(before, SENTINEL)
            L.thvm_hip_buf_write(out, fill.ctypes.data_as(C.c_void_p), n_out)
            assert L.thvm_hip_synchronize() == 0
            c0 = _counters(L)
            rc = L.thvm_hip_dispatch_uop_kernel_noalloc(out, leaves, nl, C.byref(k))
            c1 = _counters(L)
            assert rc == OK, "dispatch %d of %s: no-allocation entry returned %d" % (i, path, rc)
            assert c1[7] == c0[7], "dispatch %d: hipMalloc during the no-allocation call" % i
            assert c1[2] == c0[2], "dispatch %d: a program was compiled" % i
            got = _read(L, out, n_out)
            assert np.array_equal(got, want), "dispatch %d of %s: %d words differ" % (
                i, path.split("/")[-1], int(np.sum(got != want)))
            checked += 1
        assert L.thvm_hip_synchronize() == 0
    finally:
        rp.close()
    return checked


def test_noalloc_matches_allocating_dispatch():
    L, saved = _fresh({})
    try:
        big = _compare_trace(L, os.path.join(WL, "convblock_b64.trc"))
        small = _compare_trace(L, tt.fixtures("convblock_2x4x8.trc")[0])
        assert big >= 28 and small >= 28
        # the workspace users were exercised: matrix-core (split-K, packed) and split reductions
        assert _counters(L)[1] > 0
    finally:
        _restore(L, saved)


def test_noalloc_refuses_uncompiled_and_oversized_work():
    L, saved = _fresh({})
    try:
        path = tt.fixtures("fused_5x7.trc")[0]
        recs = trace.read_trace(path)
        rp = tt.Replay(path, L.thvm_hip_backend())
        try:
            i = next(j for j, r in enumerate(recs) if r.tag == trace.UOP)
            rp.run(0, i)
            r = recs[i]
            out = rp.live(r.f["out"])
            n_out = {q.f["id"]: q.f["bytes"] for q in recs if q.tag == trace.ALLOC}[r.f["out"]]
            fill = np.full((n_out + 3) // 4, SENTINEL, dtype=np.uint32)
            L.thvm_hip_buf_write(out, fill.ctypes.data_as(C.c_void_p), n_out)
            leaves = (C.c_uint32 * len(r.f["leaf_bufs"]))(*[rp.live(t) for t in r.f["leaf_bufs"]])
            k = rp.kernel(i)
            rc = L.thvm_hip_dispatch_uop_kernel_noalloc(out, leaves, len(r.f["leaf_bufs"]), C.byref(k))
            assert rc == ENOTREADY, rc
            assert np.array_equal(_read(L, out, n_out), fill), "a refused call wrote its output"
            assert L.thvm_hip_dispatch_uop_kernel_noalloc(0, leaves, 1, C.byref(k)) == -1
        finally:
            rp.close()
    finally:
        _restore(L, saved)

    L, saved = _fresh({"THVM_HIP_DENSE_SPLITS": "2"})
    try:
        path = os.path.join(WL, "linear_4096.trc")
        recs = trace.read_trace(path)
        rp = tt.Replay(path, L.thvm_hip_backend())
        try:
            i = next(j for j, r in enumerate(recs) if r.tag == trace.UOP)
            rp.run(0, i)
            r = recs[i]
            k = rp.kernel(i)
            a = _lib.dense_analyze(k)
            assert a and a[3] == 2 and 2 * a[0] * a[1] * 4 > (32 << 20), a
            out = rp.live(r.f["out"])
            leaves = (C.c_uint32 * len(r.f["leaf_bufs"]))(*[rp.live(t) for t in r.f["leaf_bufs"]])
            L.thvm_hip_dispatch_uop_kernel(out, leaves, len(r.f["leaf_bufs"]), C.byref(k), 0)
            c0 = _counters(L)
            rc = L.thvm_hip_dispatch_uop_kernel_noalloc(out, leaves, len(r.f["leaf_bufs"]), C.byref(k))
            assert rc == ESCRATCH, rc
            assert _counters(L)[7] == c0[7]
            assert L.thvm_hip_synchronize() == 0
        finally:
            rp.close()
    finally:
        _restore(L, saved)


def _fused_then_noalloc(L, path, m0, m1):
    """Replays [m0, m1) of `path` once with no reads (programs fuse), then
    again record by record, each UOP through the no-allocation entry point
    first and then, from the same inputs, through the allocating one."""
    recs = trace.read_trace(path)
    sizes = {r.f["id"]: r.f["bytes"] for r in recs if r.tag == trace.ALLOC}
    rp = tt.Replay(path, L.thvm_hip_backend())
    checked = 0
    try:
        lo = next(i for i, r in enumerate(recs) if r.tag == trace.MARK and r.f["text"] == m0)
        hi = next(i for i, r in enumerate(recs) if i > lo and r.tag == trace.MARK and r.f["text"] == m1) \
            if m1 else len(recs)
        rp.run(0, lo)
        c0 = (C.c_uint64 * 13)()
        L.thvm_hip_counters(c0, 13)
        rp.run(lo, hi, 1)                               # no reads: the held launches fuse
        assert L.thvm_hip_synchronize() == 0
        c1 = (C.c_uint64 * 13)()
        L.thvm_hip_counters(c1, 13)
        assert c1[12] > c0[12], "nothing fused in %s" % path
        for i in range(lo, hi):
            r = recs[i]
            if r.tag != trace.UOP:
                rp.run(i, i + 1, 1)
                continue
            k = rp.kernel(i)
            out = rp.live(r.f["out"])
            n_out = sizes[r.f["out"]]
            nl = len(r.f["leaf_bufs"])
            leaves = (C.c_uint32 * max(nl, 1))(*[rp.live(t) for t in r.f["leaf_bufs"]])
            before = _read(L, out, n_out)
            own = _reads_own_output(k, r.f["out"], r.f["leaf_bufs"])
            fill = before if own else np.full_like(before, SENTINEL)
            L.thvm_hip_buf_write(out, fill.ctypes.data_as(C.c_void_p), n_out)
            m0_ = _counters(L)
            rc = L.thvm_hip_dispatch_uop_kernel_noalloc(out, leaves, nl, C.byref(k))
            assert rc == OK, "dispatch %d of %s (run fused before): no-allocation entry returned %d" % (
                i, path.split("/")[-1], rc)
            assert _counters(L)[7] == m0_[7] and _counters(L)[2] == m0_[2]
            got = _read(L, out, n_out)
            L.thvm_hip_buf_write(out, before.ctypes.data_as(C.c_void_p), n_out)
            L.thvm_hip_dispatch_uop_kernel(out, leaves, nl, C.byref(k), 0)
            want = _read(L, out, n_out)
            assert np.array_equal(got, want), "dispatch %d of %s: %d words differ" % (
                i, path.split("/")[-1], int(np.sum(got != want)))
            checked += 1
        assert L.thvm_hip_synchronize() == 0
    finally:
        rp.close()
    return checked


def test_noalloc_after_fused_step():
    L, saved = _fresh({})
    try:
        n = _fused_then_noalloc(L, os.path.join(WL, "lenet_b256.trc"), "lenet.step", "lenet.end")
        assert n >= 50
        n = _fused_then_noalloc(L, os.path.join(WL, "mlp_64x784x128x10.trc"), "mlp.fwd", None)
        assert n >= 15
    finally:
        _restore(L, saved)
