"""Batched launches of independent generated kernels, elementwise kernels
fused into the epilogue of the contraction they follow, and loop-free
kernels merged with the loop-free kernel whose output they read.

The backend holds back launches of generated kernels and issues independent
ones together as one launch of a batch kernel. In a LeNet-5 training step at
batch 256: each fully connected layer's weight gradient (the direct MFMA
kernel), bias gradient (a group reduction) and input gradient; each
convolution's weight gradient (the outer-product kernel or its split-K sum)
and bias gradient (a run sum); the ten SGD updates. The step is replayed
twice from the same parameters in fresh backends, with batching on and with
THVM_HIP_NO_BATCH=1: the ten updated parameters, which every gradient feeds,
must be bit identical (each kernel's arithmetic is the same either way), and
the batched run must have issued at least 20 dispatches inside batch
launches.
"""
import ctypes as C
import os

import pytest

from tinyhvm_amd import _lib, trace

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TRACE = os.path.join(ROOT, "tinyhvm_amd", "workloads", "lenet_b256.trc")
PARAMS = range(2, 12)          # trace ids of W1, b1, ..., W5, b5


CONV = os.path.join(ROOT, "tinyhvm_amd", "workloads", "convblock_b64.trc")
MLP = os.path.join(ROOT, "tinyhvm_amd", "workloads", "mlp_64x784x128x10.trc")


def _run_all(path, m0, m1, no_fuse):
    """Replays [m0, m1) of a trace (the part before m0 untimed) in a fresh
    backend; returns every buffer live at the end (trace id -> bytes) and
    the number of dispatches fused into a held launch."""
    old = os.environ.get("THVM_HIP_NO_FUSE")
    os.environ["THVM_HIP_NO_FUSE"] = "1" if no_fuse else "0"
    L = _lib.lib()
    try:
        assert L.thvm_hip_init() == 0
        recs = trace.read_trace(path)
        sizes = {r.f["id"]: r.f["bytes"] for r in recs if r.tag == trace.ALLOC}
        be = L.thvm_hip_backend()
        t = L.thvm_trace_load(path.encode())
        assert t
        lo = L.thvm_trace_find_mark(t, m0.encode(), 0)
        hi = L.thvm_trace_find_mark(t, m1.encode(), lo) if m1 else L.thvm_trace_count(t)
        L.thvm_trace_replay(t, be, 0, lo, 0)
        before = (C.c_uint64 * 13)()
        L.thvm_hip_counters(before, 13)
        L.thvm_trace_replay(t, be, lo, hi, 1)
        assert L.thvm_hip_synchronize() == 0
        after = (C.c_uint64 * 13)()
        assert L.thvm_hip_counters(after, 13) == 13
        out = {}
        for tid, n in sizes.items():
            live = L.thvm_trace_live_id(t, tid)
            if live:
                buf = (C.c_uint8 * n)()
                L.thvm_hip_buf_read(live, buf, n)
                out[tid] = bytes(buf)
        L.thvm_trace_release(t, be)
        L.thvm_trace_free(t)
        return out, after[12] - before[12]
    finally:
        L.thvm_hip_shutdown()
        if old is None:
            os.environ.pop("THVM_HIP_NO_FUSE", None)
        else:
            os.environ["THVM_HIP_NO_FUSE"] = old


def _step(no_batch, no_fuse=False):
    old = {k: os.environ.get(k) for k in ("THVM_HIP_NO_BATCH", "THVM_HIP_NO_FUSE")}
    os.environ["THVM_HIP_NO_BATCH"] = "1" if no_batch else "0"
    os.environ["THVM_HIP_NO_FUSE"] = "1" if no_fuse else "0"
    L = _lib.lib()
    try:
        assert L.thvm_hip_init() == 0
        sizes = {r.f["id"]: r.f["bytes"] for r in trace.read_trace(TRACE) if r.tag == trace.ALLOC}
        be = L.thvm_hip_backend()
        t = L.thvm_trace_load(TRACE.encode())
        assert t
        lo = L.thvm_trace_find_mark(t, b"lenet.step", 0)
        hi = L.thvm_trace_find_mark(t, b"lenet.end", lo)
        L.thvm_trace_replay(t, be, 0, lo, 0)
        before = (C.c_uint64 * 13)()
        L.thvm_hip_counters(before, 13)
        L.thvm_trace_replay(t, be, lo, hi, 1)
        assert L.thvm_hip_synchronize() == 0
        after = (C.c_uint64 * 13)()
        assert L.thvm_hip_counters(after, 13) == 13
        out = {}
        for tid in PARAMS:
            buf = (C.c_uint8 * sizes[tid])()
            L.thvm_hip_buf_read(L.thvm_trace_live_id(t, tid), buf, sizes[tid])
            out[tid] = bytes(buf)
        L.thvm_trace_release(t, be)
        L.thvm_trace_free(t)
        return out, after[11] - before[11], after[12] - before[12]
    finally:
        L.thvm_hip_shutdown()
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def test_batched_launches_match_single_launches():
    single, n_single, _ = _step(no_batch=True)
    batched, n_batched, _ = _step(no_batch=False, no_fuse=True)
    assert n_single == 0
    assert n_batched >= 20, "only %d dispatches were batched" % n_batched
    bad = [tid for tid in PARAMS if single[tid] != batched[tid]]
    assert not bad, "parameters %s differ between batched and single launches" % bad


def test_fused_epilogues_match_separate_launches():
    """The bias+relu (or bias) kernels after LeNet-5's two convolutions and
    three fully connected layers, and the relu mask after fc2's input
    gradient, run in the epilogue of the contraction whose output they read
    (no launch of their own). The step's updated parameters are bit for bit
    those with THVM_HIP_NO_FUSE=1 (every kernel launched on its own), and at
    least the five forward consumers were fused."""
    separate, _, n_sep = _step(no_batch=False, no_fuse=True)
    fused, _, n_fused = _step(no_batch=False)
    assert n_sep == 0
    assert n_fused >= 5, "only %d epilogues were fused" % n_fused
    bad = [tid for tid in PARAMS if separate[tid] != fused[tid]]
    assert not bad, "parameters %s differ between fused and separate launches" % bad


def test_chained_elementwise_match_separate_launches():
    """Loop-free dispatches that read a held loop-free program's output at
    their own gid run merged with it (one launch writing both outputs): in
    the conv block at [64,64,56,56], batchnorm's variance and inverse
    deviation (the variance's input is freed in between: the free waits for
    the launch), the normalisation with its scale and shift and the relu
    after them, and the pooling backward's routing with the product by the
    scale. Every buffer live after the forward and backward step is bit for
    bit that of THVM_HIP_NO_FUSE=1, and those four dispatches were fused."""
    sep, n_sep = _run_all(CONV, "conv.fwd", None, no_fuse=True)
    fused, n_fused = _run_all(CONV, "conv.fwd", None, no_fuse=False)
    assert n_sep == 0
    assert n_fused >= 4, "only %d dispatches were fused" % n_fused
    assert sep.keys() == fused.keys()
    bad = [tid for tid in sep if sep[tid] != fused[tid]]
    assert not bad, "buffers %s differ between fused and separate launches" % bad


def test_mlp_fusions_match_separate_launches():
    """The MLP step: fc2's bias in the epilogue of its contraction, a
    softmax step merged with the one before, and the relu mask merged with
    fc2's input gradient (a generated loop that each lane runs for its own
    gid). Every buffer live after the step is bit for bit that of
    THVM_HIP_NO_FUSE=1."""
    sep, n_sep = _run_all(MLP, "mlp.fwd", None, no_fuse=True)
    fused, n_fused = _run_all(MLP, "mlp.fwd", None, no_fuse=False)
    assert n_sep == 0
    assert n_fused >= 3, "only %d dispatches were fused" % n_fused
    assert sep.keys() == fused.keys()
    bad = [tid for tid in sep if sep[tid] != fused[tid]]
    assert not bad, "buffers %s differ between fused and separate launches" % bad
