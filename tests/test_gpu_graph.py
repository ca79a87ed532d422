"""HIP graphs of a recorded training step (thvm_hip_graph_*).

One LeNet-5 training step at batch 256 (forward, backward, SGD through
ASSIGN) is replayed from its kernel trace once eagerly and once under stream
capture; the graph is then launched several times, each launch starting from
the same parameters, with the program's own eager steps, host writes and
synchronizations between the launches. Every launch must leave the ten
parameters bit-identical to the eager step (the same kernels with the same
arguments in the same order; every sum has a fixed order).
"""
import ctypes as C
import os

import numpy as np
import pytest

from tinyhvm_amd import _lib

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TRACE = os.path.join(ROOT, "tinyhvm_amd", "workloads", "lenet_b256.trc")
PARAMS = range(2, 12)          # trace ids of W1, b1, ..., W5, b5
SKIP_READS = 1


@pytest.fixture(scope="module")
def L():
    L = _lib.lib()
    assert L.thvm_hip_init() == 0, "HIP backend failed to initialise"
    yield L
    L.thvm_hip_shutdown()


def _params(L, t, sizes):
    out = {}
    for tid in PARAMS:
        n = sizes[tid]
        buf = (C.c_uint8 * n)()
        L.thvm_hip_buf_read(L.thvm_trace_live_id(t, tid), buf, n)
        out[tid] = bytes(buf)
    return out


def _restore(L, t, p0):
    for tid, data in p0.items():
        L.thvm_hip_buf_write(L.thvm_trace_live_id(t, tid), data, len(data))


def test_graph_of_training_step_matches_eager(L):
    from tinyhvm_amd import trace
    sizes = {r.f["id"]: r.f["bytes"] for r in trace.read_trace(TRACE) if r.tag == trace.ALLOC}
    be = L.thvm_hip_backend()
    t = L.thvm_trace_load(TRACE.encode())
    assert t
    g = None
    try:
        n = L.thvm_trace_count(t)
        lo = L.thvm_trace_find_mark(t, b"lenet.step", 0)
        hi = L.thvm_trace_find_mark(t, b"lenet.end", lo)
        assert 0 <= lo < hi <= n
        L.thvm_trace_replay(t, be, 0, lo, 0)
        L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)      # compiles every kernel
        assert L.thvm_hip_synchronize() == 0
        p0 = _params(L, t, sizes)
        L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)
        assert L.thvm_hip_synchronize() == 0
        eager = _params(L, t, sizes)
        assert any(eager[k] != p0[k] for k in PARAMS), "the step did not update the parameters"
        _restore(L, t, p0)
        assert L.thvm_hip_synchronize() == 0

        assert L.thvm_hip_graph_begin() == 0
        L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)
        g = L.thvm_hip_graph_end()
        assert g, "the step could not be captured"
        # capture ran nothing on the device
        assert _params(L, t, sizes) == p0

        for rep in range(3):
            _restore(L, t, p0)
            assert L.thvm_hip_graph_launch(g) == 0
            assert L.thvm_hip_synchronize() == 0
            got = _params(L, t, sizes)
            bad = [k for k in PARAMS if got[k] != eager[k]]
            assert not bad, "graph launch %d: parameters %s differ from the eager step" % (rep, bad)
            # eager work between the launches: an eager step from the same state
            _restore(L, t, p0)
            L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)
            assert L.thvm_hip_synchronize() == 0
            again = _params(L, t, sizes)
            assert all(again[k] == eager[k] for k in PARAMS), "eager step %d differs" % rep
        # two launches in a row are two training steps
        _restore(L, t, p0)
        assert L.thvm_hip_graph_launch(g) == 0 and L.thvm_hip_graph_launch(g) == 0
        assert L.thvm_hip_synchronize() == 0
        two = _params(L, t, sizes)
        _restore(L, t, p0)
        L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)
        L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)
        assert L.thvm_hip_synchronize() == 0
        assert _params(L, t, sizes) == two
        assert any(two[k] != eager[k] for k in PARAMS)
    finally:
        if g:
            L.thvm_hip_graph_destroy(g)
        L.thvm_trace_release(t, be)
        L.thvm_trace_free(t)
        L.thvm_hip_pool_reset(0)


CONV = os.path.join(ROOT, "tinyhvm_amd", "workloads", "convblock_b64.trc")


def _out_bytes(L, t, tid, n):
    buf = (C.c_uint8 * n)()
    L.thvm_hip_buf_read(L.thvm_trace_live_id(t, tid), buf, n)
    return bytes(buf)


def test_graph_of_conv_block_matches_eager(L):
    """The conv block step at batch 64 under graph launches (the matrix-core
    convolutions with their packed weights and the weight gradient's split-K
    workspace, the split reductions of batchnorm and the loss): three
    launches, with eager steps between them, each leave the three
    convolution outputs bit-identical to the eager step's (every sum has a
    fixed order)."""
    from tinyhvm_amd import trace
    recs = trace.read_trace(CONV)
    sizes = {r.f["id"]: r.f["bytes"] for r in recs if r.tag == trace.ALLOC}
    be = L.thvm_hip_backend()
    t = L.thvm_trace_load(CONV.encode())
    assert t
    g = None
    try:
        n = L.thvm_trace_count(t)
        lo = L.thvm_trace_find_mark(t, b"conv.fwd", 0)
        assert 0 <= lo < n
        outs = [r.f["out"] for r in recs[lo:] if r.tag == trace.UOP]
        watch = [outs[1], outs[23], outs[27]]          # conv forward, dW, dX
        L.thvm_trace_replay(t, be, 0, lo, 0)
        L.thvm_trace_replay(t, be, lo, n, SKIP_READS)      # compiles every kernel
        assert L.thvm_hip_synchronize() == 0
        eager = {tid: _out_bytes(L, t, tid, sizes[tid]) for tid in watch}
        assert L.thvm_hip_graph_begin() == 0
        L.thvm_trace_replay(t, be, lo, n, SKIP_READS)
        g = L.thvm_hip_graph_end()
        assert g, "the step could not be captured"
        for rep in range(3):
            assert L.thvm_hip_graph_launch(g) == 0
            assert L.thvm_hip_synchronize() == 0
            got = {tid: _out_bytes(L, t, tid, sizes[tid]) for tid in watch}
            bad = [tid for tid in watch if got[tid] != eager[tid]]
            assert not bad, "graph launch %d: outputs %s differ from the eager step" % (rep, bad)
            L.thvm_trace_replay(t, be, lo, n, SKIP_READS)
            assert L.thvm_hip_synchronize() == 0
            again = {tid: _out_bytes(L, t, tid, sizes[tid]) for tid in watch}
            assert again == eager, "eager step %d differs" % rep
    finally:
        if g:
            L.thvm_hip_graph_destroy(g)
        L.thvm_trace_release(t, be)
        L.thvm_trace_free(t)
        L.thvm_hip_pool_reset(0)


def test_capture_with_a_host_read_is_refused(L):
    """A host read inside the captured calls cannot be repeated by a graph:
    the capture is abandoned, graph_end returns NULL, and the backend keeps
    working eagerly."""
    buf = L.thvm_hip_buf_alloc(4096)
    data = np.arange(1024, dtype=np.float32)
    L.thvm_hip_buf_write(buf, data.ctypes.data_as(C.c_void_p), 4096)
    L.thvm_hip_buf_write(buf, data.ctypes.data_as(C.c_void_p), 4096)
    assert L.thvm_hip_synchronize() == 0
    other = L.thvm_hip_buf_alloc(4096)
    L.thvm_hip_buf_copy(other, buf, 4096)
    assert L.thvm_hip_graph_begin() == 0
    out = np.zeros(1024, dtype=np.float32)
    L.thvm_hip_buf_read(other, out.ctypes.data_as(C.c_void_p), 4096)
    assert not L.thvm_hip_graph_end()
    L.thvm_hip_buf_read(other, out.ctypes.data_as(C.c_void_p), 4096)
    assert np.array_equal(out, data)
    L.thvm_hip_buf_free(buf)
    L.thvm_hip_buf_free(other)


def test_graph_memory_is_not_handed_out_again(L):
    """Blocks a graph writes stay reserved while it lives: the step's
    temporaries, allocated and freed inside the capture, are not given to
    buffers allocated after it, so launching the graph leaves those buffers
    intact; once the graph is destroyed the blocks are reusable."""
    from tinyhvm_amd import trace
    recs = trace.read_trace(TRACE)
    be = L.thvm_hip_backend()
    t = L.thvm_trace_load(TRACE.encode())
    assert t
    g = None
    extra = []
    try:
        lo = L.thvm_trace_find_mark(t, b"lenet.step", 0)
        hi = L.thvm_trace_find_mark(t, b"lenet.end", lo)
        L.thvm_trace_replay(t, be, 0, lo, 0)
        L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)
        assert L.thvm_hip_synchronize() == 0
        assert L.thvm_hip_graph_begin() == 0
        L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)
        g = L.thvm_hip_graph_end()
        assert g, "the step could not be captured"
        cnt = (C.c_uint64 * 10)()
        L.thvm_hip_counters(cnt, 10)
        assert cnt[8] > 0, "no device block was pinned by the capture"
        # buffers of every size the step allocates, each with its own pattern
        step_sizes = [r.f["bytes"] for r in recs[lo:hi] if r.tag == trace.ALLOC]
        assert len(step_sizes) > 20
        for j, nb in enumerate(step_sizes):
            b = L.thvm_hip_buf_alloc(nb)
            assert b
            pat = np.full((nb + 3) // 4, np.float32(1000 + j), dtype=np.float32)
            L.thvm_hip_buf_write(b, pat.ctypes.data_as(C.c_void_p), nb)
            extra.append((b, nb, pat))
        assert L.thvm_hip_synchronize() == 0
        for _ in range(2):
            assert L.thvm_hip_graph_launch(g) == 0
        assert L.thvm_hip_synchronize() == 0
        for b, nb, pat in extra:
            out = np.zeros((nb + 3) // 4, dtype=np.float32)
            L.thvm_hip_buf_read(b, out.ctypes.data_as(C.c_void_p), nb)
            assert np.array_equal(out[:nb // 4], pat[:nb // 4]), "a graph launch wrote a later buffer"
        L.thvm_hip_graph_destroy(g)
        g = None
        L.thvm_hip_counters(cnt, 10)
        assert cnt[8] == 0 and cnt[9] == 0, "blocks still pinned after the graph was destroyed"
    finally:
        if g:
            L.thvm_hip_graph_destroy(g)
        for b, _nb, _p in extra:
            L.thvm_hip_buf_free(b)
        L.thvm_trace_release(t, be)
        L.thvm_trace_free(t)
        L.thvm_hip_pool_reset(0)
