"""HIP graphs of a recorded training step (thvm_hip_graph_*).

For LeNet-5 at batch 256 (forward, backward, SGD through ASSIGN), the 2-layer
MLP at batch 64 and the conv block at batch 64 ([64,64,56,56], forward and
backward), one step is replayed from its kernel trace eagerly, and then, from
the same state, under stream capture; the graph is then launched three times,
each launch from that same state, with other eager work (another trace's
kernels, host writes, synchronizations) between the launches. After every
launch every buffer live at the end of the step (parameters, gradients,
activations, batchnorm statistics, the loss and the step's temporaries) must
be bit-identical to the eager step's: the same kernels with the same
arguments in the same order, and every sum in a fixed order. For LeNet-5,
two launches in a row must also equal two eager steps.
"""
import ctypes as C
import os

import numpy as np
import pytest

from tests import tracetools as tt
from tinyhvm_amd import _lib, trace

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
WL = os.path.join(ROOT, "tinyhvm_amd", "workloads")
TRACE = os.path.join(WL, "lenet_b256.trc")
PARAMS = range(2, 12)          # trace ids of W1, b1, ..., W5, b5
SKIP_READS = 1
STEPS = {
    "lenet": ("lenet_b256.trc", "lenet.step", "lenet.end"),
    "mlp": ("mlp_64x784x128x10.trc", "mlp.fwd", None),
    "convblock": ("convblock_b64.trc", "conv.fwd", None),
}


@pytest.fixture(scope="module")
def L():
    L = _lib.lib()
    assert L.thvm_hip_init() == 0, "HIP backend failed to initialise"
    yield L
    L.thvm_hip_shutdown()


def _live(L, t, sizes, ids=None):
    out = {}
    for tid in (sizes if ids is None else ids):
        live = L.thvm_trace_live_id(t, tid)
        if live:
            buf = (C.c_uint8 * sizes[tid])()
            L.thvm_hip_buf_read(live, buf, sizes[tid])
            out[tid] = bytes(buf)
    return out


def _restore(L, t, snap):
    for tid, data in snap.items():
        L.thvm_hip_buf_write(L.thvm_trace_live_id(t, tid), data, len(data))


def _other_eager_work(L, rep):
    """Kernels of another trace, in buffers of their own, a host write and a
    synchronization, between two graph launches."""
    other = tt.Replay(tt.fixtures("fused_64x256.trc")[0], L.thvm_hip_backend())
    try:
        other.run(0, other.n, SKIP_READS)
        b = L.thvm_hip_buf_alloc(4096)
        pat = np.full(1024, float(rep), dtype=np.float32)
        L.thvm_hip_buf_write(b, pat.ctypes.data_as(C.c_void_p), 4096)
        assert L.thvm_hip_synchronize() == 0
        L.thvm_hip_buf_free(b)
    finally:
        other.close()


@pytest.mark.parametrize("name", list(STEPS))
def test_graph_of_step_matches_eager_on_every_buffer(L, name):
    path = os.path.join(WL, STEPS[name][0])
    sizes = {r.f["id"]: r.f["bytes"] for r in trace.read_trace(path) if r.tag == trace.ALLOC}
    be = L.thvm_hip_backend()
    t = L.thvm_trace_load(path.encode())
    assert t
    g = None
    try:
        lo = L.thvm_trace_find_mark(t, STEPS[name][1].encode(), 0)
        hi = L.thvm_trace_find_mark(t, STEPS[name][2].encode(), lo) if STEPS[name][2] else L.thvm_trace_count(t)
        assert 0 <= lo < hi
        L.thvm_trace_replay(t, be, 0, lo, 0)
        s0 = _live(L, t, sizes)                             # the state before the step
        L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)      # compiles every kernel
        assert L.thvm_hip_synchronize() == 0
        _restore(L, t, s0)
        L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)
        assert L.thvm_hip_synchronize() == 0
        eager = _live(L, t, sizes)
        assert len(eager) > len(s0)
        _restore(L, t, s0)
        assert L.thvm_hip_synchronize() == 0

        assert L.thvm_hip_graph_begin() == 0
        L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)
        g = L.thvm_hip_graph_end()
        assert g, "the step could not be captured"
        # capture ran nothing on the device
        assert _live(L, t, sizes, s0) == s0
        for rep in range(3):
            _restore(L, t, s0)
            assert L.thvm_hip_graph_launch(g) == 0
            assert L.thvm_hip_synchronize() == 0
            got = _live(L, t, sizes)
            assert got.keys() == eager.keys()
            bad = sorted(k for k in eager if got[k] != eager[k])
            assert not bad, "%s, graph launch %d: buffers %s differ from the eager step" % (name, rep, bad)
            _other_eager_work(L, rep)
        if name == "lenet":
            # two launches in a row are two training steps: the same parameters
            # as a second launch from the state the first left
            _restore(L, t, s0)
            assert L.thvm_hip_graph_launch(g) == 0 and L.thvm_hip_graph_launch(g) == 0
            assert L.thvm_hip_synchronize() == 0
            two = _live(L, t, sizes, PARAMS)
            one = {k: eager[k] for k in PARAMS}
            assert any(two[k] != one[k] for k in PARAMS), "the second launch did not update the parameters"
            _restore(L, t, one)
            assert L.thvm_hip_graph_launch(g) == 0
            assert L.thvm_hip_synchronize() == 0
            assert _live(L, t, sizes, PARAMS) == two
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
