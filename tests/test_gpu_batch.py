"""The shipped dispatch mode against single launches, on every buffer.

The per-dispatch oracle harness (tests/test_gpu_parity.py, the full-size
tests) reads every input and output around each dispatch, so it sees each
kernel launched on its own. What the benchmark runs is another mode: no read
between dispatches, so the backend holds launches back and
  - issues independent ones together as one launch of a batch kernel,
  - runs an elementwise consumer in the epilogue of the matrix-core
    contraction whose output it reads,
  - merges a loop-free consumer with the held program whose output it reads,
  - and, captured into a HIP graph, replays the whole step as one submission.
Each of these must leave memory exactly as single launches do.

For LeNet-5 at batch 256 (one training step), the 2-layer MLP at batch 64
and the conv block at batch 64 ([64,64,56,56], forward and backward), the
step is replayed without reads in a fresh backend in four modes:
  single   THVM_HIP_NO_BATCH=1 THVM_HIP_NO_FUSE=1: every dispatch its own
           launch (the mode the oracle harness checks dispatch by dispatch);
  shipped  the defaults: batched, fused, merged (the benchmark's mode);
  batched  THVM_HIP_NO_FUSE=1 alone: batched launches, nothing fused;
  graph    the defaults, the step captured once into a HIP graph (after an
           eager step that compiles every kernel, and with the state before
           the step restored) and then launched.
Every buffer live at the end of the step (parameters, gradients,
activations, batchnorm statistics, the loss, every temporary still bound)
must be bit for bit that of the single launches. The shipped mode must have
batched and fused what it does in these steps.
"""
import ctypes as C
import os

import pytest

from tinyhvm_amd import _lib, trace

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
WL = os.path.join(ROOT, "tinyhvm_amd", "workloads")
SKIP_READS = 1
KNOBS = ("THVM_HIP_NO_BATCH", "THVM_HIP_NO_FUSE")

# name -> trace, first mark of the step, mark after it (None: the trace's end),
# least dispatches batched, fused and issued as sequence steps (the softmax
# and its gradient: two runs of dependent small programs) in the shipped mode
STEPS = {
    "lenet": ("lenet_b256.trc", "lenet.step", "lenet.end", 20, 5, 6),
    "mlp": ("mlp_64x784x128x10.trc", "mlp.fwd", None, 2, 3, 6),
    "convblock": ("convblock_b64.trc", "conv.fwd", None, 2, 4, 0),
}
MODES = {
    "single": {"THVM_HIP_NO_BATCH": "1", "THVM_HIP_NO_FUSE": "1"},
    "shipped": {},
    "batched": {"THVM_HIP_NO_FUSE": "1"},
    "graph": {},
}


def _live(L, t, sizes):
    out = {}
    for tid, n in sizes.items():
        live = L.thvm_trace_live_id(t, tid)
        if live:
            buf = (C.c_uint8 * n)()
            L.thvm_hip_buf_read(live, buf, n)
            out[tid] = bytes(buf)
    return out


def _restore(L, t, snap):
    for tid, data in snap.items():
        live = L.thvm_trace_live_id(t, tid)
        if live:
            L.thvm_hip_buf_write(live, data, len(data))


def _step(name, mode):
    """Every buffer live after one step of workload `name` in `mode`, and the
    dispatches batched and fused during the step."""
    path, m0, m1 = (os.path.join(WL, STEPS[name][0]),) + STEPS[name][1:3]
    L = _lib.lib()
    L.thvm_hip_shutdown()
    saved = {k: os.environ.pop(k, None) for k in KNOBS}
    os.environ.update(MODES[mode])
    try:
        assert L.thvm_hip_init() == 0
        sizes = {r.f["id"]: r.f["bytes"] for r in trace.read_trace(path) if r.tag == trace.ALLOC}
        be = L.thvm_hip_backend()
        t = L.thvm_trace_load(path.encode())
        assert t
        g = None
        try:
            lo = L.thvm_trace_find_mark(t, m0.encode(), 0)
            hi = L.thvm_trace_find_mark(t, m1.encode(), lo) if m1 else L.thvm_trace_count(t)
            assert 0 <= lo < hi
            L.thvm_trace_replay(t, be, 0, lo, 0)
            before = (C.c_uint64 * 16)()
            after = (C.c_uint64 * 16)()
            if mode == "graph":
                s0 = _live(L, t, sizes)
                L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)      # compiles every kernel
                assert L.thvm_hip_synchronize() == 0
                _restore(L, t, s0)
                assert L.thvm_hip_graph_begin() == 0
                L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)
                g = L.thvm_hip_graph_end()
                assert g, "the step could not be captured"
                _restore(L, t, s0)
                L.thvm_hip_counters(before, 16)
                assert L.thvm_hip_graph_launch(g) == 0
            else:
                L.thvm_hip_counters(before, 16)
                L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)
            assert L.thvm_hip_synchronize() == 0
            assert L.thvm_hip_counters(after, 16) >= 16
            out = _live(L, t, sizes)
        finally:
            if g:
                L.thvm_hip_graph_destroy(g)
            L.thvm_trace_release(t, be)
            L.thvm_trace_free(t)
        return out, after[11] - before[11], after[12] - before[12], after[15] - before[15]
    finally:
        L.thvm_hip_shutdown()
        for k in KNOBS:
            os.environ.pop(k, None)
            if saved[k] is not None:
                os.environ[k] = saved[k]


_single = {}


@pytest.mark.parametrize("mode", ["shipped", "batched", "graph"])
@pytest.mark.parametrize("name", list(STEPS))
def test_step_matches_single_launches(name, mode):
    if name not in _single:
        ref, nb, nf, ns = _step(name, "single")
        assert nb == 0 and nf == 0 and ns == 0
        _single[name] = ref
    ref = _single[name]
    got, n_batched, n_fused, n_seq = _step(name, mode)
    print("%s %s: %d buffers, %d dispatches batched (%d as sequence steps), %d fused" %
          (name, mode, len(got), n_batched, n_seq, n_fused))
    assert got.keys() == ref.keys()
    bad = sorted(tid for tid in ref if got[tid] != ref[tid])
    assert not bad, "%s, %s mode: buffers %s differ from single launches" % (name, mode, bad)
    if mode == "shipped":
        assert n_batched >= STEPS[name][3], "only %d dispatches were batched" % n_batched
        assert n_fused >= STEPS[name][4], "only %d dispatches were fused" % n_fused
        assert n_seq >= STEPS[name][5], "only %d dispatches were sequence steps" % n_seq
    if mode == "batched":
        assert n_batched >= STEPS[name][3] and n_fused == 0, (n_batched, n_fused)
