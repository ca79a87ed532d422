"""Single-pass combines that give up waiting are reported to the host.

A split reduction whose grid fits on the GPU at once combines its
workgroups' partial sums in the same launch: the last workgroup of each
output waits (a bounded number of polls) for the other workgroups' partials.
If a wait runs out, the partial is taken as a NaN, the kernel still ends
normally, and the host must learn of it: the kernel sets a host-visible word,
and the next wait on the stream counts it (counter 13), prints it, and makes
thvm_hip_synchronize return -1.

The condition is forced from the host: THVM_HIP_COMB_WITHHOLD=1 builds the
kernels so that split 0 of output 0 never publishes its partial, and
THVM_HIP_COMB_SPIN bounds each wait at a few thousand polls, so every wait
ends quickly. Over the long-reduction fixture (three split reductions of 3-4
outputs over 20,000 values: two run sums and one generated reduction; with
THVM_HIP_NO_WINDOW=1 all three are generated reductions), each dispatch runs
alone, and then:
  - a split reduction: thvm_hip_synchronize returns -1 once (0 afterwards),
    the counter goes up by one, every other output is bit for bit that of a
    run without the knob, and a sum's output 0 is a NaN (a max combines
    with the engine's a > b ? a : b, which may drop the NaN taken for the
    missing partial: there the report is the signal);
  - any other dispatch: synchronize returns 0 and the output is bit for bit
    that of the run without the knob.
After each split reduction the correct output is written back, so that later
dispatches read the same inputs in both runs.
"""
import ctypes as C
import os

import numpy as np
import pytest

from tests import tracetools as tt
from tinyhvm_amd import _lib, abi, trace

pytestmark = pytest.mark.gpu

PATH = os.path.join(tt.GOLDEN, "longreduce_4x20000.trc")
KNOBS = ("THVM_HIP_COMB_WITHHOLD", "THVM_HIP_COMB_SPIN", "THVM_HIP_NO_WINDOW")


def _single_pass(k, no_window):
    """Whether the backend runs kernel k as a split reduction combined in
    its own launch (a run sum of several workgroups per output, or a
    generated split reduction with the combine words as its last buffer)."""
    w = None if no_window else _lib.window_analyze(k)
    if w is not None:
        return w[0] == 2 and w[1] > 1
    return "unsigned long long* sl_" in _lib.kernel_source(k)[0]


def _is_max(k):
    """Whether the program's accumulator combines with the engine's max."""
    return any(k.ops[j].type == abi.KOP_ACC and k.ops[j].imm.u == abi.UOP_RMAX for j in range(k.n_ops))


def _run(env, fix=None):
    """Every UOP of the fixture alone, in a fresh backend with `env`; returns
    (outputs by record index, synchronize codes, give-up counts, the kernels).
    fix: record index -> the output written back after that dispatch."""
    L = _lib.lib()
    L.thvm_hip_shutdown()
    saved = {k: os.environ.pop(k, None) for k in KNOBS}
    os.environ.update(env)
    outs, rcs, gave, ks = {}, {}, {}, {}
    try:
        assert L.thvm_hip_init() == 0
        recs = trace.read_trace(PATH)
        sizes = {r.f["id"]: r.f["bytes"] for r in recs if r.tag == trace.ALLOC}
        rp = tt.Replay(PATH, L.thvm_hip_backend())
        try:
            for i, r in enumerate(recs):
                rp.run(i, i + 1, 1)
                if r.tag != trace.UOP:
                    continue
                c0 = (C.c_uint64 * 14)()
                L.thvm_hip_counters(c0, 14)
                rcs[i] = L.thvm_hip_synchronize()
                c1 = (C.c_uint64 * 14)()
                assert L.thvm_hip_counters(c1, 14) == 16
                gave[i] = c1[13] - c0[13]
                n = sizes[r.f["out"]]
                buf = np.zeros(n // 4, dtype=np.float32)
                L.thvm_hip_buf_read(rp.live(r.f["out"]), buf.ctypes.data_as(C.c_void_p), n)
                outs[i] = buf
                ks[i] = trace.to_uop_kernel(r)
                if fix and i in fix:
                    L.thvm_hip_buf_write(rp.live(r.f["out"]), fix[i].ctypes.data_as(C.c_void_p), n)
                assert L.thvm_hip_synchronize() == 0, "a second synchronize still reports the give-up"
        finally:
            rp.close()
    finally:
        L.thvm_hip_shutdown()
        for k in KNOBS:
            os.environ.pop(k, None)
            if saved[k] is not None:
                os.environ[k] = saved[k]
    return outs, rcs, gave, ks


@pytest.mark.parametrize("no_window", [False, True], ids=["run_sums", "generated"])
def test_combine_give_up_is_reported(no_window):
    base = {"THVM_HIP_NO_WINDOW": "1"} if no_window else {}
    ref, rc_ref, gave_ref, ks = _run(dict(base))
    assert all(rc == 0 for rc in rc_ref.values()) and not any(gave_ref.values())
    split = [i for i in ref if _single_pass(ks[i], no_window)]
    assert len(split) == 3, split
    env = dict(base, THVM_HIP_COMB_WITHHOLD="1", THVM_HIP_COMB_SPIN="4096")
    got, rcs, gave, _ = _run(env, fix={i: ref[i] for i in split})
    for i in ref:
        if i in split:
            assert rcs[i] == -1, "dispatch %d: the give-up was not reported" % i
            assert gave[i] == 1, (i, gave[i])
            if not _is_max(ks[i]):
                # a sum takes the missing partial as a NaN; the engine's max
                # rule (a > b ? a : b) may drop it, so a max is only reported
                assert np.isnan(got[i][0]), "dispatch %d: output 0 is %r, not a NaN" % (i, got[i][0])
            assert got[i][1:].tobytes() == ref[i][1:].tobytes(), "dispatch %d: other outputs differ" % i
        else:
            assert rcs[i] == 0 and gave[i] == 0, (i, rcs[i], gave[i])
            assert got[i].tobytes() == ref[i].tobytes(), "dispatch %d differs" % i


def _long_sum(trip):
    """One output summing `trip` consecutive floats of its leaf: a run sum
    the backend splits over up to 1024 workgroups."""
    k = abi.UOpKernel()
    ops = [(abi.KOP_GID, (0, 0, 0), None), (abi.KOP_ACC_INIT, (0, 0, 0), 0.0), (abi.KOP_RANGE, (0, 0, 0), trip),
           (abi.KOP_LOAD, (2, 0, 0), 1), (abi.KOP_ACC, (1, 3, 0), abi.UOP_SUM), (abi.KOP_ENDRANGE, (2, 0, 0), 0),
           (abi.KOP_STORE, (0, 1, 0), 0)]
    for j, (t, a, imm) in enumerate(ops):
        k.ops[j].type = t
        for q in range(3):
            k.ops[j].arg[q] = a[q]
        if isinstance(imm, float):
            k.ops[j].imm.f = imm
        elif imm is not None:
            k.ops[j].imm.u = imm
    k.n_ops, k.n_leaves, k.n_bufs = len(ops), 1, 2
    k.leaf_dtypes[0] = abi.DTYPE_F32
    k.out_dtype = abi.DTYPE_F32
    k.grid[0], k.grid[1], k.grid[2] = 1, 1, 1
    k.local_size, k.reduce_numel = 256, trip
    return k


def _sum_once(k, x, env):
    L = _lib.lib()
    L.thvm_hip_shutdown()
    saved = {n: os.environ.pop(n, None) for n in KNOBS}
    os.environ.update(env)
    try:
        assert L.thvm_hip_init() == 0
        xb, ob = L.thvm_hip_buf_alloc(x.nbytes), L.thvm_hip_buf_alloc(4)
        L.thvm_hip_buf_write(xb, x.ctypes.data_as(C.c_void_p), x.nbytes)
        c0 = (C.c_uint64 * 14)()
        L.thvm_hip_counters(c0, 14)
        leaves = (C.c_uint32 * 1)(xb)
        L.thvm_hip_dispatch_uop_kernel(ob, leaves, 1, C.byref(k), 0)
        rc = L.thvm_hip_synchronize()
        c1 = (C.c_uint64 * 14)()
        L.thvm_hip_counters(c1, 14)
        out = np.zeros(1, dtype=np.float32)
        L.thvm_hip_buf_read(ob, out.ctypes.data_as(C.c_void_p), 4)
        return out[0], rc, c1[13] - c0[13]
    finally:
        L.thvm_hip_shutdown()
        for n in KNOBS:
            os.environ.pop(n, None)
            if saved[n] is not None:
                os.environ[n] = saved[n]


def test_give_up_with_several_partials_per_lane():
    """A sum split over more workgroups than a workgroup has lanes (1024
    here): the combining workgroup reads all of a lane's partial words first
    and then waits for each. A withheld partial is still a NaN, reported
    once, and the sum without the knob is the plain one."""
    trip = 1 << 21
    k = _long_sum(trip)
    w = _lib.window_analyze(k)
    assert w == (2, 1024), w
    x = np.random.default_rng(5).standard_normal(trip).astype(np.float32)
    ref, rc, gave = _sum_once(k, x, {})
    assert rc == 0 and gave == 0
    assert abs(float(ref) - float(x.astype(np.float64).sum())) <= 1e-4 * float(np.abs(x).astype(np.float64).sum())
    got, rc, gave = _sum_once(k, x, {"THVM_HIP_COMB_WITHHOLD": "1", "THVM_HIP_COMB_SPIN": "4096"})
    assert rc == -1 and gave == 1 and np.isnan(got), (got, rc, gave)
