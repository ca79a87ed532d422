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
                assert L.thvm_hip_counters(c1, 14) == 14
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
