"""The wave tile's split tail tiles on the GPU (dense.c, plan_wave_tail).

The 3x3 64->64 convolution at batch 64 has 6272 tiles of 32 output pixels
for 1024 SIMDs: 6144 run whole, 4 to a workgroup, and each of the last 128
is split over the waves of one workgroup in K chunks added through LDS. The
whole tiles keep the summation order of the one-tile-per-wave grid
(THVM_HIP_DENSE_NOTAIL=1), so they match it bit for bit; the split tiles
add their chunks in chunk order, within the contractions' 1e-4 normwise
class of it. Split widths of 2, 4 (the default) and 8 waves
(THVM_HIP_WAVE_TAIL_S) are compared, and every output is written."""
import ctypes as C
import os

import numpy as np
import pytest

from tests import tracetools as tt
from tinyhvm_amd import _lib, trace

pytestmark = pytest.mark.gpu

PATH = os.path.join(tt.ROOT, "tinyhvm_amd", "workloads", "convblock_b64.trc")
KNOBS = ("THVM_HIP_DENSE_NOTAIL", "THVM_HIP_WAVE_TAIL_S")
N_OUT = 64 * 64 * 56 * 56


def _conv_record():
    """(record index, output trace id, kernel) of the step's forward convolution"""
    recs = trace.read_trace(PATH)
    for i, r in enumerate(recs):
        if r.tag == trace.UOP:
            k = trace.to_uop_kernel(r)
            a = _lib.dense_analyze(k)
            if a and a[:3] == (200704, 64, 576):
                return i, r.f["out"], k
    raise AssertionError("no forward convolution in the trace")


def _conv_output(env):
    idx, out_tid, _k = _conv_record()
    L = _lib.lib()
    L.thvm_hip_shutdown()
    saved = {k: os.environ.pop(k, None) for k in KNOBS}
    os.environ.update(env)
    try:
        assert L.thvm_hip_init() == 0
        rp = tt.Replay(PATH, L.thvm_hip_backend())
        try:
            rp.run(0, idx)
            assert L.thvm_hip_synchronize() == 0
            out = rp.live(out_tid)
            assert out
            # NaN sentinels: an output the kernel does not write stays NaN
            nan = np.full(N_OUT, np.nan, dtype=np.float32)
            L.thvm_hip_buf_write(out, nan.ctypes.data_as(C.c_void_p), N_OUT * 4)
            before = (C.c_uint64 * 2)()
            L.thvm_hip_counters(before, 2)
            rp.run(idx, idx + 1)
            assert L.thvm_hip_synchronize() == 0
            after = (C.c_uint64 * 2)()
            L.thvm_hip_counters(after, 2)
            assert after[1] - before[1] == 1, "the convolution did not run on matrix cores"
            buf = (C.c_uint8 * (N_OUT * 4))()
            L.thvm_hip_buf_read(out, buf, N_OUT * 4)
            return np.frombuffer(bytes(buf), dtype=np.float32).copy()
        finally:
            rp.close()
    finally:
        L.thvm_hip_shutdown()
        for k in KNOBS:
            os.environ.pop(k, None)
            if saved[k] is not None:
                os.environ[k] = saved[k]


@pytest.mark.timeout(300)
def test_split_tail_matches_whole_tiles():
    base = _conv_output({})
    whole = _conv_output({"THVM_HIP_DENSE_NOTAIL": "1"})
    i = np.arange(N_OUT)
    pixel = (i // (64 * 3136)) * 3136 + i % 3136
    tail = pixel >= 6144 * 32
    assert np.isfinite(base).all() and np.isfinite(whole).all()
    assert np.array_equal(base[~tail], whole[~tail])
    scale = float(np.max(np.abs(whole)))
    for env in ({}, {"THVM_HIP_WAVE_TAIL_S": "2"}, {"THVM_HIP_WAVE_TAIL_S": "8"}):
        got = base if not env else _conv_output(env)
        assert np.isfinite(got).all(), env
        assert np.array_equal(got[~tail], whole[~tail]), env
        err = float(np.max(np.abs(got[tail].astype(np.float64) - whole[tail]))) / scale
        assert err <= 1e-5, (env, err)
