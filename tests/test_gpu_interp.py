"""The KOp interpreter (static kernel thvm_kop), the path of a program the
kernel generator or hipRTC cannot compile, on the GPU.

With THVM_HIP_INTERP=1 every lowered program of every committed trace runs on
the interpreter (matrix cores off). It executes each gid's whole program with
its reduce loops in order, as the reference interpreter does
(src/backend/cpu/uop.c:29-155), so every dispatch must match the oracle bit
for bit (1e-6 per element where EXP or LOG appear: device libm). With
THVM_HIP_RTC_FAIL=1 every compile fails: the dispatches must still produce
the oracle's outputs, and the fallback counter must count each of them.
"""
import ctypes as C
import os

import pytest

from tests import tracetools as tt
from tests.test_gpu_parity import _has_transcendental_uop, _oracle, kernel_parity
from tinyhvm_amd import _lib

pytestmark = pytest.mark.gpu

KNOBS = ("THVM_HIP_INTERP", "THVM_HIP_RTC_FAIL", "THVM_HIP_NO_DENSE", "THVM_HIP_DENSE_FORCE")


def _init(env):
    """A fresh backend that reads these knobs (init reads them once)."""
    L = _lib.lib()
    L.thvm_hip_shutdown()
    saved = {k: os.environ.pop(k, None) for k in KNOBS}
    os.environ.update(env)
    assert L.thvm_hip_init() == 0, "HIP backend failed to initialise"
    return L, saved


def _fini(L, saved):
    L.thvm_hip_shutdown()
    for k in KNOBS:
        os.environ.pop(k, None)
        if saved[k] is not None:
            os.environ[k] = saved[k]


def _serial_tolerance(k):
    return ("elem", 1e-6) if _has_transcendental_uop(k) else ("exact", 0.0)


@pytest.fixture(scope="module")
def interp():
    L, saved = _init({"THVM_HIP_INTERP": "1", "THVM_HIP_NO_DENSE": "1"})
    yield L
    _fini(L, saved)


@pytest.mark.parametrize("path", [p for p in tt.fixtures() if "/rs_" not in p], ids=lambda p: p.split("/")[-1])
def test_interpreter_parity(interp, path):
    print("interpreter parity: %s" % path.split("/")[-1], flush=True)
    before = (C.c_uint64 * 10)()
    interp.thvm_hip_counters(before, 10)
    kr, e2e = kernel_parity(interp.thvm_hip_backend(), interp.thvm_hip_buf_read, interp.thvm_hip_synchronize,
                            _oracle(), path, tol_fn=_serial_tolerance)
    bad = [r for r in kr if not r[1]]
    assert not bad, "kernel parity: %s" % bad
    bad_e2e = [r for r in e2e if not r[1]]
    assert not bad_e2e, "end-to-end vs reference: %s" % bad_e2e
    after = (C.c_uint64 * 10)()
    interp.thvm_hip_counters(after, 10)
    from tinyhvm_amd import trace
    n_uop = sum(1 for r in trace.read_trace(path) if r.tag == trace.UOP)
    assert after[4] - before[4] == n_uop, "every lowered program should have run on the interpreter"


def test_failed_compiles_fall_back_to_the_interpreter():
    L, saved = _init({"THVM_HIP_RTC_FAIL": "1", "THVM_HIP_NO_DENSE": "1"})
    try:
        path = os.path.join(tt.GOLDEN, "fused_64x256.trc")
        kr, e2e = kernel_parity(L.thvm_hip_backend(), L.thvm_hip_buf_read, L.thvm_hip_synchronize,
                                _oracle(), path, tol_fn=_serial_tolerance)
        assert kr and all(r[1] for r in kr), kr
        assert all(r[1] for r in e2e), e2e
        cnt = (C.c_uint64 * 10)()
        L.thvm_hip_counters(cnt, 10)
        assert cnt[4] == len(kr), "fallback count %d for %d dispatches" % (cnt[4], len(kr))
        assert cnt[2] == 0, "nothing should have compiled"
    finally:
        _fini(L, saved)
