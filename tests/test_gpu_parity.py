"""GPU parity: every committed kernel trace is replayed through the HIP
backend's C ABI and each dispatch's output is compared with the reference CPU
backend's output recorded in the trace.

Tolerances: bit-exact for kernels that run in the
reference's own order (serial mode: elementwise, index/view work, RMAX, and
reductions a single lane walks in order) except for EXP/LOG, 1e-6 relative for
those, and 1e-4 relative (with a floor at 1e-3 of the output's max) for
reductions split across a workgroup, whose summation order differs."""
import ctypes as C
import sys

import numpy as np
import pytest

from tests import tracetools as tt
from tinyhvm_amd import _lib, abi

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    L = _lib.lib()
    assert L.thvm_hip_init() == 0, "HIP backend failed to initialise"
    yield L
    L.thvm_hip_shutdown()


def _has_transcendental(k):
    return any(k.ops[i].type == abi.KOP_ALU and k.ops[i].imm.u in (abi.UOP_EXP, abi.UOP_LOG)
               for i in range(k.n_ops))


def _kernel_tolerance(k):
    _src, mode, _vec = _lib.kernel_source(k)
    if mode == 1:
        has_sum = any(k.ops[i].type == abi.KOP_ACC and k.ops[i].imm.u != abi.UOP_RMAX
                      for i in range(k.n_ops))
        if has_sum:
            return 1e-4
    return 1e-6 if _has_transcendental(k) else 0.0


def replay_and_compare(L, path):
    be = L.thvm_hip_backend()
    rp = tt.Replay(path, be)
    results = []
    last_kernel = None
    last_rs = False
    try:
        for i in range(rp.n):
            tag = rp.tag(i)
            if tag == tt.TRC_SNAPSHOT:
                tid, ref = rp.snapshot(i)
                live = rp.live(tid)
                buf = (C.c_uint8 * len(ref))()
                L.thvm_hip_buf_read(live, buf, len(ref))
                got = bytes(buf)
                if last_rs or last_kernel is None:
                    tol = 0.0
                    dt = np.float32
                else:
                    tol = _kernel_tolerance(last_kernel)
                    dt = tt.dtype_of_kernel(last_kernel)
                if tol == 0.0:
                    ok = got == ref
                    msg = "bit-exact" if ok else "differs (%d of %d bytes)" % (
                        sum(a != b for a, b in zip(got, ref)), len(ref))
                else:
                    ok, msg = tt.close(np.frombuffer(got, dtype=dt), np.frombuffer(ref, dtype=dt), tol)
                results.append((i, ok, msg))
                print("  %s record %d: %s" % (path.split("/")[-1], i, msg), flush=True)
            else:
                if tag == tt.TRC_UOP:
                    last_kernel = rp.kernel(i)
                    last_rs = False
                elif tag == tt.TRC_RS:
                    last_rs = True
                print("  %s record %d tag %d" % (path.split("/")[-1], i, tag), file=sys.stderr, flush=True)
                rp.run(i, i + 1)
        assert L.thvm_hip_synchronize() == 0
    finally:
        rp.close()
    return results


@pytest.mark.parametrize("path", tt.fixtures(), ids=lambda p: p.split("/")[-1])
def test_trace_parity(hip, path):
    res = replay_and_compare(hip, path)
    assert res, "trace has no snapshots"
    bad = [r for r in res if not r[1]]
    assert not bad, bad
