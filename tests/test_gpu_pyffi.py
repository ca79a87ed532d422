"""The engine's Python FFI surface (py/csrc/libthvm.m:52-215) with hip_backend
as the engine's device: the py_* calls of tests/pyffi.py, unchanged from the
CPU test, on a context made by thvm_init("hip") (the "hip" branch of the
engine's thvm_init, tests/live/hip_init.h, compiled into the library with the
engine's sources).

Run in a child process (python -m tests.pyffi hip), so that the engine
context and the backend it owns live and end with that process:
  - thvm_init("hip") made the HIP backend the default device (index 2);
  - the MLP step's loss, dW1 and dW2 match the fixture's read-backs of the
    engine's own MLP workload within 1e-4 normwise (float32 sums in another
    order; the CPU test holds the same calls to 1e-5);
  - the README's relu(linear) example gives [0, 2.6, 0, 5.0] within 1e-5;
  - the HIP backend ran the MLP's kernels (its dispatch counter);
  - py_free (thvm_free) shut the backend down each time.
With THVM_HIP_DEVICE naming a device that does not exist, the backend's init
fails: thvm_init("hip") stays on the CPU (default device 0), the same calls
give the CPU's results (1e-5) and the HIP backend runs nothing.
"""
import json
import os
import subprocess
import sys

import pytest

from tests import pyffi
from tests import tracetools as tt

pytestmark = pytest.mark.gpu


def _child(env=None):
    cmd = [sys.executable, "-m", "tests.pyffi", "hip"]
    print("running:", " ".join(cmd), env or "", flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=240, cwd=tt.ROOT,
                       env=dict(os.environ, **(env or {})))
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
    assert lines, "no result (exit %d): %s" % (r.returncode, r.stderr[-2000:])
    res = json.loads(lines[-1])
    print("py ffi on hip:", json.dumps(res), flush=True)
    assert r.returncode == 0 and res["device"] == "hip"
    return res, r.stderr


@pytest.mark.skipif(not os.path.exists(pyffi.LIB),
                    reason="oracle/_ref/libthvm_py.so is built where the engine sources are present")
def test_py_exports_drive_hip_backend():
    res, _ = _child()
    assert res["default_device"] == [2, 2], res
    assert res["mlp_shapes_ok"]
    for name, err in res["mlp"].items():
        assert err <= 1e-4, (name, err)
    assert max(abs(a - b) for a, b in zip(res["readme"], [0.0, 2.6, 0.0, 5.0])) <= 1e-5, res["readme"]
    assert res["mlp_hip_dispatches"] >= 5, res
    assert res["shut_down_by_free"] == [True, True], res


@pytest.mark.skipif(not os.path.exists(pyffi.LIB),
                    reason="oracle/_ref/libthvm_py.so is built where the engine sources are present")
def test_thvm_init_hip_falls_back_to_cpu():
    res, err = _child({"THVM_HIP_DEVICE": "99"})
    assert res["default_device"] == [0, 0], res
    assert "requested hip backend unavailable; using cpu" in err
    for name, e in res["mlp"].items():
        assert e <= 1e-5, (name, e)
    assert max(abs(a - b) for a, b in zip(res["readme"], [0.0, 2.6, 0.0, 5.0])) <= 1e-6, res["readme"]
    assert res["mlp_hip_dispatches"] == 0, res
