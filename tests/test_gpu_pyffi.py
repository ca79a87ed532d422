"""The engine's Python FFI surface (py/csrc/libthvm.m:52-215) with hip_backend
as the engine's device: the py_* calls of tests/pyffi.py, unchanged from the
CPU test, with py_init_hip (tests/live/py_hip.c) registering the backend the
way a "hip" branch of thvm_init would.

Run in a child process (python -m tests.pyffi hip), so that the engine
context and the backend it owns live and end with that process:
  - the MLP step's loss, dW1 and dW2 match the fixture's read-backs of the
    engine's own MLP workload within 1e-4 normwise (float32 sums in another
    order; the CPU test holds the same calls to 1e-5);
  - the README's relu(linear) example gives [0, 2.6, 0, 5.0] within 1e-5;
  - the HIP backend ran the MLP's kernels (its dispatch counter).
"""
import json
import os
import subprocess
import sys

import pytest

from tests import pyffi
from tests import tracetools as tt

pytestmark = pytest.mark.gpu


@pytest.mark.skipif(not os.path.exists(pyffi.LIB),
                    reason="oracle/_ref/libthvm_py.so is built where the engine sources are present")
def test_py_exports_drive_hip_backend():
    cmd = [sys.executable, "-m", "tests.pyffi", "hip"]
    print("running:", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=240, cwd=tt.ROOT)
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
    assert lines, "no result (exit %d): %s" % (r.returncode, r.stderr[-2000:])
    res = json.loads(lines[-1])
    print("py ffi on hip:", json.dumps(res), flush=True)
    assert r.returncode == 0 and res["device"] == "hip"
    assert res["mlp_shapes_ok"]
    for name, err in res["mlp"].items():
        assert err <= 1e-4, (name, err)
    assert max(abs(a - b) for a, b in zip(res["readme"], [0.0, 2.6, 0.0, 5.0])) <= 1e-5, res["readme"]
    assert res["mlp_hip_dispatches"] >= 5, res
