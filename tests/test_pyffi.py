"""The engine's Python FFI surface (py/csrc/libthvm.m:52-215) as a second
consumer of the backend vtable, checked on the CPU (the engine's own CPU
backend behind the same py_* calls):
  - the MLP step of tests/pyffi.py built from py_* calls alone matches the
    three read-backs the fixture recorded from the engine's own MLP workload
    (loss, dW1, dW2) within 1e-5 normwise;
  - the README's relu(linear) example gives its stated [0, 2.6, 0, 5.0].
The same calls with the HIP backend registered as the device are
tests/test_gpu_pyffi.py."""
import os

import numpy as np
import pytest

from tests import pyffi

pytestmark = pytest.mark.skipif(not os.path.exists(pyffi.LIB),
                                reason="oracle/_ref/libthvm_py.so is built where the engine sources are present")


def test_mlp_gradients_through_py_exports_match_fixture():
    got = pyffi.mlp_step("cpu")
    want = pyffi.fixture_readbacks()
    assert len(want) == 3
    for name, g, w in zip(("loss", "dW1", "dW2"), got, want):
        err = pyffi.normwise(g, w)
        print("%s: normwise %.2e" % (name, err))
        assert g.shape == w.shape and err <= 1e-5, (name, err)


def test_readme_linear_known_answer():
    np.testing.assert_allclose(pyffi.readme_linear("cpu"), [0.0, 2.6, 0.0, 5.0], rtol=0, atol=1e-6)


def test_thvm_init_hip_falls_back_to_cpu_without_the_device():
    """thvm_init("hip") with a backend whose init fails (no such device, here
    and on a GPU host alike) prints the engine's message, stays on the CPU
    (default device 0) and gives the CPU's results."""
    import json
    import subprocess
    import sys
    r = subprocess.run([sys.executable, "-m", "tests.pyffi", "hip"], capture_output=True, text=True, timeout=240,
                       cwd=pyffi.tt.ROOT, env=dict(os.environ, THVM_HIP_DEVICE="99"))
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
    assert r.returncode == 0 and lines, r.stderr[-2000:]
    res = json.loads(lines[-1])
    assert res["default_device"] == [0, 0], res
    assert "requested hip backend unavailable; using cpu" in r.stderr
    for name, err in res["mlp"].items():
        assert err <= 1e-5, (name, err)
    assert res["mlp_hip_dispatches"] == 0
