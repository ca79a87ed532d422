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
