"""The kernel-boundary parity harness of the GPU tests, exercised on the CPU
with the oracle standing in for the device: every dispatch must then match
bit for bit, and every recorded reference output end to end."""
import ctypes as C

import pytest

from tests import tracetools as tt
from tests.test_gpu_parity import _oracle, kernel_parity


@pytest.mark.parametrize("path", tt.fixtures(), ids=lambda p: p.split("/")[-1])
def test_harness_on_oracle_device(path):
    ora = _oracle()
    be = ora.oracle_backend_ptr()
    be.contents.init()

    def read(live, buf, n):
        C.memmove(buf, ora.oracle_buf_ptr(live), n)

    try:
        kr, e2e = kernel_parity(be, read, lambda: 0, ora, path, tol_fn=lambda k: ("exact", 0.0))
    finally:
        be.contents.shutdown()
    assert kr and all(ok for _i, ok, _m in kr), [r for r in kr if not r[1]]
    assert all(ok for _i, ok, _m in e2e), [r for r in e2e if not r[1]]
