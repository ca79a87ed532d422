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


@pytest.mark.parametrize("name", ["convblock_2x4x8.trc", "lenet_b2.trc", "linear_33x300x40.trc"])
def test_prefix_oracle_is_exact(name):
    """The prefix check of large kernels: the oracle run over a grid of T
    computes exactly the first T outputs of the full run (group reductions,
    convolutions and matmuls alike), bit for bit."""
    ora = _oracle()
    be = ora.oracle_backend_ptr()
    be.contents.init()

    def read(live, buf, n):
        C.memmove(buf, ora.oracle_buf_ptr(live), n)

    def prefix(k):
        total = k.grid[0] if k.local_size > 0 else k.grid[0] * k.grid[1] * k.grid[2]
        return max(1, total // 3) if total > 3 else None

    try:
        kr, _e2e = kernel_parity(be, read, lambda: 0, ora, tt.fixtures(name)[0],
                                 tol_fn=lambda k: ("exact", 0.0), prefix_fn=prefix)
    finally:
        be.contents.shutdown()
    assert sum(1 for _i, _ok, m in kr if "first" in m) >= 3
    assert kr and all(ok for _i, ok, _m in kr), [r for r in kr if not r[1]]
