"""The kernel-boundary parity harness of the GPU tests, exercised on the CPU
with the oracle standing in for the device: every dispatch must then match
bit for bit, and every recorded reference output end to end."""
import ctypes as C

import numpy as np
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


@pytest.mark.parametrize("name", ["convblock_2x4x8.trc", "lenet_b2.trc", "linear_33x300x40.trc"])
def test_sampled_oracle_is_exact(name):
    """The sampled check of large kernels: the oracle run over a list of gids
    stores exactly those gids' outputs of the full run, bit for bit; the
    device output is filled with the sentinel before the dispatch and must
    come out fully written."""
    ora = _oracle()
    be = ora.oracle_backend_ptr()
    be.contents.init()
    rng = np.random.default_rng(3)

    def read(live, buf, n):
        C.memmove(buf, ora.oracle_buf_ptr(live), n)

    def write(live, data, n):
        be.contents.buf_write(live, data, n)

    def sample(k):
        total = k.grid[0] if k.local_size > 0 else k.grid[0] * k.grid[1] * k.grid[2]
        if total < 8:
            return None
        return np.concatenate([[0, total - 1], rng.choice(total, total // 3, replace=False)])

    try:
        kr, _e2e = kernel_parity(be, read, lambda: 0, ora, tt.fixtures(name)[0],
                                 tol_fn=lambda k: ("exact", 0.0), sample_fn=sample, write_fn=write)
    finally:
        be.contents.shutdown()
    assert sum(1 for _i, _ok, m in kr if "every output written" in m) >= 3
    assert kr and all(ok for _i, ok, _m in kr), [r for r in kr if not r[1]]


def test_sampled_check_catches_an_unwritten_output():
    """A device that leaves one output of a sampled kernel unwritten fails the
    sentinel check even where the sample does not look."""
    ora = _oracle()
    be = ora.oracle_backend_ptr()
    be.contents.init()
    proto = type(be.contents.dispatch_uop_kernel)
    orig_ptr = C.cast(be.contents.dispatch_uop_kernel, C.c_void_p).value
    orig = proto(orig_ptr)
    state = {"hit": 0}

    def lossy(out, leaves, n, k, key):
        orig(out, leaves, n, k, key)
        total = k.contents.grid[0] * k.contents.grid[1] * k.contents.grid[2]
        if total >= 64 and not state["hit"]:
            state["hit"] = 1
            p = ora.oracle_buf_ptr(out)
            C.memmove(p + 4 * (total - 1), (C.c_uint32 * 1)(0xFFFFFFFF), 4)

    cb = proto(lossy)
    be.contents.dispatch_uop_kernel = cb

    def read(live, buf, n):
        C.memmove(buf, ora.oracle_buf_ptr(live), n)

    def write(live, data, n):
        be.contents.buf_write(live, data, n)

    try:
        kr, _e2e = kernel_parity(be, read, lambda: 0, ora, tt.fixtures("convblock_2x4x8.trc")[0],
                                 tol_fn=lambda k: ("exact", 0.0), sample_fn=lambda k: np.array([0]),
                                 write_fn=write)
    finally:
        be.contents.dispatch_uop_kernel = proto(orig_ptr)
        be.contents.shutdown()
    assert state["hit"]
    bad = [r for r in kr if not r[1]]
    # the planted hole is caught at its own dispatch (the sentinel it leaves
    # then flows on into later kernels' inputs)
    assert bad and "; 1 outputs never written" in bad[0][2], bad[:3]
