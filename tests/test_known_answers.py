"""The engine's own known-answer tests, on the oracle and on the GPU.

tests/golden/known.trc restates them (tests/golden/capture.c wl_known: the
same engine API calls on the same inputs, each case behind a "known.<case>"
mark, ending in the readback the test checks). Replaying it must give the
values the tests expect:

  conv         [7,9,13,15]   test/archive/test_tensor_nn_layers.m:19-36 (tol 1e-3)
  pool         4             test/archive/test_tensor_nn_layers.m:39-50
  bn_eval      y0 1, y3 4    test/archive/test_tensor_nn_layers.m:52-67 (tol 5e-3)
  relu_linear  [0,2.6,0,5]   test/archive/test_readme_verify.m:22-41 (tol 1e-3)
  multiview    160           test/archive/test_lower_multiview_kernel.m:14-33 (exact)
  dtype_*      [7,-16], [6], [1,20,3], [1,0]   test/archive/test_dtype_cast.m:28-56

Four more fail on the engine itself, on its CPU backend, upstream of any
backend: built from their own sources (`make -C oracle known`) they print
  test_cpu_metal_cmp      [0.0000, 0.0000]  (expect [20, 86])
  test_fused_reduce       total: 0.0        (expect 165888)
  test_dup_chain          got 9, 9, 9, 9    (expect 5)
  test_mm_dup_2arm        dw ptr NULL       (no gradient tensor)
(their low-level ASSIGN of a lazy sum leaves the destination unwritten, and
the DUP-chain gradient counts arms twice). The replay must reproduce exactly
those outputs, and nothing is read back where the engine reads nothing.
"""
import ctypes as C

import numpy as np
import pytest

from tests import tracetools as tt
from tinyhvm_amd import _lib, trace

PATH = tt.fixtures("known.trc")[0]


def _reads(backend, read_fn, sync_fn=None):
    """case -> list of (trace id, bytes) read back in that case."""
    recs = trace.read_trace(PATH)
    sizes = {}
    out = {}
    case = None
    rp = tt.Replay(PATH, backend)
    try:
        for i, r in enumerate(recs):
            if r.tag == trace.ALLOC:
                sizes[r.f["id"]] = r.f["bytes"]
            rp.run(i, i + 1)
            if r.tag == trace.MARK:
                case = r.f["text"]
            elif r.tag == trace.READ:
                n = r.f["bytes"]
                buf = (C.c_uint8 * max(n, 4))()
                read_fn(rp.live(r.f["id"]), buf, n)
                out.setdefault(case, []).append((r.f["id"], bytes(buf)[:n]))
        if sync_fn:
            assert sync_fn() == 0
    finally:
        rp.close()
    return out


def _f32(b):
    return np.frombuffer(b, np.float32)


def _i32(b):
    return np.frombuffer(b, np.int32)


def check_known(reads):
    last = {k: v[-1][1] for k, v in reads.items()}
    assert np.allclose(_f32(last["known.conv"]), [7, 9, 13, 15], atol=1e-3, rtol=0)
    assert abs(_f32(last["known.pool"])[0] - 4.0) <= 1e-3
    bn = _f32(last["known.bn_eval"])
    assert abs(bn[0] - 1.0) <= 5e-3 and abs(bn[3] - 4.0) <= 5e-3
    assert np.allclose(_f32(last["known.relu_linear"]), [0, 2.6, 0, 5.0], atol=1e-3, rtol=0)
    assert _f32(last["known.multiview"])[0] == 160.0
    assert list(_i32(last["known.dtype_add_i32"])) == [7, -16]
    assert list(_i32(last["known.dtype_sum_i32"])) == [6]
    assert list(_i32(last["known.dtype_where_i32"])) == [1, 20, 3]
    assert list(_i32(last["known.dtype_argmax"])) == [1, 0]
    # the engine's own failures, reproduced as its programs print them
    assert _f32(last["known.fused_reduce"])[0] == 0.0
    assert list(_f32(last["known.mul_sum"])) == [0.0, 0.0]
    assert list(_f32(last["known.dup_chain"])) == [9.0, 9.0, 9.0, 9.0]
    assert "known.mm_dup" not in reads and "known.readme_grad" not in reads


def test_known_answers_on_the_oracle():
    ora = tt.oracle()
    be = ora.oracle_backend_ptr()
    be.contents.init()

    def read(live, buf, n):
        C.memmove(buf, ora.oracle_buf_ptr(live), n)

    try:
        check_known(_reads(be, read))
    finally:
        be.contents.shutdown()


@pytest.mark.gpu
def test_known_answers_on_the_gpu():
    L = _lib.lib()
    assert L.thvm_hip_init() == 0, "HIP backend failed to initialise"
    try:
        check_known(_reads(L.thvm_hip_backend(), L.thvm_hip_buf_read, L.thvm_hip_synchronize))
    finally:
        L.thvm_hip_shutdown()
