"""The contraction recognizer (tinyhvm_amd/csrc/dense.c) on the committed
traces, without a GPU: every matmul and convolution kernel the engine lowers
is recognized with the GEMM shape its workload implies, nothing else is, and
the generated matrix-core kernels compile for gfx950."""
import os

import pytest

from tests import tracetools as tt
from tinyhvm_amd import _lib, trace


def _kernels(name):
    return [(r.f["full_dims"][:r.f["full_rank"]], trace.to_uop_kernel(r))
            for r in trace.read_trace(os.path.join(tt.GOLDEN, name)) if r.tag == trace.UOP]


@pytest.fixture(autouse=True)
def force_dense(monkeypatch):
    # size heuristics off: the fixtures are small
    monkeypatch.setenv("THVM_HIP_DENSE_FORCE", "1")


def _analyze_forced(k):
    # thvm_hip_dense_analyze reads the environment once per process; the
    # forced setting is exported by conftest for the whole CPU run
    return _lib.dense_analyze(k)


def test_matmul_forward_and_backward_shapes():
    ks = _kernels("linear_33x300x40.trc")
    shapes = [_analyze_forced(k) for _full, k in ks]
    # y = X @ W (M=33, N=40, K=300); dX = G @ W^T (33, 300, 40); dW = X^T @ G (300, 40, 33)
    assert shapes[0][:3] == (33, 40, 300)
    assert (33, 300, 40) in [s[:3] for s in shapes if s]
    assert (300, 40, 33) in [s[:3] for s in shapes if s]
    # bias+relu and the relu mask are not contractions
    assert sum(1 for s in shapes if s is None) == 3


def test_conv_kernels_are_contractions():
    got = {tuple(full): _analyze_forced(k) for full, k in _kernels("convblock_2x4x8.trc")}
    # conv3x3 forward: M = B*H*W = 128, N = Co = 4, K = Ci*3*3 = 36 (padded views)
    assert got[(2, 1, 4, 8, 8, 4, 3, 3)][:3] == (128, 4, 36)
    # weight gradient: M = Ci*3*3 = 36, N = Co = 4, K = B*H*W = 128
    assert got[(4, 4, 3, 3, 2, 8, 8)][:3] == (36, 4, 128)


def test_reductions_without_a_product_are_not_contractions():
    for name in ("fused_64x256.trc", "dtypes.trc"):
        for _full, k in _kernels(name):
            assert _analyze_forced(k) is None


@pytest.mark.parametrize("name", ["linear_33x300x40.trc", "convblock_2x4x8.trc", "lenet_b2.trc"])
def test_matrix_core_kernels_compile(name):
    n = 0
    for _full, k in _kernels(name):
        if _analyze_forced(k):
            assert _lib.dense_compile_check(k) > 0
            n += 1
    assert n > 0
