"""The pooling-window and run-sum kernels (window.c), without a device.

- Every program of every committed trace that the window recognizer takes
  compiles with hipRTC for gfx950.
- The benchmark workloads route to them as intended: in the conv block at
  [64,64,56,56] the max-pool forward is a window max and the six batchnorm
  sums over [0,2,3] and the loss sum are run sums (the BN sums split over 16
  workgroups per channel, the loss sum over 1024: 1024 workgroups, all
  resident at once, so the partials combine in the launch); in LeNet-5 at batch 256 the
  two max-pools (and the row maxima of the softmax) are window maxes and the
  two convolution bias gradients are run sums. No other kernel of those steps
  is taken (a change to the recognizer that widens or narrows it shows here).
- The window max reads each window row with one 8-byte load and keeps the
  engine's order of the maximum; a run sum reads 16-byte vectors along the
  runs and combines the workgroups in the same launch.
- Shapes the recognizer must refuse: the fused forward's 8192 row sums (many
  outputs), short loops, and a sum whose loads are strided along the loop.
"""
import os
import re

import pytest

from tests import tracetools as tt
from tinyhvm_amd import _lib, trace

WL = os.path.join(tt.ROOT, "tinyhvm_amd", "workloads")


def _all_traces():
    return tt.fixtures() + sorted(os.path.join(WL, f) for f in os.listdir(WL) if f.endswith(".trc"))


def _routes(path):
    out = []
    n = 0
    for r in trace.read_trace(path):
        if r.tag != trace.UOP:
            continue
        a = _lib.window_analyze(trace.to_uop_kernel(r))
        if a:
            out.append((n, a[0], a[1]))
        n += 1
    return out


@pytest.mark.parametrize("path", _all_traces(), ids=lambda p: p.split("/")[-1])
def test_window_kernels_compile(path):
    for r in trace.read_trace(path):
        if r.tag == trace.UOP:
            k = trace.to_uop_kernel(r)
            if _lib.window_analyze(k):
                assert _lib.window_compile_check(k) > 0


def test_conv_block_routes():
    routes = _routes(os.path.join(WL, "convblock_b64.trc"))
    assert routes == [(2, 2, 16), (5, 2, 16), (13, 1, 1), (14, 2, 1024), (17, 2, 16), (18, 2, 16),
                      (21, 2, 16), (22, 2, 16)], routes


def test_lenet_routes():
    routes = _routes(os.path.join(WL, "lenet_b256.trc"))
    kinds = [(n, kind) for n, kind, _s in routes]
    assert kinds == [(3, 1), (6, 1), (13, 1), (18, 1), (36, 2), (43, 2)], routes


def test_window_max_source_shape():
    recs = [r for r in trace.read_trace(os.path.join(WL, "convblock_b64.trc")) if r.tag == trace.UOP]
    src = _lib.window_source(trace.to_uop_kernel(recs[13])).split('extern "C" __global__')[1]
    n_units = len(re.findall(r"const u32 o\d+_ =", src))
    # two adjacent windows per 16-byte load, two window rows per pair
    assert n_units >= 1 and src.count("(const v4f_*)") == 2 * n_units and "make_float2(a0_, a1_)" in src
    order = re.findall(r"e_ = v0_(\d)_\.([xyzw]); a(\d)_", src)
    # the engine's r order for each output: (ky, kx) = (0,0), (0,1), (1,0), (1,1)
    assert order[:4] == [("0", "x", "0"), ("0", "y", "0"), ("1", "x", "0"), ("1", "y", "0")]
    assert order[4:8] == [("0", "z", "1"), ("0", "w", "1"), ("1", "z", "1"), ("1", "w", "1")]
    src = _lib.window_source(trace.to_uop_kernel(recs[5]))
    assert "ld4nt_u(" in src and "comb_take(" in src and "_fin" not in src


def test_refused_shapes():
    fused = [r for r in trace.read_trace(os.path.join(WL, "fused_8192x8192.trc")) if r.tag == trace.UOP]
    assert _lib.window_analyze(trace.to_uop_kernel(fused[0])) is None      # 8192 outputs
    mlp = [r for r in trace.read_trace(os.path.join(WL, "mlp_64x784x128x10.trc")) if r.tag == trace.UOP]
    for r in mlp:
        k = trace.to_uop_kernel(r)
        a = _lib.window_analyze(k)
        if a and a[0] == 2:
            raise AssertionError("a run sum in the MLP, whose sums run across rows with stride")
