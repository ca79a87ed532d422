"""The engine itself driving the HIP backend: thvm_eval's scheduler, lowering
and dispatch calling `hip_backend` live, with no trace in between.

oracle/_ref/engine_live (tests/live/engine_live.c, built with the engine's
sources by `make -C oracle ref`) runs each workload twice in one process:
on the engine's CPU backend, then with hip_backend registered as the
engine's default device, the way the thvm_init branch for "hip" registers
it. Every buffer the workload reads back must agree: the same sequence and
sizes, and values within 1e-3 normwise (the order of the GPU's sums
differs). The reads are the workloads' losses, gradients, updated parameters
and outputs.
"""
import json
import os
import subprocess

import pytest

from tests import tracetools as tt

pytestmark = pytest.mark.gpu

EXE = os.path.join(tt.ROOT, "oracle", "_ref", "engine_live")
LIB = os.path.join(tt.ROOT, "tinyhvm_amd", "libthvm_hip.so")

CASES = [
    ("mlp", []),
    ("fused", [256, 1024]),
    ("linear", [128, 256, 96]),
    ("lenet", [8, 1]),
    ("convblock", [2, 8, 16]),
    ("adam", []),
    ("known", []),
]


@pytest.mark.skipif(not os.path.exists(EXE), reason="oracle/_ref/engine_live is built only where the "
                                                    "engine sources are present (make -C oracle ref)")
@pytest.mark.parametrize("workload,sizes", CASES, ids=[c[0] for c in CASES])
def test_engine_drives_hip_backend(workload, sizes):
    cmd = [EXE, LIB, workload] + [str(s) for s in sizes]
    print("running:", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=240)
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
    assert lines, "no result (exit %d): %s" % (r.returncode, r.stderr[-2000:])
    res = json.loads(lines[-1])
    print("%s: %d reads, worst %.2e, cpu %.2fs, gpu %.2fs" % (workload, res["reads"][0], res["worst"],
                                                             res["cpu_seconds"], res["gpu_seconds"]))
    assert res["reads"][0] == res["reads"][1] and res["reads"][0] > 0
    assert res["ok"] and r.returncode == 0, res
