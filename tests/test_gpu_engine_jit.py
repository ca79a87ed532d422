"""Capture and replay of a training step that the engine itself drives: the
Metal backend's JIT record/replay (src/backend/metal/jit.m:24-631, used at
test/archive/test_jit_dense.m:95-157) done with the HIP backend's graphs.

oracle/_ref/engine_live in jit mode (tests/live/engine_live.c) makes its
context with thvm_init("hip"), then runs N training steps through thvm_eval
(eager), and from the same initial parameters captures one thvm_eval step
into a HIP graph and launches it N times; before each step or launch it
writes that step's labels into the persistent one-hot tensor, after each it
reads the loss the step assigns to a persistent tensor. Every loss and every
final parameter of the graph launches must equal the eager steps' bit for
bit, the parameters must have moved, and the graph launches, which skip the
engine's host work, must be faster than the eager steps.
"""
import json
import os
import subprocess

import pytest

from tests import tracetools as tt

pytestmark = pytest.mark.gpu

EXE = os.path.join(tt.ROOT, "oracle", "_ref", "engine_live")
LIB = os.path.join(tt.ROOT, "tinyhvm_amd", "libthvm_hip.so")

CASES = [("lenet", 12, 256), ("mlp", 30, 64)]


@pytest.mark.timeout(300)
@pytest.mark.skipif(not os.path.exists(EXE), reason="oracle/_ref/engine_live is built only where the "
                                                    "engine sources are present (make -C oracle ref)")
@pytest.mark.parametrize("workload,steps,batch", CASES, ids=[c[0] for c in CASES])
def test_graph_replays_equal_engine_steps(workload, steps, batch):
    cmd = [EXE, LIB, "jit", workload, str(steps), str(batch)]
    print("running:", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=280)
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
    assert lines, "no result (exit %d): %s" % (r.returncode, r.stderr[-2000:])
    res = json.loads(lines[-1])
    print("engine jit:", json.dumps(res), flush=True)
    assert res["losses_equal"], "graph launches gave other losses than the engine's steps"
    assert res["params_equal"], "graph launches left other parameters than the engine's steps"
    assert res["params_moved"] and res["ok"] and r.returncode == 0, res
    assert res["graph"]["steps_per_s"] > res["eager"]["steps_per_s"], res
