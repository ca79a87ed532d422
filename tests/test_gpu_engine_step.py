"""The engine's own training step driving hip_backend, timed (no trace).

oracle/_ref/engine_live in timing mode runs LeNet-5 at batch 256 and the
2-layer MLP at batch 64 through thvm_eval with hip_backend as the default
device (the scheduler's dispatch loop, src/schedule/_.c:2268-2411): two
warm-up steps, then timed steps, each including the engine's host work and
the step's read-backs (LeNet: its loss and ten updated parameters; MLP: its
loss and two weight gradients). Every backend slot is wrapped to count the
host's waits on the stream inside it:
  - no slot but buf_read (the engine's sync point) may wait: the dispatches,
    uploads, copies, frees and pool resets of a step are all enqueued
    without a host synchronization;
  - the waits per step are at most the read-backs per step.
The same steps on the engine's CPU backend give the baseline the rate is
printed beside.
"""
import json
import os
import subprocess

import pytest

from tests import tracetools as tt

pytestmark = pytest.mark.gpu

EXE = os.path.join(tt.ROOT, "oracle", "_ref", "engine_live")
LIB = os.path.join(tt.ROOT, "tinyhvm_amd", "libthvm_hip.so")

CASES = [("lenet", 20, 256), ("mlp", 50, 64)]


@pytest.mark.timeout(400)
@pytest.mark.skipif(not os.path.exists(EXE), reason="oracle/_ref/engine_live is built only where the "
                                                    "engine sources are present (make -C oracle ref)")
@pytest.mark.parametrize("workload,steps,batch", CASES, ids=[c[0] for c in CASES])
def test_engine_step_has_no_sync_between_dispatches(workload, steps, batch):
    cmd = [EXE, LIB, "time", workload, str(steps), str(batch)]
    print("running:", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=380)
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
    assert lines, "no result (exit %d): %s" % (r.returncode, r.stderr[-2000:])
    res = json.loads(lines[-1])
    print("engine step:", json.dumps(res), flush=True)
    g = res["gpu"]
    assert r.returncode == 0 and g["steps_per_s"] > 0
    assert g["waits_outside_reads"] == 0, "a slot other than buf_read waited on the stream: %s" % g["wait_slot"]
    assert g["reads_per_step"] > 0 and g["host_waits_per_step"] <= g["reads_per_step"]
    assert g["dispatches_per_step"] > 10
    assert res["cpu"]["steps_per_s"] > 0
