"""The CPU baseline's replayer (oracle/_ref/ref_replay) reproduces the engine.

ref_replay times the engine's own CPU backend (src/backend/cpu/) on a kernel
trace. With --guard every buffer sits at the start of a zero-filled guard
region, so kernels whose masked loads leave their buffer (the zero-padded
convolutions of LeNet and the conv block) run on the engine's interpreter
unchanged. Its --check mode replays a fixture and compares every SNAPSHOT (the
engine's own outputs, recorded by tests/golden/capture.c) with the live buffer
at that point, bit for bit: the baseline that bench.py times computes exactly
what the engine computes.
"""
import os
import subprocess

import pytest

from tests import tracetools as tt

EXE = os.path.join(tt.ROOT, "oracle", "_ref", "ref_replay")

# the fixtures whose every record the engine's CPU backend implements
# (assign.trc needs contiguify and adam.trc adam_step, slots that backend lacks)
FIXTURES = ["lenet_b2.trc", "convblock_2x4x8.trc", "convblock_1x64x8.trc", "pooltie_2x4x16.trc",
            "mlp_64x784x128x10.trc", "fused_64x256.trc", "linear_33x300x40.trc",
            "longreduce_4x20000.trc", "known.trc", "dtypes.trc", "legacy.trc", "rs_convblock_2x4x8.trc"]


@pytest.mark.skipif(not os.path.exists(EXE), reason="oracle/_ref/ref_replay is built only where the "
                                                    "engine sources are present (make -C oracle ref)")
@pytest.mark.parametrize("name", FIXTURES)
def test_guarded_engine_replay_matches_snapshots(name):
    r = subprocess.run([EXE, os.path.join(tt.GOLDEN, name), "x", "-", "1", "--check", "--guard"],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert '"check_mismatches": 0' in r.stdout


LIVE = os.path.join(tt.ROOT, "oracle", "_ref", "engine_live")


@pytest.mark.skipif(not os.path.exists(LIVE), reason="oracle/_ref/engine_live is built only where the "
                                                     "engine sources are present (make -C oracle ref)")
def test_engine_cpu_leg_runs_guarded():
    """The CPU leg of the engine-driven step timing (engine_live with "-" for
    the library): LeNet's zero-padded convolutions run on the engine's own
    interpreter over guard regions, and the step closes."""
    import json
    r = subprocess.run([LIVE, "-", "time", "lenet", "1", "4"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    res = json.loads([ln for ln in r.stdout.splitlines() if ln.startswith("{")][-1])
    assert res["cpu"]["steps_per_s"] > 0 and res["gpu"]["steps_per_s"] == 0
