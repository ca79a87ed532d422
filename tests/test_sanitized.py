"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

  pool_test     the buffer pool (pool.c) against the engine's buffer contract
                with a host-memory stand-in for the HIP runtime
                (tests/cpu/fake_hip.c): the 16383-id limit, idempotent frees,
                pool_reset(keep), the persistent floor, out-of-memory returning
                0, graph-held blocks kept out of the free lists until their
                graph is destroyed, and write/read round trips; no leak at
                shutdown.
  analyze_all   the device-free program analyses (kernel generator, lane
                classification, matrix-core and window recognizers, the merge
                of consecutive programs) over every lowered kernel of every
                committed trace, plus truncated programs and dangling
                operands.

Both are built with gcc (host code only; no device code is instrumented).
"""
import os
import subprocess

import pytest

from tests import tracetools as tt

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
CSRC = os.path.join(tt.ROOT, "tinyhvm_amd", "csrc")
CPU = os.path.join(tt.ROOT, "tests", "cpu")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all"]
CFLAGS = ["-std=gnu11", "-g", "-O1", "-Wall", "-Wno-unused-function", "-Wno-deprecated-declarations",
          "-D__HIP_PLATFORM_AMD__", "-I" + os.path.join(ROCM, "include"),
          "-I" + os.path.join(tt.ROOT, "include"), "-I" + CSRC]
ENV = dict(os.environ, ASAN_OPTIONS="abort_on_error=0:detect_leaks=1",
           UBSAN_OPTIONS="print_stacktrace=1")


def _build(out, sources, libs=()):
    cmd = ["gcc"] + CFLAGS + SAN + sources + list(libs) + ["-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]


def test_pool_contract_sanitized(tmp_path):
    exe = str(tmp_path / "pool_test")
    _build(exe, [os.path.join(CSRC, "pool.c"), os.path.join(CPU, "fake_hip.c"),
                 os.path.join(CPU, "pool_test.c")])
    r = subprocess.run([exe], capture_output=True, text=True, env=ENV, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr[-4000:]
    assert "checks passed" in r.stdout


def test_program_analysis_sanitized(tmp_path):
    from tinyhvm_amd import build
    blob = os.path.join(tt.ROOT, "_build", "static_kernels_blob.c")
    if not os.path.exists(blob):
        build.build_kernels()
    # the static-workspace object (hipcc, not instrumented: it holds no analysis code)
    objs = [os.path.join(tt.ROOT, "_build", os.path.splitext(h)[0] + ".o") for h in build.HIP_OBJECTS]
    if not all(os.path.exists(o) for o in objs):
        objs = build.build_hip_objects()
    exe = str(tmp_path / "analyze_all")
    srcs = [os.path.join(CSRC, f) for f in ("backend.c", "pool.c", "kgen.c", "rtc.c", "affine.c", "dense.c", "window.c", "chain.c", "replay.c")]
    _build(exe, srcs + [blob, os.path.join(CPU, "analyze_all.c")] + objs,
           ["-L" + os.path.join(ROCM, "lib"), "-lamdhip64", "-lhiprtc", "-lstdc++", "-lpthread", "-lm",
            "-Wl,-rpath," + os.path.join(ROCM, "lib")])
    traces = tt.fixtures() + sorted(
        os.path.join(tt.ROOT, "tinyhvm_amd", "workloads", f)
        for f in os.listdir(os.path.join(tt.ROOT, "tinyhvm_amd", "workloads")) if f.endswith(".trc"))
    r = subprocess.run([exe] + traces, capture_output=True, text=True, env=ENV, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr[-4000:]
    words = r.stdout.split("analyze_all:")[1].split()
    n, merged = int(words[0]), int(words[2])
    assert n > 300
    assert merged > 10, "only %d consecutive pairs merged" % merged
