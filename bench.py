"""Benchmark of the HIP backend on the TinyHVM kernel-dispatch hot path.

A step is one replay of the engine's recorded Backend calls for the workload
(kernel trace, inputs already resident in HBM): for the fused workload that is
y = sum(relu(a*b + c), -1) (one group-reduce kernel) and its gradient
dA = (a*b + c > 0) * b (one elementwise kernel), a/b/c ~ N(0,1) of [8192,8192] f32.

value  = algorithmic HBM bytes of one step / time per step (GB/s).
roofline: the dominant kernel's algorithmic bytes per launch / its average
          launch time, from HIP events recorded on the backend's stream.
cpu_baseline: the engine's own CPU backend (oracle/_ref/ref_replay, built from
          the engine sources) replaying the same trace on one host core.
"""
import argparse
import ctypes as C
import json
import os
import shutil
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from tinyhvm_amd import _lib  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_F32_PEAK_TFLOPS = 157.3
METRIC = "fused-kernel HBM GB/s (% peak); f32 matmul TFLOPS; LeNet-5 train steps/sec"

WORKLOADS = {
    "fused": {
        "trace": os.path.join(ROOT, "tinyhvm_amd", "workloads", "fused_8192x8192.trc"),
        "step_marks": ("fused.fwd", None),
        "kernels": {
            # mark -> algorithmic HBM bytes of the kernel that follows it
            "fused.fwd": 3 * 8192 * 8192 * 4 + 8192 * 4,
            "fused.bwd": 4 * 8192 * 8192 * 4,
        },
        "dominant": "fused.bwd",
        "config": {"workload": "fused elementwise+reduce f32: y = sum(relu(a*b+c), -1) and dA",
                   "shape": [8192, 8192], "dist": "N(0,1)"},
        "cpu_sample": "full fused fwd+bwd step at [8192,8192], 1 replay",
        "profile": "fused_8192x8192.md",
    },
}


class Hip:
    """hipEvent timing on the backend's stream (libamdhip64 via ctypes)."""

    def __init__(self, stream):
        self.h = C.CDLL("libamdhip64.so")
        self.stream = C.c_void_p(stream)
        self.h.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.h.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.h.hipEventSynchronize.argtypes = [C.c_void_p]
        self.h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.h.hipEventDestroy.argtypes = [C.c_void_p]

    def event(self):
        e = C.c_void_p()
        assert self.h.hipEventCreate(C.byref(e)) == 0
        return e

    def record(self, e):
        assert self.h.hipEventRecord(e, self.stream) == 0

    def ms(self, a, b):
        self.h.hipEventSynchronize(b)
        out = C.c_float()
        assert self.h.hipEventElapsedTime(C.byref(out), a, b) == 0
        return out.value


def measured_traffic(profile, kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 summary
    (its ```json block), or None when no counter run has been recorded."""
    path = os.path.join(ROOT, "profiles", profile)
    if not os.path.exists(path):
        return None
    text = open(path).read()
    if "```json" not in text:
        return None
    block = text.split("```json", 1)[1].split("```", 1)[0]
    return json.loads(block).get("traffic_bytes", {}).get(kernel)


def find_mark(L, t, text, start=0):
    return L.thvm_trace_find_mark(t, text.encode(), start)


def cpu_baseline(wl, lo_mark):
    exe = os.path.join(ROOT, "oracle", "_ref", "ref_replay")
    if not os.path.exists(exe):
        return None
    cmd = [exe, wl["trace"], lo_mark, "-", "1"]
    if shutil.which("taskset"):
        cmd = ["taskset", "-c", "0"] + cmd
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    if r.returncode != 0:
        sys.stderr.write(r.stderr)
        return None
    res = json.loads(r.stdout.strip().splitlines()[-1])
    step_bytes = sum(wl["kernels"].values())
    return {"value": step_bytes / res["per_rep"] / 1e9, "unit": "GB/s", "cores": 1,
            "kind": "reference", "sample": wl["cpu_sample"], "seconds": res["per_rep"]}


def copy_calibration(nbytes=256 << 20, reps=5):
    """A plain copy kernel of known size through the same generated-kernel
    path (out[i] = src[i]): the reference reading for the HBM byte counters."""
    from tinyhvm_amd import abi
    L = _lib.lib()
    if L.thvm_hip_init() != 0:
        raise SystemExit("HIP backend failed to initialise")
    n = nbytes // 4
    k = abi.UOpKernel()
    k.n_ops, k.n_leaves, k.n_bufs, k.rank = 3, 1, 2, 1
    k.full_shape.rank, k.full_shape.dims[0] = 1, n
    k.grid[0], k.grid[1], k.grid[2] = n, 1, 1
    k.ops[0].type = abi.KOP_GID
    k.ops[1].type = abi.KOP_LOAD
    k.ops[1].arg[0], k.ops[1].imm.u = 0, 1
    k.ops[2].type = abi.KOP_STORE
    k.ops[2].arg[0], k.ops[2].arg[1] = 0, 1
    src, dst = L.thvm_hip_buf_alloc(nbytes), L.thvm_hip_buf_alloc(nbytes)
    leaves = (C.c_uint32 * 1)(src)
    L.thvm_hip_dispatch_uop_kernel(dst, leaves, 1, C.byref(k), 0)
    assert L.thvm_hip_synchronize() == 0
    hip = Hip(L.thvm_hip_stream())
    e0, e1 = hip.event(), hip.event()
    hip.record(e0)
    for _ in range(reps):
        L.thvm_hip_dispatch_uop_kernel(dst, leaves, 1, C.byref(k), 0)
    hip.record(e1)
    ms = hip.ms(e0, e1) / reps
    assert L.thvm_hip_synchronize() == 0
    L.thvm_hip_shutdown()
    print(json.dumps({"copy_calibration_bytes_read": nbytes, "bytes_written": nbytes, "reps": reps,
                      "ms_per_copy": round(ms, 4), "GBps": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="fused")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a 256 MiB copy kernel (HBM counter calibration)")
    args = ap.parse_args()
    if args.calibrate_copy:
        copy_calibration()
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(use --gpus 1)", file=sys.stderr)
        sys.exit(2)
    wl = WORKLOADS[args.workload]
    L = _lib.lib()
    if L.thvm_hip_init() != 0:
        raise SystemExit("HIP backend failed to initialise")
    be = L.thvm_hip_backend()
    t = L.thvm_trace_load(wl["trace"].encode())
    if not t:
        raise SystemExit("cannot load %s" % wl["trace"])
    n = L.thvm_trace_count(t)
    lo = find_mark(L, t, wl["step_marks"][0])
    hi = n if wl["step_marks"][1] is None else find_mark(L, t, wl["step_marks"][1], lo)
    SKIP_READS = 1
    # setup: allocate and upload the inputs (not timed)
    L.thvm_trace_replay(t, be, 0, lo, 0)
    L.thvm_trace_drop_gen_cache(t)
    assert L.thvm_hip_synchronize() == 0
    print("setup done: %d records, step = records [%d, %d)" % (n, lo, hi), file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)
    assert L.thvm_hip_synchronize() == 0

    hip = Hip(L.thvm_hip_stream())
    # pass 1: whole steps, no per-kernel events (the reported value)
    e0, e1 = hip.event(), hip.event()
    assert L.thvm_hip_synchronize() == 0
    t0 = time.perf_counter()
    hip.record(e0)
    for _ in range(args.steps):
        L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)
    hip.record(e1)
    assert L.thvm_hip_synchronize() == 0
    wall = time.perf_counter() - t0
    gpu_ms = hip.ms(e0, e1)
    print("timed %d steps: %.3f ms/step wall, %.3f ms/step on the stream"
          % (args.steps, wall / args.steps * 1e3, gpu_ms / args.steps), file=sys.stderr, flush=True)
    # pass 2: the same steps split at the workload's marks, with events around
    # each kernel's records on the backend stream
    marks = sorted((find_mark(L, t, m, lo), m) for m in wl["kernels"])
    bounds = []
    for i in range(len(marks)):
        a = marks[i][0]
        b = marks[i + 1][0] if i + 1 < len(marks) else hi
        u = next(j for j in range(a, b) if L.thvm_trace_tag(t, j) in (7, 8))  # the dispatch
        bounds.append((a, u, b, marks[i][1]))
    ev = [(hip.event(), hip.event()) for _ in bounds]
    k_ms = {m: 0.0 for m in wl["kernels"]}
    for _ in range(args.steps):
        for (a, u, b, m), (ea, eb) in zip(bounds, ev):
            L.thvm_trace_replay(t, be, a, u, SKIP_READS)
            hip.record(ea)
            L.thvm_trace_replay(t, be, u, u + 1, SKIP_READS)
            hip.record(eb)
            L.thvm_trace_replay(t, be, u + 1, b, SKIP_READS)
        for (a, u, b, m), (ea, eb) in zip(bounds, ev):
            k_ms[m] += hip.ms(ea, eb)
    assert L.thvm_hip_synchronize() == 0
    step_s = wall / args.steps
    step_bytes = sum(wl["kernels"].values())
    value = step_bytes / step_s / 1e9
    dom = wl["dominant"]
    dom_ms = k_ms[dom] / args.steps
    achieved = wl["kernels"][dom] / (dom_ms * 1e-3) / 1e9
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": wl["config"],
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(wl["profile"], dom),
                     "kernel": dom},
        "kernels_ms": {m: round(v / args.steps, 4) for m, v in k_ms.items()},
        "gpu_ms_per_step": round(gpu_ms / args.steps, 4),
    }
    L.thvm_trace_release(t, be)
    L.thvm_trace_free(t)
    L.thvm_hip_shutdown()
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(wl, wl["step_marks"][0])
    print(json.dumps(out))


if __name__ == "__main__":
    main()
