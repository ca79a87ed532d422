"""Benchmark of the HIP backend on TinyHVM's kernel-dispatch hot path.

A step is one replay of the engine's recorded Backend calls for a workload
(a kernel trace; inputs already resident in HBM, results not read back):

  fused   y = sum(relu(a*b + c), -1) and dA = (a*b + c > 0) * b, a/b/c ~ N(0,1)
          [8192,8192] f32 (one group-reduce kernel + one elementwise kernel).
          This is the headline: `value` = algorithmic HBM bytes / step time.
  matmul  y = relu(X @ W + b), dX = G @ W^T, dW = X^T @ G at 4096^3 f32
          (three matrix-core contractions + three elementwise kernels):
          TFLOP/s = GEMM FLOPs / step time.
  lenet   one LeNet-5 training step at batch 256 (forward, backward, SGD
          through ASSIGN: 54 kernels): steps/s.
  convblock  conv3x3 64->64 pad 1, batchnorm (train), relu, maxpool 2, sum
          loss, and the backward to dW and dX, x [64,64,56,56] ~ N(0,1)
          (28 kernels): TFLOP/s = the three convolutions' FLOPs / step time.
  mlp     2-layer MLP x [64,784] -> 128 -> 10, relu, softmax cross-entropy,
          forward and backward to dW1, dW2 (20 kernels): steps/s (latency-bound).

lenet, mlp and convblock are also captured once into a HIP graph and timed as
graph launches (one launch = one whole step): `graph_value` beside `value`
(the replayed step).

Warmup: untimed replays of the step before the timed ones, at least
--warmup of them and at least WARM_MIN_S of them back to back after the
first (which compiles), as far as the backend's buffer ids allow;
`warmup_replays` says how many ran. The timed region is always exactly
--steps replays.

roofline: the dominant kernel's algorithmic bytes (or FLOPs) per launch / its
average duration, from HIP events on the backend's stream: around that one
dispatch for the HBM-bound kernels, around the contraction's main kernel
alone for the matrix-core ones (thvm_hip_time_contraction; the kernel that
rocprof's statistics name, without the operand pack or split-K sum kernel of
the same dispatch, which `kernels_ms` includes and `main_kernels_ms` does
not); `traffic` comes from the committed rocprofv3 counter summary.
cpu_baseline: the engine's own CPU backend (oracle/_ref/ref_replay, built from
the engine sources) on one host core, on the same trace or a stated slice;
LeNet and the conv block replay with every buffer in a zero-filled guard
region, since the engine's interpreter loads masked pad elements before the
mask discards them.

lenet_engine, mlp_engine: the same training steps driven by the engine itself
(thvm_eval on a context made by thvm_init("hip"); oracle/_ref/engine_live in
a child process): the rate a user of the engine gets, host work included,
with the host's stream waits per step counted beside the step's read-backs.

lenet_engine_graph, mlp_engine_graph: such an engine-driven step captured
once into a HIP graph and launched for every later step with new labels
written in between (the Metal backend's JIT record/replay role): steps/s with
the label write and the loss read, checked bit for bit against the same
number of eager engine steps.
"""
import argparse
import ctypes as C
import json
import os
import platform
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
WL = os.path.join(ROOT, "tinyhvm_amd", "workloads")
F4096 = 2 * 4096 ** 3
FCONV = 2 * 64 * 64 * 64 * 56 * 56 * 9          # one 3x3 64->64 conv over [64,64,56,56]
TAG_UOP, TAG_RS = 7, 8
TAG_ALLOC = 1
# buffer ids the backend hands out before a pool_reset recycles them (the
# engine's epoch table ends there, src/tinyhvm.h:720); every replay of a step
# allocates its temporaries afresh
MAX_BUFFER_IDS = 16383
# untimed warmup of each workload: at least this long of back-to-back step
# replays (as well as the --warmup count)
WARM_MIN_S = 0.05
SKIP_READS = 1

WORKLOADS = {
    "fused": {
        "trace": os.path.join(WL, "fused_8192x8192.trc"),
        "step": ("fused.fwd", None),
        # dispatch ordinal within the step -> (name, algorithmic bytes or FLOPs)
        "kernels": {0: ("fused.fwd", 3 * 8192 * 8192 * 4 + 8192 * 4),
                    1: ("fused.bwd", 4 * 8192 * 8192 * 4)},
        "unit": "GB/s", "bound": "hbm", "dominant": "fused.bwd",
        "config": {"workload": "fused elementwise+reduce f32: y = sum(relu(a*b+c), -1) and its "
                               "gradient dA = (a*b+c > 0) * b", "shape": [8192, 8192],
                   "dist": "N(0,1)", "kernels_per_step": 2},
        "profile": "fused_8192x8192.md",
        "cpu": {"exe": "oracle/_ref/ref_replay", "kind": "reference",
                "trace": os.path.join(WL, "fused_8192x8192.trc"), "marks": ("fused.fwd", "-"), "reps": 2,
                "sample": "the full step (fwd+bwd) at [8192,8192], 2 replays"},
    },
    "matmul": {
        "trace": os.path.join(WL, "linear_4096.trc"),
        "step": ("linear.fwd", None),
        "kernels": {0: ("gemm.fwd", F4096), 3: ("gemm.dx", F4096), 5: ("gemm.dw", F4096)},
        "unit": "TFLOP/s", "bound": "mfma", "dominant": "gemm.fwd",
        "config": {"workload": "dense f32 matmul + bias + relu (linear forward) and backward "
                               "dX, dW", "shape": [4096, 4096, 4096], "dist": "U(-1,1)",
                   "kernels_per_step": 6},
        "profile": "matmul_4096.md",
        "cpu": {"exe": "oracle/_ref/ref_replay", "kind": "reference",
                "trace": os.path.join(WL, "linear_8x4096x4096.trc"),
                "marks": ("linear.fwd", "linear.bwd.dx"), "flops": 2 * 8 * 4096 * 4096, "reps": 3,
                "sample": "forward (GEMM + bias + relu) on an 8-row slice of X (8x4096 @ 4096x4096), "
                          "the same kernels, 3 replays; GEMM throughput is linear in the rows"},
    },
    "lenet": {
        "trace": os.path.join(WL, "lenet_b256.trc"),
        "step": ("lenet.step", "lenet.end"),
        "kernels": {},
        "unit": "steps/s", "bound": None, "dominant": None, "graph": True,
        "config": {"workload": "LeNet-5 training step f32 (conv5x5 pad2 -> 6, relu, maxpool2, "
                               "conv5x5 -> 16, relu, maxpool2, fc 400-120-84-10, softmax CE, "
                               "backward, SGD via ASSIGN)", "batch": 256,
                   "input": "U(0,1) [256,1,28,28]", "kernels_per_step": 54},
        "cpu": {"exe": "oracle/_ref/ref_replay", "kind": "reference", "args": ["--guard"],
                "trace": os.path.join(WL, "lenet_b256.trc"), "marks": ("lenet.step", "lenet.end"),
                "reps": 1,
                "sample": "one training step at batch 256 on the engine's CPU backend, its buffers "
                          "placed in zero-filled guard regions (its interpreter loads masked pad "
                          "elements before discarding them)"},
    },
    "mlp": {
        "trace": os.path.join(WL, "mlp_64x784x128x10.trc"),
        "step": ("mlp.fwd", None),
        "kernels": {},
        "unit": "steps/s", "bound": None, "dominant": None, "graph": True,
        "config": {"workload": "2-layer MLP f32 forward + backward: x [64,784] ~ N(0,1), W1 [784,128], "
                               "W2 [128,10] Kaiming-uniform, relu, softmax cross-entropy; outputs loss, "
                               "dW1, dW2", "batch": 64, "kernels_per_step": 20},
        "cpu": {"exe": "oracle/_ref/ref_replay", "kind": "reference",
                "trace": os.path.join(WL, "mlp_64x784x128x10.trc"), "marks": ("mlp.fwd", "-"), "reps": 60,
                "sample": "the full step, 60 replays (the engine's CPU backend)"},
    },
    "convblock": {
        "trace": os.path.join(WL, "convblock_b64.trc"),
        "step": ("conv.fwd", None),
        "kernels": {1: ("conv.fwd", FCONV), 23: ("conv.dw", FCONV), 27: ("conv.dx", FCONV)},
        "unit": "TFLOP/s", "bound": "mfma", "dominant": "conv.fwd", "graph": True,
        "config": {"workload": "conv block f32 fwd+bwd: conv3x3 64->64 pad 1, batchnorm (train, "
                               "eps 1e-5), relu, maxpool 2, sum loss; backward dW and dX",
                   "batch": 64, "input": "N(0,1) [64,64,56,56]", "kernels_per_step": 28},
        "profile": "convblock_b64.md",
        "cpu": {"exe": "oracle/_ref/ref_replay", "kind": "reference", "args": ["--guard"],
                "trace": os.path.join(WL, "convblock_b1.trc"), "marks": ("conv.fwd", "-"),
                "flops": 3 * FCONV // 64,
                "sample": "the full step at batch 1 (the same 28 kernels; the convolutions' "
                          "FLOPs are linear in the batch) on the engine's CPU backend, its "
                          "buffers placed in zero-filled guard regions (its interpreter loads "
                          "masked pad elements before discarding them)"},
    },
}


class Hip:
    """hipEvent timing on the backend's stream (libamdhip64 via ctypes)."""

    def __init__(self, stream, flush=None):
        self.h = C.CDLL("libamdhip64.so")
        self.stream = C.c_void_p(stream)
        self.flush = flush
        self.h.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.h.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.h.hipEventSynchronize.argtypes = [C.c_void_p]
        self.h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]

    def event(self):
        e = C.c_void_p()
        assert self.h.hipEventCreate(C.byref(e)) == 0
        return e

    def record(self, e):
        # the backend holds some launches back to batch them: issue them
        # first, so that the event follows every earlier dispatch
        if self.flush:
            self.flush()
        assert self.h.hipEventRecord(e, self.stream) == 0

    def ms(self, a, b):
        self.h.hipEventSynchronize(b)
        out = C.c_float()
        assert self.h.hipEventElapsedTime(C.byref(out), a, b) == 0
        return out.value


def measured_traffic(profile, kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 summary
    (its ```json block), or None when no counter run has been recorded."""
    if not profile:
        return None
    path = os.path.join(ROOT, "profiles", profile)
    if not os.path.exists(path):
        return None
    text = open(path).read()
    if "```json" not in text:
        return None
    block = text.split("```json", 1)[1].split("```", 1)[0]
    return json.loads(block).get("traffic_bytes", {}).get(kernel)


def host_info():
    """The host the CPU baselines ran on: CPU model, cores visible, glibc."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        nproc = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        nproc = os.cpu_count()
    return {"cpu": model, "nproc": nproc, "cpu_count": os.cpu_count(),
            "glibc": "-".join(platform.libc_ver())}


def cpu_baseline(spec, wl):
    exe = os.path.join(ROOT, spec["exe"])
    if not os.path.exists(exe):
        print("cpu baseline: %s is not built" % spec["exe"], file=sys.stderr)
        return None
    cmd = [exe, spec["trace"], spec["marks"][0], spec["marks"][1], str(spec.get("reps", 1))] + spec.get("args", [])
    if shutil.which("taskset"):
        cmd = ["taskset", "-c", "0"] + cmd
    print("cpu baseline: %s" % " ".join(cmd), file=sys.stderr, flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    if r.returncode != 0:
        sys.stderr.write(r.stderr)
        return None
    sec = json.loads(r.stdout.strip().splitlines()[-1])["per_rep"]
    out = {"unit": wl["unit"], "cores": 1, "kind": spec["kind"], "sample": spec["sample"],
           "seconds": round(sec, 3), "host": host_info()}
    if wl["unit"] == "GB/s":
        out["value"] = round(sum(b for _n, b in wl["kernels"].values()) / sec / 1e9, 4)
    elif wl["unit"] == "TFLOP/s":
        out["value"] = round(spec["flops"] / sec / 1e12, 6)
    else:
        out["value"] = round(1.0 / (sec * spec.get("batch_scale", 1.0)), 5)
    return out


def dispatch_count(L):
    c = (C.c_uint64 * 13)()
    L.thvm_hip_counters(c, 13)
    return c[0]


def run_workload(L, name, steps, warmup, want_cpu):
    wl = WORKLOADS[name]
    be = L.thvm_hip_backend()
    t = L.thvm_trace_load(wl["trace"].encode())
    if not t:
        raise SystemExit("cannot load %s" % wl["trace"])
    n = L.thvm_trace_count(t)
    lo = L.thvm_trace_find_mark(t, wl["step"][0].encode(), 0)
    hi = n if wl["step"][1] is None else L.thvm_trace_find_mark(t, wl["step"][1].encode(), lo)
    assert 0 <= lo < hi <= n
    allocs = sum(1 for j in range(0, hi) if L.thvm_trace_tag(t, j) == TAG_ALLOC)
    step_allocs = sum(1 for j in range(lo, hi) if L.thvm_trace_tag(t, j) == TAG_ALLOC)
    replays = max(warmup, 1) + 2 * steps + (1 if wl.get("graph") else 0)
    # replays the buffer ids allow beyond those (extra untimed warmup)
    spare = (MAX_BUFFER_IDS - allocs) // step_allocs - replays if step_allocs else 1 << 20
    if allocs + replays * step_allocs > MAX_BUFFER_IDS:
        raise SystemExit("%s: %d step replays need %d buffer ids, more than the %d the backend holds without a "
                         "pool reset; use fewer --steps" % (name, replays, allocs + replays * step_allocs,
                                                            MAX_BUFFER_IDS))
    L.thvm_trace_replay(t, be, 0, lo, 0)           # inputs: allocate and upload (untimed)
    L.thvm_trace_drop_gen_cache(t)
    assert L.thvm_hip_synchronize() == 0
    t_c = time.perf_counter()
    L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)  # the first replay compiles every kernel
    assert L.thvm_hip_synchronize() == 0
    # the warmup: at least `warmup` replays, and at least WARM_MIN_S of
    # back-to-back replays after the first (the GPU's clocks settle under
    # sustained load: the conv block's timed steps ran 0.670-0.679 ms after
    # 5 warmup steps, 0.641-0.645 ms after 40), as far as the buffer ids allow
    done, t_w = 1, time.perf_counter()
    while done < max(warmup, 1) or (time.perf_counter() - t_w < WARM_MIN_S and done - max(warmup, 1) < spare):
        t_r = time.perf_counter()
        L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)
        done += 1
        if time.perf_counter() - t_r > WARM_MIN_S:   # it compiled (batch kernels of a later replay)
            t_w = time.perf_counter()
        if done % 4 == 0:
            assert L.thvm_hip_synchronize() == 0
    assert L.thvm_hip_synchronize() == 0
    print("%s: setup + warmup %.1fs (%d warmup replays), step = records [%d, %d)" %
          (name, time.perf_counter() - t_c, done, lo, hi), file=sys.stderr, flush=True)
    hip = Hip(L.thvm_hip_stream(), L.thvm_hip_flush)
    n_disp = sum(1 for j in range(lo, hi) if L.thvm_trace_tag(t, j) in (TAG_UOP, TAG_RS))
    d0 = dispatch_count(L)
    # pass 1: whole steps (the reported throughput)
    e0, e1 = hip.event(), hip.event()
    t0 = time.perf_counter()
    hip.record(e0)
    for _ in range(steps):
        L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)
    hip.record(e1)
    assert L.thvm_hip_synchronize() == 0
    wall = time.perf_counter() - t0
    # every dispatch of every step ran (none skipped for a missing buffer)
    assert dispatch_count(L) - d0 == steps * n_disp, "%s: dispatches skipped" % name
    gpu_ms = hip.ms(e0, e1)
    step_s = wall / steps
    # pass 2: events around each listed dispatch on the backend stream
    disp = [j for j in range(lo, hi) if L.thvm_trace_tag(t, j) in (TAG_UOP, TAG_RS)]
    k_ms, km_ms = {}, {}
    if wl["kernels"]:
        ev = {o: (hip.event(), hip.event()) for o in wl["kernels"]}
        # matrix-core workloads: a second pair of events right around each
        # contraction's main kernel (thvm_hip_time_contraction), the kernel
        # the roofline and the rocprof statistics name; the dispatch's pair
        # also holds its pack or split-K sum kernel
        evm = {o: (hip.event(), hip.event()) for o in wl["kernels"]} if wl["bound"] == "mfma" else {}
        for _ in range(steps):
            prev = lo
            for o in sorted(ev):
                u = disp[o]
                L.thvm_trace_replay(t, be, prev, u, SKIP_READS)
                hip.record(ev[o][0])
                if o in evm:
                    L.thvm_hip_time_contraction(evm[o][0], evm[o][1])
                L.thvm_trace_replay(t, be, u, u + 1, SKIP_READS)
                if o in evm:
                    assert L.thvm_hip_time_contraction(None, None) == 1, "%s: dispatch %d is no contraction" % (name, o)
                hip.record(ev[o][1])
                prev = u + 1
            L.thvm_trace_replay(t, be, prev, hi, SKIP_READS)
            for o, (ea, eb) in ev.items():
                nm = wl["kernels"][o][0]
                k_ms[nm] = k_ms.get(nm, 0.0) + hip.ms(ea, eb)
                if o in evm:
                    km_ms[nm] = km_ms.get(nm, 0.0) + hip.ms(*evm[o])
        k_ms = {k: v / steps for k, v in k_ms.items()}
        km_ms = {k: v / steps for k, v in km_ms.items()}
    assert L.thvm_hip_synchronize() == 0
    gpu_ms_eager = gpu_ms
    # pass 3: the step captured once into a HIP graph, launched `steps` times
    # (each launch is a whole step on the current parameters)
    graph_s = None
    if wl.get("graph"):
        g = None
        if L.thvm_hip_graph_begin() == 0:
            L.thvm_trace_replay(t, be, lo, hi, SKIP_READS)
            g = L.thvm_hip_graph_end()
        if g:
            assert L.thvm_hip_graph_launch(g) == 0
            assert L.thvm_hip_synchronize() == 0
            t0 = time.perf_counter()
            hip.record(e0)
            for _ in range(steps):
                assert L.thvm_hip_graph_launch(g) == 0
            hip.record(e1)
            assert L.thvm_hip_synchronize() == 0
            graph_s = (time.perf_counter() - t0) / steps
            gpu_ms = hip.ms(e0, e1)
            L.thvm_hip_graph_destroy(g)
        else:
            print("%s: the step could not be captured into a graph" % name, file=sys.stderr)
    L.thvm_trace_release(t, be)
    L.thvm_trace_free(t)
    L.thvm_hip_pool_reset(0)
    res = {"value": None, "unit": wl["unit"], "ms_per_step": round(step_s * 1e3, 4),
           "gpu_ms_per_step": round(gpu_ms_eager / steps, 4), "config": wl["config"],
           "kernels_ms": {k: round(v, 4) for k, v in k_ms.items()}, "warmup_replays": done}
    if km_ms:
        res["main_kernels_ms"] = {k: round(v, 4) for k, v in km_ms.items()}
    if graph_s is not None:
        res["graph_ms_per_step"] = round(graph_s * 1e3, 4)
        res["graph_gpu_ms_per_step"] = round(gpu_ms / steps, 4)
    work = sum(w for _n, w in wl["kernels"].values())
    if wl["unit"] == "GB/s":
        res["value"] = round(work / step_s / 1e9, 2)
    elif wl["unit"] == "TFLOP/s":
        res["value"] = round(work / step_s / 1e12, 3)
        if graph_s is not None:
            res["graph_value"] = round(work / graph_s / 1e12, 3)
    else:
        res["value"] = round(1.0 / step_s, 3)
        if graph_s is not None:
            res["graph_value"] = round(1.0 / graph_s, 3)
    if wl["dominant"]:
        dom = wl["dominant"]
        dom_w = next(w for nm, w in wl["kernels"].values() if nm == dom)
        if wl["bound"] == "hbm":
            ach, peak, unit = dom_w / (k_ms[dom] * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s"
        else:
            ach, peak, unit = dom_w / (km_ms.get(dom, k_ms[dom]) * 1e-3) / 1e12, MFMA_F32_PEAK_TFLOPS, "TFLOP/s"
        res["roofline"] = {"bound": wl["bound"], "achieved": round(ach, 2), "peak": peak,
                           "unit": unit, "frac": round(ach / peak, 4),
                           "traffic": measured_traffic(wl.get("profile"), dom), "kernel": dom}
    if want_cpu and wl.get("cpu"):
        res["cpu_baseline"] = cpu_baseline(wl["cpu"], wl)
    print("%s: %s" % (name, json.dumps(res)), file=sys.stderr, flush=True)
    return res


ENGINE_STEPS = {
    "lenet_engine": ("lenet", 20, 256, "LeNet-5 training step at batch 256 through the engine"),
    "mlp_engine": ("mlp", 50, 64, "2-layer MLP forward + backward at batch 64 through the engine"),
}


def engine_step(name, want_cpu):
    """The workload's training step driven by the engine itself (thvm_eval with
    hip_backend as the default device: scheduling, lowering, dispatch and the
    step's read-backs, timed on the host clock), via oracle/_ref/engine_live in
    a child process. Its CPU leg runs the same steps on the engine's CPU backend."""
    exe = os.path.join(ROOT, "oracle", "_ref", "engine_live")
    if not os.path.exists(exe):
        print("engine step: oracle/_ref/engine_live is not built", file=sys.stderr)
        return None
    wl, steps, batch, what = ENGINE_STEPS[name]
    cmd = [exe, os.path.join(ROOT, "tinyhvm_amd", "libthvm_hip.so"), "time", wl, str(steps), str(batch)]
    print("engine step: %s" % " ".join(cmd), file=sys.stderr, flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
    if r.returncode != 0 or not lines:
        sys.stderr.write(r.stderr[-2000:])
        return None
    e = json.loads(lines[-1])
    g = e["gpu"]
    res = {"value": g["steps_per_s"], "unit": "steps/s", "ms_per_step": g["median_ms"],
           "mean_ms_per_step": g["mean_ms"],
           "config": {"workload": what + " (thvm_eval -> hip_backend; host work, dispatches and "
                                         "read-backs on the host clock, median of %d steps)" % steps,
                      "batch": batch},
           "dispatches_per_step": g["dispatches_per_step"], "reads_per_step": g["reads_per_step"],
           "host_waits_per_step": g["host_waits_per_step"], "waits_outside_reads": g["waits_outside_reads"],
           "backend_slots_ms_per_step": g.get("backend_slots_ms_per_step"),
           "read_ms_per_step": g.get("read_ms_per_step")}
    if want_cpu and e["cpu"]["steps_per_s"] > 0:
        res["cpu_baseline"] = {"value": e["cpu"]["steps_per_s"], "unit": "steps/s", "cores": 1,
                               "kind": "reference", "seconds": e["cpu"]["seconds_per_step"],
                               "sample": "the same step through thvm_eval on the engine's CPU "
                                         "backend (%s)" % ("one step" if wl == "lenet" else
                                                           "median of three steps"),
                               "host": host_info()}
    print("%s: %s" % (name, json.dumps(res)), file=sys.stderr, flush=True)
    return res


ENGINE_JIT = {
    "lenet_engine_graph": ("lenet", 50, 256, "LeNet-5 training step at batch 256 through the engine, captured "
                                             "once into a HIP graph and replayed"),
    "mlp_engine_graph": ("mlp", 100, 64, "2-layer MLP training step (SGD) at batch 64 through the engine, "
                                         "captured once into a HIP graph and replayed"),
}


def engine_jit(name):
    """A training step the engine drives (thvm_eval on a context made by
    thvm_init("hip")), captured once into a HIP graph and launched for every
    later step, the role of the Metal backend's JIT record/replay: each step
    writes its labels into the persistent one-hot tensor, launches the graph
    and reads the loss back (host clock). oracle/_ref/engine_live runs the
    same steps eagerly through the engine first and checks that every loss and
    the final parameters agree bit for bit."""
    exe = os.path.join(ROOT, "oracle", "_ref", "engine_live")
    if not os.path.exists(exe):
        print("engine jit: oracle/_ref/engine_live is not built", file=sys.stderr)
        return None
    wl, steps, batch, what = ENGINE_JIT[name]
    cmd = [exe, os.path.join(ROOT, "tinyhvm_amd", "libthvm_hip.so"), "jit", wl, str(steps), str(batch)]
    print("engine jit: %s" % " ".join(cmd), file=sys.stderr, flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
    if not lines:
        sys.stderr.write(r.stderr[-2000:])
        return None
    e = json.loads(lines[-1])
    res = {"value": e["graph"]["steps_per_s"], "unit": "steps/s", "ms_per_step": e["graph"]["ms_per_step"],
           "eager_value": e["eager"]["steps_per_s"], "eager_ms_per_step": e["eager"]["ms_per_step"],
           "config": {"workload": what + " (label write, graph launch and loss read per step, host clock, "
                                         "%d steps)" % steps, "batch": batch},
           "losses_equal_eager": e["losses_equal"], "params_equal_eager": e["params_equal"],
           "loss_first": e["loss_first"], "loss_last": e["loss_last"]}
    if r.returncode != 0:
        res["error"] = "graph replays differ from the engine's eager steps"
    print("%s: %s" % (name, json.dumps(res)), file=sys.stderr, flush=True)
    return res


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
    hip = Hip(L.thvm_hip_stream(), L.thvm_hip_flush)
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
    ap.add_argument("--workloads", default="fused,matmul,lenet,convblock,mlp,lenet_engine,mlp_engine,"
                                           "lenet_engine_graph,mlp_engine_graph",
                    help="comma list; the first one gives the headline value")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a 256 MiB copy kernel (HBM counter calibration)")
    args = ap.parse_args()
    if args.calibrate_copy:
        copy_calibration()
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: this backend has no multi-GPU path "
              "(use --gpus 1)", file=sys.stderr)
        sys.exit(2)
    names = [w for w in args.workloads.split(",") if w]
    for nm in names:
        if nm not in WORKLOADS and nm not in ENGINE_STEPS and nm not in ENGINE_JIT:
            raise SystemExit("unknown workload %r (have %s)" % (
                nm, ", ".join(list(WORKLOADS) + list(ENGINE_STEPS) + list(ENGINE_JIT))))
    if names[0] not in WORKLOADS:
        raise SystemExit("the first workload gives the headline value: one of %s" % ", ".join(WORKLOADS))
    L = _lib.lib()
    if L.thvm_hip_init() != 0:
        raise SystemExit("HIP backend failed to initialise")
    results = {nm: run_workload(L, nm, args.steps, args.warmup, not args.no_cpu) for nm in names
               if nm in WORKLOADS}
    L.thvm_hip_shutdown()
    for nm in names:
        if nm in ENGINE_STEPS:
            results[nm] = engine_step(nm, not args.no_cpu)
        elif nm in ENGINE_JIT:
            results[nm] = engine_jit(nm)
    head = results[names[0]]
    out = {
        "metric": METRIC,
        "value": head["value"],
        "unit": head["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": head["config"],
        "roofline": head.get("roofline"),
        "cpu_baseline": head.get("cpu_baseline"),
        "kernels_ms": head.get("kernels_ms"),
        "workloads": {nm: r for nm, r in results.items() if nm != names[0]},
    }
    if head.get("main_kernels_ms"):
        out["main_kernels_ms"] = head["main_kernels_ms"]
    print(json.dumps(out))


if __name__ == "__main__":
    main()
