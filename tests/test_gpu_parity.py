"""GPU parity, through the HIP backend's C ABI, for every committed kernel trace.

Kernel-boundary parity: before each dispatch the GPU's actual input buffers
are read back and the oracle (oracle/oracle.c, the CPU restatement of the
engine's interpreter) runs the same kernel on them; the GPU output must match
the oracle's under the kernel's tolerance class:
  - bit-exact: kernels a single lane evaluates in the reference's own order
    (elementwise, index/view work, casts, RMAX), the FusedOp fallback, the
    legacy per-op slots, strided copies (contiguify) and buffer copies;
  - 1e-6 relative per element (floor 1e-3 of the output's max): the same with
    EXP or LOG, whose last bit may differ between GPU and host libm;
  - 1e-4 normwise (max |x - y| <= 1e-4 max |y|): sums whose order differs
    (split across a workgroup, or accumulated by matrix cores). Where the
    reference's own serial float sum is farther than that from the exact sum
    of the same terms (the oracle with double accumulators), the GPU result
    must be within 1e-4 of the exact sum instead.
End-to-end: the outputs the trace recorded from the reference CPU backend
(SNAPSHOT records) must match the GPU run within 1e-3 normwise, the GPU's
reordered sums propagating through whole training steps.
"""
import ctypes as C
import os

import numpy as np
import pytest

from tests import tracetools as tt
from tinyhvm_amd import _lib, abi, trace

pytestmark = pytest.mark.gpu

DT = {0: np.float32, 1: np.uint16, 2: np.int32, 3: np.uint32}


@pytest.fixture(scope="module")
def hip():
    # default heuristics: small contractions stay on the generated kernels
    saved = os.environ.pop("THVM_HIP_DENSE_FORCE", None)
    L = _lib.lib()
    assert L.thvm_hip_init() == 0, "HIP backend failed to initialise"
    yield L
    L.thvm_hip_shutdown()
    if saved is not None:
        os.environ["THVM_HIP_DENSE_FORCE"] = saved


def _oracle():
    ora = tt.oracle()
    u64, vp = C.c_uint64, C.c_void_p
    ora.ora_dispatch_uop.argtypes = [vp, u64, C.POINTER(vp), C.POINTER(u64), C.c_uint32,
                                     C.POINTER(abi.UOpKernel)]
    ora.ora_dispatch_uop_exact.argtypes = ora.ora_dispatch_uop.argtypes
    ora.ora_dispatch_uop_gids.argtypes = ora.ora_dispatch_uop.argtypes + [vp, u64]
    ora.ora_dispatch_rs.argtypes = [vp, u64, C.POINTER(vp), C.POINTER(u64),
                                    C.POINTER(C.POINTER(abi.View)),
                                    C.POINTER(C.POINTER(abi.ShapeTracker)), C.c_uint32,
                                    C.POINTER(abi.FusedOp), C.c_uint32, C.POINTER(abi.Shape),
                                    C.POINTER(abi.ReduceSpec), C.POINTER(C.c_uint32), C.c_uint32]
    u32, PV = C.c_uint32, C.POINTER(abi.View)
    ora.ora_contiguify.argtypes = [vp, u64, vp, u64, u32, PV, u32]
    ora.ora_op_unary.argtypes = [u32, vp, u64, PV, u32, vp, u64, PV, u32]
    ora.ora_op_binary.argtypes = [u32, vp, u64, PV, u32, vp, u64, PV, u32, vp, u64, PV, u32]
    ora.ora_op_mm.argtypes = [vp, u64, u32, vp, u64, PV, u32, vp, u64, PV, u32, u32, u32, u32]
    ora.ora_op_reduce.argtypes = [u32, vp, u64, u32, u32, vp, u64, u32, u32]
    f32 = C.c_float
    ora.ora_adam_step.argtypes = [vp, vp, vp, vp, f32, f32, f32, f32, f32, f32, u32]
    return ora


def _legacy_oracle(ora, r, host):
    """Runs a CONTIG or legacy per-op record through the oracle on the GPU's
    inputs; returns (expected bytes, output dtype, tolerance kind, rtol)."""
    f = r.f
    cast = lambda b: C.cast(b, C.c_void_p)  # noqa: E731
    if r.tag == trace.CONTIG:
        out, n = host.read(f["dst"])
        src, sn = host.read(f["src"])
        esize = 2 if n == f["numel"] * 2 else 4
        v = f["view"].to_c()
        ora.ora_contiguify(cast(out), n, cast(src), sn, f["numel"], C.byref(v), esize)
        return out, n, {2: 1, 4: 0}[esize], "exact", 0.0
    out, n = host.read(f["dst"])
    a, an = host.read(f["a"])
    tr = f.get("uop") in (abi.UOP_EXP, abi.UOP_LOG)
    kind, rtol = ("elem", 1e-6) if tr and r.tag != trace.OPRED else ("exact", 0.0)
    if r.tag == trace.OPUN:
        dv, av = f["dv"].to_c(), f["av"].to_c()
        ora.ora_op_unary(f["uop"], cast(out), n, C.byref(dv), f["dd"], cast(a), an, C.byref(av), f["ad"])
    elif r.tag == trace.OPBIN:
        b, bn = host.read(f["b"])
        dv, av, bv = f["dv"].to_c(), f["av"].to_c(), f["bv"].to_c()
        ora.ora_op_binary(f["uop"], cast(out), n, C.byref(dv), f["dd"], cast(a), an, C.byref(av), f["ad"],
                          cast(b), bn, C.byref(bv), f["bd"])
    elif r.tag == trace.OPMM:
        b, bn = host.read(f["b"])
        av, bv = f["av"].to_c(), f["bv"].to_c()
        ora.ora_op_mm(cast(out), n, f["dd"], cast(a), an, C.byref(av), f["ad"], cast(b), bn, C.byref(bv),
                      f["bd"], f["M"], f["K"], f["N"])
    else:
        ora.ora_op_reduce(f["uop"], cast(out), n, f["dn"], f["dd"], cast(a), an, f["ad"], f["rdim"])
    return out, n, f["dd"], kind, rtol


def _has_transcendental_uop(k):
    return any(k.ops[i].type == abi.KOP_ALU and k.ops[i].imm.u in (abi.UOP_EXP, abi.UOP_LOG)
               for i in range(k.n_ops))


def uop_tolerance(k):
    """(kind, rtol) for a lowered kernel, from how the backend runs it."""
    if _lib.dense_analyze(k):
        return "norm", 1e-4
    w = _lib.window_analyze(k)
    if w and w[0] == 2:                 # run sum: reordered across lanes and workgroups
        return "norm", 1e-4
    if w and w[0] == 1:                 # window max: the engine's order
        return "exact", 0.0
    _src, mode, _vec = _lib.kernel_source(k)
    has_sum = any(k.ops[i].type == abi.KOP_ACC and k.ops[i].imm.u != abi.UOP_RMAX
                  for i in range(k.n_ops))
    if mode == 1 and has_sum:
        return "norm", 1e-4
    if _has_transcendental_uop(k):
        return "elem", 1e-6
    return "exact", 0.0


def compare(got, want, dtype, kind, rtol):
    if kind == "exact" or dtype != 0:
        if got == want:
            return True, "bit-exact"
        g = np.frombuffer(got, dtype=np.uint8)
        w = np.frombuffer(want, dtype=np.uint8)
        return False, "differs in %d of %d bytes" % (int(np.sum(g != w)), len(w))
    x = np.frombuffer(got, dtype=np.float32).astype(np.float64)
    y = np.frombuffer(want, dtype=np.float32).astype(np.float64)
    both_nan = np.isnan(x) & np.isnan(y)
    x, y = np.where(both_nan, 0, x), np.where(both_nan, 0, y)
    ymax = float(np.max(np.abs(y))) if y.size else 0.0
    if kind == "norm":
        err = float(np.max(np.abs(x - y))) / max(ymax, 1e-30)
        return err <= rtol, "normwise %.2e (tol %.0e)" % (err, rtol)
    scale = np.maximum(np.abs(y), 1e-3 * max(ymax, 1e-30))
    err = float(np.max(np.abs(x - y) / scale)) if y.size else 0.0
    return err <= rtol, "elementwise %.2e (tol %.0e)" % (err, rtol)


class Host:
    """Host copies of the device's buffers, read just before a dispatch."""

    def __init__(self, read_fn, rp, sizes):
        self.read_fn, self.rp, self.sizes = read_fn, rp, sizes

    def read(self, trace_id):
        live = self.rp.live(trace_id)
        n = self.sizes.get(trace_id, 0)
        buf = (C.c_uint8 * max(n, 4))()
        if live and n:
            self.read_fn(live, buf, n)
        return buf, n if live else 0


def _rs_args(r):
    f = r.f
    n = f["n_leaves"]
    views = [v.to_c() for v in f["views"]]
    sts = []
    for s in f["sts"]:
        if s is None:
            sts.append(None)
            continue
        st = abi.ShapeTracker()
        st.n_views = len(s)
        for j, v in enumerate(s):
            v.to_c(st.views[j])
        sts.append(st)
    vptr = (C.POINTER(abi.View) * max(n, 1))(*[C.pointer(v) for v in views])
    sptr = (C.POINTER(abi.ShapeTracker) * max(n, 1))(*[C.pointer(s) if s is not None else None
                                                      for s in sts])
    ops = (abi.FusedOp * max(len(f["ops"]), 1))()
    for j, (u, a, b, aux) in enumerate(f["ops"]):
        ops[j].uop, ops[j].arg_a, ops[j].arg_b, ops[j].aux = u, a, b, aux
    full = abi.Shape()
    full.rank = f["full_rank"]
    for d in range(8):
        full.dims[d] = f["full_dims"][d]
    red = None
    if f["has_reduce"]:
        red = abi.ReduceSpec()
        rr = f["reduce"]
        for d in range(8):
            red.is_reduce[d] = rr["is_reduce"][d]
            red.is_reduce2[d] = rr["is_reduce2"][d]
        red.reduce_type, red.post_reduce_start = rr["reduce_type"], rr["post_reduce_start"]
        red.n_post_leaves, red.reduce2_type = rr["n_post_leaves"], rr["reduce2_type"]
        red.reduce2_start = rr["reduce2_start"]
    dts = (C.c_uint32 * max(n, 1))(*f["leaf_dtypes"]) if f["has_dtypes"] else None
    keep = (views, sts)
    return keep, vptr, sptr, ops, full, red, dts


SENTINEL = 0xFFFFFFFF      # a NaN bit pattern no kernel of these workloads produces


def _reads_own_output(k, out_id, leaf_ids):
    return out_id in leaf_ids or any(k.ops[i].type == abi.KOP_LOAD and k.ops[i].imm.u == 0
                                     for i in range(k.n_ops))


def kernel_parity(backend, read_fn, sync_fn, ora, path, tol_fn=None, prefix_fn=None, sample_fn=None,
                  extra_fn=None, write_fn=None):
    """Replays `path` against `backend`, checking every dispatch against the
    oracle on the same inputs and every SNAPSHOT against the reference.

    prefix_fn(k) -> T or None: for a kernel too large for the oracle, check
    its first T outputs only. A lowered kernel's index arithmetic decodes the
    flat output index from GID by constants of its own, not from the grid, so
    the oracle run over a grid of T computes exactly those T outputs.

    sample_fn(k) -> array of gids or None: for such a kernel, the oracle runs
    those gids only (into a sentinel-filled buffer, so exactly the outputs
    they store are compared), and, with write_fn(live_id, bytes) given, the
    device output is filled with the sentinel before the dispatch and no
    sentinel may survive it: every output is written, whatever the sample.

    extra_fn(i, k, leaves, got) -> (ok, message) or None: a further check of
    dispatch i on its input buffers and the device output (bytes)."""
    tol_fn = tol_fn or uop_tolerance
    recs = trace.read_trace(path)
    rp = tt.Replay(path, backend)
    host = Host(read_fn, rp, {})
    dtype_of = {}
    kernel_results, e2e = [], []
    try:
        for i, r in enumerate(recs):
            if r.tag == trace.ALLOC:
                host.sizes[r.f["id"]] = r.f["bytes"]
            if r.tag == trace.WRITE and r.f["enc"] == trace.ENC_GEN:
                dtype_of[r.f["id"]] = r.f["dtype"]
            if r.tag in (trace.UOP, trace.RS):
                out_id = r.f["out"]
                out_buf, out_n = host.read(out_id)
                leaves = [host.read(t) for t in r.f["leaf_bufs"]]
                n = len(leaves)
                lp = (C.c_void_p * max(n, 1))(*[C.cast(b, C.c_void_p) if m else None for b, m in leaves])
                lb = (C.c_uint64 * max(n, 1))(*[m for _b, m in leaves])
                cmp_n, note, sampled, filled = out_n, "", None, False
                if r.tag == trace.UOP:
                    k = trace.to_uop_kernel(r)
                    T = prefix_fn(k) if prefix_fn else None
                    gids = sample_fn(k) if sample_fn else None
                    if gids is not None and _reads_own_output(k, out_id, r.f["leaf_bufs"]):
                        gids = None           # its old contents are an input: run it whole
                    kp = k
                    if gids is not None:
                        gids = np.ascontiguousarray(gids, dtype=np.uint32)
                        ctypes_fill = np.frombuffer(out_buf, dtype=np.uint32, count=out_n // 4)
                        ctypes_fill[:] = SENTINEL
                        ora.ora_dispatch_uop_gids(C.cast(out_buf, C.c_void_p), out_n, lp, lb, n, C.byref(k),
                                                  gids.ctypes.data_as(C.c_void_p), len(gids))
                        sampled = np.frombuffer(bytes(out_buf)[:out_n], dtype=np.uint32)
                        note = " [%d sampled gids]" % len(gids)
                        if write_fn is not None and k.out_dtype != 1 and \
                                not _reads_own_output(k, out_id, r.f["leaf_bufs"]):
                            fill = np.full(out_n // 4, SENTINEL, dtype=np.uint32)
                            write_fn(rp.live(out_id), fill.ctypes.data_as(C.c_void_p), out_n)
                            filled = True
                            note += ", every output written"
                    elif T:
                        kp = trace.to_uop_kernel(r)
                        kp.grid[0], kp.grid[1], kp.grid[2] = T, 1, 1
                        cmp_n = min(out_n, T * (2 if k.out_dtype == 1 else 4))
                        note = " [first %d outputs]" % T
                        ora.ora_dispatch_uop(C.cast(out_buf, C.c_void_p), out_n, lp, lb, n, C.byref(kp))
                    else:
                        ora.ora_dispatch_uop(C.cast(out_buf, C.c_void_p), out_n, lp, lb, n, C.byref(kp))
                    kind, rtol = tol_fn(k)
                    dtype = k.out_dtype
                else:
                    keep, vptr, sptr, ops, full, red, dts = _rs_args(r)
                    ora.ora_dispatch_rs(C.cast(out_buf, C.c_void_p), out_n, lp, lb, vptr, sptr, n, ops,
                                        len(r.f["ops"]), C.byref(full),
                                        C.byref(red) if red is not None else None, dts,
                                        r.f["out_dtype"])
                    has_tr = any(o[0] in (abi.UOP_EXP, abi.UOP_LOG) for o in r.f["ops"])
                    kind, rtol = ("elem", 1e-6) if has_tr else ("exact", 0.0)
                    dtype = r.f["out_dtype"]
                rp.run(i, i + 1)
                dtype_of[out_id] = dtype
                got, _ = host.read(out_id)
                if sampled is not None:
                    g32 = np.frombuffer(bytes(got)[:out_n], dtype=np.uint32)
                    sel = sampled != SENTINEL
                    ok, msg = compare(g32[sel].tobytes(), sampled[sel].tobytes(), dtype, kind, rtol)
                    msg += " over %d outputs" % int(sel.sum())
                    if filled:
                        total = k.grid[0] if k.local_size > 0 else k.grid[0] * k.grid[1] * k.grid[2]
                        unwritten = int(np.sum(g32[:min(total, len(g32))] == SENTINEL))
                        if unwritten:
                            ok, msg = False, msg + "; %d outputs never written" % unwritten
                    if extra_fn is not None:
                        xr = extra_fn(i, k, [bytes(b)[:m] for b, m in leaves], bytes(got)[:out_n])
                        if xr is not None:
                            ok, msg = ok and xr[0], msg + "; " + xr[1]
                    kernel_results.append((i, ok, msg + note))
                    print("  %s dispatch %d (%s): %s%s" % (path.split("/")[-1], i, kind, msg, note), flush=True)
                    continue
                ok, msg = compare(bytes(got)[:cmp_n], bytes(out_buf)[:cmp_n], dtype, kind, rtol)
                if not ok and kind == "norm" and r.tag == trace.UOP:
                    # a long serial float sum in the reference can itself be
                    # farther than the tolerance from the exact sum: then the
                    # GPU must be within the tolerance of the exact sum
                    exact = (C.c_uint8 * max(out_n, 4))()
                    ora.ora_dispatch_uop_exact(C.cast(exact, C.c_void_p), out_n, lp, lb, n, C.byref(kp))
                    ok, m_gpu = compare(bytes(got)[:cmp_n], bytes(exact)[:cmp_n], dtype, kind, rtol)
                    _ok, m_ref = compare(bytes(out_buf)[:cmp_n], bytes(exact)[:cmp_n], dtype, kind, rtol)
                    msg = "vs reference %s; vs the exact sum: gpu %s, reference %s" % (msg, m_gpu, m_ref)
                msg += note
                kernel_results.append((i, ok, msg))
                print("  %s dispatch %d (%s): %s" % (path.split("/")[-1], i, kind, msg), flush=True)
            elif r.tag == trace.CONTIG or r.tag in trace.LEGACY:
                want, n, dtype, kind, rtol = _legacy_oracle(ora, r, host)
                rp.run(i, i + 1)
                dst = r.f["dst"]
                dtype_of[dst] = dtype
                got, _ = host.read(dst)
                ok, msg = compare(bytes(got)[:n], bytes(want)[:n], dtype, kind, rtol)
                kernel_results.append((i, ok, msg))
                print("  %s %s %d (%s): %s" % (path.split("/")[-1], trace.TAG_NAMES[r.tag], i, kind, msg),
                      flush=True)
            elif r.tag == trace.ADAM:
                f = r.f
                nb = f["n"] * 4
                host_in = {k: np.frombuffer(bytes(host.read(f[k])[0])[:nb], dtype=np.float32).copy()
                           for k in ("param", "grad", "m", "v")}
                ora.ora_adam_step(*(host_in[k].ctypes.data for k in ("param", "grad", "m", "v")),
                                  f["lr"], f["beta1"], f["beta2"], f["eps"], f["bc1"], f["bc2"], f["n"])
                rp.run(i, i + 1)
                for k in ("param", "m", "v"):
                    dtype_of[f[k]] = 0
                    got, _ = host.read(f[k])
                    ok, msg = compare(bytes(got)[:nb], host_in[k].tobytes(), 0, "exact", 0.0)
                    kernel_results.append((i, ok, "%s: %s" % (k, msg)))
                    print("  %s ADAM %d %s (exact): %s" % (path.split("/")[-1], i, k, msg), flush=True)
            elif r.tag == trace.SNAPSHOT:
                got, n = host.read(r.f["id"])
                dt = dtype_of.get(r.f["id"], 0)
                ok, msg = compare(bytes(got)[:n], r.f["data"][:n], dt, "norm", 1e-3)
                e2e.append((i, ok, msg))
            else:
                if r.tag == trace.COPY:
                    dtype_of[r.f["dst"]] = dtype_of.get(r.f["src"], 0)
                rp.run(i, i + 1)
        assert sync_fn() == 0
    finally:
        rp.close()
    return kernel_results, e2e


@pytest.mark.parametrize("path", tt.fixtures(), ids=lambda p: p.split("/")[-1])
def test_trace_parity(hip, path):
    ora = _oracle()
    kr, e2e = kernel_parity(hip.thvm_hip_backend(), hip.thvm_hip_buf_read, hip.thvm_hip_synchronize,
                            ora, path)
    assert kr, "trace has no dispatches"
    bad = [r for r in kr if not r[1]]
    assert not bad, "kernel parity: %s" % bad
    bad_e2e = [r for r in e2e if not r[1]]
    assert not bad_e2e, "end-to-end vs reference: %s" % bad_e2e
