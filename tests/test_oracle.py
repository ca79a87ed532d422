"""The oracle (oracle/oracle.c) against the golden vectors: every SNAPSHOT in
the committed kernel traces holds the reference CPU backend's output for the
dispatch before it (source 0; source 2 where the engine ran over zero-guarded
leaves because its interpreter loads masked elements outside the buffer);
replaying the trace through the oracle must reproduce them bit for bit. Plus
closed-form checks that do not depend on the traces."""
import ctypes as C

import numpy as np
import pytest

from tests import tracetools as tt
from tinyhvm_amd import trace


@pytest.mark.parametrize("path", tt.fixtures(), ids=lambda p: p.split("/")[-1])
def test_oracle_reproduces_reference_snapshots(path):
    ora = tt.oracle()
    be = ora.oracle_backend_ptr()
    be.contents.init()
    rp = tt.Replay(path, be)
    n_snap = 0
    sources = {r_i: r.f["source"] for r_i, r in enumerate(trace.read_trace(path)) if r.tag == trace.SNAPSHOT}
    try:
        for i in range(rp.n):
            if rp.tag(i) == tt.TRC_SNAPSHOT:
                tid, ref = rp.snapshot(i)
                live = rp.live(tid)
                p = ora.oracle_buf_ptr(live)
                got = C.string_at(p, len(ref))
                assert got == ref, "%s: snapshot %d differs (source %d)" % (path, i, sources[i])
                n_snap += sources[i] in (0, 2)
            else:
                rp.run(i, i + 1)
    finally:
        rp.close()
        be.contents.shutdown()
    assert n_snap > 0
    # every golden vector comes from the engine itself (none from the oracle)
    assert all(v in (0, 2) for v in sources.values())


def _fused_closed_form(path):
    recs = trace.read_trace(path)
    gens = [r for r in recs if r.tag == trace.WRITE and r.f["enc"] == trace.ENC_GEN]
    assert len(gens) == 3
    ups = [r for r in recs if r.tag == trace.UOP]
    R, Cc = ups[0].f["full_dims"][:2]
    a, b, c = [np.frombuffer(trace.gen_data(g.f["dist"], g.f["dtype"], g.f["seed"], g.f["p0"],
                                            g.f["p1"], g.f["bytes"]), dtype=np.float32).reshape(R, Cc)
               for g in gens]
    snaps = [r for r in recs if r.tag == trace.SNAPSHOT]
    return a, b, c, snaps


@pytest.mark.parametrize("path", tt.fixtures("fused_*.trc"), ids=lambda p: p.split("/")[-1])
def test_fused_snapshots_match_closed_form(path):
    """y = sum(relu(a*b + c), -1) in f64 (within 1e-5 of the f32 sequential
    sum) and dA = (a*b + c > 0) * b (exact: the mask and one f32 product)."""
    a, b, c, snaps = _fused_closed_form(path)
    y_ref = np.maximum(a.astype(np.float64) * b + c, 0).sum(axis=1)
    y = np.frombuffer(snaps[0].f["data"], dtype=np.float32)
    ok, msg = tt.close(y, y_ref, 1e-5)
    assert ok, msg
    pre = (a * b) + c  # f32, same two roundings as the kernel
    da_ref = np.where(pre > 0, 1.0, 0.0).astype(np.float32) * b
    da = np.frombuffer(snaps[1].f["data"], dtype=np.float32).reshape(a.shape)
    assert np.array_equal(da, da_ref)


def test_planted_mistake_is_caught():
    """A wrong sign in the closed form must fail the same comparison."""
    a, b, c, snaps = _fused_closed_form(tt.fixtures("fused_64x256.trc")[0])
    y_wrong = np.maximum(a.astype(np.float64) * b - c, 0).sum(axis=1)
    y = np.frombuffer(snaps[0].f["data"], dtype=np.float32)
    ok, _ = tt.close(y, y_wrong, 1e-5)
    assert not ok


def _run_uop(fn, rec, leaves_by_id, out_elems):
    k = trace.to_uop_kernel(rec)
    arrs = [leaves_by_id[t] for t in rec.f["leaf_bufs"]]
    n = len(arrs)
    lp = (C.c_void_p * n)(*[a.ctypes.data for a in arrs])
    lb = (C.c_uint64 * n)(*[a.nbytes for a in arrs])
    out = np.zeros(out_elems, dtype=np.float32)
    fn(C.c_void_p(out.ctypes.data), out.nbytes, lp, lb, n, C.byref(k))
    return out


@pytest.mark.parametrize("path", tt.fixtures("fused_3x1000.trc") + tt.fixtures("fused_64x256.trc"),
                         ids=lambda p: p.split("/")[-1])
def test_exact_accumulation_mode(path):
    """ora_dispatch_uop_exact (the reference for long sums): the fused forward's
    row sums equal the float64 sum of the same float32 terms rounded once, and
    a kernel without a sum (the backward) is bit-identical to the float mode."""
    from tests.test_gpu_parity import _oracle
    ora = _oracle()
    recs = trace.read_trace(path)
    leaves = {}
    for r in recs:
        if r.tag == trace.WRITE:
            f = r.f
            if f["enc"] == trace.ENC_GEN:
                data = trace.gen_data(f["dist"], f["dtype"], f["seed"], f["p0"], f["p1"], f["bytes"])
            else:
                data = f["data"]
            leaves[f["id"]] = np.frombuffer(data, dtype=np.float32).copy()
    ups = [r for r in recs if r.tag == trace.UOP]
    R, Cc = ups[0].f["full_dims"][:2]
    a, b, c = (leaves[t].reshape(R, Cc) for t in ups[0].f["leaf_bufs"][:3])
    y = _run_uop(ora.ora_dispatch_uop_exact, ups[0], leaves, R)
    terms = np.maximum((a * b) + c, np.float32(0))
    want = terms.astype(np.float64).sum(axis=1).astype(np.float32)
    assert np.array_equal(y, want)
    y32 = _run_uop(ora.ora_dispatch_uop, ups[0], leaves, R)
    assert not np.array_equal(y32, want) or Cc < 512   # the serial float sum rounds at each step
    d_exact = _run_uop(ora.ora_dispatch_uop_exact, ups[1], leaves, R * Cc)
    d_float = _run_uop(ora.ora_dispatch_uop, ups[1], leaves, R * Cc)
    assert np.array_equal(d_exact, d_float)
