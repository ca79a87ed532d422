"""The code generator's vector-lane index analysis, checked against the op
semantics by brute force (no device needed).

One thread-vector of the generated kernels handles four consecutive gids
(elementwise) or four consecutive counter values of a reduce loop. For each
u32 op the generator claims: the same value on every lane (kind 0), or lane v
= lane 0 + off[v] with offsets fixed at generation (kind 1); a divisor of the
lane-0 value; and an upper bound of the value. The generated code computes
such ops once per thread-vector and forms 128-bit loads from them, so a wrong
claim reads wrong addresses. Here every u32 op of every generated kernel of
the committed traces is evaluated, with the interpreter's semantics (u32 wrap
on IDX, x/0 = x%0 = 0), on sampled thread-vectors and loop counters, and
every claim is checked against the values.
"""
import glob
import os

import numpy as np
import pytest

from tinyhvm_amd import abi, _lib, trace

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TRACES = sorted(glob.glob(os.path.join(ROOT, "tests", "golden", "*.trc")) +
                glob.glob(os.path.join(ROOT, "tinyhvm_amd", "workloads", "*.trc")))
M32 = np.uint64(0xFFFFFFFF)


def _kernels(path):
    seen = set()
    for r in trace.read_trace(path):
        if r.tag != trace.UOP:
            continue
        k = trace.to_uop_kernel(r)
        key = bytes(memoryview(k.ops)[:k.n_ops * C_KOP]) + bytes(k.grid) + bytes([k.local_size & 255])
        if key in seen:
            continue
        seen.add(key)
        yield k


C_KOP = 20   # sizeof(KOp): type, arg[3], imm


def _values(k, mode, V, S, rng):
    """u32 values of every op on S sampled thread-vectors x V lanes (None for
    float-valued ops and for ops computed from them)."""
    n = k.n_ops
    total = k.grid[0] if (mode == 1) else k.grid[0] * k.grid[1] * k.grid[2]
    if mode == 0:
        nvec = (total + V - 1) // V
        x = np.concatenate([np.arange(min(nvec, 64)), np.arange(max(nvec - 64, 0), nvec),
                            rng.integers(0, nvec, S)]).astype(np.uint64)
        gid = x[:, None] * np.uint64(V) + np.arange(V, dtype=np.uint64)[None, :]
    else:
        g = np.concatenate([np.arange(min(total, 16)), rng.integers(0, total, S)]).astype(np.uint64)
        gid = np.repeat(g[:, None], V, axis=1)
    rows = gid.shape[0]
    vals = [None] * n
    depth = 0
    for i in range(n):
        op = k.ops[i]
        t, a0, a1, imm = op.type, op.arg[0], op.arg[1], op.imm.u
        if t == abi.KOP_GID:
            vals[i] = gid
        elif t == abi.KOP_CONST_U:
            vals[i] = np.full((rows, V), imm, np.uint64)
        elif t == abi.KOP_RANGE:
            trip = max(imm, 1)
            if mode == 1 and depth == 0:
                q = rng.integers(0, max(trip // V, 1), rows).astype(np.uint64)
                q[:2] = [0, max(trip // V, 1) - 1]
                vals[i] = q[:, None] * np.uint64(V) + np.arange(V, dtype=np.uint64)[None, :]
            else:
                r = rng.integers(0, trip, rows).astype(np.uint64)
                r[:2] = [0, trip - 1]
                vals[i] = np.repeat(r[:, None], V, axis=1)
            depth += 1
        elif t == abi.KOP_ENDRANGE:
            depth -= 1
        elif t in (abi.KOP_DIV, abi.KOP_MOD):
            a = vals[a0]
            if a is not None:
                if imm == 0:
                    vals[i] = np.zeros_like(a)
                else:
                    vals[i] = a // np.uint64(imm) if t == abi.KOP_DIV else a % np.uint64(imm)
        elif t == abi.KOP_IDX:
            a, b = vals[a0], vals[a1]
            if a is not None and b is not None:
                vals[i] = (a * np.uint64(imm) + b) & M32
    return vals


def check_claims(k, mode, V, rows, vals):
    """Names of the ops whose claimed classification the values contradict."""
    bad = []
    for i, (kind, o0, o1, o2, o3, dv, hi) in enumerate(rows):
        x = vals[i]
        if x is None or kind >= 2:
            continue
        if x.max() > hi:
            bad.append("op %d: value %d above the bound %d" % (i, int(x.max()), hi))
        off = np.array([o0, o1, o2, o3][:V], np.uint64)
        if kind == 0 and not (off == 0).all():
            bad.append("op %d: invariant with offsets" % i)
        if not (x == x[:, :1] + off[None, :]).all():
            bad.append("op %d: lanes are not lane 0 + %s" % (i, off.tolist()))
        if dv == 0:
            if (x[:, 0] != 0).any():
                bad.append("op %d: lane 0 claimed zero" % i)
        elif (x[:, 0] % np.uint64(dv) != 0).any():
            bad.append("op %d: lane 0 not divisible by %d" % (i, dv))
    return bad


@pytest.mark.parametrize("path", TRACES, ids=[os.path.basename(p) for p in TRACES])
def test_lane_claims_hold(path):
    rng = np.random.default_rng(7)
    n_checked = 0
    for k in _kernels(path):
        if _lib.dense_analyze(k):
            continue
        mode, V, rows = _lib.kernel_lanes(k)
        if V == 1:
            continue
        vals = _values(k, mode, V, 2048, rng)
        bad = check_claims(k, mode, V, rows, vals)
        assert not bad, "%s: %s" % (os.path.basename(path), bad[:5])
        n_checked += 1
    if n_checked == 0:
        pytest.skip("no vectorised generated kernels in this trace")


def test_checker_catches_a_wrong_claim():
    """The check itself has teeth: a claimed offset, divisor or bound that the
    values do not bear out is reported."""
    path = os.path.join(ROOT, "tinyhvm_amd", "workloads", "convblock_b64.trc")
    rng = np.random.default_rng(3)
    for k in _kernels(path):
        if _lib.dense_analyze(k):
            continue
        mode, V, rows = _lib.kernel_lanes(k)
        lin = [i for i, r in enumerate(rows) if r[0] == 1 and r[2] != r[3] and r[5] != 0]
        if mode != 0 or V != 4 or not lin:
            continue
        vals = _values(k, mode, V, 512, rng)
        assert not check_claims(k, mode, V, rows, vals)
        i = lin[0]
        r = list(rows[i])
        wrong = [list(rows) for _ in range(3)]
        wrong[0][i] = tuple(r[:2] + [r[2] + 1] + r[3:])             # an offset
        wrong[1][i] = tuple(r[:5] + [r[5] * 7] + r[6:])      # a divisor
        wrong[2][i] = tuple(r[:6] + [0])                            # the bound
        for w in wrong:
            assert check_claims(k, mode, V, w, vals)
        return
    pytest.fail("no lane-offset op with unequal offsets found")
