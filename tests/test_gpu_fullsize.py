"""Parity at the benchmark workloads' full sizes, on the GPU.

  fused 8192x8192   dA = (a*b + c > 0) * b checked bit for bit against numpy
                    float32 (the same two roundings per element); y =
                    sum(relu(a*b + c), -1) within 1e-4 normwise of float64
                    sums (the group reduction reorders the sum).
  matmul 4096^3     y = relu(X @ W + b), dX = G @ W^T, dW = X^T @ G with
                    G = (y > 0): 64 sampled rows of y and dX and 64 sampled
                    columns of dW against float64 dot products, 1e-4 normwise
                    (matrix-core accumulation order), and the relu mask G
                    bit for bit against y.
  LeNet-5 B=256     every dispatch of one training step against the oracle on
                    the GPU's own inputs (the kernel-boundary parity of
                    tests/test_gpu_parity.py at the benchmark batch).
  conv block B=64   the same for the 28 dispatches of the conv block's forward
                    and backward at [64,64,56,56]. The three 14.8 GFLOP
                    convolutions are too large for the oracle whole: each is
                    checked (1) on the oracle over a sample of outputs that
                    takes one output from every run of 64 consecutive pixels
                    (every 64-row tile of the forward and input-gradient
                    GEMMs, 3136 of them) or every 64 consecutive weights
                    (every tile of the weight gradient), plus random ones and
                    both ends; (2) with the output filled with a NaN sentinel
                    before the dispatch, none of which may survive it: every
                    output, in every tile and split, is written; (3) against
                    the textbook sliding-window convolution in float64 on
                    2048 sampled outputs, computed from the kernel's own input
                    buffers.

Inputs are the traces' generator specs materialized on the host, so the
numpy side sees exactly the bytes the GPU was given.
"""
import ctypes as C
import os

import numpy as np
import pytest

from tests import tracetools as tt
from tests.test_gpu_parity import _oracle, kernel_parity
from tinyhvm_amd import _lib, trace

pytestmark = pytest.mark.gpu

WL = os.path.join(tt.ROOT, "tinyhvm_amd", "workloads")


@pytest.fixture(scope="module")
def hip():
    saved = os.environ.pop("THVM_HIP_DENSE_FORCE", None)
    L = _lib.lib()
    assert L.thvm_hip_init() == 0, "HIP backend failed to initialise"
    yield L
    L.thvm_hip_shutdown()
    if saved is not None:
        os.environ["THVM_HIP_DENSE_FORCE"] = saved


def _gen_inputs(recs):
    """seed -> (trace id, float32 array) for every generated input."""
    out = {}
    for r in recs:
        if r.tag == trace.WRITE and r.f["enc"] == trace.ENC_GEN:
            f = r.f
            data = trace.gen_data(f["dist"], f["dtype"], f["seed"], f["p0"], f["p1"], f["bytes"])
            out[f["seed"]] = (f["id"], np.frombuffer(data, dtype=np.float32))
    return out


def _replay_outputs(L, path):
    """Replays the whole trace on the GPU; returns (records, generated inputs,
    [output array of each dispatch, read right after it])."""
    recs = trace.read_trace(path)
    sizes = {}
    outs = []
    rp = tt.Replay(path, L.thvm_hip_backend())
    try:
        for i, r in enumerate(recs):
            if r.tag == trace.ALLOC:
                sizes[r.f["id"]] = r.f["bytes"]
            rp.run(i, i + 1)
            if r.tag == trace.UOP:
                n = sizes[r.f["out"]]
                buf = np.empty(n // 4, dtype=np.float32)
                L.thvm_hip_buf_read(rp.live(r.f["out"]), buf.ctypes.data_as(C.c_void_p), n)
                outs.append(buf)
        assert L.thvm_hip_synchronize() == 0
    finally:
        rp.close()
    return recs, _gen_inputs(recs), outs


def normwise(x, y):
    x, y = np.asarray(x, np.float64), np.asarray(y, np.float64)
    return float(np.max(np.abs(x - y))) / max(float(np.max(np.abs(y))), 1e-30)


def test_fused_8192(hip):
    recs, gens, outs = _replay_outputs(hip, os.path.join(WL, "fused_8192x8192.trc"))
    R = Cn = 8192
    a, b, c = (gens[s][1].reshape(R, Cn) for s in (2001, 2002, 2003))
    y, da = outs[0][:R], outs[1].reshape(R, Cn)
    pre = (a * b) + c                      # float32, the kernel's two roundings
    want_da = (pre > 0).astype(np.float32) * b
    assert np.array_equal(da, want_da), "dA differs in %d elements" % int(np.sum(da != want_da))
    y_ref = np.maximum(a.astype(np.float64) * b + c, 0).sum(axis=1)
    err = normwise(y, y_ref)
    assert err <= 1e-4, "y normwise %.2e" % err


def test_matmul_4096(hip):
    recs, gens, outs = _replay_outputs(hip, os.path.join(WL, "linear_4096.trc"))
    n = 4096
    X, W, bias = gens[3001][1].reshape(n, n), gens[3002][1].reshape(n, n), gens[3003][1]
    y0, y, G, dX, G2, dW = (o[:n * n].reshape(n, n) for o in outs)
    rng = np.random.default_rng(7)
    rows = rng.choice(n, 64, replace=False)
    cols = rng.choice(n, 64, replace=False)
    Xd, Wd = X.astype(np.float64), W.astype(np.float64)
    err = normwise(y0[rows], Xd[rows] @ Wd)
    assert err <= 1e-4, "X @ W normwise %.2e" % err
    # bias + relu and the masks are elementwise on the GPU's own y0 / y: exact
    assert np.array_equal(y, np.maximum(y0 + bias, np.float32(0)))
    assert np.array_equal(G, (y > 0).astype(np.float32)) and np.array_equal(G2, G)
    Gd = G.astype(np.float64)
    err = normwise(dX[rows], Gd[rows] @ Wd.T)
    assert err <= 1e-4, "dX normwise %.2e" % err
    err = normwise(dW[:, cols], Xd.T @ Gd[:, cols])
    assert err <= 1e-4, "dW normwise %.2e" % err


@pytest.mark.timeout(600)
def test_lenet_b256_kernel_parity(hip):
    ora = _oracle()
    kr, _e2e = kernel_parity(hip.thvm_hip_backend(), hip.thvm_hip_buf_read, hip.thvm_hip_synchronize,
                             ora, os.path.join(WL, "lenet_b256.trc"))
    assert len(kr) >= 54
    bad = [r for r in kr if not r[1]]
    assert not bad, "kernel parity: %s" % bad


ORACLE_MACS = 150_000_000
B, CH, HW, W = 64, 64, 56 * 56, 56


def _total(k):
    return k.grid[0] if k.local_size > 0 else k.grid[0] * k.grid[1] * k.grid[2]


def _conv_sample(k):
    """gids of a too-large contraction for the oracle: one per 64-row tile
    and random extras (see the module docstring); None for the rest."""
    a = _lib.dense_analyze(k)
    if not a:
        return None
    M, N, K, _splits = a
    if M * N * K <= ORACLE_MACS:
        return None
    total = _total(k)
    rng = np.random.default_rng(K)
    if total == B * CH * HW:
        # output [B, C, 56, 56]: pixel m = b*HW + p, one per run of 64 pixels
        m = np.arange(0, B * HW, 64) + rng.integers(0, 64, B * HW // 64)
        b, p = m // HW, m % HW
        gids = (b * CH + rng.integers(0, CH, len(m))) * HW + p
        extra = rng.integers(0, total, 20000)
    else:
        # weight gradient [Co, Ci, 3, 3]: one per run of 64 consecutive weights
        gids = np.arange(0, total, 64) + rng.integers(0, 64, (total + 63) // 64)
        extra = rng.integers(0, total, 64)
    gids = np.concatenate([[0, total - 1], gids, extra])
    return np.unique(np.minimum(gids, total - 1))


def _textbook_conv(i, k, leaves, got):
    """The 3x3 convolutions in float64 from the kernel's own inputs:
    out[b,o,y,x] = sum_{i,ky,kx} big[b,i,y+ky,x+kx] * w[o,i,ky,kx] (forward,
    and the input gradient with the flipped transposed kernel), or
    dW[o,i,ky,kx] = sum_{b,y,x} xp[b,i,y+ky,x+kx] * dz[b,o,y,x]."""
    big_n, w_n, dz_n = B * CH * 58 * 58 * 4, CH * CH * 9 * 4, B * CH * HW * 4
    by = {len(x): np.frombuffer(x, dtype=np.float32) for x in leaves}
    out = np.frombuffer(got, dtype=np.float32)
    rng = np.random.default_rng(i)
    if big_n in by and w_n in by:
        big = by[big_n].reshape(B, CH, 58, 58)
        w = by[w_n].reshape(CH, CH, 3, 3).astype(np.float64)
        sel = rng.integers(0, B * CH * HW, 2048)
        b, o, y, x = sel // (CH * HW), sel // HW % CH, sel % HW // W, sel % W
        want = np.array([np.sum(big[bb, :, yy:yy + 3, xx:xx + 3].astype(np.float64) * w[oo])
                         for bb, oo, yy, xx in zip(b, o, y, x)])
        have = out[sel]
    elif big_n in by and dz_n in by:
        xp = by[big_n].reshape(B, CH, 58, 58)
        dz = by[dz_n].reshape(B, CH, 56, 56).astype(np.float64)
        sel = rng.integers(0, CH * CH * 9, 64)
        o, ii, ky, kx = sel // (CH * 9), sel // 9 % CH, sel % 9 // 3, sel % 3
        want = np.array([np.sum(xp[:, ci, a:a + 56, c:c + 56].astype(np.float64) * dz[:, oo])
                         for oo, ci, a, c in zip(o, ii, ky, kx)])
        have = out[sel]
    else:
        return None
    err = normwise(have, want)
    return err <= 1e-4, "textbook float64 conv %.2e over %d outputs" % (err, len(sel))


@pytest.mark.timeout(900)
def test_convblock_b64_kernel_parity(hip):
    ora = _oracle()
    kr, _e2e = kernel_parity(hip.thvm_hip_backend(), hip.thvm_hip_buf_read, hip.thvm_hip_synchronize,
                             ora, os.path.join(WL, "convblock_b64.trc"), sample_fn=_conv_sample,
                             extra_fn=_textbook_conv, write_fn=hip.thvm_hip_buf_write)
    assert len(kr) >= 28
    sampled = [r for r in kr if "sampled" in r[2]]
    assert len(sampled) == 3, [r[2] for r in kr]
    assert all("every output written" in r[2] and "textbook" in r[2] for r in sampled), sampled
    bad = [r for r in kr if not r[1]]
    assert not bad, "kernel parity: %s" % bad
