"""Textbook checks of the convolution-shaped kernels in the LeNet-5 and conv
block fixtures, on the oracle's own inputs and outputs.

The golden vectors pin the oracle to the engine bit for bit; these checks pin
what the workloads compute against the mathematics, independent of both, so a
kernel program that is faithfully reproduced but computes the wrong function
(a lost pad mask, a wrong stride) is caught too. Each dispatch is classified
by its iteration domain and restated in numpy float64:

  conv       out[b,o,i,j] = sum_{c,u,v} x[b,c,i+u,j+v] * w[o,c,u,v]
             (the input is already zero padded: forward convs, and the input
             gradient as the conv of padded dz with the flipped, transposed
             kernel)
  conv dW    dW[o,c,u,v]  = sum_{b,i,j} x[b,c,i+u,j+v] * dz[b,o,i,j]
  pad        xp = x zero-padded by p on both spatial sides (bit-exact)
  pool bwd   dz = up2(dp) * (1 - (up2(pooled) > a)) * (a > 0)   (ties-to-all
             routing, src/interact/grad.c:405-425; bit-exact in f32)

Sums are compared normwise within 1e-5 (f32 sequential accumulation against
f64). A planted mistake (an unflipped kernel, a shifted window, a dropped
relu mask) must fail the same checks.

Ties: ties at positive values, where ties-to-all and first-max routing
differ, do not occur in random data. The pooltie fixture (integer-valued
activations) has them in most windows; its engine snapshots of the forward
pools and of both routings are checked bit for bit against brute force with
the ties-to-all rule, and a first-max rule must fail the same check.
"""
import ctypes as C

import numpy as np
import pytest
from numpy.lib.stride_tricks import sliding_window_view

from tests import tracetools as tt
from tinyhvm_amd import trace

FIXTURES = {"lenet_b2.trc": {"conv": 3, "conv_dw": 2, "pool_bwd": 2, "pad": 2},
            "convblock_2x4x8.trc": {"conv": 2, "conv_dw": 1, "pool_bwd": 1, "pad": 2},
            "rs_convblock_2x4x8.trc": {"conv": 2, "conv_dw": 1, "pool_bwd": 1, "pad": 2}}


def conv_ref(x, w):
    K = w.shape[-1]
    win = sliding_window_view(x.astype(np.float64), (K, K), axis=(2, 3))   # [B,C,OH,OW,K,K]
    return np.einsum("bcijuv,ocuv->boij", win, w.astype(np.float64))


def conv_dw_ref(x, dz, K):
    win = sliding_window_view(x.astype(np.float64), (K, K), axis=(2, 3))
    return np.einsum("bcijuv,boij->ocuv", win, dz.astype(np.float64))


def maxpool2(a):
    B, Cc, H, W = a.shape
    return a.reshape(B, Cc, H // 2, 2, W // 2, 2).max(axis=(3, 5))


def pool_relu_bwd_ref(dp, pooled, a6, relu_mask=True):
    """a6 is the activation in [B,C,H/2,2,W/2,2]; dp and pooled are [B,C,H/2,W/2]."""
    up = lambda t: t[:, :, :, None, :, None]  # noqa: E731  stride-0 upsample
    routed = np.float32(1.0) - (up(pooled) > a6).astype(np.float32)
    g = up(dp) * routed
    return g * (a6 > 0).astype(np.float32) if relu_mask else g


def normwise(x, y):
    x, y = np.asarray(x, np.float64), np.asarray(y, np.float64)
    return float(np.max(np.abs(x - y))) / max(float(np.max(np.abs(y))), 1e-30)


def _dispatches(path):
    """(record index, record, leaf arrays, output array) for every dispatch of
    the trace, replayed through the oracle."""
    recs = trace.read_trace(path)
    ora = tt.oracle()
    be = ora.oracle_backend_ptr()
    be.contents.init()
    rp = tt.Replay(path, be)
    sizes, out = {}, []

    def grab(tid):
        n = sizes.get(tid, 0)
        if not n:
            return np.zeros(0, np.float32)
        return np.frombuffer(C.string_at(ora.oracle_buf_ptr(rp.live(tid)), n), dtype=np.float32).copy()

    try:
        for i, r in enumerate(recs):
            if r.tag == trace.ALLOC:
                sizes[r.f["id"]] = r.f["bytes"]
            if r.tag in (trace.UOP, trace.RS):
                leaves = [grab(t) for t in r.f["leaf_bufs"]]
                rp.run(i, i + 1)
                out.append((i, r, leaves, grab(r.f["out"])))
            else:
                rp.run(i, i + 1)
    finally:
        rp.close()
        be.contents.shutdown()
    return out


def _square_side(n):
    s = int(round(n ** 0.5))
    return s if s * s == n else None


def check_dispatch(r, leaves, got, mistake=None):
    """Returns (kind, ok, msg), or None for a dispatch of another shape."""
    d = list(r.f["full_dims"][:r.f["full_rank"]])
    if len(d) == 8 and d[1] == 1 and len(leaves) in (2, 3):    # [B,1,Co,OH,OW,Ci,K,K]: conv
        B, _, Co, OH, OW, Ci, K, K2 = d
        H = OH + K - 1
        ws = [a for a in leaves if a.size == Co * Ci * K * K]
        xs = [a for a in leaves if a.size == B * Ci * H * H]
        if K != K2 or OH != OW or not ws or not xs:
            return None
        x, w = xs[0].reshape(B, Ci, H, H), ws[-1].reshape(Co, Ci, K, K)
        if mistake == "flip":
            w = w[:, :, ::-1, ::-1]
        want = conv_ref(x, w)
        g = got.reshape(B, Co, OH, OW)
        if mistake == "shift":
            g = np.roll(g, 1, axis=3)
        # a fused bias + relu epilogue is not part of these kernels
        err = normwise(g, want)
        return "conv", err <= 1e-5, "normwise %.2e" % err
    if len(d) == 7 and len(leaves) == 2:                       # [Co,Ci,K,K,B,OY,OX]: conv dW
        Co, Ci, K, _, B, OY, OX = d
        H = OY + K - 1
        errs = []
        # x and dz can have the same size: try both roles (swapping them is a
        # different function, so only the right one matches)
        for dz, x in (leaves, leaves[::-1]):
            if dz.size != B * Co * OY * OX or x.size != B * Ci * H * H:
                continue
            xx = x.reshape(B, Ci, H, H)
            if mistake == "shift":
                xx = np.roll(xx, 1, axis=3)
            errs.append(normwise(got.reshape(Co, Ci, K, K), conv_dw_ref(xx, dz.reshape(B, Co, OY, OX), K)))
        if not errs:
            return None
        err = min(errs)
        return "conv_dw", err <= 1e-5, "normwise %.2e" % err
    if len(d) == 6 and d[3] == 2 and d[5] == 2 and len(leaves) >= 3:   # pool + relu backward
        B, Cc, h, _, w, _ = d
        big = [a for a in leaves if a.size == B * Cc * h * w * 4]
        halves = [a.reshape(B, Cc, h, w) for a in leaves if a.size == B * Cc * h * w]
        if not big or not halves:
            return None
        a6 = big[0].reshape(B, Cc, h, 2, w, 2)
        a4 = a6.reshape(B, Cc, 2 * h, 2 * w)
        pooled_ix = [j for j, t in enumerate(halves) if np.array_equal(t, maxpool2(a4))]
        if not pooled_ix:
            return "pool_bwd", False, "no leaf equals maxpool2(a)"
        pooled = halves[pooled_ix[0]]
        others = [t for j, t in enumerate(halves) if j != pooled_ix[0]]
        dp = others[0] if others else pooled
        want = pool_relu_bwd_ref(dp, pooled, a6, relu_mask=(mistake != "no_relu"))
        ok = np.array_equal(got.reshape(a6.shape), want)
        return "pool_bwd", ok, "bit-exact" if ok else "differs"
    if len(d) == 4 and len(leaves) == 2 and d[2] == d[3]:      # zero padding (times 1)
        B, Cc, Hp, _ = d
        xs = [a for a in leaves if a.size > 1 and _square_side(a.size // (B * Cc))]
        if not xs or got.size != B * Cc * Hp * Hp:
            return None
        H = _square_side(xs[0].size // (B * Cc))
        p = (Hp - H) // 2
        if p <= 0 or H + 2 * p != Hp:
            return None
        want = np.pad(xs[0].reshape(B, Cc, H, H), ((0, 0), (0, 0), (p, p), (p, p)))
        if mistake == "shift":
            want = np.roll(want, 1, axis=3)
        ok = np.array_equal(got.reshape(B, Cc, Hp, Hp), want)
        return "pad", ok, "bit-exact" if ok else "differs"
    return None


@pytest.mark.parametrize("name", sorted(FIXTURES))
def test_conv_kernels_match_textbook(name):
    counts = {}
    for i, r, leaves, got in _dispatches(tt.fixtures(name)[0]):
        res = check_dispatch(r, leaves, got)
        if res is None:
            continue
        kind, ok, msg = res
        assert ok, "%s dispatch record %d (%s): %s" % (name, i, kind, msg)
        counts[kind] = counts.get(kind, 0) + 1
    assert counts == FIXTURES[name]


def test_planted_mistakes_fail():
    first = {}
    for i, r, leaves, got in _dispatches(tt.fixtures("lenet_b2.trc")[0]):
        res = check_dispatch(r, leaves, got)
        if res is not None:
            first.setdefault(res[0], (r, leaves, got))
    assert set(first) == {"conv", "conv_dw", "pool_bwd", "pad"}
    r, leaves, got = first["conv"]
    assert not check_dispatch(r, leaves, got, mistake="flip")[1]
    assert not check_dispatch(r, leaves, got, mistake="shift")[1]
    r, leaves, got = first["conv_dw"]
    assert not check_dispatch(r, leaves, got, mistake="shift")[1]
    r, leaves, got = first["pad"]
    assert not check_dispatch(r, leaves, got, mistake="shift")[1]
    # windows of zeros (relu outputs) route to all four inputs, where only the
    # relu mask zeroes the gradient: dropping it must be caught
    r, leaves, got = first["pool_bwd"]
    assert not check_dispatch(r, leaves, got, mistake="no_relu")[1]


def _pooltie():
    path = tt.fixtures("pooltie_2x4x16.trc")[0]
    recs = trace.read_trace(path)
    gens, snaps = {}, {}
    for r in recs:
        if r.tag == trace.WRITE and r.f["enc"] == trace.ENC_GEN:
            f = r.f
            gens[f["seed"]] = np.frombuffer(trace.gen_data(f["dist"], f["dtype"], f["seed"], f["p0"], f["p1"],
                                                           f["bytes"]), dtype=np.float32)
        if r.tag == trace.SNAPSHOT:
            snaps[r.f["id"]] = np.frombuffer(r.f["data"], dtype=np.float32)
    B, Cc, H = 2, 4, 16
    x = gens[8001].reshape(B, Cc, H, H)
    g = gens[8002].reshape(B, Cc, H // 2, H // 2)
    return x, g, snaps


def _first_max_bwd(dp, a):
    """The alternative rule: only the first maximum of each window (row-major)
    receives the gradient."""
    B, Cc, H, W = a.shape
    win = a.reshape(B, Cc, H // 2, 2, W // 2, 2).transpose(0, 1, 2, 4, 3, 5).reshape(B, Cc, H // 2, W // 2, 4)
    first = np.argmax(win, axis=-1)
    out = np.zeros_like(win)
    np.put_along_axis(out, first[..., None], dp[..., None], axis=-1)
    return out.reshape(B, Cc, H // 2, W // 2, 2, 2).transpose(0, 1, 2, 4, 3, 5).reshape(B, Cc, H, W)


def test_pool_ties_fixture_has_positive_ties():
    x, _g, _s = _pooltie()
    a = np.maximum(x, 0)
    win = a.reshape(2, 4, 8, 2, 8, 2).transpose(0, 1, 2, 4, 3, 5).reshape(-1, 4)
    mx = win.max(axis=1)
    ties = (win == mx[:, None]).sum(axis=1)
    assert np.sum((mx > 0) & (ties >= 2)) >= 20
    assert set(np.unique(x)) == {-1.0, 0.0, 1.0, 2.0}


def test_pool_ties_routing_is_ties_to_all():
    """Engine snapshots of the pooltie workload: forward pools, the pool+relu
    routing of g and the plain routing of g, bit for bit against brute force;
    a first-max rule differs from them."""
    x, g, snaps = _pooltie()
    a = np.maximum(x, np.float32(0))
    p, px = maxpool2(a), maxpool2(x)
    assert np.array_equal(snaps[8].reshape(p.shape), p)
    assert np.array_equal(snaps[13].reshape(px.shape), px)
    s6 = (2, 4, 8, 2, 8, 2)
    da = pool_relu_bwd_ref(g, p, a.reshape(s6)).reshape(x.shape)
    dx = pool_relu_bwd_ref(g, px, x.reshape(s6), relu_mask=False).reshape(x.shape)
    assert np.array_equal(snaps[20].reshape(x.shape), da)
    assert np.array_equal(snaps[28].reshape(x.shape), dx)
    # every tied maximum got the window's gradient: the routed total per window
    # is g times the number of maxima, not g
    assert not np.array_equal(snaps[28].reshape(x.shape), _first_max_bwd(g, x))
    first_relu = _first_max_bwd(g, a) * (a > 0)
    assert not np.array_equal(snaps[20].reshape(x.shape), first_relu)
