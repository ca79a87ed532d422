"""A ctypes driver of the engine's Python FFI library (py/csrc/libthvm.m:52-215,
built with the HIP backend registered as a device into
oracle/_ref/libthvm_py.so by tests/live/py_hip.c).

mlp_step() builds the 2-layer MLP step of the mlp_64x784x128x10 fixture from
py_* calls alone: inputs from the fixture's generator specs (x ~ N(0,1),
Kaiming-uniform W1/W2, zero biases, integer labels), forward
h = relu(x @ W1 + b1), logits = h @ W2 + b2, the softmax cross-entropy loss
-sum(onehot * log_softmax(logits)) / B, and the backward the fixture composes:
d2 = (softmax(logits) - onehot) / B, dW2 = h^T d2, dz1 = (d2 W2^T) * (h > 0),
dW1 = x^T dz1. Returns (loss, dW1, dW2), the fixture's three read-backs.

The engine's lazy terms are linear: an operation consumes the terms it is
given, so a term may feed one consumer only. Input tensors (py_tensor) may be
used any number of times; every intermediate needed twice is therefore built
again from the inputs (the engine's lowering fuses each copy into the kernels
of its consumer), and only the three results are realized and read.
"""
import ctypes as C
import json
import os
import sys

import numpy as np

from tests import tracetools as tt
from tinyhvm_amd import trace

LIB = os.path.join(tt.ROOT, "oracle", "_ref", "libthvm_py.so")
HIP = os.path.join(tt.ROOT, "tinyhvm_amd", "libthvm_hip.so")
FIXTURE = os.path.join(tt.GOLDEN, "mlp_64x784x128x10.trc")

UOP_EXP, UOP_LOG, UOP_RELU = 4, 5, 6
UOP_ADD, UOP_MUL, UOP_DIV, UOP_CMP, UOP_SUB = 9, 10, 11, 13, 14
UOP_SUM, UOP_RMAX, UOP_MM = 15, 16, 17
GEN_UNIFORM, GEN_NORMAL, GEN_INT = 1, 2, 3

_lib = None
STATS = {}


def lib():
    global _lib
    if _lib is None:
        L = C.CDLL(LIB)
        u32, u64, vp = C.c_uint32, C.c_uint64, C.c_void_p
        pu32 = C.POINTER(u32)
        sigs = {
            "py_init": (vp, [C.c_char_p]),
            "py_init_hip": (vp, [C.c_char_p]),
            "py_default_device": (u32, [vp]),
            "py_free": (None, [vp]),
            "py_tensor": (u64, [vp, C.POINTER(C.c_float), pu32, u32]),
            "py_scalar": (u64, [vp, C.c_float]),
            "py_op": (u64, [vp, u32, u64, u64]),
            "py_reduce": (u64, [vp, u64]),
            "py_to_host": (C.POINTER(C.c_float), [vp, u64]),
            "py_numel": (u32, [vp, u64]),
            "py_reshape": (u64, [vp, u64, pu32, u32]),
            "py_expand": (u64, [vp, u64, pu32, u32]),
            "py_permute": (u64, [vp, u64, pu32, u32]),
            "py_era": (u64, []),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def _dims(*d):
    return (C.c_uint32 * len(d))(*d)


class Ctx:
    def __init__(self, device):
        L = lib()
        self.L = L
        self.device = device
        self.ctx = L.py_init_hip(HIP.encode()) if device == "hip" else L.py_init(b"cpu")
        if not self.ctx:
            raise RuntimeError("engine context for %s unavailable" % device)
        # thvm_init("hip") made the HIP backend the default device (2), or
        # stayed on the CPU (0) when the backend's init failed
        STATS.setdefault("default_device", []).append(int(L.py_default_device(self.ctx)))

    def tensor(self, arr):
        a = np.ascontiguousarray(arr, dtype=np.float32)
        return self.L.py_tensor(self.ctx, a.ctypes.data_as(C.POINTER(C.c_float)), _dims(*a.shape), a.ndim)

    def scalar(self, v):
        return self.L.py_scalar(self.ctx, float(v))

    def op(self, uop, a, b=None):
        return self.L.py_op(self.ctx, uop, a, self.L.py_era() if b is None else b)

    def reduce(self, uop, t, axis):
        return self.op(uop, t, self.scalar(axis))

    def reshape(self, t, *d):
        return self.L.py_reshape(self.ctx, t, _dims(*d), len(d))

    def expand(self, t, *d):
        return self.L.py_expand(self.ctx, t, _dims(*d), len(d))

    def transpose(self, t):
        return self.L.py_permute(self.ctx, t, _dims(1, 0), 2)

    def realize(self, t):
        """Evaluate a lazy term into a tensor term that can be used again (the
        engine's lazy terms are consumed by the operation that uses them)."""
        return self.L.py_reduce(self.ctx, t)

    def host(self, t, n):
        p = self.L.py_to_host(self.ctx, t)
        return np.ctypeslib.as_array(p, shape=(n,)).copy()

    def hip_dispatches(self):
        """Kernels the HIP backend has run in this process (its first counter);
        the library is the one py_init_hip loaded, so the counts are its own."""
        h = C.CDLL(HIP)
        h.thvm_hip_counters.restype = C.c_int
        h.thvm_hip_counters.argtypes = [C.POINTER(C.c_uint64), C.c_uint32]
        v = (C.c_uint64 * 16)()
        return int(v[0]) if h.thvm_hip_counters(v, 16) > 0 else -1

    def free(self):
        self.L.py_free(self.ctx)
        if self.device == "hip":
            # thvm_free shut the registered backend down: the library no
            # longer synchronizes
            h = C.CDLL(HIP)
            h.thvm_hip_synchronize.restype = C.c_int
            STATS.setdefault("shut_down_by_free", []).append(h.thvm_hip_synchronize() == -1)


def _gen(dist, dtype, seed, p0, p1, n):
    return np.frombuffer(trace.gen_data(dist, dtype, seed, p0, p1, 4 * n),
                         dtype=np.int32 if dtype == 2 else np.float32)


def mlp_inputs(B=64, IN=784, H=128, NC=10):
    b1 = np.float32(np.sqrt(np.float32(6.0) / np.float32(IN)))
    b2 = np.float32(np.sqrt(np.float32(6.0) / np.float32(H)))
    x = _gen(GEN_NORMAL, 0, 1001, 0.0, 1.0, B * IN).reshape(B, IN)
    W1 = _gen(GEN_UNIFORM, 0, 1002, -b1, b1, IN * H).reshape(IN, H)
    W2 = _gen(GEN_UNIFORM, 0, 1004, -b2, b2, H * NC).reshape(H, NC)
    lab = _gen(GEN_INT, 2, 1006, 0.0, 10.0, B)
    onehot = np.zeros((B, NC), np.float32)
    onehot[np.arange(B), lab] = 1.0
    return x, W1, W2, onehot


def mlp_step(device, B=64, IN=784, H=128, NC=10):
    """(loss, dW1, dW2) of the fixture's MLP step, built from py_* calls."""
    x, W1, W2, onehot = mlp_inputs(B, IN, H, NC)
    c = Ctx(device)
    try:
        tx, tW1, tW2, toh = c.tensor(x), c.tensor(W1), c.tensor(W2), c.tensor(onehot)
        tb1, tb2 = c.tensor(np.zeros(H, np.float32)), c.tensor(np.zeros(NC, np.float32))

        def h():
            z1 = c.op(UOP_ADD, c.op(UOP_MM, tx, tW1), c.expand(c.reshape(tb1, 1, H), B, H))
            return c.op(UOP_RELU, z1)

        def logits():
            return c.op(UOP_ADD, c.op(UOP_MM, h(), tW2), c.expand(c.reshape(tb2, 1, NC), B, NC))

        def shifted():                                                  # logits - rowmax
            return c.op(UOP_SUB, logits(), c.expand(c.reduce(UOP_RMAX, logits(), 1), B, NC))

        def rowsum_exp():                                               # [B, 1]
            return c.reduce(UOP_SUM, c.op(UOP_EXP, shifted()), 1)

        def d2():
            p = c.op(UOP_DIV, c.op(UOP_EXP, shifted()), c.expand(rowsum_exp(), B, NC))
            return c.op(UOP_MUL, c.op(UOP_SUB, p, toh), c.scalar(1.0 / B))

        logp = c.op(UOP_SUB, shifted(), c.expand(c.op(UOP_LOG, rowsum_exp()), B, NC))
        nll = c.reduce(UOP_SUM, c.reduce(UOP_SUM, c.op(UOP_MUL, logp, toh), 1), 0)
        loss = c.realize(c.op(UOP_MUL, nll, c.scalar(-1.0 / B)))
        dW2 = c.realize(c.op(UOP_MM, c.transpose(h()), d2()))
        dz1 = c.op(UOP_MUL, c.op(UOP_MM, d2(), c.transpose(tW2)), c.op(UOP_CMP, h(), c.scalar(0.0)))
        dW1 = c.realize(c.op(UOP_MM, c.transpose(tx), dz1))
        out = c.host(loss, 1), c.host(dW1, IN * H), c.host(dW2, H * NC)
        if device == "hip":
            STATS["mlp_hip_dispatches"] = c.hip_dispatches()
        return out
    finally:
        c.free()


def readme_linear(device):
    """relu(x @ w + b) of the engine README's example (README.md:106-124):
    x [2,3] = 1..6, w [3,2], b [1,2]; the README states [0, 2.6, 0, 5.0]."""
    c = Ctx(device)
    try:
        x = c.tensor(np.arange(1, 7, dtype=np.float32).reshape(2, 3))
        w = c.tensor(np.array([[0.1, -0.2], [0.3, 0.4], [-0.5, 0.6]], np.float32))
        b = c.tensor(np.array([[-0.1, 0.2]], np.float32))
        y = c.realize(c.op(UOP_RELU, c.op(UOP_ADD, c.op(UOP_MM, x, w), c.expand(b, 2, 2))))
        return c.host(y, 4)
    finally:
        c.free()


def fixture_readbacks(path=FIXTURE):
    """The reference engine's read-backs recorded in a fixture, in order."""
    last = {}
    out = []
    for r in trace.read_trace(path):
        if r.tag == trace.SNAPSHOT:
            last[r.f["id"]] = np.frombuffer(r.f["data"], dtype=np.float32)
        elif r.tag == trace.READ:
            out.append(last[r.f["id"]][:r.f["bytes"] // 4])
    return out


def normwise(x, y):
    x, y = np.asarray(x, np.float64), np.asarray(y, np.float64)
    return float(np.max(np.abs(x - y))) / max(float(np.max(np.abs(y))), 1e-30)


def main(device):
    """Runs both workloads on one device and prints one JSON line: the MLP's
    normwise errors against the fixture's read-backs, the README result and,
    for the HIP device, the kernels the backend ran."""
    got = mlp_step(device)
    want = fixture_readbacks()
    res = {"device": device,
           "mlp": {n: normwise(g, w) for n, g, w in zip(("loss", "dW1", "dW2"), got, want)},
           "mlp_shapes_ok": all(g.shape == w.shape for g, w in zip(got, want)) and len(want) == 3,
           "readme": [float(v) for v in readme_linear(device)]}
    res.update(STATS)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "cpu")
