"""Shared test helpers: fixture discovery, the oracle binding, trace replay
against a Backend vtable and the tolerance rules for comparing outputs."""
import ctypes as C
import glob
import os
import subprocess

import numpy as np

from tinyhvm_amd import _lib, abi, trace

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "liboracle.so")

TRC_SNAPSHOT = 13
TRC_UOP = 7
TRC_RS = 8

_oracle = None


def oracle():
    """The C restatement (oracle/oracle.c), built on demand with make."""
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_SO):
            subprocess.run(["make", "-s", "-C", ORACLE_DIR, "liboracle.so"], check=True)
        L = C.CDLL(ORACLE_SO)
        L.oracle_backend_ptr.restype = C.POINTER(abi.Backend)
        L.oracle_buf_ptr.restype = C.c_void_p
        L.oracle_buf_ptr.argtypes = [C.c_uint32]
        L.oracle_buf_size.restype = C.c_uint64
        L.oracle_buf_size.argtypes = [C.c_uint32]
        _oracle = L
    return _oracle


def fixtures(pattern="*.trc"):
    return sorted(glob.glob(os.path.join(GOLDEN, pattern)))


def close(x, y, rtol):
    """|x - y| <= rtol * max(|y|, 1e-3 * max|y|): relative error with a floor
    for entries that cross zero."""
    x = np.asarray(x, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    if x.shape != y.shape:
        return False, "shape %s vs %s" % (x.shape, y.shape)
    if x.size == 0:
        return True, "empty"
    scale = np.maximum(np.abs(y), 1e-3 * max(np.max(np.abs(y)), 1e-30))
    err = np.abs(x - y) / scale
    worst = float(np.max(err))
    return worst <= rtol, "max scaled error %.3e (rtol %.1e)" % (worst, rtol)


class Replay:
    """A loaded trace replayed record by record against one Backend."""

    def __init__(self, path, backend_ptr):
        self.L = _lib.lib()
        self.path = path
        self.t = self.L.thvm_trace_load(path.encode())
        if not self.t:
            raise RuntimeError("cannot load trace %s" % path)
        self.be = backend_ptr
        self.n = self.L.thvm_trace_count(self.t)

    def tag(self, i):
        return self.L.thvm_trace_tag(self.t, i)

    def run(self, lo, hi, flags=0):
        return self.L.thvm_trace_replay(self.t, self.be, lo, hi, flags)

    def live(self, trace_id):
        return self.L.thvm_trace_live_id(self.t, trace_id)

    def snapshot(self, i):
        nb = self.L.thvm_trace_rec_bytes(self.t, i)
        p = self.L.thvm_trace_rec_data(self.t, i)
        return self.L.thvm_trace_rec_id(self.t, i), C.string_at(p, nb) if nb else b""

    def kernel(self, i):
        k = self.L.thvm_trace_rec_kernel(self.t, i)
        return k.contents if k else None

    def close(self):
        if self.t:
            self.L.thvm_trace_release(self.t, self.be)
            self.L.thvm_trace_free(self.t)
            self.t = None


def dtype_of_kernel(k):
    return {0: np.float32, 1: np.uint16, 2: np.int32, 3: np.uint32}[k.out_dtype]
