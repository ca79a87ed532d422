"""Matrix-core (f32 MFMA) contraction kernels on the GPU: every committed trace
replayed with every contraction forced onto the matrix-core path (most
fixtures are below the size heuristics), once with the tile shape and split-K
chosen by size, and once per tile shape (128x128, 64x64, 256x32, 32x256,
and the direct per-wave kernel) with
fixed split-K factors, under the same kernel-boundary parity as
tests/test_gpu_parity.py; the matrix-core kernels fall in the 1e-4 normwise
class."""
import os

import pytest

from tests import tracetools as tt
from tests.test_gpu_parity import _oracle, kernel_parity, uop_tolerance
from tinyhvm_amd import _lib

pytestmark = pytest.mark.gpu


# (split-K factor, tile shape): 0 = chosen by size, 1 = 128x128, 2 = 64x64,
# 3 = 256x32, 4 = 32x256, 5 = direct (per-wave 32x32 blocks, no LDS), 6 = 256x64,
# 7 = 128x64, 8 = skinny (a row per lane, for at most 16 columns; wider
# contractions keep the chosen tile), 9 = outer-product reduction (a k per
# lane, for few outputs; others keep the chosen tile), 11 = the wave tile (no
# LDS, a wave per 32 rows by 64 columns; contractions of 64 columns with the
# B side packed, others keep the 64x64 tile). The direct and
# outer-product kernels combine their split-K partials in the same launch;
# "nocomb" sends them through the workspace and the sum kernel instead.
CONFIGS = [("1", "0"), ("2", "0"), ("1", "1"), ("3", "2"), ("1", "3"), ("2", "4"), ("1", "5"), ("3", "5"),
           ("1", "6"), ("3", "6"), ("1", "7"), ("2", "7"), ("8", "2"), ("16", "7"), ("1", "2", "pack"),
           ("2", "7", "pack"), ("1", "8"), ("1", "8", "noskblk"), ("1", "9"), ("8", "5"), ("3", "5", "nocomb"),
           ("1", "9", "nocomb"), ("1", "11", "pack")]


@pytest.fixture(scope="module", params=CONFIGS,
                ids=["whole-K", "split-K", "tile128x128", "tile64x64-split3", "tile256x32",
                     "tile32x256-split2", "direct", "direct-split3", "tile256x64", "tile256x64-split3",
                     "tile128x64", "tile128x64-split2", "tile64x64-split8", "tile128x64-split16",
                     "tile64x64-packed", "tile128x64-split2-packed", "skinny", "skinny-per-k",
                     "outer-product", "direct-split8", "direct-split3-sum-kernel", "outer-product-sum-kernel",
                     "wave-tile-packed"])
def hip_dense(request):
    saved = {k: os.environ.get(k) for k in ("THVM_HIP_DENSE_FORCE", "THVM_HIP_DENSE_SPLITS",
                                             "THVM_HIP_DENSE_TILE", "THVM_HIP_DENSE_PACK", "THVM_HIP_DENSE_NOSKBLK",
                                             "THVM_HIP_DENSE_NOCOMB")}
    os.environ["THVM_HIP_DENSE_FORCE"] = "1"
    os.environ["THVM_HIP_DENSE_SPLITS"], os.environ["THVM_HIP_DENSE_TILE"] = request.param[:2]
    os.environ["THVM_HIP_DENSE_PACK"] = "1" if request.param[2:] == ("pack",) else "0"
    os.environ["THVM_HIP_DENSE_NOSKBLK"] = "1" if request.param[2:] == ("noskblk",) else "0"
    os.environ["THVM_HIP_DENSE_NOCOMB"] = "1" if request.param[2:] == ("nocomb",) else "0"
    L = _lib.lib()
    assert L.thvm_hip_init() == 0
    yield L
    L.thvm_hip_shutdown()
    for k, v in saved.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v


def dense_tolerance(k):
    if _lib.dense_analyze(k):
        return "norm", 1e-4
    return uop_tolerance(k)


@pytest.mark.parametrize("path", tt.fixtures(), ids=lambda p: p.split("/")[-1])
def test_trace_parity_matrix_cores(hip_dense, path):
    L = hip_dense
    kr, e2e = kernel_parity(L.thvm_hip_backend(), L.thvm_hip_buf_read, L.thvm_hip_synchronize,
                            _oracle(), path, tol_fn=dense_tolerance)
    bad = [r for r in kr if not r[1]]
    assert not bad, "kernel parity: %s" % bad
    bad_e2e = [r for r in e2e if not r[1]]
    assert not bad_e2e, "end-to-end vs reference: %s" % bad_e2e


def test_contraction_timing_events():
    """thvm_hip_time_contraction: armed with two events, the next contraction
    dispatch records them on the backend stream around its main kernel (it
    reports 1 when disarmed after it, and the pair measures a positive
    time); a dispatch that is no contraction leaves them unrecorded (0). The
    buffers after the step match a run without the events bit for bit."""
    import ctypes as C
    from tinyhvm_amd import trace
    path = os.path.join(tt.ROOT, "tests", "golden", "mlp_64x784x128x10.trc")
    sizes = {r.f["id"]: r.f["bytes"] for r in trace.read_trace(path) if r.tag == trace.ALLOC}
    hip = C.CDLL("libamdhip64.so")
    hip.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
    hip.hipEventSynchronize.argtypes = [C.c_void_p]
    hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
    hip.hipEventDestroy.argtypes = [C.c_void_p]
    L = _lib.lib()

    def run(timed):
        L.thvm_hip_shutdown()
        assert L.thvm_hip_init() == 0
        rp = tt.Replay(path, L.thvm_hip_backend())
        fired, ms = [], []
        try:
            for i in range(rp.n):
                k = rp.kernel(i) if rp.tag(i) == trace.UOP else None
                if not (timed and k is not None):
                    rp.run(i, i + 1)
                    continue
                ea, eb = C.c_void_p(), C.c_void_p()
                assert hip.hipEventCreate(C.byref(ea)) == 0 and hip.hipEventCreate(C.byref(eb)) == 0
                assert L.thvm_hip_time_contraction(ea, eb) == 0
                rp.run(i, i + 1)
                f = L.thvm_hip_time_contraction(None, None)
                fired.append((bool(_lib.dense_analyze(k)), f))
                if f == 1:
                    assert hip.hipEventSynchronize(eb) == 0
                    t = C.c_float()
                    assert hip.hipEventElapsedTime(C.byref(t), ea, eb) == 0
                    ms.append(t.value)
                hip.hipEventDestroy(ea)
                hip.hipEventDestroy(eb)
            assert L.thvm_hip_synchronize() == 0
            outs = {}
            for tid, n in sizes.items():
                live = rp.live(tid)
                if live:
                    buf = (C.c_uint8 * n)()
                    L.thvm_hip_buf_read(live, buf, n)
                    outs[tid] = bytes(buf)
            return fired, ms, outs
        finally:
            rp.close()

    fired, ms, got = run(True)
    _f, _m, want = run(False)
    L.thvm_hip_shutdown()
    assert any(c for c, _ in fired) and any(not c for c, _ in fired), fired
    assert all(f == (1 if c else 0) for c, f in fired), fired
    assert ms and all(t > 0.0 for t in ms), ms
    assert got.keys() == want.keys() and got == want
