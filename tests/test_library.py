"""CPU-side checks of the HIP backend library: it loads, exports every symbol
declared in include/*.h, its struct layouts match the engine's ABI, and the
kernel generator produces HIP that hipRTC compiles for gfx950 for every
kernel in the committed traces (no GPU needed for any of this)."""
import ctypes as C
import os
import re
import shutil
import subprocess

import pytest

from tests import tracetools as tt
from tinyhvm_amd import _lib, abi, trace

INCLUDE = os.path.join(tt.ROOT, "include")


def _declared_functions():
    names = set()
    for h in ("thvm_hip.h", "thvm_replay.h"):
        text = open(os.path.join(INCLUDE, h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(thvm_\w+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    missing = [n for n in sorted(_declared_functions() | {"hip_backend"}) if not hasattr(L, n)]
    assert not missing, missing


def test_struct_sizes_match_abi():
    L = _lib.lib()
    out = (C.c_uint32 * 4)()
    L.thvm_hip_abi_sizes(out, 4)
    assert list(out) == [212, 852, 24184, 208]
    assert [C.sizeof(abi.View), C.sizeof(abi.ShapeTracker), C.sizeof(abi.UOpKernel),
            C.sizeof(abi.Backend)] == list(out)


PROBE = r'''
#include <stddef.h>
#include <stdio.h>
#include "%s"
#define O(T, f) printf(#T "." #f " %%zu\n", offsetof(T, f))
#define S(T) printf(#T " %%zu\n", sizeof(T))
int main(void) {
  S(Shape); S(View); S(ShapeTracker); S(FusedOp); S(ReduceSpec); S(KOp); S(UOpKernel); S(Backend);
  O(View, strides); O(View, offset); O(View, numel); O(View, has_mask); O(View, mask_begin);
  O(View, mask_end); O(View, n_compound_masks); O(View, compound_masks); O(View, mod_size);
  O(ShapeTracker, n_views); O(ReduceSpec, reduce_type); O(ReduceSpec, is_reduce2);
  O(UOpKernel, n_ops); O(UOpKernel, leaf_views); O(UOpKernel, leaf_dtypes); O(UOpKernel, rank);
  O(UOpKernel, full_shape); O(UOpKernel, grid); O(UOpKernel, local_size); O(UOpKernel, out_dtype);
  O(Backend, dispatch_kernel_rs); O(Backend, dispatch_uop_kernel); O(Backend, adam_step);
  O(Backend, pool_reset); O(Backend, profile_reset);
  return 0;
}
'''


def _probe(header, incdir, tmp_path, tag):
    src = tmp_path / ("probe_%s.c" % tag)
    src.write_text(PROBE % header)
    exe = tmp_path / ("probe_%s" % tag)
    subprocess.run(["gcc", "-std=gnu11", "-w", "-I" + incdir, str(src), "-o", str(exe)], check=True)
    return subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout


@pytest.mark.skipif(not os.path.exists("/root/reference/src/tinyhvm.h"),
                    reason="engine sources not present")
def test_layout_matches_engine_header(tmp_path):
    """Every offset the backend depends on, compiled against the engine's own
    header (src/tinyhvm.h) and against include/thvm_abi.h."""
    ours = _probe("thvm_abi.h", INCLUDE, tmp_path, "ours")
    theirs = _probe("tinyhvm.h", "/root/reference/src", tmp_path, "engine")
    assert ours == theirs


def _has_uop(path):
    return any(r.tag == trace.UOP for r in trace.read_trace(path))


@pytest.mark.parametrize("path", [p for p in tt.fixtures() if _has_uop(p)], ids=lambda p: p.split("/")[-1])
def test_generated_kernels_compile(path):
    for r in trace.read_trace(path):
        if r.tag == trace.UOP:
            assert _lib.compile_check(trace.to_uop_kernel(r)) > 0


def test_generator_rejects_malformed_programs():
    k = abi.UOpKernel()
    k.n_ops = 2
    k.ops[0].type = abi.KOP_RANGE
    k.ops[0].imm.u = 4
    k.ops[1].type = abi.KOP_GID
    with pytest.raises(ValueError, match="unterminated"):
        _lib.kernel_source(k)
    k2 = abi.UOpKernel()
    k2.n_ops = 1
    k2.ops[0].type = abi.KOP_IDX
    k2.ops[0].arg[0] = 5
    with pytest.raises(ValueError, match="earlier op"):
        _lib.kernel_source(k2)


def test_init_without_gpu_fails_cleanly():
    """Without a device, init reports failure instead of crashing (the engine
    then keeps the CPU backend)."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    assert _lib.lib().thvm_hip_init() == -1
