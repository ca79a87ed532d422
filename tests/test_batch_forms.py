"""Device-function forms of the generated modules (no device needed).

Independent dispatches are held back and issued as one launch of a batch
kernel that calls each generated module's kernels as device functions on
their own workgroup ranges. Every distinct kernel of the LeNet-5 and conv-block
traces (generated elementwise and reduction kernels, matrix-core contractions,
window max and run sums) is put into batch kernels of eight, which must
compile for gfx950; a module the form cannot take (none of these) would be
launched on its own instead.
"""
import os
import re

import pytest

from tinyhvm_amd import _lib, trace

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
WL = os.path.join(ROOT, "tinyhvm_amd", "workloads")
MAIN = re.compile(r'extern "C" __global__ __launch_bounds__\((\d+)\) (?:__attribute__\(\(\w+\([\d, ]*\)\)\) )?void (\w+)\(')


def _modules(name):
    out, seen = [], set()
    for r in trace.read_trace(os.path.join(WL, name)):
        if r.tag != trace.UOP:
            continue
        k = trace.to_uop_kernel(r)
        if _lib.dense_analyze(k):
            src = _lib.dense_source(k)
        elif _lib.window_analyze(k):
            src = _lib.window_source(k)
        else:
            src = _lib.kernel_source(k)[0]
        mains = [(int(t), n) for t, n in MAIN.findall(src) if not n.endswith(("_sum", "_fin", "_pack"))]
        assert mains, src[:2000]
        threads, kname = mains[0]
        if kname in seen:
            continue
        seen.add(kname)
        out.append((src, kname, threads, 3, 1))
    return out


@pytest.mark.parametrize("name", ["lenet_b256.trc", "convblock_b64.trc"])
def test_generated_modules_compile_as_batches(name):
    mods = _modules(name)
    assert len(mods) >= 10
    for i in range(0, len(mods), 8):
        group = mods[i:i + 8]
        assert _lib.batch_compile_check(group) > 0, [g[1] for g in group]


def test_lenet_epilogues_fuse_and_compile():
    """Elementwise dispatches that read a matrix-core contraction's output at
    their own index fuse into its epilogue: LeNet-5's five forward bias+relu
    (or bias) kernels after conv1, conv2, fc1, fc2, fc3 and the relu mask
    after fc2's input gradient; the fused modules compile. Consumers that
    read the output elsewhere (the pool backward after fc1's input gradient
    and conv2's, and the pad after the weight flip) are refused."""
    recs = trace.read_trace(os.path.join(WL, "lenet_b256.trc"))
    lo = next(i for i, r in enumerate(recs) if r.tag == trace.MARK and r.f["text"] == "lenet.step")
    hi = next(i for i, r in enumerate(recs) if i > lo and r.tag == trace.MARK and r.f["text"] == "lenet.end")
    uops = [r for r in recs[lo:hi] if r.tag == trace.UOP]
    fused, refused = [], []
    for p, c in zip(uops, uops[1:]):
        kp = trace.to_uop_kernel(p)
        a = _lib.dense_analyze(kp)
        if not a or p.f["out"] not in c.f["leaf_bufs"]:
            continue
        kc = trace.to_uop_kernel(c)
        try:
            assert _lib.epilogue_compile_check(kp, kc, c.f["leaf_bufs"].index(p.f["out"]) + 1) > 0
            fused.append(a[:3])
        except ValueError as e:
            assert "own index" in str(e), str(e)
            refused.append(a[:3])
    # (the CPU run routes every contraction to the matrix cores, so smaller
    # ones fuse too)
    for want in [(200704, 6, 25), (25600, 16, 150), (256, 120, 400), (256, 84, 120), (256, 10, 84),
                 (256, 120, 84)]:
        assert want in fused, (want, fused)
    assert refused == [(256, 400, 120), (96, 25, 25), (50176, 6, 400)], refused


def test_upload_kernel_compiles_in_a_batch():
    """Host writes of at most 64 KiB are copied by the upload kernel, read
    from pinned coherent host memory, so that the copy goes out in one batch
    launch with independent held work instead of as a copy of its own: its
    module compiles alone and batched with generated modules."""
    src = _lib.upload_source()
    assert 'void thvm_upload(' in src and "__launch_bounds__(256)" in src
    mods = _modules("lenet_b256.trc")[:3]
    assert _lib.batch_compile_check([(src, "thvm_upload", 256, 3, 1)]) > 0
    assert _lib.batch_compile_check([(src, "thvm_upload", 256, 3, 1)] + mods) > 0


def test_weight_pack_kernels_compile_in_a_batch():
    """The B-operand pack kernel of a contraction (the 3x3 convolutions'
    weights packed K x N) is held like a generated kernel, so that it goes
    out in one launch with the independent work before it: its module
    compiles batched with generated modules."""
    packs = []
    for r in trace.read_trace(os.path.join(WL, "convblock_b64.trc")):
        if r.tag != trace.UOP:
            continue
        k = trace.to_uop_kernel(r)
        if not _lib.dense_analyze(k):
            continue
        src = _lib.dense_source(k)
        m = re.search(r'void (thvm_gemm_[0-9a-f]+_pack)\(', src)
        if m and all(m.group(1) != p[1] for p in packs):
            packs.append((src, m.group(1), 256, 144, 1))
    assert packs
    mods = _modules("convblock_b64.trc")[:2]
    assert _lib.batch_compile_check(packs + mods) > 0


def _region(name, mark, lo, hi):
    """(source, main kernel, lanes, gx, gy) of dispatches lo..hi-1 after mark
    (the generated and window-max programs; grids as the backend launches them)"""
    recs = trace.read_trace(os.path.join(WL, name))
    start = next(i for i, r in enumerate(recs) if r.tag == trace.MARK and r.f["text"] == mark)
    out, n = [], 0
    for r in recs[start:]:
        if r.tag != trace.UOP:
            continue
        if lo <= n < hi:
            k = trace.to_uop_kernel(r)
            assert not _lib.dense_analyze(k)
            src = _lib.window_source(k) if _lib.window_analyze(k) else _lib.kernel_source(k)[0]
            mains = [(int(t), nm) for t, nm in MAIN.findall(src) if not nm.endswith(("_sum", "_fin", "_pack"))]
            out.append((src, mains[0][1], mains[0][0], 1, 1))
        n += 1
        if n >= hi:
            break
    return out


@pytest.mark.parametrize("name,mark,lo,hi", [
    ("lenet_b256.trc", "lenet.step", 13, 23),
    ("mlp_64x784x128x10.trc", "mlp.fwd", 4, 14),
])
def test_softmax_steps_compile_as_sequences(name, mark, lo, hi):
    """The softmax cross-entropy and its gradient on [batch, 10] are tiny
    dependent programs: the backend holds them as steps of a sequence and
    issues each run of them as one launch of a sequence kernel (one
    workgroup runs the programs in order, a barrier after each). The group
    reduction among them runs one wave per output and reduces in registers
    (no LDS, no barrier), so the whole run compiles as one sequence."""
    items = _region(name, mark, lo, hi)
    assert len(items) == hi - lo
    reds = [it for it in items if it[1].startswith("thvm_red_")]
    assert len(reds) == 1 and reds[0][2] == 64
    assert "__shared__" not in reds[0][0].split(reds[0][1])[1] and "wsum0(" in reds[0][0]
    assert _lib.seq_compile_check(items) > 0, [it[1] for it in items]
