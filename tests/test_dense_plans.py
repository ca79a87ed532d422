"""The matrix-core plans the benchmark workloads get (no device needed).

The plan choices are what the measured numbers rest on; this pins them so a
change to the planner that silently drops one shows up here:
- the 3x3 64->64 convolution (forward and input gradient): the LDS-free wave
  tile (a wave per 32 pixels by 64 channels, buffer loads with scalar k
  offsets), K-reordered loaders, its weights packed, the epilogue along the
  pixels;
- its weight gradient: 64x64 tiles, 128 K splits, K-reordered loaders over
  image rows padded 56 -> 64, two stages of loads in flight;
- the 4096^3 GEMMs: 128x128 tiles, K-reordered loaders, 16-byte loads, the
  epilogue along n (row-major output);
- LeNet-5's fully connected weight gradients: the direct kernel with 8 waves.
The device-free entry points read the tuning environment once per process;
the CPU test run exports only THVM_HIP_DENSE_FORCE (routing), which leaves
these contractions' plans as they are.
"""
import os
import re

from tinyhvm_amd import _lib, trace

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
WL = os.path.join(ROOT, "tinyhvm_amd", "workloads")


def _plans(name):
    out = {}
    for r in trace.read_trace(os.path.join(WL, name)):
        if r.tag != trace.UOP:
            continue
        k = trace.to_uop_kernel(r)
        a = _lib.dense_analyze(k)
        if not a:
            continue
        src = _lib.dense_source(k)
        cst = re.search(r"constexpr u32 BM = (\d+), BN = (\d+), BK = (\d+)", src)
        nw = re.search(r"NW = (\d+)u", src)
        kw = re.search(r"KW = (\d+)u, KCW", src)
        ke = re.search(r"constexpr u32 E = (\d+)u, NBLK", src)
        ro = re.search(r"MG = (\d+)u, V = \d+u, VP = \d+u, KCH = (\d+)u", src)
        tl = re.search(r"constexpr u32 S = (\d+)u, FULL = (\d+)u, NFW = FULL / S, KPC = KP / S, PFT = (\d+)u", src)
        out[a] = {
            "tile": (int(cst.group(1)), int(cst.group(2))) if cst else "direct",
            "kperm": "kbase_p(" in src,
            "padded": "lim_" in src,
            "packed": "_pack(" in src,
            "transposed": "(b[kk][j], a[kk][i]" in src or "(rb0[q], ra[q]" in src,
            "wave": "__amdgpu_buffer_rsrc_t rA" in src,
            "vec16": "*(const float4*)(ps" in src,
            "two_stage": "ra1[" in src,
            "waves": int(nw.group(1)) if nw else 4,
            "skinny": "KCW = " in src,
            "skinny_waves": int(kw.group(1)) if kw else None,
            "skinny_block": int(ke.group(1)) if ke else None,
            "outer": (int(ro.group(1)), int(ro.group(2))) if ro else None,
            "comb": "comb_pub(sl_" in src,
            "tail": (int(tl.group(2)), int(tl.group(1)), int(tl.group(3))) if tl else None,
            "prio": "__builtin_amdgcn_s_setprio(1)" in src,
        }
    return out


def test_convolution_plans():
    p = _plans("convblock_b64.trc")
    fwd = p[(200704, 64, 576, 1)]
    assert fwd["wave"] and fwd["kperm"] and fwd["packed"] and fwd["transposed"]
    assert not fwd["padded"]
    # the weight gradient's splits fill the 1024 workgroup slots of 256 CUs
    # exactly once: 9 row tiles x 112 splits of 2048 (padded, reordered) K
    dw = p[(576, 64, 200704, 112)]
    assert dw["tile"] == (64, 64) and dw["kperm"] and dw["padded"] and dw["two_stage"]
    assert not dw["packed"]
    # the long-K weight gradient raises a wave's priority over its math; the
    # forward (wave tile) has no stages to do so
    assert dw["prio"] and not fwd["prio"]


def test_gemm_4096_plans():
    p = _plans("linear_4096.trc")
    assert len(p) == 1 or all(v == list(p.values())[0] for v in p.values())
    for a, v in p.items():
        assert a[:3] == (4096, 4096, 4096)
        assert v["tile"] == (128, 128) and v["kperm"] and v["vec16"]
        assert not v["transposed"] and not v["packed"] and not v["two_stage"] and not v["prio"]


def test_lenet_few_channel_convolutions_are_skinny():
    # conv1 forward (6 channels), conv2 forward (16) and conv2 dX (6): a row
    # per lane with every column sum in registers; K walks in blocks of the
    # 5x5 window (25), whose offsets are constants, and the waves of a row
    # group split the blocks evenly, as many as keep the grid at most 8192
    # waves (conv2: its 6 blocks on 6 waves; conv2 dX: 16 blocks on 8)
    p = _plans("lenet_b256.trc")
    for shape, waves in [((200704, 6, 25, 1), 1), ((25600, 16, 150, 1), 6), ((50176, 6, 400, 1), 8)]:
        src = p[shape]
        assert src["skinny"] and src["skinny_waves"] == waves and src["skinny_block"] == 25, (shape, src)


def test_lenet_convolution_weight_gradients_are_outer_product_reductions():
    # conv1 dW (25x6 over 200704 pixels) and conv2 dW (150x16 over 25600):
    # a k per lane, row groups of at most 96 / N rows, K chunks of at least
    # 8 k per lane; conv2's 12 splits combined in the same launch, conv1's 98
    # through the split-K sum kernel
    p = _plans("lenet_b256.trc")
    assert p[(25, 6, 200704, 98)]["outer"] == (13, 2048) and not p[(25, 6, 200704, 98)]["comb"]
    assert p[(150, 16, 25600, 12)]["outer"] == (6, 2134) and p[(150, 16, 25600, 12)]["comb"]


def test_lenet_fc_weight_gradients_use_eight_waves():
    p = _plans("lenet_b256.trc")
    for shape in [(400, 120, 256, 1), (120, 84, 256, 1), (84, 10, 256, 1)]:
        assert p[shape]["tile"] == "direct" and p[shape]["waves"] == 8, (shape, p[shape])



def test_conv_wave_tile_splits_its_last_tiles():
    # the 3x3 64->64 convolution at batch 64 (forward and dX): 6272 wave
    # tiles on 1024 SIMDs; 6144 run whole, 4 to a workgroup, and the last
    # 128 are split over the 4 waves of a workgroup in K chunks of 72
    # k-pairs (a ring of 8 loads), so that no SIMD gets a seventh tile
    p = _plans("convblock_b64.trc")
    hit = [v for a, v in p.items() if a[:3] == (200704, 64, 576)]
    assert hit and all(v["tail"] == (6144, 4, 8) for v in hit), hit
