"""Run-sum groups (window.c), without a device.

Batchnorm's statistics (src/nn/batchnorm.c:35-111) reach the backend as run
sums over a [N, C, H, W] tensor, each followed by small per-channel
programs, and the loss is a run sum over the pooled output. The backend runs
such a sequence as one launch:

- run sums of one shape (outputs, loop, runs, splits) that follow each other
  read what they share once (backward: sum(dy) and sum(dy * xhat));
- a held elementwise program or window max whose output a run sum reads is
  computed where the sum loads it, and stored there by the same lane
  (forward: the centring c = y - mean with sum(c^2); the max-pool with the
  loss sum; backward: the pooling backward with sum(dy));
- elementwise programs over the sums' outputs run in the workgroup that
  combines each output (the mean; the variance and the inverse deviation).

Here, on the conv block's recorded dispatches: which sequences group, that
their kernels compile for gfx950, what the generated source does (no
memory load of a tensor the producer computes), and that sequences that
must not group do not. Every value in a group is computed by the same
operations in the same order as in the separate launches; the GPU tests
compare the grouped step with single launches bit for bit on every buffer.
"""
import os
import re

import pytest

from tinyhvm_amd import _lib, trace as T

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
WL = os.path.join(ROOT, "tinyhvm_amd", "workloads")


@pytest.fixture(scope="module")
def conv():
    recs = [r for r in T.read_trace(os.path.join(WL, "convblock_b64.trc")) if r.tag == T.UOP]
    return [(T.to_uop_kernel(r), [r.f["out"]] + list(r.f["leaf_bufs"])) for r in recs]


def _group(seq, idx, producer=False):
    ks = [seq[i][0] for i in idx]
    bs = [seq[i][1] for i in idx]
    return ks, bs, producer


def test_forward_statistics_group(conv):
    # sum(y) with the mean: one sum, one consumer in the combining workgroup
    ks, bs, pr = _group(conv, [2, 3])
    src = _lib.group_source(ks, bs, pr)
    assert "tl0_(gid, v0_" in src and "prod_" not in src
    assert _lib.group_compile_check(ks, bs, pr) > 0
    # c = y - mean, sum(c^2), the variance and the inverse deviation
    ks, bs, pr = _group(conv, [4, 5, 6, 7], producer=True)
    src = _lib.group_source(ks, bs, pr)
    main = src.split('extern "C" __global__')[1]
    c_buf = bs[0][0]
    assert bs[1][1] == c_buf                      # the sum reads the centred tensor
    assert "ld4nt_u(m0_p1" not in main            # ... from the producer, not memory
    assert "prod_(pb_ + o_, ok_" in main
    assert "st4nt(p0" in src                      # the producer still stores c
    assert "tl1_(gid, u0_" in main                # the inverse deviation takes the variance
    assert _lib.group_compile_check(ks, bs, pr) > 0


def test_pooling_and_loss_group(conv):
    ks, bs, pr = _group(conv, [13, 14], producer=True)
    src = _lib.group_source(ks, bs, pr)
    # the window max reads its rows as 16-byte vectors, maxima in the engine's order
    fn = src[src.index("void prod_"):src.index('extern "C" __global__')]
    assert fn.count("__builtin_nontemporal_load((const v4f_*)") == 4
    assert re.search(r"a_\[0\] = \(a_\[0\] > e_\) \? a_\[0\] : e_", fn)
    assert _lib.group_compile_check(ks, bs, pr) > 0


def test_backward_group(conv):
    # the pooling backward merged with the relu backward (chain.c), then
    # sum(dy) and sum(dy * xhat): the merged program is the producer
    (k15, d15), (k16, d16) = conv[15], conv[16]
    m, mb = _lib.chain_merge(k15, d15, k16, d16[0], d16[1:])
    ks = [m, conv[17][0], conv[18][0]]
    bs = [list(mb), conv[17][1], conv[18][1]]
    src = _lib.group_source(ks, bs, True)
    main = src.split('extern "C" __global__')[1]
    dy = conv[17][1][1]
    assert dy in mb and conv[18][1][1] == dy
    # dy is the producer's value in both sums; xhat is read from memory once
    assert "m0_f" in main and "m1_f" in main
    assert main.count("ld4nt_u(") == 1
    assert _lib.group_compile_check(ks, bs, True) > 0
    # the second pair of sums over the pooling backward's output: siblings
    ks, bs, pr = _group(conv, [21, 22])
    main = _lib.group_source(ks, bs, pr).split('extern "C" __global__')[1]
    # dyp and xhat loaded once each: the second sum takes the first's dyp values
    assert main.count("ld4nt_u(") == 2
    assert re.search(r"const float m1_f\d+_0 = m0_f\d+_0;", main)
    assert "comb_put(sl_, gid + 64u" in main      # the second sum's partials after the first's
    assert _lib.group_compile_check(ks, bs, pr) > 0


def test_sequences_that_do_not_group(conv):
    # a sum of another shape (the loss sum: one output) does not join the statistics
    with pytest.raises(ValueError, match="does not join"):
        _lib.group_source(*_group(conv, [2, 14]))
    # a consumer that reads no output of the group
    with pytest.raises(ValueError, match="does not join"):
        _lib.group_source(*_group(conv, [2, 7]))
    # a big elementwise program is no consumer (other size): c = y - mean after sum(y)
    with pytest.raises(ValueError, match="does not join"):
        _lib.group_source(*_group(conv, [2, 3, 4]))
    # the sum must read the producer's output: sum(y) does not read c
    with pytest.raises(ValueError, match="does not join"):
        _lib.group_source(*_group(conv, [4, 2], producer=True))
    # the loss sum over a tensor the window max does not write
    k14, b14 = conv[14]
    ks, bs, pr = _group(conv, [13, 14], producer=True)
    with pytest.raises(ValueError, match="does not join"):
        _lib.group_source(ks, [bs[0], [b14[0], 999]], pr)
    # a sum that does not read every element of the producer's tensor once:
    # sum(y) over the pooled output (a quarter of its loop's elements exist)
    k2, b2 = conv[2]
    with pytest.raises(ValueError, match="does not join"):
        _lib.group_source([ks[0], k2], [bs[0], [b2[0], bs[0][0]]], pr)
