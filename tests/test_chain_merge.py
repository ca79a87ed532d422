"""Elementwise programs fused in sequence (chain.c), without a device.

A loop-free dispatch C that reads the output of a held loop-free program P
at its own gid runs as one merged program M: P's ops, then C's with each
load of P's output replaced by the value P stores there, and C's STORE into
a new leaf slot holding C's output. Here, over the dispatch sequences of the
recorded workloads:

- the pairs that merge are the expected ones (batchnorm's variance and
  inverse deviation, normalisation then scale and shift, the pooling
  backward's routing then the product with the scale; in LeNet-5 and the
  MLP a softmax step and the relu mask after the last layer's input
  gradient, whose producer is a loop each lane runs for its own gid; one
  pair in the linear stack), and pairs where the second does not read the
  first's output at its own gid do not;
- M, run by a small interpreter of per-gid KOp programs on random
  inputs, leaves every buffer exactly as P followed by C does (both sides
  use the same interpreter, so this checks the merge, not the arithmetic;
  the GPU tests compare the fused launches with separate ones bit for bit);
- M compiles for gfx950 (hipRTC, no device).
"""
import ctypes as C
import os

import numpy as np
import pytest

from tinyhvm_amd import _lib, abi, trace as T

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
WL = os.path.join(ROOT, "tinyhvm_amd", "workloads")


class Skip(Exception):
    pass


def run(k, bufs, ids):
    """Evaluates program k (no loop, or loops each lane runs for its own
    gid) over every gid, in place on bufs (id -> float32 array); ids =
    [output, leaves...] (0: absent)."""
    n = k.local_size and k.grid[0] or k.grid[0] * k.grid[1] * k.grid[2]
    gid = np.arange(n, dtype=np.uint32)
    val = {}
    isf = {}
    end = {}
    stack = []
    for i in range(k.n_ops):
        if k.ops[i].type == abi.KOP_RANGE:
            stack.append(i)
        elif k.ops[i].type == abi.KOP_ENDRANGE:
            end[stack.pop()] = i
    i = 0
    loops = []                   # [range op, r]
    while i < k.n_ops:
        op = k.ops[i]
        t, a0, a1 = op.type, op.arg[0], op.arg[1]
        if t == abi.KOP_RANGE:
            if op.imm.u == 0:
                i = end[i] + 1
                continue
            loops.append([i, 0])
            val[i], isf[i] = np.zeros(n, np.uint32), False
            i += 1
            continue
        if t == abi.KOP_ENDRANGE:
            lp = loops[-1]
            lp[1] += 1
            if lp[1] < k.ops[lp[0]].imm.u:
                val[lp[0]] = np.full(n, lp[1], np.uint32)
                i = lp[0] + 1
            else:
                loops.pop()
                i += 1
            continue
        i = step(k, i, op, t, a0, a1, n, gid, val, isf, bufs, ids)


def step(k, i, op, t, a0, a1, n, gid, val, isf, bufs, ids):
    if True:

        def f(j):
            return val[j] if isf[j] else val[j].astype(np.float32)

        def u(j):
            if isf[j]:
                raise Skip("float index")
            return val[j]

        if t == abi.KOP_GID:
            if op.imm.u != 0:
                raise Skip("grid axis")
            val[i], isf[i] = gid, False
        elif t == abi.KOP_CONST_U:
            val[i], isf[i] = np.full(n, op.imm.u, np.uint32), False
        elif t == abi.KOP_CONST_F:
            val[i], isf[i] = np.full(n, op.imm.f, np.float32), True
        elif t == abi.KOP_IDX:
            val[i], isf[i] = (u(a0) * np.uint32(op.imm.u) + u(a1)).astype(np.uint32), False
        elif t in (abi.KOP_MOD, abi.KOP_DIV):
            q = op.imm.u
            x = u(a0)
            val[i] = np.zeros(n, np.uint32) if q == 0 else (x % np.uint32(q) if t == abi.KOP_MOD else x // np.uint32(q))
            isf[i] = False
        elif t == abi.KOP_LOAD:
            s = op.imm.u
            if s > k.n_leaves:
                val[i] = np.zeros(n, np.float32)
            else:
                dt = k.out_dtype if s == 0 else k.leaf_dtypes[s - 1]
                if dt != abi.DTYPE_F32:
                    raise Skip("dtype")
                b = bufs.get(ids[s])
                idx = u(a0)
                if b is None:
                    val[i] = np.zeros(n, np.float32)
                else:
                    ok = idx < b.size
                    val[i] = np.where(ok, b[np.where(ok, idx, 0)], np.float32(0))
            isf[i] = True
        elif t == abi.KOP_STORE:
            s = op.imm.u
            dt = k.out_dtype if s == 0 else k.leaf_dtypes[s - 1]
            if dt != abi.DTYPE_F32:
                raise Skip("dtype")
            b = bufs[ids[s]]
            idx = u(a0)
            ok = idx < b.size
            b[idx[ok]] = f(a1)[ok]
        elif t == abi.KOP_ACC_INIT:
            val[i], isf[i] = np.full(n, op.imm.f, np.float32), True
        elif t == abi.KOP_ACC:
            x = val[a0]
            y = val[a1] if isf[a1] else val[a1].astype(np.float32)
            val[a0] = (np.where(x > y, x, y) if op.imm.u == abi.UOP_RMAX else x + y).astype(np.float32)
        elif t == abi.KOP_MASK:
            val[i], isf[i] = np.where(f(a0) != 0, f(a1), np.float32(0)).astype(np.float32), True
        elif t == abi.KOP_ALU:
            uop = op.imm.u
            x = f(a0)
            y = f(a1) if uop not in abi.UNARY_UOPS else None
            with np.errstate(all="ignore"):
                if uop == abi.UOP_ADD: r = x + y
                elif uop == abi.UOP_SUB: r = x - y
                elif uop == abi.UOP_MUL: r = x * y
                elif uop == abi.UOP_DIV: r = np.where(y != 0, x / np.where(y != 0, y, 1), np.float32(0))
                elif uop == abi.UOP_MAX: r = np.where(x > y, x, y)
                elif uop == abi.UOP_CMP: r = np.where(x > y, np.float32(1), np.float32(0))
                elif uop == abi.UOP_NEG: r = -x
                elif uop == abi.UOP_RELU: r = np.where(x > 0, x, np.float32(0))
                elif uop == abi.UOP_EXP: r = np.exp(x)
                elif uop == abi.UOP_LOG: r = np.log(x)
                elif uop == abi.UOP_SQRT: r = np.sqrt(x)
                else: raise Skip("alu %d" % uop)
            val[i], isf[i] = r.astype(np.float32), True
        else:
            raise Skip("op %d" % t)
    return i + 1


def dispatches(name, m0=None, m1=None):
    recs = T.read_trace(os.path.join(WL, name))
    lo = 0 if m0 is None else next(i for i, r in enumerate(recs) if r.tag == T.MARK and r.f["text"] == m0)
    hi = len(recs) if m1 is None else next(i for i, r in enumerate(recs)
                                           if i > lo and r.tag == T.MARK and r.f["text"] == m1)
    sizes = {r.f["id"]: r.f["bytes"] for r in recs if r.tag == T.ALLOC}
    out = []
    for r in recs[lo:hi]:
        if r.tag == T.UOP:
            out.append((T.to_uop_kernel(r), [r.f["out"]] + list(r.f["leaf_bufs"])))
    return out, sizes


def chains(seq):
    """Each dispatch merged into the one before when the pair merges (the
    chain continuing with the merged program): [(first, last, m, mb), ...].
    The backend offers a producer only when it runs as a generated program:
    a contraction it routes to the matrix cores takes its consumer as a
    fused epilogue instead (the MLP's fc2 forward and its bias, 2 and 3)."""
    found = []
    prev, first = None, 0
    for n, (k, ids) in enumerate(seq):
        if prev is not None:
            r = _lib.chain_merge(prev[0], prev[1], k, ids[0], ids[1:])
            if r is not None:
                prev = r
                if found and found[-1][0] == first:
                    found[-1] = (first, n, r[0], r[1])
                else:
                    found.append((first, n, r[0], r[1]))
                continue
        prev, first = (k, ids), n
    return found


CASES = [
    # LeNet-5: 1-2, 4-5, 9-10, 11-12 and 29-30 are contractions with their
    # bias/relu consumers (fused epilogues in the backend)
    ("lenet_b256.trc", "lenet.step", "lenet.end", [(1, 2), (4, 5), (9, 10), (11, 12), (21, 22), (25, 26), (29, 30)]),
    ("convblock_b64.trc", None, None, [(6, 7), (8, 9), (15, 16)]),
    ("mlp_64x784x128x10.trc", None, None, [(2, 3), (12, 13), (16, 17)]),
    ("linear_8x4096x4096.trc", None, None, [(1, 2)]),
]


@pytest.mark.parametrize("name,m0,m1,want", CASES, ids=[c[0] for c in CASES])
def test_pairs_that_merge(name, m0, m1, want):
    seq, _ = dispatches(name, m0, m1)
    got = [(a, b) for a, b, _, _ in chains(seq)]
    assert got == want


@pytest.mark.parametrize("name,m0,m1", [("lenet_b64.trc", "lenet.step", "lenet.end"),
                                        ("convblock_b1.trc", None, None),
                                        ("mlp_64x784x128x10.trc", None, None)])
def test_merged_program_equals_the_pair(name, m0, m1):
    seq, sizes = dispatches(name, m0, m1)
    found = chains(seq)
    assert found, "no pair merged"
    rng = np.random.default_rng(7)
    checked = 0
    for first, last, m, mb in found:
        ids = {i for _, d in seq[first:last + 1] for i in d if i} | {i for i in mb if i}
        init = {i: rng.standard_normal(sizes[i] // 4).astype(np.float32) for i in ids}
        a = {i: v.copy() for i, v in init.items()}
        b = {i: v.copy() for i, v in init.items()}
        try:
            for k, d in seq[first:last + 1]:
                run(k, a, d)
            run(m, b, mb)
        except Skip:
            continue
        for i in ids:
            assert a[i].tobytes() == b[i].tobytes(), "buffer %d differs after dispatches %d..%d" % (i, first, last)
        # the merged program writes every output of the pair, each once
        def stores(k):
            return [k.ops[j].imm.u for j in range(k.n_ops) if k.ops[j].type == abi.KOP_STORE]
        assert len(stores(m)) == sum(len(stores(k)) for k, _ in seq[first:last + 1])
        assert sorted(mb[s] for s in stores(m)) == sorted(d[0] for _, d in seq[first:last + 1])
        checked += 1
    assert checked, "every merged pair was skipped"


def test_merged_programs_compile():
    seq, _ = dispatches("convblock_b64.trc")
    for first, last, m, _ in chains(seq):
        assert _lib.compile_check(m) > 0, "merged dispatches %d..%d" % (first, last)


def test_no_merge_without_a_gid_read():
    """A consumer that reads the producer's output anywhere but at its own
    gid (a padded copy) does not merge, nor one whose output is a buffer the
    producer reads at other elements than each lane's own, nor one that does
    not read the producer's output."""
    seq, _ = dispatches("convblock_b64.trc")
    k20, d20 = seq[20]           # batchnorm backward dc
    k26, d26 = seq[26]           # the padded copy of dc: reads it shifted
    assert d20[0] in d26[1:]
    assert _lib.chain_merge(k20, d20, k26, d26[0], d26[1:]) is None
    k8, d8 = seq[8]              # xhat = c * rstd[channel]
    k9, d9 = seq[9]
    assert _lib.chain_merge(k8, d8, k9, d8[2], d9[1:]) is None    # into rstd, read per channel
    k10, d10 = seq[10]           # running mean, then running variance:
    k11, d11 = seq[11]           # independent of each other
    assert _lib.chain_merge(k10, d10, k11, d11[0], d11[1:]) is None


def test_in_place_update_merges():
    """A consumer whose output is a buffer the producer reads only at each
    lane's own element (ASSIGN writing an updated value back over the input
    it came from) merges: each lane loads its element before the merged
    store, so M leaves every buffer as P followed by C does."""
    seq, sizes = dispatches("convblock_b1.trc")
    k8, d8 = seq[8]              # xhat = c * rstd[channel], c read at gid
    k9, d9 = seq[9]
    r = _lib.chain_merge(k8, d8, k9, d8[1], d9[1:])
    assert r is not None
    m, mb = r
    rng = np.random.default_rng(11)
    ids = {i for i in list(d8) + list(d9) + list(mb) if i}
    init = {i: rng.standard_normal(sizes[i] // 4).astype(np.float32) for i in ids}
    a = {i: v.copy() for i, v in init.items()}
    b = {i: v.copy() for i, v in init.items()}
    run(k8, a, d8)
    run(k9, a, [d8[1]] + list(d9[1:]))
    run(m, b, mb)
    for i in ids:
        assert a[i].tobytes() == b[i].tobytes(), "buffer %d differs" % i
    assert _lib.compile_check(m) > 0


def _with_extra_store(k, slot):
    """A copy of loop-free producer k whose last STORE is followed by a
    second STORE at the same index into `slot`, of the negated value."""
    m = abi.UOpKernel()
    C.memmove(C.byref(m), C.byref(k), C.sizeof(abi.UOpKernel))
    st = [j for j in range(k.n_ops) if k.ops[j].type == abi.KOP_STORE][-1]
    n = m.n_ops
    m.ops[n].type = abi.KOP_ALU
    m.ops[n].arg[0] = m.ops[n].arg[1] = k.ops[st].arg[1]
    m.ops[n].imm.u = abi.UOP_NEG
    m.ops[n + 1].type = abi.KOP_STORE
    m.ops[n + 1].arg[0] = k.ops[st].arg[0]
    m.ops[n + 1].arg[1] = n
    m.ops[n + 1].imm.u = slot
    m.n_ops = n + 2
    return m


def test_producer_storing_one_buffer_twice():
    """A producer whose STOREs write one buffer twice leaves the last value
    there. Stored twice through the same slot, it is not a producer at all;
    through two slots that name the same buffer (its output also passed as
    a leaf), the consumer's load takes the second, later value, as P then C
    leaves it."""
    seq, sizes = dispatches("convblock_b1.trc")
    found = chains(seq)
    assert found
    first, _, _, _ = found[0]
    kp, dp = seq[first]
    kc, dc = seq[first + 1]
    assert _lib.chain_merge(kp, dp, kc, dc[0], dc[1:]) is not None
    twice = _with_extra_store(kp, 0)
    assert _lib.chain_merge(twice, dp, kc, dc[0], dc[1:]) is None

    # the output passed again as an extra leaf (slot kp.n_leaves + 1), stored through it last
    alias = _with_extra_store(kp, kp.n_leaves + 1)
    alias.leaf_dtypes[kp.n_leaves] = kp.out_dtype
    alias.n_leaves = kp.n_leaves + 1
    alias.n_bufs = alias.n_leaves + 1
    ids = list(dp) + [dp[0]]
    r = _lib.chain_merge(alias, ids, kc, dc[0], dc[1:])
    assert r is not None
    m, mb = r
    rng = np.random.default_rng(11)
    used = {i for i in ids + list(dc) + list(mb) if i}
    init = {i: rng.standard_normal(sizes[i] // 4).astype(np.float32) for i in used}
    a = {i: v.copy() for i, v in init.items()}
    b = {i: v.copy() for i, v in init.items()}
    run(alias, a, ids)
    run(kc, a, dc)
    run(m, b, mb)
    for i in used:
        assert a[i].tobytes() == b[i].tobytes(), "buffer %d differs" % i
