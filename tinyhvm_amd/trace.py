"""Reader and writer for the kernel-trace format described in include/thvm_trace.h.

A trace is the recorded sequence of Backend calls the engine made for one
workload (what src/schedule/_.c:2268-2411 dispatches, plus the buffer traffic
around it). Records are parsed into plain Python objects; `to_uop_kernel`
builds the ctypes UOpKernel that dispatch_uop_kernel receives.
"""
import struct
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

from . import abi

MAGIC = b"THVMTRC1"
(ALLOC, FREE, INCREF, DECREF, WRITE, READ, UOP, RS, COPY, CONTIG, RESET, PERSIST,
 SNAPSHOT, MARK, OPUN, OPBIN, OPMM, OPRED, ADAM) = range(1, 20)
LEGACY = (OPUN, OPBIN, OPMM, OPRED)
ENC_RAW, ENC_GEN = 0, 1
GEN_UNIFORM, GEN_NORMAL, GEN_INT, GEN_CONST = 1, 2, 3, 4
TAG_NAMES = {ALLOC: "ALLOC", FREE: "FREE", INCREF: "INCREF", DECREF: "DECREF", WRITE: "WRITE",
             READ: "READ", UOP: "UOP", RS: "RS", COPY: "COPY", CONTIG: "CONTIG",
             RESET: "RESET", PERSIST: "PERSIST", SNAPSHOT: "SNAPSHOT", MARK: "MARK",
             OPUN: "OPUN", OPBIN: "OPBIN", OPMM: "OPMM", OPRED: "OPRED", ADAM: "ADAM"}


@dataclass
class ViewRec:
    rank: int
    dims: List[int]
    strides: List[int]
    offset: int
    numel: int
    contiguous: int
    has_mask: int
    mask_begin: List[int]
    mask_end: List[int]
    n_compound: int
    compound: List[tuple]      # (dim_a, dim_b, stride_a, begin, end) x 2
    mod_size: List[int]

    def to_c(self, v: Optional[abi.View] = None) -> abi.View:
        v = v if v is not None else abi.View()
        v.shape.rank = self.rank
        for d in range(abi.MAX_DIM):
            v.shape.dims[d] = self.dims[d]
            v.strides[d] = self.strides[d]
            v.mask_begin[d] = self.mask_begin[d]
            v.mask_end[d] = self.mask_end[d]
            v.mod_size[d] = self.mod_size[d]
        v.offset = self.offset
        v.numel = self.numel
        v.contiguous = self.contiguous
        v.has_mask = self.has_mask
        v.n_compound_masks = self.n_compound
        for i in range(2):
            a, b, s, lo, hi = self.compound[i]
            cm = v.compound_masks[i]
            cm.dim_a, cm.dim_b, cm.stride_a, cm.begin, cm.end = a, b, s, lo, hi
        return v


@dataclass
class Rec:
    tag: int
    f: dict = field(default_factory=dict)

    @property
    def name(self):
        return TAG_NAMES.get(self.tag, str(self.tag))


class _Cur:
    def __init__(self, b: bytes):
        self.b = b
        self.o = 0

    def u32(self):
        v = struct.unpack_from("<I", self.b, self.o)[0]
        self.o += 4
        return v

    def i32(self):
        v = struct.unpack_from("<i", self.b, self.o)[0]
        self.o += 4
        return v

    def u64(self):
        v = struct.unpack_from("<Q", self.b, self.o)[0]
        self.o += 8
        return v

    def f32(self):
        v = struct.unpack_from("<f", self.b, self.o)[0]
        self.o += 4
        return v

    def words(self, n, fmt="I"):
        v = list(struct.unpack_from("<%d%s" % (n, fmt), self.b, self.o))
        self.o += 4 * n
        return v

    def raw(self, n):
        v = self.b[self.o:self.o + n]
        self.o += n
        return v

    def shape(self):
        rank = self.u32()
        return rank, self.words(8)

    def view(self) -> ViewRec:
        rank, dims = self.shape()
        strides = self.words(8, "i")
        offset = self.i32()
        numel, contiguous, has_mask = self.u32(), self.u32(), self.u32()
        mb, me = self.words(8), self.words(8)
        ncm = self.u32()
        cms = []
        for _ in range(2):
            a, b = self.u32(), self.u32()
            s = self.i32()
            lo, hi = self.u32(), self.u32()
            cms.append((a, b, s, lo, hi))
        mod = self.words(8)
        return ViewRec(rank, dims, strides, offset, numel, contiguous, has_mask, mb, me, ncm,
                       cms, mod)


def _parse_payload(tag, p: bytes) -> dict:
    c = _Cur(p)
    f = {}
    if tag == ALLOC:
        f["id"] = c.u32(); c.u32(); f["bytes"] = c.u64()
    elif tag in (FREE, INCREF, DECREF):
        f["id"] = c.u32()
    elif tag == WRITE:
        f["id"], f["enc"], f["bytes"] = c.u32(), c.u32(), c.u64()
        if f["enc"] == ENC_RAW:
            f["data"] = c.raw(f["bytes"])
        else:
            f["dist"], f["dtype"] = c.u32(), c.u32()
            f["seed"] = c.u64()
            f["p0"], f["p1"] = c.f32(), c.f32()
    elif tag == READ:
        f["id"], f["has_data"], f["bytes"] = c.u32(), c.u32(), c.u64()
        if f["has_data"]:
            f["data"] = c.raw(f["bytes"])
    elif tag == UOP:
        f["out"] = c.u32()
        n = c.u32()
        f["n_leaves"] = n
        f["leaf_bufs"] = c.words(n)
        f["cache_key"] = c.u64()
        f["n_ops"], f["n_bufs"], f["rank"] = c.u32(), c.u32(), c.u32()
        f["full_rank"], f["full_dims"] = c.shape()
        f["grid"] = c.words(3)
        f["tg"] = c.words(3)
        f["local_size"], f["reduce_numel"], f["out_dtype"] = c.u32(), c.u32(), c.u32()
        f["coord_uop"] = c.words(8)
        f["ops"] = [tuple(c.words(5)) for _ in range(f["n_ops"])]
        f["views"] = [c.view() for _ in range(n)]
        f["leaf_dtypes"] = c.words(n)
    elif tag == RS:
        f["out"] = c.u32()
        n = c.u32()
        f["n_leaves"] = n
        f["leaf_bufs"] = c.words(n)
        f["views"] = [c.view() for _ in range(n)]
        has_st = c.words(n)
        sts = []
        for i in range(n):
            if has_st[i]:
                nv = c.u32()
                sts.append([c.view() for _ in range(nv)])
            else:
                sts.append(None)
        f["sts"] = sts
        nops = c.u32()
        f["ops"] = [tuple(c.words(4)) for _ in range(nops)]
        f["full_rank"], f["full_dims"] = c.shape()
        f["has_reduce"] = c.u32()
        if f["has_reduce"]:
            w = c.words(21)
            f["reduce"] = dict(is_reduce=w[0:8], reduce_type=w[8], post_reduce_start=w[9],
                               n_post_leaves=w[10], reduce2_type=w[11], reduce2_start=w[12],
                               is_reduce2=w[13:21])
        f["n_side"] = ns = c.u32()
        f["side_bufs"] = c.words(ns)
        f["side_idx"] = c.words(ns)
        f["has_dtypes"] = c.u32()
        f["leaf_dtypes"] = c.words(n) if f["has_dtypes"] else [0] * n
        f["out_dtype"] = c.u32()
    elif tag == COPY:
        f["dst"], f["src"], f["bytes"] = c.u32(), c.u32(), c.u64()
    elif tag == CONTIG:
        f["dst"], f["numel"], f["src"] = c.u32(), c.u32(), c.u32()
        f["view"] = c.view()
    elif tag == RESET:
        f["keep"] = c.u32()
    elif tag == PERSIST:
        f["max_buf"] = c.u32()
    elif tag == SNAPSHOT:
        f["id"] = c.u32(); f["source"] = c.u32(); f["bytes"] = c.u64()
        f["data"] = c.raw(f["bytes"])
    elif tag == MARK:
        n = c.u32()
        f["text"] = c.raw(n).decode()
    elif tag in (OPUN, OPBIN):
        f["uop"], f["dst"], f["dd"] = c.u32(), c.u32(), c.u32()
        f["dv"] = c.view()
        f["a"], f["ad"] = c.u32(), c.u32()
        f["av"] = c.view()
        if tag == OPBIN:
            f["b"], f["bd"] = c.u32(), c.u32()
            f["bv"] = c.view()
    elif tag == OPMM:
        f["dst"], f["dd"] = c.u32(), c.u32()
        f["a"], f["ad"] = c.u32(), c.u32()
        f["av"] = c.view()
        f["b"], f["bd"] = c.u32(), c.u32()
        f["bv"] = c.view()
        f["M"], f["K"], f["N"] = c.u32(), c.u32(), c.u32()
    elif tag == OPRED:
        f["uop"], f["dst"], f["dn"], f["dd"] = c.u32(), c.u32(), c.u32(), c.u32()
        f["a"], f["sn"], f["ad"], f["rdim"] = c.u32(), c.u32(), c.u32(), c.u32()
    elif tag == ADAM:
        f["param"], f["grad"], f["m"], f["v"] = c.u32(), c.u32(), c.u32(), c.u32()
        for k in ("lr", "beta1", "beta2", "eps", "bc1", "bc2"):
            f[k] = c.f32()
        f["n"] = c.u32()
    return f


def read_trace(path) -> List[Rec]:
    with open(path, "rb") as fh:
        b = fh.read()
    if b[:8] != MAGIC:
        raise ValueError("%s: not a kernel trace (bad magic)" % path)
    o = 8
    out = []
    while o < len(b):
        tag, _flags, ln = struct.unpack_from("<IIQ", b, o)
        o += 16
        out.append(Rec(tag, _parse_payload(tag, b[o:o + ln])))
        o += ln
    return out


def to_uop_kernel(r: Rec) -> abi.UOpKernel:
    """Build the ctypes UOpKernel for a UOP record."""
    f = r.f
    k = abi.UOpKernel()
    k.n_ops = f["n_ops"]
    k.n_bufs = f["n_bufs"]
    k.n_leaves = f["n_leaves"]
    k.rank = f["rank"]
    k.full_shape.rank = f["full_rank"]
    for d in range(8):
        k.full_shape.dims[d] = f["full_dims"][d]
        k.coord_uop[d] = f["coord_uop"][d]
    for i in range(3):
        k.grid[i] = f["grid"][i]
        k.tg[i] = f["tg"][i]
    k.local_size = f["local_size"]
    k.reduce_numel = f["reduce_numel"]
    k.out_dtype = f["out_dtype"]
    for i, (t, a0, a1, a2, imm) in enumerate(f["ops"]):
        op = k.ops[i]
        op.type = t
        op.arg[0], op.arg[1], op.arg[2] = a0, a1, a2
        op.imm.u = imm
    for i, v in enumerate(f["views"]):
        v.to_c(k.leaf_views[i])
        k.leaf_dtypes[i] = f["leaf_dtypes"][i]
    return k


def gen_data(dist, dtype, seed, p0, p1, nbytes) -> bytes:
    """Materialize a WRITE/GEN record with the shared generator (include/thvm_gen.h)."""
    from . import _lib
    return _lib.gen_bytes(dist, dtype, seed, p0, p1, nbytes)


def describe(recs: List[Rec]) -> str:
    lines = []
    for r in recs:
        f = r.f
        if r.tag == UOP:
            lines.append("UOP out=%d leaves=%s full=%s grid=%s local=%d rn=%d nops=%d" % (
                f["out"], f["leaf_bufs"], f["full_dims"][:f["full_rank"]], f["grid"],
                f["local_size"], f["reduce_numel"], f["n_ops"]))
        elif r.tag == RS:
            lines.append("RS out=%d leaves=%s full=%s nops=%d reduce=%s" % (
                f["out"], f["leaf_bufs"], f["full_dims"][:f["full_rank"]], len(f["ops"]),
                f.get("reduce", {}).get("reduce_type")))
        elif r.tag in (WRITE, READ, SNAPSHOT, ALLOC):
            lines.append("%s id=%d bytes=%d%s" % (r.name, f["id"], f["bytes"],
                                                  " gen" if f.get("enc") == ENC_GEN else ""))
        elif r.tag == MARK:
            lines.append("MARK %s" % f["text"])
        else:
            lines.append("%s %s" % (r.name, {k: v for k, v in f.items() if k != "data"}))
    return "\n".join(lines)


def kop_listing(r: Rec) -> str:
    out = []
    for i, (t, a0, a1, a2, imm) in enumerate(r.f["ops"]):
        name = abi.KOP_NAMES[t] if t < len(abi.KOP_NAMES) else str(t)
        if t in (abi.KOP_CONST_F, abi.KOP_ACC_INIT):
            immv = struct.unpack("<f", struct.pack("<I", imm))[0]
        else:
            immv = imm
        out.append("%3d %-8s %4d %4d %4d imm=%s" % (i, name, a0, a1, a2, immv))
    return "\n".join(out)


def snapshot_array(r: Rec, dtype=np.float32) -> np.ndarray:
    return np.frombuffer(r.f["data"], dtype=dtype)
