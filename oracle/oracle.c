/*
 * oracle.c - CPU restatement of the TinyHVM CPU backend's kernel semantics.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the reference
 * results are compared against (or as the timed CPU baseline). The product path (tinyhvm_amd) never calls it.
 *
 * It exports a host-memory Backend vtable (`oracle_backend`) so that kernel
 * traces can be replayed through it exactly as through the GPU backend.
 *
 * Functions and the reference code they restate:
 *   ora_h2f / ora_f2h ............ src/tinyhvm.h:433-486 (f16 with the engine's
 *                                  round-half-up on the first dropped bit)
 *   ora_load / ora_store / cast .. src/tinyhvm.h:488-526
 *   ora_alu ...................... src/backend/cpu/dispatch.c:5-21
 *   ora_uop_exec / ora_dispatch_uop
 *                                  src/backend/cpu/uop.c:3-155
 *   ora_dispatch_uop_gids ........ the same interpreter over a chosen list of
 *                                  gids only (sampled checks of kernels too
 *                                  large to interpret whole)
 *   ora_dispatch_uop_exact ....... the same with SUM accumulators kept in
 *                                  double (a checker of long sums, not a
 *                                  restatement: the reference adds in float)
 *   ora_view_read / ora_st_read / ora_dispatch_rs
 *                                  src/backend/cpu/dispatch.c:23-282
 *   ora_contiguify ............... strided masked copy, src/ops/_.c:338-357
 *   ora_op_unary/binary/mm/reduce  legacy per-op slots, src/backend/cpu/ops.c:1-130
 *   ora_adam_step ................ the adam_step slot with the lazy update's
 *                                  arithmetic, src/nn/adam.c:75-88
 *   pool (alloc ids, reset) ...... src/backend/cpu/pool.c:6-26
 *
 * Deliberate difference from the reference: every load and store is checked
 * against the buffer size (out-of-range loads read 0, stores are dropped).
 * The reference reads out of range for masked pad positions and faults there
 * (its LOAD runs before the MASK select); masked values are discarded, so the
 * results are identical wherever the reference does not fault.
 *
 * Parity pins (tests/): bit-exact against the reference CPU backend's own
 * outputs recorded in tests/golden/*.trc (SNAPSHOT records; for kernels whose
 * masked loads leave their buffer, the reference run over zero-filled guard
 * memory); the fused workload's closed form in f64; textbook restatements of
 * the convolution, padding and pool-backward kernels.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "thvm_abi.h"

/* ---------------- dtype helpers ---------------- */
f32 ora_h2f(u16 h) {
    u32 sign = ((u32)h & 0x8000u) << 16;
    u32 ex = ((u32)h >> 10) & 0x1Fu;
    u32 man = (u32)h & 0x03FFu;
    u32 bits;
    if (ex == 0) {
        if (man == 0) bits = sign;
        else {
            ex = 1;
            while ((man & 0x0400u) == 0) { man <<= 1; ex -= 1; }
            man &= 0x03FFu;
            bits = sign | ((ex + 127 - 15) << 23) | (man << 13);
        }
    } else if (ex == 0x1Fu) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((ex + 127 - 15) << 23) | (man << 13);
    }
    f32 out;
    memcpy(&out, &bits, 4);
    return out;
}

u16 ora_f2h(f32 f) {
    u32 x;
    memcpy(&x, &f, 4);
    u32 sign = (x >> 16) & 0x8000u;
    i32 ex = (i32)((x >> 23) & 0xFFu) - 127 + 15;
    u32 man = x & 0x7FFFFFu;
    if (ex <= 0) {
        if (ex < -10) return (u16)sign;
        man = (man | 0x800000u) >> (1 - ex);
        if (man & 0x1000u) man += 0x2000u;
        return (u16)(sign | (man >> 13));
    }
    if (ex >= 31) return (u16)(sign | 0x7C00u | (man ? 0x0200u : 0));
    if (man & 0x1000u) {
        man += 0x2000u;
        if (man & 0x800000u) {
            man = 0;
            ex += 1;
            if (ex >= 31) return (u16)(sign | 0x7C00u);
        }
    }
    return (u16)(sign | ((u32)ex << 10) | (man >> 13));
}

static u32 dt_size(u32 dt) { return dt == DTYPE_F16 ? 2u : 4u; }

/* Loads that fell outside their buffer since the counter was last cleared
 * (where the reference interpreter would have read out of bounds). */
u64 ora_oob_loads;

/* Host C conversions on x86-64: the same instructions the reference build uses. */
f32 ora_load(const void *base, u64 nbytes, u32 dt, u32 i) {
    if (!base || (u64)i * dt_size(dt) + dt_size(dt) > nbytes) {
        ora_oob_loads++;
        return 0.0f;
    }
    switch (dt) {
    case DTYPE_F32: return ((const f32 *)base)[i];
    case DTYPE_F16: return ora_h2f(((const u16 *)base)[i]);
    case DTYPE_I32: return (f32)((const i32 *)base)[i];
    case DTYPE_U32: return (f32)((const u32 *)base)[i];
    default: return 0.0f;
    }
}

void ora_store(void *base, u64 nbytes, u32 dt, u32 i, f32 v) {
    if (!base || (u64)i * dt_size(dt) + dt_size(dt) > nbytes) return;
    switch (dt) {
    case DTYPE_F32: ((f32 *)base)[i] = v; break;
    case DTYPE_F16: ((u16 *)base)[i] = ora_f2h(v); break;
    case DTYPE_I32: ((i32 *)base)[i] = (i32)v; break;
    case DTYPE_U32: ((u32 *)base)[i] = (u32)v; break;
    default: break;
    }
}

f32 ora_cast(f32 v, u32 dt) {
    switch (dt) {
    case DTYPE_F32: return v;
    case DTYPE_F16: return ora_h2f(ora_f2h(v));
    case DTYPE_I32: return (f32)(i32)v;
    case DTYPE_U32: return (f32)(u32)v;
    default: return v;
    }
}

f32 ora_alu(u32 uop, u32 aux, f32 a, f32 b) {
    switch (uop) {
    case UOP_ADD: return a + b;
    case UOP_MUL: return a * b;
    case UOP_DIV: return b != 0.f ? a / b : 0.f;
    case UOP_SUB: return a - b;
    case UOP_MAX: return a > b ? a : b;
    case UOP_CMP: return a > b ? 1.f : 0.f;
    case UOP_NEG: return -a;
    case UOP_RELU: return a > 0.f ? a : 0.f;
    case UOP_EXP: return expf(a);
    case UOP_LOG: return logf(a);
    case UOP_SQRT: return sqrtf(a);
    case UOP_CAST: return ora_cast(a, aux);
    default: return a;
    }
}

/* ---------------- KOp interpreter ---------------- */
typedef struct {
    const UOpKernel *k;
    const u32 *range_end;
    void *out;
    u64 out_bytes;
    const void **leaf;
    const u64 *leaf_bytes;
    u32 n_leaf_ptrs;
    u32 *uv;
    f32 *fv;
    double *dv;    /* exact mode: SUM accumulators in double, else NULL */
} OraCtx;

static int is_ftype(const UOpKernel *k, u32 id) {
    if (id >= k->n_ops) return 0;
    switch (k->ops[id].type) {
    case KOP_CONST_F: case KOP_LOAD: case KOP_ALU: case KOP_ACC_INIT: case KOP_MASK: return 1;
    default: return 0;
    }
}
static u32 as_u(const OraCtx *c, u32 id) {
    if (id >= c->k->n_ops) return 0;
    return is_ftype(c->k, id) ? (u32)c->fv[id] : c->uv[id];
}
static f32 as_f(const OraCtx *c, u32 id) {
    if (id >= c->k->n_ops) return 0.0f;
    return is_ftype(c->k, id) ? c->fv[id] : (f32)c->uv[id];
}

/* Returns 0 where the reference interpreter would abandon the dispatch. */
static int ora_uop_exec(OraCtx *c, u32 start, u32 stop, u32 gid) {
    const UOpKernel *k = c->k;
    for (u32 i = start; i < stop; i++) {
        const KOp *op = &k->ops[i];
        switch (op->type) {
        case KOP_GID: c->uv[i] = gid; break;
        case KOP_CONST_U: c->uv[i] = op->imm.u; break;
        case KOP_CONST_F: c->fv[i] = op->imm.f; break;
        case KOP_MOD: c->uv[i] = op->imm.u ? as_u(c, op->arg[0]) % op->imm.u : 0; break;
        case KOP_DIV: c->uv[i] = op->imm.u ? as_u(c, op->arg[0]) / op->imm.u : 0; break;
        case KOP_IDX: c->uv[i] = as_u(c, op->arg[0]) * op->imm.u + as_u(c, op->arg[1]); break;
        case KOP_LOAD: {
            u32 bi = op->imm.u;
            if (bi == 0) c->fv[i] = ora_load(c->out, c->out_bytes, k->out_dtype, as_u(c, op->arg[0]));
            else if (bi - 1 < k->n_leaves && bi - 1 < c->n_leaf_ptrs)
                c->fv[i] = ora_load(c->leaf[bi - 1], c->leaf_bytes[bi - 1], k->leaf_dtypes[bi - 1],
                                    as_u(c, op->arg[0]));
            else c->fv[i] = 0.0f;
            break;
        }
        case KOP_MASK: c->fv[i] = as_f(c, op->arg[0]) != 0.0f ? as_f(c, op->arg[1]) : 0.0f; break;
        case KOP_ALU: c->fv[i] = ora_alu(op->imm.u, op->arg[2], as_f(c, op->arg[0]), as_f(c, op->arg[1])); break;
        case KOP_ACC_INIT:
            c->fv[i] = op->imm.f;
            if (c->dv) c->dv[i] = op->imm.f;
            break;
        case KOP_ACC: {
            u32 a = op->arg[0];
            f32 v = as_f(c, op->arg[1]);
            if (a >= k->n_ops) break;
            if (op->imm.u == UOP_RMAX) {
                c->fv[a] = c->fv[a] > v ? c->fv[a] : v;
                if (c->dv) c->dv[a] = c->fv[a];
            } else if (c->dv) {
                c->dv[a] += (double)v;
                c->fv[a] = (f32)c->dv[a];
            } else {
                c->fv[a] = c->fv[a] + v;
            }
            break;
        }
        case KOP_RANGE: {
            u32 end = c->range_end[i];
            if (end == 0xFFFFFFFFu || end <= i) return 0;
            for (u32 r = 0; r < op->imm.u; r++) {
                c->uv[i] = r;
                if (!ora_uop_exec(c, i + 1, end, gid)) return 0;
            }
            i = end;
            break;
        }
        case KOP_ENDRANGE: break;
        case KOP_STORE: ora_store(c->out, c->out_bytes, k->out_dtype, as_u(c, op->arg[0]), as_f(c, op->arg[1])); break;
        default: return 0;
        }
    }
    return 1;
}

static void ora_dispatch_uop_mode(void *out, u64 out_bytes, const void **leaf, const u64 *leaf_bytes,
                                  u32 n_leaves, const UOpKernel *k, int exact, const u32 *gids, u64 n_gids) {
    if (!k || !out || k->n_ops > KOP_MAX) return;
    u32 range_end[KOP_MAX], stack[KOP_MAX], sp = 0;
    for (u32 i = 0; i < KOP_MAX; i++) range_end[i] = 0xFFFFFFFFu;
    for (u32 i = 0; i < k->n_ops; i++) {
        if (k->ops[i].type == KOP_RANGE) stack[sp++] = i;
        else if (k->ops[i].type == KOP_ENDRANGE) {
            if (sp == 0) return;
            range_end[stack[--sp]] = i;
        }
    }
    if (sp != 0) return;
    u32 uv[KOP_MAX];
    f32 fv[KOP_MAX];
    double dv[KOP_MAX];
    OraCtx c = {k, range_end, out, out_bytes, leaf, leaf_bytes, n_leaves, uv, fv, exact ? dv : NULL};
    u32 total = k->local_size > 0 ? k->grid[0] : k->grid[0] * k->grid[1] * k->grid[2];
    if (gids) {
        for (u64 j = 0; j < n_gids; j++) {
            if (gids[j] >= total) continue;
            memset(uv, 0, sizeof uv);
            memset(fv, 0, sizeof fv);
            if (!ora_uop_exec(&c, 0, k->n_ops, gids[j])) return;
        }
        return;
    }
    for (u32 gid = 0; gid < total; gid++) {
        memset(uv, 0, sizeof uv);
        memset(fv, 0, sizeof fv);
        if (!ora_uop_exec(&c, 0, k->n_ops, gid)) return;
    }
}

void ora_dispatch_uop(void *out, u64 out_bytes, const void **leaf, const u64 *leaf_bytes, u32 n_leaves,
                      const UOpKernel *k) {
    ora_dispatch_uop_mode(out, out_bytes, leaf, leaf_bytes, n_leaves, k, 0, NULL, 0);
}

/* The interpreter for the listed gids only (each runs its whole program, so
 * its stores are exactly those of the full dispatch); gids past the launch
 * are skipped. */
void ora_dispatch_uop_gids(void *out, u64 out_bytes, const void **leaf, const u64 *leaf_bytes, u32 n_leaves,
                           const UOpKernel *k, const u32 *gids, u64 n_gids) {
    if (!gids) return;
    ora_dispatch_uop_mode(out, out_bytes, leaf, leaf_bytes, n_leaves, k, 0, gids, n_gids);
}

/* The kernel with every SUM accumulated in double and rounded to float when
 * an op reads it: the exact sum of the same float terms, to tell a reordered
 * GPU sum's error from the float rounding of the reference's own serial one
 * over long reductions. */
void ora_dispatch_uop_exact(void *out, u64 out_bytes, const void **leaf, const u64 *leaf_bytes, u32 n_leaves,
                            const UOpKernel *k) {
    ora_dispatch_uop_mode(out, out_bytes, leaf, leaf_bytes, n_leaves, k, 1, NULL, 0);
}

/* ---------------- FusedOp interpreter ---------------- */
static f32 ora_st_read(const void *buf, u64 nb, u32 dt, const ShapeTracker *st, const u32 *coords, u32 rank,
                       const u32 *full_dims) {
    if (!st || st->n_views <= 1) return 0.f;
    u32 si = 0;
    {
        u32 stride = 1;
        for (i32 d = (i32)rank - 1; d >= 0; d--) {
            si += coords[d] * stride;
            stride *= full_dims[d];
        }
    }
    for (i32 vi = (i32)st->n_views - 2; vi >= 0; vi--) {
        const View *vw = &st->views[vi];
        const View *outer = &st->views[vi + 1];
        u32 outer_flat = 0;
        {
            u32 udiv = 1, ostr[MAX_DIM];
            u32 orank = outer->shape.rank < MAX_DIM ? outer->shape.rank : MAX_DIM;
            if (orank > 0) {
                ostr[orank - 1] = 1;
                for (i32 d = (i32)orank - 2; d >= 0; d--) ostr[d] = ostr[d + 1] * outer->shape.dims[d + 1];
            }
            for (i32 d = (i32)orank - 1; d >= 0; d--) {
                u32 dim = outer->shape.dims[d];
                if (dim <= 1) { udiv *= dim; continue; }
                u32 cc = udiv ? (si / udiv) % dim : 0;
                outer_flat += cc * ostr[d];
                udiv *= dim;
            }
        }
        i32 idx = vw->offset;
        {
            u32 rem = outer_flat, istr[MAX_DIM];
            u32 irank = vw->shape.rank < MAX_DIM ? vw->shape.rank : MAX_DIM;
            if (irank > 0) {
                istr[irank - 1] = 1;
                for (i32 d = (i32)irank - 2; d >= 0; d--) istr[d] = istr[d + 1] * vw->shape.dims[d + 1];
            }
            for (u32 d = 0; d < irank; d++) {
                u32 cc = istr[d] ? rem / istr[d] : 0;
                rem = istr[d] ? rem % istr[d] : rem;
                if (vw->has_mask && (cc < vw->mask_begin[d] || cc >= vw->mask_end[d])) return 0.f;
                if (vw->strides[d] != 0) idx = (i32)((u32)idx + cc * (u32)vw->strides[d]);
            }
        }
        if (idx < 0) return 0.f;
        si = (u32)idx;
    }
    return ora_load(buf, nb, dt, si);
}

static f32 ora_view_read(const void *buf, u64 nb, u32 dt, const View *v, const u32 *coords, u32 rank) {
    if (v->has_mask) {
        for (u32 d = 0; d < rank && d < v->shape.rank; d++)
            if (coords[d] < v->mask_begin[d] || coords[d] >= v->mask_end[d]) return 0.f;
        for (u32 cm = 0; cm < v->n_compound_masks; cm++) {
            u32 da = v->compound_masks[cm].dim_a, db = v->compound_masks[cm].dim_b;
            if (da >= MAX_DIM || db >= MAX_DIM) return 0.f;
            i32 composed = (i32)coords[da] * v->compound_masks[cm].stride_a + (i32)coords[db];
            if (composed < (i32)v->compound_masks[cm].begin || composed >= (i32)v->compound_masks[cm].end)
                return 0.f;
        }
    }
    i32 idx = v->offset;
    for (u32 d = 0; d < rank && d < v->shape.rank; d++) {
        u32 dim = v->shape.dims[d];
        u32 cc = dim ? coords[d] % dim : 0;
        idx = (i32)((u32)idx + cc * (u32)v->strides[d]);
    }
    if (idx < 0) return 0.f;
    return ora_load(buf, nb, dt, (u32)idx);
}

void ora_dispatch_rs(void *out, u64 out_bytes, const void **leaf, const u64 *leaf_bytes, const View **views,
                     const ShapeTracker *const *sts, u32 n_leaves, const FusedOp *ops, u32 n_ops,
                     const Shape *full, const ReduceSpec *reduce, const u32 *leaf_dtypes, u32 out_dtype) {
    u32 rank = full->rank ? full->rank : 1;
    if (rank > MAX_DIM) return;
    int has_reduce = reduce && reduce->reduce_type;
    u32 out_numel = 1, full_numel = 1, out_shape[MAX_DIM];
    for (u32 d = 0; d < rank; d++) {
        full_numel *= full->dims[d];
        out_shape[d] = (has_reduce && reduce->is_reduce[d]) ? 1 : full->dims[d];
        out_numel *= out_shape[d];
    }
    if (has_reduce) {
        f32 init = reduce->reduce_type == UOP_RMAX ? -1e30f : 0.f;
        for (u32 i = 0; i < out_numel; i++) ora_store(out, out_bytes, out_dtype, i, init);
    }
    u32 fs[MAX_DIM], os[MAX_DIM];
    fs[rank - 1] = 1;
    os[rank - 1] = 1;
    for (i32 d = (i32)rank - 2; d >= 0; d--) {
        fs[d] = fs[d + 1] * full->dims[d + 1];
        os[d] = os[d + 1] * out_shape[d + 1];
    }
    f32 vals[FUSE_MAX_LEAVES + FUSE_MAX_OPS];
    memset(vals, 0, sizeof vals);
    for (u32 flat = 0; flat < full_numel; flat++) {
        u32 coords[MAX_DIM], rem = flat;
        for (u32 d = 0; d < rank; d++) {
            coords[d] = fs[d] ? rem / fs[d] : 0;
            rem = fs[d] ? rem % fs[d] : rem;
        }
        for (u32 i = 0; i < n_leaves; i++) {
            u32 dt = leaf_dtypes ? leaf_dtypes[i] : DTYPE_F32;
            if (sts && sts[i] && sts[i]->n_views >= 2)
                vals[i] = ora_st_read(leaf[i], leaf_bytes[i], dt, sts[i], coords, rank, full->dims);
            else
                vals[i] = ora_view_read(leaf[i], leaf_bytes[i], dt, views[i], coords, rank);
        }
        u32 en = (has_reduce && reduce->post_reduce_start) ? reduce->post_reduce_start : n_ops;
        for (u32 i = 0; i < en; i++) {
            u32 aa = ops[i].arg_a, bb = ops[i].arg_b;
            if (aa >= n_leaves + en || bb >= n_leaves + en) break;
            vals[n_leaves + i] = ora_alu(ops[i].uop, ops[i].aux, vals[aa], vals[bb]);
        }
        f32 result = en > 0 ? vals[n_leaves + en - 1] : vals[0];
        if (has_reduce) {
            u32 oi = 0;
            for (u32 d = 0; d < rank; d++) if (!reduce->is_reduce[d]) oi += coords[d] * os[d];
            f32 cur = ora_load(out, out_bytes, out_dtype, oi);
            if (reduce->reduce_type == UOP_SUM) ora_store(out, out_bytes, out_dtype, oi, cur + result);
            else if (reduce->reduce_type == UOP_RMAX) ora_store(out, out_bytes, out_dtype, oi, result > cur ? result : cur);
        } else {
            ora_store(out, out_bytes, out_dtype, flat, result);
        }
    }
    if (has_reduce && reduce->post_reduce_start && reduce->post_reduce_start < n_ops) {
        u32 ps = reduce->post_reduce_start;
        u32 zero_dims[MAX_DIM] = {0};
        const u32 LIM = FUSE_MAX_LEAVES + FUSE_MAX_OPS;
        for (u32 oi = 0; oi < out_numel; oi++) {
            u32 coords[MAX_DIM], rem = oi;
            for (u32 d = 0; d < rank; d++) {
                coords[d] = os[d] ? rem / os[d] : 0;
                rem = os[d] ? rem % os[d] : rem;
            }
            f32 rr = ora_load(out, out_bytes, out_dtype, oi);
            u32 npre = n_leaves - reduce->n_post_leaves;
            for (u32 i = 0; i < n_leaves; i++) {
                if (i < npre) { vals[i] = 0; continue; }
                u32 dt = leaf_dtypes ? leaf_dtypes[i] : DTYPE_F32;
                if (sts && sts[i] && sts[i]->n_views >= 2)
                    vals[i] = ora_st_read(leaf[i], leaf_bytes[i], dt, sts[i], coords, rank, zero_dims);
                else
                    vals[i] = ora_view_read(leaf[i], leaf_bytes[i], dt, views[i], coords, rank);
            }
            if (ps > 0 && n_leaves + ps - 1 < LIM) vals[n_leaves + ps - 1] = rr;
            for (u32 i = ps; i < n_ops; i++) {
                u32 aa = ops[i].arg_a, bb = ops[i].arg_b;
                f32 a = aa < LIM ? vals[aa] : 0.f, b = bb < LIM ? vals[bb] : 0.f;
                vals[n_leaves + i] = ora_alu(ops[i].uop, ops[i].aux, a, b);
            }
            ora_store(out, out_bytes, out_dtype, oi, vals[n_leaves + n_ops - 1]);
        }
    }
}

/* ASSIGN from a strided view into a dense buffer. The engine's CPU backend
 * has no contiguify slot; without it ASSIGN reads the source to the host
 * (thvm_to_host_raw, src/ops/_.c:338-357) and writes it back, so that read is
 * the semantics: per-dim mask checked, strides below 0 counted as 0 (:348),
 * compound masks not consulted, element size from the dtype. esize is the
 * destination's bytes per element (dtypes agree, src/interact/tensor_ops.c:116). */
void ora_contiguify(void *dst, u64 dst_bytes, const void *src, u64 src_bytes, u32 numel, const View *v,
                    u32 esize) {
    for (u32 t = 0; t < numel && (u64)(t + 1) * esize <= dst_bytes; t++) {
        u32 rem = t;
        i32 idx = v->offset;
        int masked = 0;
        for (i32 d = (i32)v->shape.rank - 1; d >= 0; d--) {
            u32 dim = v->shape.dims[d];
            u32 cc = dim ? rem % dim : 0;
            rem = dim ? rem / dim : 0;
            if (v->has_mask && (cc < v->mask_begin[d] || cc >= v->mask_end[d])) masked = 1;
            idx += (i32)cc * (v->strides[d] > 0 ? v->strides[d] : 0);
        }
        int ok = !masked && idx >= 0 && (u64)((u32)idx + 1) * esize <= src_bytes;
        if (esize == 2) ((u16 *)dst)[t] = ok ? ((const u16 *)src)[(u32)idx] : 0;
        else ((u32 *)dst)[t] = ok ? ((const u32 *)src)[(u32)idx] : 0;
    }
}

/* ---------------- legacy per-op slots (src/backend/cpu/ops.c) ---------------- */

/* strided_index, src/backend/cpu/ops.c:3-13: u32 arithmetic, no masks. */
static u32 ora_strided_index(u32 flat, const View *v) {
    u32 idx = (u32)v->offset, rem = flat;
    for (i32 d = (i32)v->shape.rank - 1; d >= 0; d--) {
        u32 dim = v->shape.dims[d];
        u32 coord = dim ? rem % dim : 0;
        rem = dim ? rem / dim : 0;
        idx += coord * (u32)v->strides[d];
    }
    return idx;
}

/* cpu_op_unary, src/backend/cpu/ops.c:15-33 */
void ora_op_unary(u32 uop, void *dst, u64 dst_bytes, const View *dv, u32 dd, const void *src, u64 src_bytes,
                  const View *sv, u32 sd) {
    for (u32 i = 0; i < dv->numel; i++) {
        f32 val = ora_load(src, src_bytes, sd, ora_strided_index(i, sv));
        switch (uop) {
        case UOP_NEG: val = -val; break;
        case UOP_RELU: val = val > 0.0f ? val : 0.0f; break;
        case UOP_EXP: val = expf(val); break;
        case UOP_LOG: val = logf(val); break;
        case UOP_SQRT: val = sqrtf(val); break;
        default: break;
        }
        ora_store(dst, dst_bytes, dd, i, val);
    }
}

/* cpu_op_binary, src/backend/cpu/ops.c:35-60 */
void ora_op_binary(u32 uop, void *dst, u64 dst_bytes, const View *dv, u32 dd, const void *a, u64 a_bytes,
                   const View *av, u32 ad, const void *b, u64 b_bytes, const View *bv, u32 bd) {
    for (u32 i = 0; i < dv->numel; i++) {
        f32 va = ora_load(a, a_bytes, ad, ora_strided_index(i, av));
        f32 vb = ora_load(b, b_bytes, bd, ora_strided_index(i, bv));
        f32 vr;
        switch (uop) {
        case UOP_ADD: vr = va + vb; break;
        case UOP_MUL: vr = va * vb; break;
        case UOP_DIV: vr = vb != 0.0f ? va / vb : 0.0f; break;
        case UOP_SUB: vr = va - vb; break;
        case UOP_MAX: vr = va > vb ? va : vb; break;
        case UOP_CMP: vr = va > vb ? 1.0f : 0.0f; break;
        default: vr = va; break;
        }
        ora_store(dst, dst_bytes, dd, i, vr);
    }
}

/* cpu_op_mm without BLAS, src/backend/cpu/ops.c:80-113: k innermost, in order */
void ora_op_mm(void *dst, u64 dst_bytes, u32 dd, const void *a, u64 a_bytes, const View *av, u32 ad,
               const void *b, u64 b_bytes, const View *bv, u32 bd, u32 M, u32 K, u32 N) {
    for (u32 i = 0; i < M; i++)
        for (u32 j = 0; j < N; j++) {
            f32 acc = 0;
            for (u32 k = 0; k < K; k++) {
                f32 va = ora_load(a, a_bytes, ad, ora_strided_index(i * K + k, av));
                f32 vb = ora_load(b, b_bytes, bd, ora_strided_index(k * N + j, bv));
                acc += va * vb;
            }
            ora_store(dst, dst_bytes, dd, i * N + j, acc);
        }
}

/* cpu_op_reduce, src/backend/cpu/ops.c:115-130: innermost reduce_dim elements */
void ora_op_reduce(u32 uop, void *dst, u64 dst_bytes, u32 dst_numel, u32 dd, const void *src, u64 src_bytes,
                   u32 sd, u32 reduce_dim) {
    for (u32 o = 0; o < dst_numel; o++) {
        f32 acc = uop == UOP_RMAX ? -1e30f : 0.0f;
        for (u32 r = 0; r < reduce_dim; r++) {
            f32 v = ora_load(src, src_bytes, sd, o * reduce_dim + r);
            if (uop == UOP_SUM) acc += v;
            else if (uop == UOP_RMAX) acc = v > acc ? v : acc;
        }
        ora_store(dst, dst_bytes, dd, o, acc);
    }
}

/* ---------------- Adam ---------------- */

/* The adam_step slot (src/tinyhvm.h:1033-1035) with the arithmetic of the
 * engine's lazy update, which is what the CPU backend computes (it has no
 * slot): every product, quotient and sum rounded to f32 in the order of the
 * op composition of src/nn/adam.c:75-88,
 *   m' = beta1*m + (1-beta1)*g
 *   v' = beta2*v + (1-beta2)*(g*g)
 *   p' = p - lr * ((m'/bc1) / (sqrt(v'/bc2) + eps))
 * with the engine's guarded DIV (src/backend/cpu/dispatch.c:5-21). */
void ora_adam_step(f32 *p, const f32 *g, f32 *m, f32 *v, f32 lr, f32 beta1, f32 beta2, f32 eps, f32 bc1, f32 bc2,
                   u32 n) {
    const f32 omb1 = 1.0f - beta1, omb2 = 1.0f - beta2;
    for (u32 i = 0; i < n; i++) {
        const f32 gi = g[i];
        f32 mi = ora_alu(UOP_ADD, 0, ora_alu(UOP_MUL, 0, beta1, m[i]), ora_alu(UOP_MUL, 0, omb1, gi));
        f32 vi = ora_alu(UOP_ADD, 0, ora_alu(UOP_MUL, 0, beta2, v[i]),
                         ora_alu(UOP_MUL, 0, omb2, ora_alu(UOP_MUL, 0, gi, gi)));
        f32 m_hat = ora_alu(UOP_DIV, 0, mi, bc1);
        f32 v_hat = ora_alu(UOP_DIV, 0, vi, bc2);
        f32 denom = ora_alu(UOP_ADD, 0, ora_alu(UOP_SQRT, 0, v_hat, 0.0f), eps);
        f32 step = ora_alu(UOP_MUL, 0, lr, ora_alu(UOP_DIV, 0, m_hat, denom));
        m[i] = mi;
        v[i] = vi;
        p[i] = ora_alu(UOP_SUB, 0, p[i], step);
    }
}

/* ---------------- host-memory Backend ---------------- */
static struct {
    void **bufs;
    u64 *sizes;
    u32 cap, count;
} OP;

static int ob_init(void) {
    free(OP.bufs);
    free(OP.sizes);
    OP.cap = 1024;
    OP.bufs = calloc(OP.cap, sizeof(void *));
    OP.sizes = calloc(OP.cap, sizeof(u64));
    OP.count = 1;
    return (OP.bufs && OP.sizes) ? 0 : -1;
}
static void ob_shutdown(void) {
    for (u32 i = 1; i < OP.count; i++) free(OP.bufs[i]);
    free(OP.bufs);
    free(OP.sizes);
    memset(&OP, 0, sizeof OP);
}
static u32 ob_alloc(u64 b) {
    if (!OP.bufs && ob_init() != 0) return 0;
    if (OP.count >= OP.cap) {
        u32 nc = OP.cap * 2;
        void **nb = realloc(OP.bufs, nc * sizeof(void *));
        u64 *ns = realloc(OP.sizes, nc * sizeof(u64));
        if (!nb || !ns) return 0;
        memset(nb + OP.cap, 0, (nc - OP.cap) * sizeof(void *));
        memset(ns + OP.cap, 0, (nc - OP.cap) * sizeof(u64));
        OP.bufs = nb;
        OP.sizes = ns;
        OP.cap = nc;
    }
    u32 id = OP.count++;
    OP.bufs[id] = calloc(1, b ? b : 4);
    OP.sizes[id] = b;
    return OP.bufs[id] ? id : 0;
}
static void *ob_ptr(u32 id) { return (id && id < OP.count) ? OP.bufs[id] : NULL; }
static u64 ob_size(u32 id) { return (id && id < OP.count && OP.bufs[id]) ? OP.sizes[id] : 0; }
static void ob_free(u32 id) {
    if (id && id < OP.count) {
        free(OP.bufs[id]);
        OP.bufs[id] = NULL;
        OP.sizes[id] = 0;
    }
}
static void ob_write(u32 id, const void *d, u64 b) {
    void *p = ob_ptr(id);
    if (p && d) memcpy(p, d, b < ob_size(id) ? b : ob_size(id));
}
static void ob_read(u32 id, void *o, u64 b) {
    void *p = ob_ptr(id);
    u64 n = b < ob_size(id) ? b : ob_size(id);
    if (p) memcpy(o, p, n);
    if (n < b) memset((u8 *)o + n, 0, b - n);
}
static void ob_reset(u32 keep) {
    u32 first = keep + 1;
    for (u32 i = first; i < OP.count; i++) ob_free(i);
    if (first < OP.count) OP.count = first;
}
static void ob_uop(u32 out, const u32 *leaves, u32 n, const UOpKernel *k, u64 key) {
    (void)key;
    const void *lp[FUSE_MAX_LEAVES];
    u64 lb[FUSE_MAX_LEAVES];
    for (u32 i = 0; i < n && i < FUSE_MAX_LEAVES; i++) {
        lp[i] = ob_ptr(leaves[i]);
        lb[i] = ob_size(leaves[i]);
    }
    ora_dispatch_uop(ob_ptr(out), ob_size(out), lp, lb, n < FUSE_MAX_LEAVES ? n : FUSE_MAX_LEAVES, k);
}
static void ob_rs(u32 out, u32 *leaves, const View **views, const ShapeTracker *const *sts, u32 n, FusedOp *ops,
                  u32 n_ops, const Shape *full, const ReduceSpec *reduce, u32 *sb, const u32 *si, u32 ns,
                  const u32 *dts, u32 odt) {
    (void)sb; (void)si; (void)ns;
    const void *lp[FUSE_MAX_LEAVES];
    u64 lb[FUSE_MAX_LEAVES];
    for (u32 i = 0; i < n && i < FUSE_MAX_LEAVES; i++) {
        lp[i] = ob_ptr(leaves[i]);
        lb[i] = ob_size(leaves[i]);
    }
    ora_dispatch_rs(ob_ptr(out), ob_size(out), lp, lb, views, sts, n, ops, n_ops, full, reduce, dts, odt);
}
static void ob_copy(u32 d, u32 s, u64 b) {
    void *dp = ob_ptr(d), *sp = ob_ptr(s);
    u64 n = b;
    if (n > ob_size(d)) n = ob_size(d);
    if (n > ob_size(s)) n = ob_size(s);
    if (dp && sp) memmove(dp, sp, n);
}
static void ob_contig(u32 d, u32 numel, u32 s, const View *v) {
    if (ob_ptr(d) && v)
        ora_contiguify(ob_ptr(d), ob_size(d), ob_ptr(s), ob_size(s), numel, v,
                       ob_size(d) == (u64)numel * 2 ? 2 : 4);
}

static void ob_op_unary(u32 uop, u32 dst, const View *dv, u32 dd, u32 src, const View *sv, u32 sd) {
    ora_op_unary(uop, ob_ptr(dst), ob_size(dst), dv, dd, ob_ptr(src), ob_size(src), sv, sd);
}
static void ob_op_binary(u32 uop, u32 dst, const View *dv, u32 dd, u32 a, const View *av, u32 ad, u32 b,
                         const View *bv, u32 bd) {
    ora_op_binary(uop, ob_ptr(dst), ob_size(dst), dv, dd, ob_ptr(a), ob_size(a), av, ad, ob_ptr(b), ob_size(b),
                  bv, bd);
}
static void ob_op_mm(u32 dst, u32 dd, u32 a, const View *av, u32 ad, u32 b, const View *bv, u32 bd, u32 M,
                     u32 K, u32 N) {
    ora_op_mm(ob_ptr(dst), ob_size(dst), dd, ob_ptr(a), ob_size(a), av, ad, ob_ptr(b), ob_size(b), bv, bd, M, K,
              N);
}
static void ob_op_reduce(u32 uop, u32 dst, u32 dn, u32 dd, u32 src, u32 sn, u32 sd, u32 rdim) {
    (void)sn;
    ora_op_reduce(uop, ob_ptr(dst), ob_size(dst), dn, dd, ob_ptr(src), ob_size(src), sd, rdim);
}

static void ob_adam(u32 p, u32 g, u32 m, u32 v, f32 lr, f32 b1, f32 b2, f32 eps, f32 bc1, f32 bc2, u32 n) {
    const u64 need = (u64)n * 4;
    if (ob_size(p) < need || ob_size(g) < need || ob_size(m) < need || ob_size(v) < need) return;
    ora_adam_step(ob_ptr(p), ob_ptr(g), ob_ptr(m), ob_ptr(v), lr, b1, b2, eps, bc1, bc2, n);
}

Backend oracle_backend = {
    .init = ob_init,
    .shutdown = ob_shutdown,
    .buf_alloc = ob_alloc,
    .buf_free = ob_free,
    .buf_write = ob_write,
    .buf_read = ob_read,
    .buf_read_nosync = ob_read,
    .op_unary = ob_op_unary,
    .op_binary = ob_op_binary,
    .op_mm = ob_op_mm,
    .op_reduce = ob_op_reduce,
    .dispatch_kernel_rs = ob_rs,
    .dispatch_uop_kernel = ob_uop,
    .contiguify = ob_contig,
    .buf_copy = ob_copy,
    .pool_reset = ob_reset,
    .adam_step = ob_adam,
};

const Backend *oracle_backend_ptr(void) { return &oracle_backend; }
void *oracle_buf_ptr(u32 id) { return ob_ptr(id); }
u64 oracle_buf_size(u32 id) { return ob_size(id); }
