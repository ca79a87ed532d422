/*
 * chain.c - an elementwise program fused into the launch of the elementwise
 * program whose output it reads.
 *
 * The engine dispatches each realized node as its own UOP_KERNEL
 * (src/schedule/_.c:2268-2411): batchnorm's normalisation and its scale and
 * shift, the relu after them, the routing mask of the pooling backward and
 * its product with the scale are separate launches, each reading the tensor
 * the one before wrote. When such a program P (no loop, or one loop that
 * each lane runs for its own gid, every STORE after it and at its own gid)
 * is held back for a batched launch and the next dispatch C (no loop, one
 * STORE at gid) reads P's output only at its own gid, the two run
 * as one program M: P's ops, then C's, with each load of P's output taking
 * the value P stores there and C's STORE naming the leaf slot that holds C's
 * output (a KOp STORE names its buffer in imm.u, src/tinyhvm.h:683; the
 * engine's own programs always store to buffer 0). M still writes both
 * outputs; it saves C's launch and C's read of P's output. A lane computes
 * P's and C's values for one gid from the same loads in the same order, so
 * the results are those of the two launches bit for bit.
 */
#include <stdlib.h>
#include <string.h>

#include "hipb.h"
#include "affine.h"

static u32 launch_total(const UOpKernel *k) {
    return k->local_size > 0 ? k->grid[0] : k->grid[0] * k->grid[1] * k->grid[2];
}

/* op-index operands of an op (the generator's own rule: unary ALUs carry
 * an earlier op in arg[1] too) */
static u32 op_refs(KOpType t) {
    switch (t) {
    case KOP_MOD: case KOP_DIV: case KOP_LOAD: return 1;
    case KOP_IDX: case KOP_MASK: case KOP_STORE: case KOP_ALU: return 2;
    default: return 0;
    }
}

static int loop_free(const UOpKernel *k) {
    if (k->n_ops == 0 || k->n_ops > CHAIN_MAX_OPS || k->local_size != 0) return 0;
    for (u32 i = 0; i < k->n_ops; i++) {
        const KOpType t = k->ops[i].type;
        if (t <= KOP_NOOP || t > KOP_MASK || t == KOP_RANGE || t == KOP_ENDRANGE || t == KOP_ACC_INIT ||
            t == KOP_ACC)
            return 0;
        for (u32 a = 0; a < op_refs(t); a++)
            if (k->ops[i].arg[a] >= i) return 0;
    }
    return 1;
}

/* A producer: loop-free, or one top-level loop (the generator's serial
 * form: each lane loops for its own gid) with every STORE after it. */
static int producer_form(const UOpKernel *k) {
    if (k->n_ops == 0 || k->n_ops > CHAIN_MAX_OPS || k->local_size != 0) return 0;
    int depth = 0, loops = 0;
    for (u32 i = 0; i < k->n_ops; i++) {
        const KOp *op = &k->ops[i];
        const KOpType t = op->type;
        if (t <= KOP_NOOP || t > KOP_MASK) return 0;
        for (u32 a = 0; a < op_refs(t); a++)
            if (op->arg[a] >= i) return 0;
        if (t == KOP_RANGE) {
            if (depth++ == 0) loops++;
        } else if (t == KOP_ENDRANGE) {
            if (--depth < 0 || op->arg[0] >= i || k->ops[op->arg[0]].type != KOP_RANGE) return 0;
        } else if (t == KOP_ACC && (op->arg[0] >= i || k->ops[op->arg[0]].type != KOP_ACC_INIT)) {
            return 0;
        } else if (t == KOP_STORE && depth > 0) {
            return 0;
        }
    }
    return depth == 0 && loops <= 1;
}

static u32 slot_dtype(const UOpKernel *k, u32 slot) { return slot ? k->leaf_dtypes[slot - 1] : k->out_dtype; }

u64 chain_store_slots(const UOpKernel *k) {
    u64 m = 0;
    for (u32 i = 0; i < k->n_ops; i++)
        if (k->ops[i].type == KOP_STORE && k->ops[i].imm.u > 0 && k->ops[i].imm.u <= k->n_leaves &&
            k->ops[i].imm.u < 64)
            m |= 1ull << k->ops[i].imm.u;
    return m;
}

ChainInfo *chain_info_make(const UOpKernel *k, const KOp *ops) {
    if (!k || !ops || !producer_form(k) || k->n_leaves > FUSE_MAX_LEAVES) return NULL;
    const u32 total = launch_total(k);
    if (total == 0) return NULL;
    Aff *aff = calloc(k->n_ops, sizeof(Aff));
    ChainInfo *ci = calloc(1, sizeof *ci);
    if (!aff || !ci) {
        free(aff);
        free(ci);
        return NULL;
    }
    DCtx dc = {k, total, 1, -1, aff};
    analyze_aff(&dc);
    int ok = 1;
    for (u32 i = 0; i < k->n_ops && ok; i++) {
        const KOp *op = &k->ops[i];
        if (op->type != KOP_STORE) continue;
        const u32 slot = op->imm.u;
        ok = ci->n_st < CHAIN_MAX_STORES && slot <= k->n_leaves && aff_is_gid(&dc, &aff[op->arg[0]]) &&
             op_type_is_float(k->ops[op->arg[1]].type);
        /* a slot stored twice holds the last value: not a producer */
        for (u32 s = 0; s < ci->n_st && ok; s++) ok = ci->st_slot[s] != slot;
        if (!ok) break;
        ci->st_slot[ci->n_st] = slot;
        ci->st_val[ci->n_st] = op->arg[1];
        ci->st_f32[ci->n_st] = slot_dtype(k, slot) == DTYPE_F32;
        ci->n_st++;
    }
    ci->gid_loads = ~0ull;
    for (u32 i = 0; i < k->n_ops && ok; i++) {
        const KOp *op = &k->ops[i];
        if (op->type == KOP_LOAD && op->imm.u < 64 && !aff_is_gid(&dc, &aff[op->arg[0]]))
            ci->gid_loads &= ~(1ull << op->imm.u);
    }
    free(aff);
    if (!ok || ci->n_st == 0) {
        free(ci);
        return NULL;
    }
    ci->ops = ops;
    ci->n_ops = k->n_ops;
    ci->n_leaves = k->n_leaves;
    ci->total = total;
    memcpy(ci->grid, k->grid, sizeof ci->grid);
    ci->out_dtype = k->out_dtype;
    memcpy(ci->leaf_dtypes, k->leaf_dtypes, sizeof ci->leaf_dtypes);
    return ci;
}

int chain_merge(const ChainInfo *p, const u32 *pb, const UOpKernel *c, u32 c_out, const u32 *c_leaves,
                u32 c_nl, UOpKernel *m, u32 *mb) {
    if (!p || !pb || !c || !c_leaves || !m || !mb || c->n_leaves > c_nl || c->n_leaves > FUSE_MAX_LEAVES ||
        !loop_free(c) || launch_total(c) != p->total || p->n_ops + c->n_ops > CHAIN_MAX_OPS || c_out == 0)
        return 0;
    /* C's output is none of P's buffers, except one P only reads, each lane
     * its own element (an in-place update: the lane's load comes before the
     * merged store), and not read by C */
    for (u32 s = 0; s <= p->n_leaves; s++) {
        if (pb[s] != c_out) continue;
        if (s == 0 || s >= 64 || !((p->gid_loads >> s) & 1u)) return 0;
        for (u32 j = 0; j < p->n_st; j++)
            if (p->st_slot[j] == s) return 0;
    }
    for (u32 j = 0; j < c->n_leaves; j++)
        if (c_leaves[j] == c_out) return 0;
    Aff *aff = calloc(c->n_ops, sizeof(Aff));
    if (!aff) return 0;
    DCtx dc = {c, p->total, 1, -1, aff};
    analyze_aff(&dc);
    /* each of C's leaf slots: P's stored value (sub >= 0) or a slot of M */
    i32 sub[FUSE_MAX_LEAVES];
    u32 slot[FUSE_MAX_LEAVES];
    for (u32 j = 0; j < FUSE_MAX_LEAVES; j++) sub[j] = -1;
    u32 nl = p->n_leaves;
    memcpy(mb, pb, (1u + p->n_leaves) * sizeof(u32));
    memset(m->leaf_dtypes, 0, sizeof m->leaf_dtypes);
    memcpy(m->leaf_dtypes, p->leaf_dtypes, p->n_leaves * sizeof(u32));
    int ok = 1, stores = 0;
    for (u32 j = 0; j < c->n_leaves && ok; j++) {
        const u32 id = c_leaves[j], dt = c->leaf_dtypes[j];
        sub[j] = -1;
        slot[j] = 0;
        /* two of P's slots may name the same buffer: it holds the last store */
        for (u32 s = 0; s < p->n_st; s++)
            if (id && pb[p->st_slot[s]] == id) sub[j] = (i32)s;
        if (sub[j] >= 0) ok = p->st_f32[sub[j]] && dt == DTYPE_F32;
        if (sub[j] >= 0 || !ok) continue;
        for (u32 s = 1; s <= nl && !slot[j]; s++)
            if (mb[s] == id && m->leaf_dtypes[s - 1] == dt) slot[j] = s;
        if (slot[j]) continue;
        if (nl + 1 >= FUSE_MAX_LEAVES) { ok = 0; break; }   /* one slot stays for C's output */
        nl++;
        mb[nl] = id;
        m->leaf_dtypes[nl - 1] = dt;
        slot[j] = nl;
    }
    const u32 out_slot = nl + 1;
    ok = ok && out_slot < 64;   /* written slots are tracked in a 64-bit mask */
    /* M's ops: P's, then C's renumbered */
    u32 map[KOP_MAX];
    u32 n = p->n_ops;
    if (ok) memcpy(m->ops, p->ops, p->n_ops * sizeof(KOp));
    /* P's loads past its leaves read 0 there: keep them past M's */
    for (u32 i = 0; i < p->n_ops && ok; i++)
        if (m->ops[i].type == KOP_LOAD && m->ops[i].imm.u > p->n_leaves) m->ops[i].imm.u = FUSE_MAX_LEAVES + 1u;
    for (u32 i = 0; i < c->n_ops && ok; i++) {
        KOp op = c->ops[i];
        if (op.type == KOP_LOAD && op.imm.u == 0) { ok = 0; break; }   /* C reads its own output */
        if (op.type == KOP_LOAD && op.imm.u >= 1 && op.imm.u <= c->n_leaves && sub[op.imm.u - 1] >= 0) {
            /* a load of P's output: only at gid, where P's lane stored it */
            ok = aff_is_gid(&dc, &aff[op.arg[0]]);
            map[i] = p->st_val[sub[op.imm.u - 1]];
            continue;
        }
        for (u32 a = 0; a < op_refs(op.type); a++) op.arg[a] = map[op.arg[a]];
        if (op.type == KOP_LOAD) op.imm.u = (op.imm.u >= 1 && op.imm.u <= c->n_leaves) ? slot[op.imm.u - 1]
                                                                                        : FUSE_MAX_LEAVES + 1u;
        if (op.type == KOP_STORE) {
            ok = stores++ == 0 && op.imm.u == 0 && aff_is_gid(&dc, &aff[c->ops[i].arg[0]]);
            op.imm.u = out_slot;
        }
        map[i] = n;
        m->ops[n++] = op;
    }
    free(aff);
    int reads = 0;
    for (u32 j = 0; j < c->n_leaves; j++) reads |= sub[j] >= 0;
    if (!ok || stores != 1 || !reads) return 0;   /* C reads an output of P */
    mb[out_slot] = c_out;
    m->leaf_dtypes[out_slot - 1] = c->out_dtype;
    m->n_ops = n;
    m->n_leaves = out_slot;
    m->n_bufs = out_slot + 1;
    memcpy(m->grid, p->grid, sizeof m->grid);
    m->local_size = 0;
    m->out_dtype = p->out_dtype;
    return 1;
}
