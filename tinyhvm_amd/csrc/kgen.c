/*
 * kgen.c - lowers a UOpKernel (the engine's linear KOp program) to HIP source
 * for hipRTC.
 *
 * Semantics follow the engine's CPU interpreter (src/backend/cpu/uop.c:1-155)
 * and its ALU (src/backend/cpu/dispatch.c:5-21), with the storage helpers of
 * src/tinyhvm.h:433-526:
 *   - ops are SSA values; CONST_F, LOAD, ALU, ACC_INIT and MASK are float
 *     valued, the rest u32 valued; a u32 value read as float is (float)u and
 *     a float read as u32 is the x86-64 conversion (u32)(int64)trunc(f);
 *   - index arithmetic wraps modulo 2^32, MOD/DIV by 0 give 0;
 *   - RANGE..ENDRANGE is a loop over [0, imm); ACC folds SUM (a+b) or RMAX
 *     (a > b ? a : b) into the accumulator op named by arg[0];
 *   - a launch covers grid[0] outputs when local_size > 0, else the product
 *     of the grid.
 * Deliberate difference: every LOAD and STORE is bounds-checked against the
 * buffer's size (out of range loads read 0, stores are dropped). The CPU
 * interpreter reads out of range for masked pad positions; masked values are
 * discarded by MASK, so results agree wherever the CPU does not fault.
 *
 * Two execution shapes:
 *   SERIAL  one thread runs the whole program for V consecutive gids (V = 4 or
 *           1); loops run sequentially, so SUM order matches the CPU exactly.
 *   GROUP   (local_size > 0) one workgroup per output; the lanes split each
 *           top-level reduce loop, keep per-lane partials, and combine them
 *           with wavefront shuffles and LDS. SUM order differs from the CPU.
 *
 * Vectorization: inside the vector variable's scope (gid in SERIAL, the loop
 * counter in GROUP) each u32 op is classified as invariant (INV), lane-offset
 * (LIN: value at lane v = value at lane 0 + off[v], the offsets known when the
 * kernel is generated) or varying. Lane-offset ops are computed once per
 * thread-vector. The classification tracks a known divisor of the lane-0 value
 * and an upper bound of the value over every lane: dividing or reducing a
 * lane-offset value by d keeps it lane-offset when d divides the divisor, or
 * when every offset is below gcd(divisor, d) (the lanes then share the
 * quotient), as long as the bound proves the u32 arithmetic never wrapped.
 * Loads whose offsets are 0,1,2,3 on a lane-0 index divisible by 4 become one
 * 128-bit load (stores likewise); lanes with equal offsets share one load.
 * In GROUP mode, loads whose index is affine in the loop counter over the
 * whole loop are range-checked once per workgroup and then loaded unchecked.
 */
#include <stdarg.h>
#include <stdlib.h>
#include <string.h>

#include "hipb.h"

/* ---------------- string builder ---------------- */
typedef struct { char *p; size_t n, cap; } SB;

static void sb_put(SB *s, const char *fmt, ...) {
    va_list ap;
    for (;;) {
        size_t room = s->cap - s->n;
        va_start(ap, fmt);
        int w = vsnprintf(s->p ? s->p + s->n : NULL, s->p ? room : 0, fmt, ap);
        va_end(ap);
        if (w < 0) return;
        if (s->p && (size_t)w < room) {
            s->n += (size_t)w;
            return;
        }
        size_t nc = s->cap ? s->cap * 2 : 16384;
        while (nc < s->n + (size_t)w + 1) nc *= 2;
        char *np = realloc(s->p, nc);
        if (!np) return;
        s->p = np;
        s->cap = nc;
    }
}

/* ---------------- analysis ---------------- */
enum { K_INV = 0, K_LIN = 1, K_VAR = 2 };
enum { G_INV = 0, G_LIN = 1, G_NOT = 2 };

typedef struct {
    u8  ft;        /* float valued */
    u8  kind;      /* K_* w.r.t. the vector variable */
    u32 off[4];    /* K_LIN: value(v) = value(0) + off[v] (off[0] = 0) */
    u32 dv;        /* a divisor of value(0); 0 means "value(0) is 0" */
    u64 hi;        /* upper bound of the u32 value over every lane and thread */
    u8  gk;        /* G_* w.r.t. the enclosing parallel loop counter */
    u32 gs;        /* G_LIN slope */
    u8  pure;      /* value equals the parallel loop counter */
    i32 depth;     /* loop nesting depth at this op */
    i32 ploop;     /* enclosing parallel (top-level) loop RANGE op, or -1 */
    u32 end;       /* RANGE: index of its ENDRANGE */
    u8  acc_tgt;   /* target of ACC ops inside a parallel loop */
    u32 acc_type;  /* UOP_SUM / UOP_RMAX */
    u8  used_after;/* referenced after its enclosing top-level loop ends */
} OpI;

typedef struct {
    const UOpKernel *k;
    OpI *oi;
    int mode;
    u32 V;
    u32 block;
    u32 total;
    u32 gx;            /* GROUP: workgroups per grid row */
    u32 unroll;        /* GROUP: unroll depth of the parallel loop */
    int nt;            /* streaming (non-temporal) 128-bit loads/stores */
    u32 per_thread;    /* SERIAL: thread-vectors per thread */
    u32 ew_block;      /* SERIAL: workgroup size (0: chosen by size) */
    u32 red_block;     /* GROUP: largest workgroup size */
    u32 split_target;  /* split GROUP: workgroups to aim for (outputs x splits) */
    u32 split_max;     /* split GROUP: most workgroups per output */
    int combine_launch; /* split GROUP: partials to a workspace and a separate combine kernel */
    int combine_mode;   /* THVM_HIP_SPLIT_COMBINE: 0 by the split count, 1 "launch", 2 "single" */
    u32 splits;        /* GROUP: workgroups per output (1: whole loop in one) */
    u32 split_acc;     /* GROUP split: the accumulator op */
    i32 *scal;         /* per op: index into the inline scalar list, or -1 */
    u32 n_scal;
    SB sb;
    char err[256];
} Gen;

static int op_is_float(KOpType t) {
    return t == KOP_CONST_F || t == KOP_LOAD || t == KOP_ALU || t == KOP_ACC_INIT || t == KOP_MASK;
}

static int op_nargs(KOpType t) {
    switch (t) {
    case KOP_MOD: case KOP_DIV: case KOP_LOAD: case KOP_ENDRANGE: return 1;
    case KOP_IDX: case KOP_MASK: case KOP_ACC: case KOP_STORE: case KOP_ALU: return 2;
    default: return 0;
    }
}

static int alu_is_unary(u32 uop) {
    return uop == UOP_NEG || uop == UOP_EXP || uop == UOP_LOG || uop == UOP_RELU ||
           uop == UOP_CAST || uop == UOP_SQRT;
}

static u32 gcd_u32(u32 a, u32 b) {
    while (b) { u32 t = a % b; a = b; b = t; }
    return a;
}
/* divisor facts: 0 stands for "the value is 0" (divisible by anything) */
static u32 dv_gcd(u32 a, u32 b) {
    if (a == 0) return b;
    if (b == 0) return a;
    return gcd_u32(a, b);
}
static u32 dv_mul(u32 a, u32 s) {
    /* a divisor of value*s where a divides value (no wrap: checked by the caller) */
    if (a == 0 || s == 0) return 0;
    u64 r = (u64)a * (u64)s;
    return r > 0xFFFFFFFFull ? (a > s ? a : s) : (u32)r;
}

int kgen_validate(const UOpKernel *k, char *err, size_t errlen) {
    if (!k) { snprintf(err, errlen, "null kernel"); return 0; }
    if (k->n_ops == 0 || k->n_ops > KOP_MAX) { snprintf(err, errlen, "bad n_ops %u", k->n_ops); return 0; }
    if (k->n_leaves > FUSE_MAX_LEAVES) { snprintf(err, errlen, "bad n_leaves %u", k->n_leaves); return 0; }
    if (k->out_dtype >= DTYPE_COUNT) { snprintf(err, errlen, "bad out dtype %u", k->out_dtype); return 0; }
    for (u32 i = 0; i < k->n_leaves; i++)
        if (k->leaf_dtypes[i] >= DTYPE_COUNT) { snprintf(err, errlen, "bad leaf dtype"); return 0; }
    int sp = 0;   /* open RANGEs; ENDRANGE closes the innermost, as the interpreter pairs them */
    for (u32 i = 0; i < k->n_ops; i++) {
        const KOp *op = &k->ops[i];
        if (op->type <= KOP_NOOP || op->type > KOP_MASK) {
            snprintf(err, errlen, "op %u: unsupported type %d", i, (int)op->type);
            return 0;
        }
        int na = op_nargs(op->type);
        for (int a = 0; a < na; a++) {
            if (op->type == KOP_ENDRANGE) break;
            if (op->arg[a] >= i) {
                snprintf(err, errlen, "op %u: arg %d = %u is not an earlier op", i, a, op->arg[a]);
                return 0;
            }
        }
        if (op->type == KOP_ACC && k->ops[op->arg[0]].type != KOP_ACC_INIT) {
            snprintf(err, errlen, "op %u: accumulator %u is not an ACC_INIT op", i, op->arg[0]);
            return 0;
        }
        if (op->type == KOP_RANGE) sp++;
        if (op->type == KOP_ENDRANGE) {
            if (sp == 0) { snprintf(err, errlen, "op %u: ENDRANGE without RANGE", i); return 0; }
            sp--;
        }
    }
    if (sp != 0) { snprintf(err, errlen, "unterminated RANGE"); return 0; }
    return 1;
}

/* Structure: loop ends, depths, enclosing top-level loop. */
static void analyze_structure(Gen *g) {
    const UOpKernel *k = g->k;
    i32 stack[KOP_MAX];
    int sp = 0;
    i32 top = -1;
    for (u32 i = 0; i < k->n_ops; i++) {
        OpI *o = &g->oi[i];
        o->ft = (u8)op_is_float(k->ops[i].type);
        o->ploop = top;
        o->depth = sp;
        if (k->ops[i].type == KOP_RANGE) {
            if (sp == 0) top = (i32)i;
            o->ploop = (sp == 0) ? (i32)i : top;
            stack[sp++] = (i32)i;
        } else if (k->ops[i].type == KOP_ENDRANGE) {
            i32 r = stack[--sp];
            g->oi[r].end = i;
            o->depth = sp;
            o->ploop = top;
            if (sp == 0) top = -1;
        }
    }
    /* references that escape a top-level loop */
    for (u32 i = 0; i < k->n_ops; i++) {
        const KOp *op = &k->ops[i];
        int na = op_nargs(op->type);
        if (op->type == KOP_ENDRANGE) na = 0;
        for (int a = 0; a < na; a++) {
            u32 j = op->arg[a];
            i32 lj = g->oi[j].ploop;
            if (lj >= 0 && g->oi[j].depth > 0 && (u32)lj != (u32)g->oi[i].ploop)
                g->oi[j].used_after = 1;
            if (lj >= 0 && (u32)lj == j && g->oi[i].ploop != lj) g->oi[j].used_after = 1;
        }
    }
}

/* May the top-level loops be split across the lanes of a workgroup? */
static int group_ok(Gen *g, char *why, size_t wlen) {
    const UOpKernel *k = g->k;
    int n_loops = 0;
    for (u32 i = 0; i < k->n_ops; i++) {
        if (k->ops[i].type != KOP_RANGE || g->oi[i].depth != 0) continue;
        n_loops++;
        u32 e = g->oi[i].end;
        if (g->oi[i].used_after) { snprintf(why, wlen, "loop counter used after loop"); return 0; }
        for (u32 j = i + 1; j < e; j++) {
            const KOp *op = &k->ops[j];
            if (op->type == KOP_STORE) { snprintf(why, wlen, "store inside loop"); return 0; }
            if (g->oi[j].used_after && op->type != KOP_ACC_INIT) {
                snprintf(why, wlen, "op %u used after its loop", j);
                return 0;
            }
            if (op->type == KOP_ACC) {
                u32 t = op->arg[0];
                if (k->ops[t].type != KOP_ACC_INIT || t > i || g->oi[t].depth != 0) {
                    snprintf(why, wlen, "accumulator %u not initialised outside the loop", t);
                    return 0;
                }
                u32 ty = op->imm.u == UOP_RMAX ? UOP_RMAX : UOP_SUM;
                if (g->oi[t].acc_tgt && g->oi[t].acc_type != ty) {
                    snprintf(why, wlen, "mixed reductions on one accumulator");
                    return 0;
                }
                g->oi[t].acc_tgt = 1;
                g->oi[t].acc_type = ty;
            }
        }
        /* an accumulator may only be read by its ACC ops inside the loop */
        for (u32 j = i + 1; j < e; j++) {
            const KOp *op = &k->ops[j];
            int na = op_nargs(op->type);
            if (op->type == KOP_ENDRANGE) na = 0;
            for (int a = 0; a < na; a++) {
                u32 t = op->arg[a];
                if (!(op->type == KOP_ACC && a == 0) && g->oi[t].acc_tgt && t < i) {
                    snprintf(why, wlen, "accumulator %u read inside its loop", t);
                    return 0;
                }
            }
        }
    }
    if (n_loops == 0) { snprintf(why, wlen, "no reduce loop"); return 0; }
    return 1;
}

/* At most 64 outputs, and a top-level loop of at least 64 steps.
 * THVM_HIP_TINY_SERIAL=1 keeps such kernels serial (in the CPU's order). */
static int tiny_long_reduce(const Gen *g, u32 total) {
    static int keep = -1;
    if (keep < 0) { const char *e = getenv("THVM_HIP_TINY_SERIAL"); keep = e && e[0] == '1'; }
    if (keep || total == 0 || total > 64) return 0;
    const UOpKernel *k = g->k;
    for (u32 i = 0; i < k->n_ops; i++)
        if (k->ops[i].type == KOP_RANGE && g->oi[i].depth == 0 && k->ops[i].imm.u >= 64) return 1;
    return 0;
}

/* Vector classification. In SERIAL mode the vector variable is the gid; in
 * GROUP mode it is the counter of the enclosing top-level loop, and ops
 * outside top-level loops are uniform. */
static int lin_zero(const u32 *off, u32 V) {
    for (u32 v = 0; v < V; v++) if (off[v]) return 0;
    return 1;
}
static u32 lin_max(const u32 *off, u32 V) {
    u32 m = 0;
    for (u32 v = 0; v < V; v++) if (off[v] > m) m = off[v];
    return m;
}
/* 0,1,2,3 on a lane-0 value divisible by 4: one 128-bit access */
static int lin_unit4(const OpI *o, u32 V) {
    if (V != 4 || o->ft || o->kind != K_LIN || (o->dv != 0 && o->dv % 4 != 0)) return 0;
    for (u32 v = 0; v < 4; v++) if (o->off[v] != v) return 0;
    return 1;
}

/* 0,0,1,1 on an even lane-0 value (an upsample-by-2 broadcast read with 4
 * gids per lane): one 64-bit access serves the four lanes */
static int lin_pair2(const OpI *o, u32 V) {
    if (V != 4 || o->ft || o->kind != K_LIN || (o->dv != 0 && o->dv % 2 != 0)) return 0;
    return o->off[0] == 0 && o->off[1] == 0 && o->off[2] == 1 && o->off[3] == 1;
}

static void analyze_vector(Gen *g) {
    const UOpKernel *k = g->k;
    u32 V = g->V;
    const u64 U32MAX = 0xFFFFFFFFull;
    for (u32 i = 0; i < k->n_ops; i++) {
        const KOp *op = &k->ops[i];
        OpI *o = &g->oi[i];
        o->kind = K_VAR;
        memset(o->off, 0, sizeof o->off);
        o->dv = 1;
        /* value bound over every gid, lane and loop counter */
        switch (op->type) {
        case KOP_GID:
            o->hi = g->mode == KG_MODE_SERIAL ? ((u64)g->total + V - 1) / V * V - 1
                                              : (g->total ? (u64)g->total - 1 : 0);
            break;
        case KOP_CONST_U: o->hi = op->imm.u; break;
        case KOP_RANGE: o->hi = op->imm.u ? (u64)op->imm.u - 1 : 0; break;
        case KOP_DIV: o->hi = op->imm.u ? g->oi[op->arg[0]].hi / op->imm.u : 0; break;
        case KOP_MOD: {
            u64 h = g->oi[op->arg[0]].hi;
            o->hi = op->imm.u ? (h < (u64)op->imm.u - 1 ? h : (u64)op->imm.u - 1) : 0;
            break;
        }
        case KOP_IDX: {
            u64 h = g->oi[op->arg[0]].hi * (u64)op->imm.u + g->oi[op->arg[1]].hi;
            o->hi = h;   /* > U32MAX: may wrap */
            break;
        }
        default: o->hi = U32MAX; break;   /* float valued (f2u when used as an index) */
        }
        int wrap = o->hi > U32MAX;
        if (wrap) o->hi = U32MAX;
        int inscope = (g->mode == KG_MODE_SERIAL) || (o->ploop >= 0 && o->depth > 0) ||
                      op->type == KOP_RANGE;
        if ((g->mode == KG_MODE_GROUP && !inscope) || V == 1) {
            /* uniform across the vector */
            o->kind = K_INV;
            if (op->type == KOP_CONST_U) o->dv = op->imm.u;
            continue;
        }
        switch (op->type) {
        case KOP_GID:
            if (g->mode == KG_MODE_SERIAL) {
                o->kind = K_LIN; o->dv = V;
                for (u32 v = 0; v < V; v++) o->off[v] = v;
            } else o->kind = K_INV;
            break;
        case KOP_CONST_U:
            o->kind = K_INV; o->dv = op->imm.u;
            break;
        case KOP_CONST_F:
            o->kind = K_INV;
            break;
        case KOP_RANGE:
            if (g->mode == KG_MODE_GROUP && o->depth == 0) {
                o->kind = K_LIN; o->dv = V;
                for (u32 v = 0; v < V; v++) o->off[v] = v;
            } else o->kind = K_INV;
            break;
        case KOP_IDX: {
            const OpI *a = &g->oi[op->arg[0]], *b = &g->oi[op->arg[1]];
            if (a->kind == K_VAR || b->kind == K_VAR || ((a->ft || b->ft) && !(a->kind == K_INV && b->kind == K_INV))) {
                o->kind = K_VAR;
                break;
            }
            if (a->kind == K_INV && b->kind == K_INV) {
                o->kind = K_INV;
                o->dv = (wrap || a->ft || b->ft) ? 1 : dv_gcd(dv_mul(a->dv, op->imm.u), b->dv);
                break;
            }
            if (wrap) { o->kind = K_VAR; break; }
            for (u32 v = 0; v < V; v++) o->off[v] = a->off[v] * op->imm.u + b->off[v];
            o->dv = dv_gcd(dv_mul(a->dv, op->imm.u), b->dv);
            o->kind = lin_zero(o->off, V) ? K_INV : K_LIN;
            break;
        }
        case KOP_MOD: case KOP_DIV: {
            const OpI *a = &g->oi[op->arg[0]];
            u32 d = op->imm.u;
            int is_mod = op->type == KOP_MOD;
            if (d == 0) { o->kind = K_INV; o->dv = 0; break; }
            if (a->ft) { o->kind = a->kind == K_INV ? K_INV : K_VAR; break; }
            if (a->kind == K_VAR) break;
            u32 A = a->dv;
            if (A != 0 && A % d != 0 && a->kind == K_LIN && lin_max(a->off, V) >= gcd_u32(A, d)) break;
            /* Here either d divides A (lane values split exactly), or every
             * offset is below G = gcd(A, d): value(0) mod d is a multiple of G
             * and at most d - G, so no lane crosses a multiple of d. */
            if (A == 0 || A % d == 0) {
                for (u32 v = 0; v < V; v++) o->off[v] = is_mod ? a->off[v] % d : a->off[v] / d;
                o->dv = is_mod ? 0 : (A == 0 ? 0 : A / d);
            } else {
                for (u32 v = 0; v < V; v++) o->off[v] = is_mod ? a->off[v] : 0;
                o->dv = is_mod ? gcd_u32(A, d) : 1;
            }
            o->kind = lin_zero(o->off, V) ? K_INV : K_LIN;
            break;
        }
        case KOP_LOAD:
            o->kind = g->oi[op->arg[0]].kind == K_INV ? K_INV : K_VAR;
            break;
        case KOP_MASK:
        case KOP_ALU: {
            const OpI *a = &g->oi[op->arg[0]], *b = &g->oi[op->arg[1]];
            int unary = op->type == KOP_ALU && alu_is_unary(op->imm.u);
            o->kind = (a->kind == K_INV && (unary || b->kind == K_INV)) ? K_INV : K_VAR;
            break;
        }
        case KOP_ACC_INIT:
            o->kind = (g->mode == KG_MODE_GROUP) ? K_INV : K_VAR;
            break;
        default:
            o->kind = K_INV;
            break;
        }
    }
}

/* A SERIAL program whose loop body loads with lane offsets 0, s, 2s, 3s for
 * s >= 2 (a 2x2 stride-2 pooling window read for 4 adjacent outputs): each
 * such load instruction touches s times the cache lines it uses, once per
 * loop step, so one gid per lane is better (measured: the maxpool forward
 * over [64,64,56,56] 16.8 -> 14.9 us, LeNet-5's fc3 input gradient 5.9 ->
 * 3.8 us). THVM_HIP_STRIDED_V4=1 keeps 4 gids per lane. */
static int serial_strided(const Gen *g) {
    static int keep = -1;
    if (keep < 0) { const char *e = getenv("THVM_HIP_STRIDED_V4"); keep = e && e[0] == '1'; }
    if (keep) return 0;
    const UOpKernel *k = g->k;
    for (u32 i = 0; i < k->n_ops; i++) {
        const KOp *op = &k->ops[i];
        if (op->type != KOP_LOAD || g->oi[i].depth == 0 || op->imm.u > k->n_leaves) continue;
        const OpI *ix = &g->oi[op->arg[0]];
        if (ix->ft || ix->kind != K_LIN) continue;
        const u32 st = ix->off[1];
        if (st >= 2 && ix->off[2] == 2 * st && ix->off[3] == 3 * st) return 1;
    }
    return 0;
}

/* Global affine analysis of u32 ops inside GROUP parallel loops, w.r.t. the
 * loop counter over its whole range [0, trip). */
static void analyze_global(Gen *g) {
    const UOpKernel *k = g->k;
    for (u32 i = 0; i < k->n_ops; i++) {
        const KOp *op = &k->ops[i];
        OpI *o = &g->oi[i];
        o->gk = G_NOT; o->gs = 0; o->pure = 0;
        if (g->mode != KG_MODE_GROUP) continue;
        int inloop = o->ploop >= 0 && o->depth > 0;
        if (!inloop) {
            if (op->type == KOP_RANGE && o->depth == 0) { o->gk = G_LIN; o->gs = 1; o->pure = 1; }
            else o->gk = o->ft ? G_NOT : G_INV;
            continue;
        }
        u32 trip = k->ops[o->ploop].imm.u;
        switch (op->type) {
        case KOP_CONST_U: case KOP_GID: o->gk = G_INV; break;
        case KOP_RANGE: o->gk = G_NOT; break;  /* nested loop counter */
        case KOP_IDX: {
            const OpI *a = &g->oi[op->arg[0]], *b = &g->oi[op->arg[1]];
            if (a->gk == G_NOT || b->gk == G_NOT) break;
            u64 s = (u64)a->gs * op->imm.u + b->gs;
            if (s * (u64)(trip ? trip - 1 : 0) >= (1ull << 31)) break;
            o->gs = (u32)s;
            o->gk = s ? G_LIN : G_INV;
            o->pure = (a->pure && op->imm.u == 1 && b->gk == G_INV && k->ops[op->arg[1]].type == KOP_CONST_U &&
                       k->ops[op->arg[1]].imm.u == 0) ||
                      (b->pure && a->gk == G_INV && k->ops[op->arg[0]].type == KOP_CONST_U &&
                       k->ops[op->arg[0]].imm.u == 0);
            break;
        }
        case KOP_MOD: {
            const OpI *a = &g->oi[op->arg[0]];
            if (op->imm.u == 0) { o->gk = G_INV; break; }
            if (a->gk == G_INV) { o->gk = G_INV; break; }
            if (a->pure && op->imm.u >= trip) { o->gk = G_LIN; o->gs = 1; o->pure = 1; }
            break;
        }
        case KOP_DIV: {
            const OpI *a = &g->oi[op->arg[0]];
            if (op->imm.u == 0) { o->gk = G_INV; break; }
            if (a->gk == G_INV) { o->gk = G_INV; break; }
            if (op->imm.u == 1) { o->gk = a->gk; o->gs = a->gs; o->pure = a->pure; break; }
            if (a->pure && op->imm.u >= trip) { o->gk = G_INV; }
            break;
        }
        default: break;
        }
    }
}

/* ---------------- expression accessors ---------------- */
static const char *U(Gen *g, u32 j, u32 v, char *buf);

static const char *Fx(Gen *g, u32 j, u32 v, char *buf) {
    const OpI *o = &g->oi[j];
    if (o->ft) {
        if (o->kind == K_INV || g->V == 1) snprintf(buf, 64, "f%u", j);
        else snprintf(buf, 64, "f%u_%u", j, v);
    } else {
        char t[64];
        snprintf(buf, 96, "((float)%s)", U(g, j, v, t));
    }
    return buf;
}

static const char *U(Gen *g, u32 j, u32 v, char *buf) {
    const OpI *o = &g->oi[j];
    if (o->ft) {
        char t[96];
        snprintf(buf, 128, "f2u(%s)", Fx(g, j, v, t));
        return buf;
    }
    if (o->kind == K_INV || g->V == 1) snprintf(buf, 64, "n%u", j);
    else if (o->kind == K_LIN) {
        if (o->off[v] == 0) snprintf(buf, 64, "n%u", j);
        else snprintf(buf, 64, "(n%u+%uu)", j, o->off[v]);
    } else snprintf(buf, 64, "n%u_%u", j, v);
    return buf;
}

/* Value of u32 op j at loop counter 0 (GROUP range-check prologue). */
static const char *G0(Gen *g, u32 j, i32 loop, char *buf) {
    const OpI *o = &g->oi[j];
    if ((i32)j == loop) snprintf(buf, 64, "0u");
    else if (o->ploop == loop && o->depth > 0) snprintf(buf, 64, "g%u", j);
    else snprintf(buf, 64, "n%u", j);
    return buf;
}

static const char *dt_ld(u32 dt) {
    switch (dt) {
    case DTYPE_F16: return "ld_f16";
    case DTYPE_I32: return "ld_i32";
    case DTYPE_U32: return "ld_u32";
    default: return "ld_f32";
    }
}
static const char *dt_st(u32 dt) {
    switch (dt) {
    case DTYPE_F16: return "st_f16";
    case DTYPE_I32: return "st_i32";
    case DTYPE_U32: return "st_u32";
    default: return "st_f32";
    }
}

static void fmt_float(char *buf, f32 f) {
    u32 bits;
    memcpy(&bits, &f, 4);
    snprintf(buf, 64, "__uint_as_float(0x%08xu)", bits);
}

/* Declare every op variable once, zero-initialised (the CPU interpreter
 * clears its value arrays for each gid). */
static void emit_decls(Gen *g) {
    const UOpKernel *k = g->k;
    for (u32 i = 0; i < k->n_ops; i++) {
        const OpI *o = &g->oi[i];
        KOpType t = k->ops[i].type;
        if (t == KOP_ENDRANGE || t == KOP_STORE || t == KOP_ACC) continue;
        const char *ty = o->ft ? "float" : "u32";
        const char *z = o->ft ? "0.0f" : "0u";
        char pf = o->ft ? 'f' : 'n';
        if (o->kind == K_VAR && g->V > 1) {
            sb_put(&g->sb, "  %s", ty);
            for (u32 v = 0; v < g->V; v++) sb_put(&g->sb, "%s %c%u_%u = %s", v ? "," : "", pf, i, v, z);
            sb_put(&g->sb, ";\n");
        } else {
            sb_put(&g->sb, "  %s %c%u = %s;\n", ty, pf, i, z);
        }
    }
}

/* The engine's ALU (src/backend/cpu/dispatch.c:5-21) on float operands a and
 * b as one HIP expression: guarded DIV, strict-comparison MAX/CMP/RELU. */
int kgen_alu_expr(u32 uop, u32 aux, const char *a, const char *b, char *out, size_t n) {
    switch (uop) {
    case UOP_ADD:  return snprintf(out, n, "%s + %s", a, b);
    case UOP_SUB:  return snprintf(out, n, "%s - %s", a, b);
    case UOP_MUL:  return snprintf(out, n, "%s * %s", a, b);
    case UOP_DIV:  return snprintf(out, n, "(%s != 0.0f) ? (%s / %s) : 0.0f", b, a, b);
    case UOP_MAX:  return snprintf(out, n, "(%s > %s) ? %s : %s", a, b, a, b);
    case UOP_CMP:  return snprintf(out, n, "(%s > %s) ? 1.0f : 0.0f", a, b);
    case UOP_NEG:  return snprintf(out, n, "-%s", a);
    case UOP_RELU: return snprintf(out, n, "(%s > 0.0f) ? %s : 0.0f", a, a);
    case UOP_EXP:  return snprintf(out, n, "expf(%s)", a);
    case UOP_LOG:  return snprintf(out, n, "logf(%s)", a);
    case UOP_SQRT: return snprintf(out, n, "sqrtf(%s)", a);
    case UOP_CAST: return snprintf(out, n, "cast_f(%s, %uu)", a, aux);
    default:       return snprintf(out, n, "%s", a);
    }
}

static void emit_alu(Gen *g, const KOp *op, u32 i, u32 v) {
    char a[128], b[128], d[64], x[512];
    Fx(g, op->arg[0], v, a);
    Fx(g, op->arg[1], v, b);
    const OpI *o = &g->oi[i];
    if (o->kind == K_VAR && g->V > 1) snprintf(d, sizeof d, "f%u_%u", i, v);
    else snprintf(d, sizeof d, "f%u", i);
    kgen_alu_expr(op->imm.u, op->arg[2], a, b, x, sizeof x);
    sb_put(&g->sb, "    %s = %s;\n", d, x);
}

/* Emit one op (all vector lanes). `fast` selects unchecked loads for indices
 * proven in range by the GROUP prologue. `ploop_active`: inside a parallel loop. */
static void emit_op(Gen *g, u32 i, int fast, int in_ploop) {
    const UOpKernel *k = g->k;
    const KOp *op = &k->ops[i];
    const OpI *o = &g->oi[i];
    u32 V = g->V;
    int single = (o->kind != K_VAR) || V == 1;
    char a[128], b[128], fb[64];
    switch (op->type) {
    case KOP_GID:
        if (g->mode == KG_MODE_SERIAL) sb_put(&g->sb, "    n%u = X0;\n", i);
        else sb_put(&g->sb, "    n%u = gid;\n", i);
        break;
    case KOP_CONST_U:
        sb_put(&g->sb, "    n%u = %uu;\n", i, op->imm.u);
        break;
    case KOP_CONST_F:
        fmt_float(fb, op->imm.f);
        sb_put(&g->sb, "    f%u = %s;\n", i, fb);
        break;
    case KOP_MOD: case KOP_DIV: case KOP_IDX: {
        u32 nv = single ? 1 : V;
        for (u32 v = 0; v < nv; v++) {
            char d[32];
            if (single) snprintf(d, sizeof d, "n%u", i);
            else snprintf(d, sizeof d, "n%u_%u", i, v);
            U(g, op->arg[0], v, a);
            if (op->type == KOP_IDX) {
                U(g, op->arg[1], v, b);
                sb_put(&g->sb, "    %s = %s * %uu + %s;\n", d, a, op->imm.u, b);
            } else if (op->imm.u == 0) {
                sb_put(&g->sb, "    %s = 0u;\n", d);
            } else {
                sb_put(&g->sb, "    %s = %s %c %uu;\n", d, a, op->type == KOP_MOD ? '%' : '/', op->imm.u);
            }
        }
        break;
    }
    case KOP_LOAD: {
        u32 bi = op->imm.u;
        if (bi > k->n_leaves) {
            if (single) sb_put(&g->sb, "    f%u = 0.0f;\n", i);
            else for (u32 v = 0; v < V; v++) sb_put(&g->sb, "    f%u_%u = 0.0f;\n", i, v);
            break;
        }
        u32 dt = bi == 0 ? k->out_dtype : k->leaf_dtypes[bi - 1];
        const OpI *ix = &g->oi[op->arg[0]];
        int unchecked = fast && ix->gk != G_NOT && !ix->ft && o->depth == 1;
        if (g->scal && g->scal[i] >= 0) {
            u32 j = (u32)g->scal[i];
            U(g, op->arg[0], 0, a);
            if (single)
                sb_put(&g->sb, "    f%u = ((sm_ >> %uu) & 1u) ? sv%u : %s(p%u, c%u, %s);\n", i, j, j, dt_ld(dt), bi,
                       bi, a);
            else
                for (u32 v = 0; v < V; v++)
                    sb_put(&g->sb, "    f%u_%u = ((sm_ >> %uu) & 1u) ? sv%u : %s(p%u, c%u, %s);\n", i, v, j, j,
                           dt_ld(dt), bi, bi, a);
            break;
        }
        if (single) {
            U(g, op->arg[0], 0, a);
            if (unchecked) sb_put(&g->sb, "    f%u = %s_u(p%u, %s);\n", i, dt_ld(dt), bi, a);
            else sb_put(&g->sb, "    f%u = %s(p%u, c%u, %s);\n", i, dt_ld(dt), bi, bi, a);
        } else if (lin_unit4(ix, V) && dt == DTYPE_F32) {
            U(g, op->arg[0], 0, a);
            const char *sfx = (g->nt & 1) ? "nt" : "";
            if (unchecked)
                sb_put(&g->sb, "    { float4 t_ = ld4%s_u(p%u, %s); f%u_0 = t_.x; f%u_1 = t_.y; f%u_2 = t_.z; f%u_3 = t_.w; }\n",
                       sfx, bi, a, i, i, i, i);
            else
                sb_put(&g->sb, "    { float4 t_ = ld4%s(p%u, c%u, %s); f%u_0 = t_.x; f%u_1 = t_.y; f%u_2 = t_.z; f%u_3 = t_.w; }\n",
                       sfx, bi, bi, a, i, i, i, i);
        } else if (lin_pair2(ix, V) && dt == DTYPE_F32) {
            U(g, op->arg[0], 0, a);
            if (unchecked)
                sb_put(&g->sb, "    { float2 t_ = ld2_u(p%u, %s); f%u_0 = t_.x; f%u_1 = t_.x; f%u_2 = t_.y; f%u_3 = t_.y; }\n",
                       bi, a, i, i, i, i);
            else
                sb_put(&g->sb, "    { float2 t_ = ld2(p%u, c%u, %s); f%u_0 = t_.x; f%u_1 = t_.x; f%u_2 = t_.y; f%u_3 = t_.y; }\n",
                       bi, bi, a, i, i, i, i);
        } else {
            for (u32 v = 0; v < V; v++) {
                u32 u = v;
                if (ix->kind == K_LIN && !ix->ft)
                    for (u = 0; u < v && ix->off[u] != ix->off[v]; u++) {}
                if (u < v) {   /* same address as lane u */
                    sb_put(&g->sb, "    f%u_%u = f%u_%u;\n", i, v, i, u);
                    continue;
                }
                U(g, op->arg[0], v, a);
                if (unchecked) sb_put(&g->sb, "    f%u_%u = %s_u(p%u, %s);\n", i, v, dt_ld(dt), bi, a);
                else sb_put(&g->sb, "    f%u_%u = %s(p%u, c%u, %s);\n", i, v, dt_ld(dt), bi, bi, a);
            }
        }
        break;
    }
    case KOP_MASK: {
        u32 nv = single ? 1 : V;
        for (u32 v = 0; v < nv; v++) {
            Fx(g, op->arg[0], v, a);
            Fx(g, op->arg[1], v, b);
            if (single) sb_put(&g->sb, "    f%u = (%s != 0.0f) ? %s : 0.0f;\n", i, a, b);
            else sb_put(&g->sb, "    f%u_%u = (%s != 0.0f) ? %s : 0.0f;\n", i, v, a, b);
        }
        break;
    }
    case KOP_ALU: {
        u32 nv = single ? 1 : V;
        for (u32 v = 0; v < nv; v++) emit_alu(g, op, i, v);
        break;
    }
    case KOP_ACC_INIT:
        fmt_float(fb, op->imm.f);
        if (single) sb_put(&g->sb, "    f%u = %s;\n", i, fb);
        else for (u32 v = 0; v < V; v++) sb_put(&g->sb, "    f%u_%u = %s;\n", i, v, fb);
        break;
    case KOP_ACC: {
        /* SERIAL: one accumulator per vector lane (per gid). GROUP inside a
         * parallel loop: per-lane partials p<t>_<v>. V == 1: a single one. */
        u32 t = op->arg[0];
        int rmax = op->imm.u == UOP_RMAX;
        int group = in_ploop && g->mode == KG_MODE_GROUP;
        u32 nv = (group || g->oi[t].kind == K_VAR) ? V : 1;
        for (u32 v = 0; v < nv; v++) {
            char d[32];
            if (group) snprintf(d, sizeof d, "p%u_%u", t, v);
            else if (nv > 1) snprintf(d, sizeof d, "f%u_%u", t, v);
            else snprintf(d, sizeof d, "f%u", t);
            Fx(g, op->arg[1], v, a);
            if (rmax) sb_put(&g->sb, "    %s = (%s > %s) ? %s : %s;\n", d, d, a, d, a);
            else sb_put(&g->sb, "    %s = %s + %s;\n", d, d, a);
        }
        break;
    }
    case KOP_STORE: {
        const OpI *ix = &g->oi[op->arg[0]];
        /* buffer imm.u: the engine's programs store to 0 (the output); a
         * chain of fused elementwise programs also stores to leaf slots */
        const u32 sb_ = op->imm.u <= k->n_leaves ? op->imm.u : 0u;
        const u32 sdt = sb_ ? k->leaf_dtypes[sb_ - 1] : k->out_dtype;
        if (g->mode == KG_MODE_GROUP) {
            U(g, op->arg[0], 0, a);
            Fx(g, op->arg[1], 0, b);
            sb_put(&g->sb, "    if (lane == 0) %s(p%u, c%u, %s, %s);\n", dt_st(sdt), sb_, sb_, a, b);
            break;
        }
        if (lin_unit4(ix, V) && sdt == DTYPE_F32) {
            char b1[128], b2[128], b3[128];
            U(g, op->arg[0], 0, a);
            Fx(g, op->arg[1], 0, b);
            Fx(g, op->arg[1], 1, b1);
            Fx(g, op->arg[1], 2, b2);
            Fx(g, op->arg[1], 3, b3);
            sb_put(&g->sb, "    if (X0 + 3u < TOTAL) st4%s(p%u, c%u, %s, make_float4(%s, %s, %s, %s));\n",
                   (g->nt & 2) ? "nt" : "", sb_, sb_, a, b, b1, b2, b3);
            sb_put(&g->sb, "    else {\n");
            for (u32 v = 0; v < V; v++) {
                U(g, op->arg[0], v, a);
                Fx(g, op->arg[1], v, b);
                sb_put(&g->sb, "      if (X0 + %uu < TOTAL) %s(p%u, c%u, %s, %s);\n", v, dt_st(sdt), sb_, sb_, a, b);
            }
            sb_put(&g->sb, "    }\n");
        } else {
            for (u32 v = 0; v < V; v++) {
                U(g, op->arg[0], v, a);
                Fx(g, op->arg[1], v, b);
                sb_put(&g->sb, "    if (X0 + %uu < TOTAL) %s(p%u, c%u, %s, %s);\n", v, dt_st(sdt), sb_, sb_, a, b);
            }
        }
        break;
    }
    default:
        break;
    }
}

/* Emit ops [lo, hi) sequentially; nested RANGEs become sequential loops. */
static void emit_range_seq(Gen *g, u32 lo, u32 hi, int fast, int in_ploop);

static void emit_seq_loop(Gen *g, u32 r, int fast, int in_ploop) {
    const KOp *op = &g->k->ops[r];
    u32 e = g->oi[r].end;
    sb_put(&g->sb, "    for (u32 r%u = 0u; r%u < %uu; r%u++) {\n    n%u = r%u;\n", r, r, op->imm.u, r, r, r);
    emit_range_seq(g, r + 1, e, fast, in_ploop);
    sb_put(&g->sb, "    }\n");
}

static void emit_range_seq(Gen *g, u32 lo, u32 hi, int fast, int in_ploop) {
    for (u32 i = lo; i < hi; i++) {
        const KOp *op = &g->k->ops[i];
        if (op->type == KOP_RANGE) {
            emit_seq_loop(g, i, fast, in_ploop);
            i = g->oi[i].end;
            continue;
        }
        if (op->type == KOP_ENDRANGE) continue;
        emit_op(g, i, fast, in_ploop);
    }
}

static const char *PRELUDE_BODY =
"#ifndef THVM_COMB_SPIN\n#define THVM_COMB_SPIN (1u << 22)\n#endif\n"
"#ifndef THVM_COMB_WITHHOLD\n#define THVM_COMB_WITHHOLD 0\n#endif\n"
"typedef unsigned int u32;\n"
"typedef unsigned short u16;\n"
"/* f16 decode (exact) */\n"
"__device__ __forceinline__ float h2f(u32 h) {\n"
"  u32 sign = (h & 0x8000u) << 16, ex = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;\n"
"  if (ex == 0u) {\n"
"    if (man == 0u) bits = sign;\n"
"    else { ex = 1u; while ((man & 0x400u) == 0u) { man <<= 1; ex -= 1u; } man &= 0x3FFu;\n"
"           bits = sign | ((ex + 112u) << 23) | (man << 13); }\n"
"  } else if (ex == 0x1Fu) bits = sign | 0x7F800000u | (man << 13);\n"
"  else bits = sign | ((ex + 112u) << 23) | (man << 13);\n"
"  return __uint_as_float(bits);\n"
"}\n"
"/* f16 encode: round half up on the first dropped bit (engine rule) */\n"
"__device__ __forceinline__ u32 f2h(float f) {\n"
"  u32 x = __float_as_uint(f), sign = (x >> 16) & 0x8000u, man = x & 0x7FFFFFu;\n"
"  int ex = (int)((x >> 23) & 0xFFu) - 112;\n"
"  if (ex <= 0) { if (ex < -10) return sign; man = (man | 0x800000u) >> (1 - ex);\n"
"                 if (man & 0x1000u) man += 0x2000u; return sign | (man >> 13); }\n"
"  if (ex >= 31) return sign | 0x7C00u | (man ? 0x200u : 0u);\n"
"  if (man & 0x1000u) { man += 0x2000u; if (man & 0x800000u) { man = 0u; ex += 1; if (ex >= 31) return sign | 0x7C00u; } }\n"
"  return sign | ((u32)ex << 10) | (man >> 13);\n"
"}\n"
"/* x86-64 conversions: (u32)f goes through a 64-bit truncation; (i32)f gives INT_MIN out of range */\n"
"__device__ __forceinline__ u32 f2u(float f) {\n"
"  if (!(fabsf(f) < 9.2233720368547758e18f)) return 0u;\n"
"  return (u32)(unsigned long long)(long long)f;\n"
"}\n"
"__device__ __forceinline__ int f2i(float f) {\n"
"  if (!(f >= -2147483648.0f && f < 2147483648.0f)) return (int)0x80000000u;\n"
"  return (int)f;\n"
"}\n"
"__device__ __forceinline__ float cast_f(float v, u32 dt) {\n"
"  if (dt == 1u) return h2f(f2h(v));\n"
"  if (dt == 2u) return (float)f2i(v);\n"
"  if (dt == 3u) return (float)f2u(v);\n"
"  return v;\n"
"}\n"
"/* checked loads without branches: an out-of-range index loads element 0\n"
" * instead and the value is replaced by 0 (every pointer argument points at\n"
" * least 4 valid bytes, also for empty or absent buffers) */\n"
"__device__ __forceinline__ float ld_f32(const char* p, u32 n, u32 i) {\n"
"  const float v = ((const float*)p)[i < n ? i : 0u]; return i < n ? v : 0.0f;\n"
"}\n"
"__device__ __forceinline__ float ld_f16(const char* p, u32 n, u32 i) {\n"
"  const float v = h2f(((const u16*)p)[i < n ? i : 0u]); return i < n ? v : 0.0f;\n"
"}\n"
"__device__ __forceinline__ float ld_i32(const char* p, u32 n, u32 i) {\n"
"  const float v = (float)((const int*)p)[i < n ? i : 0u]; return i < n ? v : 0.0f;\n"
"}\n"
"__device__ __forceinline__ float ld_u32(const char* p, u32 n, u32 i) {\n"
"  const float v = (float)((const u32*)p)[i < n ? i : 0u]; return i < n ? v : 0.0f;\n"
"}\n"
"__device__ __forceinline__ float ld_f32_u(const char* p, u32 i) { return ((const float*)p)[i]; }\n"
"__device__ __forceinline__ float ld_f16_u(const char* p, u32 i) { return h2f(((const u16*)p)[i]); }\n"
"__device__ __forceinline__ float ld_i32_u(const char* p, u32 i) { return (float)((const int*)p)[i]; }\n"
"__device__ __forceinline__ float ld_u32_u(const char* p, u32 i) { return (float)((const u32*)p)[i]; }\n"
"__device__ __forceinline__ float4 ld4_u(const char* p, u32 i) { return *(const float4*)((const float*)p + i); }\n"
"__device__ __forceinline__ float2 ld2_u(const char* p, u32 i) { return *(const float2*)((const float*)p + i); }\n"
"__device__ __forceinline__ float2 ld2(const char* p, u32 n, u32 i) {\n"
"  if (i + 1u < n && i + 1u >= i) return *(const float2*)((const float*)p + i);\n"
"  return make_float2(ld_f32(p, n, i), ld_f32(p, n, i + 1u));\n"
"}\n"
"__device__ __forceinline__ float4 ld4(const char* p, u32 n, u32 i) {\n"
"  if (i + 3u < n && i + 3u >= i) return *(const float4*)((const float*)p + i);\n"
"  return make_float4(ld_f32(p, n, i), ld_f32(p, n, i + 1u), ld_f32(p, n, i + 2u), ld_f32(p, n, i + 3u));\n"
"}\n"
"typedef float v4f_ __attribute__((ext_vector_type(4)));\n"
"__device__ __forceinline__ float4 ld4nt_u(const char* p, u32 i) {\n"
"  v4f_ t = __builtin_nontemporal_load((const v4f_*)((const float*)p + i)); return make_float4(t.x, t.y, t.z, t.w);\n"
"}\n"
"__device__ __forceinline__ float4 ld4nt(const char* p, u32 n, u32 i) {\n"
"  if (i + 3u < n && i + 3u >= i) return ld4nt_u(p, i);\n"
"  return make_float4(ld_f32(p, n, i), ld_f32(p, n, i + 1u), ld_f32(p, n, i + 2u), ld_f32(p, n, i + 3u));\n"
"}\n"
"__device__ __forceinline__ void st_f32(char* p, u32 n, u32 i, float v) { if (i < n) ((float*)p)[i] = v; }\n"
"__device__ __forceinline__ void st_f16(char* p, u32 n, u32 i, float v) { if (i < n) ((u16*)p)[i] = (u16)f2h(v); }\n"
"__device__ __forceinline__ void st_i32(char* p, u32 n, u32 i, float v) { if (i < n) ((int*)p)[i] = f2i(v); }\n"
"__device__ __forceinline__ void st_u32(char* p, u32 n, u32 i, float v) { if (i < n) ((u32*)p)[i] = f2u(v); }\n"
"__device__ __forceinline__ void st4(char* p, u32 n, u32 i, float4 v) {\n"
"  if (i + 3u < n && i + 3u >= i) { *(float4*)((float*)p + i) = v; return; }\n"
"  st_f32(p, n, i, v.x); st_f32(p, n, i + 1u, v.y); st_f32(p, n, i + 2u, v.z); st_f32(p, n, i + 3u, v.w);\n"
"}\n"
"__device__ __forceinline__ void st4nt(char* p, u32 n, u32 i, float4 v) {\n"
"  if (i + 3u < n && i + 3u >= i) { v4f_ t = {v.x, v.y, v.z, v.w}; __builtin_nontemporal_store(t, (v4f_*)((float*)p + i)); return; }\n"
"  st_f32(p, n, i, v.x); st_f32(p, n, i + 1u, v.y); st_f32(p, n, i + 2u, v.z); st_f32(p, n, i + 3u, v.w);\n"
"}\n"
"__device__ __forceinline__ float wsum(float x) {\n"
"  for (int o = 32; o > 0; o >>= 1) x = x + __shfl_xor(x, o, 64);\n"
"  return x;\n"
"}\n"
"__device__ __forceinline__ float wmax(float x) {\n"
"  for (int o = 32; o > 0; o >>= 1) { float y = __shfl_xor(x, o, 64); x = (x > y) ? x : y; }\n"
"  return x;\n"
"}\n"
/* a single-wave workgroup's total, lane 0's value in every lane (the same
 * bits a block-wide helper returns, without LDS or barriers) */
"__device__ __forceinline__ float wsum0(float x) { return __shfl(wsum(x), 0, 64); }\n"
"__device__ __forceinline__ float wmax0(float x) { return __shfl(wmax(x), 0, 64); }\n"
"__device__ __forceinline__ float bsum(float x, float* red) {\n"
"  x = wsum(x);\n"
"  __syncthreads();\n"
"  if ((threadIdx.x & 63u) == 0u) red[threadIdx.x >> 6] = x;\n"
"  __syncthreads();\n"
"  float s = red[0];\n"
"  for (u32 w = 1u; w < (blockDim.x >> 6); w++) s = s + red[w];\n"
"  return s;\n"
"}\n"
"__device__ __forceinline__ float bmax(float x, float* red) {\n"
"  x = wmax(x);\n"
"  __syncthreads();\n"
"  if ((threadIdx.x & 63u) == 0u) red[threadIdx.x >> 6] = x;\n"
"  __syncthreads();\n"
"  float s = red[0];\n"
"  for (u32 w = 1u; w < (blockDim.x >> 6); w++) { float y = red[w]; s = (s > y) ? s : y; }\n"
"  return s;\n"
"}\n"
/* The same with the workgroup's wave count fixed (a batched launch's
 * workgroups can be larger than the program's) */
"template <u32 NW> __device__ __forceinline__ float bsum_n(float x, float* red) {\n"
"  x = wsum(x);\n"
"  __syncthreads();\n"
"  if ((threadIdx.x & 63u) == 0u) red[threadIdx.x >> 6] = x;\n"
"  __syncthreads();\n"
"  float s = red[0];\n"
"  for (u32 w = 1u; w < NW; w++) s = s + red[w];\n"
"  return s;\n"
"}\n"
"template <u32 NW> __device__ __forceinline__ float bmax_n(float x, float* red) {\n"
"  x = wmax(x);\n"
"  __syncthreads();\n"
"  if ((threadIdx.x & 63u) == 0u) red[threadIdx.x >> 6] = x;\n"
"  __syncthreads();\n"
"  float s = red[0];\n"
"  for (u32 w = 1u; w < NW; w++) { float y = red[w]; s = (s > y) ? s : y; }\n"
"  return s;\n"
"}\n"
/* Where a single-pass combine reports that it gave up waiting for a
 * partial: a word of host-visible memory whose device address the host
 * writes into every module it loads (NULL: not reported). */
"extern \"C\" { __device__ unsigned int* thvm_comb_err_ = nullptr; }\n"
"__device__ __forceinline__ void comb_gave_up() {\n"
"  unsigned int* e = thvm_comb_err_;\n"
"  if (e) __hip_atomic_store(e, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);\n"
"}\n"
/* Single-pass combine of per-workgroup partials. Each of the S workgroups
 * of output o but the last publishes its partial as one 64-bit word (a ready
 * flag in the high half, the float's bits in the low half) with an
 * agent-scope atomic store. The workgroup with split index S-1 takes the
 * words in index order, its lanes each waiting (bounded) until their word is
 * marked ready, clears them for the next launch, and combines them with its
 * own partial in a fixed order. Flag and value share one word, so no fence
 * is needed, no cache is written back and no word is contended; the result
 * does not depend on timing. The host uses it only for grids that fit on
 * the GPU at once (every workgroup resident together), so the waiting
 * workgroup never holds back one it waits for. A wait that runs out
 * (THVM_COMB_SPIN polls) takes a NaN for the partial and reports it through
 * comb_gave_up. THVM_COMB_WITHHOLD (a test knob) keeps the partial of
 * split 0 of output 0 unpublished, so that its wait runs out. */
"__device__ __forceinline__ void comb_put(unsigned long long* sl, u32 o, u32 sp, u32 S, float part) {\n"
"  if (THVM_COMB_WITHHOLD && o == 0u && sp == 0u) return;\n"
"  if (threadIdx.x == 0u)\n"
"    __hip_atomic_store(sl + (unsigned long long)o * S + sp, (1ull << 32) | (unsigned long long)__float_as_uint(part),\n"
"                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n"
"}\n"
"__device__ __forceinline__ float comb_take(unsigned long long* sl, u32 o, u32 s, u32 S) {\n"
"  unsigned long long* w = sl + (unsigned long long)o * S + s;\n"
"  unsigned long long v = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n"
"  for (u32 n = 0u; (v >> 32) == 0ull && n < THVM_COMB_SPIN; n++) {\n"
"    __builtin_amdgcn_s_sleep(2);\n"
"    v = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n"
"  }\n"
"  __hip_atomic_store(w, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n"
"  if ((v >> 32) == 0ull) comb_gave_up();\n"
"  return (v >> 32) ? __uint_as_float((u32)v) : __uint_as_float(0x7fc00000u);\n"
"}\n"
/* The same words for a block of partials: comb_pub publishes one,
 * comb_peek reads one without waiting (a batch of them issued together),
 * comb_ready waits (bounded) for a peeked word to be marked ready and
 * returns its float (a NaN if it never became ready), comb_clear clears it
 * for the next launch (the clears of a batch issued after all its waits, so
 * that no wait is for a clear). */
"__device__ __forceinline__ void comb_pub(unsigned long long* w, float x) {\n"
"  __hip_atomic_store(w, (1ull << 32) | (unsigned long long)__float_as_uint(x), __ATOMIC_RELAXED,\n"
"                     __HIP_MEMORY_SCOPE_AGENT);\n"
"}\n"
"__device__ __forceinline__ unsigned long long comb_peek(unsigned long long* w) {\n"
"  return __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n"
"}\n"
"__device__ __forceinline__ float comb_ready(unsigned long long* w, unsigned long long v) {\n"
"  for (u32 n = 0u; (v >> 32) == 0ull && n < THVM_COMB_SPIN; n++) {\n"
"    __builtin_amdgcn_s_sleep(2);\n"
"    v = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n"
"  }\n"
"  if ((v >> 32) == 0ull) comb_gave_up();\n"
"  return (v >> 32) ? __uint_as_float((u32)v) : __uint_as_float(0x7fc00000u);\n"
"}\n"
"__device__ __forceinline__ void comb_clear(unsigned long long* w) {\n"
"  __hip_atomic_store(w, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);\n"
"}\n";

/* The prelude with the combine's wait bound and test knob
 * (THVM_HIP_COMB_SPIN, THVM_HIP_COMB_WITHHOLD), read when it is first built
 * after each kgen_prelude_reset (backend init). */
static char *prelude_buf;

void kgen_prelude_reset(void) {
    free(prelude_buf);
    prelude_buf = NULL;
}

const char *kgen_prelude(void) {
    if (prelude_buf) return prelude_buf;
    const char *e = getenv("THVM_HIP_COMB_SPIN");
    unsigned long spin = e ? strtoul(e, NULL, 10) : 0;
    if (spin == 0 || spin > (1ul << 24)) spin = 1ul << 22;
    const char *w = getenv("THVM_HIP_COMB_WITHHOLD");
    const int withhold = w && w[0] && strcmp(w, "0") != 0;
    const size_t cap = strlen(PRELUDE_BODY) + 128;
    char *b = malloc(cap);
    if (!b) return PRELUDE_BODY;   /* the knobs' defaults are in the body too */
    snprintf(b, cap, "#define THVM_COMB_SPIN %luu\n#define THVM_COMB_WITHHOLD %d\n%s", spin, withhold, PRELUDE_BODY);
    prelude_buf = b;
    return prelude_buf;
}

/* Scalar straight-line code for the ops flagged in `cone` (in op order), as
 * the body of a device function: GID reads `gid_expr`, the top-level RANGE
 * reads `r_expr`. Buffers are the kernel parameters p<i>/c<i>. Returns the
 * number of bytes written, or -1 if an op cannot be emitted this way. */
static int emit_cone_subst(const UOpKernel *k, const u8 *cone, const char *gid_expr, const char *r_expr,
                           u32 subst_leaf, const char *subst_expr, const i32 *scal, char *out, size_t outlen);

int kgen_emit_cone(const UOpKernel *k, const u8 *cone, const char *gid_expr, const char *r_expr,
                   char *out, size_t outlen) {
    return emit_cone_subst(k, cone, gid_expr, r_expr, ~0u, NULL, NULL, out, outlen);
}

/* kgen_emit_cone, with every LOAD of leaf buffer subst_leaf (1 + leaf)
 * reading subst_expr instead, and each LOAD i with scal[i] >= 0 taking
 * argument sv<scal[i]> when bit scal[i] of sm_ is set (an inline scalar) */
static int emit_cone_subst(const UOpKernel *k, const u8 *cone, const char *gid_expr, const char *r_expr,
                           u32 subst_leaf, const char *subst_expr, const i32 *scal, char *out, size_t outlen) {
    SB sb = {0};
    char a[96], b[96], fb[64];
    for (u32 i = 0; i < k->n_ops; i++) {
        if (!cone[i]) continue;
        const KOp *op = &k->ops[i];
        /* operand types; the args of ops without operands may hold anything */
        int fa = op->arg[0] < k->n_ops && op_is_float(k->ops[op->arg[0]].type);
        int fbt = op->arg[1] < k->n_ops && op_is_float(k->ops[op->arg[1]].type);
#define UA(x, ft) ((ft) ? (snprintf(a, sizeof a, "f2u(f%u)", (x)), a) : (snprintf(a, sizeof a, "n%u", (x)), a))
        switch (op->type) {
        case KOP_GID: sb_put(&sb, "  const u32 n%u = %s;\n", i, gid_expr); break;
        case KOP_RANGE: sb_put(&sb, "  const u32 n%u = %s;\n", i, r_expr); break;
        case KOP_CONST_U: sb_put(&sb, "  const u32 n%u = %uu;\n", i, op->imm.u); break;
        case KOP_CONST_F: fmt_float(fb, op->imm.f); sb_put(&sb, "  const float f%u = %s;\n", i, fb); break;
        case KOP_MOD: case KOP_DIV:
            if (op->imm.u == 0) sb_put(&sb, "  const u32 n%u = 0u;\n", i);
            else sb_put(&sb, "  const u32 n%u = %s %c %uu;\n", i, UA(op->arg[0], fa),
                        op->type == KOP_MOD ? '%' : '/', op->imm.u);
            break;
        case KOP_IDX: {
            char t[96];
            snprintf(t, sizeof t, "%s", UA(op->arg[0], fa));
            if (fbt) snprintf(b, sizeof b, "f2u(f%u)", op->arg[1]);
            else snprintf(b, sizeof b, "n%u", op->arg[1]);
            sb_put(&sb, "  const u32 n%u = %s * %uu + %s;\n", i, t, op->imm.u, b);
            break;
        }
        case KOP_LOAD: {
            u32 bi = op->imm.u;
            if (bi == subst_leaf) { sb_put(&sb, "  const float f%u = %s;\n", i, subst_expr); break; }
            if (bi > k->n_leaves) { sb_put(&sb, "  const float f%u = 0.0f;\n", i); break; }
            u32 dt = bi == 0 ? k->out_dtype : k->leaf_dtypes[bi - 1];
            if (scal && scal[i] >= 0)
                sb_put(&sb, "  const float f%u = ((sm_ >> %uu) & 1u) ? sv%d : %s(p%u, c%u, %s);\n", i, (u32)scal[i],
                       scal[i], dt_ld(dt), bi, bi, UA(op->arg[0], fa));
            else
                sb_put(&sb, "  const float f%u = %s(p%u, c%u, %s);\n", i, dt_ld(dt), bi, bi, UA(op->arg[0], fa));
            break;
        }
        case KOP_MASK: {
            char x[96], y[96];
            if (fa) snprintf(x, sizeof x, "f%u", op->arg[0]); else snprintf(x, sizeof x, "(float)n%u", op->arg[0]);
            if (fbt) snprintf(y, sizeof y, "f%u", op->arg[1]); else snprintf(y, sizeof y, "(float)n%u", op->arg[1]);
            sb_put(&sb, "  const float f%u = (%s != 0.0f) ? %s : 0.0f;\n", i, x, y);
            break;
        }
        case KOP_ALU: {
            char x[96], y[96];
            if (fa) snprintf(x, sizeof x, "f%u", op->arg[0]); else snprintf(x, sizeof x, "((float)n%u)", op->arg[0]);
            if (fbt) snprintf(y, sizeof y, "f%u", op->arg[1]); else snprintf(y, sizeof y, "((float)n%u)", op->arg[1]);
            switch (op->imm.u) {
            case UOP_ADD: sb_put(&sb, "  const float f%u = %s + %s;\n", i, x, y); break;
            case UOP_SUB: sb_put(&sb, "  const float f%u = %s - %s;\n", i, x, y); break;
            case UOP_MUL: sb_put(&sb, "  const float f%u = %s * %s;\n", i, x, y); break;
            case UOP_DIV: sb_put(&sb, "  const float f%u = (%s != 0.0f) ? (%s / %s) : 0.0f;\n", i, y, x, y); break;
            case UOP_MAX: sb_put(&sb, "  const float f%u = (%s > %s) ? %s : %s;\n", i, x, y, x, y); break;
            case UOP_CMP: sb_put(&sb, "  const float f%u = (%s > %s) ? 1.0f : 0.0f;\n", i, x, y); break;
            case UOP_NEG: sb_put(&sb, "  const float f%u = -%s;\n", i, x); break;
            case UOP_RELU: sb_put(&sb, "  const float f%u = (%s > 0.0f) ? %s : 0.0f;\n", i, x, x); break;
            case UOP_EXP: sb_put(&sb, "  const float f%u = expf(%s);\n", i, x); break;
            case UOP_LOG: sb_put(&sb, "  const float f%u = logf(%s);\n", i, x); break;
            case UOP_SQRT: sb_put(&sb, "  const float f%u = sqrtf(%s);\n", i, x); break;
            case UOP_CAST: sb_put(&sb, "  const float f%u = cast_f(%s, %uu);\n", i, x, op->arg[2]); break;
            default: sb_put(&sb, "  const float f%u = %s;\n", i, x); break;
            }
            break;
        }
        default:
            free(sb.p);
            return -1;
        }
#undef UA
    }
    if (!sb.p) {
        if (outlen) out[0] = 0;
        return 0;
    }
    size_t n = strlen(sb.p);
    if (n + 1 > outlen) { free(sb.p); return -1; }
    memcpy(out, sb.p, n + 1);
    free(sb.p);
    return (int)n;
}

/* inline scalars of an elementwise program: its loads at a constant index
 * of a leaf other than skip_leaf (1 + leaf; ~0u: none) */
static void find_scalars(const UOpKernel *k, u32 skip_leaf, i32 *scal, KGenScalars *sc) {
    sc->n = 0;
    for (u32 i = 0; i < k->n_ops; i++) {
        const KOp *op = &k->ops[i];
        scal[i] = -1;
        if (op->type == KOP_LOAD && op->imm.u >= 1 && op->imm.u <= k->n_leaves && op->imm.u != skip_leaf &&
            op->arg[0] < k->n_ops && k->ops[op->arg[0]].type == KOP_CONST_U && sc->n < KGEN_MAX_SCALARS) {
            sc->leaf[sc->n] = op->imm.u - 1;
            sc->index[sc->n] = k->ops[op->arg[0]].imm.u;
            scal[i] = (i32)sc->n++;
        }
    }
}

static void put_buffer_params(SB *sb, const UOpKernel *k, const KGenScalars *sc) {
    for (u32 b = 0; b <= k->n_leaves; b++) sb_put(sb, ", char* p%u", b);
    for (u32 b = 0; b <= k->n_leaves; b++) sb_put(sb, ", u32 c%u", b);
    if (sc->n) {
        sb_put(sb, ", u32 sm_");
        for (u32 j = 0; j < sc->n; j++) sb_put(sb, ", float sv%u", j);
    }
}

static int sb_out(SB *sb, char *out, size_t outlen) {
    if (!sb->p) return -1;
    const size_t n = strlen(sb->p);
    if (n + 1 > outlen) { free(sb->p); return -1; }
    memcpy(out, sb->p, n + 1);
    free(sb->p);
    return (int)n;
}

/* An elementwise program as the epilogue of the kernel that produces one of
 * its leaves: a device function fname(gid_, v_, p0.., c0..) that computes
 * the program for output gid_ with every load of leaf buffer o_leaf (1 +
 * leaf) taking v_ (the value the producer just stored there, at gid_),
 * stores the result as the program's STORE does and returns the value it
 * stored (before the conversion of a non-f32 output). The program has no loop
 * and one STORE; the caller checks that its loads of o_leaf and its STORE
 * index are gid itself. Buffers are the function's own p<b>/c<b> (0: its
 * output). Returns the length written, or -1. */
int kgen_epilogue_fn(const UOpKernel *k, u32 o_leaf, const char *fname, char *out, size_t outlen,
                     KGenScalars *sc) {
    u8 cone[KOP_MAX];
    i32 st = -1, scal[KOP_MAX];
    if (k->n_ops == 0 || k->n_ops > KOP_MAX) return -1;
    find_scalars(k, o_leaf, scal, sc);
    for (u32 i = 0; i < k->n_ops; i++) {
        const KOpType t = k->ops[i].type;
        if (t == KOP_RANGE || t == KOP_ENDRANGE || t == KOP_ACC_INIT || t == KOP_ACC) return -1;
        if (t == KOP_STORE) {
            if (st >= 0) return -1;
            st = (i32)i;
        }
        cone[i] = t != KOP_STORE;
    }
    if (st < 0) return -1;
    const KOp *so = &k->ops[st];
    if (so->arg[0] >= k->n_ops || so->arg[1] >= k->n_ops) return -1;
    char body[32768];
    if (emit_cone_subst(k, cone, "gid_", "0u", o_leaf, "v_", scal, body, sizeof body) < 0) return -1;
    SB sb = {0};
    sb_put(&sb, "__device__ __forceinline__ float %s(u32 gid_, float v_", fname);
    put_buffer_params(&sb, k, sc);
    const int fv = op_is_float(k->ops[so->arg[1]].type);
    char v[48];
    if (fv) snprintf(v, sizeof v, "f%u", so->arg[1]);
    else snprintf(v, sizeof v, "(float)n%u", so->arg[1]);
    sb_put(&sb, ") {\n%s  %s(p0, c0, n%u, %s);\n  return %s;\n}\n", body, dt_st(k->out_dtype), so->arg[0], v, v);
    return sb_out(&sb, out, outlen);
}

int kgen_epilogue(const UOpKernel *k, u32 o_leaf, char *out, size_t outlen, KGenScalars *sc) {
    return kgen_epilogue_fn(k, o_leaf, "epi_", out, outlen, sc);
}

/* A loop-free elementwise program inlined where its output is read: a
 * device function fname(gid_, st_, r0_.., p0.., c0..) that computes the
 * program for gid_, stores each of its STOREs there when st_ is set, and
 * returns the value of STORE j in *r<j>_ (STOREs in program order). Its
 * STOREs must all be at gid and it must not load a buffer it stores (the
 * caller checks both). Returns the length written, or -1. */
int kgen_producer_fn(const UOpKernel *k, const char *fname, char *out, size_t outlen, KGenScalars *sc) {
    u8 cone[KOP_MAX];
    i32 scal[KOP_MAX];
    u32 st[CHAIN_MAX_STORES], nst = 0;
    if (k->n_ops == 0 || k->n_ops > KOP_MAX) return -1;
    find_scalars(k, ~0u, scal, sc);
    for (u32 i = 0; i < k->n_ops; i++) {
        const KOp *op = &k->ops[i];
        if (op->type == KOP_RANGE || op->type == KOP_ENDRANGE || op->type == KOP_ACC_INIT || op->type == KOP_ACC)
            return -1;
        if (op->type == KOP_STORE) {
            if (nst >= CHAIN_MAX_STORES || op->arg[0] >= k->n_ops || op->arg[1] >= k->n_ops ||
                op->imm.u > k->n_leaves)
                return -1;
            st[nst++] = i;
        }
        cone[i] = op->type != KOP_STORE;
    }
    if (!nst) return -1;
    char body[32768];
    if (emit_cone_subst(k, cone, "gid_", "0u", ~0u, NULL, scal, body, sizeof body) < 0) return -1;
    SB sb = {0};
    sb_put(&sb, "__device__ __forceinline__ void %s(u32 gid_, bool st_", fname);
    for (u32 j = 0; j < nst; j++) sb_put(&sb, ", float* r%u_", j);
    put_buffer_params(&sb, k, sc);
    sb_put(&sb, ") {\n%s  if (st_) {\n", body);
    for (u32 j = 0; j < nst; j++) {
        const KOp *so = &k->ops[st[j]];
        const u32 slot = so->imm.u, dt = slot ? k->leaf_dtypes[slot - 1] : k->out_dtype;
        char v[48];
        if (op_is_float(k->ops[so->arg[1]].type)) snprintf(v, sizeof v, "f%u", so->arg[1]);
        else snprintf(v, sizeof v, "(float)n%u", so->arg[1]);
        sb_put(&sb, "    %s(p%u, c%u, n%u, %s);\n", dt_st(dt), slot, slot, so->arg[0], v);
    }
    sb_put(&sb, "  }\n");
    for (u32 j = 0; j < nst; j++) {
        const KOp *so = &k->ops[st[j]];
        if (op_is_float(k->ops[so->arg[1]].type)) sb_put(&sb, "  *r%u_ = f%u;\n", j, so->arg[1]);
        else sb_put(&sb, "  *r%u_ = (float)n%u;\n", j, so->arg[1]);
    }
    sb_put(&sb, "}\n");
    return sb_out(&sb, out, outlen);
}

static void plan_inline_scalars(Gen *g, KGenResult *out);

/* kgen_producer_fn for four consecutive gids X0..X0+3 (X0 a multiple of 4,
 * at most `total` gids): the serial generator's vector form of the program,
 * so that loads along gid are 16-byte loads and values the four share are
 * computed once. fname(X0, st_, r0_.., p0.., c0..) stores the STOREs when st_
 * is set and returns STORE j's four values in *r<j>_ (a float4). */
int kgen_producer4_fn(const UOpKernel *k, u32 total, const char *fname, char *out, size_t outlen,
                      KGenScalars *sc) {
    u32 st[CHAIN_MAX_STORES], nst = 0;
    char err[128];
    if (k->n_ops == 0 || k->n_ops > KOP_MAX || total == 0 || !kgen_validate(k, err, sizeof err)) return -1;
    for (u32 i = 0; i < k->n_ops; i++) {
        const KOp *op = &k->ops[i];
        if (op->type == KOP_RANGE || op->type == KOP_ENDRANGE || op->type == KOP_ACC_INIT || op->type == KOP_ACC)
            return -1;
        if (op->type == KOP_STORE) {
            if (nst >= CHAIN_MAX_STORES || op->arg[0] >= k->n_ops || op->arg[1] >= k->n_ops ||
                op->imm.u > k->n_leaves)
                return -1;
            st[nst++] = i;
        }
    }
    if (!nst) return -1;
    Gen G;
    memset(&G, 0, sizeof G);
    G.k = k;
    G.mode = KG_MODE_SERIAL;
    G.V = 4;
    G.total = total;
    G.block = 256;
    G.nt = 3;
    G.oi = calloc(k->n_ops, sizeof(OpI));
    G.scal = malloc(k->n_ops * sizeof(i32));
    KGenResult kr;
    memset(&kr, 0, sizeof kr);
    if (!G.oi || !G.scal) {
        free(G.oi);
        free(G.scal);
        return -1;
    }
    analyze_structure(&G);
    plan_inline_scalars(&G, &kr);
    analyze_vector(&G);
    analyze_global(&G);
    sc->n = kr.n_scal;
    for (u32 j = 0; j < kr.n_scal; j++) {
        sc->leaf[j] = kr.scal_leaf[j];
        sc->index[j] = kr.scal_index[j];
    }
    SB *s = &G.sb;
    sb_put(s, "__device__ __forceinline__ void %s(u32 X0, bool st_", fname);
    for (u32 j = 0; j < nst; j++) sb_put(s, ", float4* r%u_", j);
    put_buffer_params(s, k, sc);
    sb_put(s, ") {\n  const u32 TOTAL = %uu;\n", total);
    emit_decls(&G);
    for (u32 i = 0; i < k->n_ops; i++)
        if (k->ops[i].type != KOP_STORE) emit_op(&G, i, 0, 0);
    sb_put(s, "  if (st_) {\n");
    for (u32 j = 0; j < nst; j++) emit_op(&G, st[j], 0, 0);
    sb_put(s, "  }\n");
    for (u32 j = 0; j < nst; j++) {
        const u32 val = k->ops[st[j]].arg[1];
        char a[4][128];
        for (u32 v = 0; v < 4; v++) Fx(&G, val, v, a[v]);
        sb_put(s, "  *r%u_ = make_float4(%s, %s, %s, %s);\n", j, a[0], a[1], a[2], a[3]);
    }
    sb_put(s, "}\n");
    free(G.oi);
    free(G.scal);
    return sb_out(s, out, outlen);
}

static void emit_params(Gen *g) {
    u32 nb = g->k->n_leaves + 1;
    for (u32 b = 0; b < nb; b++) sb_put(&g->sb, "%schar* p%u", b ? ", " : "", b);
    for (u32 b = 0; b < nb; b++) sb_put(&g->sb, ", u32 c%u", b);
    if (g->n_scal) {
        sb_put(&g->sb, ", u32 sm_");
        for (u32 j = 0; j < g->n_scal; j++) sb_put(&g->sb, ", float sv%u", j);
    }
}

/* Loads of a leaf element at a constant index (the engine's scalar leaves:
 * learning rates, constants, counts) can take their value from a kernel
 * argument: when the host still holds the leaf's contents (written by the
 * host, not by a kernel since), it passes the value and sets bit j of sm_,
 * and the leaf need not be uploaded at all. */
static void plan_inline_scalars(Gen *g, KGenResult *out) {
    const UOpKernel *k = g->k;
    u32 scal_only = 0, other = 0;
    g->n_scal = 0;
    for (u32 i = 0; i < k->n_ops; i++) {
        g->scal[i] = -1;
        const KOp *op = &k->ops[i];
        if (op->type != KOP_LOAD) continue;
        u32 bi = op->imm.u;
        if (bi == 0 || bi > k->n_leaves) continue;
        u32 bit = bi <= 32 ? 1u << (bi - 1) : 0u;
        if (k->ops[op->arg[0]].type == KOP_CONST_U && g->n_scal < KGEN_MAX_SCALARS) {
            out->scal_leaf[g->n_scal] = bi - 1;
            out->scal_index[g->n_scal] = k->ops[op->arg[0]].imm.u;
            g->scal[i] = (i32)g->n_scal++;
            scal_only |= bit;
        } else {
            other |= bit;
        }
    }
    out->n_scal = g->n_scal;
    out->scal_only_leaves = scal_only & ~other;
}

/* GROUP kernels with few outputs and a long reduction (per-channel sums of
 * a whole batch: a handful of outputs over 10^5 elements) would leave most
 * CUs idle with one workgroup per output. When the program is a single
 * reduce loop whose accumulator is stored as is at gid, each output is split
 * over several workgroups: each writes its partial to a workspace, and a
 * second kernel combines the partials of an output in a fixed order
 * (SUM: init + p0 + p1 + ..., RMAX: the engine's a > b ? a : b). */
#define SPLIT_MAX_OUTPUTS 256u
#define SPLIT_MIN_TRIP 8192u
#define SPLIT_MIN_CHUNK 2048u

static void group_split_plan(Gen *g) {
    const UOpKernel *k = g->k;
    i32 r = -1;
    for (u32 i = 0; i < k->n_ops; i++) {
        if (k->ops[i].type == KOP_RANGE && g->oi[i].depth == 0) {
            if (r >= 0) return;                       /* more than one loop */
            r = (i32)i;
        }
    }
    if (r < 0) return;
    u32 e = g->oi[r].end, trip = k->ops[r].imm.u;
    if (g->total > SPLIT_MAX_OUTPUTS || trip < SPLIT_MIN_TRIP) return;
    /* after the loop: exactly STORE(gid op, accumulator) */
    if (e + 2 != k->n_ops) return;
    const KOp *st = &k->ops[e + 1];
    if (st->type != KOP_STORE || k->ops[st->arg[0]].type != KOP_GID) return;
    u32 t = st->arg[1];
    if (k->ops[t].type != KOP_ACC_INIT || !g->oi[t].acc_tgt) return;
    for (u32 i = 0; i < k->n_ops; i++)
        if (i != t && g->oi[i].acc_tgt) return;       /* one accumulator */
    u32 S = 1;
    while (g->total * S < g->split_target && trip / (S * 2) >= SPLIT_MIN_CHUNK && S < g->split_max) S *= 2;
    if (S < 2) return;
    g->splits = S;
    g->split_acc = t;
}

/* The end of a split workgroup (its partial t_ reduced): publish it, or, in
 * the workgroup with the last split index, combine the output's partials in
 * index order (lane l: partials l, l + block, ...; then the fixed
 * shuffle/LDS tree), add the accumulator's initial value and store. */
static void emit_single_pass(Gen *g, u32 t, int rmax) {
    const KOp *init = &g->k->ops[t];
    sb_put(&g->sb, "      t_ = %s(t_, red_);\n"
                   "      if (sp_ != %uu) {\n"
                   "        comb_put(sl_, gid, sp_, %uu, t_);\n"
                   "      } else {\n"
                   "        float w_ = %s;\n"
                   "        for (u32 s_ = lane; s_ < %uu; s_ += %uu) {\n"
                   "          const float x_ = (s_ == %uu) ? t_ : comb_take(sl_, gid, s_, %uu);\n"
                   "          %s\n"
                   "        }\n"
                   "        w_ = %s(w_, red_);\n"
                   "        if (lane == 0u) {\n"
                   "          float f_ = __uint_as_float(0x%08xu);\n"
                   "          %s\n"
                   "          %s(p0, c0, gid, f_);\n"
                   "        }\n"
                   "      }\n"
                   "    }\n",
           rmax ? "bmax" : "bsum", g->splits - 1, g->splits, rmax ? "__uint_as_float(0xff800000u)" : "0.0f",
           g->splits, g->block, g->splits - 1, g->splits, rmax ? "w_ = (w_ > x_) ? w_ : x_;" : "w_ = w_ + x_;",
           rmax ? "bmax" : "bsum", init->imm.u, rmax ? "f_ = (f_ > w_) ? f_ : w_;" : "f_ = f_ + w_;",
           dt_st(g->k->out_dtype));
}

/* One parallel loop of GROUP mode. */
static void emit_group_loop(Gen *g, u32 r) {
    const UOpKernel *k = g->k;
    u32 e = g->oi[r].end;
    u32 trip = k->ops[r].imm.u;
    u32 V = g->V;
    char a[128], b[128];
    sb_put(&g->sb, "  {\n");
    /* partials */
    for (u32 t = 0; t < r; t++) {
        if (!g->oi[t].acc_tgt) continue;
        int used = 0;
        for (u32 j = r + 1; j < e; j++)
            if (k->ops[j].type == KOP_ACC && k->ops[j].arg[0] == t) used = 1;
        if (!used) continue;
        for (u32 v = 0; v < V; v++) {
            if (g->oi[t].acc_type == UOP_RMAX) sb_put(&g->sb, "    float p%u_%u = f%u;\n", t, v, t);
            else sb_put(&g->sb, "    float p%u_%u = 0.0f;\n", t, v);
        }
    }
    /* prologue: index values at counter 0 and the one-time range check */
    sb_put(&g->sb, "    bool ok_ = true;\n");
    for (u32 j = r + 1; j < e; j++) {
        const OpI *o = &g->oi[j];
        const KOp *op = &k->ops[j];
        if (o->ft || o->gk == G_NOT || o->depth != 1) continue;
        if (op->type == KOP_CONST_U) { sb_put(&g->sb, "    const u32 g%u = %uu;\n", j, op->imm.u); continue; }
        if (op->type == KOP_GID) { sb_put(&g->sb, "    const u32 g%u = gid;\n", j); continue; }
        G0(g, op->arg[0], (i32)r, a);
        if (op->type == KOP_IDX) {
            G0(g, op->arg[1], (i32)r, b);
            sb_put(&g->sb, "    const u32 g%u = %s * %uu + %s;\n", j, a, op->imm.u, b);
        } else if (op->imm.u == 0) {
            sb_put(&g->sb, "    const u32 g%u = 0u;\n", j);
        } else {
            sb_put(&g->sb, "    const u32 g%u = %s %c %uu;\n", j, a, op->type == KOP_MOD ? '%' : '/', op->imm.u);
        }
    }
    for (u32 j = r + 1; j < e; j++) {
        const KOp *op = &k->ops[j];
        if (op->type != KOP_LOAD || g->oi[j].depth != 1) continue;
        const OpI *ix = &g->oi[op->arg[0]];
        if (ix->ft || ix->gk == G_NOT) continue;
        u32 bi = op->imm.u;
        if (bi > k->n_leaves) continue;
        char gv[64];
        G0(g, op->arg[0], (i32)r, gv);
        u64 span = (u64)ix->gs * (u64)(trip ? trip - 1 : 0);
        sb_put(&g->sb, "    ok_ = ok_ && (%s + %lluu >= %s) && (%s + %lluu < c%u);\n", gv,
               (unsigned long long)span, gv, gv, (unsigned long long)span, bi);
    }
    u32 nq = trip / V;
    if (g->splits > 1) {
        u32 cq = (nq + g->splits - 1) / g->splits;
        sb_put(&g->sb, "    const u32 qlo_ = sp_ * %uu, qhi_ = (qlo_ + %uu < %uu) ? qlo_ + %uu : %uu;\n", cq, cq, nq,
               cq, nq);
    } else {
        sb_put(&g->sb, "    const u32 qlo_ = 0u, qhi_ = %uu;\n", nq);
    }
    for (int pass = 0; pass < 2; pass++) {
        sb_put(&g->sb, pass == 0 ? "    if (ok_) {\n" : "    } else {\n");
        if (g->unroll > 1) sb_put(&g->sb, "    #pragma unroll %u\n", g->unroll);
        sb_put(&g->sb, "    for (u32 q_ = qlo_ + lane; q_ < qhi_; q_ += %uu) {\n    n%u = q_ * %uu;\n", g->block, r, V);
        emit_range_seq(g, r + 1, e, pass == 0, 1);
        sb_put(&g->sb, "    }\n");
    }
    sb_put(&g->sb, "    }\n");
    /* combine partials across the workgroup */
    for (u32 t = 0; t < r; t++) {
        if (!g->oi[t].acc_tgt) continue;
        int used = 0;
        for (u32 j = r + 1; j < e; j++)
            if (k->ops[j].type == KOP_ACC && k->ops[j].arg[0] == t) used = 1;
        if (!used) continue;
        if (g->oi[t].acc_type == UOP_RMAX) {
            sb_put(&g->sb, "    { float t_ = p%u_0;\n", t);
            for (u32 v = 1; v < V; v++) sb_put(&g->sb, "      t_ = (t_ > p%u_%u) ? t_ : p%u_%u;\n", t, v, t, v);
            if (g->splits > 1 && g->combine_launch)
                sb_put(&g->sb, "      t_ = bmax(t_, red_);\n"
                               "      if (lane == 0) ws_[(unsigned long long)gid * %uu + sp_] = t_; }\n", g->splits);
            else if (g->splits > 1)
                emit_single_pass(g, t, 1);
            else
                sb_put(&g->sb, g->block == 64 ? "      f%u = wmax0(t_); }\n" : "      f%u = bmax(t_, red_); }\n", t);
        } else {
            if (V == 4) sb_put(&g->sb, "    { float t_ = (p%u_0 + p%u_1) + (p%u_2 + p%u_3);\n", t, t, t, t);
            else {
                sb_put(&g->sb, "    { float t_ = p%u_0;\n", t);
                for (u32 v = 1; v < V; v++) sb_put(&g->sb, "      t_ = t_ + p%u_%u;\n", t, v);
            }
            if (g->splits > 1 && g->combine_launch)
                sb_put(&g->sb, "      t_ = bsum(t_, red_);\n"
                               "      if (lane == 0) ws_[(unsigned long long)gid * %uu + sp_] = t_; }\n", g->splits);
            else if (g->splits > 1)
                emit_single_pass(g, t, 0);
            else
                sb_put(&g->sb, g->block == 64 ? "      f%u = f%u + wsum0(t_); }\n" : "      f%u = f%u + bsum(t_, red_); }\n", t, t);
        }
    }
    sb_put(&g->sb, "  }\n");
}

int kgen_uop(const UOpKernel *k, KGenResult *out, char *err, size_t errlen) {
    return kgen_uop_lanes(k, out, NULL, err, errlen);
}

int kgen_uop_lanes(const UOpKernel *k, KGenResult *out, u32 *lanes, char *err, size_t errlen) {
    memset(out, 0, sizeof(*out));
    if (!kgen_validate(k, err, errlen)) return 0;
    Gen G;
    memset(&G, 0, sizeof(G));
    G.k = k;
    G.oi = calloc(k->n_ops, sizeof(OpI));
    if (!G.oi) { snprintf(err, errlen, "oom"); return 0; }
    analyze_structure(&G);
    {
        const char *e;
        G.unroll = (e = getenv("THVM_HIP_UNROLL")) ? (u32)atoi(e) : 1;
        G.nt = (e = getenv("THVM_HIP_NT")) ? atoi(e) : 1;   /* bit 0: loads, bit 1: stores */
        G.ew_block = (e = getenv("THVM_HIP_EW_BLOCK")) ? (u32)atoi(e) : 0;   /* 0: by size */
        if (G.ew_block != 0 && G.ew_block != 128 && G.ew_block != 256 && G.ew_block != 512 &&
            G.ew_block != 1024) G.ew_block = 0;
        G.red_block = (e = getenv("THVM_HIP_RED_BLOCK")) ? (u32)atoi(e) : 256;
        if (G.red_block != 64 && G.red_block != 128 && G.red_block != 512 && G.red_block != 1024)
            G.red_block = 256;
        G.split_target = (e = getenv("THVM_HIP_SPLIT_TARGET")) ? (u32)atoi(e) : 4096;
        if (G.split_target < 1) G.split_target = 4096;
        G.split_max = (e = getenv("THVM_HIP_SPLIT_MAX")) ? (u32)atoi(e) : 512;
        if (G.split_max < 2 || G.split_max > 1024) G.split_max = 512;
        e = getenv("THVM_HIP_SPLIT_COMBINE");
        G.combine_mode = !e ? 0 : strcmp(e, "launch") == 0 ? 1 : strcmp(e, "single") == 0 ? 2 : 0;
        G.per_thread = (e = getenv("THVM_HIP_EW_PER_THREAD")) ? (u32)atoi(e) : 1;
        if (G.per_thread < 1) G.per_thread = 1;
        if (G.per_thread > 8) G.per_thread = 8;
    }

    u32 total = k->local_size > 0 ? k->grid[0] : k->grid[0] * k->grid[1] * k->grid[2];
    G.total = total;
    char why[128] = {0};
    G.mode = KG_MODE_SERIAL;
    if (k->local_size > 0 && group_ok(&G, why, sizeof why)) G.mode = KG_MODE_GROUP;
    else if (k->local_size == 0 && tiny_long_reduce(&G, total) && group_ok(&G, why, sizeof why)) {
        /* a handful of outputs over a long loop (a loss summed over the batch
         * rows) would run as one or two threads walking the loop in order;
         * a workgroup per output splits it across lanes instead, so its sum
         * is ordered differently (the reductions' tolerance, not bit-exact) */
        G.mode = KG_MODE_GROUP;
    }
    if (G.mode == KG_MODE_SERIAL) {
        for (u32 i = 0; i < k->n_ops; i++) { G.oi[i].acc_tgt = 0; G.oi[i].acc_type = 0; }
    }

    if (G.mode == KG_MODE_GROUP) {
        u32 min_trip = 0xFFFFFFFFu;
        int all4 = 1;
        for (u32 i = 0; i < k->n_ops; i++) {
            if (k->ops[i].type == KOP_RANGE && G.oi[i].depth == 0) {
                u32 t = k->ops[i].imm.u;
                if (t < min_trip) min_trip = t;
                if (t % 4 != 0) all4 = 0;
            }
        }
        G.V = (all4 && min_trip >= 64) ? 4 : 1;
        u32 nq = min_trip / G.V;
        G.block = 64;
        while (G.block < G.red_block && G.block < nq) G.block *= 2;
    } else {
        G.V = (total >= 1024 && k->n_ops <= 256) ? 4 : 1;
        /* Streaming kernels over >= 4M thread-vectors run best with 1024-lane
         * workgroups (fewer, longer-lived groups); smaller grids keep 256 so
         * every CU still gets work. */
        u64 nv = ((u64)total + G.V - 1) / G.V;
        G.block = G.ew_block ? G.ew_block : (nv >= (4ull << 20) ? 1024 : 256);
    }
    G.splits = 1;
    if (G.mode == KG_MODE_GROUP) group_split_plan(&G);
    /* The partials combine in the same launch when the whole grid fits on
     * the GPU at once; a larger grid writes them to a workspace for a
     * combine kernel. */
    G.combine_launch = G.combine_mode == 1 || hipb.force_combine_launch ||
                       (G.combine_mode == 0 && (u64)G.total * G.splits * (G.block / 64) > hipb_resident_waves());
    G.scal = malloc(k->n_ops * sizeof(i32));
    if (!G.scal) { free(G.oi); snprintf(err, errlen, "oom"); return 0; }
    plan_inline_scalars(&G, out);
    analyze_vector(&G);
    if (G.mode == KG_MODE_SERIAL && G.V == 4 && serial_strided(&G)) {
        /* loads whose 4 lanes sit 2 or more elements apart inside a loop:
         * one gid per lane keeps each load instruction on contiguous lines */
        G.V = 1;
        u64 nv = total;
        G.block = G.ew_block ? G.ew_block : (nv >= (4ull << 20) ? 1024 : 256);
        analyze_vector(&G);
    }
    analyze_global(&G);

    SB *s = &G.sb;
    sb_put(s, "%s\n", kgen_prelude());
    {
        int has_loop = 0;
        for (u32 i = 0; i < k->n_ops; i++) if (k->ops[i].type == KOP_RANGE) has_loop = 1;
        const char *kind = G.mode == KG_MODE_GROUP ? "red" : (has_loop ? "loop" : "ew");
        snprintf(out->name, sizeof out->name, "thvm_%s_%08x", kind, (u32)(uop_signature(k) & 0xFFFFFFFFu));
    }
    sb_put(s, "extern \"C\" __global__ __launch_bounds__(%u) void %s(", G.block, out->name);
    emit_params(&G);
    if (G.splits > 1) sb_put(s, G.combine_launch ? ", float* ws_" : ", unsigned long long* sl_");
    sb_put(s, ") {\n");
    if (G.mode == KG_MODE_SERIAL) {
        u64 nvec = ((u64)total + G.V - 1) / G.V;          /* thread-vectors */
        u32 W = G.per_thread;
        if (nvec < (u64)W * G.block * 256) W = 1;
        u64 nthreads = (nvec + W - 1) / W;
        sb_put(s, "  const u32 TOTAL = %uu;\n", total);
        sb_put(s, "  const unsigned long long t_ = ((unsigned long long)blockIdx.y * gridDim.x + blockIdx.x) * %uull + threadIdx.x;\n", G.block);
        sb_put(s, "  if (t_ >= %lluull) return;\n", (unsigned long long)nthreads);
        if (W > 1) {
            sb_put(s, "  #pragma unroll\n  for (u32 w_ = 0; w_ < %uu; w_++) {\n", W);
            sb_put(s, "  const unsigned long long v_ = t_ + (unsigned long long)w_ * %lluull;\n", (unsigned long long)nthreads);
            sb_put(s, "  if (v_ >= %lluull) break;\n", (unsigned long long)nvec);
            sb_put(s, "  const u32 X0 = (u32)v_ * %uu;\n", G.V);
        } else {
            sb_put(s, "  const u32 X0 = (u32)t_ * %uu;\n", G.V);
        }
        emit_decls(&G);
        emit_range_seq(&G, 0, k->n_ops, 0, 0);
        if (W > 1) sb_put(s, "  }\n");
        out->n_threads = nthreads;
    } else {
        if (G.splits > 1) {
            sb_put(s, "  const u32 bid_ = blockIdx.y * gridDim.x + blockIdx.x;\n");
            sb_put(s, "  const u32 gid = bid_ / %uu, sp_ = bid_ %% %uu;\n", G.splits, G.splits);
        } else {
            sb_put(s, "  const u32 gid = blockIdx.y * gridDim.x + blockIdx.x;\n");
        }
        sb_put(s, "  if (gid >= %uu) return;\n", total);
        sb_put(s, "  const u32 lane = threadIdx.x;\n");
        /* a one-wave workgroup without splits reduces in registers */
        if (G.block > 64 || G.splits > 1) sb_put(s, "  __shared__ float red_[%u];\n", G.block / 64);
        emit_decls(&G);
        for (u32 i = 0; i < k->n_ops; i++) {
            const KOp *op = &k->ops[i];
            if (op->type == KOP_RANGE && G.oi[i].depth == 0) {
                emit_group_loop(&G, i);
                i = G.oi[i].end;
                if (G.splits > 1) break;      /* the store happens in the combine kernel */
                continue;
            }
            if (op->type == KOP_ENDRANGE) continue;
            emit_op(&G, i, 0, 0);
        }
        out->n_threads = total;
    }
    sb_put(s, "}\n");
    if (G.splits > 1 && G.combine_launch) {
        /* combine: one workgroup per output; lane l takes partials l, l + 256,
         * ... in order, then a fixed shuffle/LDS tree, then the initial value */
        const KOp *init = &k->ops[G.split_acc];
        u32 bits = init->imm.u;
        int rmax = G.oi[G.split_acc].acc_type == UOP_RMAX;
        sb_put(s, "extern \"C\" __global__ __launch_bounds__(256) void %s_fin(char* p0, u32 c0, const float* ws_) {\n"
                  "  const u32 o = blockIdx.x;\n"
                  "  if (o >= %uu) return;\n"
                  "  __shared__ float red_[4];\n"
                  "  float w_ = %s;\n"
                  "  for (u32 s = threadIdx.x; s < %uu; s += 256u) {\n"
                  "    const float x_ = ws_[(unsigned long long)o * %uu + s];\n"
                  "    %s\n"
                  "  }\n"
                  "  w_ = %s(w_, red_);\n"
                  "  if (threadIdx.x == 0u) {\n"
                  "    float f = __uint_as_float(0x%08xu);\n"
                  "    %s\n"
                  "    %s(p0, c0, o, f);\n"
                  "  }\n}\n",
               out->name, total, rmax ? "__uint_as_float(0xff800000u)" : "0.0f", G.splits, G.splits,
               rmax ? "w_ = (w_ > x_) ? w_ : x_;" : "w_ = w_ + x_;", rmax ? "bmax" : "bsum", bits,
               rmax ? "f = (f > w_) ? f : w_;" : "f = f + w_;", dt_st(k->out_dtype));
    }
    if (lanes)
        for (u32 i = 0; i < k->n_ops; i++) {
            const OpI *o = &G.oi[i];
            u32 *l = lanes + 7 * i;
            l[0] = o->ft ? 3u : o->kind;
            for (u32 v = 0; v < 4; v++) l[1 + v] = o->off[v];
            l[5] = o->dv;
            l[6] = (u32)o->hi;
        }
    free(G.oi);
    free(G.scal);
    if (!s->p) { snprintf(err, errlen, "oom"); return 0; }
    out->src = s->p;
    out->mode = G.mode;
    out->vec = G.V;
    out->block = G.block;
    out->total = total;
    out->splits = G.splits;
    out->combine_launch = G.splits > 1 && G.combine_launch;
    return 1;
}

void kgen_free(KGenResult *r) {
    if (r && r->src) free(r->src);
    if (r) r->src = NULL;
}
