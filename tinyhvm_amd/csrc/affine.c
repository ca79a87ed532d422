/*
 * affine.c - digit analysis of KOp index programs (see affine.h).
 */
#include <string.h>

#include "affine.h"

int op_type_is_float(KOpType t) {
    return t == KOP_CONST_F || t == KOP_LOAD || t == KOP_ALU || t == KOP_ACC_INIT || t == KOP_MASK;
}

u64 var_range(const DCtx *c, u8 var) { return var ? c->trip : c->total; }

void digit_norm(const DCtx *c, Digit *d, int *is_zero) {
    u64 r = var_range(c, d->var);
    *is_zero = 0;
    if ((u64)d->div >= r) { *is_zero = 1; return; }
    if (d->mod && (u64)d->div * d->mod >= r) d->mod = 0;
}

int aff_add_term(Aff *a, Digit d, u32 coef) {
    if (coef == 0) return 1;
    for (u32 i = 0; i < a->n; i++) {
        if (a->d[i].var == d.var && a->d[i].div == d.div && a->d[i].mod == d.mod) {
            a->coef[i] += coef;
            if (a->coef[i] == 0) {
                a->d[i] = a->d[a->n - 1];
                a->coef[i] = a->coef[a->n - 1];
                a->n--;
            }
            return 1;
        }
    }
    if (a->n >= DG_MAX) return 0;
    a->d[a->n] = d;
    a->coef[a->n] = coef;
    a->n++;
    return 1;
}

int is_single_digit(const Aff *a) { return a->ok && a->cst == 0 && a->n == 1 && a->coef[0] == 1; }

void analyze_aff(DCtx *c) {
    const UOpKernel *k = c->k;
    for (u32 i = 0; i < k->n_ops; i++) {
        const KOp *op = &k->ops[i];
        Aff *o = &c->aff[i];
        memset(o, 0, sizeof *o);
        switch (op->type) {
        case KOP_GID: {
            Digit d = {0, 1, 0};
            int z;
            digit_norm(c, &d, &z);
            o->ok = 1;
            if (!z) aff_add_term(o, d, 1);
            break;
        }
        case KOP_RANGE: {
            if ((i32)i != c->range_op) break;
            Digit d = {1, 1, 0};
            int z;
            digit_norm(c, &d, &z);
            o->ok = 1;
            if (!z) aff_add_term(o, d, 1);
            break;
        }
        case KOP_CONST_U:
            o->ok = 1;
            o->cst = op->imm.u;
            break;
        case KOP_IDX: {
            const Aff *a = &c->aff[op->arg[0]], *b = &c->aff[op->arg[1]];
            if (!a->ok || !b->ok) break;
            u32 s = op->imm.u;
            o->ok = 1;
            o->cst = a->cst * s + b->cst;
            for (u32 t = 0; t < a->n && o->ok; t++) o->ok = aff_add_term(o, a->d[t], a->coef[t] * s);
            for (u32 t = 0; t < b->n && o->ok; t++) o->ok = aff_add_term(o, b->d[t], b->coef[t]);
            break;
        }
        case KOP_MOD: case KOP_DIV: {
            const Aff *a = &c->aff[op->arg[0]];
            u32 q = op->imm.u;
            if (!a->ok) break;
            if (q == 0) { o->ok = 1; break; }
            if (a->n == 0) {
                o->ok = 1;
                o->cst = op->type == KOP_MOD ? a->cst % q : a->cst / q;
                break;
            }
            if (!is_single_digit(a)) break;
            Digit d = a->d[0];
            if (op->type == KOP_MOD) {
                if (d.mod == 0 || d.mod % q == 0) d.mod = q;
                else if (q % d.mod == 0) { /* already smaller */ }
                else break;
            } else {
                if (q == 1) { *o = *a; break; }
                if (d.mod == 0) d.div *= q;
                else if (d.mod % q == 0) { d.div *= q; d.mod /= q; }
                else break;
            }
            int z;
            digit_norm(c, &d, &z);
            o->ok = 1;
            if (!z) aff_add_term(o, d, 1);
            break;
        }
        default:
            break;
        }
    }
}

/* Marks the cone of op `root` (all ops it depends on). */
void mark_cone(const UOpKernel *k, u32 root, u8 *cone) {
    u32 stack[KOP_MAX];
    u32 sp = 0;
    stack[sp++] = root;
    while (sp) {
        u32 i = stack[--sp];
        if (cone[i]) continue;
        cone[i] = 1;
        const KOp *op = &k->ops[i];
        int na = 0;
        switch (op->type) {
        case KOP_MOD: case KOP_DIV: case KOP_LOAD: na = 1; break;
        case KOP_IDX: case KOP_MASK: case KOP_ALU: na = 2; break;
        default: na = 0; break;
        }
        if (op->type == KOP_ALU) {
            u32 u = op->imm.u;
            if (u == UOP_NEG || u == UOP_EXP || u == UOP_LOG || u == UOP_RELU || u == UOP_CAST || u == UOP_SQRT)
                na = 1;
        }
        for (int a = 0; a < na; a++)
            if (op->arg[a] < i && sp < KOP_MAX) stack[sp++] = op->arg[a];
    }
}

/* Length of the contiguous run of an affine index along one variable: its
 * fastest digit with coefficient 1, extended by each next digit whose
 * coefficient equals the run so far (e.g. [y, x] of a row-major image); 0
 * when the fastest digit is not unit-stride. Along k (var 1) the next digit
 * must follow in k itself (divisor = the run's); along the output rows
 * (var 0) it is the side's next gid digit, wherever the other side's digits
 * sit between them in gid. */
u64 contiguous_run(const DCtx *c, const Aff *a, u8 var) {
    u64 run = 0, div = 0;
    for (;;) {
        int t = -1;
        for (u32 i = 0; i < a->n; i++) {
            if (a->d[i].var != var) continue;
            if (var == 1 && a->d[i].div != (div ? div : 1)) continue;
            if (var == 0 && a->d[i].div <= div) continue;
            if (t < 0 || a->d[i].div < a->d[t].div) t = (int)i;
        }
        if (t < 0 || a->coef[t] != (run ? run : 1)) break;
        u64 ext = a->d[t].mod ? a->d[t].mod : (var_range(c, var) + a->d[t].div - 1) / a->d[t].div;
        run = run ? run * ext : ext;
        div = a->d[t].div;
        if (!a->d[t].mod) break;
        if (var == 1) div *= ext;
        if (div > 0xFFFFFFFFull || run > 0xFFFFFFFFull) break;
    }
    return run;
}

u64 aff_eval(const Aff *a, u32 gid, u32 r) {
    u64 v = a->cst;
    for (u32 t = 0; t < a->n; t++) {
        u64 x = a->d[t].var ? r : gid;
        x /= a->d[t].div;
        if (a->d[t].mod) x %= a->d[t].mod;
        v += (u64)a->coef[t] * x;
    }
    return v;
}

u64 aff_max(const DCtx *c, const Aff *a) {
    u64 v = a->cst;
    for (u32 t = 0; t < a->n; t++) {
        u64 range = var_range(c, a->d[t].var);
        u64 hi = range ? (range - 1) / a->d[t].div : 0;
        if (a->d[t].mod && hi > a->d[t].mod - 1) hi = a->d[t].mod - 1;
        v += (u64)a->coef[t] * hi;
    }
    return v;
}

int aff_is_gid(const DCtx *c, const Aff *a) {
    if (!a->ok || a->cst != 0 || a->n == 0 || a->n > DG_MAX) return 0;
    /* digits of gid alone, in increasing div, each step the previous one's
     * div * mod, the coefficient its div, the last without a mod */
    u32 ord[DG_MAX];
    for (u32 t = 0; t < a->n; t++) ord[t] = t;
    for (u32 i = 1; i < a->n; i++)
        for (u32 j = i; j > 0 && a->d[ord[j - 1]].div > a->d[ord[j]].div; j--) {
            const u32 x = ord[j];
            ord[j] = ord[j - 1];
            ord[j - 1] = x;
        }
    u64 step = 1;
    for (u32 i = 0; i < a->n; i++) {
        const Digit *d = &a->d[ord[i]];
        if (d->var != 0 || d->div != step || a->coef[ord[i]] != d->div) return 0;
        if (i + 1 == a->n) return d->mod == 0 || (u64)d->div * d->mod >= var_range(c, 0);
        if (d->mod == 0) return 0;
        step = (u64)d->div * d->mod;
        if (step > 0xFFFFFFFFull) return 0;
    }
    return 0;
}
