/*
 * affine.h - digit analysis of KOp index programs, shared by the recognizers
 * that route UOpKernels to hand-written kernels (dense.c: contractions;
 * window.c: pooling windows and per-channel reductions).
 *
 * Every index op of a program is rewritten as
 *     c + sum_i a_i * digit_i,   digit = (x / div) % mod   (mod 0: none)
 * of x = gid (range [0, total)) or x = r, the counter of the program's one
 * top-level loop (range [0, trip)). The lowerer builds coordinates exactly
 * this way (MOD/DIV chains over GID and the RANGE counter,
 * src/lower/_.c:828-876) and leaf indices as strided sums of them
 * (src/lower/_.c:435-494). u32 arithmetic is exact in this form as long as
 * no intermediate wraps; the recognizers check value bounds where they rely
 * on it.
 */
#ifndef THVM_AFFINE_H
#define THVM_AFFINE_H

#include "thvm_abi.h"

#define DG_MAX 8

typedef struct { u8 var; u32 div, mod; } Digit;      /* var 0: gid, 1: r */
typedef struct {
    int ok;
    u32 cst;
    u32 n;
    Digit d[DG_MAX];
    u32 coef[DG_MAX];
} Aff;

typedef struct {
    const UOpKernel *k;
    u32 total, trip;
    i32 range_op;
    Aff *aff;
} DCtx;

int  op_type_is_float(KOpType t);
u64  var_range(const DCtx *c, u8 var);
void digit_norm(const DCtx *c, Digit *d, int *is_zero);
int  aff_add_term(Aff *a, Digit d, u32 coef);
int  is_single_digit(const Aff *a);
/* c->aff[i] for every op i of c->k (ok = 0 where the op is not such a sum) */
void analyze_aff(DCtx *c);
/* cone[i] = 1 for every op the value of `root` depends on */
void mark_cone(const UOpKernel *k, u32 root, u8 *cone);
u64  contiguous_run(const DCtx *c, const Aff *a, u8 var);
/* the value of an affine sum at x = gid (var 0) and r (var 1) */
u64  aff_eval(const Aff *a, u32 gid, u32 r);
/* the largest value an affine sum takes over its digits' ranges */
u64  aff_max(const DCtx *c, const Aff *a);
/* whether an affine sum is gid itself for every gid in [0, total) */
int  aff_is_gid(const DCtx *c, const Aff *a);

#endif
