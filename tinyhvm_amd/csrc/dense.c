/*
 * dense.c - routes contraction-shaped UOpKernels to f32 matrix-core kernels.
 *
 * The engine has no matmul or convolution op on this path: a matmul is
 * EXPAND+MUL+SUM over [M,K,N] (src/ctx/init.c:555-612) and a convolution is
 * a pool view times the weight, summed over (ci,kh,kw) of an 8-D domain
 * (src/nn/conv.c:390-481). Both reach the backend as a KOp program of the
 * form
 *     acc = 0;  for r in [0,K): acc += P(gid, r) * Q(gid, r);  out[gid] = acc
 * This file proves that shape and splits the output index into M and N.
 *
 * Digit analysis. Every index op of the program is rewritten as
 *     c + sum_i a_i * digit_i,   digit = (x / div) % mod   (mod 0: none)
 * of x = gid (range [0, total)) or x = r (range [0, K)). The lowerer builds
 * coordinates exactly this way (MOD/DIV chains over GID and the RANGE
 * counter, src/lower/_.c:828-876) and leaf indices as strided sums of them
 * (src/lower/_.c:435-494). A program is a contraction when
 *   - the loop body is one SUM ACC of MUL(P, Q), and nothing else escapes;
 *   - the gid digits P depends on and the gid digits Q depends on are
 *     disjoint, and together tile gid exactly (a mixed-radix decomposition);
 *   - the output index is gid itself.
 * Then out[gid_m(m) + gid_n(n)] = init + sum_r P(gid_m(m), r) * Q(gid_n(n), r)
 * for m in [0,M), n in [0,N): a GEMM whose operands are *evaluated*, not
 * loaded: the generated kernel runs P's and Q's own KOp code per element
 * (bounds-checked loads, pad masks, fused elementwise prologues), so the
 * operand values are exactly the engine's; only the summation order differs
 * (matrix-core accumulation, tolerance 1e-4 normwise).
 *
 * Kernel: 256 lanes, 128x128 output tile, K staged 16 at a time through
 * double-buffered LDS, each wavefront accumulating 64x64 with
 * v_mfma_f32_32x32x2_f32 (2x2 blocks). Operand tiles are loaded with the
 * lane order that is contiguous in memory for that operand (found from the
 * digit form of its first load). Tiles are assigned so that each XCD works on
 * a compact block of the tile grid (L2 reuse); long reductions are split
 * over K across workgroups and summed in a second, fixed-order pass.
 */
#include <stdlib.h>
#include <string.h>

#include "hipb.h"
#include "thvm_hip.h"

#define DENSE_MIN_K 16
#define DENSE_MIN_WORK (1ull << 12)

#include "affine.h"

typedef struct {
    int ok;
    u32 M, N, K;
    f32 init;
    u8 coneP[KOP_MAX], coneQ[KOP_MAX];
    u32 rootP, rootQ;
    /* gid digits of each side, sorted by div descending */
    u32 np, nq;
    u32 pdiv[DG_MAX], pext[DG_MAX], qdiv[DG_MAX], qext[DG_MAX];
    int p_kmajor, q_kmajor;       /* lanes along k when loading the tile */
    /* separable operands: the side is one LOAD whose index is f(gid) + g(r)
     * (no digit mixes gid and r); the loader then adds a per-row base and a
     * per-k offset instead of evaluating the operand's program per element */
    int sep[2];
    u32 sep_buf[2], sep_dt[2];
    Aff sep_aff[2];
} Contraction;

/* The gid digits an operand consumes: those of the integer values its float
 * ops read (load indices, integers converted for ALU/MASK). Intermediate
 * index ops (the raw GID, partial MOD/DIV chains) do not count. */
static int add_digits(const DCtx *c, u32 arg, Digit *out, u32 *n, int *uses_r) {
    if (op_type_is_float(c->k->ops[arg].type)) return 1;
    const Aff *a = &c->aff[arg];
    if (!a->ok) return 0;
    for (u32 t = 0; t < a->n; t++) {
        if (a->d[t].var == 1) { *uses_r = 1; continue; }
        int dup = 0;
        for (u32 j = 0; j < *n; j++)
            if (out[j].div == a->d[t].div && out[j].mod == a->d[t].mod) dup = 1;
        if (!dup) {
            if (*n >= DG_MAX) return 0;
            out[(*n)++] = a->d[t];
        }
    }
    return 1;
}

static int collect_gdigits(const DCtx *c, const u8 *cone, Digit *out, u32 *n, int *uses_r) {
    *n = 0;
    *uses_r = 0;
    for (u32 i = 0; i < c->k->n_ops; i++) {
        if (!cone[i]) continue;
        const KOp *op = &c->k->ops[i];
        switch (op->type) {
        case KOP_LOAD:
            if (!add_digits(c, op->arg[0], out, n, uses_r)) return 0;
            break;
        case KOP_MASK:
        case KOP_ALU:
            if (!add_digits(c, op->arg[0], out, n, uses_r)) return 0;
            if (!add_digits(c, op->arg[1], out, n, uses_r)) return 0;
            break;
        default:
            break;
        }
    }
    return 1;
}

/* Is the first load of the cone contiguous along r (k) rather than gid? The
 * longer contiguous run wins: an image's rows (56 floats along the output
 * pixels of a convolution) over the 3 taps of a kernel row along k. */
static int cone_kmajor(const DCtx *c, const u8 *cone) {
    for (u32 i = 0; i < c->k->n_ops; i++) {
        if (!cone[i] || c->k->ops[i].type != KOP_LOAD) continue;
        const Aff *a = &c->aff[c->k->ops[i].arg[0]];
        if (!a->ok) return 1;
        return contiguous_run(c, a, 1) >= contiguous_run(c, a, 0);
    }
    return 1;
}

static int cmp_digit_div_desc(const void *x, const void *y) {
    const Digit *a = x, *b = y;
    return a->div < b->div ? 1 : (a->div > b->div ? -1 : 0);
}

static int dense_debug(void) {
    static int v = -1;
    if (v < 0) { const char *e = getenv("THVM_HIP_DENSE_DEBUG"); v = e && e[0] == '1'; }
    return v;
}
#define REJECT(why) do { if (dense_debug()) fprintf(stderr, "dense: not a contraction: %s\n", why); return 0; } while (0)

static int recognize(const UOpKernel *k, Contraction *ct) {
    memset(ct, 0, sizeof *ct);
    if (k->n_ops == 0 || k->n_ops > KOP_MAX) REJECT("line 2");
    /* operands name earlier ops, loops nest, types are known: the analyses
     * below follow operand indices without further checks */
    char verr[128];
    if (!kgen_validate(k, verr, sizeof verr)) REJECT("invalid program");
    /* one top-level loop, no nesting */
    i32 R = -1;
    u32 E = 0;
    int depth = 0;
    for (u32 i = 0; i < k->n_ops; i++) {
        if (k->ops[i].type == KOP_RANGE) {
            if (depth || R >= 0) REJECT("line 9");
            R = (i32)i;
            depth = 1;
        } else if (k->ops[i].type == KOP_ENDRANGE) {
            if (!depth) REJECT("line 13");
            depth = 0;
            E = i;
        }
    }
    if (R < 0 || depth) REJECT("line 18");
    /* the body: exactly one ACC, SUM, of a MUL */
    i32 acc_op = -1;
    for (u32 i = (u32)R + 1; i < E; i++) {
        const KOp *op = &k->ops[i];
        if (op->type == KOP_STORE || op->type == KOP_ACC_INIT) REJECT("line 23");
        if (op->type == KOP_ACC) {
            if (acc_op >= 0 || op->imm.u == UOP_RMAX) REJECT("line 25");
            acc_op = (i32)i;
        }
    }
    if (acc_op < 0) REJECT("line 29");
    u32 tgt = k->ops[acc_op].arg[0];
    if (k->ops[tgt].type != KOP_ACC_INIT || tgt > (u32)R) REJECT("line 31");
    const KOp *mul = &k->ops[k->ops[acc_op].arg[1]];
    if (mul->type != KOP_ALU || mul->imm.u != UOP_MUL) REJECT("line 33");
    ct->rootP = mul->arg[0];
    ct->rootQ = mul->arg[1];
    ct->init = k->ops[tgt].imm.f;
    /* after the loop: one STORE of the accumulator at index gid; no other
     * side effects anywhere */
    i32 store = -1;
    for (u32 i = 0; i < k->n_ops; i++) {
        if (k->ops[i].type == KOP_STORE) {
            if (store >= 0 || i < E) REJECT("line 42");
            store = (i32)i;
        }
    }
    if (store < 0 || k->ops[store].arg[1] != tgt) REJECT("line 46");

    DCtx c = {k, k->local_size > 0 ? k->grid[0] : k->grid[0] * k->grid[1] * k->grid[2],
              k->ops[R].imm.u, R, NULL};
    if (c.total == 0 || c.trip == 0) REJECT("line 50");
    Aff aff[KOP_MAX];
    c.aff = aff;
    analyze_aff(&c);
    /* output index must be exactly gid */
    const Aff *sa = &aff[k->ops[store].arg[0]];
    if (!sa->ok || sa->cst != 0 || sa->n != 1 || sa->coef[0] != 1 || sa->d[0].var != 0 ||
        sa->d[0].div != 1 || sa->d[0].mod != 0)
        REJECT("line 58");
    mark_cone(k, ct->rootP, ct->coneP);
    mark_cone(k, ct->rootQ, ct->coneQ);
    /* every op of the loop body belongs to P, Q, or is the MUL/ACC */
    for (u32 i = (u32)R + 1; i < E; i++) {
        if ((i32)i == acc_op || &k->ops[i] == mul) continue;
        if (!ct->coneP[i] && !ct->coneQ[i]) REJECT("line 64");
    }
    /* no float op is shared between the operands */
    for (u32 i = 0; i < k->n_ops; i++)
        if (ct->coneP[i] && ct->coneQ[i] && op_type_is_float(k->ops[i].type)) REJECT("line 68");
    /* the accumulator itself must not feed the operands */
    if (ct->coneP[tgt] || ct->coneQ[tgt]) REJECT("line 70");
    Digit gp[DG_MAX], gq[DG_MAX];
    u32 np = 0, nq = 0;
    int pr = 0, qr = 0;
    if (!collect_gdigits(&c, ct->coneP, gp, &np, &pr)) REJECT("line 74");
    if (!collect_gdigits(&c, ct->coneQ, gq, &nq, &qr)) REJECT("line 75");
    if (np == 0 || nq == 0) REJECT("line 76");
    /* disjoint, and together a mixed-radix tiling of [0,total) */
    Digit all[2 * DG_MAX];
    u32 na = 0;
    for (u32 i = 0; i < np; i++) all[na++] = gp[i];
    for (u32 i = 0; i < nq; i++) {
        for (u32 j = 0; j < np; j++)
            if (gp[j].div == gq[i].div) REJECT("line 83");
        all[na++] = gq[i];
    }
    qsort(all, na, sizeof(Digit), cmp_digit_div_desc);
    u64 expect_div = 1;
    for (i32 i = (i32)na - 1; i >= 0; i--) {
        if (all[i].div != expect_div) REJECT("line 89");
        if (i > 0) {
            if (all[i].mod == 0) REJECT("line 91");
            expect_div *= all[i].mod;
        } else if (all[i].mod != 0) {
            REJECT("line 94");
        }
    }
    qsort(gp, np, sizeof(Digit), cmp_digit_div_desc);
    qsort(gq, nq, sizeof(Digit), cmp_digit_div_desc);
    u64 M = 1, N = 1;
    for (u32 i = 0; i < np; i++) {
        u32 e = gp[i].mod ? gp[i].mod : (u32)((c.total + gp[i].div - 1) / gp[i].div);
        ct->pdiv[i] = gp[i].div;
        ct->pext[i] = e;
        M *= e;
    }
    for (u32 i = 0; i < nq; i++) {
        u32 e = gq[i].mod ? gq[i].mod : (u32)((c.total + gq[i].div - 1) / gq[i].div);
        ct->qdiv[i] = gq[i].div;
        ct->qext[i] = e;
        N *= e;
    }
    if (M * N != c.total || M > 0xFFFFFFFFull || N > 0xFFFFFFFFull) REJECT("line 112");
    ct->np = np;
    ct->nq = nq;
    ct->M = (u32)M;
    ct->N = (u32)N;
    ct->K = c.trip;
    ct->p_kmajor = cone_kmajor(&c, ct->coneP);
    ct->q_kmajor = cone_kmajor(&c, ct->coneQ);
    for (int side = 0; side < 2 && !hipb.dense_nosep; side++) {
        const KOp *ld = &k->ops[side ? ct->rootQ : ct->rootP];
        if (ld->type != KOP_LOAD || ld->imm.u > k->n_leaves || !c.aff[ld->arg[0]].ok) continue;
        ct->sep[side] = 1;
        ct->sep_buf[side] = ld->imm.u;
        ct->sep_dt[side] = ld->imm.u == 0 ? k->out_dtype : k->leaf_dtypes[ld->imm.u - 1];
        ct->sep_aff[side] = c.aff[ld->arg[0]];
    }
    ct->ok = 1;
    return 1;
}

/* ---------------- code generation ---------------- */

typedef struct { char *p; size_t n, cap; } DSB;
static void dsb_put(DSB *s, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
#include <stdarg.h>
static void dsb_put(DSB *s, const char *fmt, ...) {
    va_list ap;
    for (;;) {
        size_t room = s->cap - s->n;
        va_start(ap, fmt);
        int w = vsnprintf(s->p ? s->p + s->n : NULL, s->p ? room : 0, fmt, ap);
        va_end(ap);
        if (w < 0) return;
        if (s->p && (size_t)w < room) { s->n += (size_t)w; return; }
        size_t nc = s->cap ? s->cap * 2 : 32768;
        while (nc < s->n + (size_t)w + 1) nc *= 2;
        char *np = realloc(s->p, nc);
        if (!np) return;
        s->p = np;
        s->cap = nc;
    }
}

static void emit_params(DSB *s, u32 n_leaves) {
    for (u32 b = 0; b <= n_leaves; b++) dsb_put(s, "%schar* p%u", b ? ", " : "", b);
    for (u32 b = 0; b <= n_leaves; b++) dsb_put(s, ", u32 c%u", b);
}
static void emit_args(DSB *s, u32 n_leaves) {
    for (u32 b = 0; b <= n_leaves; b++) dsb_put(s, "%sp%u", b ? ", " : "", b);
    for (u32 b = 0; b <= n_leaves; b++) dsb_put(s, ", c%u", b);
}

/* flat index over one side's digits -> the gid contribution */
static void emit_gid_fn(DSB *s, const char *name, u32 n, const u32 *div, const u32 *ext) {
    dsb_put(s, "__device__ __forceinline__ u32 %s(u32 x) {\n  u32 g = 0u;\n", name);
    for (i32 i = (i32)n - 1; i >= 0; i--) {
        if (i > 0) dsb_put(s, "  g += (x %% %uu) * %uu; x /= %uu;\n", ext[i], div[i], ext[i]);
        else dsb_put(s, "  g += x * %uu;\n", div[i]);
    }
    dsb_put(s, "  return g;\n}\n");
}

/* Tile shapes. Every shape uses v_mfma_f32_32x32x2f32 blocks and 4 waves:
 * a wave owns wm_b x wn_b blocks (32x32 each); the waves form a gm x gn grid. */
typedef struct {
    u32 bm, bn, bk;
    u32 wm_b, wn_b;
    u32 gm, gn;
    const char *tag;
    int direct;    /* no LDS: 1 = each wave owns one 32x32 block and loads its MFMA operands
                      itself; 2 = skinny (see CFG_SKINNY) */
} TileCfg;

/* bk: K per LDS stage (32 halves the barriers per K of 16; measured 2-3%
 * faster on the 128x128 tile, and long split reductions on the 64x64 tile
 * take half as many load-latency-bound steps). */
static const TileCfg CFG_BIG = {128, 128, 32, 2, 2, 2, 2, "128x128"};   /* large square GEMMs */
static const TileCfg CFG_MID = {64, 64, 32, 1, 1, 2, 2, "64x64"};       /* small GEMMs: more tiles */
static const TileCfg CFG_TALL = {256, 32, 16, 2, 1, 4, 1, "256x32"};    /* N <= 32 (conv channels) */
static const TileCfg CFG_WIDE = {32, 256, 16, 1, 2, 1, 4, "32x256"};    /* M <= 32 */
/* 64 output channels: waves stacked along M, each 64x64 like the big tile;
 * K 16 per stage keeps the stages at 42 KB of LDS (3 workgroups per CU) */
static const TileCfg CFG_C64 = {256, 64, 16, 2, 2, 4, 1, "256x64"};
static const TileCfg CFG_C64S = {128, 64, 32, 2, 1, 2, 2, "128x64"};
/* 64 output channels: four waves stacked along M, each 32 rows by all 64
 * columns (two accumulator chains sharing each A fragment) */
static const TileCfg CFG_C64W = {128, 64, 16, 1, 2, 4, 1, "128x64w"};
/* Small and skinny contractions (conv channels, fc layers, weight gradients):
 * with operands that fit in L2 there is little to gain from sharing tiles
 * through LDS, and everything to gain from keeping many independent loads in
 * flight without barriers. Each wave computes one 32x32 block, loading 32 K
 * of both MFMA operands per iteration straight into registers. */
static const TileCfg CFG_DIRECT = {32, 32, 32, 1, 1, 1, 1, "direct32", 1};
/* 64 output channels over many rows (3x3 64->64 convolutions): no LDS and
 * no barriers. Each wave owns 32 rows by all 64 columns (two accumulator
 * chains sharing each A fragment) and loads its MFMA fragments straight from
 * memory with buffer loads: a lane's row offset is fixed, the k offset is
 * uniform (scalar), and the B side is the packed K x 64 weight matrix. A ring
 * of k-pairs of fragments is in flight ahead of the MFMAs. Measured on the
 * 3x3 64->64 convolution over [64,64,56,56] in a standalone probe: 141 us
 * against 242 us for the same probe's 64x64 LDS tile. */
static const TileCfg CFG_WAVE = {32, 64, 2, 1, 2, 1, 1, "wave32x64", 4};
/* Skinny contractions: at most 16 columns over many rows (the convolutions
 * of a few channels: LeNet-5's 6 and 16). A 32-wide MFMA block would leave
 * most of its columns empty; here each lane owns one row and keeps all N
 * column sums in registers, reading its operand element once per k and the
 * k-th row of the small side as wave-uniform (scalar) loads, with the
 * workgroup's waves splitting K and adding their sums in wave order. VALU
 * FMAs, no LDS tiles, no split-K workspace. */
static const TileCfg CFG_SKINNY = {64, 16, 1, 1, 1, 1, 1, "skinny", 2};
/* Outer-product reductions: few outputs (M*N <= RED_MAX_MN) over a long K
 * (the weight gradients of a few-channel convolution: LeNet-5's conv1,
 * 25x6 over 200704 pixels, and conv2, 150x16 over 25600). On MFMA blocks
 * most of each 32x32 block is empty and the split-K chain is long. Here a
 * lane walks k (a pixel: unit stride along the image rows) and keeps the
 * outer products of a group of MG rows with all N columns in registers;
 * a workgroup takes one row group and one K chunk, halves its partials
 * across the wavefront's lanes by shuffles, adds the four waves in order, and
 * the chunks' partials go through the split-K sum. Both sides separable. */
static const TileCfg CFG_RED = {1, 1, 1, 1, 1, 1, 1, "outer", 3};
#define RED_MAX_MN 4096
#define RED_MIN_K 8192
#define RED_MAX_ACC 96        /* MG * N */
#define RED_K_PER_LANE 8
#define SKINNY_MAX_N 16
#define SKINNY_MAX_KN 8192   /* the small side in LDS: at most 32 KB */
#define SKINNY_MIN_M 4096
#define SKINNY_TARGET_WAVES 4096
#define SKINNY_TARGET_WAVES_BLK 8192

/* K-reordered affine loading of separable operands. K is split into atomic
 * digits (the finest mixed radix both operands' k offsets decompose into);
 * the largest digit whose extent is a multiple of the stage depth becomes the
 * innermost, so that within a stage both offsets are a uniform base (a
 * function of the stage's start) plus a per-lane constant. The sum visits the
 * same (m, n, k) terms in another order. Loads are unchecked: the dispatch
 * verifies that the largest index each side can form lies inside its buffer. */
#define KP_MAX (4 * DG_MAX + 2)
typedef struct {
    int on;
    u32 E;                       /* extent of the inner digit */
    u32 Ep;                      /* E rounded up to the stage depth: k runs over Ep per outer step and
                                    the loaders zero elements whose inner index is E or more */
    u32 Kl;                      /* the reordered K the GEMM loops over: K / E * Ep */
    u32 ndig;                    /* outer digits, fastest first */
    u32 oext[KP_MAX];
    u32 ocoef[2][KP_MAX];
    u32 icoef[2];                /* per side: coefficient of the inner digit */
    u64 maxidx[2];               /* largest element index a side can form */
    u32 buf[2];                  /* the buffer each side loads (1 + leaf) */
    int lin[2];                  /* tile rows map to offsets linearly (no digit carry inside a tile) */
    u32 lcoef[2];                /* the row coefficient of a linear side */
    int vec[2];                  /* a linear side loaded 4 contiguous, 16-byte aligned elements per lane */
} KPerm;

typedef struct {
    char name[48];
    TileCfg cfg;
    u32 pad_a, pad_b;      /* LDS row padding (floats) of the A and B stages */
    u32 splits;
    u32 splits_want;       /* split count asked for; splits is what the K chunks give */
    u32 depth;             /* stages of global loads in flight ahead of the math (1 or 2) */
    u32 nw;                /* direct kernel: waves per block, each taking every nw-th K step */
    u32 kchunk;
    u32 tiles_m, tiles_n;
    KPerm kp;
    int swap;              /* output m-contiguous: MFMA blocks computed transposed so that lanes
                              run along m in the epilogue (coalesced stores) */
    int pack;              /* the B side is first copied into a K x N row-major buffer in the
                              reordered k order (a small operand with scattered loads) */
    KPerm kpo;             /* the K-reordered plan before packing (the pack kernel's loads) */
    u32 ske;               /* skinny: K walked in blocks of ske (a digit boundary of both sides'
                              k offsets), whose in-block offsets are constants; 0 = per k */
    u64 skmax;             /* skinny: largest index the row side's loads form (unchecked loads
                              when the buffer holds it), or ~0 */
    u32 skbuf;             /* skinny: the buffer of the row side (1 + leaf) */
    u32 red_mg;            /* outer-product reduction: rows per group */
    u64 red_max[2];        /* ... the largest index each side forms (unchecked loads) */
    u32 red_buf[2];        /* ... and the buffer it reads (1 + leaf) */
    u32 tail_full;         /* wave tile: tiles run whole, tail_s per workgroup (a multiple of the SIMD
                              count); each of the rest is split over the tail_s waves of a workgroup */
    u32 tail_s;            /* ... in K chunks, added through LDS; 0 = one wave per workgroup, no split */
    u32 tail_pf;           /* ... whose k-pairs go through a ring of tail_pf loads */
    int dvec[2];           /* direct kernel: side s read 4 consecutive k per lane with one 16-byte load */
    u32 dvec_buf[2];       /* ... from this buffer (p<b>) */
    int comb;              /* direct and outer-product kernels: split-K partials combined in the
                              same launch by the last split's workgroup through the combine words */
    int prio;              /* LDS tiles: the wave's priority raised over its stage's fragment reads
                              and MFMAs */
} GemmPlan;

#define GEMM_THREADS 256
/* Workgroups of the 64x64 tile a compute unit holds at once: four waves
 * each, about 34 KB of LDS (two stages) and at most 128 VGPRs, so LDS and
 * registers both stop at four. */
#define GEMM_SLOTS_PER_CU 4u

static u32 dense_cus(void) { return hipb.n_cu ? hipb.n_cu : 256u; }

/* lanes of an LDS tile's workgroup: one wave per gm x gn position (the
 * kernels without LDS tiles plan their loaders against GEMM_THREADS) */
static u32 lds_threads(const TileCfg *cf) { return cf->direct ? GEMM_THREADS : 64u * cf->gm * cf->gn; }

/* workgroup size of a plan's main kernel */
static u32 dense_threads(const GemmPlan *pl) {
    if (pl->cfg.direct == 4) return 64u * (pl->tail_s ? pl->tail_s : 1u);
    return pl->cfg.direct == 3 ? GEMM_THREADS : pl->cfg.direct ? 64u * pl->nw : lds_threads(&pl->cfg);
}

/* wave tile: k-pairs of fragments in flight (a divisor of the K-pair count) */
static u32 wave_ring(u32 kpairs) {
    static const u32 pf[] = {8, 6, 4, 3, 2, 1};
    for (u32 i = 0; i < sizeof pf / sizeof pf[0]; i++)
        if (kpairs % pf[i] == 0) return pf[i];
    return 1;
}
#define SUM_WAVE_MIN_SPLITS 16   /* split-K sums this long use a wavefront per output, */
#define SUM_WAVE_MAX_OUTPUTS 8192 /* unless there are enough outputs for a lane each */

/* Split-K sum shape: a wavefront per output for few outputs with long sums
 * (its lanes read one output's partials, strided), else a lane per output
 * (consecutive lanes read consecutive partials, coalesced). Both add the
 * splits in a fixed order. */
static int sum_per_wave(const GemmPlan *pl, u64 outputs) {
    return pl->splits >= SUM_WAVE_MIN_SPLITS && outputs < SUM_WAVE_MAX_OUTPUTS;
}

/* f(gid) (var 0) or g(r) (var 1) part of a separable operand index */
static void emit_sep_fn(DSB *s, const char *name, const Aff *a, u8 var) {
    dsb_put(s, "__device__ __forceinline__ u32 %s(u32 x) {\n  return %uu", name, var == 0 ? a->cst : 0u);
    for (u32 t = 0; t < a->n; t++) {
        if (a->d[t].var != var) continue;
        if (a->d[t].mod) dsb_put(s, " + ((x / %uu) %% %uu) * %uu", a->d[t].div, a->d[t].mod, a->coef[t]);
        else dsb_put(s, " + (x / %uu) * %uu", a->d[t].div, a->coef[t]);
    }
    dsb_put(s, ";\n}\n");
}

static const char *ld_name(u32 dt) {
    return dt == DTYPE_F16 ? "ld_f16" : dt == DTYPE_I32 ? "ld_i32" : dt == DTYPE_U32 ? "ld_u32" : "ld_f32";
}

/* Loader lane map for one operand: x in [0, BX) along the tile's M or N side,
 * k in [0, BK). k-major operands put 16 consecutive lanes on consecutive k,
 * the others put consecutive lanes on consecutive x (coalesced either way). */
static void emit_map(DSB *s, int kmajor, u32 bx, const TileCfg *cf, const char *xname) {
    const u32 bk = cf->bk, T = lds_threads(cf);
    if (kmajor) {
        if (bk == 16)
            dsb_put(s, "const u32 kk = tid & 15u, %s = (tid >> 4) + e * %uu;", xname, T / 16u);
        else
            dsb_put(s, "const u32 kk = (tid & 15u) + (e %% %uu) * 16u, %s = (tid >> 4) + (e / %uu) * %uu;", bk / 16,
                    xname, bk / 16, T / 16u);
    } else if (bx == T) {
        dsb_put(s, "const u32 %s = tid, kk = e;", xname);
    } else {
        dsb_put(s, "const u32 %s = tid %% %uu, kk = tid / %uu + e * %uu;", xname, bx, bx, T / bx);
    }
}

static void out_store_fn(const UOpKernel *k, const Contraction *ct, char *fb, size_t fblen, const char **st) {
    u32 bits;
    memcpy(&bits, &ct->init, 4);
    snprintf(fb, fblen, "__uint_as_float(0x%08xu)", bits);
    *st = k->out_dtype == DTYPE_F16 ? "st_f16" : k->out_dtype == DTYPE_I32 ? "st_i32"
          : k->out_dtype == DTYPE_U32 ? "st_u32" : "st_f32";
}

/* A fused epilogue (set only while a fused module is generated): the
 * consumer's device function epi_, the main kernel's extra parameters for
 * the consumer's buffers (q<b>, qc<b>) and the call made after every output
 * store with the stored value v_ at output index o_. */
static const char *g_epi_src, *g_epi_params, *g_epi_call;

/* "st(p0, c0, idx, val);" or, with a fused epilogue, the same store followed
 * by the consumer's epilogue for that output */
static void emit_out_store(DSB *s, const char *indent, const char *st, const char *idx, const char *val) {
    if (!g_epi_call) {
        dsb_put(s, "%s%s(p0, c0, %s, %s);\n", indent, st, idx, val);
        return;
    }
    dsb_put(s, "%s{ const u32 o_ = %s; const float v_ = %s; %s(p0, c0, o_, v_); %s; }\n", indent, idx, val, st,
            g_epi_call);
}

/* Closes the epilogue opened by the caller (inside `if (m < M && n < N) {`
 * with the accumulator value c[v]): stores the result (or the split's partial
 * into the workspace), closes the kernel, and emits the split-K sum kernel. */
static void emit_sum_kernel(DSB *s_, const UOpKernel *k, const Contraction *ct, const GemmPlan *pl);

static void emit_store_tail(DSB *sp, const UOpKernel *k, const Contraction *ct, const GemmPlan *pl) {
    DSB *s_ = sp;
    char fb[64];
    const char *st;
    out_store_fn(k, ct, fb, sizeof fb, &st);
    if (pl->comb)
        /* the direct kernel's in-launch combine (the words taken into cb_) */
        dsb_put(s_, "        if (sl_ == nullptr) {\n"
                    "          ws[((unsigned long long)spl * M + m) * N + n] = c[v];\n"
                    "        } else if (spl != S - 1u) {\n"
                    "          comb_pub(sl_ + (unsigned long long)spl * MN + m * N + n, c[v]);\n"
                    "        } else {\n"
                    "          float a_ = 0.0f;\n"
                    "          #pragma unroll\n"
                    "          for (u32 sp = 0; sp + 1u < S; sp++) a_ = a_ + cb_[(sp * 16u + v) * 64u + lane];\n"
                    "          %s(p0, c0, gid_m(m) + gid_n(n), %s + (a_ + c[v]));\n"
                    "        }\n", st, fb);
    else if (pl->splits > 1 && pl->swap)
        dsb_put(s_, "        ws[((unsigned long long)spl * N + n) * M + m] = c[v];\n");
    else if (pl->splits > 1)
        dsb_put(s_, "        ws[((unsigned long long)spl * M + m) * N + n] = c[v];\n");
    else {
        char val[96];
        snprintf(val, sizeof val, "%s + c[v]", fb);
        emit_out_store(s_, "        ", st, "gid_m(m) + gid_n(n)", val);
    }
    dsb_put(s_, "      }\n    }\n  }\n}\n");
    emit_sum_kernel(s_, k, ct, pl);
}

/* The split-K sum kernel (<name>_sum) of a plan with splits > 1: adds the
 * splits' partials ws[split][m][n] (or [split][n][m] with swap) per output in
 * a fixed order and stores init + the sum. */
static void emit_sum_kernel(DSB *s_, const UOpKernel *k, const Contraction *ct, const GemmPlan *pl) {
    char fb[64];
    const char *st;
    out_store_fn(k, ct, fb, sizeof fb, &st);
    const u32 M = ct->M, N = ct->N;
    if (pl->splits <= 1) return;
    if (sum_per_wave(pl, (u64)M * N)) {
        /* many splits: one wavefront per output; lane l adds splits l, l+64, ...
         * in order, then a fixed shuffle tree (deterministic) */
        dsb_put(s_, "extern \"C\" __global__ __launch_bounds__(256) void %s_sum(char* p0, u32 c0, const float* ws) {\n"
                    "  const unsigned long long t = (unsigned long long)blockIdx.x * 4u + (threadIdx.x >> 6);\n"
                    "  const u32 lane = threadIdx.x & 63u;\n"
                    "  if (t >= %lluull) return;\n"
                    "  const u32 %s = (u32)(t / %uu), %s = (u32)(t %% %uu);\n"
                    "  float a = 0.0f;\n"
                    "  for (u32 s = lane; s < %uu; s += 64u) a = a + ws[(unsigned long long)s * %lluull + t];\n"
                    "  a = wsum(a);\n"
                    "  if (lane == 0u) %s(p0, c0, gid_m(m) + gid_n(n), %s + a);\n}\n",
                pl->name, (unsigned long long)M * N, pl->swap ? "n" : "m", pl->swap ? M : N, pl->swap ? "m" : "n",
                pl->swap ? M : N, pl->splits, (unsigned long long)M * N, st, fb);
    } else {
        /* many outputs: a workgroup per 64 outputs, lane l of wave w adding
         * splits w, w+4, ... of output l in order; the 4 wave sums are then
         * added in a fixed order (four times the workgroups of a lane per
         * output over all splits, which is bound by its serial loads) */
        dsb_put(s_, "extern \"C\" __global__ __launch_bounds__(256) void %s_sum(char* p0, u32 c0, const float* ws) {\n"
                    "  __shared__ float part_[3][64];\n"
                    "  const u32 lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;\n"
                    "  const unsigned long long t = (unsigned long long)blockIdx.x * 64u + lane;\n"
                    "  float a = 0.0f;\n"
                    "  if (t < %lluull) {\n"
                    "    #pragma unroll 4\n"
                    "    for (u32 s = wave; s < %uu; s += 4u) a = a + ws[(unsigned long long)s * %lluull + t];\n"
                    "  }\n"
                    "  if (wave > 0u) part_[wave - 1u][lane] = a;\n"
                    "  __syncthreads();\n"
                    "  if (wave > 0u || t >= %lluull) return;\n"
                    "  a = ((a + part_[0][lane]) + part_[1][lane]) + part_[2][lane];\n"
                    "  const u32 %s = (u32)(t / %uu), %s = (u32)(t %% %uu);\n"
                    "  %s(p0, c0, gid_m(m) + gid_n(n), %s + a);\n}\n",
                pl->name, (unsigned long long)M * N, pl->splits, (unsigned long long)M * N, (unsigned long long)M * N,
                pl->swap ? "n" : "m", pl->swap ? M : N, pl->swap ? "m" : "n", pl->swap ? M : N, st, fb);
    }
}

/* Operand element (m, k) of one side: separable loads add a row base and a
 * k offset; other operands run their own KOp program. */
static void emit_operand_expr(DSB *s, const UOpKernel *k, const Contraction *ct, int side, const char *base,
                              const char *x, const char *kv) {
    if (ct->sep[side]) {
        dsb_put(s, "%s(p%u, c%u, %s + koff_%c(%s))", ld_name(ct->sep_dt[side]), ct->sep_buf[side], ct->sep_buf[side],
                base, side ? 'q' : 'p', kv);
    } else {
        dsb_put(s, "operand_%c(gid_%c(%s), %s, ", side ? 'q' : 'p', side ? 'n' : 'm', x, kv);
        emit_args(s, k->n_leaves);
        dsb_put(s, ")");
    }
}

/* Outer-product reduction kernel (CFG_RED): workgroup (g, s) takes rows
 * [g*MG, g*MG + MG) and k in chunk s; lane l of wave w walks k = kbeg + 64w + l,
 * kbeg + 256 + 64w + l, ... in order. The MG*N sums of the 64 lanes are added
 * through an LDS transpose, 32 sums at a time (lane j adds sum j over the
 * lanes in order; a shuffle tree per value, every shuffle waited for, took
 * 12 of 19 us on LeNet-5's conv1 dW); wave 0 then adds the four waves in
 * order and writes the chunk's partials for the split-K sum. Loads are
 * unchecked: the dispatch sees that both buffers hold the largest index
 * their sides form. Deterministic. */
static void emit_red_kernel(DSB *s, const UOpKernel *k, const Contraction *ct, const GemmPlan *pl) {
    const u32 M = ct->M, N = ct->N, K = ct->K, MG = pl->red_mg, V = MG * N;
    const u32 VP = (V + 63) / 64 * 64;
    dsb_put(s, "extern \"C\" __global__ __launch_bounds__(256) void %s(", pl->name);
    emit_params(s, k->n_leaves);
    dsb_put(s, pl->comb ? ", float* ws, unsigned long long* sl_) {\n" : ", float* ws) {\n");
    /* the loads as buffer loads: the lane's k offset in a VGPR and the
     * row's base (uniform) in an SGPR, so that no load needs a 64-bit
     * address of its own; the byte offsets fit 32 bits (the dispatch checks
     * that the buffers hold every index formed) */
    const int bufld = pl->red_max[0] < (1ull << 30) && pl->red_max[1] < (1ull << 30);
    dsb_put(s,
            "  constexpr u32 M = %uu, N = %uu, K = %uu, MG = %uu, V = %uu, VP = %uu, KCH = %uu;\n"
            "  const u32 lane = threadIdx.x & 63u, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);\n"
            "  const u32 m0 = blockIdx.x * MG, spl = blockIdx.y;\n",
            M, N, K, MG, V, VP, pl->kchunk);
    for (int sd = 0; sd < 2; sd++) {
        const u32 b = ct->sep_buf[sd];
        const char S = sd ? 'Q' : 'P';
        if (bufld)
            dsb_put(s, "  const __amdgpu_buffer_rsrc_t r%c_ = __builtin_amdgcn_make_buffer_rsrc((void*)p%u, (short)0,\n"
                       "      (int)((unsigned long long)c%u * 4ull < 0xFFFFFFFFull ? c%u * 4u : 0xFFFFFFFFu), 0x00020000);\n"
                       "  auto LD%c_ = [&](u32 base, u32 off) {\n"
                       "    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r%c_, (int)(off * 4u), (int)(base * 4u), 0));\n"
                       "  };\n", S, b, b, b, S, S);
        else
            dsb_put(s, "  auto LD%c_ = [&](u32 base, u32 off) { return ld_f32_u(p%u, base + off); };\n", S, b);
    }
    dsb_put(s,
            "  const u32 kbeg = spl * KCH, kend = (kbeg + KCH < K) ? kbeg + KCH : K;\n"
            "  u32 rb[MG];\n"
            "  #pragma unroll\n"
            "  for (u32 i = 0; i < MG; i++) rb[i] = rowb_p(gid_m(m0 + i < M ? m0 + i : M - 1u));\n"
            "  float acc[V];\n"
            "  #pragma unroll\n"
            "  for (u32 j = 0; j < V; j++) acc[j] = 0.0f;\n"
            "  #pragma unroll 2\n"
            "  for (u32 k = kbeg + wave * 64u + lane; k < kend; k += 256u) {\n"
            "    const u32 op = koff_p(k), oq = koff_q(k);\n"
            "    float a[MG], b[N];\n"
            "    #pragma unroll\n"
            "    for (u32 i = 0; i < MG; i++) a[i] = (m0 + i < M) ? LDP_(rb[i], op) : 0.0f;\n"
            "    #pragma unroll\n"
            "    for (u32 n = 0; n < N; n++) b[n] = LDQ_(rowb_q(gid_n(n)), oq);\n"
            "    #pragma unroll\n"
            "    for (u32 i = 0; i < MG; i++)\n"
            "      #pragma unroll\n"
            "      for (u32 n = 0; n < N; n++) acc[i * N + n] = fmaf(a[i], b[n], acc[i * N + n]);\n"
            "  }\n"
            "  /* each chunk of 32 sums through LDS: lane l writes its 32 values as\n"
            "   * column l, lane j < 32 adds row j over the 64 lanes in order */\n"
            "  constexpr u32 NQ = (V + 31u) / 32u;\n"
            "  __shared__ float tr_[4][32][65];\n"
            "  __shared__ float tot_[4][NQ * 32u];\n"
            "  #pragma unroll\n"
            "  for (u32 q = 0; q < NQ; q++) {\n"
            "    #pragma unroll\n"
            "    for (u32 j = 0; j < 32u; j++) tr_[wave][j][lane] = (32u * q + j < V) ? acc[32u * q + j] : 0.0f;\n"
            "    __syncthreads();\n"
            "    if (lane < 32u) {\n"
            "      float t = 0.0f;\n"
            "      #pragma unroll 16\n"
            "      for (u32 i = 0; i < 64u; i++) t = t + tr_[wave][lane][i];\n"
            "      tot_[wave][32u * q + lane] = t;\n"
            "    }\n"
            "    __syncthreads();\n"
            "  }\n"
            "  __syncthreads();\n");
    if (pl->comb) {
        char fb[64];
        const char *st;
        out_store_fn(k, ct, fb, sizeof fb, &st);
        /* in-launch combine: the splits but the last publish their partials
         * (word s*M*N + m*N + n); the last split's 256 threads take the other
         * splits' words into LDS (the transpose buffer, free by now), all of a
         * thread's words peeked at once and cleared after, and lane idx of wave 0
         * adds output idx's partials in split order, its own last */
        dsb_put(s,
                "  constexpr u32 S = %uu, MN = M * N, NTK = (S - 1u) * V;\n"
                "  if (sl_ != nullptr) {\n"
                "    if (spl != S - 1u) {\n"
                "      if (wave > 0u) return;\n"
                "      for (u32 idx = lane; idx < V; idx += 64u) {\n"
                "        const float t = ((tot_[0][idx] + tot_[1][idx]) + tot_[2][idx]) + tot_[3][idx];\n"
                "        if (m0 + idx / N < M) comb_pub(sl_ + (unsigned long long)spl * MN + m0 * N + idx, t);\n"
                "      }\n"
                "      return;\n"
                "    }\n"
                "    float* cb_ = &tr_[0][0][0];\n"
                "    constexpr u32 NB = (NTK + 255u) / 256u;\n"
                "    unsigned long long w_[NB];\n"
                "    #pragma unroll\n"
                "    for (u32 u = 0; u < NB; u++) {\n"
                "      const u32 j = threadIdx.x + 256u * u, sp = j / V, idx = j %% V;\n"
                "      w_[u] = (j < NTK && m0 + idx / N < M) ? comb_peek(sl_ + (unsigned long long)sp * MN + m0 * N + idx)\n"
                "                                          : (1ull << 32);\n"
                "    }\n"
                "    #pragma unroll\n"
                "    for (u32 u = 0; u < NB; u++) {\n"
                "      const u32 j = threadIdx.x + 256u * u, sp = j / V, idx = j %% V;\n"
                "      if (j < NTK && m0 + idx / N < M) cb_[j] = comb_ready(sl_ + (unsigned long long)sp * MN + m0 * N + idx, w_[u]);\n"
                "    }\n"
                "    #pragma unroll\n"
                "    for (u32 u = 0; u < NB; u++) {\n"
                "      const u32 j = threadIdx.x + 256u * u, sp = j / V, idx = j %% V;\n"
                "      if (j < NTK && m0 + idx / N < M) comb_clear(sl_ + (unsigned long long)sp * MN + m0 * N + idx);\n"
                "    }\n"
                "    __syncthreads();\n"
                "    if (wave > 0u) return;\n"
                "    for (u32 idx = lane; idx < V; idx += 64u) {\n"
                "      const u32 i = idx / N, n = idx %% N, m = m0 + i;\n"
                "      if (m >= M) continue;\n"
                "      float a = 0.0f;\n"
                "      #pragma unroll\n"
                "      for (u32 sp = 0; sp + 1u < S; sp++) a = a + cb_[sp * V + idx];\n"
                "      a = a + (((tot_[0][idx] + tot_[1][idx]) + tot_[2][idx]) + tot_[3][idx]);\n"
                "      %s(p0, c0, gid_m(m) + gid_n(n), %s + a);\n"
                "    }\n"
                "    return;\n"
                "  }\n",
                pl->splits, st, fb);
    }
    dsb_put(s,
            "  if (wave > 0u) return;\n"
            "  for (u32 idx = lane; idx < V; idx += 64u) {\n"
            "    const float t = ((tot_[0][idx] + tot_[1][idx]) + tot_[2][idx]) + tot_[3][idx];\n"
            "    const u32 i = idx / N, n = idx %% N, m = m0 + i;\n"
            "    if (m < M) ws[((unsigned long long)spl * M + m) * N + n] = t;\n"
            "  }\n"
            "}\n");
}

/* Skinny kernel (CFG_SKINNY): lane = row m, all N column sums in registers.
 * The small side (K x N, at most SKINNY_MAX_KN elements) is first copied by
 * the workgroup into LDS as K rows of N, so that each k's row is a broadcast
 * LDS read (scalar loads of it, one k at a time, each waited for, ran 5x
 * slower). Wave w of the workgroup takes k in [w*KCW, (w+1)*KCW), its lanes
 * loading SKU operand elements ahead of the FMAs of the previous SKU (one
 * set of 8 loads waited for before its FMAs: 32 us on LeNet-5's conv2 dX,
 * 50176x6x400); wave 0 then adds the other waves' sums in wave order
 * (deterministic). */
static void emit_skinny_kernel(DSB *s, const UOpKernel *k, const Contraction *ct, const GemmPlan *pl) {
    const u32 M = ct->M, N = ct->N, K = ct->K, KW = pl->nw;
    const u32 kcw = (K + KW - 1) / KW;
    char fb[64];
    const char *st;
    out_store_fn(k, ct, fb, sizeof fb, &st);
    dsb_put(s, "extern \"C\" __global__ __launch_bounds__(%u) void %s(", 64u * KW, pl->name);
    emit_params(s, k->n_leaves);
    dsb_put(s, ", float* ws%s) {\n", g_epi_params ? g_epi_params : "");
    dsb_put(s,
            "  constexpr u32 M = %uu, N = %uu, K = %uu, KW = %uu, KCW = %uu, SKU = %uu;\n"
            "  __shared__ float bs_[K * N];\n"
            "  for (u32 i = threadIdx.x; i < K * N; i += 64u * KW) {\n"
            "    const u32 k = i / N, n = i %% N;\n"
            "    bs_[i] = ",
            M, N, K, KW, kcw, 16u);
    emit_operand_expr(s, k, ct, 1, "rowb_q(gid_n(n))", "n", "k");
    dsb_put(s, ";\n"
               "  }\n"
               "  __syncthreads();\n"
               "  const u32 lane = threadIdx.x & 63u, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);\n"
               "  const u32 m = blockIdx.x * 64u + lane, ma = m < M ? m : M - 1u;\n"
               "  const u32 kbeg = wave * KCW, kend = (kbeg + KCW < K) ? kbeg + KCW : K;\n"
               "  float acc[N];\n"
               "  #pragma unroll\n"
               "  for (u32 n = 0; n < N; n++) acc[n] = 0.0f;\n");
    if (ct->sep[0]) dsb_put(s, "  const u32 bA = rowb_p(gid_m(ma));\n");
    if (pl->ske) {
        /* K in blocks of E: the block's row-side offset once, the in-block
         * offsets koff_p(i) constants; E loads in flight, then E*N FMAs with
         * the block's rows of the small side from LDS */
        const u32 E = pl->ske, nblk = K / E, bpw = (nblk + KW - 1) / KW;
        char ldx[96];
        if (pl->skmax != ~0ull)   /* the dispatch checks the buffer holds skmax; the block's
                                   * 64-bit base once, its loads at constant offsets from it */
            snprintf(ldx, sizeof ldx, "pa_[koff_p(i)]");
        else
            snprintf(ldx, sizeof ldx, "%s(p%u, c%u, oa + koff_p(i))", ld_name(ct->sep_dt[0]), ct->sep_buf[0],
                     ct->sep_buf[0]);
        dsb_put(s, "  constexpr u32 E = %uu, NBLK = %uu, BPW = %uu;\n"
                   "  const u32 bbeg = wave * BPW, bend = (bbeg + BPW < NBLK) ? bbeg + BPW : NBLK;\n"
                   "  for (u32 bk = bbeg; bk < bend; bk++) {\n"
                   "    const u32 kb = bk * E, oa = bA + koff_p(kb);\n"
                   "    const float* pa_ = (const float*)p%u + oa;\n"
                   "    float a[E];\n"
                   "    #pragma unroll\n"
                   "    for (u32 i = 0; i < E; i++) a[i] = %s;\n"
                   "    const float* br = bs_ + kb * N;\n"
                   "    #pragma unroll\n"
                   "    for (u32 i = 0; i < E; i++)\n"
                   "      #pragma unroll\n"
                   "      for (u32 n = 0; n < N; n++) acc[n] = fmaf(a[i], br[i * N + n], acc[n]);\n"
                   "  }\n",
                E, nblk, bpw, ct->sep_buf[0], ldx);
    } else {
    /* two register sets of SKU operand elements: the next set's loads are
     * issued before the current set's FMAs */
    dsb_put(s, "  auto fetch = [&](u32 k0, float (&a)[SKU]) {\n"
               "    #pragma unroll\n"
               "    for (u32 u = 0; u < SKU; u++) {\n"
               "      const u32 k = (k0 + u < kend) ? k0 + u : kbeg;\n"
               "      const float v = ");
    emit_operand_expr(s, k, ct, 0, "bA", "ma", "k");
    dsb_put(s, ";\n"
               "      a[u] = (k0 + u < kend) ? v : 0.0f;\n"
               "    }\n"
               "  };\n"
               "  auto fmas = [&](u32 k0, const float (&a)[SKU]) {\n"
               "    #pragma unroll\n"
               "    for (u32 u = 0; u < SKU; u++) {\n"
               "      const float* br = bs_ + ((k0 + u < kend) ? k0 + u : kbeg) * N;\n"
               "      #pragma unroll\n"
               "      for (u32 n = 0; n < N; n++) acc[n] = fmaf(a[u], br[n], acc[n]);\n"
               "    }\n"
               "  };\n"
               "  float a0[SKU], a1[SKU];\n"
               "  if (kbeg < kend) fetch(kbeg, a0);\n"
               "  for (u32 k0 = kbeg; k0 < kend; k0 += 2u * SKU) {\n"
               "    if (k0 + SKU < kend) fetch(k0 + SKU, a1);\n"
               "    fmas(k0, a0);\n"
               "    if (k0 + SKU >= kend) break;\n"
               "    if (k0 + 2u * SKU < kend) fetch(k0 + 2u * SKU, a0);\n"
               "    fmas(k0 + SKU, a1);\n"
               "  }\n");
    }
    if (KW > 1)
        dsb_put(s, "  __shared__ float part_[KW - 1u][N][64];\n"
                   "  if (wave > 0u) {\n"
                   "    #pragma unroll\n"
                   "    for (u32 n = 0; n < N; n++) part_[wave - 1u][n][lane] = acc[n];\n"
                   "  }\n"
                   "  __syncthreads();\n"
                   "  if (wave > 0u) return;\n"
                   "  for (u32 w = 0; w + 1u < KW; w++)\n"
                   "    #pragma unroll\n"
                   "    for (u32 n = 0; n < N; n++) acc[n] = acc[n] + part_[w][n][lane];\n");
    dsb_put(s, "  if (m < M) {\n"
               "    #pragma unroll\n"
               "    for (u32 n = 0; n < N; n++)\n");
    char val[96];
    snprintf(val, sizeof val, "%s + acc[n]", fb);
    emit_out_store(s, "      ", st, "gid_m(m) + gid_n(n)", val);
    dsb_put(s, "  }\n}\n");
}

/* Direct kernel: a side whose k offset is k itself (one loop digit, unit
 * coefficient, no wrap below K) and whose row bases are multiples of 4 reads
 * 4 consecutive k per lane as one 16-byte load, for K a multiple of 4 (then
 * a group of 4 never straddles the end of K or of a split's chunk). The
 * buffer's 16-byte alignment is checked when the kernel is dispatched. */
static int direct_vec_side(const Contraction *ct, int side) {
    if (!ct->sep[side] || ct->sep_dt[side] != DTYPE_F32 || ct->K % 4u || hipb.dense_novec) return 0;
    const Aff *a = &ct->sep_aff[side];
    if (a->cst % 4u) return 0;
    u32 nr = 0;
    for (u32 t = 0; t < a->n; t++) {
        if (a->d[t].var == 1) {
            if (a->d[t].div != 1u || a->coef[t] != 1u || (a->d[t].mod && a->d[t].mod < ct->K)) return 0;
            nr++;
        } else if (a->coef[t] % 4u) {
            return 0;
        }
    }
    return nr == 1;
}

/* Direct kernel: a workgroup of 4 waves owns one 32x32 output block; the
 * waves take alternate KU-long steps of the workgroup's K range, each wave
 * keeping 4 independent accumulator chains and loading the next step's
 * operands before it multiplies the current ones. The 4 waves' partial blocks
 * are summed through LDS in a fixed order. */
static void emit_direct_kernel(DSB *s, const UOpKernel *k, const Contraction *ct, const GemmPlan *pl) {
    const u32 M = ct->M, N = ct->N, K = ct->K, KU = pl->cfg.bk;
    const u32 blocks = pl->tiles_m * pl->tiles_n;
    dsb_put(s, "extern \"C\" __global__ __launch_bounds__(%u) void %s(", 64u * pl->nw, pl->name);
    emit_params(s, k->n_leaves);
    if (pl->comb) dsb_put(s, ", float* ws, unsigned long long* sl_) {\n");
    else dsb_put(s, ", float* ws%s) {\n", g_epi_params ? g_epi_params : "");
    dsb_put(s,
            "  constexpr u32 M = %uu, N = %uu, K = %uu, TN = %uu, BLOCKS = %uu, KCH = %uu, KU = %uu, NW = %uu;\n"
            "  const u32 lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;\n"
            "  const u32 blk = blockIdx.x;\n"
            "  if (blk >= BLOCKS) return;\n"
            "  const u32 m0 = (blk / TN) * 32u, n0 = (blk %% TN) * 32u;\n"
            "  const u32 spl = blockIdx.y;\n"
            "  const u32 kbeg = spl * KCH;\n"
            "  const u32 kend = (kbeg + KCH < K) ? kbeg + KCH : K;\n"
            "  const u32 i = lane & 31u, kh = lane >> 5;\n"
            "  const u32 ma = m0 + i, nb = n0 + i;\n",
            M, N, K, pl->tiles_n, blocks, pl->kchunk, KU, pl->nw);
    if (ct->sep[0]) dsb_put(s, "  const u32 bA = ma < M ? rowb_p(gid_m(ma)) : 0u;\n");
    if (ct->sep[1]) dsb_put(s, "  const u32 bB = nb < N ? rowb_q(gid_n(nb)) : 0u;\n");
    if (pl->dvec[0] || pl->dvec[1]) {
        /* MFMA step q = 4j + t takes k = k0 + 8j + 4h + t in the lanes of
         * half h: a lane's 4 k of a group of 8 are consecutive */
        dsb_put(s,
                "  float a[KU / 2u], b[KU / 2u];\n"
                "  auto fetch = [&](u32 k0) {\n"
                "    #pragma unroll\n"
                "    for (u32 j = 0; j < KU / 8u; j++) {\n"
                "      const u32 kk = k0 + 8u * j + 4u * kh;\n");
        for (int side = 0; side < 2; side++) {
            const char *arr = side ? "b" : "a", *base = side ? "bB" : "bA", *x = side ? "nb" : "ma",
                       *lim = side ? "N" : "M";
            if (pl->dvec[side]) {
                dsb_put(s,
                        "      {\n"
                        "        float4 v4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);\n"
                        "        if (%s < %s && kk < kend) v4 = ld4(p%u, c%u, %s + kk);\n"
                        "        %s[4u * j] = v4.x; %s[4u * j + 1u] = v4.y; %s[4u * j + 2u] = v4.z; %s[4u * j + 3u] = v4.w;\n"
                        "      }\n",
                        x, lim, ct->sep_buf[side], ct->sep_buf[side], base, arr, arr, arr, arr);
            } else {
                dsb_put(s,
                        "      #pragma unroll\n"
                        "      for (u32 t = 0; t < 4u; t++) {\n"
                        "        const u32 k = kk + t;\n"
                        "        const float v = ");
                emit_operand_expr(s, k, ct, side, base, x, "k");
                dsb_put(s, ";\n        %s[4u * j + t] = __uint_as_float(__float_as_uint(v) & ((%s < %s && k < kend) ? "
                           "0xFFFFFFFFu : 0u));\n      }\n", arr, x, lim);
            }
        }
        dsb_put(s, "    }\n  };\n");
    } else {
        dsb_put(s,
                "  float a[KU / 2u], b[KU / 2u];\n"
                "  auto fetch = [&](u32 k0) {\n"
                "    #pragma unroll\n"
                "    for (u32 q = 0; q < KU / 2u; q++) {\n"
                "      const u32 k = k0 + 2u * q + kh;\n"
                "      const float va = ");
        emit_operand_expr(s, k, ct, 0, "bA", "ma", "k");
        dsb_put(s, ";\n      const float vb = ");
        emit_operand_expr(s, k, ct, 1, "bB", "nb", "k");
        dsb_put(s, ";\n      a[q] = __uint_as_float(__float_as_uint(va) & ((ma < M && k < kend) ? 0xFFFFFFFFu : 0u));\n"
                   "      b[q] = __uint_as_float(__float_as_uint(vb) & ((nb < N && k < kend) ? 0xFFFFFFFFu : 0u));\n"
                   "    }\n  };\n");
    }
    dsb_put(s, "  f32x16 acc0 = {0}, acc1 = {0}, acc2 = {0}, acc3 = {0};\n"
               "  u32 k0 = kbeg + wave * KU;\n"
               "  if (k0 < kend) fetch(k0);\n"
               "  while (k0 < kend) {\n"
               "    float ca[KU / 2u], cb[KU / 2u];\n"
               "    #pragma unroll\n"
               "    for (u32 q = 0; q < KU / 2u; q++) { ca[q] = a[q]; cb[q] = b[q]; }\n"
               "    const u32 kn = k0 + NW * KU;\n"
               "    if (kn < kend) fetch(kn);\n"
               "    #pragma unroll\n"
               "    for (u32 q = 0; q < KU / 2u; q += 4u) {\n"
               "      acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(ca[q], cb[q], acc0, 0, 0, 0);\n"
               "      acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(ca[q + 1u], cb[q + 1u], acc1, 0, 0, 0);\n"
               "      acc2 = __builtin_amdgcn_mfma_f32_32x32x2f32(ca[q + 2u], cb[q + 2u], acc2, 0, 0, 0);\n"
               "      acc3 = __builtin_amdgcn_mfma_f32_32x32x2f32(ca[q + 3u], cb[q + 3u], acc3, 0, 0, 0);\n"
               "    }\n"
               "    k0 = kn;\n"
               "  }\n"
               "  f32x16 acc = (acc0 + acc1) + (acc2 + acc3);\n"
               "  __shared__ float part_[NW - 1u][16][64];\n"
               "  if (wave > 0u) {\n"
               "    #pragma unroll\n"
               "    for (u32 v = 0; v < 16u; v++) part_[wave - 1u][v][lane] = acc[v];\n"
               "  }\n"
               "  __syncthreads();\n");
    if (pl->comb)
        /* in-launch combine: the last split's threads take the other splits'
         * words of the block's 1024 outputs into LDS (slot s*1024 + v*64 +
         * lane, the output of accumulator v in lane `lane`), all of a thread's
         * words peeked at once; the epilogue adds them in split order */
        dsb_put(s,
               "  constexpr u32 S = %uu, MN = M * N, NTK = (S - 1u) * 1024u;\n"
               "  __shared__ float cb_[NTK];\n"
               "  if (sl_ != nullptr && spl == S - 1u) {\n"
               "    constexpr u32 NB = (NTK + NW * 64u - 1u) / (NW * 64u);\n"
               "    unsigned long long w_[NB];\n"
               "    u32 o_[NB];\n"
               "    #pragma unroll\n"
               "    for (u32 u = 0; u < NB; u++) {\n"
               "      const u32 j = threadIdx.x + NW * 64u * u, l = j & 1023u, v = l >> 6, ln = l & 63u;\n"
               "      const u32 m = m0 + 8u * (v >> 2) + 4u * (ln >> 5) + (v & 3u), n = n0 + (ln & 31u);\n"
               "      o_[u] = (j < NTK && m < M && n < N) ? m * N + n : ~0u;\n"
               "      w_[u] = o_[u] != ~0u ? comb_peek(sl_ + (unsigned long long)(j >> 10) * MN + o_[u]) : (1ull << 32);\n"
               "    }\n"
               "    #pragma unroll\n"
               "    for (u32 u = 0; u < NB; u++) {\n"
               "      const u32 j = threadIdx.x + NW * 64u * u;\n"
               "      if (o_[u] != ~0u) cb_[j] = comb_ready(sl_ + (unsigned long long)(j >> 10) * MN + o_[u], w_[u]);\n"
               "    }\n"
               "    #pragma unroll\n"
               "    for (u32 u = 0; u < NB; u++) {\n"
               "      const u32 j = threadIdx.x + NW * 64u * u;\n"
               "      if (o_[u] != ~0u) comb_clear(sl_ + (unsigned long long)(j >> 10) * MN + o_[u]);\n"
               "    }\n"
               "    __syncthreads();\n"
               "  }\n",
               pl->splits);
    dsb_put(s, "  if (wave > 0u) return;\n"
               "  #pragma unroll\n"
               "  for (u32 w = 0; w < NW - 1u; w++)\n"
               "    #pragma unroll\n"
               "    for (u32 v = 0; v < 16u; v++) acc[v] = acc[v] + part_[w][v][lane];\n"
               "  {\n"
               "    const f32x16 c = acc;\n"
               "    const u32 n = n0 + (lane & 31u);\n"
               "    #pragma unroll\n"
               "    for (u32 v = 0; v < 16u; v++) {\n"
               "      const u32 m = m0 + 8u * (v >> 2) + 4u * (lane >> 5) + (v & 3u);\n"
               "      if (m < M && n < N) {\n");
}

/* The wave-tile kernel (CFG_WAVE): one wave per 32-row tile of the output,
 * all 64 columns. A k-pair kp covers reordered k = 2kp (lanes 0-31) and
 * 2kp + 1 (lanes 32-63), which lie in the same run of the inner digit (its
 * extent is even): the A fragment of row m is at rowb_p(gid_m(m)) +
 * kbase_p(2kp) + h * icoef (h the lane's half), the B fragment at packed row
 * 2kp + h. Buffer loads take the lane's offset as a VGPR and kbase as an SGPR;
 * loads past the buffer read 0. Rows past M are clamped to M - 1 (their
 * products are never stored). */
static void emit_wave_kernel(DSB *s, const UOpKernel *k, const Contraction *ct, const GemmPlan *pl) {
    const KPerm *kp = &pl->kp;
    const u32 M = ct->M, N = ct->N, KPAIRS = kp->Kl / 2u, PF = wave_ring(KPAIRS);
    const u32 tiles = pl->tiles_m;
    const char *mf_a = pl->swap ? "rb0[q]" : "ra[q]", *mf_b = pl->swap ? "ra[q]" : "rb0[q]";
    const char *mf_a1 = pl->swap ? "rb1[q]" : "ra[q]", *mf_b1 = pl->swap ? "ra[q]" : "rb1[q]";
    /* at least six waves per SIMD: the register budget the compiler keeps
     * to (measured 141 against 145 us with four or five) */
    const u32 S = pl->tail_s ? pl->tail_s : 1u;
    dsb_put(s, "extern \"C\" __global__ __launch_bounds__(%u) __attribute__((amdgpu_waves_per_eu(6, 8))) void %s(",
            64u * S, pl->name);
    emit_params(s, k->n_leaves);
    dsb_put(s, ", float* ws, const float* pk%s) {\n", g_epi_params ? g_epi_params : "");
    dsb_put(s,
            "  constexpr u32 M = %uu, N = %uu, KP = %uu, PF = %uu, TILES = %uu, ICA = %uu;\n"
            "  constexpr u32 S = %uu, FULL = %uu, NFW = FULL / S, KPC = KP / S, PFT = %uu;\n"
            "  const u32 lane = threadIdx.x & 63u, h = lane >> 5;\n"
            "  const u32 wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);\n"
            "  u32 tile = blockIdx.x, kp0 = 0u;\n"
            "  bool tail = false;\n"
            "  if (S > 1u && tile >= NFW) {\n"
            "    /* the tiles past FULL (fewer than one per SIMD): each split over\n"
            "     * the S waves of one workgroup in K chunks of KPC k-pairs, so that\n"
            "     * no SIMD gets a whole extra tile */\n"
            "    tile = FULL + (tile - NFW);\n"
            "    if (tile >= TILES) return;\n"
            "    kp0 = wave * KPC;\n"
            "    tail = true;\n"
            "  } else if (S > 1u) {\n"
            "    /* workgroup b runs on XCD b %% 8: consecutive tiles (rows that share\n"
            "     * their neighbourhood of A) on one XCD's L2 */\n"
            "    if (NFW %% 8u == 0u) tile = (tile %% 8u) * (NFW / 8u) + tile / 8u;\n"
            "    tile = tile * S + wave;\n"
            "  } else {\n"
            "    if (tile >= TILES) return;\n"
            "    if (TILES %% 8u == 0u) tile = (tile %% 8u) * (TILES / 8u) + tile / 8u;\n"
            "  }\n"
            "  const u32 m0 = tile * 32u, n0 = 0u, wm = 0u, wn = 0u;\n"
            "  const u32 ma = (m0 + (lane & 31u) < M) ? m0 + (lane & 31u) : M - 1u;\n"
            "  const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc((void*)p%u, (short)0,\n"
            "      (int)((unsigned long long)c%u * 4ull < 0xFFFFFFFFull ? c%u * 4u : 0xFFFFFFFFu), 0x00020000);\n"
            "  const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc((void*)pk, (short)0, (int)(%uu * 4u), 0x00020000);\n"
            "  const int vA = (int)((rowb_p(gid_m(ma)) + h * ICA) * 4u);\n"
            "  const int vB = (int)((h * N + (lane & 31u)) * 4u);\n"
            "  float ra[PF], rb0[PF], rb1[PF];\n"
            "  auto load = [&](u32 kp, u32 q) {\n"
            "    const int so = (int)(kbase_p(2u * kp) * 4u);\n"
            "    ra[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rA, vA, so, 0));\n"
            "    rb0[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rB, vB, (int)(kp * 2u * N * 4u), 0));\n"
            "    rb1[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rB, vB + 128, (int)(kp * 2u * N * 4u), 0));\n"
            "  };\n"
            "  f32x16 acc[2];\n"
            "  acc[0] = (f32x16){0};\n"
            "  acc[1] = (f32x16){0};\n"
            "  if (!tail) {\n"
            "    #pragma unroll\n"
            "    for (u32 q = 0; q < PF; q++) load(q, q);\n"
            "    for (u32 kb = 0; kb + PF < KP; kb += PF) {\n"
            "      #pragma unroll\n"
            "      for (u32 q = 0; q < PF; q++) {\n"
            "        acc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(%s, %s, acc[0], 0, 0, 0);\n"
            "        acc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(%s, %s, acc[1], 0, 0, 0);\n"
            "        load(kb + PF + q, q);\n"
            "        /* each step's loads go out right after its MFMAs: PF k-pairs ahead */\n"
            "        __builtin_amdgcn_sched_barrier(0);\n"
            "      }\n"
            "    }\n"
            "    #pragma unroll\n"
            "    for (u32 q = 0; q < PF; q++) {\n"
            "      acc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(%s, %s, acc[0], 0, 0, 0);\n"
            "      acc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(%s, %s, acc[1], 0, 0, 0);\n"
            "    }\n"
            "  }\n",
            M, N, KPAIRS, PF, tiles, kp->icoef[0], S, pl->tail_full, pl->tail_pf ? pl->tail_pf : 1u,
            ct->sep_buf[0], ct->sep_buf[0], ct->sep_buf[0],
            kp->Kl * N, mf_a, mf_b, mf_a1, mf_b1, mf_a, mf_b, mf_a1, mf_b1);
    if (S > 1u)
        /* a tail chunk: its KPC k-pairs through the first PFT slots of the
         * ring; then waves 1..S-1 hand their partials to wave 0 through LDS
         * one after the other, and wave 0 adds them in wave (chunk) order
         * and makes the stores */
        dsb_put(s,
                "  __shared__ float tl_[32][64];\n"
                "  if (tail) {\n"
                "    #pragma unroll\n"
                "    for (u32 q = 0; q < PFT; q++) load(kp0 + q, q);\n"
                "    for (u32 kb = kp0; kb + PFT < kp0 + KPC; kb += PFT) {\n"
                "      #pragma unroll\n"
                "      for (u32 q = 0; q < PFT; q++) {\n"
                "        acc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(%s, %s, acc[0], 0, 0, 0);\n"
                "        acc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(%s, %s, acc[1], 0, 0, 0);\n"
                "        load(kb + PFT + q, q);\n"
                "        __builtin_amdgcn_sched_barrier(0);\n"
                "      }\n"
                "    }\n"
                "    #pragma unroll\n"
                "    for (u32 q = 0; q < PFT; q++) {\n"
                "      acc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(%s, %s, acc[0], 0, 0, 0);\n"
                "      acc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(%s, %s, acc[1], 0, 0, 0);\n"
                "    }\n"
                "    for (u32 j = 1u; j < S; j++) {\n"
                "      if (wave == j) {\n"
                "        #pragma unroll\n"
                "        for (u32 v = 0; v < 16u; v++) { tl_[v][lane] = acc[0][v]; tl_[16u + v][lane] = acc[1][v]; }\n"
                "      }\n"
                "      __syncthreads();\n"
                "      if (wave == 0u) {\n"
                "        #pragma unroll\n"
                "        for (u32 v = 0; v < 16u; v++) { acc[0][v] = acc[0][v] + tl_[v][lane]; acc[1][v] = acc[1][v] + tl_[16u + v][lane]; }\n"
                "      }\n"
                "      __syncthreads();\n"
                "    }\n"
                "    if (wave != 0u) return;\n"
                "  }\n",
                mf_a, mf_b, mf_a1, mf_b1, mf_a, mf_b, mf_a1, mf_b1);
    /* the LDS tile's epilogue: blocks (m, n) = (0, 0) and (0, 32) of the wave's tile */
    dsb_put(s,
            "  #pragma unroll\n"
            "  for (u32 blk = 0; blk < 2u; blk++) {\n"
            "    const f32x16 c = acc[blk];\n"
            "    const u32 bm = wm, bn = wn + blk * 32u;\n"
            "    #pragma unroll\n"
            "    for (u32 v = 0; v < 16u; v++) {\n"
            "      const u32 %s = %s0 + b%s + (lane & 31u);\n"
            "      const u32 %s = %s0 + b%s + 8u * (v >> 2) + 4u * (lane >> 5) + (v & 3u);\n"
            "      if (m < M && n < N) {\n", pl->swap ? "m" : "n", pl->swap ? "m" : "n",
            pl->swap ? "m" : "n", pl->swap ? "n" : "m", pl->swap ? "n" : "m", pl->swap ? "n" : "m");
}

/* Whether a plan made for CFG_WAVE can run it: K-reordered loads with an
 * even inner digit and no padding, the B side packed as K x 64, one split. */
static int wave_plan_ok(const Contraction *ct, const GemmPlan *pl) {
    const KPerm *kp = &pl->kp;
    return pl->cfg.direct == 4 && kp->on && pl->pack && kp->E == kp->Ep && kp->E % 2 == 0 && kp->Kl % 2 == 0 &&
           ct->N == 64 && pl->splits == 1 && kp->maxidx[0] < (1ull << 30) && (u64)kp->Kl * ct->N < (1ull << 28);
}

/* Uniform k base of one side at the stage starting at reordered index k. */
static void emit_kbase_fn(DSB *s, const KPerm *kp, int side, const char *name) {
    dsb_put(s, "__device__ __forceinline__ u32 %s(u32 k) {\n  u32 o = k / %uu;\n  u32 u = (k %% %uu) * %uu;\n",
            name, kp->Ep, kp->Ep, kp->icoef[side]);
    for (u32 t = 0; t < kp->ndig; t++) {
        if (t + 1 < kp->ndig)
            dsb_put(s, "  u += (o %% %uu) * %uu; o /= %uu;\n", kp->oext[t], kp->ocoef[side][t], kp->oext[t]);
        else
            dsb_put(s, "  u += o * %uu;\n", kp->ocoef[side][t]);
    }
    dsb_put(s, "  return u;\n}\n");
}

/* Lane map of a 16-byte loader: each lane holds 4 contiguous elements, along
 * k (k-major) or along the tile's rows; e counts the lane's groups of 4. */
static void emit_map4(DSB *s, int kmajor, u32 bx, const TileCfg *cf, const char *xname) {
    const u32 T = lds_threads(cf);
    if (kmajor) {
        const u32 g = cf->bk / 4u;
        dsb_put(s, "const u32 kk = (tid %% %uu) * 4u, %s = tid / %uu + %uu * e;", g, xname, g, T / g);
    } else {
        const u32 h = bx / 4u;
        dsb_put(s, "const u32 %s = (tid %% %uu) * 4u, kk = tid / %uu + %uu * e;", xname, h, h, T / h);
    }
}

/* K-reordered loaders (see KPerm): per-lane offsets once per tile, then one
 * uniform base per stage and an unchecked load per element. Rows past the
 * end of M (N) are clamped to the last row; their products are never stored. */
static void emit_kperm_loaders(DSB *s, const Contraction *ct, const GemmPlan *pl) {
    const TileCfg *cf = &pl->cfg;
    const KPerm *kp = &pl->kp;
    const u32 EX[2] = {cf->bm * cf->bk / lds_threads(cf), cf->bn * cf->bk / lds_threads(cf)};
    /* padded inner digit: elements whose inner index i0 + kk reaches E load
     * as 0 from a clamped (in-range) address; lim_ = E - i0 >= 1 because i0
     * is a multiple of the stage depth below Ep */
    const int padded = kp->Ep != kp->E;
    for (int side = 0; side < 2; side++) {
        const char S = side ? 'q' : 'p', X = side ? 'B' : 'A';
        const char *xn = side ? "nn" : "mm";
        const int kmaj = side ? ct->q_kmajor : ct->p_kmajor;
        const u32 bx = side ? cf->bn : cf->bm;
        const char rr = side ? 'b' : 'a';
        const int packed = side == 1 && pl->pack;     /* zero rows written by the pack kernel */
        const int mask = padded && !packed;
        if (packed) {
            dsb_put(s, "  const u32 oB = n0;\n");
        } else if (kp->lin[side]) {
            dsb_put(s, "  const u32 o%c = rowb_%c(gid_%c(%s));\n", X, S, side ? 'n' : 'm', side ? "n0" : "m0");
        } else {
            dsb_put(s, "  u32 o%c[%u];\n  #pragma unroll\n  for (u32 e = 0; e < %uu; e++) { ", X, EX[side], EX[side]);
            emit_map(s, kmaj, bx, cf, xn);
            char kt[48] = "";
            if (!mask) snprintf(kt, sizeof kt, " + kk * %uu", kp->icoef[side]);
            dsb_put(s, "\n    const u32 x = %s + %s;\n"
                       "    o%c[e] = rowb_%c(gid_%c(x < %uu ? x : %uu))%s; }\n",
                    side ? "n0" : "m0", xn, X, S, side ? 'n' : 'm', side ? ct->N : ct->M,
                    (side ? ct->N : ct->M) - 1, kt);
        }
        char src[40], lim[64], kv[16];
        if (packed) snprintf(src, sizeof src, "pk");
        else snprintf(src, sizeof src, "(const float*)p%u", ct->sep_buf[side]);
        snprintf(lim, sizeof lim, mask ? "\n    const u32 lim_ = %uu - k0 %% %uu;" : "", kp->E, kp->Ep);
        snprintf(kv, sizeof kv, mask ? "kv_" : "kk");
        /* offset of one element: row base, row, and the (clamped) k */
        char off[160];
        if (kp->lin[side] || packed)
            snprintf(off, sizeof off, "o%c + %s * %uu + %s * %uu", X, xn, kp->lcoef[side], kv, kp->icoef[side]);
        else
            snprintf(off, sizeof off, mask ? "o%c[e] + kv_ * %uu" : "o%c[e]", X, kp->icoef[side]);
        if (kp->vec[side]) {
            dsb_put(s, "  auto load%c = [&](u32 k0, float (&r%c)[%u]) {\n"
                       "    const float* ps = %s + kbase_%c(k0);%s\n"
                       "    #pragma unroll\n    for (u32 e = 0; e < %uu; e++) { ",
                    X, rr, EX[side], src, S, lim, EX[side] / 4u);
            emit_map4(s, kmaj, bx, cf, xn);
            if (mask) dsb_put(s, "\n      const u32 kv_ = kk < lim_ ? kk : 0u;");
            dsb_put(s, "\n      float4 v = *(const float4*)(ps + %s);\n", off);
            if (mask) {
                /* 16-byte groups never straddle E (E, i0 and the group start are multiples of 4) */
                dsb_put(s, "      if (kk >= lim_) v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);\n");
            }
            dsb_put(s, "      r%c[4u * e] = v.x; r%c[4u * e + 1u] = v.y; r%c[4u * e + 2u] = v.z; r%c[4u * e + 3u] = v.w; }\n"
                       "  };\n", rr, rr, rr, rr);
            continue;
        }
        dsb_put(s, "  auto load%c = [&](u32 k0, float (&r%c)[%u]) {\n"
                   "    const float* ps = %s + kbase_%c(k0);%s\n"
                   "    #pragma unroll\n    for (u32 e = 0; e < %uu; e++) { ",
                X, rr, EX[side], src, S, lim, EX[side]);
        emit_map(s, kmaj, bx, cf, xn);
        if (mask)
            dsb_put(s, "\n      const u32 kv_ = kk < lim_ ? kk : 0u;\n"
                       "      const float v = ps[%s];\n      r%c[e] = kk < lim_ ? v : 0.0f; }\n  };\n", off, rr);
        else
            dsb_put(s, "\n      r%c[e] = ps[%s]; }\n  };\n", rr, off);
    }
}

static char *gen_gemm_source(const UOpKernel *k, const Contraction *ct_in, const GemmPlan *pl, char *err,
                             size_t errlen) {
    /* the big tile evaluates its operands in place: separable row bases would
     * hold 16 more registers across its whole K loop (measured slower) */
    Contraction ctl = *ct_in;
    if (pl->cfg.bm == 128 && !pl->kp.on) ctl.sep[0] = ctl.sep[1] = 0;
    if (pl->pack) ctl.q_kmajor = 0;
    const Contraction *ct = &ctl;
    DSB s = {0};
    const TileCfg *cf = &pl->cfg;
    dsb_put(&s, "%s\n", kgen_prelude());
    if (g_epi_src) dsb_put(&s, "%s\n", g_epi_src);
    dsb_put(&s, "typedef float f32x16 __attribute__((ext_vector_type(16)));\n");
    emit_gid_fn(&s, "gid_m", ct->np, ct->pdiv, ct->pext);
    emit_gid_fn(&s, "gid_n", ct->nq, ct->qdiv, ct->qext);
    for (int side = 0; side < 2; side++) {
        if (!ct->sep[side]) continue;
        emit_sep_fn(&s, side ? "rowb_q" : "rowb_p", &ct->sep_aff[side], 0);
        emit_sep_fn(&s, side ? "koff_q" : "koff_p", &ct->sep_aff[side], 1);
        if (pl->kp.on) emit_kbase_fn(&s, &pl->kp, side, side ? "kbase_q" : "kbase_p");
        if (pl->pack && side == 1) emit_kbase_fn(&s, &pl->kpo, 1, "kbase_qo");
    }
    static char body[1 << 16];
    for (int side = 0; side < 2; side++) {
        const u8 *cone = side ? ct->coneQ : ct->coneP;
        u32 root = side ? ct->rootQ : ct->rootP;
        if (kgen_emit_cone(k, cone, "gid", "r", body, sizeof body) < 0) {
            snprintf(err, errlen, "operand cone cannot be emitted");
            free(s.p);
            return NULL;
        }
        dsb_put(&s, "__device__ __forceinline__ float operand_%c(u32 gid, u32 r, ", side ? 'q' : 'p');
        emit_params(&s, k->n_leaves);
        dsb_put(&s, ") {\n%s", body);
        if (op_type_is_float(k->ops[root].type)) dsb_put(&s, "  return f%u;\n}\n", root);
        else dsb_put(&s, "  return (float)n%u;\n}\n", root);
    }
    const u32 M = ct->M, N = ct->N, K = pl->kp.on ? pl->kp.Kl : ct->K;   /* the reordered (padded) K */
    const u32 tiles = pl->tiles_m * pl->tiles_n;
    if (cf->direct == 2) {
        emit_skinny_kernel(&s, k, ct, pl);
        return s.p;
    }
    if (cf->direct == 3) {
        emit_red_kernel(&s, k, ct, pl);
        emit_sum_kernel(&s, k, ct, pl);
        return s.p;
    }
    if (cf->direct && cf->direct != 4) {
        emit_direct_kernel(&s, k, ct, pl);
        emit_store_tail(&s, k, ct, pl);
        return s.p;
    }
    const u32 BK = cf->bk;
    const u32 EA = cf->bm * BK / lds_threads(cf), EB = cf->bn * BK / lds_threads(cf);
    const u32 NB = cf->wm_b * cf->wn_b;
    if (pl->pack) {
        /* B in the reordered k order, row-major K x N (n contiguous) */
        dsb_put(&s, "extern \"C\" __global__ __launch_bounds__(256) void %s_pack(", pl->name);
        emit_params(&s, k->n_leaves);
        dsb_put(&s, ", float* pk) {\n"
                    "  const u32 t = blockIdx.x * 256u + threadIdx.x;\n"
                    "  if (t >= %uu) return;\n"
                    "  const u32 k = t / %uu, n = t %% %uu;\n"
                    "  pk[t] = (k %% %uu < %uu) ? ld_f32(p%u, c%u, kbase_qo(k) + rowb_q(gid_n(n))) : 0.0f;\n}\n",
                pl->kp.Kl * N, N, N, pl->kp.Ep, pl->kp.E, ct->sep_buf[1], ct->sep_buf[1]);
    }
    if (cf->direct == 4) {
        emit_wave_kernel(&s, k, ct, pl);
        emit_store_tail(&s, k, ct, pl);
        return s.p;
    }
    dsb_put(&s, "extern \"C\" __global__ __launch_bounds__(%u) void %s(", lds_threads(cf), pl->name);
    emit_params(&s, k->n_leaves);
    dsb_put(&s, pl->pack ? ", float* ws, const float* pk%s) {\n" : ", float* ws%s) {\n", g_epi_params ? g_epi_params : "");
    dsb_put(&s,
            "  constexpr u32 BM = %u, BN = %u, BK = %u, LDA = BM + %uu, LDB = BN + %uu;\n"
            "  constexpr u32 M = %uu, N = %uu, K = %uu, TM = %uu, TN = %uu, TILES = %uu, KCH = %uu, SPLITS = %uu;\n"
            "  constexpr u32 WM = %uu, WN = %uu, GN = %uu;\n",
            cf->bm, cf->bn, BK, pl->pad_a, pl->pad_b, M, N, K, pl->tiles_m, pl->tiles_n, tiles, pl->kchunk, pl->splits,
            cf->wm_b * 32, cf->wn_b * 32, cf->gn);
    dsb_put(&s,
            "  __shared__ __attribute__((aligned(16))) float As[2][BK * LDA];\n"
            "  __shared__ __attribute__((aligned(16))) float Bs[2][BK * LDB];\n"
            "  const u32 tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;\n"
            "  /* XCD-aware tile order: workgroups go round-robin over 8 XCDs; give\n"
            "   * each XCD a compact block of tiles so their operand panels share L2 */\n"
            "  u32 bid = blockIdx.x, spl = blockIdx.y;\n"
            "  /* split K with few tiles: every tile of one split on the same XCD\n"
            "   * (workgroup w runs on XCD w %% 8), so the split's shared panel is\n"
            "   * fetched into one L2 */\n"
            "  if (SPLITS > 1u && SPLITS %% 8u == 0u && TILES %% 8u != 0u) {\n"
            "    const u32 lin = blockIdx.y * TILES + blockIdx.x, j = lin / 8u;\n"
            "    spl = (j / TILES) * 8u + lin %% 8u; bid = j %% TILES; }\n"
            "  u32 tile = bid;\n"
            "  if (TILES %% 8u == 0u) tile = (bid %% 8u) * (TILES / 8u) + bid / 8u;\n"
            "  u32 tm, tn;\n"
            "  { const u32 G = 8u; const u32 grp = tile / (G * TN), first = grp * G;\n"
            "    const u32 gsz = (TM - first) < G ? (TM - first) : G;\n"
            "    tm = first + (tile %% (G * TN)) %% gsz; tn = (tile %% (G * TN)) / gsz; }\n"
            "  const u32 m0 = tm * BM, n0 = tn * BN;\n"
            "  const u32 kbeg = spl * KCH;\n"
            "  const u32 kend = (kbeg + KCH < K) ? kbeg + KCH : K;\n"
            "  float ra0[%u], rb0[%u];\n", EA, EB);
    if (pl->depth == 2) dsb_put(&s, "  float ra1[%u], rb1[%u];\n", EA, EB);
    if (pl->kp.on) emit_kperm_loaders(&s, ct, pl);
    /* separable operands: per-row index bases, once per tile */
    if (!pl->kp.on && ct->sep[0]) {
        dsb_put(&s, "  u32 bA[%u];\n  #pragma unroll\n  for (u32 e = 0; e < %uu; e++) { ", EA, EA);
        emit_map(&s, ct->p_kmajor, cf->bm, cf, "mm");
        dsb_put(&s, " (void)kk; bA[e] = rowb_p(gid_m(m0 + mm)); }\n");
    }
    if (!pl->kp.on && ct->sep[1]) {
        dsb_put(&s, "  u32 bB[%u];\n  #pragma unroll\n  for (u32 e = 0; e < %uu; e++) { ", EB, EB);
        emit_map(&s, ct->q_kmajor, cf->bn, cf, "nn");
        dsb_put(&s, " (void)kk; bB[e] = rowb_q(gid_n(n0 + nn)); }\n");
    }
    if (!pl->kp.on) {
    dsb_put(&s, "  auto loadA = [&](u32 k0, float (&ra)[%u]) {\n    #pragma unroll\n    for (u32 e = 0; e < %uu; e++) { ",
            EA, EA);
    emit_map(&s, ct->p_kmajor, cf->bm, cf, "mm");
    /* operands are evaluated unconditionally (every load is range-checked,
     * so any (m, k) is safe) and masked after: no divergent branches */
    dsb_put(&s, "\n      const u32 m = m0 + mm, k = k0 + kk;\n");
    /* the mask is applied to the bits (a select would let the compiler move
     * the load under a branch and wait for each load in turn); it is left out
     * where the tile grid and K split divide the problem exactly */
    const int full_k = (K % pl->kchunk == 0) && (pl->kchunk % BK == 0);
    const char *gm = (M % cf->bm == 0) ? "true" : "(m < M)";
    const char *gn = (N % cf->bn == 0) ? "true" : "(n < N)";
    const char *gk = full_k ? "true" : "(k < kend)";
    if (ct->sep[0]) {
        dsb_put(&s, "      const float v = %s(p%u, c%u, bA[e] + koff_p(k));\n",
                ld_name(ct->sep_dt[0]), ct->sep_buf[0], ct->sep_buf[0]);
    } else {
        dsb_put(&s, "      const float v = operand_p(gid_m(m), k, ");
        emit_args(&s, k->n_leaves);
        dsb_put(&s, ");\n");
    }
    dsb_put(&s, "      ra[e] = __uint_as_float(__float_as_uint(v) & ((%s && %s) ? 0xFFFFFFFFu : 0u)); }\n  };\n", gm,
            gk);
    dsb_put(&s, "  auto loadB = [&](u32 k0, float (&rb)[%u]) {\n    #pragma unroll\n    for (u32 e = 0; e < %uu; e++) { ",
            EB, EB);
    emit_map(&s, ct->q_kmajor, cf->bn, cf, "nn");
    dsb_put(&s, "\n      const u32 n = n0 + nn, k = k0 + kk;\n");
    if (ct->sep[1]) {
        dsb_put(&s, "      const float v = %s(p%u, c%u, bB[e] + koff_q(k));\n",
                ld_name(ct->sep_dt[1]), ct->sep_buf[1], ct->sep_buf[1]);
    } else {
        dsb_put(&s, "      const float v = operand_q(gid_n(n), k, ");
        emit_args(&s, k->n_leaves);
        dsb_put(&s, ");\n");
    }
    dsb_put(&s, "      rb[e] = __uint_as_float(__float_as_uint(v) & ((%s && %s) ? 0xFFFFFFFFu : 0u)); }\n  };\n", gn,
            gk);
    }
    for (int side = 0; side < 2; side++) {
        const char X = side ? 'B' : 'A', r = side ? 'b' : 'a';
        const char *xn = side ? "nn" : "mm", *ld = side ? "LDB" : "LDA";
        const int kmaj = side ? ct->q_kmajor : ct->p_kmajor;
        const u32 bx = side ? cf->bn : cf->bm, ex = side ? EB : EA;
        if (pl->kp.on && pl->kp.vec[side]) {
            dsb_put(&s, "  auto store%c = [&](u32 buf, const float (&r%c)[%u]) {\n    #pragma unroll\n"
                        "    for (u32 e = 0; e < %uu; e++) { ", X, r, ex, ex / 4u);
            emit_map4(&s, kmaj, bx, cf, xn);
            if (kmaj)
                dsb_put(&s, "\n      #pragma unroll\n      for (u32 j = 0; j < 4u; j++) %cs[buf][(kk + j) * %s + %s] = r%c[4u * e + j]; }\n  };\n",
                        X, ld, xn, r);
            else
                dsb_put(&s, "\n      *(float4*)&%cs[buf][kk * %s + %s] = make_float4(r%c[4u * e], r%c[4u * e + 1u], "
                            "r%c[4u * e + 2u], r%c[4u * e + 3u]); }\n  };\n",
                        X, ld, xn, r, r, r, r);
            continue;
        }
        dsb_put(&s, "  auto store%c = [&](u32 buf, const float (&r%c)[%u]) {\n    #pragma unroll\n"
                    "    for (u32 e = 0; e < %uu; e++) { ", X, r, ex, ex);
        emit_map(&s, kmaj, bx, cf, xn);
        dsb_put(&s, " %cs[buf][kk * %s + %s] = r%c[e]; }\n  };\n", X, ld, xn, r);
    }
    dsb_put(&s,
            "  f32x16 acc[%u];\n"
            "  #pragma unroll\n  for (u32 b = 0; b < %uu; b++) acc[b] = (f32x16){0};\n"
            "  const u32 wm = (wave / GN) * WM, wn = (wave %% GN) * WN;\n"
            "  const u32 nst = (kend > kbeg) ? (kend - kbeg + BK - 1u) / BK : 0u;\n",
            NB, NB);
    /* One stage: issue the global loads of stage st + depth into a register
     * set, multiply the current LDS buffer, then move the registers of stage
     * st + 1 (loaded depth - 1 stages earlier) into the other buffer. With
     * depth 2 a load has two stages of math to arrive; the loop is unrolled
     * by two so that each register set is a fixed array. */
    char stage[4096];
    const char *mfma_a = pl->swap ? "b[kk][j]" : "a[kk][i]", *mfma_b = pl->swap ? "a[kk][i]" : "b[kk][j]";
    const char *prio_on = pl->prio ? "    __builtin_amdgcn_s_setprio(1);\n" : "";
    const char *prio_off = pl->prio ? "    __builtin_amdgcn_s_setprio(0);\n" : "";
    for (u32 ph = 0; ph < pl->depth; ph++) {
        const u32 ls = pl->depth == 2 ? ph : 0u, ss = pl->depth == 2 ? 1u - ph : 0u;
        snprintf(stage, sizeof stage,
                 "    {\n"
                 "    const u32 cur = st & 1u;\n"
                 "    if (st + %uu < nst) { loadA(kbeg + (st + %uu) * BK, ra%u); loadB(kbeg + (st + %uu) * BK, rb%u); }\n"
                 "    const float* A = As[cur];\n"
                 "    const float* B = Bs[cur];\n"
                 "    /* the stage's fragments; the compiler interleaves their reads with the\n"
                 "     * MFMAs (measured faster than pinning every read ahead of the math, which\n"
                 "     * costs registers and occupancy: 8-24 %% slower) */\n"
                 "%s"
                 "    float a[BK / 2u][%u], b[BK / 2u][%u];\n"
                 "    #pragma unroll\n"
                 "    for (u32 kk = 0; kk < BK; kk += 2u) {\n"
                 "      const u32 kr = kk + (lane >> 5);\n"
                 "      #pragma unroll\n"
                 "      for (u32 i = 0; i < %uu; i++) a[kk / 2u][i] = A[kr * LDA + wm + i * 32u + (lane & 31u)];\n"
                 "      #pragma unroll\n"
                 "      for (u32 j = 0; j < %uu; j++) b[kk / 2u][j] = B[kr * LDB + wn + j * 32u + (lane & 31u)];\n"
                 "    }\n"
                 "    #pragma unroll\n"
                 "    for (u32 kk = 0; kk < BK / 2u; kk++)\n"
                 "      #pragma unroll\n"
                 "      for (u32 i = 0; i < %uu; i++)\n"
                 "        #pragma unroll\n"
                 "        for (u32 j = 0; j < %uu; j++)\n"
                 "          acc[i * %uu + j] = __builtin_amdgcn_mfma_f32_32x32x2f32(%s, %s, acc[i * %uu + j], 0, 0, 0);\n"
                 "%s"
                 "    /* the next stages' global loads stay in flight across the MFMAs: the\n"
                 "     * LDS stores (which need them) may not move above the math */\n"
                 "    __builtin_amdgcn_sched_barrier(0);\n"
                 "    if (st + 1u < nst) { storeA(cur ^ 1u, ra%u); storeB(cur ^ 1u, rb%u); }\n"
                 "    __syncthreads();\n"
                 "    }\n",
                 pl->depth, pl->depth, ls, pl->depth, ls, prio_on, cf->wm_b, cf->wn_b, cf->wm_b, cf->wn_b, cf->wm_b,
                 cf->wn_b, cf->wn_b, mfma_a, mfma_b, cf->wn_b, prio_off, ss, ss);
        if (ph == 0) {
            if (pl->depth == 2)
                dsb_put(&s, "  if (nst > 0u) { loadA(kbeg, ra0); loadB(kbeg, rb0); storeA(0u, ra0); storeB(0u, rb0); }\n"
                            "  if (nst > 1u) { loadA(kbeg + BK, ra1); loadB(kbeg + BK, rb1); }\n"
                            "  __syncthreads();\n"
                            "  for (u32 st = 0; st < nst; st += 2u) {\n");
            else
                dsb_put(&s, "  if (nst > 0u) { loadA(kbeg, ra0); loadB(kbeg, rb0); storeA(0u, ra0); storeB(0u, rb0); }\n"
                            "  __syncthreads();\n"
                            "  for (u32 st = 0; st < nst; st++) {\n");
            dsb_put(&s, "%s", stage);
        } else {
            dsb_put(&s, "  if (st + 1u < nst) {\n  const u32 st1 = st + 1u;\n  { const u32 st = st1;\n%s  }\n  }\n", stage);
        }
    }
    dsb_put(&s, "  }\n");
    /* epilogue: D[i][j] of a 32x32 block sits in lane j + 32*((i/4)%%2), register (i%%4) + 4*(i/8);
     * D is the (m, n) block, or with swap its transpose (the MFMA took B as its first operand), so
     * that the 32 lanes of a store run along whichever output index is contiguous */
    dsb_put(&s,
            "  #pragma unroll\n"
            "  for (u32 blk = 0; blk < %uu; blk++) {\n"
            "    const f32x16 c = acc[blk];\n"
            "    const u32 bm = wm + (blk / %uu) * 32u, bn = wn + (blk %% %uu) * 32u;\n"
            "    #pragma unroll\n"
            "    for (u32 v = 0; v < 16u; v++) {\n"
            "      const u32 %s = %s0 + b%s + (lane & 31u);\n"
            "      const u32 %s = %s0 + b%s + 8u * (v >> 2) + 4u * (lane >> 5) + (v & 3u);\n"
            "      if (m < M && n < N) {\n", NB, cf->wn_b, cf->wn_b, pl->swap ? "m" : "n", pl->swap ? "m" : "n",
            pl->swap ? "m" : "n", pl->swap ? "n" : "m", pl->swap ? "n" : "m", pl->swap ? "n" : "m");
    emit_store_tail(&s, k, ct, pl);
    return s.p;
}

/* ---------------- plan cache and dispatch ---------------- */

typedef struct {
    u64 key;
    KOp *ops;
    u32 n_ops, n_leaves;
    u32 meta[5 + FUSE_MAX_LEAVES];
    int is_dense;                 /* 0: not a contraction (negative cache) */
    hipModule_t mod;
    hipFunction_t fn, fn_sum, fn_pack;
    GemmPlan plan;
    u32 M, N;
    CoForm co, co_sum, co_pack;   /* co-launch forms of the main, split-K sum and pack kernels */
    u32 serial;                   /* unique in the process (entries move when the table grows) */
    UOpKernel *kcopy;             /* the program, kept when its launch can take a fused epilogue */
    u32 cap;                      /* workgroups of the main kernel the GPU holds at once */
} DenseEntry;

/* Modules of a contraction with the elementwise program that consumes its
 * output fused into its epilogue (fn NULL: the pair was refused). */
#define FUSED_MAX 128
#define EPI_SOLO_MAX_LDS 8192u
typedef struct {
    u64 key;
    hipModule_t mod;
    hipFunction_t fn;
    CoForm co;
    KGenScalars sc;    /* the consumer's inline scalars (the fused kernel's last parameters) */
} FusedEntry;
static struct {
    FusedEntry e[FUSED_MAX];
    u32 n;
    u32 next_serial;
} F;

static struct {
    DenseEntry *tab;
    u32 cap, n;
    Scratch ws;            /* split-K partial sums */
    Scratch pk;            /* packed B operands */
} D;

static void meta_of(const UOpKernel *k, u32 *m) {
    memset(m, 0, (5 + FUSE_MAX_LEAVES) * sizeof(u32));
    m[0] = k->grid[0]; m[1] = k->grid[1]; m[2] = k->grid[2];
    m[3] = k->local_size; m[4] = k->out_dtype;
    for (u32 i = 0; i < k->n_leaves && i < FUSE_MAX_LEAVES; i++) m[5 + i] = k->leaf_dtypes[i];
}

/* Whether a plan's one launch writes every output once in an epilogue that
 * can take a fused consumer: unsplit, no packed operand, f32 output, on the
 * tiled, direct or row-per-lane kernel. */
static int plan_takes_epilogue(const GemmPlan *pl, const UOpKernel *k) {
    return pl->splits == 1 && !pl->comb && !pl->pack && pl->cfg.direct <= 2 && k->out_dtype == DTYPE_F32;
}

static DenseEntry *lookup(u64 key, const UOpKernel *k) {
    if (!D.tab) return NULL;
    u32 mk = D.cap - 1;
    for (u32 p = (u32)key & mk, probes = 0; probes < D.cap; p = (p + 1) & mk, probes++) {
        DenseEntry *e = &D.tab[p];
        if (!e->key) return NULL;
        if (e->key != key || e->n_ops != k->n_ops || e->n_leaves != k->n_leaves) continue;
        u32 m[5 + FUSE_MAX_LEAVES];
        meta_of(k, m);
        if (memcmp(m, e->meta, sizeof m) == 0 && memcmp(e->ops, k->ops, (size_t)k->n_ops * sizeof(KOp)) == 0)
            return e;
    }
    return NULL;
}

static DenseEntry *insert(u64 key, const UOpKernel *k) {
    if (!D.tab || (D.n + 1) * 2 > D.cap) {
        u32 nc = D.cap ? D.cap * 2 : 256;
        DenseEntry *nt = calloc(nc, sizeof(DenseEntry));
        if (!nt) return NULL;
        for (u32 i = 0; i < D.cap; i++) {
            if (!D.tab[i].key) continue;
            u32 p = (u32)D.tab[i].key & (nc - 1);
            while (nt[p].key) p = (p + 1) & (nc - 1);
            nt[p] = D.tab[i];
        }
        free(D.tab);
        D.tab = nt;
        D.cap = nc;
    }
    u32 p = (u32)key & (D.cap - 1);
    while (D.tab[p].key) p = (p + 1) & (D.cap - 1);
    DenseEntry *e = &D.tab[p];
    memset(e, 0, sizeof *e);
    e->key = key;
    e->serial = ++F.next_serial;
    e->n_ops = k->n_ops;
    e->n_leaves = k->n_leaves;
    meta_of(k, e->meta);
    e->ops = malloc((size_t)k->n_ops * sizeof(KOp));
    if (e->ops) memcpy(e->ops, k->ops, (size_t)k->n_ops * sizeof(KOp));
    D.n++;
    return e;
}

/* Measured on MI355X over the LeNet-5, conv-block and 4096^3 contractions:
 * big tiles when both sides are large; the LDS-staged 256x32 (32x256) tile
 * for very tall (wide) and thin operands such as convolutions over a batch of
 * images, where its four waves share each operand stage; for 64 channels
 * (33..64 columns) the 64x64 tile on a tall convolution (231 us against 282
 * for 256x64 and 480 for the direct kernel on a 3x3 64->64 conv over
 * [64,64,56,56]) and also on a weight gradient's long K (see long_k); the
 * direct kernel for the rest (fully connected layers, small weight
 * gradients). */
static TileCfg pick_cfg(u32 M, u32 N, u32 K) {
    u64 big_tiles = (u64)((M + 127) / 128) * ((N + 127) / 128);
    if (M >= 128 && N >= 128 && big_tiles >= 128) return CFG_BIG;
    if (N <= SKINNY_MAX_N && M >= SKINNY_MIN_M && (u64)K * N <= SKINNY_MAX_KN && !hipb.dense_noskinny)
        return CFG_SKINNY;
    if (N <= 32 && M >= 4096) return CFG_TALL;
    if (M <= 32 && N >= 4096) return CFG_WIDE;
    if (N > 32 && N <= 64 && M >= 4096) return CFG_MID;
    if (N > 32 && N <= 64 && M >= 256 && K >= 16384) return CFG_MID;
    return CFG_DIRECT;
}

/* A weight gradient's shape: few output tiles (64-channel columns, a few
 * hundred rows) over a long K. Such a contraction is bound by each
 * workgroup's chain of dependent stages, so it takes twice the workgroups
 * (about 1024) and two stages of loads in flight. Measured on the 3x3 64->64
 * weight gradient over [64,64,56,56] (576x64x200704): 64x64 tiles with 128
 * splits 190 us + 7.5 us sum, against 200 + 7.5 for 128x64 tiles with 128
 * splits (their fifth row tile is half empty) and 210 for 64x64 with 64. */
static int long_k(u32 M, u32 N, u32 K) {
    return N > 32 && N <= 64 && M >= 256 && M < 4096 && K >= 16384;
}

static int cmp_u64(const void *x, const void *y) {
    u64 a = *(const u64 *)x, b = *(const u64 *)y;
    return a < b ? -1 : a > b;
}

/* Largest value one digit of an affine index takes. */
static u64 digit_max(const Digit *d, u64 range) {
    if (d->mod) return d->mod - 1;
    return (range + d->div - 1) / d->div - 1;
}

static int plan_kperm(const Contraction *ct, GemmPlan *pl) {
    KPerm *kp = &pl->kp;
    memset(kp, 0, sizeof *kp);
    const TileCfg *cf = &pl->cfg;
    if (hipb.dense_nokperm || (cf->direct && cf->direct != 4)) return 0;
    const u64 K = ct->K, total = (u64)ct->M * ct->N;
    for (int s = 0; s < 2; s++)
        if (!ct->sep[s] || ct->sep_dt[s] != DTYPE_F32 || ct->sep_buf[s] == 0) return 0;
    /* digit boundaries of both sides' k offsets */
    u64 b[KP_MAX + 2];
    u32 nb = 0;
    b[nb++] = 1;
    b[nb++] = K;
    for (int s = 0; s < 2; s++) {
        const Aff *a = &ct->sep_aff[s];
        for (u32 t = 0; t < a->n; t++) {
            if (a->d[t].var != 1) continue;
            if (nb + 2 > KP_MAX + 2) return 0;
            b[nb++] = a->d[t].div;
            b[nb++] = a->d[t].mod ? (u64)a->d[t].div * a->d[t].mod : K;
        }
    }
    qsort(b, nb, sizeof b[0], cmp_u64);
    u32 nu = 0;
    for (u32 i = 0; i < nb; i++)
        if (nu == 0 || b[i] != b[nu - 1]) b[nu++] = b[i];
    if (b[nu - 1] != K) return 0;
    u32 nd = nu - 1;                      /* atomic digit j: div b[j], extent b[j+1] / b[j] */
    u64 ext[KP_MAX], co[2][KP_MAX];
    for (u32 j = 0; j < nd; j++) {
        if (b[j + 1] % b[j]) return 0;
        ext[j] = b[j + 1] / b[j];
        co[0][j] = co[1][j] = 0;
    }
    for (int s = 0; s < 2; s++) {
        const Aff *a = &ct->sep_aff[s];
        u64 mx = a->cst;
        for (u32 t = 0; t < a->n; t++) {
            const Digit *d = &a->d[t];
            if (d->var == 0) {
                mx += (u64)a->coef[t] * digit_max(d, total);
                continue;
            }
            u64 end = d->mod ? (u64)d->div * d->mod : K;
            for (u32 j = 0; j < nd; j++)
                if (b[j] >= d->div && b[j + 1] <= end) co[s][j] += (u64)a->coef[t] * (b[j] / d->div);
        }
        for (u32 j = 0; j < nd; j++) {
            if (co[s][j] > 0xFFFFFFFFull) return 0;
            mx += co[s][j] * (ext[j] - 1);
        }
        kp->maxidx[s] = mx;
        if (mx > 0xFFFFFFFFull) return 0;
    }
    /* the inner digit: the longest whose extent the stage depth divides;
     * lanes along k stay coalesced only on a unit-stride inner digit, and a
     * strided one is fine only for an operand that stays in cache (weights).
     * Failing that, a digit that is unit-stride on every k-major side, padded
     * up to a multiple of the stage depth (at most 1/4 more work): the image
     * rows of a weight gradient (56 -> 64) */
    int best = -1;
    for (int pass = 0; pass < 2 && best < 0; pass++) {
        for (u32 j = 0; j < nd; j++) {
            const u64 ep = (ext[j] + cf->bk - 1) / cf->bk * cf->bk;
            if (pass == 0 ? ext[j] % cf->bk != 0 : (ext[j] % cf->bk == 0 || ext[j] % 4 != 0 || ep * 4 > ext[j] * 5))
                continue;
            int ok = 1;
            for (int s = 0; s < 2; s++) {
                int kmaj = s ? ct->q_kmajor : ct->p_kmajor;
                if (kmaj && co[s][j] != 1 && (pass == 1 || kp->maxidx[s] * 4 > (8ull << 20))) ok = 0;
            }
            if (ok && (best < 0 || ext[j] > ext[best])) best = (int)j;
        }
    }
    if (best < 0) return 0;
    kp->E = (u32)ext[best];
    kp->Ep = (u32)((ext[best] + cf->bk - 1) / cf->bk * cf->bk);
    kp->Kl = (u32)(K / kp->E * kp->Ep);
    kp->buf[0] = ct->sep_buf[0];
    kp->buf[1] = ct->sep_buf[1];
    for (int s = 0; s < 2; s++) kp->icoef[s] = (u32)co[s][best];
    for (u32 j = 0; j < nd; j++) {
        if ((int)j == best) continue;
        kp->oext[kp->ndig] = (u32)ext[j];
        kp->ocoef[0][kp->ndig] = (u32)co[0][j];
        kp->ocoef[1][kp->ndig] = (u32)co[1][j];
        kp->ndig++;
    }
    /* rows of a tile that never carry into the next gid digit map linearly */
    for (int s = 0; s < 2; s++) {
        u32 nx = s ? ct->nq : ct->np;
        u32 fdiv = s ? ct->qdiv[nx - 1] : ct->pdiv[nx - 1];
        u32 fext = s ? ct->qext[nx - 1] : ct->pext[nx - 1];
        u32 bx = s ? cf->bn : cf->bm, mx = s ? ct->N : ct->M;
        if (fext % bx || mx % bx) continue;
        const Aff *a = &ct->sep_aff[s];
        int ok = 1;
        u32 lc = 0;
        for (u32 t = 0; t < a->n; t++) {
            const Digit *d = &a->d[t];
            if (d->var != 0 || d->div != fdiv) continue;
            if (d->mod && d->mod != fext) ok = 0;
            lc = a->coef[t];
        }
        kp->lin[s] = ok;
        kp->lcoef[s] = lc;
    }
    /* 16-byte loads: a linear side whose lanes run along a unit-stride
     * dimension, with every other coefficient and the constant a multiple of
     * 4, reads 4 contiguous elements from a 16-byte aligned address (buffers
     * start 256-byte aligned) */
    for (int s = 0; s < 2 && !hipb.dense_novec; s++) {
        if (!kp->lin[s]) continue;
        const int kmaj = s ? ct->q_kmajor : ct->p_kmajor;
        const u32 unit = kmaj ? kp->icoef[s] : kp->lcoef[s];
        const u32 other = kmaj ? kp->lcoef[s] : kp->icoef[s];
        const u32 nx = s ? ct->nq : ct->np;
        const u32 fdiv = s ? ct->qdiv[nx - 1] : ct->pdiv[nx - 1];
        const Aff *a = &ct->sep_aff[s];
        const u32 per_lane = (s ? cf->bn : cf->bm) * cf->bk / lds_threads(cf);
        int ok = unit == 1 && other % 4 == 0 && a->cst % 4 == 0 && kp->E % 4 == 0 && per_lane % 4 == 0;
        for (u32 t = 0; t < kp->ndig; t++) ok = ok && kp->ocoef[s][t] % 4 == 0;
        for (u32 t = 0; t < a->n; t++)
            if (a->d[t].var == 0 && a->d[t].div != fdiv) ok = ok && a->coef[t] % 4 == 0;
        kp->vec[s] = ok;
    }
    /* the 128x128 tile keeps no per-lane offset arrays (registers) */
    if (cf->bm == 128 && cf->bn == 128 && !(kp->lin[0] && kp->lin[1])) {
        memset(kp, 0, sizeof *kp);
        return 0;
    }
    kp->on = 1;
    return 1;
}

/* LDS row padding (floats). A k-major operand is stored with its lanes along
 * k, so each store spreads over LDS rows; 32 four-byte banks serve a half
 * wavefront at a time. 4-byte stores put 16 lanes on consecutive k and 2
 * rows per half wavefront: a row stride of 2 mod 32 keeps all 32 in distinct
 * banks. 16-byte loaders store 4 k-rows per lane with 8 lane groups along k
 * and 4 rows per half wavefront: a stride of 1 mod 32. Operands stored along
 * their rows are conflict-free at any stride; 4 keeps 16-byte alignment.
 * (Measured: the 16-byte 4096^3 GEMM 2-6 % faster with 1 than 4; the
 * 64-channel convolutions lost a third of their LDS cycles to conflicts with
 * the wrong stride.) THVM_HIP_GEMM_PAD overrides the k-major padding. */
static void plan_pads(const Contraction *ct, GemmPlan *pl) {
    for (int s = 0; s < 2; s++) {
        const int kmaj = s ? (pl->pack ? 0 : ct->q_kmajor) : ct->p_kmajor;
        const u32 bx = s ? pl->cfg.bn : pl->cfg.bm;
        u32 pad = 4;
        if (kmaj) {
            const u32 want = pl->kp.on && pl->kp.vec[s] ? 1u : 2u;
            pad = hipb.gemm_pad_k_set ? hipb.gemm_pad_k : (want + 32u - bx % 32u) % 32u;
        }
        if (s) pl->pad_b = pad;
        else pl->pad_a = pad;
    }
}

/* Packing the B side. A small B (the weights of a convolution) reused by
 * many row tiles, whose reordered-k loads are scattered (lanes along k on a
 * strided digit: 3x3 weights put consecutive input channels 9 floats apart),
 * costs the address unit and L1 far more than its bytes: each 64-lane load
 * touches dozens of cache lines. A pack kernel first copies it into a K x N
 * row-major buffer in the reordered k order; the GEMM then reads that buffer
 * like a linear side with 16-byte loads along n. In K-reordered terms the
 * packed side has row coefficient 1, inner coefficient N and outer digit
 * coefficients N times the place value of each digit in k. */
static void plan_pack(const Contraction *ct, GemmPlan *pl) {
    KPerm *kp = &pl->kp;
    pl->pack = 0;
    if (!kp->on || hipb.dense_nopack || kp->vec[1] || (pl->cfg.direct && pl->cfg.direct != 4)) return;
    const u32 per_lane = pl->cfg.bn * pl->cfg.bk / lds_threads(&pl->cfg);
    if ((u64)kp->Kl * ct->N > (4u << 20) || ct->N % 4 != 0 || ct->N % pl->cfg.bn != 0 || per_lane % 4 != 0 ||
        (pl->tiles_m < 64 && !hipb.dense_pack))
        return;
    pl->kpo = *kp;
    pl->pack = 1;
    kp->lin[1] = 1;
    kp->lcoef[1] = 1;
    kp->icoef[1] = ct->N;
    u64 place = kp->Ep;
    for (u32 t = 0; t < kp->ndig; t++) {
        kp->ocoef[1][t] = (u32)(place * ct->N);
        place *= kp->oext[t];
    }
    kp->vec[1] = !hipb.dense_novec;
    kp->maxidx[1] = (u64)kp->Kl * ct->N - 1;
}

/* K chunk per split, in stage multiples, over the K the kernel loops on (the
 * padded reordered K of a K-reordered plan). */
static void plan_chunks(const Contraction *ct, GemmPlan *pl) {
    const u32 K = pl->kp.on ? pl->kp.Kl : ct->K, splits = pl->splits_want ? pl->splits_want : 1;
    u32 kch = (K + splits - 1) / splits;
    kch = (kch + pl->cfg.bk - 1) / pl->cfg.bk * pl->cfg.bk;
    pl->kchunk = kch;
    pl->splits = (K + kch - 1) / kch;
    /* direct kernel: its waves walk the chunk's K steps in turn, each step a
     * chain of dependent loads and MFMAs; 8 waves when an unsplit K has more
     * than 4 steps (measured on LeNet-5's fully connected weight gradients:
     * 7.5 -> 6.2 us; its split-K convolution weight gradients got slower, 16
     * -> 17 us, and 16 waves were slower everywhere, 12 -> 31 us on fc1: wave
     * 0 then adds 15 partial blocks from 60 KB of LDS) */
    pl->nw = 4;
    if (pl->cfg.direct == 4) {
        pl->nw = 1;
        return;
    }
    if (pl->cfg.direct == 3) {
        /* row groups of at most RED_MAX_ACC / N rows, balanced; K chunks of
         * at least RED_K_PER_LANE k per lane, about 1024 workgroups at most */
        const u32 mgmax = RED_MAX_ACC / ct->N, ng = (ct->M + mgmax - 1) / mgmax;
        pl->red_mg = (ct->M + ng - 1) / ng;
        pl->tiles_m = (ct->M + pl->red_mg - 1) / pl->red_mg;
        pl->tiles_n = 1;
        u32 sp = ct->K / (GEMM_THREADS * RED_K_PER_LANE);
        if (sp > 1024 / pl->tiles_m) sp = 1024 / pl->tiles_m;
        if (sp < 2) sp = 2;
        pl->kchunk = (ct->K + sp - 1) / sp;
        pl->splits = (ct->K + pl->kchunk - 1) / pl->kchunk;
        for (int sd = 0; sd < 2; sd++) {
            const Aff *a = &ct->sep_aff[sd];
            u64 mx = a->cst;
            for (u32 t = 0; t < a->n; t++)
                mx += (u64)a->coef[t] * digit_max(&a->d[t], a->d[t].var == 0 ? (u64)ct->M * ct->N : ct->K);
            pl->red_max[sd] = mx;
            pl->red_buf[sd] = ct->sep_buf[sd];
        }
        return;
    }
    if (pl->cfg.direct == 2) {
        /* skinny: waves per workgroup splitting K, aiming at SKINNY_TARGET_WAVES
         * waves in all with at least 8 k per wave */
        const u32 rows = pl->tiles_m;
        u32 kw = 1;
        while (kw < 16 && (u64)rows * kw * 2 <= SKINNY_TARGET_WAVES && ct->K / (kw * 2) >= 8) kw *= 2;
        pl->nw = hipb.direct_waves ? hipb.direct_waves : kw;
        pl->kchunk = ct->K;
        pl->splits = 1;
        return;
    }
    if (pl->cfg.direct) {
        const u32 steps = (kch + pl->cfg.bk - 1) / pl->cfg.bk;
        if (hipb.direct_waves) pl->nw = hipb.direct_waves;
        else if (steps > 4 && pl->splits == 1) pl->nw = 8;
    }
}

static void make_plan_cfg(const Contraction *ct, GemmPlan *pl, u64 sig, const TileCfg *cfg);

/* Skinny block size: the largest E <= SKINNY_MAX_E dividing K such that no
 * k digit of either side straddles it (each lies wholly below E or wholly at
 * or above it), so that koff(kb + i) = koff(kb) + koff(i) for kb a multiple
 * of E and i < E: the kernel unrolls i and every in-block offset is a
 * constant. And the largest index the row side forms. */
#define SKINNY_MAX_E 64
static void plan_skinny(const Contraction *ct, GemmPlan *pl) {
    pl->ske = 0;
    pl->skmax = ~0ull;
    if (pl->cfg.direct != 2) return;
    pl->skbuf = ct->sep[0] ? ct->sep_buf[0] : 0;
    if (ct->sep[0] && ct->sep_dt[0] == DTYPE_F32) {
        const Aff *a = &ct->sep_aff[0];
        u64 mx = a->cst;
        for (u32 t = 0; t < a->n; t++)
            mx += (u64)a->coef[t] * digit_max(&a->d[t], a->d[t].var == 0 ? (u64)ct->M * ct->N : ct->K);
        pl->skmax = mx;
    }
    if (!ct->sep[0] || !ct->sep[1] || hipb.dense_noskinny_blocks) return;
    for (u32 E = SKINNY_MAX_E < ct->K ? SKINNY_MAX_E : ct->K; E >= 2; E--) {
        if (ct->K % E) continue;
        int ok = 1;
        for (int sd = 0; sd < 2 && ok; sd++) {
            const Aff *a = &ct->sep_aff[sd];
            for (u32 t = 0; t < a->n && ok; t++) {
                const Digit *d = &a->d[t];
                if (d->var != 1) continue;
                const u64 end = d->mod ? (u64)d->div * d->mod : ct->K;
                if (!(end <= E && E % end == 0) && !(d->div >= E && d->div % E == 0)) ok = 0;
            }
        }
        if (ok) {
            pl->ske = E;
            /* waves per row group: a divisor of the block count (no wave
             * without a block, every wave the same number of blocks), the
             * largest with at most SKINNY_TARGET_WAVES_BLK waves in all
             * (LeNet-5's conv2 input gradient: 16 blocks over 8 waves
             * instead of 4, conv2: 6 blocks over 6 waves instead of 8) */
            const u32 nblk = ct->K / E, rows = pl->tiles_m;
            if (!hipb.direct_waves) {
                u32 kw = 1;
                for (u32 w = 1; w <= 16 && w <= nblk; w++)
                    if (nblk % w == 0 && (u64)rows * w <= SKINNY_TARGET_WAVES_BLK) kw = w;
                pl->nw = kw;
            }
            return;
        }
    }
}

/* In-launch combine of split-K partials (direct and outer-product kernels):
 * the splits but the last publish their partials as combine words, the last
 * split's workgroup takes them into LDS and adds every output's partials in
 * split order (deterministic), so no workspace and no sum kernel. It needs a
 * word per partial in the combine area and the taken partials in LDS: the
 * direct kernel's 1024 outputs for at most COMB_DIRECT_MAX_SPLITS - 1 splits,
 * the outer-product kernel's within its transpose buffer. At most
 * COMB_MAX_SPLITS splits: the last split's workgroup takes every other
 * split's words after its own chunk, which LeNet-5's conv1 weight gradient
 * (98 splits) paid for with 7 us over the 3 us of its sum kernel, while its
 * conv2 weight gradient (12 splits) saved 2.5 us. */
#define COMB_DIRECT_MAX_SPLITS 8u
#define COMB_RED_LDS_FLOATS (4u * 32u * 65u)
#define COMB_MAX_SPLITS 16u
static void plan_comb(const Contraction *ct, GemmPlan *pl) {
    pl->comb = 0;
    if (hipb.dense_nocomb || pl->splits < 2 || pl->splits > COMB_MAX_SPLITS ||
        (u64)pl->splits * ct->M * ct->N > COMB_SLOTS)
        return;
    if (pl->cfg.direct == 1) pl->comb = pl->splits <= COMB_DIRECT_MAX_SPLITS && !pl->pack;
    else if (pl->cfg.direct == 3) pl->comb = (u64)(pl->splits - 1) * pl->red_mg * ct->N <= COMB_RED_LDS_FLOATS;
}

/* Wave tile: its grid is one wave per 32-row tile, and the waves of a SIMD
 * share its matrix pipe, so the kernel takes as long as the SIMD with the
 * most tiles. With S waves per workgroup, the tiles up to the largest
 * multiple of the SIMD count run whole (S per workgroup) and each of the
 * rest (fewer than one per SIMD) is split over the S waves of a workgroup in
 * K chunks, added through LDS in chunk order: on the 3x3 64->64 convolution
 * at batch 64, 6272 tiles on 1024 SIMDs are 6144 whole tiles and 128 tiles in
 * 4 chunks, at most 6.25 tiles of work per SIMD instead of 7. */
static void plan_wave_tail(GemmPlan *pl) {
    pl->tail_full = pl->tail_s = pl->tail_pf = 0;
    if (hipb.dense_notail) return;
    const u32 simds = 4u * dense_cus(), tiles = pl->tiles_m * pl->tiles_n, kpairs = pl->kp.Kl / 2u;
    const u32 full = tiles / simds * simds, rem = tiles - full;
    if (!full || !rem) return;
    for (u32 S = hipb.wave_tail_s ? hipb.wave_tail_s : 4u; S >= 2u; S /= 2u) {
        if (full % (8u * S) || kpairs % S) continue;
        const u32 kpc = kpairs / S;
        u32 pft = 0;
        for (u32 d = wave_ring(kpairs); d >= 2u && !pft; d--)
            if (kpc % d == 0) pft = d;
        if (!pft) continue;
        pl->tail_full = full;
        pl->tail_s = S;
        pl->tail_pf = pft;
        return;
    }
}

static void make_plan(const Contraction *ct, GemmPlan *pl, u64 sig) {
    static const TileCfg *forced[12] = {NULL, &CFG_BIG, &CFG_MID, &CFG_TALL, &CFG_WIDE, &CFG_DIRECT, &CFG_C64,
                                        &CFG_C64S, &CFG_SKINNY, &CFG_RED, &CFG_C64W, &CFG_WAVE};
    const int red_fits = ct->sep[0] && ct->sep[1] && ct->sep_dt[0] == DTYPE_F32 && ct->sep_dt[1] == DTYPE_F32 &&
                         ct->M >= 2 && ct->N >= 2 &&
                         (u64)ct->M * ct->N <= RED_MAX_MN && ct->N <= RED_MAX_ACC;
    /* the skinny kernel keeps N sums per lane and the outer-product one MG*N:
     * forced only where they apply */
    const int forced_ok = hipb.dense_tile &&
                          !(hipb.dense_tile == 8 && (ct->N > SKINNY_MAX_N || (u64)ct->K * ct->N > SKINNY_MAX_KN)) &&
                          !(hipb.dense_tile == 9 && !red_fits);
    TileCfg cfg = forced_ok ? *forced[hipb.dense_tile] : pick_cfg(ct->M, ct->N, ct->K);
    if (!forced_ok && !hipb.dense_nored && red_fits && ct->K >= RED_MIN_K) cfg = CFG_RED;
    if (!forced_ok && !hipb.dense_nowave && ct->N == 64 && ct->M >= 4096 && !long_k(ct->M, ct->N, ct->K)) {
        make_plan_cfg(ct, pl, sig, &CFG_WAVE);
        if (wave_plan_ok(ct, pl)) {
            plan_wave_tail(pl);
            return;
        }
    }
    if (cfg.direct == 4) cfg = CFG_MID;
    make_plan_cfg(ct, pl, sig, &cfg);
    if (pl->cfg.direct == 4 && !wave_plan_ok(ct, pl)) make_plan_cfg(ct, pl, sig, &CFG_MID);
    if (pl->cfg.direct == 4) plan_wave_tail(pl);
}

static void make_plan_cfg(const Contraction *ct, GemmPlan *pl, u64 sig, const TileCfg *cfg) {
    memset(pl, 0, sizeof *pl);
    pl->cfg = *cfg;
    /* two stages of loads in flight on the 128x64 tile and for long K (the
     * weight gradients: measured 5-7 % faster there, 3 % slower on the 64x64
     * convolution and the 128x128 GEMM, whose occupancy it lowers) */
    const int lk = long_k(ct->M, ct->N, ct->K) && !hipb.dense_tile;
    pl->depth = hipb.gemm_depth ? hipb.gemm_depth : ((cfg->bm == 128 && cfg->bn == 64) || lk) ? 2u : 1u;
    /* a wave's priority raised over its stage's math (the SIMD's other wave
     * then issues its loads and LDS stores around it): the long-K weight
     * gradient 162 -> 158 us, the 4096^3 GEMM 4 % slower */
    pl->prio = hipb.gemm_prio == 1 || (hipb.gemm_prio == 0 && lk);
    if (!pl->cfg.direct && hipb.gemm_bk) pl->cfg.bk = hipb.gemm_bk;
    pl->tiles_m = (ct->M + pl->cfg.bm - 1) / pl->cfg.bm;
    pl->tiles_n = (ct->N + pl->cfg.bn - 1) / pl->cfg.bn;
    u32 tiles = pl->tiles_m * pl->tiles_n;
    /* split K until the grid covers the 256 CUs about twice, keeping each
     * split at least min_chunk long (512 for the big tiles, whose per-tile
     * setup is larger; 64 otherwise) */
    /* direct: 4 waves per block share its K range, so a split of c gives
     * each wave c/4; keep that >= 64 and aim for ~2048 waves */
    u32 min_chunk = pl->cfg.bm == 128 ? 512 : pl->cfg.direct ? (hipb.direct_min_chunk ? hipb.direct_min_chunk : 256) : 64;
    u64 target = lk ? 1024 : 512;    /* workgroups */
    u32 splits = 1;
    while ((u64)tiles * splits < target && ct->K / (splits * 2) >= min_chunk && splits < 1024) splits *= 2;
    if (lk && tiles <= GEMM_SLOTS_PER_CU * dense_cus()) {
        /* a long-K weight gradient fills the GPU's workgroup slots once: a
         * second, mostly empty round of splits costs most of a split's time
         * (576x64x200704 on 256 CUs: 9 tiles x 128 splits = 1152 workgroups
         * on 1024 slots, 182 us; 9 x 112 = 1008, 160 us) */
        splits = GEMM_SLOTS_PER_CU * dense_cus() / tiles;
        if (splits > 1024) splits = 1024;
    }
    if (hipb.dense_splits) splits = hipb.dense_splits;
    if (pl->cfg.direct == 2 || pl->cfg.direct == 4) splits = 1;
    if (pl->cfg.direct == 3) splits = 2;   /* the chunks are chosen with the row groups */
    pl->splits_want = splits;
    snprintf(pl->name, sizeof pl->name, "thvm_gemm_%08x", (u32)(sig & 0xFFFFFFFFu));
    pl->swap = (!pl->cfg.direct || pl->cfg.direct == 4) && !hipb.dense_noswap && ct->np > 0 && ct->pdiv[ct->np - 1] == 1 &&
               !(ct->nq > 0 && ct->qdiv[ct->nq - 1] == 1);
    plan_kperm(ct, pl);
    plan_pack(ct, pl);
    plan_pads(ct, pl);
    plan_chunks(ct, pl);
    plan_skinny(ct, pl);
    plan_comb(ct, pl);
    if (pl->cfg.direct == 1 && pl->cfg.bk % 8u == 0)
        for (int side = 0; side < 2; side++) {
            pl->dvec[side] = direct_vec_side(ct, side);
            pl->dvec_buf[side] = ct->sep_buf[side];
        }
}

/* Contraction analysis without a device: returns 1 and fills M/N/K when the
 * kernel would take the matrix-core path. */
int dense_analyze(const UOpKernel *k, u32 *M, u32 *N, u32 *K, u32 *splits) {
    Contraction ct;
    if (!recognize(k, &ct)) return 0;
    GemmPlan pl;
    make_plan(&ct, &pl, 0);
    /* Matrix cores pay off once the contraction is more than a few hundred
     * thousand multiply-adds with a reduction of at least one K step: the
     * tile loaders then evaluate each operand element once instead of once
     * per output, and split-K spreads short outputs over the CUs. Smaller
     * ones stay on the generated kernels (one lane or workgroup per output). */
    if (!hipb.dense_force &&
        (ct.M < 2 || ct.N < 2 || ct.K < DENSE_MIN_K || (u64)ct.M * ct.N * ct.K < DENSE_MIN_WORK))
        return 0;
    if (M) *M = ct.M;
    if (N) *N = ct.N;
    if (K) *K = ct.K;
    if (splits) *splits = pl.splits;
    return 1;
}

/* Generated source of the matrix-core kernel (no device needed). */
char *dense_source(const UOpKernel *k) {
    Contraction ct;
    if (!dense_analyze(k, NULL, NULL, NULL, NULL) || !recognize(k, &ct)) return NULL;
    GemmPlan pl;
    make_plan(&ct, &pl, uop_signature(k));
    char err[128];
    return gen_gemm_source(k, &ct, &pl, err, sizeof err);
}

/* The unchecked loads of a K-reordered plan stay inside the buffers they
 * read: every index a side can form is below that buffer's element count,
 * and 16-byte loads start from 16-byte aligned buffers. */
static int kperm_fits(const GemmPlan *pl, const u32 *counts, void *const *ptrs) {
    const KPerm *kp = &pl->kp;
    for (int s = 0; s < 2; s++) {
        if (s == 1 && pl->pack) continue;    /* reads the pack buffer, sized K x N */
        if (kp->maxidx[s] >= counts[kp->buf[s]]) return 0;
        if (kp->vec[s] && ((uintptr_t)ptrs[kp->buf[s]] & 15u)) return 0;
    }
    return 1;
}

/* Records that a program is not a contraction (the entry dense_try_dispatch
 * would leave), without dispatching it: for a program that ran only fused
 * into another launch, so that a later dispatch without allocation finds it.
 * A contraction is left alone (its entry is made by its first dispatch). */
void dense_note_plain(const UOpKernel *k) {
    if (!k || k->n_leaves > FUSE_MAX_LEAVES) return;
    u64 key = uop_signature(k) ^ 0xD5E5E5E5D5E5E5E5ull;
    if (!key) key = 1;
    if (lookup(key, k)) return;
    u32 M, N, K, sp;
    if (dense_analyze(k, &M, &N, &K, &sp)) return;
    insert(key, k);
}

int dense_try_dispatch(u32 out_buf, const u32 *leaf_bufs, u32 n_leaves, const UOpKernel *k) {
    void *ptrs[FUSE_MAX_LEAVES + 1];
    u32 counts[FUSE_MAX_LEAVES + 1];
    if (k->n_leaves > FUSE_MAX_LEAVES) return 0;
    ptrs[0] = pool_ptr(out_buf);
    counts[0] = (u32)(pool_bytes(out_buf) / (k->out_dtype == DTYPE_F16 ? 2 : 4));
    for (u32 i = 0; i < k->n_leaves; i++) {
        void *lp = i < n_leaves ? pool_ptr(leaf_bufs[i]) : NULL;
        ptrs[i + 1] = lp ? lp : hipb.dummy;   /* loads index an absent buffer's element 0 */
        u64 b = lp ? pool_bytes(leaf_bufs[i]) : 0;
        counts[i + 1] = (u32)(b / (k->leaf_dtypes[i] == DTYPE_F16 ? 2 : 4));
    }
    u64 key = uop_signature(k) ^ 0xD5E5E5E5D5E5E5E5ull;
    if (!key) key = 1;
    DenseEntry *e = lookup(key, k);
    if (!e && hipb.noalloc) {
        hipb.noalloc_err = THVM_HIP_ENOTREADY;   /* never compiles without allocating */
        return 0;
    }
    if (!e) {
        e = insert(key, k);
        if (!e) return 0;
        Contraction ct;
        u32 M, N, K, sp;
        if (!dense_analyze(k, &M, &N, &K, &sp) || !recognize(k, &ct)) return 0;
        make_plan(&ct, &e->plan, uop_signature(k));
        if (e->plan.kp.on && !kperm_fits(&e->plan, counts, ptrs)) {
            memset(&e->plan.kp, 0, sizeof e->plan.kp);
            e->plan.pack = 0;
            plan_pads(&ct, &e->plan);
            plan_chunks(&ct, &e->plan);
            plan_comb(&ct, &e->plan);
        }
        char err[256] = {0};
        char *src = gen_gemm_source(k, &ct, &e->plan, err, sizeof err);
        if (!src) {
            fprintf(stderr, "tinyhvm-hip: dense kernel generation failed: %s\n", err);
            return 0;
        }
        if (hipb.dump_src) fprintf(stderr, "---- dense kernel ----\n%s\n", src);
        if (!rtc_build_module(src, &e->mod, err, sizeof err)) {
            fprintf(stderr, "tinyhvm-hip: dense kernel build failed: %s\n", err);
            free(src);
            return 0;
        }
        if (hipModuleGetFunction(&e->fn, e->mod, e->plan.name) != hipSuccess) {
            free(src);
            return 0;
        }
        co_form_make(&e->co, src, e->plan.name, dense_threads(&e->plan), e->fn);
        e->cap = rtc_capacity(e->fn, dense_threads(&e->plan));
        if (e->plan.pack) {
            char nm[64];
            snprintf(nm, sizeof nm, "%s_pack", e->plan.name);
            if (hipModuleGetFunction(&e->fn_pack, e->mod, nm) != hipSuccess) {
                free(src);
                return 0;
            }
            co_form_make(&e->co_pack, src, nm, 256, e->fn_pack);
        }
        if (e->plan.splits > 1) {
            char nm[64];
            snprintf(nm, sizeof nm, "%s_sum", e->plan.name);
            if (hipModuleGetFunction(&e->fn_sum, e->mod, nm) != hipSuccess) {
                free(src);
                return 0;
            }
            co_form_make(&e->co_sum, src, nm, 256, e->fn_sum);
        }
        free(src);
        e->M = ct.M;
        e->N = ct.N;
        e->is_dense = 1;
        if (plan_takes_epilogue(&e->plan, k) && !hipb.no_fuse) {
            e->kcopy = malloc(sizeof(UOpKernel));
            if (e->kcopy) memcpy(e->kcopy, k, sizeof(UOpKernel));
        }
        if (hipb.verbose)
            fprintf(stderr, "tinyhvm-hip: dense %s M=%u N=%u K=%u tile %s splits=%u kperm=%u\n", e->plan.name, ct.M,
                    ct.N, ct.K, e->plan.cfg.tag, e->plan.splits, e->plan.kp.on ? e->plan.kp.E : 0);
    }
    if (!e->is_dense) return 0;
    /* buffers smaller than the plan was made for: the generated kernels */
    if (e->plan.kp.on && !kperm_fits(&e->plan, counts, ptrs)) return 0;
    for (int side = 0; side < 2; side++)
        if (e->plan.dvec[side] && ((uintptr_t)ptrs[e->plan.dvec_buf[side]] & 15u)) return 0;
    if (e->plan.cfg.direct == 2 && e->plan.ske && e->plan.skmax != ~0ull && e->plan.skmax >= counts[e->plan.skbuf])
        return 0;
    if (e->plan.cfg.direct == 3 &&
        (e->plan.red_max[0] >= counts[e->plan.red_buf[0]] || e->plan.red_max[1] >= counts[e->plan.red_buf[1]]))
        return 0;
    for (u32 i = 0; i < n_leaves && i < FUSE_MAX_LEAVES; i++) pool_sync_device(leaf_bufs[i]);
    u32 tiles = e->plan.tiles_m * e->plan.tiles_n;
    const u32 threads = dense_threads(&e->plan);
    /* in-launch combine only when every workgroup of the grid is on the GPU at
     * once (the last split's workgroups wait for the others' words);
     * otherwise the partials go through the workspace and the sum kernel */
    unsigned long long *sl = NULL;
    if (e->plan.comb && (u64)tiles * e->plan.splits <= e->cap) sl = hipb.comb_slots;
    /* split-K workspace */
    float *ws = NULL;
    if (e->plan.splits > 1 && !sl) {
        ws = scratch_reserve(&D.ws, (u64)e->plan.splits * e->M * e->N * sizeof(float));
        if (!ws) return 0;
    }
    /* packed B side */
    float *pk = NULL;
    if (e->plan.pack) {
        pk = scratch_reserve(&D.pk, (u64)e->plan.kp.maxidx[1] * sizeof(float) + sizeof(float));
        if (!pk) return 0;
    }
    void *params[2 * (FUSE_MAX_LEAVES + 1) + 2];
    u32 nb = k->n_leaves + 1;
    for (u32 b = 0; b < nb; b++) {
        params[b] = &ptrs[b];
        params[nb + b] = &counts[b];
    }
    params[2 * nb] = &ws;
    params[2 * nb + 1] = e->plan.comb ? (void *)&sl : (void *)&pk;
    if (e->plan.pack) {
        void *pp[2 * (FUSE_MAX_LEAVES + 1) + 1];
        for (u32 b = 0; b < 2 * nb; b++) pp[b] = params[b];
        pp[2 * nb] = &pk;
        const u64 kn = e->plan.kp.maxidx[1] + 1;
        /* held: it goes out in one launch with the independent work held
         * before it (the forward convolution's pack with the padding of its
         * input), and the main kernel's launch below issues it first */
        HbMem hp;
        hp.n = 0;
        hbm_add(&hp, pk, kn * sizeof(float), 1);
        for (u32 i = 0; i < n_leaves && i < FUSE_MAX_LEAVES; i++)
            hbm_add(&hp, pool_ptr(leaf_bufs[i]), pool_bytes(leaf_bufs[i]), 0);
        if (!hipb_hold(&e->co_pack, e->fn_pack, (u32)((kn + 255) / 256), 1, pp, &hp, 0, -1, 0) &&
            !hipb_launch_grid(e->fn_pack, (u32)((kn + 255) / 256), 1, 256, pp))
            return 0;
    }
    /* held for a batch with the next independent dispatches (the split-K sum
     * then joins them, its main kernel going out first) */
    const u64 mn = (u64)e->M * e->N, wsb = (u64)e->plan.splits * mn * sizeof(float);
    HbMem hm;
    hm.n = 0;
    hbm_add(&hm, ws ? (void *)ws : ptrs[0], ws ? wsb : pool_bytes(out_buf), 1);
    for (u32 i = 0; i < n_leaves && i < FUSE_MAX_LEAVES; i++)
        hbm_add(&hm, pool_ptr(leaf_bufs[i]), pool_bytes(leaf_bufs[i]), 0);
    /* a timed contraction (thvm_hip_time_contraction) goes out on its own,
     * between its two events */
    const int timed = hipb.time_ev[0] != NULL;
    int held = !timed && !e->plan.pack && hipb_hold(&e->co, e->fn, tiles, e->plan.splits, params, &hm, sl != NULL,
                                                    sl ? (int)(2 * nb + 1) : -1, sl ? (u64)e->plan.splits * mn : 0);
    /* a larger launch that an elementwise consumer may still fuse into is
     * held alone if its workgroups use little LDS (the fused module adds no
     * LDS; big LDS tiles are the headline GEMMs, left as they are) */
    if (!held && !timed && e->kcopy && e->co.src && e->co.lds <= EPI_SOLO_MAX_LDS)
        held = hipb_hold_solo(&e->co, e->fn, tiles, e->plan.splits, params, &hm);
    if (!held) {
        /* wave tile with split tail tiles: S whole tiles per workgroup, then a
         * workgroup per split tile */
        const u32 gx = e->plan.tail_s ? e->plan.tail_full / e->plan.tail_s + (tiles - e->plan.tail_full) : tiles;
        if (timed) {
            hipb_before_stream();
            HIPB_CHECK(hipEventRecord((hipEvent_t)hipb.time_ev[0], hipb.stream));
        }
        const int ok = hipb_launch_grid(e->fn, gx, e->plan.splits, threads, params);
        if (timed) {
            HIPB_CHECK(hipEventRecord((hipEvent_t)hipb.time_ev[1], hipb.stream));
            hipb.time_ev[0] = hipb.time_ev[1] = NULL;
            hipb.time_fired = 1;
        }
        if (!ok) return 0;
    } else if (e->kcopy && !ws) {
        /* held: the next dispatch may fuse into its epilogue */
        hipb_hold_tag(key, e->serial, out_buf);
    }
    if (ws) {
        void *p2[] = {&ptrs[0], &counts[0], &ws};
        const u64 per_block = sum_per_wave(&e->plan, mn) ? 4 : 64;
        const u32 blocks = (u32)((mn + per_block - 1) / per_block);
        HbMem hs;
        hs.n = 0;
        hbm_add(&hs, ptrs[0], pool_bytes(out_buf), 1);
        hbm_add(&hs, ws, wsb, 0);
        if (!hipb_hold(&e->co_sum, e->fn_sum, blocks, 1, p2, &hs, 0, -1, 0) &&
            !hipb_launch_grid(e->fn_sum, blocks, 1, 256, p2))
            return 0;
    }
    return 1;
}

void dense_reset_stats(void) {}

void dense_shutdown(void) {
    if (D.tab) {
        for (u32 i = 0; i < D.cap; i++) {
            if (!D.tab[i].key) continue;
            if (D.tab[i].is_dense) HIPB_CHECK(hipModuleUnload(D.tab[i].mod));
            co_form_free(&D.tab[i].co);
            co_form_free(&D.tab[i].co_sum);
            co_form_free(&D.tab[i].co_pack);
            free(D.tab[i].kcopy);
            free(D.tab[i].ops);
        }
        free(D.tab);
    }
    for (u32 i = 0; i < F.n; i++) {
        if (F.e[i].fn) HIPB_CHECK(hipModuleUnload(F.e[i].mod));
        co_form_free(&F.e[i].co);
    }
    F.n = 0;
    scratch_release(&D.ws);
    scratch_release(&D.pk);
    memset(&D, 0, sizeof D);
}


/* Whether the elementwise program `c` can be the fused epilogue of a
 * contraction with M x N outputs that it reads as leaf buffer o_leaf (1 +
 * leaf): no loop, one STORE at gid, that leaf read only at gid and as f32,
 * as many outputs as the contraction. */
static int epi_fits(u32 M, u32 N, const UOpKernel *c, u32 o_leaf) {
    if (!c || o_leaf == 0 || o_leaf > c->n_leaves || c->n_leaves > FUSE_MAX_LEAVES || c->n_ops == 0 ||
        c->n_ops > KOP_MAX || c->leaf_dtypes[o_leaf - 1] != DTYPE_F32)
        return 0;
    const u32 total = c->local_size > 0 ? c->grid[0] : c->grid[0] * c->grid[1] * c->grid[2];
    if ((u64)total != (u64)M * N) return 0;
    Aff *aff = calloc(c->n_ops, sizeof(Aff));
    if (!aff) return 0;
    DCtx dc = {c, total, 1, -1, aff};
    analyze_aff(&dc);
    int ok = 1, stores = 0;
    for (u32 i = 0; i < c->n_ops && ok; i++) {
        const KOp *op = &c->ops[i];
        if (op->type == KOP_RANGE || op->type == KOP_ENDRANGE || op->type == KOP_ACC_INIT || op->type == KOP_ACC)
            ok = 0;
        else if (op->type == KOP_STORE) {
            stores++;
            ok = op->arg[0] < c->n_ops && aff_is_gid(&dc, &aff[op->arg[0]]);
        } else if (op->type == KOP_LOAD && op->imm.u == o_leaf)
            ok = op->arg[0] < c->n_ops && aff_is_gid(&dc, &aff[op->arg[0]]);
    }
    free(aff);
    return ok && stores == 1;
}

/* The fused module's source: the contraction's kernel (plan pl, its name
 * replaced by `name`) with c's program, a device function over c's own
 * buffers (the kernel's extra parameters q<b>, qc<b>), run by the lane that
 * stores each output on the value it stores. */
static char *epi_source(const UOpKernel *k, const Contraction *ct, const GemmPlan *pl0, const UOpKernel *c,
                        u32 o_leaf, const char *name, KGenScalars *sc, char *err, size_t errlen) {
    char *epi = malloc(65536), params[2048], call[2048];
    if (!epi || kgen_epilogue(c, o_leaf, epi, 65536, sc) < 0) {
        free(epi);
        snprintf(err, errlen, "epilogue generation failed");
        return NULL;
    }
    size_t wp = 0, wc = (size_t)snprintf(call, sizeof call, "epi_(o_, v_");
    for (u32 b = 0; b <= c->n_leaves; b++) {
        wp += (size_t)snprintf(params + wp, sizeof params - wp, ", char* q%u", b);
        wc += (size_t)snprintf(call + wc, sizeof call - wc, ", q%u", b);
    }
    for (u32 b = 0; b <= c->n_leaves; b++) {
        wp += (size_t)snprintf(params + wp, sizeof params - wp, ", u32 qc%u", b);
        wc += (size_t)snprintf(call + wc, sizeof call - wc, ", qc%u", b);
    }
    if (sc->n) {
        wp += (size_t)snprintf(params + wp, sizeof params - wp, ", u32 qsm_");
        wc += (size_t)snprintf(call + wc, sizeof call - wc, ", qsm_");
        for (u32 j = 0; j < sc->n; j++) {
            wp += (size_t)snprintf(params + wp, sizeof params - wp, ", float qsv%u", j);
            wc += (size_t)snprintf(call + wc, sizeof call - wc, ", qsv%u", j);
        }
    }
    snprintf(call + wc, sizeof call - wc, ")");
    GemmPlan pl = *pl0;
    snprintf(pl.name, sizeof pl.name, "%s", name);
    g_epi_src = epi;
    g_epi_params = params;
    g_epi_call = call;
    char *src = gen_gemm_source(k, ct, &pl, err, errlen);
    g_epi_src = g_epi_params = g_epi_call = NULL;
    free(epi);
    return src;
}

/* The contraction (key, serial) held for launch with the elementwise program
 * `c`, which reads its output as leaf buffer o_leaf, fused into its
 * epilogue (the same arithmetic as the two launches). Returns 1 with the
 * fused module's function and co-launch form, 0 when the pair does not fuse
 * (remembered, like the modules, per pair). */
int dense_epilogue(u64 key, u32 serial, const UOpKernel *c, u32 o_leaf, hipFunction_t *fn, CoForm *co,
                   KGenScalars *sc) {
    if (hipb.no_fuse || !c || o_leaf == 0 || o_leaf > c->n_leaves) return 0;
    u64 fk = key ^ (uop_signature(c) * 0x9E3779B97F4A7C15ull) ^ ((u64)o_leaf << 56) ^ ((u64)serial << 40);
    if (!fk) fk = 1;
    for (u32 i = 0; i < F.n; i++)
        if (F.e[i].key == fk) {
            if (!F.e[i].fn) return 0;
            *fn = F.e[i].fn;
            *co = F.e[i].co;
            *sc = F.e[i].sc;
            return 1;
        }
    if (F.n >= FUSED_MAX) return 0;
    FusedEntry *fe = &F.e[F.n++];
    memset(fe, 0, sizeof *fe);
    fe->key = fk;
    DenseEntry *e = NULL;
    for (u32 i = 0; D.tab && i < D.cap && !e; i++)
        if (D.tab[i].key == key && D.tab[i].serial == serial && D.tab[i].is_dense && D.tab[i].kcopy) e = &D.tab[i];
    Contraction ct;
    if (!e || !epi_fits(e->M, e->N, c, o_leaf) || !recognize(e->kcopy, &ct)) return 0;
    char name[48], err[256] = {0};
    snprintf(name, sizeof name, "thvm_gemmep_%08x", (u32)(fk & 0xFFFFFFFFu));
    char *src = epi_source(e->kcopy, &ct, &e->plan, c, o_leaf, name, &fe->sc, err, sizeof err);
    if (!src) return 0;
    if (hipb.dump_src) fprintf(stderr, "---- dense kernel with fused epilogue ----\n%s\n", src);
    if (!rtc_build_module(src, &fe->mod, err, sizeof err)) {
        fprintf(stderr, "tinyhvm-hip: fused epilogue build failed: %s\n", err);
        free(src);
        return 0;
    }
    hipFunction_t f = NULL;
    if (hipModuleGetFunction(&f, fe->mod, name) != hipSuccess ||
        !co_form_make(&fe->co, src, name, dense_threads(&e->plan), f) ||
        fe->co.np != e->co.np + 2u * (c->n_leaves + 1u) + (fe->sc.n ? 1u + fe->sc.n : 0u)) {
        HIPB_CHECK(hipModuleUnload(fe->mod));
        co_form_free(&fe->co);
        free(src);
        return 0;
    }
    free(src);
    fe->fn = f;
    hipb.n_compile++;
    if (hipb.verbose)
        fprintf(stderr, "tinyhvm-hip: %s = %s + epilogue thvm_%s_%08x\n", name, e->plan.name, "ew",
                (u32)(uop_signature(c) & 0xFFFFFFFFu));
    *fn = f;
    *co = fe->co;
    *sc = fe->sc;
    return 1;
}

/* Device-free: the fused module of contraction k and elementwise program c
 * (reading k's output as leaf buffer o_leaf) when the pair fuses, else NULL
 * with the reason in err. */
char *dense_epilogue_source(const UOpKernel *k, const UOpKernel *c, u32 o_leaf, char *err, size_t errlen) {
    Contraction ct;
    if (!dense_analyze(k, NULL, NULL, NULL, NULL) || !recognize(k, &ct)) {
        snprintf(err, errlen, "not a matrix-core contraction");
        return NULL;
    }
    GemmPlan pl;
    make_plan(&ct, &pl, uop_signature(k));
    if (!plan_takes_epilogue(&pl, k)) {
        snprintf(err, errlen, "the contraction's plan takes no epilogue");
        return NULL;
    }
    if (!epi_fits(ct.M, ct.N, c, o_leaf)) {
        snprintf(err, errlen, "not an elementwise consumer of the output at its own index");
        return NULL;
    }
    KGenScalars sc;
    return epi_source(k, &ct, &pl, c, o_leaf, "thvm_gemmep_check", &sc, err, errlen);
}
