/*
 * window.c - hand-written kernels for the pooling windows and the
 * per-channel reductions of the engine's max-pool and batchnorm.
 *
 * The engine has no max-pool or batchnorm op on this path. thvm_maxpool2d
 * (src/nn/conv.c:484-514) is an RMAX over the window axes of a pool view,
 * and batchnorm (src/nn/batchnorm.c:35-111) is built from SUMs over axes
 * [0,2,3] and elementwise kernels. Both reach the backend as KOp programs of
 * the form
 *     acc = init;  for r in [0,T): acc = acc (+|max) f(loads(gid, r));  out[gid] = acc
 * This file recognises two such shapes, with the digit analysis of
 * affine.c, and runs them on kernels written for them:
 *
 *   window max      RMAX over a small window (T <= 16): one load whose index
 *                   is base(gid) + off(r). Each output is one lane; the
 *                   window's elements are read with 8- or 16-byte loads
 *                   (lanes along the output columns read contiguous memory,
 *                   where the generated kernel's 4-byte loads sit two floats
 *                   apart), and the maximum is taken in the engine's r order
 *                   with its rule acc > v ? acc : v, so the result, tied and
 *                   signed zeros and NaNs included, is the engine's bit for
 *                   bit (src/backend/cpu/uop.c:80-88).
 *   run sums        SUM over a long loop (T >= 4096) of an elementwise
 *                   function of loads that either read contiguous runs along
 *                   r (a channel's image rows, [0,2,3]: runs of H*W floats, one
 *                   per image) or do not depend on r (a per-channel mean).
 *                   The reduction is split over workgroups along the runs;
 *                   lanes read 16-byte vectors and keep per-lane partials in
 *                   sequence; a wavefront shuffle tree and an LDS tree give a
 *                   workgroup's partial, and the last workgroup of each output
 *                   combines the partials in index order in the same launch
 *                   (the single-pass combine of the generator's prelude). The
 *                   order of the sum differs from the engine's serial one:
 *                   tolerance 1e-4 normwise.
 *
 * Anything else, or a dispatch whose buffers are smaller than the plan's
 * largest index or not aligned for its vector loads, takes the generated
 * kernels.
 */
#include <stdarg.h>
#include <stdlib.h>
#include <string.h>

#include "hipb.h"
#include "thvm_hip.h"
#include "affine.h"

#define WIN_MAX_TRIP 16          /* window max: at most this many elements per window */
#define WIN_SUM_MIN_TRIP 4096    /* run sums: reductions at least this long */
#define WIN_SUM_MIN_RUN 16       /* ... over contiguous runs at least this long */
#define WIN_SUM_TARGET_WG 1024   /* workgroups to aim for in all (256 lanes each: all resident at once) */
#define WIN_SUM_MIN_CHUNK 512    /* vectors per workgroup, at least */
#define WIN_SUM_MAX_OUTPUTS 256  /* run sums: few outputs (more take the generated group kernels) */
#define WIN_SUM_MAX_FIXED 16     /* run sums: vectors per lane up to which all loads are issued at once */
#define WIN_MAX_LOADS 16
#define WIN_BLOCK 256u

enum { WIN_NONE = 0, WIN_MAX = 1, WIN_SUM = 2 };

typedef struct {
    int kind;
    u32 total;                   /* outputs (= gids) */
    u32 trip;                    /* loop length */
    u32 init_bits;               /* the accumulator's initial value */
    u32 R, E, acc, value;        /* op indices: RANGE, ENDRANGE, ACC, accumulated value */
    u32 n_ld;
    u32 ld_op[WIN_MAX_LOADS];
    Aff ld_aff[WIN_MAX_LOADS];
    u8 ld_r[WIN_MAX_LOADS];      /* the index depends on r */
    u64 ld_max[WIN_MAX_LOADS];   /* the largest index it forms */
    u32 W;                       /* elements per vector load: 2 or 4 (window max), 1 or 4 (sums) */
    /* window max */
    u32 off[WIN_MAX_TRIP];       /* r-offset of window element r */
    u64 cover_max;               /* the largest index its vector loads touch */
    /* run sums */
    u32 L;                       /* run length along r */
    u32 n_outer;
    u32 outer_div[DG_MAX], outer_mod[DG_MAX], outer_coef[DG_MAX];
    u32 S;                       /* workgroups per output */
    u32 unroll;                  /* run sums: loop unroll */
    int launch;                  /* run sums: partials through a workspace and a combine kernel */
    u32 U;                       /* window max: units (outputs, or pairs of outputs) per lane */
    u32 P;                       /* window max: adjacent outputs per vector load (1 or 2) */
    u32 c1;                      /* window max: input step between adjacent outputs */
    u8 cone[KOP_MAX];
} WinPlan;

static u32 env_u32(const char *name, u32 dflt) {
    const char *e = getenv(name);
    return e && e[0] ? (u32)atoi(e) : dflt;
}

/* ---------------- recognition ---------------- */

static int win_debug(void) {
    static int v = -1;
    if (v < 0) { const char *e = getenv("THVM_HIP_WINDOW_DEBUG"); v = e && e[0] == '1'; }
    return v;
}
#define WREJECT(why) do { if (win_debug()) fprintf(stderr, "window: not recognised: %s\n", why); return 0; } while (0)

static int alu_unary(u32 uop) {
    return uop == UOP_NEG || uop == UOP_EXP || uop == UOP_LOG || uop == UOP_RELU || uop == UOP_CAST || uop == UOP_SQRT;
}

/* Index sums must not wrap in u32 (the kernel computes them in u32, the
 * plan in u64): small coefficients and constant, and a largest value below
 * 2^32. */
static int aff_no_wrap(const DCtx *c, const Aff *a) {
    if (!a->ok || a->cst >= 0x80000000u) return 0;
    for (u32 t = 0; t < a->n; t++)
        if (a->coef[t] >= 0x80000000u) return 0;
    return aff_max(c, a) < 0xFFFFFFFFull;
}

static int same_r_part(const Aff *a, const Aff *b) {
    u32 na = 0, nb = 0;
    for (u32 t = 0; t < a->n; t++) na += a->d[t].var == 1;
    for (u32 t = 0; t < b->n; t++) nb += b->d[t].var == 1;
    if (na != nb) return 0;
    for (u32 t = 0; t < a->n; t++) {
        if (a->d[t].var != 1) continue;
        int found = 0;
        for (u32 u = 0; u < b->n; u++)
            if (b->d[u].var == 1 && b->d[u].div == a->d[t].div && b->d[u].mod == a->d[t].mod &&
                b->coef[u] == a->coef[t]) found = 1;
        if (!found) return 0;
    }
    return 1;
}

static int win_recognize(const UOpKernel *k, WinPlan *p) {
    memset(p, 0, sizeof *p);
    char err[128];
    if (!kgen_validate(k, err, sizeof err)) WREJECT("invalid program");
    if (k->out_dtype != DTYPE_F32) WREJECT("output not f32");
    i32 R = -1, E = -1;
    for (u32 i = 0; i < k->n_ops; i++) {
        if (k->ops[i].type == KOP_RANGE) {
            if (R >= 0) WREJECT("more than one loop");
            R = (i32)i;
        } else if (k->ops[i].type == KOP_ENDRANGE) {
            E = (i32)i;
        }
    }
    if (R < 0 || E < 0) WREJECT("no loop");
    if ((u32)E + 2 != k->n_ops) WREJECT("ops after the store");
    const KOp *st = &k->ops[E + 1];
    if (st->type != KOP_STORE) WREJECT("no store after the loop");
    u32 t = st->arg[1];
    if (t >= (u32)R || k->ops[t].type != KOP_ACC_INIT) WREJECT("store is not the accumulator");
    i32 acc = -1;
    for (u32 i = 0; i < k->n_ops; i++) {
        if (k->ops[i].type != KOP_ACC) continue;
        if (acc >= 0 || i <= (u32)R || i >= (u32)E || k->ops[i].arg[0] != t) WREJECT("accumulators");
        acc = (i32)i;
    }
    if (acc < 0) WREJECT("no accumulation");
    for (u32 i = 0; i < (u32)R; i++)
        if (op_type_is_float(k->ops[i].type) && i != t) WREJECT("float work before the loop");
    u32 value = k->ops[acc].arg[1];
    if (value <= (u32)R || value >= (u32)acc || !op_type_is_float(k->ops[value].type)) WREJECT("accumulated value");
    mark_cone(k, value, p->cone);
    if (p->cone[t]) WREJECT("the accumulator feeds its own value");
    for (u32 i = (u32)R + 1; i < (u32)E; i++) {
        const KOp *op = &k->ops[i];
        if (i == (u32)acc || !op_type_is_float(op->type)) continue;
        if (!p->cone[i]) WREJECT("float work outside the accumulated value");
        if (op->type == KOP_MASK || op->type == KOP_ACC_INIT) WREJECT("masked or nested accumulation");
        if (op->type == KOP_ALU) {
            if (!op_type_is_float(k->ops[op->arg[0]].type)) WREJECT("integer operand");
            if (!alu_unary(op->imm.u) && !op_type_is_float(k->ops[op->arg[1]].type)) WREJECT("integer operand");
        }
        if (op->type == KOP_LOAD) {
            u32 bi = op->imm.u;
            if (bi == 0 || bi > k->n_leaves || k->leaf_dtypes[bi - 1] != DTYPE_F32) WREJECT("load buffer");
            if (p->n_ld >= WIN_MAX_LOADS) WREJECT("too many loads");
            p->ld_op[p->n_ld++] = i;
        }
    }
    u64 total = k->local_size > 0 ? (u64)k->grid[0] : (u64)k->grid[0] * k->grid[1] * k->grid[2];
    if (total == 0 || total > 0xFFFFFFFFull) WREJECT("launch size");
    p->total = (u32)total;
    p->trip = k->ops[R].imm.u;
    if (p->trip == 0) WREJECT("empty loop");
    p->init_bits = k->ops[t].imm.u;
    p->R = (u32)R;
    p->E = (u32)E;
    p->acc = (u32)acc;
    p->value = value;

    Aff aff[KOP_MAX];
    DCtx c = {k, p->total, p->trip, R, aff};
    analyze_aff(&c);
    const Aff *sa = &aff[st->arg[0]];
    int is_gid = sa->ok && sa->cst == 0 &&
                 ((sa->n == 1 && sa->coef[0] == 1 && sa->d[0].var == 0 && sa->d[0].div == 1 && sa->d[0].mod == 0) ||
                  (sa->n == 0 && p->total == 1));   /* one output: gid is the constant 0 */
    if (!is_gid) WREJECT("store index is not gid");
    for (u32 j = 0; j < p->n_ld; j++) {
        const Aff *a = &aff[k->ops[p->ld_op[j]].arg[0]];
        if (!aff_no_wrap(&c, a)) WREJECT("load index not a bounded digit sum");
        p->ld_aff[j] = *a;
        p->ld_max[j] = aff_max(&c, a);
        for (u32 q = 0; q < a->n; q++) p->ld_r[j] |= a->d[q].var == 1;
    }

    if (k->ops[acc].imm.u == UOP_RMAX) {
        /* window max: the accumulated value is the one load itself */
        if (p->trip > WIN_MAX_TRIP || p->n_ld != 1 || p->ld_op[0] != value) WREJECT("not a window max");
        const Aff *a = &p->ld_aff[0];
        for (u32 r = 0; r < p->trip; r++) p->off[r] = (u32)(aff_eval(a, 0, r) - a->cst);
        for (u32 W = 4; W >= 2; W /= 2) {
            int ok = a->cst % W == 0;
            for (u32 q = 0; q < a->n; q++)
                if (a->d[q].var == 0 && a->coef[q] % W) ok = 0;
            /* vectors cover the window with little waste */
            u32 groups[WIN_MAX_TRIP], ng = 0;
            for (u32 r = 0; r < p->trip && ok; r++) {
                u32 g = p->off[r] / W, seen = 0;
                for (u32 x = 0; x < ng; x++) seen |= groups[x] == g;
                if (!seen) groups[ng++] = g;
            }
            if (ok && ng * W <= 2 * p->trip) {
                p->W = W;
                u32 max_off = 0, end = 0;
                for (u32 r = 0; r < p->trip; r++) if (p->off[r] > max_off) max_off = p->off[r];
                for (u32 x = 0; x < ng; x++) if (groups[x] * W + W - 1 > end) end = groups[x] * W + W - 1;
                p->cover_max = p->ld_max[0] - max_off + end;
                break;
            }
        }
        if (!p->W) WREJECT("window rows not vector aligned");
        /* pairs of adjacent outputs in one 16-byte vector: the innermost output
         * digit steps the input by c1, every window element and its
         * neighbour's sit in the same aligned 4 floats */
        p->P = 1;
        if (env_u32("THVM_HIP_WIN_PAIR", 1)) {
            int inner = -1, ok = a->cst % 4 == 0 && p->total % 2 == 0;
            for (u32 q = 0; q < a->n; q++) {
                if (a->d[q].var != 0) continue;
                if (a->d[q].div == 1) inner = (int)q;
                else if (a->coef[q] % 4) ok = 0;
            }
            if (inner < 0 || a->d[inner].mod % 2 || (2 * a->coef[inner]) % 4) ok = 0;
            u32 c1 = inner >= 0 ? a->coef[inner] : 0;
            for (u32 r = 0; r < p->trip && ok; r++)
                if (p->off[r] % 4 + c1 > 3) ok = 0;
            if (ok) {
                p->P = 2;
                p->W = 4;
                p->c1 = c1;
                u32 max_off = 0, end = 0;
                for (u32 r = 0; r < p->trip; r++) {
                    if (p->off[r] > max_off) max_off = p->off[r];
                    if (p->off[r] / 4 * 4 + 3 > end) end = p->off[r] / 4 * 4 + 3;
                }
                /* the last output of a pair is odd: its vectors end where the even one's do */
                p->cover_max = p->ld_max[0] - max_off - c1 + end;
            }
        }
        p->U = env_u32("THVM_HIP_WIN_OUT", 2);
        if (p->U != 1 && p->U != 2 && p->U != 4 && p->U != 8) p->U = 2;
        p->kind = WIN_MAX;
        return 1;
    }
    if (k->ops[acc].imm.u != UOP_SUM) WREJECT("reduction type");
    if (p->trip < WIN_SUM_MIN_TRIP) WREJECT("short reduction");
    if (p->total > WIN_SUM_MAX_OUTPUTS) WREJECT("many outputs");
    /* run sums: every r-dependent load has the same r part, a contiguous run
     * (digits div = run, coef = run, from run 1) and outer digits beyond it */
    i32 first = -1;
    for (u32 j = 0; j < p->n_ld; j++) {
        if (!p->ld_r[j]) continue;
        if (first < 0) first = (i32)j;
        else if (!same_r_part(&p->ld_aff[first], &p->ld_aff[j])) WREJECT("loads with different r parts");
    }
    if (first < 0) WREJECT("nothing depends on r");
    const Aff *a = &p->ld_aff[first];
    u8 inner[DG_MAX] = {0};
    u64 run = 1;
    for (;;) {
        int hit = -1;
        for (u32 q = 0; q < a->n; q++)
            if (a->d[q].var == 1 && !inner[q] && a->d[q].div == run && a->coef[q] == run) hit = (int)q;
        if (hit < 0) break;
        inner[hit] = 1;
        if (!a->d[hit].mod) { run = p->trip; break; }
        run *= a->d[hit].mod;
        if (run >= p->trip) { run = p->trip; break; }
    }
    if (run < WIN_SUM_MIN_RUN || p->trip % run) WREJECT("no long contiguous runs");
    p->L = (u32)run;
    for (u32 q = 0; q < a->n; q++) {
        if (a->d[q].var != 1 || inner[q]) continue;
        if (a->d[q].div < p->L || a->d[q].div % p->L) WREJECT("outer digit inside a run");
        if (p->n_outer >= DG_MAX) WREJECT("too many outer digits");
        p->outer_div[p->n_outer] = a->d[q].div / p->L;
        p->outer_mod[p->n_outer] = a->d[q].mod;
        p->outer_coef[p->n_outer] = a->coef[q];
        p->n_outer++;
    }
    /* 16-byte vectors when every run and every base is 4-float aligned */
    p->W = p->L % 4 == 0 ? 4 : 1;
    for (u32 j = 0; j < p->n_ld && p->W == 4; j++) {
        if (!p->ld_r[j]) continue;
        const Aff *b = &p->ld_aff[j];
        if (b->cst % 4) p->W = 1;
        for (u32 q = 0; q < b->n; q++)
            if ((b->d[q].var == 0 || !(b->d[q].div < p->L)) && b->coef[q] % 4) p->W = 1;
    }
    u32 units = p->trip / p->W;
    /* workgroups per output: up to the number the GPU holds at once (the
     * combine then stays in the launch), each with at least a minimum chunk */
    p->S = 1;
    while (p->S < 1024 && (u64)p->total * p->S * 2 <= WIN_SUM_TARGET_WG && units / (p->S * 2) >= WIN_SUM_MIN_CHUNK)
        p->S *= 2;
    {
        u32 fs = env_u32("THVM_HIP_WIN_S", 0);
        if (fs && (fs & (fs - 1)) == 0 && fs <= 1024) p->S = fs;
    }
    p->unroll = env_u32("THVM_HIP_WIN_UNROLL", 2);
    if (p->unroll < 1 || p->unroll > 16) p->unroll = 2;
    {
        const char *e = getenv("THVM_HIP_WIN_COMBINE");
        if (e && strcmp(e, "single") == 0) p->launch = 0;
        else if (e && strcmp(e, "launch") == 0) p->launch = 1;
        else p->launch = 0;
    }
    /* one pass only when the whole grid is on the GPU at once */
    if (p->S > 1 && !p->launch &&
        ((u64)p->total * p->S > COMB_SLOTS || (u64)p->total * p->S * (WIN_BLOCK / 64) > hipb_resident_waves()))
        p->launch = 1;
    if ((u64)p->total * p->S > 0xFFFFFFFFull / WIN_BLOCK) WREJECT("launch size");
    p->kind = WIN_SUM;
    return 1;
}

/* ---------------- code generation ---------------- */

typedef struct { char *p; size_t n, cap; } WSB;
static void wsb_put(WSB *s, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
static void wsb_put(WSB *s, const char *fmt, ...) {
    va_list ap;
    for (;;) {
        size_t room = s->cap - s->n;
        va_start(ap, fmt);
        int w = s->p ? vsnprintf(s->p + s->n, room, fmt, ap) : -1;
        va_end(ap);
        if (w >= 0 && (size_t)w < room) { s->n += (size_t)w; return; }
        size_t nc = s->cap ? s->cap * 2 : 16384;
        while (w >= 0 && nc < s->n + (size_t)w + 1) nc *= 2;
        char *np = realloc(s->p, nc);
        if (!np) return;
        s->p = np;
        s->cap = nc;
    }
}

/* gid part of a load's index as a u32 expression of the variable `g` */
static void emit_base_expr(WSB *s, const Aff *a, const char *g) {
    wsb_put(s, "%uu", a->cst);
    for (u32 q = 0; q < a->n; q++) {
        if (a->d[q].var != 0) continue;
        if (a->d[q].mod) wsb_put(s, " + %uu * ((%s / %uu) %% %uu)", a->coef[q], g, a->d[q].div, a->d[q].mod);
        else wsb_put(s, " + %uu * (%s / %uu)", a->coef[q], g, a->d[q].div);
    }
}

/* gid part of a load's index as a u32 expression of `gid` */
static void emit_base(WSB *s, const char *name, const Aff *a) {
    wsb_put(s, "  const u32 %s = %uu", name, a->cst);
    for (u32 q = 0; q < a->n; q++) {
        if (a->d[q].var != 0) continue;
        if (a->d[q].mod) wsb_put(s, " + %uu * ((gid / %uu) %% %uu)", a->coef[q], a->d[q].div, a->d[q].mod);
        else wsb_put(s, " + %uu * (gid / %uu)", a->coef[q], a->d[q].div);
    }
    wsb_put(s, ";\n");
}

static void float_bits(char *out, size_t n, u32 bits) { snprintf(out, n, "__uint_as_float(0x%08xu)", bits); }

static char *gen_window_max(const UOpKernel *k, const WinPlan *p, const char *name) {
    WSB s = {0};
    (void)k;
    const u32 U = p->U, P = p->P;
    const u64 units = (u64)p->total / P;          /* P = 2 only when total is even */
    const u64 lanes = (units + U - 1) / U;
    /* one vector per distinct group of W elements, in first-use order */
    u32 groups[WIN_MAX_TRIP], ng = 0;
    for (u32 r = 0; r < p->trip; r++) {
        u32 g = p->off[r] / p->W, seen = 0;
        for (u32 x = 0; x < ng; x++) seen |= groups[x] == g;
        if (!seen) groups[ng++] = g;
    }
    const char *vt = p->W == 4 ? "v4f_" : "v2f_";
    wsb_put(&s, "%s\n", kgen_prelude());
    wsb_put(&s, "typedef float v2f_ __attribute__((ext_vector_type(2)));\n");
    wsb_put(&s, "extern \"C\" __global__ __launch_bounds__(%u) void %s(char* p0, const char* px) {\n", WIN_BLOCK, name);
    wsb_put(&s, "  const unsigned long long t_ = ((unsigned long long)blockIdx.y * gridDim.x + blockIdx.x) * %uull + "
                "threadIdx.x;\n", WIN_BLOCK);
    wsb_put(&s, "  if (t_ >= %lluull) return;\n", (unsigned long long)lanes);
    /* lane t takes units t, t + lanes, ... (a unit: P adjacent outputs); a
     * unit past the end reads unit 0's windows (in range) and stores nothing */
    for (u32 j = 0; j < U; j++) {
        char g[16];
        snprintf(g, sizeof g, "g%u_", j);
        wsb_put(&s, "  const u32 o%u_ = (u32)t_ + %lluu;\n", j, (unsigned long long)(lanes * j));
        wsb_put(&s, "  const u32 g%u_ = (o%u_ < %lluu) ? o%u_ * %uu : 0u;\n", j, j, (unsigned long long)units, j, P);
        wsb_put(&s, "  const u32 b%u_ = ", j);
        emit_base_expr(&s, &p->ld_aff[0], g);
        wsb_put(&s, ";\n");
    }
    /* every unit's loads before any use: U * groups loads in flight per lane */
    for (u32 j = 0; j < U; j++)
        for (u32 x = 0; x < ng; x++)
            wsb_put(&s, "  const %s v%u_%u_ = __builtin_nontemporal_load((const %s*)((const float*)px + b%u_ + %uu));\n",
                    vt, j, x, vt, j, groups[x] * p->W);
    char fb[64];
    float_bits(fb, sizeof fb, p->init_bits);
    static const char comp[4] = {'x', 'y', 'z', 'w'};
    for (u32 j = 0; j < U; j++) {
        wsb_put(&s, "  if (o%u_ < %lluu) {\n", j, (unsigned long long)units);
        for (u32 q = 0; q < P; q++) {
            wsb_put(&s, "    float a%u_ = %s;\n", q, fb);
            for (u32 r = 0; r < p->trip; r++) {
                u32 g = p->off[r] / p->W, x = 0;
                while (groups[x] != g) x++;
                wsb_put(&s, "    { const float e_ = v%u_%u_.%c; a%u_ = (a%u_ > e_) ? a%u_ : e_; }\n", j, x,
                        comp[(p->off[r] + q * p->c1) % p->W], q, q, q);
            }
        }
        if (P == 2) wsb_put(&s, "    *(float2*)((float*)p0 + g%u_) = make_float2(a0_, a1_);\n  }\n", j);
        else wsb_put(&s, "    ((float*)p0)[g%u_] = a0_;\n  }\n", j);
    }
    wsb_put(&s, "}\n");
    return s.p;
}

/* one body op for vector component v (loads were emitted before) */
static void emit_body_op(WSB *s, const UOpKernel *k, const WinPlan *p, u32 i, u32 v) {
    const KOp *op = &k->ops[i];
    char a[64], b[64], x[256], fb[64];
    switch (op->type) {
    case KOP_CONST_F:
        float_bits(fb, sizeof fb, op->imm.u);
        wsb_put(s, "    const float f%u_%u = %s;\n", i, v, fb);
        break;
    case KOP_ALU:
        snprintf(a, sizeof a, "f%u_%u", op->arg[0], v);
        snprintf(b, sizeof b, "f%u_%u", alu_unary(op->imm.u) ? op->arg[0] : op->arg[1], v);
        kgen_alu_expr(op->imm.u, op->arg[2], a, b, x, sizeof x);
        wsb_put(s, "    const float f%u_%u = %s;\n", i, v, x);
        break;
    default:
        break;
    }
    (void)p;
}

/* The combining workgroup's sum of an output's S partials into w_: lane l
 * adds partials l, l + 256, ... in that order (its own, t, in place of the
 * last one). With more than one per lane, all of the lane's words are read
 * first and then waited for (one round trip instead of one per word) and
 * cleared after every wait. */
static void emit_take_all(WSB *s, u32 S, const char *t, const char *o_expr) {
    if (S <= WIN_BLOCK) {
        wsb_put(s, "    float w_ = 0.0f;\n"
                   "    for (u32 s2_ = lane; s2_ < %uu; s2_ += %uu)\n"
                   "      w_ = w_ + ((s2_ == %uu) ? %s : comb_take(sl_, %s, s2_, %uu));\n",
                S, WIN_BLOCK, S - 1, t, o_expr, S);
        return;
    }
    const u32 nq = (S + WIN_BLOCK - 1) / WIN_BLOCK;
    wsb_put(s, "    float w_ = 0.0f;\n    {\n      unsigned long long* const w0_ = sl_ + (unsigned long long)(%s) * %uu;\n",
            o_expr, S);
    for (u32 q = 0; q < nq; q++)
        wsb_put(s, "      const u32 s%u_ = lane + %uu;\n"
                   "      const unsigned long long k%u_ = (s%u_ < %uu && s%u_ != %uu) ? comb_peek(w0_ + s%u_) : 0ull;\n",
                q, q * WIN_BLOCK, q, q, S, q, S - 1, q);
    for (u32 q = 0; q < nq; q++)
        wsb_put(s, "      if (s%u_ < %uu) w_ = w_ + ((s%u_ == %uu) ? %s : comb_ready(w0_ + s%u_, k%u_));\n", q, S, q,
                S - 1, t, q, q);
    for (u32 q = 0; q < nq; q++)
        wsb_put(s, "      if (s%u_ < %uu && s%u_ != %uu) comb_clear(w0_ + s%u_);\n", q, S, q, S - 1, q);
    wsb_put(s, "    }\n");
}

static char *gen_run_sum(const UOpKernel *k, const WinPlan *p, const char *name) {
    WSB s = {0};
    const u32 W = p->W, L4 = p->L / W, units = p->trip / W;
    const u32 chunk = (units + p->S - 1) / p->S;
    wsb_put(&s, "%s\n", kgen_prelude());
    wsb_put(&s, "extern \"C\" __global__ __launch_bounds__(%u) void %s(char* p0", WIN_BLOCK, name);
    for (u32 i = 0; i < k->n_leaves; i++) wsb_put(&s, ", const char* p%u", i + 1);
    if (p->S > 1 && p->launch) wsb_put(&s, ", float* ws_) {\n");
    else wsb_put(&s, ", unsigned long long* sl_) {\n");
    wsb_put(&s, "  __shared__ float red_[%u];\n", WIN_BLOCK / 64);
    wsb_put(&s, "  const u32 gid = blockIdx.x / %uu, sp_ = blockIdx.x %% %uu;\n", p->S, p->S);
    wsb_put(&s, "  const u32 lane = threadIdx.x;\n");
    for (u32 j = 0; j < p->n_ld; j++) {
        char nm[16];
        snprintf(nm, sizeof nm, "b%u_", p->ld_op[j]);
        emit_base(&s, nm, &p->ld_aff[j]);
        if (!p->ld_r[j])
            wsb_put(&s, "  const float h%u_ = ((const float*)p%u)[b%u_];\n", p->ld_op[j],
                    k->ops[p->ld_op[j]].imm.u, p->ld_op[j]);
    }
    for (u32 v = 0; v < W; v++) wsb_put(&s, "  float q%u_ = 0.0f;\n", v);
    wsb_put(&s, "  const u32 ulo_ = sp_ * %uu, uhi_ = (ulo_ + %uu < %uu) ? ulo_ + %uu : %uu;\n", chunk, chunk, units,
            chunk, units);
    /* a lane's vectors: a fixed count when it is small, every load of the
     * lane then in flight at once (the last ones past the chunk read its
     * first vector and add nothing); else a loop */
    const u32 nit = (chunk + WIN_BLOCK - 1) / WIN_BLOCK;
    const int fixed = nit <= WIN_SUM_MAX_FIXED;
    if (fixed) {
        wsb_put(&s, "  #pragma unroll\n  for (u32 i_ = 0; i_ < %uu; i_++) {\n", nit);
        wsb_put(&s, "    const u32 uu_ = ulo_ + lane + i_ * %uu;\n    const bool ok_ = uu_ < uhi_;\n"
                    "    const u32 u_ = ok_ ? uu_ : ulo_;\n", WIN_BLOCK);
    } else {
        wsb_put(&s, "  #pragma unroll %u\n  for (u32 u_ = ulo_ + lane; u_ < uhi_; u_ += %uu) {\n", p->unroll, WIN_BLOCK);
    }
    wsb_put(&s, "    const u32 s_ = u_ / %uu, j_ = u_ - s_ * %uu;\n", L4, L4);
    wsb_put(&s, "    const u32 o_ = j_ * %uu", W);
    for (u32 q = 0; q < p->n_outer; q++) {
        if (p->outer_mod[q])
            wsb_put(&s, " + %uu * ((s_ / %uu) %% %uu)", p->outer_coef[q], p->outer_div[q], p->outer_mod[q]);
        else
            wsb_put(&s, " + %uu * (s_ / %uu)", p->outer_coef[q], p->outer_div[q]);
    }
    wsb_put(&s, ";\n");
    /* the body in op order, each op once per vector component */
    for (u32 i = p->R + 1; i < p->acc; i++) {
        if (!p->cone[i] || !op_type_is_float(k->ops[i].type)) continue;
        if (k->ops[i].type == KOP_LOAD) {
            u32 j = 0;
            while (p->ld_op[j] != i) j++;
            u32 bi = k->ops[i].imm.u;
            if (!p->ld_r[j]) {
                for (u32 v = 0; v < W; v++) wsb_put(&s, "    const float f%u_%u = h%u_;\n", i, v, i);
            } else if (W == 4) {
                wsb_put(&s, "    const float4 t%u_ = ld4nt_u(p%u, b%u_ + o_);\n", i, bi, i);
                wsb_put(&s, "    const float f%u_0 = t%u_.x, f%u_1 = t%u_.y, f%u_2 = t%u_.z, f%u_3 = t%u_.w;\n", i, i,
                        i, i, i, i, i, i);
            } else {
                wsb_put(&s, "    const float f%u_0 = ((const float*)p%u)[b%u_ + o_];\n", i, bi, i);
            }
            continue;
        }
        for (u32 v = 0; v < W; v++) emit_body_op(&s, k, p, i, v);
    }
    for (u32 v = 0; v < W; v++)
        wsb_put(&s, fixed ? "    q%u_ = q%u_ + (ok_ ? f%u_%u : 0.0f);\n" : "    q%u_ = q%u_ + f%u_%u;\n", v, v, p->value, v);
    wsb_put(&s, "  }\n");
    if (W == 4) wsb_put(&s, "  float t_ = (q0_ + q1_) + (q2_ + q3_);\n");
    else wsb_put(&s, "  float t_ = q0_;\n");
    char fb[64];
    float_bits(fb, sizeof fb, p->init_bits);
    if (p->S > 1 && p->launch) {
        /* partials to the workspace; <name>_fin: a workgroup per output, lane
         * l adds partials l, l + 256, ... in order, then the fixed trees */
        wsb_put(&s, "  t_ = bsum(t_, red_);\n  if (lane == 0u) ws_[(unsigned long long)gid * %uu + sp_] = t_;\n}\n", p->S);
        wsb_put(&s, "extern \"C\" __global__ __launch_bounds__(%u) void %s_fin(char* p0, const float* ws_) {\n"
                    "  __shared__ float red_[%u];\n"
                    "  const u32 gid = blockIdx.x;\n"
                    "  float w_ = 0.0f;\n"
                    "  for (u32 s_ = threadIdx.x; s_ < %uu; s_ += %uu) w_ = w_ + ws_[(unsigned long long)gid * %uu + s_];\n"
                    "  w_ = bsum(w_, red_);\n"
                    "  if (threadIdx.x == 0u) ((float*)p0)[gid] = %s + w_;\n}\n",
                WIN_BLOCK, name, WIN_BLOCK / 64, p->S, WIN_BLOCK, p->S, fb);
    } else if (p->S > 1) {
        wsb_put(&s, "  t_ = bsum(t_, red_);\n"
                    "  if (sp_ != %uu) {\n"
                    "    comb_put(sl_, gid, sp_, %uu, t_);\n"
                    "  } else {\n", p->S - 1, p->S);
        emit_take_all(&s, p->S, "t_", "gid");
        wsb_put(&s, "    w_ = bsum(w_, red_);\n"
                    "    if (lane == 0u) ((float*)p0)[gid] = %s + w_;\n"
                    "  }\n}\n", fb);
    } else {
        wsb_put(&s, "  t_ = bsum(t_, red_);\n  if (lane == 0u) ((float*)p0)[gid] = %s + t_;\n}\n", fb);
    }
    return s.p;
}

static char *gen_window(const UOpKernel *k, const WinPlan *p, char *name, size_t namelen) {
    snprintf(name, namelen, "thvm_%s_%08x", p->kind == WIN_MAX ? "wmax" : "rsum",
             (u32)(uop_signature(k) & 0xFFFFFFFFu));
    return p->kind == WIN_MAX ? gen_window_max(k, p, name) : gen_run_sum(k, p, name);
}

/* ---------------- cache and dispatch ---------------- */

typedef struct {
    u64 key;
    u32 n_ops, n_leaves;
    KOp *ops;
    u32 meta[5];
    u32 dts[FUSE_MAX_LEAVES];
    int kind;                    /* WIN_NONE: a program this file does not take */
    WinPlan plan;
    hipModule_t mod;
    hipFunction_t fn, fn_fin;
    CoForm co;                   /* the main kernel's co-launch form (one-launch plans) */
    char name[32];               /* its kernel's name */
    u32 cov_n[WIN_MAX_LOADS];    /* run sums: the tensor size each load was checked to tile (0: not yet) */
    u8 cov_ok[WIN_MAX_LOADS];    /* ... and the answer */
} WinEntry;

static Scratch win_ws;   /* run-sum partials of the combine-kernel form */

static struct {
    WinEntry *tab;
    u32 cap, n;
} WC;

static int win_same(const WinEntry *e, const UOpKernel *k) {
    if (e->n_ops != k->n_ops || e->n_leaves != k->n_leaves || !e->ops) return 0;
    if (e->meta[0] != k->grid[0] || e->meta[1] != k->grid[1] || e->meta[2] != k->grid[2] ||
        e->meta[3] != k->local_size || e->meta[4] != k->out_dtype)
        return 0;
    if (memcmp(e->dts, k->leaf_dtypes, (size_t)k->n_leaves * sizeof(u32)) != 0) return 0;
    return memcmp(e->ops, k->ops, (size_t)k->n_ops * sizeof(KOp)) == 0;
}

static WinEntry *win_lookup(u64 key, const UOpKernel *k) {
    if (!WC.tab) return NULL;
    u32 m = WC.cap - 1;
    for (u32 q = (u32)key & m, probes = 0; probes < WC.cap; q = (q + 1) & m, probes++) {
        WinEntry *e = &WC.tab[q];
        if (!e->key) return NULL;
        if (e->key == key && win_same(e, k)) return e;
    }
    return NULL;
}

static WinEntry *win_insert(u64 key, const UOpKernel *k) {
    if (!WC.tab || (WC.n + 1) * 2 > WC.cap) {
        u32 nc = WC.cap ? WC.cap * 2 : 256;
        WinEntry *nt = calloc(nc, sizeof(WinEntry));
        if (!nt) return NULL;
        for (u32 i = 0; i < WC.cap; i++) {
            if (!WC.tab[i].key) continue;
            u32 q = (u32)WC.tab[i].key & (nc - 1);
            while (nt[q].key) q = (q + 1) & (nc - 1);
            nt[q] = WC.tab[i];
        }
        free(WC.tab);
        WC.tab = nt;
        WC.cap = nc;
    }
    u32 m = WC.cap - 1, q = (u32)key & m;
    while (WC.tab[q].key) q = (q + 1) & m;
    WinEntry *e = &WC.tab[q];
    memset(e, 0, sizeof *e);
    e->key = key;
    e->n_ops = k->n_ops;
    e->n_leaves = k->n_leaves;
    e->ops = malloc((size_t)k->n_ops * sizeof(KOp));
    if (e->ops) memcpy(e->ops, k->ops, (size_t)k->n_ops * sizeof(KOp));
    e->meta[0] = k->grid[0]; e->meta[1] = k->grid[1]; e->meta[2] = k->grid[2];
    e->meta[3] = k->local_size; e->meta[4] = k->out_dtype;
    memcpy(e->dts, k->leaf_dtypes, (size_t)k->n_leaves * sizeof(u32));
    WC.n++;
    return e;
}

static u64 win_key(const UOpKernel *k) {
    u64 key = uop_signature(k) ^ 0x57494E444F57ull;
    return key ? key : 1;
}

static u64 win_key_of(const WinEntry *e) { return e->key; }

int window_analyze(const UOpKernel *k, u32 *kind, u32 *splits) {
    WinPlan p;
    if (!k || !win_recognize(k, &p)) {
        if (kind) *kind = WIN_NONE;
        if (splits) *splits = 0;
        return 0;
    }
    if (kind) *kind = (u32)p.kind;
    if (splits) *splits = p.kind == WIN_SUM ? p.S : 1;
    return 1;
}

char *window_source(const UOpKernel *k) {
    WinPlan p;
    char name[48];
    if (!k || !win_recognize(k, &p)) return NULL;
    return gen_window(k, &p, name, sizeof name);
}

/* Records that a program is neither a window max nor a run sum (the entry
 * window_try_dispatch would leave), without dispatching it: for a program
 * that ran only fused into another launch. */
void window_note_plain(const UOpKernel *k) {
    if (!k || k->n_leaves > FUSE_MAX_LEAVES) return;
    const u64 key = win_key(k);
    WinPlan p;
    if (win_lookup(key, k) || win_recognize(k, &p)) return;
    win_insert(key, k);
}

/* The program's entry: looked up, or recognised and compiled on first
 * sight (kind WIN_NONE: a program this file does not take). NULL only when
 * no entry could be made. */
static WinEntry *win_entry(const UOpKernel *k) {
    if (k->n_leaves > FUSE_MAX_LEAVES) return NULL;
    u64 key = win_key(k);
    WinEntry *e = win_lookup(key, k);
    if (e) return e;
    if (hipb.noalloc) {
        hipb.noalloc_err = THVM_HIP_ENOTREADY;   /* never compiles without allocating */
        return NULL;
    }
    e = win_insert(key, k);
    if (!e) return NULL;
    if (!win_recognize(k, &e->plan)) return e;    /* kind stays WIN_NONE */
    char name[48], err[256] = {0};
build:;
    char *src = gen_window(k, &e->plan, name, sizeof name);
    if (!src) return e;
    if (hipb.dump_src) fprintf(stderr, "---- window kernel ----\n%s\n", src);
    if (!rtc_build_module(src, &e->mod, err, sizeof err)) {
        fprintf(stderr, "tinyhvm-hip: window kernel build failed: %s\n", err);
        free(src);
        return e;
    }
    char fin[64];
    snprintf(fin, sizeof fin, "%s_fin", name);
    if (hipModuleGetFunction(&e->fn, e->mod, name) != hipSuccess ||
        (e->plan.kind == WIN_SUM && e->plan.S > 1 && e->plan.launch &&
         hipModuleGetFunction(&e->fn_fin, e->mod, fin) != hipSuccess)) {
        HIPB_CHECK(hipModuleUnload(e->mod));
        free(src);
        return e;
    }
    /* one pass only if the whole grid is on the GPU at once with this
     * kernel's own occupancy; else partials go to a combine kernel */
    if (e->plan.kind == WIN_SUM && e->plan.S > 1 && !e->plan.launch &&
        (u64)e->plan.total * e->plan.S > rtc_capacity(e->fn, WIN_BLOCK)) {
        HIPB_CHECK(hipModuleUnload(e->mod));
        free(src);
        e->plan.launch = 1;
        goto build;
    }
    if (!(e->plan.kind == WIN_SUM && e->plan.S > 1 && e->plan.launch))
        co_form_make(&e->co, src, name, WIN_BLOCK, e->fn);
    free(src);
    e->kind = e->plan.kind;
    snprintf(e->name, sizeof e->name, "%s", name);
    if (hipb.verbose)
        fprintf(stderr, "tinyhvm-hip: %s outputs=%u trip=%u W=%u run=%u splits=%u\n", name, e->plan.total,
                e->plan.trip, e->plan.W, e->plan.L, e->plan.S);
    return e;
}

int window_try_dispatch(u32 out_buf, const u32 *leaf_bufs, u32 n_leaves, const UOpKernel *k) {
    WinEntry *e = win_entry(k);
    if (!e || e->kind == WIN_NONE) return 0;
    const WinPlan *p = &e->plan;
    /* buffers: every index the plan forms is inside them, vector loads aligned */
    void *ptrs[FUSE_MAX_LEAVES + 1];
    HipbBuf *ob = pool_get(out_buf);
    if (!ob || ob->bytes / 4 < p->total) return 0;
    ptrs[0] = ob->ptr;
    for (u32 i = 0; i < k->n_leaves; i++) {
        void *lp = i < n_leaves ? pool_ptr(leaf_bufs[i]) : NULL;
        ptrs[i + 1] = lp ? lp : hipb.dummy;
    }
    for (u32 j = 0; j < p->n_ld; j++) {
        u32 bi = k->ops[p->ld_op[j]].imm.u;
        if (bi > n_leaves || !pool_ptr(leaf_bufs[bi - 1])) return 0;
        u64 top = p->kind == WIN_MAX ? p->cover_max : p->ld_max[j];
        if (top >= pool_bytes(leaf_bufs[bi - 1]) / 4) return 0;
        if (p->ld_r[j] && ((uintptr_t)ptrs[bi] & (4u * p->W - 1u))) return 0;
    }
    if (p->kind == WIN_MAX && p->P == 2 && ((uintptr_t)ptrs[0] & 7u)) return 0;
    float *ws = NULL;
    if (p->kind == WIN_SUM && p->S > 1 && p->launch) {
        ws = scratch_reserve(&win_ws, (u64)p->total * p->S * sizeof(float));
        if (!ws) return 0;
    }
    for (u32 i = 0; i < n_leaves && i < FUSE_MAX_LEAVES; i++) pool_sync_device(leaf_bufs[i]);
    if (p->kind == WIN_MAX) {
        u32 bi = k->ops[p->ld_op[0]].imm.u;
        void *params[] = {&ptrs[0], &ptrs[bi]};
        u64 lanes = ((u64)p->total / p->P + p->U - 1) / p->U;
        u64 blocks = (lanes + WIN_BLOCK - 1) / WIN_BLOCK;
        u32 gx = (u32)blocks, gy = 1;
        if (blocks * WIN_BLOCK >= (1ull << 32)) {
            gx = 65536;
            gy = (u32)((blocks + 65535) / 65536);
        }
        HbMem hm;
        hm.n = 0;
        hbm_add(&hm, ptrs[0], pool_bytes(out_buf), 1);
        hbm_add(&hm, ptrs[bi], pool_bytes(leaf_bufs[bi - 1]), 0);
        if (hipb_hold(&e->co, e->fn, gx, gy, params, &hm, 0, -1, 0) ||
            (gy == 1 && hipb_hold_large(&e->co, e->fn, gx, gy, params, &hm, 0, -1, 0))) {
            hipb_hold_tag_wmax(e, out_buf, leaf_bufs[bi - 1]);
            return 1;
        }
        if (!hipb_launch(e->fn, gx, gy, 1, WIN_BLOCK, params)) return 0;
    } else {
        void *params[FUSE_MAX_LEAVES + 3];
        u32 np = 0;
        for (u32 b = 0; b <= k->n_leaves; b++) params[np++] = &ptrs[b];
        if (ws) {
            params[np++] = &ws;
        } else {
            params[np++] = &hipb.comb_slots;
            /* one launch: held for a batch with the next independent dispatches */
            HbMem hm;
            hm.n = 0;
            hbm_add(&hm, ptrs[0], pool_bytes(out_buf), 1);
            for (u32 i = 0; i < n_leaves && i < FUSE_MAX_LEAVES; i++)
                hbm_add(&hm, pool_ptr(leaf_bufs[i]), pool_bytes(leaf_bufs[i]), 0);
            if (hipb_hold(&e->co, e->fn, p->total * p->S, 1, params, &hm, p->S > 1, (int)(np - 1),
                          (u64)p->total * p->S) ||
                hipb_hold_large(&e->co, e->fn, p->total * p->S, 1, params, &hm, p->S > 1, (int)(np - 1),
                                (u64)p->total * p->S)) {
                hipb_hold_tag_sum(e, out_buf, leaf_bufs, n_leaves);
                return 1;
            }
        }
        if (!hipb_launch(e->fn, p->total * p->S, 1, 1, WIN_BLOCK, params)) return 0;
        if (ws) {
            void *p2[] = {&ptrs[0], &ws};
            if (!hipb_launch(e->fn_fin, p->total, 1, 1, WIN_BLOCK, p2)) return 0;
        }
    }
    return 1;
}

/* ---------------- run-sum groups ---------------- */

/* The generated group kernels, one per shape (the key names the programs
 * and which of their loads take the producer's values); fn NULL: refused. */
#define WG_CACHE 128
typedef struct {
    u64 key;
    hipModule_t mod;
    hipFunction_t fn;
    CoForm co;
    KGenScalars psc, tsc[WG_MAX_TAILS];
    u32 cap;                     /* workgroups resident at once */
} WgEntry;
static struct {
    WgEntry e[WG_CACHE];
    u32 n;
    UOpKernel *tail[64];         /* the consumers' programs (copies, by signature) */
    u64 tail_sig[64];
    u32 n_tail;
} WGC;

static u64 wg_mix(u64 h, u64 v) {
    h ^= v + 0x9E3779B97F4A7C15ull + (h << 6) + (h >> 2);
    h *= 0xFF51AFD7ED558CCDull;
    return h ^ (h >> 33);
}

static u32 launch_total_of(const UOpKernel *k) {
    return k->local_size > 0 ? k->grid[0] : k->grid[0] * k->grid[1] * k->grid[2];
}

/* a cached entry's program as a UOpKernel (heap) */
static UOpKernel *win_kernel(const WinEntry *e) {
    UOpKernel *k = calloc(1, sizeof *k);
    if (!k) return NULL;
    memcpy(k->ops, e->ops, (size_t)e->n_ops * sizeof(KOp));
    k->n_ops = e->n_ops;
    k->n_leaves = e->n_leaves;
    k->n_bufs = e->n_leaves + 1;
    k->grid[0] = e->meta[0]; k->grid[1] = e->meta[1]; k->grid[2] = e->meta[2];
    k->local_size = e->meta[3];
    k->out_dtype = e->meta[4];
    memcpy(k->leaf_dtypes, e->dts, (size_t)e->n_leaves * sizeof(u32));
    return k;
}

static UOpKernel *chain_kernel(const ChainInfo *c) {
    UOpKernel *k = calloc(1, sizeof *k);
    if (!k) return NULL;
    memcpy(k->ops, c->ops, (size_t)c->n_ops * sizeof(KOp));
    k->n_ops = c->n_ops;
    k->n_leaves = c->n_leaves;
    k->n_bufs = c->n_leaves + 1;
    memcpy(k->grid, c->grid, sizeof k->grid);
    k->out_dtype = c->out_dtype;
    memcpy(k->leaf_dtypes, c->leaf_dtypes, sizeof c->leaf_dtypes);
    return k;
}

static int aff_same(const Aff *a, const Aff *b) {
    if (!a->ok || !b->ok || a->cst != b->cst || a->n != b->n) return 0;
    for (u32 t = 0; t < a->n; t++) {
        int found = 0;
        for (u32 u = 0; u < b->n && !found; u++)
            found = a->d[t].var == b->d[u].var && a->d[t].div == b->d[u].div && a->d[t].mod == b->d[u].mod &&
                    a->coef[t] == b->coef[u];
        if (!found) return 0;
    }
    return 1;
}

/* whether the run sum's load at `a` reads each element of [0, n) exactly
 * once over the launch: its runs, laid out for every output and outer
 * digit, tile the tensor (checked by marking them) */
static int wg_covers(const WinPlan *p, const Aff *a, u32 n) {
    if ((u64)p->total * p->trip != n) return 0;
    u8 *seen = calloc(n, 1);
    if (!seen) return 0;
    int ok = 1;
    const u32 runs = p->trip / p->L;
    for (u32 g = 0; g < p->total && ok; g++)
        for (u32 r = 0; r < runs && ok; r++) {
            const u64 st = aff_eval(a, g, r * p->L);
            if (st + p->L > n) { ok = 0; break; }
            for (u32 j = 0; j < p->L && ok; j++) ok = !seen[st + j]++;
        }
    free(seen);
    return ok;
}

static void wg_buf(WgBuf *b, u32 id, u32 dtype) {
    b->id = id;
    b->ptr = id ? pool_ptr(id) : NULL;
    b->bytes = id ? pool_bytes(id) : 0;
    b->cnt = (u32)(b->bytes / (dtype == DTYPE_F16 ? 2u : 4u));
}

static void wg_bufs(WgBufs *w, u32 out, u32 out_dt, const u32 *leaves, const u32 *dts, u32 nl) {
    w->nb = nl + 1;
    wg_buf(&w->b[0], out, out_dt);
    for (u32 i = 0; i < nl; i++) wg_buf(&w->b[i + 1], leaves[i], dts[i]);
}

/* same buffer: the id and, where the device is up, the memory */
static int wg_is(const WgBuf *b, u32 id) { return b->id && b->id == id && (!b->ptr || b->ptr == pool_ptr(id)); }

int window_group_uses(const WinGroup *g, u32 id, int writes) {
    if (!id) return 0;
    for (u32 s = 0; s < g->n_sum; s++)
        for (u32 b = 0; b < (writes ? 1u : g->sb[s].nb); b++)
            if (wg_is(&g->sb[s].b[b], id)) return 1;
    for (u32 t = 0; t < g->n_tail; t++)
        for (u32 b = 0; b < (writes ? 1u : g->tb[t].nb); b++)
            if (wg_is(&g->tb[t].b[b], id)) return 1;
    if (g->pkind == 1) {
        for (u32 b = 0; b < g->pb.nb; b++) {
            int st = 0;
            for (u32 j = 0; j < g->pc->n_st; j++) st |= g->pc->st_slot[j] == b;
            if ((!writes || st) && wg_is(&g->pb.b[b], id)) return 1;
        }
    } else if (g->pkind == 2) {
        if (wg_is(&g->pb.b[0], id) || (!writes && wg_is(&g->pb.b[1], id))) return 1;
    }
    return 0;
}

/* the producer STORE whose buffer id is (-1: none) */
static int wg_prod_store(const WinGroup *g, u32 id) {
    if (g->pkind == 1) {
        for (u32 j = 0; j < g->pc->n_st; j++)
            if (wg_is(&g->pb.b[g->pc->st_slot[j]], id)) return (int)j;
    } else if (g->pkind == 2 && wg_is(&g->pb.b[0], id)) {
        return 0;
    }
    return -1;
}

static u32 wg_prod_total(const WinGroup *g) {
    return g->pkind == 1 ? g->pc->total : g->pkind == 2 ? ((const WinEntry *)g->pw)->plan.total : 0;
}

static int wg_same_shape(const WinPlan *a, const WinPlan *b) {
    if (a->total != b->total || a->trip != b->trip || a->L != b->L || a->W != b->W || a->S != b->S ||
        a->unroll != b->unroll || a->launch != b->launch || a->n_outer != b->n_outer)
        return 0;
    for (u32 q = 0; q < a->n_outer; q++)
        if (a->outer_div[q] != b->outer_div[q] || a->outer_mod[q] != b->outer_mod[q] ||
            a->outer_coef[q] != b->outer_coef[q])
            return 0;
    return 1;
}

static void wg_clear(WinGroup *g) { memset(g, 0, sizeof *g); }

const void *window_sum_entry(const UOpKernel *k) {
    if (!k || k->n_leaves > WG_MAX_LEAVES) return NULL;
    const WinEntry *e = win_entry(k);
    if (!e || e->kind != WIN_SUM || (e->plan.S > 1 && e->plan.launch)) return NULL;
    return e;
}

/* The checks window_try_dispatch makes before a launch: every index a
 * memory load forms inside its buffer, vector loads aligned, the output
 * large enough (a load the producer's value replaces reads no memory). */
static int wg_sum_fits(const WinEntry *e, const int8_t *sub, u32 out_buf, const u32 *leaf_bufs) {
    const WinPlan *p = &e->plan;
    if (!pool_ptr(out_buf)) return 1;   /* no device: a source check */
    if (pool_bytes(out_buf) / 4 < p->total) return 0;
    for (u32 j = 0; j < p->n_ld; j++) {
        const u32 bi = e->ops[p->ld_op[j]].imm.u;
        if (sub[bi] >= 0) continue;
        const void *lp = pool_ptr(leaf_bufs[bi - 1]);
        if (!lp || p->ld_max[j] >= pool_bytes(leaf_bufs[bi - 1]) / 4) return 0;
        if (p->ld_r[j] && ((uintptr_t)lp & (4u * p->W - 1u))) return 0;
    }
    return 1;
}

int window_group_add_sum(WinGroup *g, const void *we, u32 out_buf, const u32 *leaf_bufs, u32 n_leaves) {
    const WinEntry *e = we;
    if (!e || e->kind != WIN_SUM || g->n_sum >= WG_MAX_SUMS || e->n_leaves > WG_MAX_LEAVES ||
        n_leaves < e->n_leaves || (e->plan.S > 1 && e->plan.launch) || !out_buf)
        return 0;
    const WinPlan *p = &e->plan;
    if (g->n_sum && !wg_same_shape(&((const WinEntry *)g->sum[0])->plan, p)) return 0;
    if (g->n_tail) return 0;     /* consumers run after every sum's combine: sums first */
    if (window_group_uses(g, out_buf, 0)) return 0;
    for (u32 i = 0; i < e->n_leaves; i++)
        if (leaf_bufs[i] == out_buf) return 0;
    const u32 s = g->n_sum;
    int reads = 0;
    for (u32 b = 1; b <= e->n_leaves; b++) {
        const u32 id = leaf_bufs[b - 1];
        const int K = g->pkind ? wg_prod_store(g, id) : -1;
        g->sub[s][b] = (int8_t)K;
        if (K < 0) {
            if (window_group_uses(g, id, 1)) return 0;   /* another output of the group */
            continue;
        }
        if (g->pkind == 1 && !g->pc->st_f32[K]) return 0;
        /* every load of it: along r, at the index the group reads the tensor at */
        for (u32 j = 0; j < p->n_ld; j++) {
            if (e->ops[p->ld_op[j]].imm.u != b) continue;
            if (!p->ld_r[j]) return 0;
            if (!g->has_canon) {
                const u32 pn = wg_prod_total(g);
                WinEntry *me = (WinEntry *)e;
                if (me->cov_n[j] != pn) {   /* checked once per load and size */
                    me->cov_ok[j] = (u8)wg_covers(p, &p->ld_aff[j], pn);
                    me->cov_n[j] = pn;
                }
                if (!me->cov_ok[j]) return 0;
                g->canon = p->ld_aff[j];
                g->has_canon = 1;
            } else if (!aff_same(&g->canon, &p->ld_aff[j])) {
                return 0;
            }
            reads = 1;
        }
    }
    if (g->pkind && s == 0 && !reads) return 0;
    if (!wg_sum_fits(e, g->sub[s], out_buf, leaf_bufs)) return 0;
    g->sum[s] = e;
    wg_bufs(&g->sb[s], out_buf, e->meta[4], leaf_bufs, e->dts, e->n_leaves);
    g->n_sum++;
    return 1;
}

int window_group_of_sum(WinGroup *g, const void *we, u32 out_buf, const u32 *leaf_bufs, u32 n_leaves) {
    wg_clear(g);
    return window_group_add_sum(g, we, out_buf, leaf_bufs, n_leaves);
}

int window_group_of_chain(WinGroup *g, const ChainInfo *pc, const u32 *bufs) {
    wg_clear(g);
    if (!pc || pc->n_leaves > WG_MAX_LEAVES || pc->n_ops > KOP_MAX) return 0;
    /* loop-free, and reads no buffer it stores */
    for (u32 i = 0; i < pc->n_ops; i++) {
        const KOp *op = &pc->ops[i];
        if (op->type == KOP_RANGE || op->type == KOP_ACC) return 0;
        if (op->type == KOP_LOAD)
            for (u32 j = 0; j < pc->n_st; j++)
                if (op->imm.u == pc->st_slot[j] || (op->imm.u <= pc->n_leaves && bufs[op->imm.u] &&
                                                    bufs[op->imm.u] == bufs[pc->st_slot[j]]))
                    return 0;
    }
    g->pkind = 1;
    g->pc = pc;
    UOpKernel *k = chain_kernel(pc);
    if (!k) return 0;
    g->psig = uop_signature(k);
    free(k);
    wg_bufs(&g->pb, bufs[0], pc->out_dtype, bufs + 1, pc->leaf_dtypes, pc->n_leaves);
    return 1;
}

int window_group_of_wmax(WinGroup *g, const void *we, u32 out_buf, u32 in_buf) {
    wg_clear(g);
    const WinEntry *e = we;
    if (!e || e->kind != WIN_MAX || !out_buf || !in_buf || out_buf == in_buf) return 0;
    /* its loads (one element at a time here) and stores inside the buffers */
    if (pool_ptr(out_buf) && (pool_bytes(out_buf) / 4 < e->plan.total || !pool_ptr(in_buf) ||
                              e->plan.ld_max[0] >= pool_bytes(in_buf) / 4))
        return 0;
    g->pkind = 2;
    g->pw = e;
    g->psig = win_key_of(e);
    const u32 dts[1] = {DTYPE_F32};
    wg_bufs(&g->pb, out_buf, DTYPE_F32, &in_buf, dts, 1);
    return 1;
}

static const UOpKernel *wg_tail_copy(const UOpKernel *k, u64 sig) {
    for (u32 i = 0; i < WGC.n_tail; i++)
        if (WGC.tail_sig[i] == sig && WGC.tail[i]->n_ops == k->n_ops &&
            memcmp(WGC.tail[i]->ops, k->ops, (size_t)k->n_ops * sizeof(KOp)) == 0)
            return WGC.tail[i];
    if (WGC.n_tail >= 64) return NULL;
    UOpKernel *c = malloc(sizeof *c);
    if (!c) return NULL;
    memcpy(c, k, sizeof *c);
    WGC.tail[WGC.n_tail] = c;
    WGC.tail_sig[WGC.n_tail++] = sig;
    return c;
}

int window_group_add_tail(WinGroup *g, const UOpKernel *k, u32 out_buf, const u32 *leaf_bufs, u32 n_leaves) {
    if (!g->n_sum || g->n_tail >= WG_MAX_TAILS || !k || k->n_leaves == 0 || k->n_leaves > WG_MAX_LEAVES ||
        n_leaves < k->n_leaves || k->out_dtype != DTYPE_F32 || k->n_ops == 0 || k->n_ops > KOP_MAX || !out_buf)
        return 0;
    const u32 total = ((const WinEntry *)g->sum[0])->plan.total;
    if (launch_total_of(k) != total || window_group_uses(g, out_buf, 0)) return 0;
    /* the one leaf slot that holds a value of the group */
    u32 slot = 0;
    int src = -1;
    for (u32 b = 1; b <= k->n_leaves; b++) {
        const u32 id = leaf_bufs[b - 1];
        if (id == out_buf) return 0;
        int v = -1;
        for (u32 s = 0; s < g->n_sum && v < 0; s++)
            if (wg_is(&g->sb[s].b[0], id)) v = (int)s;
        for (u32 t = 0; t < g->n_tail && v < 0; t++)
            if (wg_is(&g->tb[t].b[0], id)) v = WG_MAX_SUMS + (int)t;
        if (v >= 0) {
            if (slot) return 0;
            slot = b;
            src = v;
        } else if (window_group_uses(g, id, 1)) {
            return 0;
        }
    }
    if (!slot) return 0;
    /* loop-free, one STORE, loads of that slot and the STORE at gid */
    Aff *aff = calloc(k->n_ops, sizeof(Aff));
    if (!aff) return 0;
    DCtx dc = {k, total, 1, -1, aff};
    analyze_aff(&dc);
    int ok = 1, stores = 0;
    for (u32 i = 0; i < k->n_ops && ok; i++) {
        const KOp *op = &k->ops[i];
        if (op->type == KOP_RANGE || op->type == KOP_ENDRANGE || op->type == KOP_ACC_INIT || op->type == KOP_ACC)
            ok = 0;
        else if (op->type == KOP_STORE)
            ok = stores++ == 0 && op->imm.u == 0 && op->arg[0] < k->n_ops && aff_is_gid(&dc, &aff[op->arg[0]]) &&
                 op->arg[1] < k->n_ops && op_type_is_float(k->ops[op->arg[1]].type);
        else if (op->type == KOP_LOAD && op->imm.u == slot)
            ok = op->arg[0] < k->n_ops && aff_is_gid(&dc, &aff[op->arg[0]]);
        else if (op->type == KOP_LOAD && op->imm.u == 0)
            ok = 0;
    }
    free(aff);
    if (!ok || stores != 1 || k->leaf_dtypes[slot - 1] != DTYPE_F32) return 0;
    const u64 sig = uop_signature(k);
    const UOpKernel *c = wg_tail_copy(k, sig);
    if (!c) return 0;
    const u32 t = g->n_tail;
    g->tail[t] = c;
    g->tsig[t] = sig;
    g->tleaf[t] = slot;
    g->tsrc[t] = (u8)src;
    wg_bufs(&g->tb[t], out_buf, k->out_dtype, leaf_bufs, k->leaf_dtypes, k->n_leaves);
    g->n_tail++;
    return 1;
}

/* An earlier member's memory load that member m's load j repeats (the same
 * buffer at the same index): its value is taken instead of loading again.
 * Returns 1 with that member and load. */
static int wg_shared_load(const WinGroup *g, u32 m, u32 j, u32 *pm, u32 *pj) {
    const WinEntry *e = g->sum[m];
    const u32 bi = e->ops[e->plan.ld_op[j]].imm.u;
    if (!e->plan.ld_r[j] || g->sub[m][bi] >= 0) return 0;
    for (u32 m2 = 0; m2 < m; m2++) {
        const WinEntry *e2 = g->sum[m2];
        for (u32 j2 = 0; j2 < e2->plan.n_ld; j2++) {
            const u32 b2 = e2->ops[e2->plan.ld_op[j2]].imm.u;
            if (!e2->plan.ld_r[j2] || g->sub[m2][b2] >= 0 || g->sb[m2].b[b2].id != g->sb[m].b[bi].id ||
                !aff_same(&e2->plan.ld_aff[j2], &e->plan.ld_aff[j]))
                continue;
            *pm = m2;
            *pj = j2;
            return 1;
        }
    }
    return 0;
}

static u64 wg_key(const WinGroup *g) {
    u64 h = wg_mix(0x5347524F5550ull, ((u64)g->n_sum << 8) | ((u64)g->n_tail << 4) | (u64)g->pkind);
    for (u32 s = 0; s < g->n_sum; s++) {
        const WinEntry *e = g->sum[s];
        h = wg_mix(h, e->key);
        for (u32 b = 1; b <= e->n_leaves; b++) h = wg_mix(h, (u64)(u8)g->sub[s][b]);
        for (u32 j = 0; j < e->plan.n_ld; j++) {
            u32 pm, pj;
            if (wg_shared_load(g, s, j, &pm, &pj)) h = wg_mix(h, 0x5348ull ^ ((u64)j << 16) ^ ((u64)pm << 32) ^ ((u64)pj << 40));
        }
    }
    if (g->pkind) {
        h = wg_mix(h, g->psig);
        for (u32 q = 0; q < g->canon.n; q++)
            h = wg_mix(h, ((u64)g->canon.d[q].var << 60) ^ ((u64)g->canon.d[q].div << 32) ^ g->canon.coef[q] ^
                              ((u64)g->canon.d[q].mod << 16));
        h = wg_mix(h, g->canon.cst);
    }
    for (u32 t = 0; t < g->n_tail; t++) h = wg_mix(wg_mix(h, g->tsig[t]), ((u64)g->tleaf[t] << 8) | g->tsrc[t]);
    return h ? h : 1;
}

/* the sum whose combine a value (sum s, or tail WG_MAX_SUMS + t) belongs to */
static u32 wg_root(const WinGroup *g, u32 v) {
    while (v >= WG_MAX_SUMS) v = g->tsrc[v - WG_MAX_SUMS];
    return v;
}

/* body op i of member m for component v (loads were emitted before) */
static void emit_member_op(WSB *s, const UOpKernel *k, u32 m, u32 i, u32 v) {
    const KOp *op = &k->ops[i];
    char a[64], b[64], x[256], fb[64];
    switch (op->type) {
    case KOP_CONST_F:
        float_bits(fb, sizeof fb, op->imm.u);
        wsb_put(s, "    const float m%u_f%u_%u = %s;\n", m, i, v, fb);
        break;
    case KOP_ALU:
        snprintf(a, sizeof a, "m%u_f%u_%u", m, op->arg[0], v);
        snprintf(b, sizeof b, "m%u_f%u_%u", m, alu_unary(op->imm.u) ? op->arg[0] : op->arg[1], v);
        kgen_alu_expr(op->imm.u, op->arg[2], a, b, x, sizeof x);
        wsb_put(s, "    const float m%u_f%u_%u = %s;\n", m, i, v, x);
        break;
    default:
        break;
    }
}

/* A window-max producer read four outputs at a time as two of its pairs:
 * the plan pairs adjacent outputs in 16-byte vectors, and its input is
 * aligned for them and holds every element they read. */
static int wg_wmax_vec(const WinGroup *g) {
    const WinEntry *e = g->pw;
    if (g->pkind != 2 || !e || e->plan.P != 2 || e->plan.W != 4) return 0;
    if (!g->pb.b[1].ptr) return 1;    /* no device: a source check */
    return ((uintptr_t)g->pb.b[1].ptr & 15u) == 0 && ((uintptr_t)g->pb.b[0].ptr & 15u) == 0 &&
           e->plan.cover_max < g->pb.b[1].bytes / 4;
}

/* The group's kernel source: the run sums' loop (their shared geometry),
 * each sum's body in its own names, the producer's device function called
 * once per element at the group's index, each sum's combine, and the tails
 * in the lane that stores the sum. */
static char *gen_group(const WinGroup *g, const char *name, u32 unroll, KGenScalars *psc, KGenScalars *tsc,
                       char *err, size_t errlen) {
    const WinEntry *e0 = g->sum[0];
    const WinPlan *p = &e0->plan;
    const u32 W = p->W, L4 = p->L / W, units = p->trip / W, S = p->S, total = p->total;
    const u32 chunk = (units + S - 1) / S;
    const u32 nit = (chunk + WIN_BLOCK - 1) / WIN_BLOCK;
    const int fixed = nit <= WIN_SUM_MAX_FIXED;
    UOpKernel *ks[WG_MAX_SUMS] = {0}, *pk = NULL;
    char *fnbuf = malloc(65536);
    WSB s = {0};
    int ok = fnbuf != NULL;
    for (u32 m = 0; m < g->n_sum && ok; m++) ok = (ks[m] = win_kernel(g->sum[m])) != NULL;
    u32 nst = 0;
    memset(psc, 0, sizeof *psc);
    if (ok) wsb_put(&s, "%s\n", kgen_prelude());
    /* four consecutive elements per call */
    const int vec_prod = (g->pkind == 1 || (g->pkind == 2 && wg_wmax_vec(g))) && W == 4;
    if (ok && g->pkind == 1) {
        nst = g->pc->n_st;
        ok = (pk = chain_kernel(g->pc)) != NULL &&
             (vec_prod ? kgen_producer4_fn(pk, g->pc->total, "prod_", fnbuf, 65536, psc)
                       : kgen_producer_fn(pk, "prod_", fnbuf, 65536, psc)) >= 0;
        if (ok) wsb_put(&s, "%s", fnbuf);
        else snprintf(err, errlen, "producer generation failed");
    } else if (ok && g->pkind == 2 && W == 4 && wg_wmax_vec(g)) {
        /* four adjacent outputs as two pairs, each pair's window rows read
         * as 16-byte vectors (the window-max kernel's loads), the maximum in
         * the engine's order */
        const WinPlan *w = &((const WinEntry *)g->pw)->plan;
        u32 groups[WIN_MAX_TRIP], ng = 0;
        for (u32 r = 0; r < w->trip; r++) {
            u32 gq = w->off[r] / 4, seen = 0;
            for (u32 x = 0; x < ng; x++) seen |= groups[x] == gq;
            if (!seen) groups[ng++] = gq;
        }
        char fb[64];
        nst = 1;
        float_bits(fb, sizeof fb, w->init_bits);
        wsb_put(&s, "__device__ __forceinline__ void prod_(u32 X0, bool st_, float4* r0_, char* p0, const char* p1) {\n"
                    "  float a_[4];\n");
        for (u32 q = 0; q < 2; q++) {
            char gx[32];
            snprintf(gx, sizeof gx, "(X0 + %uu)", 2 * q);
            wsb_put(&s, "  {\n    const u32 b_ = ");
            emit_base_expr(&s, &w->ld_aff[0], gx);
            wsb_put(&s, ";\n");
            for (u32 x = 0; x < ng; x++)
                wsb_put(&s, "    const v4f_ v%u_ = __builtin_nontemporal_load((const v4f_*)((const float*)p1 + b_ + %uu));\n",
                        x, groups[x] * 4);
            for (u32 t = 0; t < 2; t++) {
                wsb_put(&s, "    a_[%u] = %s;\n", 2 * q + t, fb);
                for (u32 r = 0; r < w->trip; r++) {
                    u32 x = 0;
                    while (groups[x] != w->off[r] / 4) x++;
                    wsb_put(&s, "    { const float e_ = v%u_.%c; a_[%u] = (a_[%u] > e_) ? a_[%u] : e_; }\n", x,
                            "xyzw"[(w->off[r] + t * w->c1) % 4], 2 * q + t, 2 * q + t, 2 * q + t);
                }
            }
            wsb_put(&s, "  }\n");
        }
        wsb_put(&s, "  if (st_) {\n    *(float2*)((float*)p0 + X0) = make_float2(a_[0], a_[1]);\n"
                    "    *(float2*)((float*)p0 + X0 + 2u) = make_float2(a_[2], a_[3]);\n  }\n"
                    "  *r0_ = make_float4(a_[0], a_[1], a_[2], a_[3]);\n}\n");
    } else if (ok && g->pkind == 2) {
        const WinPlan *w = &((const WinEntry *)g->pw)->plan;
        char fb[64];
        nst = 1;
        float_bits(fb, sizeof fb, w->init_bits);
        wsb_put(&s, "__device__ __forceinline__ void prod_(u32 gid_, bool st_, float* r0_, char* p0, const char* p1) {\n"
                    "  const u32 b_ = ");
        emit_base_expr(&s, &w->ld_aff[0], "gid_");
        wsb_put(&s, ";\n  float a_ = %s;\n", fb);
        for (u32 r = 0; r < w->trip; r++)
            wsb_put(&s, "  { const float e_ = ((const float*)p1)[b_ + %uu]; a_ = (a_ > e_) ? a_ : e_; }\n", w->off[r]);
        wsb_put(&s, "  if (st_) ((float*)p0)[gid_] = a_;\n  *r0_ = a_;\n}\n");
    }
    for (u32 t = 0; t < g->n_tail && ok; t++) {
        char fname[16];
        snprintf(fname, sizeof fname, "tl%u_", t);
        ok = kgen_epilogue_fn(g->tail[t], g->tleaf[t], fname, fnbuf, 65536, &tsc[t]) >= 0;
        if (ok) wsb_put(&s, "%s", fnbuf);
        else snprintf(err, errlen, "consumer generation failed");
    }
    if (!ok) goto out;
    /* parameters */
    wsb_put(&s, "extern \"C\" __global__ __launch_bounds__(%u) void %s(", WIN_BLOCK, name);
    for (u32 m = 0; m < g->n_sum; m++)
        for (u32 b = 0; b <= ks[m]->n_leaves; b++)
            wsb_put(&s, "%s%s m%u_p%u", m || b ? ", " : "", b ? "const char*" : "char*", m, b);
    if (g->pkind == 1) {
        for (u32 b = 0; b <= pk->n_leaves; b++) wsb_put(&s, ", char* g_p%u", b);
        for (u32 b = 0; b <= pk->n_leaves; b++) wsb_put(&s, ", u32 g_c%u", b);
        if (psc->n) {
            wsb_put(&s, ", u32 g_sm");
            for (u32 j = 0; j < psc->n; j++) wsb_put(&s, ", float g_sv%u", j);
        }
    } else if (g->pkind == 2) {
        wsb_put(&s, ", char* g_p0, const char* g_p1");
    }
    for (u32 t = 0; t < g->n_tail; t++) {
        for (u32 b = 0; b <= g->tail[t]->n_leaves; b++) wsb_put(&s, ", char* t%u_p%u", t, b);
        for (u32 b = 0; b <= g->tail[t]->n_leaves; b++) wsb_put(&s, ", u32 t%u_c%u", t, b);
        if (tsc[t].n) {
            wsb_put(&s, ", u32 t%u_sm", t);
            for (u32 j = 0; j < tsc[t].n; j++) wsb_put(&s, ", float t%u_sv%u", t, j);
        }
    }
    wsb_put(&s, ", unsigned long long* sl_) {\n");
    wsb_put(&s, "  __shared__ float red_[%u];\n", WIN_BLOCK / 64);
    wsb_put(&s, "  const u32 gid = blockIdx.x / %uu, sp_ = blockIdx.x %% %uu;\n", S, S);
    wsb_put(&s, "  const u32 lane = threadIdx.x;\n");
    for (u32 m = 0; m < g->n_sum; m++) {
        const WinPlan *q = &((const WinEntry *)g->sum[m])->plan;
        for (u32 j = 0; j < q->n_ld; j++) {
            const u32 op = q->ld_op[j], bi = ks[m]->ops[op].imm.u;
            if (g->sub[m][bi] >= 0) continue;
            char nm[24];
            snprintf(nm, sizeof nm, "m%u_b%u_", m, op);
            emit_base(&s, nm, &q->ld_aff[j]);
            if (!q->ld_r[j]) wsb_put(&s, "  const float m%u_h%u_ = ((const float*)m%u_p%u)[m%u_b%u_];\n", m, op, m, bi, m, op);
        }
        for (u32 v = 0; v < W; v++) wsb_put(&s, "  float m%u_q%u_ = 0.0f;\n", m, v);
    }
    if (g->pkind) emit_base(&s, "pb_", &g->canon);
    wsb_put(&s, "  const u32 ulo_ = sp_ * %uu, uhi_ = (ulo_ + %uu < %uu) ? ulo_ + %uu : %uu;\n", chunk, chunk, units,
            chunk, units);
    /* the lane's vectors in order (the order of its partial sums); how far
     * the loop is unrolled changes only how many loads are in flight */
    if (fixed) {
        if (unroll) wsb_put(&s, "  #pragma unroll %u\n", unroll);
        else wsb_put(&s, "  #pragma unroll\n");
        wsb_put(&s, "  for (u32 i_ = 0; i_ < %uu; i_++) {\n", nit);
        wsb_put(&s, "    const u32 uu_ = ulo_ + lane + i_ * %uu;\n    const bool ok_ = uu_ < uhi_;\n"
                    "    const u32 u_ = ok_ ? uu_ : ulo_;\n", WIN_BLOCK);
    } else {
        wsb_put(&s, "  #pragma unroll %u\n  for (u32 u_ = ulo_ + lane; u_ < uhi_; u_ += %uu) {\n",
                unroll ? unroll : p->unroll, WIN_BLOCK);
    }
    wsb_put(&s, "    const u32 s_ = u_ / %uu, j_ = u_ - s_ * %uu;\n", L4, L4);
    wsb_put(&s, "    const u32 o_ = j_ * %uu", W);
    for (u32 q = 0; q < p->n_outer; q++) {
        if (p->outer_mod[q])
            wsb_put(&s, " + %uu * ((s_ / %uu) %% %uu)", p->outer_coef[q], p->outer_div[q], p->outer_mod[q]);
        else
            wsb_put(&s, " + %uu * (s_ / %uu)", p->outer_coef[q], p->outer_div[q]);
    }
    wsb_put(&s, ";\n");
    /* the producer's values at the group's index, stored by this lane */
    if (vec_prod) {
        wsb_put(&s, "    float4");
        for (u32 j = 0; j < nst; j++) wsb_put(&s, "%s pv%u_", j ? "," : "", j);
        wsb_put(&s, ";\n    prod_(pb_ + o_, %s", fixed ? "ok_" : "true");
        for (u32 j = 0; j < nst; j++) wsb_put(&s, ", &pv%u_", j);
        if (g->pkind == 2) {
            wsb_put(&s, ", g_p0, g_p1");
        } else {
            for (u32 b = 0; b <= pk->n_leaves; b++) wsb_put(&s, ", g_p%u", b);
            for (u32 b = 0; b <= pk->n_leaves; b++) wsb_put(&s, ", g_c%u", b);
            if (psc->n) {
                wsb_put(&s, ", g_sm");
                for (u32 j = 0; j < psc->n; j++) wsb_put(&s, ", g_sv%u", j);
            }
        }
        wsb_put(&s, ");\n");
        for (u32 j = 0; j < nst; j++)
            wsb_put(&s, "    const float pv%u_0 = pv%u_.x, pv%u_1 = pv%u_.y, pv%u_2 = pv%u_.z, pv%u_3 = pv%u_.w;\n", j, j,
                    j, j, j, j, j, j);
    }
    for (u32 v = 0; v < W && g->pkind && !vec_prod; v++) {
        wsb_put(&s, "    float");
        for (u32 j = 0; j < nst; j++) wsb_put(&s, "%s pv%u_%u", j ? "," : "", j, v);
        wsb_put(&s, ";\n    prod_(pb_ + o_ + %uu, %s", v, fixed ? "ok_" : "true");
        for (u32 j = 0; j < nst; j++) wsb_put(&s, ", &pv%u_%u", j, v);
        if (g->pkind == 1) {
            for (u32 b = 0; b <= pk->n_leaves; b++) wsb_put(&s, ", g_p%u", b);
            for (u32 b = 0; b <= pk->n_leaves; b++) wsb_put(&s, ", g_c%u", b);
            if (psc->n) {
                wsb_put(&s, ", g_sm");
                for (u32 j = 0; j < psc->n; j++) wsb_put(&s, ", g_sv%u", j);
            }
        } else {
            wsb_put(&s, ", g_p0, g_p1");
        }
        wsb_put(&s, ");\n");
    }
    /* each sum's body in op order, each op once per vector component */
    for (u32 m = 0; m < g->n_sum; m++) {
        const WinPlan *q = &((const WinEntry *)g->sum[m])->plan;
        const UOpKernel *k = ks[m];
        for (u32 i = q->R + 1; i < q->acc; i++) {
            if (!q->cone[i] || !op_type_is_float(k->ops[i].type)) continue;
            if (k->ops[i].type == KOP_LOAD) {
                u32 j = 0;
                while (q->ld_op[j] != i) j++;
                const u32 bi = k->ops[i].imm.u;
                u32 pm, pj;
                if (g->sub[m][bi] >= 0) {
                    for (u32 v = 0; v < W; v++) wsb_put(&s, "    const float m%u_f%u_%u = pv%d_%u;\n", m, i, v, g->sub[m][bi], v);
                } else if (wg_shared_load(g, m, j, &pm, &pj)) {
                    const u32 i2 = ((const WinEntry *)g->sum[pm])->plan.ld_op[pj];
                    for (u32 v = 0; v < W; v++) wsb_put(&s, "    const float m%u_f%u_%u = m%u_f%u_%u;\n", m, i, v, pm, i2, v);
                } else if (!q->ld_r[j]) {
                    for (u32 v = 0; v < W; v++) wsb_put(&s, "    const float m%u_f%u_%u = m%u_h%u_;\n", m, i, v, m, i);
                } else if (W == 4) {
                    wsb_put(&s, "    const float4 m%u_t%u_ = ld4nt_u(m%u_p%u, m%u_b%u_ + o_);\n", m, i, m, bi, m, i);
                    for (u32 v = 0; v < 4; v++)
                        wsb_put(&s, "    const float m%u_f%u_%u = m%u_t%u_.%c;\n", m, i, v, m, i, "xyzw"[v]);
                } else {
                    wsb_put(&s, "    const float m%u_f%u_0 = ((const float*)m%u_p%u)[m%u_b%u_ + o_];\n", m, i, m, bi, m, i);
                }
                continue;
            }
            for (u32 v = 0; v < W; v++) emit_member_op(&s, k, m, i, v);
        }
        for (u32 v = 0; v < W; v++)
            wsb_put(&s, fixed ? "    m%u_q%u_ = m%u_q%u_ + (ok_ ? m%u_f%u_%u : 0.0f);\n" : "    m%u_q%u_ = m%u_q%u_ + m%u_f%u_%u;\n",
                    m, v, m, v, m, q->value, v);
    }
    wsb_put(&s, "  }\n");
    for (u32 m = 0; m < g->n_sum; m++) {
        if (W == 4) wsb_put(&s, "  float m%u_t_ = (m%u_q0_ + m%u_q1_) + (m%u_q2_ + m%u_q3_);\n", m, m, m, m, m);
        else wsb_put(&s, "  float m%u_t_ = m%u_q0_;\n", m, m);
        wsb_put(&s, "  m%u_t_ = bsum(m%u_t_, red_);\n", m, m);
    }
    if (S > 1) {
        wsb_put(&s, "  if (sp_ != %uu) {\n", S - 1);
        for (u32 m = 0; m < g->n_sum; m++) wsb_put(&s, "    comb_put(sl_, gid + %uu, sp_, %uu, m%u_t_);\n", m * total, S, m);
        wsb_put(&s, "    return;\n  }\n");
    }
    for (u32 m = 0; m < g->n_sum; m++) {
        char fb[64];
        float_bits(fb, sizeof fb, ((const WinEntry *)g->sum[m])->plan.init_bits);
        if (S > 1) {
            char t[16], o[32];
            snprintf(t, sizeof t, "m%u_t_", m);
            snprintf(o, sizeof o, "gid + %uu", m * total);
            wsb_put(&s, "  {\n");
            emit_take_all(&s, S, t, o);
            wsb_put(&s, "    w_ = bsum(w_, red_);\n");
        } else
            wsb_put(&s, "  {\n    const float w_ = m%u_t_;\n", m);
        wsb_put(&s, "    if (lane == 0u) {\n      const float v%u_ = %s + w_;\n      ((float*)m%u_p0)[gid] = v%u_;\n", m, fb, m, m);
        for (u32 t = 0; t < g->n_tail; t++) {
            if (wg_root(g, WG_MAX_SUMS + t) != m) continue;
            char in[16];
            if (g->tsrc[t] < WG_MAX_SUMS) snprintf(in, sizeof in, "v%u_", g->tsrc[t]);
            else snprintf(in, sizeof in, "u%u_", g->tsrc[t] - WG_MAX_SUMS);
            wsb_put(&s, "      const float u%u_ = tl%u_(gid, %s", t, t, in);
            for (u32 b = 0; b <= g->tail[t]->n_leaves; b++) wsb_put(&s, ", t%u_p%u", t, b);
            for (u32 b = 0; b <= g->tail[t]->n_leaves; b++) wsb_put(&s, ", t%u_c%u", t, b);
            if (tsc[t].n) {
                wsb_put(&s, ", t%u_sm", t);
                for (u32 j = 0; j < tsc[t].n; j++) wsb_put(&s, ", t%u_sv%u", t, j);
            }
            wsb_put(&s, ");\n      (void)u%u_;\n", t);
        }
        wsb_put(&s, "    }\n  }\n");
    }
    wsb_put(&s, "}\n");
out:
    for (u32 m = 0; m < WG_MAX_SUMS; m++) free(ks[m]);
    free(pk);
    free(fnbuf);
    if (!ok) {
        free(s.p);
        return NULL;
    }
    return s.p;
}

int window_group_build(WinGroup *g) {
    if (!g->n_sum || (g->n_sum == 1 && !g->pkind && !g->n_tail)) return 0;
    const WinPlan *p = &((const WinEntry *)g->sum[0])->plan;
    const u64 key = wg_key(g);
    WgEntry *w = NULL;
    for (u32 i = 0; i < WGC.n && !w; i++)
        if (WGC.e[i].key == key) w = &WGC.e[i];
    if (!w) {
        if (WGC.n >= WG_CACHE || hipb.noalloc) return 0;
        w = &WGC.e[WGC.n++];
        memset(w, 0, sizeof *w);
        w->key = key;
        char name[48], err[256] = {0};
        snprintf(name, sizeof name, "thvm_rsg_%08x", (u32)(key & 0xFFFFFFFFu));
        /* every workgroup of an output waits for the others, so the whole
         * grid must be resident: the loop is unrolled less until the
         * kernel's registers allow that */
        static const u32 unrolls[] = {0, 8, 4, 2, 1};
        hipFunction_t f = NULL;
        for (u32 a = 0; a < sizeof unrolls / sizeof unrolls[0] && !f; a++) {
            char *src = gen_group(g, name, unrolls[a], &w->psc, w->tsc, err, sizeof err);
            if (!src) return 0;
            if (hipb.dump_src) fprintf(stderr, "---- run-sum group kernel ----\n%s\n", src);
            if (!rtc_build_module(src, &w->mod, err, sizeof err)) {
                fprintf(stderr, "tinyhvm-hip: run-sum group build failed: %s\n", err);
                free(src);
                return 0;
            }
            if (hipModuleGetFunction(&f, w->mod, name) != hipSuccess ||
                !co_form_make(&w->co, src, name, WIN_BLOCK, f)) {
                HIPB_CHECK(hipModuleUnload(w->mod));
                co_form_free(&w->co);
                w->mod = NULL;
                free(src);
                return 0;
            }
            free(src);
            w->cap = rtc_capacity(f, WIN_BLOCK);
            if (p->S > 1 && (u64)p->total * p->S > w->cap) {
                if (hipb.verbose)
                    fprintf(stderr, "tinyhvm-hip: %s (unroll %u): grid does not fit at once\n", name, unrolls[a]);
                co_form_free(&w->co);
                HIPB_CHECK(hipModuleUnload(w->mod));
                w->mod = NULL;
                f = NULL;
            }
        }
        if (!f) return 0;
        w->fn = f;
        hipb.n_compile++;
        if (hipb.verbose) {
            /* its parts by the names of their own kernels, in dispatch order */
            fprintf(stderr, "tinyhvm-hip: %s =", name);
            if (g->pkind == 1) fprintf(stderr, " thvm_ew_%08x +", (u32)(g->psig & 0xFFFFFFFFu));
            if (g->pkind == 2) fprintf(stderr, " %s +", ((const WinEntry *)g->pw)->name);
            for (u32 m = 0; m < g->n_sum; m++)
                fprintf(stderr, "%s %s", m ? " +" : "", ((const WinEntry *)g->sum[m])->name);
            for (u32 t = 0; t < g->n_tail; t++) fprintf(stderr, " + thvm_ew_%08x", (u32)(g->tsig[t] & 0xFFFFFFFFu));
            fprintf(stderr, "\n");
        }
    }
    if (!w->fn) return 0;
    g->fn = w->fn;
    g->co = &w->co;
    g->psc = &w->psc;
    g->tsc = w->tsc;
    g->grid = p->total * p->S;
    g->comb_words = p->S > 1 ? p->total * p->S * g->n_sum : 0;
    g->resident = p->S > 1;
    return 1;
}

static void wg_scalars(const KGenScalars *sc, const WgBufs *b, const u32 *dts, u32 *sm, float *sv) {
    *sm = 0;
    for (u32 j = 0; j < sc->n; j++) {
        const u32 id = b->b[1 + sc->leaf[j]].id;
        sv[j] = 0.0f;
        if (id && id != b->b[0].id && pool_host_value(id, dts[sc->leaf[j]], sc->index[j], &sv[j])) *sm |= 1u << j;
    }
}

u32 window_group_params(const WinGroup *g, WgArgs *a, void **params) {
    u32 np = 0, nptr = 0, ncnt = 0, nsv = 0;
    for (u32 m = 0; m < g->n_sum; m++)
        for (u32 b = 0; b < g->sb[m].nb; b++) {
            a->ptr[nptr] = g->sb[m].b[b].ptr ? g->sb[m].b[b].ptr : hipb.dummy;
            params[np++] = &a->ptr[nptr++];
        }
    if (g->pkind == 1) {
        for (u32 b = 0; b < g->pb.nb; b++) {
            a->ptr[nptr] = g->pb.b[b].ptr ? g->pb.b[b].ptr : hipb.dummy;
            params[np++] = &a->ptr[nptr++];
        }
        for (u32 b = 0; b < g->pb.nb; b++) {
            a->cnt[ncnt] = g->pb.b[b].ptr ? g->pb.b[b].cnt : 0u;
            params[np++] = &a->cnt[ncnt++];
        }
        if (g->psc->n) {
            wg_scalars(g->psc, &g->pb, g->pc->leaf_dtypes, &a->sm[0], &a->sv[nsv]);
            params[np++] = &a->sm[0];
            for (u32 j = 0; j < g->psc->n; j++) params[np++] = &a->sv[nsv++];
        }
    } else if (g->pkind == 2) {
        for (u32 b = 0; b < 2; b++) {
            a->ptr[nptr] = g->pb.b[b].ptr;
            params[np++] = &a->ptr[nptr++];
        }
    }
    for (u32 t = 0; t < g->n_tail; t++) {
        for (u32 b = 0; b < g->tb[t].nb; b++) {
            a->ptr[nptr] = g->tb[t].b[b].ptr ? g->tb[t].b[b].ptr : hipb.dummy;
            params[np++] = &a->ptr[nptr++];
        }
        for (u32 b = 0; b < g->tb[t].nb; b++) {
            a->cnt[ncnt] = g->tb[t].b[b].ptr ? g->tb[t].b[b].cnt : 0u;
            params[np++] = &a->cnt[ncnt++];
        }
        if (g->tsc[t].n) {
            wg_scalars(&g->tsc[t], &g->tb[t], g->tail[t]->leaf_dtypes, &a->sm[1 + t], &a->sv[nsv]);
            params[np++] = &a->sm[1 + t];
            for (u32 j = 0; j < g->tsc[t].n; j++) params[np++] = &a->sv[nsv++];
        }
    }
    params[np++] = &hipb.comb_slots;
    return np;
}

void window_group_mem(const WinGroup *g, HbMem *m) {
    m->n = 0;
    for (u32 s = 0; s < g->n_sum; s++)
        for (u32 b = 0; b < g->sb[s].nb; b++)
            hbm_add(m, g->sb[s].b[b].ptr, g->sb[s].b[b].bytes, b == 0);
    for (u32 b = 0; b < g->pb.nb && g->pkind; b++) {
        int wr = g->pkind == 2 ? b == 0 : 0;
        for (u32 j = 0; g->pkind == 1 && j < g->pc->n_st; j++) wr |= g->pc->st_slot[j] == b;
        hbm_add(m, g->pb.b[b].ptr, g->pb.b[b].bytes, wr);
    }
    for (u32 t = 0; t < g->n_tail; t++)
        for (u32 b = 0; b < g->tb[t].nb; b++)
            hbm_add(m, g->tb[t].b[b].ptr, g->tb[t].b[b].bytes, b == 0);
}

u64 window_group_tail_reads(const WinGroup *g, u32 t) {
    const UOpKernel *k = g->tail[t];
    u32 sm;
    float sv[KGEN_MAX_SCALARS];
    wg_scalars(&g->tsc[t], &g->tb[t], k->leaf_dtypes, &sm, sv);
    u64 reads = 0;
    for (u32 i = 0; i < k->n_ops; i++) {
        const KOp *op = &k->ops[i];
        if (op->type != KOP_LOAD || op->imm.u == 0 || op->imm.u > k->n_leaves || op->imm.u == g->tleaf[t]) continue;
        int inl = 0;
        for (u32 j = 0; j < g->tsc[t].n && !inl; j++)
            inl = g->tsc[t].leaf[j] == op->imm.u - 1 && ((sm >> j) & 1u) && k->ops[op->arg[0]].type == KOP_CONST_U &&
                  k->ops[op->arg[0]].imm.u == g->tsc[t].index[j];
        if (!inl && op->imm.u - 1 < 64) reads |= 1ull << (op->imm.u - 1);
    }
    return reads;
}

/* a recognised program's entry outside the cache (not compiled), or NULL */
static WinEntry *wg_temp_entry(const UOpKernel *k) {
    WinEntry *e = calloc(1, sizeof *e);
    if (!e) return NULL;
    e->key = win_key(k);
    e->n_ops = k->n_ops;
    e->n_leaves = k->n_leaves;
    e->ops = malloc((size_t)k->n_ops * sizeof(KOp) + 1);
    if (!e->ops || k->n_leaves > FUSE_MAX_LEAVES || !win_recognize(k, &e->plan)) {
        free(e->ops);
        free(e);
        return NULL;
    }
    memcpy(e->ops, k->ops, (size_t)k->n_ops * sizeof(KOp));
    e->meta[0] = k->grid[0]; e->meta[1] = k->grid[1]; e->meta[2] = k->grid[2];
    e->meta[3] = k->local_size; e->meta[4] = k->out_dtype;
    memcpy(e->dts, k->leaf_dtypes, (size_t)k->n_leaves * sizeof(u32));
    e->kind = e->plan.kind;
    return e;
}

char *window_group_source(const UOpKernel *const *ks, const u32 *const *bufs, u32 n, int producer, char *err,
                          size_t errlen) {
    static WinGroup g;
    ChainInfo *pc = NULL;
    WinEntry *tmp[1 + WG_MAX_SUMS] = {0};
    u32 ntmp = 0;
    char *src = NULL;
    wg_clear(&g);
    if (!ks || !bufs || n < 2) { snprintf(err, errlen, "need at least two programs"); return NULL; }
    u32 i = 0;
    if (producer) {
        WinEntry *we = wg_temp_entry(ks[0]);
        if (we && we->kind == WIN_MAX) {
            tmp[ntmp++] = we;
            if (!window_group_of_wmax(&g, we, bufs[0][0], bufs[0][ks[0]->ops[we->plan.ld_op[0]].imm.u])) {
                snprintf(err, errlen, "window max producer refused");
                goto out;
            }
        } else {
            if (we) { free(we->ops); free(we); }
            pc = chain_info_make(ks[0], ks[0]->ops);
            if (!pc || !window_group_of_chain(&g, pc, bufs[0])) {
                snprintf(err, errlen, "producer refused");
                goto out;
            }
        }
        i = 1;
    }
    for (; i < n; i++) {
        int loop = 0;
        for (u32 q = 0; q < ks[i]->n_ops; q++) loop |= ks[i]->ops[q].type == KOP_RANGE;
        if (loop) {
            WinEntry *we = ntmp <= WG_MAX_SUMS ? wg_temp_entry(ks[i]) : NULL;
            if (!we) { snprintf(err, errlen, "program %u not a run sum", i); goto out; }
            tmp[ntmp++] = we;
            if (we->kind != WIN_SUM || !window_group_add_sum(&g, we, bufs[i][0], bufs[i] + 1, ks[i]->n_leaves)) {
                snprintf(err, errlen, "run sum %u does not join", i);
                goto out;
            }
        } else if (!window_group_add_tail(&g, ks[i], bufs[i][0], bufs[i] + 1, ks[i]->n_leaves)) {
            snprintf(err, errlen, "consumer %u does not join", i);
            goto out;
        }
    }
    {
        KGenScalars psc, tsc[WG_MAX_TAILS];
        src = gen_group(&g, "thvm_rsg_check", 0, &psc, tsc, err, errlen);
    }
out:
    free(pc);
    for (u32 q = 0; q < ntmp; q++) { free(tmp[q]->ops); free(tmp[q]); }
    wg_clear(&g);
    return src;
}

void window_shutdown(void) {
    if (WC.tab) {
        for (u32 i = 0; i < WC.cap; i++) {
            if (!WC.tab[i].key) continue;
            if (WC.tab[i].kind != WIN_NONE) HIPB_CHECK(hipModuleUnload(WC.tab[i].mod));
            co_form_free(&WC.tab[i].co);
            free(WC.tab[i].ops);
        }
        free(WC.tab);
    }
    memset(&WC, 0, sizeof WC);
    scratch_release(&win_ws);
    for (u32 i = 0; i < WGC.n; i++) {
        if (WGC.e[i].fn) HIPB_CHECK(hipModuleUnload(WGC.e[i].mod));
        co_form_free(&WGC.e[i].co);
    }
    for (u32 i = 0; i < WGC.n_tail; i++) free(WGC.tail[i]);
    memset(&WGC, 0, sizeof WGC);
}
