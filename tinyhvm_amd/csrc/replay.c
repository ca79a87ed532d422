/*
 * replay.c - loads a kernel trace (include/thvm_trace.h) and replays it
 * against any Backend vtable.
 *
 * This is the capture/replay path of the Metal backend's JIT
 * (src/backend/metal/jit.m:24-631) done at the vtable boundary: the engine's
 * calls for one step are recorded once and re-issued without the engine.
 *
 * Buffer ids: the trace's ids are mapped to whatever ids the target backend
 * hands out. An ALLOC of a trace id that is already bound (a step replayed
 * again) first frees the old binding, so repeated steps reuse memory.
 *
 * The same source builds against the engine's own header
 * (THVM_REPLAY_ENGINE_HEADER) to drive the engine's CPU backend.
 */
#ifdef THVM_REPLAY_ENGINE_HEADER
#include "tinyhvm.h"
#else
#include "thvm_abi.h"
#endif
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "thvm_gen.h"
#include "thvm_trace.h"
#include "thvm_replay.h"

typedef struct {
    u32 tag;
    u32 id, id2;           /* primary / secondary trace buffer id */
    u64 bytes;
    const u8 *data;        /* WRITE raw / READ / SNAPSHOT payload */
    u32 enc, dist, dtype;  /* WRITE gen spec */
    u64 seed;
    f32 p0, p1;
    u32 n_leaves;
    u32 *leaf_ids;
    UOpKernel *uk;         /* UOP */
    /* RS */
    View *views;
    ShapeTracker *sts;
    u8 *has_st;
    FusedOp *ops;
    u32 n_ops;
    Shape full;
    u32 has_reduce;
    ReduceSpec reduce;
    u32 has_dtypes;
    u32 *leaf_dtypes;
    u32 out_dtype;
    View cview;            /* CONTIG */
    u32 numel;
    /* OPUN / OPBIN / OPMM / OPRED (id = dst, id2 = a or src, id3 = b) */
    u32 uop, id3, dd, ad, bd, mm_m, mm_k, mm_n, dn, sn, rdim;
    View *lv;              /* dst, a, b views */
    /* ADAM (id = param, id2 = grad, id3 = m, id4 = v, n = numel) */
    u32 id4;
    f32 ad_lr, ad_b1, ad_b2, ad_eps, ad_bc1, ad_bc2;
    char *text;            /* MARK */
    void *gen_cache;       /* materialized GEN data */
} TRec;

struct ThvmTrace {
    u8 *blob;
    size_t blob_len;
    TRec *recs;
    u32 n;
    u32 max_id;
    u32 *live;             /* trace id -> backend id */
};

typedef struct { const u8 *p, *end; int bad; } Cur;

static u32 c_u32(Cur *c) {
    u32 v = 0;
    if (c->p + 4 > c->end) { c->bad = 1; return 0; }
    memcpy(&v, c->p, 4);
    c->p += 4;
    return v;
}
static u64 c_u64(Cur *c) {
    u64 v = 0;
    if (c->p + 8 > c->end) { c->bad = 1; return 0; }
    memcpy(&v, c->p, 8);
    c->p += 8;
    return v;
}
static f32 c_f32(Cur *c) {
    u32 u = c_u32(c);
    f32 f;
    memcpy(&f, &u, 4);
    return f;
}
static const u8 *c_raw(Cur *c, u64 n) {
    if ((u64)(c->end - c->p) < n) { c->bad = 1; return NULL; }
    const u8 *r = c->p;
    c->p += n;
    return r;
}
static void c_shape(Cur *c, Shape *s) {
    memset(s, 0, sizeof *s);
    s->rank = c_u32(c);
    for (int d = 0; d < MAX_DIM; d++) s->dims[d] = c_u32(c);
}
static void c_view(Cur *c, View *v) {
    memset(v, 0, sizeof *v);
    c_shape(c, &v->shape);
    for (int d = 0; d < MAX_DIM; d++) v->strides[d] = (i32)c_u32(c);
    v->offset = (i32)c_u32(c);
    v->numel = c_u32(c);
    v->contiguous = (u8)c_u32(c);
    v->has_mask = (u8)c_u32(c);
    for (int d = 0; d < MAX_DIM; d++) v->mask_begin[d] = c_u32(c);
    for (int d = 0; d < MAX_DIM; d++) v->mask_end[d] = c_u32(c);
    v->n_compound_masks = (u8)c_u32(c);
    for (int i = 0; i < 2; i++) {
        v->compound_masks[i].dim_a = (u8)c_u32(c);
        v->compound_masks[i].dim_b = (u8)c_u32(c);
        v->compound_masks[i].stride_a = (i32)c_u32(c);
        v->compound_masks[i].begin = c_u32(c);
        v->compound_masks[i].end = c_u32(c);
    }
    for (int d = 0; d < MAX_DIM; d++) v->mod_size[d] = c_u32(c);
}

static void note_id(ThvmTrace *t, u32 id) {
    if (id > t->max_id) t->max_id = id;
}

static int parse_rec(ThvmTrace *t, TRec *r, u32 tag, const u8 *p, u64 len) {
    Cur c = {p, p + len, 0};
    r->tag = tag;
    switch (tag) {
    case TRC_ALLOC:
        r->id = c_u32(&c); c_u32(&c); r->bytes = c_u64(&c);
        note_id(t, r->id);
        break;
    case TRC_FREE: case TRC_INCREF: case TRC_DECREF:
        r->id = c_u32(&c);
        break;
    case TRC_WRITE:
        r->id = c_u32(&c); r->enc = c_u32(&c); r->bytes = c_u64(&c);
        if (r->enc == TRC_ENC_RAW) r->data = c_raw(&c, r->bytes);
        else {
            r->dist = c_u32(&c); r->dtype = c_u32(&c); r->seed = c_u64(&c);
            r->p0 = c_f32(&c); r->p1 = c_f32(&c);
        }
        break;
    case TRC_READ: {
        r->id = c_u32(&c);
        u32 has = c_u32(&c);
        r->bytes = c_u64(&c);
        if (has) r->data = c_raw(&c, r->bytes);
        break;
    }
    case TRC_UOP: {
        r->id = c_u32(&c);
        r->n_leaves = c_u32(&c);
        if (r->n_leaves > FUSE_MAX_LEAVES) return 0;
        r->leaf_ids = calloc(r->n_leaves + 1, sizeof(u32));
        for (u32 i = 0; i < r->n_leaves; i++) r->leaf_ids[i] = c_u32(&c);
        (void)c_u64(&c); /* cache key */
        UOpKernel *k = calloc(1, sizeof(UOpKernel));
        if (!k || !r->leaf_ids) return 0;
        r->uk = k;
        k->n_ops = c_u32(&c); k->n_bufs = c_u32(&c); k->rank = c_u32(&c);
        k->n_leaves = r->n_leaves;
        if (k->n_ops > KOP_MAX) return 0;
        c_shape(&c, &k->full_shape);
        for (int i = 0; i < 3; i++) k->grid[i] = c_u32(&c);
        for (int i = 0; i < 3; i++) k->tg[i] = c_u32(&c);
        k->local_size = c_u32(&c); k->reduce_numel = c_u32(&c); k->out_dtype = c_u32(&c);
        for (int d = 0; d < MAX_DIM; d++) k->coord_uop[d] = c_u32(&c);
        for (u32 i = 0; i < k->n_ops; i++) {
            k->ops[i].type = (KOpType)c_u32(&c);
            k->ops[i].arg[0] = c_u32(&c); k->ops[i].arg[1] = c_u32(&c); k->ops[i].arg[2] = c_u32(&c);
            k->ops[i].imm.u = c_u32(&c);
        }
        for (u32 i = 0; i < r->n_leaves; i++) c_view(&c, &k->leaf_views[i]);
        for (u32 i = 0; i < r->n_leaves; i++) k->leaf_dtypes[i] = c_u32(&c);
        break;
    }
    case TRC_RS: {
        r->id = c_u32(&c);
        u32 n = r->n_leaves = c_u32(&c);
        if (n > FUSE_MAX_LEAVES) return 0;
        r->leaf_ids = calloc(n + 1, sizeof(u32));
        r->views = calloc(n + 1, sizeof(View));
        r->sts = calloc(n + 1, sizeof(ShapeTracker));
        r->has_st = calloc(n + 1, 1);
        r->leaf_dtypes = calloc(n + 1, sizeof(u32));
        if (!r->leaf_ids || !r->views || !r->sts || !r->has_st || !r->leaf_dtypes) return 0;
        for (u32 i = 0; i < n; i++) r->leaf_ids[i] = c_u32(&c);
        for (u32 i = 0; i < n; i++) c_view(&c, &r->views[i]);
        for (u32 i = 0; i < n; i++) r->has_st[i] = (u8)c_u32(&c);
        for (u32 i = 0; i < n; i++) {
            if (!r->has_st[i]) continue;
            u32 nv = c_u32(&c);
            if (nv > ST_MAX_VIEWS) return 0;
            r->sts[i].n_views = (u8)nv;
            for (u32 v = 0; v < nv; v++) c_view(&c, &r->sts[i].views[v]);
        }
        r->n_ops = c_u32(&c);
        if (r->n_ops > FUSE_MAX_OPS) return 0;
        r->ops = calloc(r->n_ops + 1, sizeof(FusedOp));
        if (!r->ops) return 0;
        for (u32 i = 0; i < r->n_ops; i++) {
            r->ops[i].uop = c_u32(&c); r->ops[i].arg_a = c_u32(&c);
            r->ops[i].arg_b = c_u32(&c); r->ops[i].aux = c_u32(&c);
        }
        c_shape(&c, &r->full);
        r->has_reduce = c_u32(&c);
        if (r->has_reduce) {
            for (int d = 0; d < MAX_DIM; d++) r->reduce.is_reduce[d] = (u8)c_u32(&c);
            r->reduce.reduce_type = c_u32(&c);
            r->reduce.post_reduce_start = c_u32(&c);
            r->reduce.n_post_leaves = c_u32(&c);
            r->reduce.reduce2_type = c_u32(&c);
            r->reduce.reduce2_start = c_u32(&c);
            for (int d = 0; d < MAX_DIM; d++) r->reduce.is_reduce2[d] = (u8)c_u32(&c);
        }
        u32 ns = c_u32(&c);
        for (u32 i = 0; i < 2 * ns; i++) (void)c_u32(&c); /* side outputs: unused by the engine */
        r->has_dtypes = c_u32(&c);
        if (r->has_dtypes) for (u32 i = 0; i < n; i++) r->leaf_dtypes[i] = c_u32(&c);
        r->out_dtype = c_u32(&c);
        break;
    }
    case TRC_COPY:
        r->id = c_u32(&c); r->id2 = c_u32(&c); r->bytes = c_u64(&c);
        break;
    case TRC_CONTIG:
        r->id = c_u32(&c); r->numel = c_u32(&c); r->id2 = c_u32(&c);
        c_view(&c, &r->cview);
        break;
    case TRC_RESET:
    case TRC_PERSIST:
        r->id = c_u32(&c);
        break;
    case TRC_SNAPSHOT:
        r->id = c_u32(&c); c_u32(&c); r->bytes = c_u64(&c);
        r->data = c_raw(&c, r->bytes);
        break;
    case TRC_OPUN:
    case TRC_OPBIN:
    case TRC_OPMM:
        r->lv = calloc(3, sizeof(View));
        if (!r->lv) return 0;
        if (tag == TRC_OPMM) {
            r->id = c_u32(&c); r->dd = c_u32(&c);
            r->id2 = c_u32(&c); r->ad = c_u32(&c); c_view(&c, &r->lv[1]);
            r->id3 = c_u32(&c); r->bd = c_u32(&c); c_view(&c, &r->lv[2]);
            r->mm_m = c_u32(&c); r->mm_k = c_u32(&c); r->mm_n = c_u32(&c);
        } else {
            r->uop = c_u32(&c); r->id = c_u32(&c); r->dd = c_u32(&c); c_view(&c, &r->lv[0]);
            r->id2 = c_u32(&c); r->ad = c_u32(&c); c_view(&c, &r->lv[1]);
            if (tag == TRC_OPBIN) { r->id3 = c_u32(&c); r->bd = c_u32(&c); c_view(&c, &r->lv[2]); }
        }
        break;
    case TRC_OPRED:
        r->uop = c_u32(&c); r->id = c_u32(&c); r->dn = c_u32(&c); r->dd = c_u32(&c);
        r->id2 = c_u32(&c); r->sn = c_u32(&c); r->ad = c_u32(&c); r->rdim = c_u32(&c);
        break;
    case TRC_ADAM:
        r->id = c_u32(&c); r->id2 = c_u32(&c); r->id3 = c_u32(&c); r->id4 = c_u32(&c);
        r->ad_lr = c_f32(&c); r->ad_b1 = c_f32(&c); r->ad_b2 = c_f32(&c); r->ad_eps = c_f32(&c);
        r->ad_bc1 = c_f32(&c); r->ad_bc2 = c_f32(&c);
        r->numel = c_u32(&c);
        break;
    case TRC_MARK: {
        u32 n = c_u32(&c);
        const u8 *s = c_raw(&c, n);
        r->text = calloc(n + 1, 1);
        if (r->text && s) memcpy(r->text, s, n);
        break;
    }
    default:
        break;
    }
    return !c.bad;
}

ThvmTrace *thvm_trace_load(const char *path) {
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    fseek(f, 0, SEEK_END);
    long sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    ThvmTrace *t = calloc(1, sizeof *t);
    if (!t || sz < 8) { fclose(f); free(t); return NULL; }
    t->blob = malloc((size_t)sz);
    t->blob_len = (size_t)sz;
    if (!t->blob || fread(t->blob, 1, (size_t)sz, f) != (size_t)sz ||
        memcmp(t->blob, THVM_TRACE_MAGIC, 8) != 0) {
        fclose(f);
        thvm_trace_free(t);
        return NULL;
    }
    fclose(f);
    u32 cap = 64;
    t->recs = calloc(cap, sizeof(TRec));
    size_t o = 8;
    while (o + 16 <= t->blob_len) {
        u32 tag;
        u64 len;
        memcpy(&tag, t->blob + o, 4);
        memcpy(&len, t->blob + o + 8, 8);
        o += 16;
        if (o + len > t->blob_len) break;
        if (t->n == cap) {
            cap *= 2;
            TRec *nr = realloc(t->recs, cap * sizeof(TRec));
            if (!nr) break;
            t->recs = nr;
        }
        memset(&t->recs[t->n], 0, sizeof(TRec));
        if (!parse_rec(t, &t->recs[t->n], tag, t->blob + o, len)) {
            fprintf(stderr, "thvm_trace_load: %s: bad record %u\n", path, t->n);
            thvm_trace_free(t);
            return NULL;
        }
        t->n++;
        o += len;
    }
    t->live = calloc(t->max_id + 1, sizeof(u32));
    return t;
}

void thvm_trace_free(ThvmTrace *t) {
    if (!t) return;
    for (u32 i = 0; i < t->n; i++) {
        TRec *r = &t->recs[i];
        free(r->leaf_ids); free(r->uk); free(r->views); free(r->sts); free(r->has_st);
        free(r->ops); free(r->leaf_dtypes); free(r->text); free(r->gen_cache); free(r->lv);
    }
    free(t->recs);
    free(t->live);
    free(t->blob);
    free(t);
}

u32 thvm_trace_count(const ThvmTrace *t) { return t ? t->n : 0; }
u32 thvm_trace_tag(const ThvmTrace *t, u32 i) { return (t && i < t->n) ? t->recs[i].tag : 0; }
u32 thvm_trace_rec_id(const ThvmTrace *t, u32 i) { return (t && i < t->n) ? t->recs[i].id : 0; }
u64 thvm_trace_rec_bytes(const ThvmTrace *t, u32 i) { return (t && i < t->n) ? t->recs[i].bytes : 0; }
const void *thvm_trace_rec_data(const ThvmTrace *t, u32 i) { return (t && i < t->n) ? t->recs[i].data : NULL; }
const UOpKernel *thvm_trace_rec_kernel(const ThvmTrace *t, u32 i) { return (t && i < t->n) ? t->recs[i].uk : NULL; }

int thvm_trace_find_mark(const ThvmTrace *t, const char *text, u32 from) {
    if (!t) return -1;
    for (u32 i = from; i < t->n; i++)
        if (t->recs[i].tag == TRC_MARK && t->recs[i].text && strcmp(t->recs[i].text, text) == 0)
            return (int)i;
    return -1;
}

u32 thvm_trace_live_id(const ThvmTrace *t, u32 trace_id) {
    if (!t || trace_id > t->max_id) return 0;
    return t->live[trace_id];
}

/* ---- synthetic data: multithreaded generator fill ---- */
typedef struct { void *dst; u32 dtype, dist; u64 seed; f32 p0, p1; u64 lo, hi; } GenJob;

static void *gen_worker(void *arg) {
    GenJob *j = arg;
    thvm_gen_fill(j->dst, j->dtype, j->dist, j->seed, j->p0, j->p1, j->lo, j->hi);
    return NULL;
}

void thvm_gen_fill_parallel(void *dst, u32 dtype, u32 dist, u64 seed, f32 p0, f32 p1, u64 n, u32 threads) {
    if (threads == 0) {
        long nc = sysconf(_SC_NPROCESSORS_ONLN);
        threads = nc > 0 ? (u32)nc : 1;
        if (threads > 16) threads = 16;
    }
    if (n < 65536 || threads <= 1) {
        thvm_gen_fill(dst, dtype, dist, seed, p0, p1, 0, n);
        return;
    }
    pthread_t th[64];
    GenJob jobs[64];
    u8 joined[64];
    if (threads > 64) threads = 64;
    u64 per = (n + threads - 1) / threads;
    for (u32 i = 0; i < threads; i++) {
        u64 lo = (u64)i * per, hi = lo + per > n ? n : lo + per;
        joined[i] = 0;
        if (lo >= hi) continue;
        jobs[i] = (GenJob){dst, dtype, dist, seed, p0, p1, lo, hi};
        if (pthread_create(&th[i], NULL, gen_worker, &jobs[i]) == 0) joined[i] = 1;
        else gen_worker(&jobs[i]);
    }
    for (u32 i = 0; i < threads; i++)
        if (joined[i]) pthread_join(th[i], NULL);
}

static const void *write_payload(TRec *r) {
    if (r->enc == TRC_ENC_RAW) return r->data;
    if (!r->gen_cache) {
        r->gen_cache = malloc(r->bytes ? r->bytes : 4);
        if (!r->gen_cache) return NULL;
        thvm_gen_fill_parallel(r->gen_cache, r->dtype, r->dist, r->seed, r->p0, r->p1,
                               r->bytes / thvm_gen_esize(r->dtype), 0);
    }
    return r->gen_cache;
}

void thvm_trace_drop_gen_cache(ThvmTrace *t) {
    if (!t) return;
    for (u32 i = 0; i < t->n; i++) {
        free(t->recs[i].gen_cache);
        t->recs[i].gen_cache = NULL;
    }
}

static u32 L(ThvmTrace *t, u32 id) { return id <= t->max_id ? t->live[id] : 0; }

int thvm_trace_replay(ThvmTrace *t, const Backend *be, u32 lo, u32 hi, u32 flags) {
    if (!t || !be) return -1;
    if (hi > t->n) hi = t->n;
    int dispatched = 0;
    for (u32 i = lo; i < hi; i++) {
        TRec *r = &t->recs[i];
        switch (r->tag) {
        case TRC_ALLOC: {
            if (r->id > t->max_id) break;
            if (t->live[r->id] && be->buf_free) be->buf_free(t->live[r->id]);
            t->live[r->id] = be->buf_alloc(r->bytes);
            if (!t->live[r->id]) {
                fprintf(stderr, "thvm_trace_replay: allocation of %llu bytes failed\n",
                        (unsigned long long)r->bytes);
                return -1;
            }
            break;
        }
        case TRC_FREE:
            if (L(t, r->id) && be->buf_free) be->buf_free(L(t, r->id));
            if (r->id <= t->max_id) t->live[r->id] = 0;
            break;
        case TRC_INCREF:
            if (be->buf_incref) be->buf_incref(L(t, r->id));
            break;
        case TRC_DECREF:
            if (be->buf_decref) be->buf_decref(L(t, r->id));
            break;
        case TRC_WRITE: {
            if (flags & THVM_REPLAY_SKIP_WRITES) break;
            const void *d = write_payload(r);
            if (d && L(t, r->id)) be->buf_write(L(t, r->id), d, r->bytes);
            break;
        }
        case TRC_READ:
            if (flags & THVM_REPLAY_SKIP_READS) break;
            if (L(t, r->id)) {
                void *tmp = malloc(r->bytes ? r->bytes : 4);
                if (tmp) {
                    be->buf_read(L(t, r->id), tmp, r->bytes);
                    free(tmp);
                }
            }
            break;
        case TRC_UOP: {
            u32 leaves[FUSE_MAX_LEAVES];
            for (u32 j = 0; j < r->n_leaves; j++) leaves[j] = L(t, r->leaf_ids[j]);
            be->dispatch_uop_kernel(L(t, r->id), leaves, r->n_leaves, r->uk, 0);
            dispatched++;
            break;
        }
        case TRC_RS: {
            u32 leaves[FUSE_MAX_LEAVES];
            const View *vp[FUSE_MAX_LEAVES];
            const ShapeTracker *sp[FUSE_MAX_LEAVES];
            for (u32 j = 0; j < r->n_leaves; j++) {
                leaves[j] = L(t, r->leaf_ids[j]);
                vp[j] = &r->views[j];
                sp[j] = r->has_st[j] ? &r->sts[j] : NULL;
            }
            be->dispatch_kernel_rs(L(t, r->id), leaves, vp, sp, r->n_leaves, r->ops, r->n_ops, &r->full,
                                   r->has_reduce ? &r->reduce : NULL, NULL, NULL, 0,
                                   r->has_dtypes ? r->leaf_dtypes : NULL, r->out_dtype);
            dispatched++;
            break;
        }
        case TRC_COPY:
            if (be->buf_copy) be->buf_copy(L(t, r->id), L(t, r->id2), r->bytes);
            break;
        case TRC_CONTIG:
            if (be->contiguify) be->contiguify(L(t, r->id), r->numel, L(t, r->id2), &r->cview);
            break;
        case TRC_OPUN:
            if (be->op_unary) be->op_unary(r->uop, L(t, r->id), &r->lv[0], r->dd, L(t, r->id2), &r->lv[1], r->ad);
            dispatched++;
            break;
        case TRC_OPBIN:
            if (be->op_binary)
                be->op_binary(r->uop, L(t, r->id), &r->lv[0], r->dd, L(t, r->id2), &r->lv[1], r->ad,
                              L(t, r->id3), &r->lv[2], r->bd);
            dispatched++;
            break;
        case TRC_OPMM:
            if (be->op_mm)
                be->op_mm(L(t, r->id), r->dd, L(t, r->id2), &r->lv[1], r->ad, L(t, r->id3), &r->lv[2], r->bd,
                          r->mm_m, r->mm_k, r->mm_n);
            dispatched++;
            break;
        case TRC_OPRED:
            if (be->op_reduce) be->op_reduce(r->uop, L(t, r->id), r->dn, r->dd, L(t, r->id2), r->sn, r->ad, r->rdim);
            dispatched++;
            break;
        case TRC_ADAM:
            /* a backend without the slot leaves the buffers as they are, as
             * the engine's adam_step_direct does (src/nn/adam.c:108) */
            if (be->adam_step)
                be->adam_step(L(t, r->id), L(t, r->id2), L(t, r->id3), L(t, r->id4), r->ad_lr, r->ad_b1, r->ad_b2,
                              r->ad_eps, r->ad_bc1, r->ad_bc2, r->numel);
            dispatched++;
            break;
        case TRC_RESET:
            /* ids are remapped; the target's own pool keeps its numbering */
            break;
        case TRC_PERSIST:
            break;
        default:
            break;
        }
    }
    return dispatched;
}

void thvm_trace_release(ThvmTrace *t, const Backend *be) {
    if (!t || !be) return;
    for (u32 i = 0; i <= t->max_id; i++) {
        if (t->live[i] && be->buf_free) be->buf_free(t->live[i]);
        t->live[i] = 0;
    }
}
