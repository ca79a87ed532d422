/*
 * capture.c - records the Backend calls that the TinyHVM engine makes for
 * each benchmark workload, as kernel traces (include/thvm_trace.h).
 *
 * Built only in the development container, from the engine sources where
 * they lie (see oracle/ref.mk): this file includes src/tinyhvm.c and the
 * engine's CPU backend (src/backend/cpu/_.c), wraps every slot of the
 * cpu_backend vtable with a recorder that forwards to the original, and
 * drives the engine's public tensor API (src/tinyhvm.h:1287-1544).
 *
 * In exec mode the CPU backend runs every kernel and a SNAPSHOT record with
 * the output buffer follows each dispatch: those are the golden vectors.
 * In record-only mode (-n) the kernels are not run; that is used for the
 * full-size workloads whose CPU run would take hours, and whose inputs are
 * described by generator specs rather than stored.
 *
 * Usage: capture [-n] <workload> <out.trc> [size args...]
 */
#include "tinyhvm.c"
#include "backend/cpu/_.c"
#include "thvm_trace.h"
#include "thvm_gen.h"

static FILE *g_out;
static int g_exec = 1;
static Backend g_orig;

typedef struct { u8 *p; size_t n, cap; } RecBuf;
static RecBuf rb;

static void rb_need(size_t k) {
    if (rb.n + k > rb.cap) {
        size_t c = rb.cap ? rb.cap : 4096;
        while (c < rb.n + k) c *= 2;
        rb.p = realloc(rb.p, c);
        rb.cap = c;
    }
}
static void rb_bytes(const void *d, size_t k) { rb_need(k); memcpy(rb.p + rb.n, d, k); rb.n += k; }
static void rb_u32(u32 v) { rb_bytes(&v, 4); }
static void rb_i32(i32 v) { rb_bytes(&v, 4); }
static void rb_u64(u64 v) { rb_bytes(&v, 8); }
static void rb_f32(f32 v) { rb_bytes(&v, 4); }
static void rb_begin(void) { rb.n = 0; }
static void rb_emit(u32 tag) {
    u32 hdr[2] = {tag, 0};
    u64 len = rb.n;
    fwrite(hdr, 4, 2, g_out);
    fwrite(&len, 8, 1, g_out);
    if (rb.n) fwrite(rb.p, 1, rb.n, g_out);
}

static void rb_shape(const Shape *s) {
    rb_u32(s->rank);
    for (u32 d = 0; d < MAX_DIM; d++) rb_u32(s->dims[d]);
}
static void rb_view(const View *v) {
    rb_shape(&v->shape);
    for (u32 d = 0; d < MAX_DIM; d++) rb_i32(v->strides[d]);
    rb_i32(v->offset);
    rb_u32(v->numel);
    rb_u32(v->contiguous);
    rb_u32(v->has_mask);
    for (u32 d = 0; d < MAX_DIM; d++) rb_u32(v->mask_begin[d]);
    for (u32 d = 0; d < MAX_DIM; d++) rb_u32(v->mask_end[d]);
    rb_u32(v->n_compound_masks);
    for (u32 i = 0; i < 2; i++) {
        rb_u32(v->compound_masks[i].dim_a);
        rb_u32(v->compound_masks[i].dim_b);
        rb_i32(v->compound_masks[i].stride_a);
        rb_u32(v->compound_masks[i].begin);
        rb_u32(v->compound_masks[i].end);
    }
    for (u32 d = 0; d < MAX_DIM; d++) rb_u32(v->mod_size[d]);
}
static void rb_reduce(const ReduceSpec *r) {
    for (u32 d = 0; d < MAX_DIM; d++) rb_u32(r->is_reduce[d]);
    rb_u32(r->reduce_type);
    rb_u32(r->post_reduce_start);
    rb_u32(r->n_post_leaves);
    rb_u32(r->reduce2_type);
    rb_u32(r->reduce2_start);
    for (u32 d = 0; d < MAX_DIM; d++) rb_u32(r->is_reduce2[d]);
}

static void rec_mark(const char *text) {
    rb_begin();
    u32 n = (u32)strlen(text);
    rb_u32(n);
    rb_bytes(text, n);
    rb_emit(TRC_MARK);
}

static void rec_snapshot(u32 id) {
    if (!g_exec || id == 0 || id >= MAX_BUFS || !cpu_pool.bufs[id]) return;
    rb_begin();
    rb_u32(id);
    rb_u32(0);
    rb_u64(cpu_pool.sizes[id]);
    rb_bytes(cpu_pool.bufs[id], cpu_pool.sizes[id]);
    rb_emit(TRC_SNAPSHOT);
}

/* ---- generator spec attached to the next buf_write ---- */
static struct { int active; u32 dist, dtype; u64 seed; f32 p0, p1; } g_gen;

/* ---- recording wrappers ---- */
static int cap_init(void) { return g_orig.init ? g_orig.init() : 0; }
static void cap_shutdown(void) { if (g_orig.shutdown) g_orig.shutdown(); }

static u32 cap_buf_alloc(u64 bytes) {
    u32 id = g_orig.buf_alloc(bytes);
    rb_begin(); rb_u32(id); rb_u32(0); rb_u64(bytes); rb_emit(TRC_ALLOC);
    return id;
}
static void cap_buf_free(u32 id) {
    rb_begin(); rb_u32(id); rb_emit(TRC_FREE);
    g_orig.buf_free(id);
}
static void cap_buf_write(u32 id, const void *data, u64 bytes) {
    rb_begin();
    rb_u32(id);
    if (g_gen.active) {
        rb_u32(TRC_ENC_GEN); rb_u64(bytes);
        rb_u32(g_gen.dist); rb_u32(g_gen.dtype); rb_u64(g_gen.seed);
        rb_f32(g_gen.p0); rb_f32(g_gen.p1);
        g_gen.active = 0;
    } else {
        rb_u32(TRC_ENC_RAW); rb_u64(bytes);
        rb_bytes(data, bytes);
    }
    rb_emit(TRC_WRITE);
    if (data) g_orig.buf_write(id, data, bytes);
}
static void cap_buf_read(u32 id, void *out, u64 bytes) {
    g_orig.buf_read(id, out, bytes);
    rb_begin(); rb_u32(id); rb_u32(g_exec ? 1 : 0); rb_u64(bytes);
    if (g_exec) rb_bytes(out, bytes);
    rb_emit(TRC_READ);
}
static void cap_pool_reset(u32 keep) {
    rb_begin(); rb_u32(keep); rb_emit(TRC_RESET);
    g_orig.pool_reset(keep);
}

static void cap_dispatch_uop_kernel(u32 out_buf, const u32 *leaf_bufs, u32 n_leaves,
                                    const UOpKernel *k, u64 cache_key) {
    rb_begin();
    rb_u32(out_buf);
    rb_u32(n_leaves);
    for (u32 i = 0; i < n_leaves; i++) rb_u32(leaf_bufs[i]);
    rb_u64(cache_key);
    rb_u32(k->n_ops); rb_u32(k->n_bufs); rb_u32(k->rank);
    rb_shape(&k->full_shape);
    for (u32 i = 0; i < 3; i++) rb_u32(k->grid[i]);
    for (u32 i = 0; i < 3; i++) rb_u32(k->tg[i]);
    rb_u32(k->local_size); rb_u32(k->reduce_numel); rb_u32(k->out_dtype);
    for (u32 d = 0; d < MAX_DIM; d++) rb_u32(k->coord_uop[d]);
    for (u32 i = 0; i < k->n_ops; i++) {
        rb_u32((u32)k->ops[i].type);
        rb_u32(k->ops[i].arg[0]); rb_u32(k->ops[i].arg[1]); rb_u32(k->ops[i].arg[2]);
        rb_u32(k->ops[i].imm.u);
    }
    for (u32 i = 0; i < n_leaves; i++) rb_view(&k->leaf_views[i]);
    for (u32 i = 0; i < n_leaves; i++) rb_u32(k->leaf_dtypes[i]);
    rb_emit(TRC_UOP);
    if (g_exec) g_orig.dispatch_uop_kernel(out_buf, leaf_bufs, n_leaves, k, cache_key);
    rec_snapshot(out_buf);
}

static void cap_dispatch_kernel_rs(u32 out_buf, u32 *leaf_bufs, const View **leaf_views,
                                   const ShapeTracker *const *leaf_sts, u32 n_leaves,
                                   FusedOp *ops, u32 n_ops, const Shape *full_shape,
                                   const ReduceSpec *reduce, u32 *side_bufs,
                                   const u32 *side_idx, u32 n_side,
                                   const u32 *leaf_dtypes, u32 out_dtype) {
    rb_begin();
    rb_u32(out_buf);
    rb_u32(n_leaves);
    for (u32 i = 0; i < n_leaves; i++) rb_u32(leaf_bufs[i]);
    for (u32 i = 0; i < n_leaves; i++) rb_view(leaf_views[i]);
    for (u32 i = 0; i < n_leaves; i++)
        rb_u32(leaf_sts && leaf_sts[i] && leaf_sts[i]->n_views >= 1 ? 1 : 0);
    for (u32 i = 0; i < n_leaves; i++) {
        if (leaf_sts && leaf_sts[i] && leaf_sts[i]->n_views >= 1) {
            rb_u32(leaf_sts[i]->n_views);
            for (u32 v = 0; v < leaf_sts[i]->n_views; v++) rb_view(&leaf_sts[i]->views[v]);
        }
    }
    rb_u32(n_ops);
    for (u32 i = 0; i < n_ops; i++) {
        rb_u32(ops[i].uop); rb_u32(ops[i].arg_a); rb_u32(ops[i].arg_b); rb_u32(ops[i].aux);
    }
    rb_shape(full_shape);
    rb_u32(reduce ? 1 : 0);
    if (reduce) rb_reduce(reduce);
    rb_u32(n_side);
    for (u32 i = 0; i < n_side; i++) rb_u32(side_bufs[i]);
    for (u32 i = 0; i < n_side; i++) rb_u32(side_idx[i]);
    rb_u32(leaf_dtypes ? 1 : 0);
    if (leaf_dtypes) for (u32 i = 0; i < n_leaves; i++) rb_u32(leaf_dtypes[i]);
    rb_u32(out_dtype);
    rb_emit(TRC_RS);
    if (g_exec)
        g_orig.dispatch_kernel_rs(out_buf, leaf_bufs, leaf_views, leaf_sts, n_leaves, ops, n_ops,
                                  full_shape, reduce, side_bufs, side_idx, n_side,
                                  leaf_dtypes, out_dtype);
    rec_snapshot(out_buf);
}

static void cap_legacy_unary(u32 uop, u32 dst, const View *dv, u32 dd, u32 src,
                             const View *sv, u32 sd) {
    fprintf(stderr, "capture: legacy op_unary reached (uop %u)\n", uop);
    g_orig.op_unary(uop, dst, dv, dd, src, sv, sd);
}
static void cap_legacy_binary(u32 uop, u32 dst, const View *dv, u32 dd, u32 a, const View *av,
                              u32 ad, u32 b, const View *bv, u32 bd) {
    fprintf(stderr, "capture: legacy op_binary reached (uop %u)\n", uop);
    g_orig.op_binary(uop, dst, dv, dd, a, av, ad, b, bv, bd);
}
static void cap_legacy_mm(u32 dst, u32 dd, u32 a, const View *av, u32 ad, u32 b,
                          const View *bv, u32 bd, u32 M, u32 K, u32 N) {
    fprintf(stderr, "capture: legacy op_mm reached\n");
    g_orig.op_mm(dst, dd, a, av, ad, b, bv, bd, M, K, N);
}
static void cap_legacy_reduce(u32 uop, u32 dst, u32 dn, u32 dd, u32 src, u32 sn, u32 sd, u32 rd) {
    fprintf(stderr, "capture: legacy op_reduce reached (uop %u)\n", uop);
    g_orig.op_reduce(uop, dst, dn, dd, src, sn, sd, rd);
}

static void install_recorder(void) {
    g_orig = cpu_backend;
    cpu_backend.init = cap_init;
    cpu_backend.shutdown = cap_shutdown;
    cpu_backend.buf_alloc = cap_buf_alloc;
    cpu_backend.buf_free = cap_buf_free;
    cpu_backend.buf_write = cap_buf_write;
    cpu_backend.buf_read = cap_buf_read;
    cpu_backend.pool_reset = cap_pool_reset;
    cpu_backend.dispatch_uop_kernel = cap_dispatch_uop_kernel;
    cpu_backend.dispatch_kernel_rs = cap_dispatch_kernel_rs;
    cpu_backend.op_unary = cap_legacy_unary;
    cpu_backend.op_binary = cap_legacy_binary;
    cpu_backend.op_mm = cap_legacy_mm;
    cpu_backend.op_reduce = cap_legacy_reduce;
}

/* ---- workload helpers ---- */

/* A tensor whose contents come from the shared generator. In exec mode the
 * data is generated and written; the WRITE record carries only the spec. */
static Term gen_tensor(TinyHVM *ctx, Shape s, u32 dtype, u32 dist, u64 seed, f32 p0, f32 p1) {
    u64 n = 1;
    for (u32 d = 0; d < s.rank; d++) n *= s.dims[d];
    void *data = NULL;
    if (g_exec) {
        data = malloc(n * 4);
        thvm_gen_fill(data, dtype, dist, seed, p0, p1, 0, n);
    }
    g_gen.active = 1; g_gen.dist = dist; g_gen.dtype = dtype; g_gen.seed = seed;
    g_gen.p0 = p0; g_gen.p1 = p1;
    Term t;
    if (data) {
        t = thvm_tensor_typed(ctx, data, s, dtype);
    } else {
        t = thvm_tensor_typed(ctx, NULL, s, dtype);
        u32 id = (u32)term_val(t);
        cap_buf_write(ctx->tensors[id].buf_id, NULL, n * dtype_size(dtype));
    }
    g_gen.active = 0;
    free(data);
    return t;
}

static Term unary(TinyHVM *ctx, u32 uop, Term a) { return thvm_op(ctx, uop, a, term_era()); }
static Term binary(TinyHVM *ctx, u32 uop, Term a, Term b) { return thvm_op(ctx, uop, a, b); }

static Term realize(TinyHVM *ctx, Term t) { return thvm_eval(ctx, t); }

static void readback(TinyHVM *ctx, Term t) {
    f32 *h = thvm_to_host(ctx, t);
    (void)h;
}

/* ---- workloads ---- */

/* Fused elementwise+reduce: y = sum(relu(a*b + c), axis=-1), a/b/c ~ N(0,1).
 * Backward with the implicit ones cotangent: dA = (a*b + c > 0) * b. */
static void wl_fused(TinyHVM *ctx, u32 R, u32 C, int fwd, int bwd) {
    Term a = gen_tensor(ctx, SHAPE(R, C), DTYPE_F32, TRC_GEN_NORMAL, 2001, 0.f, 1.f);
    Term b = gen_tensor(ctx, SHAPE(R, C), DTYPE_F32, TRC_GEN_NORMAL, 2002, 0.f, 1.f);
    Term c = gen_tensor(ctx, SHAPE(R, C), DTYPE_F32, TRC_GEN_NORMAL, 2003, 0.f, 1.f);
    if (fwd) {
        rec_mark("fused.fwd");
        Term pre = binary(ctx, UOP_ADD, binary(ctx, UOP_MUL, a, b), c);
        Term y = thvm_sum_axes(ctx, unary(ctx, UOP_RELU, pre), (u32[]){1}, 1);
        y = realize(ctx, y);
        readback(ctx, y);
    }
    if (bwd) {
        rec_mark("fused.bwd");
        Term pre = binary(ctx, UOP_ADD, binary(ctx, UOP_MUL, a, b), c);
        Term mask = binary(ctx, UOP_CMP, pre, term_num_f32(0.0f));
        Term da = binary(ctx, UOP_MUL, mask, b);
        da = realize(ctx, da);
        readback(ctx, da);
    }
}

int main(int argc, char **argv) {
    int ai = 1;
    if (ai < argc && strcmp(argv[ai], "-n") == 0) { g_exec = 0; ai++; }
    if (argc - ai < 2) {
        fprintf(stderr, "usage: capture [-n] <workload> <out.trc> [sizes...]\n");
        return 2;
    }
    const char *wl = argv[ai];
    const char *path = argv[ai + 1];
    u32 sz[8] = {0};
    u32 nsz = 0;
    for (int i = ai + 2; i < argc && nsz < 8; i++) sz[nsz++] = (u32)strtoul(argv[i], NULL, 10);

    g_out = fopen(path, "wb");
    if (!g_out) { perror(path); return 1; }
    fwrite(THVM_TRACE_MAGIC, 1, 8, g_out);
    install_recorder();
    TinyHVM *ctx = thvm_init("cpu");
    char note[256];
    snprintf(note, sizeof note, "workload=%s exec=%d", wl, g_exec);
    rec_mark(note);

    if (strcmp(wl, "fused") == 0) {
        wl_fused(ctx, nsz > 0 ? sz[0] : 64, nsz > 1 ? sz[1] : 256, 1, 1);
    } else if (strcmp(wl, "fused_fwd") == 0) {
        wl_fused(ctx, nsz > 0 ? sz[0] : 64, nsz > 1 ? sz[1] : 256, 1, 0);
    } else if (strcmp(wl, "fused_bwd") == 0) {
        wl_fused(ctx, nsz > 0 ? sz[0] : 64, nsz > 1 ? sz[1] : 256, 0, 1);
    } else {
        fprintf(stderr, "unknown workload %s\n", wl);
        return 2;
    }
    fclose(g_out);
    return 0;
}
