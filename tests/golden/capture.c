/*
 * capture.c - records the Backend calls that the TinyHVM engine makes for
 * each benchmark workload, as kernel traces (include/thvm_trace.h).
 *
 * Built only in the development container, from the engine sources where
 * they lie (oracle/Makefile, target `ref`): this file includes src/tinyhvm.c and the
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
#include "nn/_.c"
#include "backend/cpu/_.c"
#include "thvm_trace.h"
#include "thvm_gen.h"

#include <sys/mman.h>

/* The oracle (oracle/oracle.c, compiled separately against the same layouts). */
extern u64 ora_oob_loads;
void ora_dispatch_rs(void *out, u64 out_bytes, const void **leaf, const u64 *leaf_bytes, const View **views,
                     const ShapeTracker *const *sts, u32 n_leaves, const FusedOp *ops, u32 n_ops,
                     const Shape *full, const ReduceSpec *reduce, const u32 *leaf_dtypes, u32 out_dtype);
void ora_dispatch_uop(void *out, u64 out_bytes, const void **leaf, const u64 *leaf_bytes, u32 n_leaves,
                      const UOpKernel *k);

static FILE *g_out;
static int g_exec = 1;
static int g_read_data = 0;   /* -r: keep READ payloads (the SNAPSHOTs already hold them) */
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

/* Called with each mark's text before it is recorded (a timing driver sets
 * it to time the steps between marks). */
static void (*g_mark_hook)(const char *text);

static void rec_mark(const char *text) {
    if (g_mark_hook) g_mark_hook(text);
    rb_begin();
    u32 n = (u32)strlen(text);
    rb_u32(n);
    rb_bytes(text, n);
    rb_emit(TRC_MARK);
}

/* Source of a SNAPSHOT: 0 = the engine's CPU backend; 2 = the engine's CPU
 * backend run over zero-guarded leaves (below), for kernels whose masked loads
 * fall outside their buffer; 1 = the oracle, only if the guarded run is not
 * possible (the mapping fails). */
static u32 g_snap_source;

/* The engine's interpreter loads a leaf element before applying the mask that
 * discards it (src/backend/cpu/uop.c:55-72), so a zero-padded view reads
 * outside its buffer at the masked positions (u32 index arithmetic wraps a
 * negative pad offset to a large index) and faults. Such a kernel is run by the
 * engine itself with every leaf copied to the start of a lazily mapped,
 * zero-filled region that spans every u32 element index of a 4-byte type: the
 * stray loads read zeros, the masks discard them, and the output is the
 * engine's own. */
#define GUARD_SPAN (((u64)1 << 34) + 65536)

typedef struct { u32 id; void *saved; void *guard; } Guarded;

static u32 guard_leaves(const u32 *leaf_bufs, u32 n_leaves, Guarded *g) {
    u32 ng = 0;
    for (u32 i = 0; i < n_leaves; i++) {
        u32 id = leaf_bufs[i];
        if (!id || id >= MAX_BUFS || !cpu_pool.bufs[id]) continue;
        int seen = 0;
        for (u32 j = 0; j < ng; j++) seen |= g[j].id == id;
        if (seen) continue;
        void *m = mmap(NULL, GUARD_SPAN, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE,
                       -1, 0);
        if (m == MAP_FAILED) {
            for (u32 j = 0; j < ng; j++) {
                cpu_pool.bufs[g[j].id] = g[j].saved;
                munmap(g[j].guard, GUARD_SPAN);
            }
            return (u32)-1;
        }
        memcpy(m, cpu_pool.bufs[id], cpu_pool.sizes[id]);
        g[ng].id = id;
        g[ng].saved = cpu_pool.bufs[id];
        g[ng].guard = m;
        cpu_pool.bufs[id] = m;
        ng++;
    }
    return ng;
}

static void unguard_leaves(Guarded *g, u32 ng, u32 out_buf) {
    for (u32 j = 0; j < ng; j++) {
        if (g[j].id == out_buf) memcpy(g[j].saved, g[j].guard, cpu_pool.sizes[out_buf]);
        cpu_pool.bufs[g[j].id] = g[j].saved;
        munmap(g[j].guard, GUARD_SPAN);
    }
}

static void rec_snapshot(u32 id) {
    if (!g_exec || id == 0 || id >= MAX_BUFS || !cpu_pool.bufs[id]) return;
    rb_begin();
    rb_u32(id);
    rb_u32(g_snap_source);
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
    int keep = g_exec && g_read_data;
    rb_begin(); rb_u32(id); rb_u32(keep ? 1 : 0); rb_u64(bytes);
    if (keep) rb_bytes(out, bytes);
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
    g_snap_source = 0;
    if (g_exec) {
        /* dry run through the oracle into a scratch copy to see whether any
         * load leaves its buffer */
        const void *lp[FUSE_MAX_LEAVES];
        u64 lb[FUSE_MAX_LEAVES];
        for (u32 i = 0; i < n_leaves && i < FUSE_MAX_LEAVES; i++) {
            lp[i] = cpu_pool.bufs[leaf_bufs[i]];
            lb[i] = cpu_pool.bufs[leaf_bufs[i]] ? cpu_pool.sizes[leaf_bufs[i]] : 0;
        }
        u64 ob = cpu_pool.sizes[out_buf];
        void *scratch = malloc(ob ? ob : 4);
        memcpy(scratch, cpu_pool.bufs[out_buf], ob);
        ora_oob_loads = 0;
        ora_dispatch_uop(scratch, ob, lp, lb, n_leaves, k);
        if (ora_oob_loads) {
            Guarded g[FUSE_MAX_LEAVES];
            u32 ng = guard_leaves(leaf_bufs, n_leaves, g);
            if (ng == (u32)-1) {
                memcpy(cpu_pool.bufs[out_buf], scratch, ob);
                g_snap_source = 1;
            } else {
                g_orig.dispatch_uop_kernel(out_buf, leaf_bufs, n_leaves, k, cache_key);
                unguard_leaves(g, ng, out_buf);
                g_snap_source = 2;
                if (memcmp(cpu_pool.bufs[out_buf], scratch, ob) != 0)
                    fprintf(stderr, "capture: oracle differs from the engine on a guarded kernel\n");
            }
        } else {
            g_orig.dispatch_uop_kernel(out_buf, leaf_bufs, n_leaves, k, cache_key);
        }
        free(scratch);
    }
    rec_snapshot(out_buf);
    g_snap_source = 0;
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
    g_snap_source = 0;
    if (g_exec) {
        const void *lp[FUSE_MAX_LEAVES];
        u64 lb[FUSE_MAX_LEAVES];
        for (u32 i = 0; i < n_leaves && i < FUSE_MAX_LEAVES; i++) {
            lp[i] = cpu_pool.bufs[leaf_bufs[i]];
            lb[i] = cpu_pool.bufs[leaf_bufs[i]] ? cpu_pool.sizes[leaf_bufs[i]] : 0;
        }
        u64 ob = cpu_pool.sizes[out_buf];
        void *scratch = malloc(ob ? ob : 4);
        memcpy(scratch, cpu_pool.bufs[out_buf], ob);
        ora_oob_loads = 0;
        ora_dispatch_rs(scratch, ob, lp, lb, leaf_views, leaf_sts, n_leaves, ops, n_ops, full_shape, reduce,
                        leaf_dtypes, out_dtype);
        Guarded g[FUSE_MAX_LEAVES];
        u32 ng = ora_oob_loads ? guard_leaves(leaf_bufs, n_leaves, g) : 0;
        if (ng == (u32)-1) {
            memcpy(cpu_pool.bufs[out_buf], scratch, ob);
            g_snap_source = 1;
        } else {
            g_orig.dispatch_kernel_rs(out_buf, leaf_bufs, leaf_views, leaf_sts, n_leaves, ops, n_ops,
                                      full_shape, reduce, side_bufs, side_idx, n_side,
                                      leaf_dtypes, out_dtype);
            if (ora_oob_loads) {
                unguard_leaves(g, ng, out_buf);
                g_snap_source = 2;
                if (memcmp(cpu_pool.bufs[out_buf], scratch, ob) != 0)
                    fprintf(stderr, "capture: oracle differs from the engine on a guarded kernel\n");
            }
        }
        free(scratch);
    }
    rec_snapshot(out_buf);
    g_snap_source = 0;
}

/* The legacy per-op slots (src/tinyhvm.h:1004-1016), reached only from the
 * engine's ENSURE/materialize path (src/fuse/materialize.c:195,672,683,700):
 * recorded, run on the engine's CPU backend (src/backend/cpu/ops.c), and
 * followed by a SNAPSHOT of the destination. */
static void cap_legacy_unary(u32 uop, u32 dst, const View *dv, u32 dd, u32 src,
                             const View *sv, u32 sd) {
    rb_begin();
    rb_u32(uop); rb_u32(dst); rb_u32(dd); rb_view(dv); rb_u32(src); rb_u32(sd); rb_view(sv);
    rb_emit(TRC_OPUN);
    if (g_exec) g_orig.op_unary(uop, dst, dv, dd, src, sv, sd);
    rec_snapshot(dst);
}
static void cap_legacy_binary(u32 uop, u32 dst, const View *dv, u32 dd, u32 a, const View *av,
                              u32 ad, u32 b, const View *bv, u32 bd) {
    rb_begin();
    rb_u32(uop); rb_u32(dst); rb_u32(dd); rb_view(dv);
    rb_u32(a); rb_u32(ad); rb_view(av); rb_u32(b); rb_u32(bd); rb_view(bv);
    rb_emit(TRC_OPBIN);
    if (g_exec) g_orig.op_binary(uop, dst, dv, dd, a, av, ad, b, bv, bd);
    rec_snapshot(dst);
}
static void cap_legacy_mm(u32 dst, u32 dd, u32 a, const View *av, u32 ad, u32 b,
                          const View *bv, u32 bd, u32 M, u32 K, u32 N) {
    rb_begin();
    rb_u32(dst); rb_u32(dd); rb_u32(a); rb_u32(ad); rb_view(av); rb_u32(b); rb_u32(bd); rb_view(bv);
    rb_u32(M); rb_u32(K); rb_u32(N);
    rb_emit(TRC_OPMM);
    if (g_exec) g_orig.op_mm(dst, dd, a, av, ad, b, bv, bd, M, K, N);
    rec_snapshot(dst);
}
static void cap_legacy_reduce(u32 uop, u32 dst, u32 dn, u32 dd, u32 src, u32 sn, u32 sd, u32 rd) {
    rb_begin();
    rb_u32(uop); rb_u32(dst); rb_u32(dn); rb_u32(dd); rb_u32(src); rb_u32(sn); rb_u32(sd); rb_u32(rd);
    rb_emit(TRC_OPRED);
    if (g_exec) g_orig.op_reduce(uop, dst, dn, dd, src, sn, sd, rd);
    rec_snapshot(dst);
}

/* The engine's CPU backend has no buf_copy/contiguify, so ASSIGN would fall
 * back to a host round trip (src/interact/tensor_ops.c:113-137). Giving the
 * recorded backend both slots makes the engine take the device-copy path a
 * GPU backend gets. */
static void cap_buf_copy(u32 dst, u32 src, u64 nbytes) {
    rb_begin(); rb_u32(dst); rb_u32(src); rb_u64(nbytes); rb_emit(TRC_COPY);
    if (cpu_pool.bufs[dst] && cpu_pool.bufs[src]) {
        u64 n = nbytes;
        if (n > cpu_pool.sizes[dst]) n = cpu_pool.sizes[dst];
        if (n > cpu_pool.sizes[src]) n = cpu_pool.sizes[src];
        memmove(cpu_pool.bufs[dst], cpu_pool.bufs[src], n);
    }
    rec_snapshot(dst);
}
/* contiguify's golden output. The engine's CPU backend has no contiguify
 * slot; without one, ASSIGN reads the source view to the host
 * (thvm_to_host_raw, src/ops/_.c:304-359) and writes the result back
 * (src/interact/tensor_ops.c:121-136). The assign workload runs each case that
 * way first and keeps the engine's result here; the recorded contiguify call
 * of the same case then produces exactly those bytes (SNAPSHOT source 0). */
static u8 *g_contig_expect;
static u64 g_contig_expect_n;

static void cap_contiguify(u32 dst, u32 numel, u32 src, const View *v) {
    rb_begin(); rb_u32(dst); rb_u32(numel); rb_u32(src); rb_view(v); rb_emit(TRC_CONTIG);
    (void)src;
    if (g_exec && cpu_pool.bufs[dst]) {
        if (!g_contig_expect || g_contig_expect_n != cpu_pool.sizes[dst]) {
            fprintf(stderr, "capture: contiguify outside the assign workload has no golden output\n");
            exit(1);
        }
        memcpy(cpu_pool.bufs[dst], g_contig_expect, g_contig_expect_n);
    }
    (void)numel;
    rec_snapshot(dst);
}

/* adam_step's golden output. The engine's CPU backend has no adam_step slot;
 * without one the engine updates through its lazy composition
 * (src/nn/adam.c:52-95). The adam workload runs each step that way first and
 * keeps the engine's results; the recorded adam_step call of the same step,
 * on copies of the same parameter and moments, then produces exactly those
 * bytes (SNAPSHOT source 0). */
static void rec_adam(u32 p, u32 g, u32 m, u32 v, f32 lr, f32 b1, f32 b2, f32 eps, f32 bc1, f32 bc2, u32 n,
                     u32 p_want, u32 m_want, u32 v_want) {
    rb_begin();
    rb_u32(p); rb_u32(g); rb_u32(m); rb_u32(v);
    rb_f32(lr); rb_f32(b1); rb_f32(b2); rb_f32(eps); rb_f32(bc1); rb_f32(bc2);
    rb_u32(n);
    rb_emit(TRC_ADAM);
    if (!g_exec) return;
    const u32 dst[3] = {p, m, v}, src[3] = {p_want, m_want, v_want};
    for (int i = 0; i < 3; i++) {
        /* only where the ids are the CPU backend's (not when the workload
         * runs on another backend, as tests/live/engine_live.c does) */
        if (dst[i] >= MAX_BUFS || src[i] >= MAX_BUFS || !cpu_pool.bufs[dst[i]] || !cpu_pool.bufs[src[i]] ||
            cpu_pool.sizes[dst[i]] < (u64)n * 4 || cpu_pool.sizes[src[i]] < (u64)n * 4)
            continue;
        memcpy(cpu_pool.bufs[dst[i]], cpu_pool.bufs[src[i]], (u64)n * 4);
        rec_snapshot(dst[i]);
    }
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
    cpu_backend.buf_copy = cap_buf_copy;
    cpu_backend.contiguify = cap_contiguify;
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

static Term realize(TinyHVM *ctx, Term t) {
    Term r = thvm_eval(ctx, t);
    if (getenv("CAP_DEBUG")) {
        const View *v = term_view(ctx, r);
        fprintf(stderr, "realize -> tag %u shape [", term_tag(r));
        for (u32 d = 0; v && d < v->shape.rank; d++) fprintf(stderr, "%u%s", v->shape.dims[d], d + 1 < v->shape.rank ? "," : "");
        fprintf(stderr, "]\n");
    }
    return r;
}

/* An eager view alias of a realized tensor with another shape (no kernel). */
static Term alias_as(TinyHVM *ctx, Term r, Shape s) {
    u8 saved = ctx->no_grad_alloc;
    ctx->no_grad_alloc = 0;
    Term a = thvm_reshape(ctx, r, s);
    ctx->no_grad_alloc = saved;
    return a;
}

/* Realize, then view the result with the intended shape. On this engine
 * snapshot thvm_eval can return a reduce kernel's raw output ([M,1,N] for a
 * matmul) without the trailing reshape, which later broadcasts wrongly. */
static Term realize_as(TinyHVM *ctx, Term t, Shape s) {
    Term r = realize(ctx, t);
    const View *v = term_view(ctx, r);
    int same = v && v->shape.rank == s.rank;
    for (u32 d = 0; same && d < s.rank; d++) same = v->shape.dims[d] == s.dims[d];
    if (same) return r;
    /* an eager view alias of the realized buffer (src/ctx/init.c:626-653):
     * a real tensor with the intended shape, no kernel */
    u8 saved = ctx->no_grad_alloc;
    ctx->no_grad_alloc = 0;
    Term a = thvm_reshape(ctx, r, s);
    ctx->no_grad_alloc = saved;
    return a;
}

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

/* Dense matmul + bias + relu (linear_forward, src/nn/tensor_api.c:93-97 via
 * thvm_tg_linear, src/nn/tg_tensor.c:34-66): y = relu(X @ W + b), X [M,K],
 * W [K,N], b [N], all U(-1,1). Backward with the ones cotangent on y:
 * G = (y > 0), dX = G @ W^T, dW = X^T @ G (transposes are permute views). */
static void wl_linear(TinyHVM *ctx, u32 M, u32 K, u32 N, int bwd) {
    Term X = gen_tensor(ctx, SHAPE(M, K), DTYPE_F32, TRC_GEN_UNIFORM, 3001, -1.f, 1.f);
    Term W = gen_tensor(ctx, SHAPE(K, N), DTYPE_F32, TRC_GEN_UNIFORM, 3002, -1.f, 1.f);
    Term b = gen_tensor(ctx, SHAPE(N), DTYPE_F32, TRC_GEN_UNIFORM, 3003, -1.f, 1.f);
    rec_mark("linear.fwd");
    Term y = unary(ctx, UOP_RELU, thvm_tg_linear(ctx, X, W, &b));
    y = realize(ctx, y);
    readback(ctx, y);
    if (!bwd) return;
    rec_mark("linear.bwd.dx");
    Term G = binary(ctx, UOP_CMP, y, term_num_f32(0.0f));
    Term dX = thvm_mm(ctx, G, thvm_permute(ctx, W, (u32[]){1, 0}, 2));
    dX = realize(ctx, dX);
    readback(ctx, dX);
    rec_mark("linear.bwd.dw");
    Term G2 = binary(ctx, UOP_CMP, y, term_num_f32(0.0f));
    Term dW = thvm_mm(ctx, thvm_permute(ctx, X, (u32[]){1, 0}, 2), G2);
    dW = realize(ctx, dW);
    readback(ctx, dW);
}

/* ---- shared pieces of the network workloads ---- */

/* Kaiming-uniform U(-sqrt(6/fan_in), +sqrt(6/fan_in)). */
static Term kaiming_u(TinyHVM *ctx, Shape s, u32 fan_in, u64 seed) {
    f32 bound = sqrtf(6.0f / (f32)fan_in);
    return gen_tensor(ctx, s, DTYPE_F32, TRC_GEN_UNIFORM, seed, -bound, bound);
}
static Term zeros(TinyHVM *ctx, Shape s, u64 seed) {
    return gen_tensor(ctx, s, DTYPE_F32, TRC_GEN_CONST, seed, 0.f, 0.f);
}
static u8 *labels_u8(u32 B, u64 seed) {
    u8 *lab = malloc(B);
    for (u32 i = 0; i < B; i++) lab[i] = (u8)thvm_gen_i32(TRC_GEN_INT, seed, i, 0.f, 10.f);
    return lab;
}
static Term onehot_tensor(TinyHVM *ctx, const u8 *lab, u32 B, u32 C) {
    f32 *oh = calloc((size_t)B * C, sizeof(f32));
    for (u32 i = 0; i < B; i++) oh[i * C + lab[i]] = 1.0f;
    Term t = thvm_tensor(ctx, oh, SHAPE(B, C));
    free(oh);
    return t;
}
static Term scalar_t(TinyHVM *ctx, f32 v) { return term_num_f32(v); }

/* x [B,in] @ W [in,out] + b, then optional relu; realized. */
static Term dense(TinyHVM *ctx, Term x, Term W, Term b, int relu, u32 B, u32 out) {
    /* thvm_tg_linear's composition (src/nn/tg_tensor.c:56-66): mm, then the
     * bias reshaped to [1,N] and expanded to [B,N]; it needs realized inputs
     * to read shapes, so it is spelled out here for view inputs. */
    Term y = thvm_mm(ctx, x, W);
    y = binary(ctx, UOP_ADD, y, thvm_expand(ctx, thvm_reshape(ctx, b, SHAPE(1, out)), SHAPE(B, out)));
    if (relu) y = unary(ctx, UOP_RELU, y);
    return realize_as(ctx, y, SHAPE(B, out));
}

/* sum over axis 0 of [B,N] -> [N] */
static Term colsum(TinyHVM *ctx, Term g, u32 N) {
    return realize_as(ctx, thvm_sum_axes(ctx, g, (u32[]){0}, 1), SHAPE(N));
}

/* a [M,K] @ b [K,N], realized as [M,N] */
static Term mm_as(TinyHVM *ctx, Term a, Term b, u32 M, u32 N) {
    return realize_as(ctx, thvm_mm(ctx, a, b), SHAPE(M, N));
}

/* Backward of y = act(x @ W + b) for the ones-free chain: given dz (the grad
 * of the pre-activation), dW = x^T @ dz, db = colsum(dz), dx = dz @ W^T. */
typedef struct { Term dW, db, dx; } DenseGrads;
static DenseGrads dense_bwd(TinyHVM *ctx, Term x, Term W, Term dz, u32 B, u32 in, u32 out, int need_dx) {
    DenseGrads g;
    g.dW = mm_as(ctx, thvm_permute(ctx, x, (u32[]){1, 0}, 2), dz, in, out);
    g.db = colsum(ctx, dz, out);
    g.dx = need_dx ? mm_as(ctx, dz, thvm_permute(ctx, W, (u32[]){1, 0}, 2), B, in) : term_era();
    return g;
}

/* softmax(logits) as src/nn/softmax.c:3-23 composes it (row max, subtract,
 * exp, row sum, divide), on realized tensors so no DUP is needed. */
static Term softmax_rows(TinyHVM *ctx, Term logits, u32 B, u32 C) {
    Term m = realize_as(ctx, thvm_rmax_axes(ctx, logits, (u32[]){1}, 1), SHAPE(B, 1));
    Term e = realize_as(ctx, unary(ctx, UOP_EXP, binary(ctx, UOP_SUB, logits, thvm_expand(ctx, m, SHAPE(B, C)))),
                        SHAPE(B, C));
    Term ssum = realize_as(ctx, thvm_sum_axes(ctx, e, (u32[]){1}, 1), SHAPE(B, 1));
    return realize_as(ctx, binary(ctx, UOP_DIV, e, thvm_expand(ctx, ssum, SHAPE(B, C))), SHAPE(B, C));
}

/* softmax cross-entropy gradient: (softmax(logits) - onehot) / B */
static Term ce_grad(TinyHVM *ctx, Term logits, Term onehot, u32 B, u32 C) {
    Term p = softmax_rows(ctx, logits, B, C);
    Term d = binary(ctx, UOP_SUB, p, onehot);
    return realize_as(ctx, binary(ctx, UOP_MUL, d, scalar_t(ctx, 1.0f / (f32)B)), SHAPE(B, C));
}

/* Zero padding of the two spatial dims of [B,C,H,W] by p, realized on its
 * own. The engine lowers a lone pad view with its mask; composed with the
 * conv's pool view (src/nn/conv.c:390-481) the mask is lost and the kernel
 * reads the neighbouring rows at the borders and runs off the buffer at the
 * ends, so the workloads pad explicitly and convolve without padding. */
static Term pad_exact(TinyHVM *ctx, Term x, u32 B, u32 C, u32 H, u32 W, u32 p) {
    /* times 1 (exact): a bare view would be folded into its consumer */
    Term t = binary(ctx, UOP_MUL, thvm_pad(ctx, x, (u32[]){0, 0, 0, 0, p, p, p, p}, 4), scalar_t(ctx, 1.0f));
    return realize_as(ctx, t, shape_of((u32[]){B, C, H + 2 * p, W + 2 * p}, 4));
}

/* Max-pool 2x2 backward with the engine's routing rule (every tied maximum
 * receives the gradient, src/interact/grad.c:405-425) fused with the relu
 * mask of the pooled activation a: dz = up(dp) * (1 - (up(pool) > a)) * (a > 0).
 * Computed in the 6-D layout [B,C,H/2,2,W/2,2] (the same memory order as
 * [B,C,H,W]) where the upsample is a plain stride-0 expand: a reshape of the
 * expanded [B,C,H/2,2,W/2,2] back to [B,C,H,W] is not a strided view and the
 * engine lowers it as a dense [B,C,H,W] read of the small tensor. */
static Term pool_relu_bwd(TinyHVM *ctx, Term dp, Term pooled, Term a, u32 B, u32 C, u32 H, u32 W) {
    Shape s6 = shape_of((u32[]){B, C, H / 2, 2, W / 2, 2}, 6);
    Shape s1 = shape_of((u32[]){B, C, H / 2, 1, W / 2, 1}, 6);
    Term pu = thvm_expand(ctx, thvm_reshape(ctx, pooled, s1), s6);
    Term du = thvm_expand(ctx, thvm_reshape(ctx, dp, s1), s6);
    Term routed = binary(ctx, UOP_SUB, scalar_t(ctx, 1.0f),
                         binary(ctx, UOP_CMP, pu, thvm_reshape(ctx, a, s6)));
    Term g = binary(ctx, UOP_MUL, du, routed);
    g = binary(ctx, UOP_MUL, g, binary(ctx, UOP_CMP, thvm_reshape(ctx, a, s6), scalar_t(ctx, 0.0f)));
    return realize_as(ctx, g, shape_of((u32[]){B, C, H, W}, 4));
}

/* Max-pool 2x2 backward without a relu mask: dx = up(dp) * (1 - (up(pool) > x)),
 * the engine's routing rule on any activation (negative and zero ties too). */
static Term pool_bwd(TinyHVM *ctx, Term dp, Term pooled, Term a, u32 B, u32 C, u32 H, u32 W) {
    Shape s6 = shape_of((u32[]){B, C, H / 2, 2, W / 2, 2}, 6);
    Shape s1 = shape_of((u32[]){B, C, H / 2, 1, W / 2, 1}, 6);
    Term pu = thvm_expand(ctx, thvm_reshape(ctx, pooled, s1), s6);
    Term du = thvm_expand(ctx, thvm_reshape(ctx, dp, s1), s6);
    Term routed = binary(ctx, UOP_SUB, scalar_t(ctx, 1.0f),
                         binary(ctx, UOP_CMP, pu, thvm_reshape(ctx, a, s6)));
    return realize_as(ctx, binary(ctx, UOP_MUL, du, routed), shape_of((u32[]){B, C, H, W}, 4));
}

/* Weight gradient of a stride-1 conv as one contraction:
 * dW[co,ci,kh,kw] = sum_{b,oy,ox} xp[b,ci,oy+kh,ox+kw] * dz[b,co,oy,ox],
 * with xp the already padded input (a pool view, src/nn/conv.c:20-388). */
static Term conv_dw(TinyHVM *ctx, Term xp, Term dz, u32 B, u32 Ci, u32 Co, u32 K, u32 OY, u32 OX) {
    Term P = thvm_pool(ctx, xp, (u32[]){K, K}, (u32[]){1, 1}, 2);          /* [B,Ci,OY,OX,K,K] */
    P = thvm_permute(ctx, P, (u32[]){1, 4, 5, 0, 2, 3}, 6);                  /* [Ci,K,K,B,OY,OX] */
    P = thvm_reshape(ctx, P, shape_of((u32[]){1, Ci, K, K, B, OY, OX}, 7));
    P = thvm_expand(ctx, P, shape_of((u32[]){Co, Ci, K, K, B, OY, OX}, 7));
    Term G = thvm_permute(ctx, dz, (u32[]){1, 0, 2, 3}, 4);                  /* [Co,B,OY,OX] */
    G = thvm_reshape(ctx, G, shape_of((u32[]){Co, 1, 1, 1, B, OY, OX}, 7));
    G = thvm_expand(ctx, G, shape_of((u32[]){Co, Ci, K, K, B, OY, OX}, 7));
    Term s = thvm_sum_axes(ctx, binary(ctx, UOP_MUL, P, G), (u32[]){4, 5, 6}, 3);
    return realize_as(ctx, s, shape_of((u32[]){Co, Ci, K, K}, 4));
}

/* The KxK spatial flip of W [Co,Ci,K,K] transposed to [Ci,Co,K,K]: an exact
 * matmul with the exchange matrix (the engine has no flip view). */
static Term flip_t(TinyHVM *ctx, Term W, u32 Co, u32 Ci, u32 K) {
    u32 KK = K * K;
    f32 *J = calloc((size_t)KK * KK, sizeof(f32));
    for (u32 p = 0; p < KK; p++) J[(KK - 1 - p) * KK + p] = 1.0f;
    Term Jt = thvm_tensor(ctx, J, SHAPE(KK, KK));
    free(J);
    Term Wf = mm_as(ctx, thvm_reshape(ctx, W, SHAPE(Co * Ci, KK)), Jt, Co * Ci, KK);
    Term Wt = thvm_permute(ctx, thvm_reshape(ctx, Wf, shape_of((u32[]){Co, Ci, K, K}, 4)),
                           (u32[]){1, 0, 2, 3}, 4);
    /* times 1 (exact) materializes the transpose, so the conv reads a dense kernel */
    return realize_as(ctx, binary(ctx, UOP_MUL, Wt, scalar_t(ctx, 1.0f)), shape_of((u32[]){Ci, Co, K, K}, 4));
}

/* Input gradient of a stride-1 conv with padding `pad`: the conv of dz with
 * the flipped, transposed kernel and padding K-1-pad. */
static Term conv_dx(TinyHVM *ctx, Term dz, Term W, u32 B, u32 Co, u32 Ci, u32 K, u32 pad, u32 H, u32 W_) {
    Term Wt = flip_t(ctx, W, Co, Ci, K);
    u32 p = K - 1 - pad;
    Term dzp = pad_exact(ctx, dz, B, Co, H + 2 * pad - K + 1, W_ + 2 * pad - K + 1, p);
    return realize_as(ctx, thvm_conv2d(ctx, dzp, Wt, term_era(), 1, (u32[]){1, 1}, (u32[]){0, 0, 0, 0}),
                      shape_of((u32[]){B, Ci, H, W_}, 4));
}

/* per-channel sum over [0,2,3] of [B,C,H,W] -> [C] */
static Term chansum(TinyHVM *ctx, Term g, u32 C) {
    return realize_as(ctx, thvm_sum_axes(ctx, g, (u32[]){0, 2, 3}, 3), SHAPE(C));
}

/* SGD through the engine's ASSIGN: p <- p - lr * g for every parameter. */
static void sgd(TinyHVM *ctx, Term *params, Term *grads, u32 n, f32 lr) {
    Term chain = term_era();
    for (u32 i = 0; i < n; i++) {
        Term upd = binary(ctx, UOP_SUB, params[i], binary(ctx, UOP_MUL, grads[i], scalar_t(ctx, lr)));
        Term a = thvm_assign(ctx, params[i], upd);
        chain = (i == 0) ? a : thvm_seq(ctx, chain, a);
    }
    thvm_eval(ctx, chain);
}

/* 2-layer MLP: x [B,784] ~ N(0,1), W1 [784,H], W2 [H,10] Kaiming-uniform, b = 0,
 * relu, softmax cross-entropy (src/nn/loss.c:8-44); outputs loss, dW1, dW2.
 * With steps > 1 the forward and backward repeat from the same inputs, each
 * step opened by an "mlp.step" mark and closed by a reset of the step's
 * tensors (one step records exactly as before). */
static void wl_mlp_steps(TinyHVM *ctx, u32 B, u32 IN, u32 H, u32 C, int steps);
static void wl_mlp(TinyHVM *ctx, u32 B, u32 IN, u32 H, u32 C) { wl_mlp_steps(ctx, B, IN, H, C, 1); }
static void wl_mlp_steps(TinyHVM *ctx, u32 B, u32 IN, u32 H, u32 C, int steps) {
    Term x = gen_tensor(ctx, SHAPE(B, IN), DTYPE_F32, TRC_GEN_NORMAL, 1001, 0.f, 1.f);
    Term W1 = kaiming_u(ctx, SHAPE(IN, H), IN, 1002);
    Term b1 = zeros(ctx, SHAPE(H), 1003);
    Term W2 = kaiming_u(ctx, SHAPE(H, C), H, 1004);
    Term b2 = zeros(ctx, SHAPE(C), 1005);
    u8 *lab = labels_u8(B, 1006);
    Term onehot = onehot_tensor(ctx, lab, B, C);
    u32 keep = ctx->tensor_count;
    for (int st = 0; st < steps; st++) {
        if (steps > 1) rec_mark("mlp.step");
        rec_mark("mlp.fwd");
        Term h = dense(ctx, x, W1, b1, 1, B, H);
        Term logits = dense(ctx, h, W2, b2, 0, B, C);
        Term loss = realize(ctx, cross_entropy_loss(ctx, logits, lab, B, C));
        readback(ctx, loss);
        rec_mark("mlp.bwd");
        Term d2 = ce_grad(ctx, logits, onehot, B, C);
        DenseGrads g2 = dense_bwd(ctx, h, W2, d2, B, H, C, 1);
        Term dz1 = realize_as(ctx, binary(ctx, UOP_MUL, g2.dx, binary(ctx, UOP_CMP, h, scalar_t(ctx, 0.0f))),
                              SHAPE(B, H));
        DenseGrads g1 = dense_bwd(ctx, x, W1, dz1, B, IN, H, 0);
        readback(ctx, g1.dW);
        readback(ctx, g2.dW);
        if (steps > 1) thvm_reset(ctx, keep);
    }
    free(lab);
}

/* The engine's cross-entropy composition (src/nn/loss.c:8-44: the row max,
 * logsumexp, minus the label's logit, summed and scaled by 1/B) with the
 * one-hot labels read from a persistent tensor, where the engine's
 * cross_entropy_loss makes a new one-hot tensor from host labels at every
 * call: the form of a step that is captured once and replayed with new
 * labels written into the same tensor (as the engine's JIT test builds its
 * loss from a persistent one-hot, test/archive/test_jit_dense.m:47-60).
 * Intermediates used twice are realized (no DUP needed). [1,1]. */
static Term ce_loss_onehot(TinyHVM *ctx, Term logits, Term onehot, u32 B, u32 C) {
    Term mx = realize_as(ctx, thvm_rmax_axes(ctx, logits, (u32[]){1}, 1), SHAPE(B, 1));
    Term sh = binary(ctx, UOP_SUB, logits, thvm_expand(ctx, mx, SHAPE(B, C)));
    Term se = realize_as(ctx, thvm_sum_axes(ctx, unary(ctx, UOP_EXP, sh), (u32[]){1}, 1), SHAPE(B, 1));
    Term lse = binary(ctx, UOP_ADD, mx, unary(ctx, UOP_LOG, se));
    Term pick = thvm_sum_axes(ctx, binary(ctx, UOP_MUL, onehot, logits), (u32[]){1}, 1);
    Term row = binary(ctx, UOP_SUB, lse, pick);
    Term tot = thvm_sum_axes(ctx, row, (u32[]){0, 1}, 2);
    return realize_as(ctx, binary(ctx, UOP_MUL, tot, scalar_t(ctx, 1.0f / (f32)B)), SHAPE(1, 1));
}

/* SGD through the engine's ASSIGN, with the loss assigned to a persistent
 * tensor in the same evaluation (nothing read back). */
static void sgd_keep_loss(TinyHVM *ctx, Term *params, Term *grads, u32 n, f32 lr, Term loss_out, Term loss) {
    Term chain = thvm_assign(ctx, loss_out, loss);
    for (u32 i = 0; i < n; i++) {
        Term upd = binary(ctx, UOP_SUB, params[i], binary(ctx, UOP_MUL, grads[i], scalar_t(ctx, lr)));
        chain = thvm_seq(ctx, chain, thvm_assign(ctx, params[i], upd));
    }
    thvm_eval(ctx, chain);
}

/* One LeNet-5 training step on persistent tensors: forward, backward, SGD
 * (lr 0.01) through ASSIGN. With host labels `lab`, the loss is the
 * engine's cross_entropy_loss, realized and read back after the forward;
 * with lab NULL it is ce_loss_onehot over the persistent one-hot tensor and
 * is assigned to loss_out with the parameter updates, nothing being read:
 * the step a caller captures once and replays. */
static void lenet_step(TinyHVM *ctx, u32 B, Term x, Term *params, Term onehot, const u8 *lab, Term loss_out) {
    Term W1 = params[0], b1 = params[1], W2 = params[2], b2 = params[3], W3 = params[4], b3 = params[5];
    Term W4 = params[6], b4 = params[7], W5 = params[8], b5 = params[9];
    rec_mark("lenet.fwd");
    Term xp = pad_exact(ctx, x, B, 1, 28, 28, 2);
    Term a1 = realize_as(ctx, unary(ctx, UOP_RELU,
                         thvm_conv2d(ctx, xp, W1, b1, 1, (u32[]){1, 1}, (u32[]){0, 0, 0, 0})),
                         shape_of((u32[]){B, 6, 28, 28}, 4));
    Term p1 = realize_as(ctx, thvm_maxpool2d(ctx, a1, (u32[]){2, 2}, (u32[]){2, 2}),
                         shape_of((u32[]){B, 6, 14, 14}, 4));
    Term a2 = realize_as(ctx, unary(ctx, UOP_RELU,
                         thvm_conv2d(ctx, p1, W2, b2, 1, (u32[]){1, 1}, (u32[]){0, 0, 0, 0})),
                         shape_of((u32[]){B, 16, 10, 10}, 4));
    Term p2 = realize_as(ctx, thvm_maxpool2d(ctx, a2, (u32[]){2, 2}, (u32[]){2, 2}),
                         shape_of((u32[]){B, 16, 5, 5}, 4));
    Term f = alias_as(ctx, p2, SHAPE(B, 400));
    Term h3 = dense(ctx, f, W3, b3, 1, B, 120);
    Term h4 = dense(ctx, h3, W4, b4, 1, B, 84);
    Term logits = dense(ctx, h4, W5, b5, 0, B, 10);
    Term loss = term_era();
    if (lab) {
        loss = realize(ctx, cross_entropy_loss(ctx, logits, (u8 *)lab, B, 10));
        readback(ctx, loss);
    } else {
        loss = ce_loss_onehot(ctx, logits, onehot, B, 10);
    }
    rec_mark("lenet.bwd");
    Term d5 = ce_grad(ctx, logits, onehot, B, 10);
    DenseGrads g5 = dense_bwd(ctx, h4, W5, d5, B, 84, 10, 1);
    Term dz4 = realize_as(ctx, binary(ctx, UOP_MUL, g5.dx, binary(ctx, UOP_CMP, h4, scalar_t(ctx, 0.0f))),
                          SHAPE(B, 84));
    DenseGrads g4 = dense_bwd(ctx, h3, W4, dz4, B, 120, 84, 1);
    Term dz3 = realize_as(ctx, binary(ctx, UOP_MUL, g4.dx, binary(ctx, UOP_CMP, h3, scalar_t(ctx, 0.0f))),
                          SHAPE(B, 120));
    DenseGrads g3 = dense_bwd(ctx, f, W3, dz3, B, 400, 120, 1);
    Term dp2 = alias_as(ctx, g3.dx, shape_of((u32[]){B, 16, 5, 5}, 4));
    Term dz2 = pool_relu_bwd(ctx, dp2, p2, a2, B, 16, 10, 10);
    Term dW2 = conv_dw(ctx, p1, dz2, B, 6, 16, 5, 10, 10);
    Term db2 = chansum(ctx, dz2, 16);
    Term dp1 = conv_dx(ctx, dz2, W2, B, 16, 6, 5, 0, 14, 14);
    Term dz1 = pool_relu_bwd(ctx, dp1, p1, a1, B, 6, 28, 28);
    Term dW1 = conv_dw(ctx, xp, dz1, B, 1, 6, 5, 28, 28);
    Term db1 = chansum(ctx, dz1, 6);
    rec_mark("lenet.sgd");
    Term grads[10] = {dW1, db1, dW2, db2, g3.dW, g3.db, g4.dW, g4.db, g5.dW, g5.db};
    if (lab) sgd(ctx, params, grads, 10, 0.01f);
    else sgd_keep_loss(ctx, params, grads, 10, 0.01f, loss_out, loss);
}

/* LeNet-5's persistent tensors: x [B,1,28,28] ~ U(0,1), the ten parameters
 * (Kaiming-uniform weights, zero biases) in the order W1, b1, ..., W5, b5. */
static Term lenet_params(TinyHVM *ctx, u32 B, Term *params) {
    Term x = gen_tensor(ctx, shape_of((u32[]){B, 1, 28, 28}, 4), DTYPE_F32, TRC_GEN_UNIFORM, 4001, 0.f, 1.f);
    params[0] = kaiming_u(ctx, shape_of((u32[]){6, 1, 5, 5}, 4), 25, 4002);
    params[1] = zeros(ctx, SHAPE(6), 4003);
    params[2] = kaiming_u(ctx, shape_of((u32[]){16, 6, 5, 5}, 4), 150, 4004);
    params[3] = zeros(ctx, SHAPE(16), 4005);
    params[4] = kaiming_u(ctx, SHAPE(400, 120), 400, 4006);
    params[5] = zeros(ctx, SHAPE(120), 4007);
    params[6] = kaiming_u(ctx, SHAPE(120, 84), 120, 4008);
    params[7] = zeros(ctx, SHAPE(84), 4009);
    params[8] = kaiming_u(ctx, SHAPE(84, 10), 84, 4010);
    params[9] = zeros(ctx, SHAPE(10), 4011);
    return x;
}

/* LeNet-5 training step: x [B,1,28,28] ~ U(0,1); conv5x5 -> 6 (pad 2, so that
 * the flatten is 16*5*5 = 400), relu, maxpool 2, conv5x5 -> 16, relu,
 * maxpool 2, fc 400 -> 120 -> 84 -> 10, softmax cross-entropy; backward and
 * SGD (lr 0.01) through ASSIGN. */
static void wl_lenet(TinyHVM *ctx, u32 B, int steps) {
    Term params[10];
    Term x = lenet_params(ctx, B, params);
    u8 *lab = labels_u8(B, 4012);
    Term onehot = onehot_tensor(ctx, lab, B, 10);
    u32 keep = ctx->tensor_count;
    for (int st = 0; st < steps; st++) {
        rec_mark("lenet.step");
        lenet_step(ctx, B, x, params, onehot, lab, term_era());
        rec_mark("lenet.end");
        for (u32 i = 0; i < 10; i++) readback(ctx, params[i]);
        thvm_reset(ctx, keep);
    }
    free(lab);
}

/* Conv block: x [B,C,H,W] ~ N(0,1), conv3x3 C->C pad 1 (Kaiming-normal
 * N(0, 2/(9C))), batchnorm train mode (gamma 1, beta 0, eps 1e-5,
 * src/nn/batchnorm.c:35-87), relu, maxpool 2, loss = sum; backward dW and dX. */
static void wl_convblock(TinyHVM *ctx, u32 B, u32 C, u32 H) {
    u32 W_ = H;
    Term x = gen_tensor(ctx, shape_of((u32[]){B, C, H, W_}, 4), DTYPE_F32, TRC_GEN_NORMAL, 5001, 0.f, 1.f);
    Term Wc = gen_tensor(ctx, shape_of((u32[]){C, C, 3, 3}, 4), DTYPE_F32, TRC_GEN_NORMAL, 5002, 0.f,
                         sqrtf(2.0f / (f32)(9 * C)));
    Term gamma = gen_tensor(ctx, SHAPE(C), DTYPE_F32, TRC_GEN_CONST, 5003, 1.f, 1.f);
    Term beta = zeros(ctx, SHAPE(C), 5004);
    Term rmean = zeros(ctx, SHAPE(C), 5005);
    Term rvar = gen_tensor(ctx, SHAPE(C), DTYPE_F32, TRC_GEN_CONST, 5006, 1.f, 1.f);
    u32 N = B * H * W_;
    /* d loss / d p = 1: an input of the step, like the weights */
    Term ones = gen_tensor(ctx, shape_of((u32[]){B, C, H / 2, W_ / 2}, 4), DTYPE_F32, TRC_GEN_CONST, 5007, 1.f, 1.f);
    rec_mark("conv.fwd");
    Shape full = shape_of((u32[]){B, C, H, W_}, 4);
    Shape cshape = shape_of((u32[]){1, C, 1, 1}, 4);
    Term xp = pad_exact(ctx, x, B, C, H, W_, 1);
    Term c = realize_as(ctx, thvm_conv2d(ctx, xp, Wc, term_era(), 1, (u32[]){1, 1}, (u32[]){0, 0, 0, 0}), full);
    /* batchnorm, train mode, as src/nn/batchnorm.c:35-87 computes it (mean and
     * biased variance over [0,2,3], eps 1e-5, momentum 0.1, unbiased running
     * variance), on realized tensors: the engine's own variance composition
     * shares one lazy term on both sides of a MUL and does not terminate. */
    f32 inv_n = 1.0f / (f32)N;
    Term mean = realize_as(ctx, binary(ctx, UOP_MUL, thvm_sum_axes(ctx, c, (u32[]){0, 2, 3}, 3), scalar_t(ctx, inv_n)),
                           cshape);
    Term cen = realize_as(ctx, binary(ctx, UOP_SUB, c, thvm_expand(ctx, mean, full)), full);
    Term var = realize_as(ctx, binary(ctx, UOP_MUL, thvm_sum_axes(ctx, binary(ctx, UOP_MUL, cen, cen), (u32[]){0, 2, 3}, 3),
                                      scalar_t(ctx, inv_n)), cshape);
    Term invstd = realize_as(ctx, binary(ctx, UOP_DIV, scalar_t(ctx, 1.0f),
                                         unary(ctx, UOP_SQRT, binary(ctx, UOP_ADD, var, scalar_t(ctx, 1e-5f)))), cshape);
    Term g4 = thvm_expand(ctx, thvm_reshape(ctx, gamma, cshape), full);
    Term b4 = thvm_expand(ctx, thvm_reshape(ctx, beta, cshape), full);
    Term xhat = realize_as(ctx, binary(ctx, UOP_MUL, cen, thvm_expand(ctx, invstd, full)), full);
    Term yb = realize_as(ctx, binary(ctx, UOP_ADD, binary(ctx, UOP_MUL, xhat, g4), b4), full);
    {
        f32 mom = 0.1f, bessel = (f32)N / (f32)(N - 1);
        Term m1 = alias_as(ctx, mean, SHAPE(C));
        Term v1 = alias_as(ctx, var, SHAPE(C));
        Term nrm = binary(ctx, UOP_ADD, binary(ctx, UOP_MUL, rmean, scalar_t(ctx, 1.0f - mom)),
                          binary(ctx, UOP_MUL, m1, scalar_t(ctx, mom)));
        Term nrv = binary(ctx, UOP_ADD, binary(ctx, UOP_MUL, rvar, scalar_t(ctx, 1.0f - mom)),
                          binary(ctx, UOP_MUL, v1, scalar_t(ctx, mom * bessel)));
        thvm_eval(ctx, thvm_seq(ctx, thvm_assign(ctx, rmean, nrm), thvm_assign(ctx, rvar, nrv)));
    }
    Term a = realize_as(ctx, unary(ctx, UOP_RELU, yb), full);
    Term p = realize_as(ctx, thvm_maxpool2d(ctx, a, (u32[]){2, 2}, (u32[]){2, 2}),
                        shape_of((u32[]){B, C, H / 2, W_ / 2}, 4));
    Term loss = realize(ctx, thvm_sum_axes(ctx, p, (u32[]){0, 1, 2, 3}, 4));
    readback(ctx, loss);
    rec_mark("conv.bwd");
    /* pool + relu backward */
    Term dya = pool_relu_bwd(ctx, ones, p, a, B, C, H, W_);
    /* batchnorm backward (gamma = g):
     *   xhat = (c - mean) * invstd, dxhat = dy * g
     *   dc = invstd / N * (N * dxhat - sum(dxhat) - xhat * sum(dxhat * xhat)) */
    /* lazy terms are consumed by the eval that uses them: a fresh gamma view */
    Term g4b = thvm_expand(ctx, thvm_reshape(ctx, gamma, cshape), full);
    Term dxhat = realize_as(ctx, binary(ctx, UOP_MUL, dya, g4b), full);
    Term s1 = realize_as(ctx, thvm_sum_axes(ctx, dxhat, (u32[]){0, 2, 3}, 3), cshape);
    Term s2 = realize_as(ctx, thvm_sum_axes(ctx, binary(ctx, UOP_MUL, dxhat, xhat), (u32[]){0, 2, 3}, 3), cshape);
    Term t = binary(ctx, UOP_SUB, binary(ctx, UOP_MUL, dxhat, scalar_t(ctx, (f32)N)), thvm_expand(ctx, s1, full));
    t = binary(ctx, UOP_SUB, t, binary(ctx, UOP_MUL, xhat, thvm_expand(ctx, s2, full)));
    Term dc = realize_as(ctx, binary(ctx, UOP_MUL, t,
                                     thvm_expand(ctx, binary(ctx, UOP_MUL, invstd, scalar_t(ctx, 1.0f / (f32)N)), full)),
                         full);
    Term dgamma = realize_as(ctx, thvm_sum_axes(ctx, binary(ctx, UOP_MUL, dya, xhat), (u32[]){0, 2, 3}, 3), cshape);
    Term dbeta = chansum(ctx, dya, C);
    Term dW = conv_dw(ctx, xp, dc, B, C, C, 3, H, W_);
    Term dx = conv_dx(ctx, dc, Wc, B, C, C, 3, 1, H, W_);
    readback(ctx, dW);
    readback(ctx, dx);
    (void)dgamma; (void)dbeta;
}

/* Max-pool ties: x [B,C,H,H] takes the integer values -1, 0, 1, 2, so most
 * 2x2 windows hold their maximum more than once, at positive values too.
 * Forward: a = relu(x), p = maxpool2(a) (src/nn/conv.c:484-514), and
 * maxpool2(x); backward with upstream gradients g of distinct integer values
 * 1..4: the pool+relu routing of the conv block and LeNet (every tied
 * maximum receives the gradient, src/interact/grad.c:405-425) and the same
 * routing on x itself. */
static void wl_pooltie(TinyHVM *ctx, u32 B, u32 C, u32 H) {
    Shape full = shape_of((u32[]){B, C, H, H}, 4), half = shape_of((u32[]){B, C, H / 2, H / 2}, 4);
    Term x = gen_tensor(ctx, full, DTYPE_F32, TRC_GEN_INT, 8001, -1.f, 3.f);
    Term g = gen_tensor(ctx, half, DTYPE_F32, TRC_GEN_INT, 8002, 1.f, 5.f);
    rec_mark("pool.fwd");
    Term a = realize_as(ctx, unary(ctx, UOP_RELU, x), full);
    Term p = realize_as(ctx, thvm_maxpool2d(ctx, a, (u32[]){2, 2}, (u32[]){2, 2}), half);
    Term px = realize_as(ctx, thvm_maxpool2d(ctx, x, (u32[]){2, 2}, (u32[]){2, 2}), half);
    readback(ctx, p);
    readback(ctx, px);
    rec_mark("pool.bwd");
    Term da = pool_relu_bwd(ctx, g, p, a, B, C, H, H);
    Term dx = pool_bwd(ctx, g, px, x, B, C, H, H);
    readback(ctx, da);
    readback(ctx, dx);
}

/* Adam (beta1 0.9, beta2 0.999, eps 1e-8, lr 0.01) on two parameters, [1000]
 * and [37,111] (a length that is not a multiple of 4), for two steps. Each
 * step runs the engine's lazy update (the path it takes when the backend has
 * no adam_step slot, src/nn/adam.c:52-95). At this engine version that update
 * writes the moments but not the parameter (its APP-sequenced ASSIGN of the
 * parameter does not take effect), so the parameter's update is realized on
 * its own, with the same op composition (src/nn/adam.c:83-88) over the new
 * moments, and assigned. The parameters and moments are then snapshotted, and
 * the adam_step call of the same step is recorded on copies (the slot's
 * signature, src/tinyhvm.h:1033-1035, called as adam_step_direct does,
 * src/nn/adam.c:103-118). */
static void wl_adam(TinyHVM *ctx) {
    Shape shp[2] = {SHAPE(1000), SHAPE(37, 111)};
    u32 n[2] = {1000, 37 * 111};
    Term P[2], G[2], Pc[2], Mc[2], Vc[2];
    for (int i = 0; i < 2; i++) {
        P[i] = gen_tensor(ctx, shp[i], DTYPE_F32, TRC_GEN_NORMAL, 6001 + i, 0.f, 1.f);
        G[i] = gen_tensor(ctx, shp[i], DTYPE_F32, TRC_GEN_NORMAL, 6011 + i, 0.f, 0.1f);
        Pc[i] = gen_tensor(ctx, shp[i], DTYPE_F32, TRC_GEN_NORMAL, 6001 + i, 0.f, 1.f);
        Mc[i] = zeros(ctx, shp[i], 6021 + i);
        Vc[i] = zeros(ctx, shp[i], 6031 + i);
    }
    Adam opt = adam_init(ctx, 0.01f, 2);
    u32 gids[2];
    for (int i = 0; i < 2; i++) {
        adam_add_param(ctx, &opt, (u32)i, (u32)term_val(P[i]), n[i]);
        gids[i] = (u32)term_val(G[i]);
    }
#define BUF(t) (ctx->tensors[(u32)term_val(t)].buf_id)
#define TBUF(id) (ctx->tensors[(id)].buf_id)
    for (int st = 0; st < 2; st++) {
        rec_mark("adam.lazy");
        thvm_eval(ctx, adam_step_lazy(ctx, &opt, gids));
        f32 bc1 = 1.0f - powf(opt.beta1, (f32)opt.t);
        f32 bc2 = 1.0f - powf(opt.beta2, (f32)opt.t);
        rec_mark("adam.param");
        for (int i = 0; i < 2; i++) {
            Term m = term_new(TAG_TEN, 0, opt.m_bufs[i]);
            Term v = term_new(TAG_TEN, 0, opt.v_bufs[i]);
            Term m_hat = binary(ctx, UOP_DIV, m, scalar_t(ctx, bc1));
            Term v_hat = binary(ctx, UOP_DIV, v, scalar_t(ctx, bc2));
            Term denom = binary(ctx, UOP_ADD, unary(ctx, UOP_SQRT, v_hat), scalar_t(ctx, opt.eps));
            Term step = binary(ctx, UOP_MUL, scalar_t(ctx, opt.lr), binary(ctx, UOP_DIV, m_hat, denom));
            Term p_new = realize_as(ctx, binary(ctx, UOP_SUB, P[i], step), shp[i]);
            thvm_eval(ctx, thvm_assign(ctx, P[i], p_new));
            readback(ctx, P[i]);
            rec_snapshot(BUF(P[i]));
            rec_snapshot(TBUF(opt.m_bufs[i]));
            rec_snapshot(TBUF(opt.v_bufs[i]));
        }
        rec_mark("adam.slot");
        for (int i = 0; i < 2; i++)
            rec_adam(BUF(Pc[i]), BUF(G[i]), BUF(Mc[i]), BUF(Vc[i]), opt.lr, opt.beta1, opt.beta2, opt.eps, bc1,
                     bc2, n[i], BUF(P[i]), TBUF(opt.m_bufs[i]), TBUF(opt.v_bufs[i]));
    }
#undef BUF
#undef TBUF
    adam_free(&opt);
}

/* The engine's own known-answer tests, restated: the same API calls on the
 * same inputs (in one engine context rather than one per case), each case
 * behind a "known.<case>" mark and ending in the readback its test checks. The expected values are the tests' own:
 *   conv        [7,9,13,15]        test/archive/test_tensor_nn_layers.m:19-36
 *   pool        4                  test/archive/test_tensor_nn_layers.m:39-50
 *   bn_eval     y0 1, y3 4         test/archive/test_tensor_nn_layers.m:52-67
 *   relu_linear [0,2.6,0,5.0]      test/archive/test_readme_verify.m:22-41
 *   multiview   160                test/archive/test_lower_multiview_kernel.m:14-33
 *   fused_reduce 165888            test/archive/test_fused_reduce.m:9-36
 *   mul_sum     [20,86]            test/archive/test_cpu_metal_cmp.m:12-28
 *   mm_dup      2*colsum(x)        test/test_mm_dup_2arm.m:22-47
 *   dup_chain   5                  test/test_dup_chain.m:26-66
 *   readme_grad [5,7,9]            README.md:127-146
 *   dtype_*     the printed values test/archive/test_dtype_cast.m:10-61 */
static void known_assign_eval(TinyHVM *ctx, Term dst, Term val) {
    u64 loc = heap_alloc(ctx, 2);
    ctx->heap[loc] = dst;
    ctx->heap[loc + 1] = val;
    u64 ac = heap_alloc(ctx, 1);
    ctx->heap[ac] = term_new(TAG_TOP, UOP_ASSIGN, loc);
    thvm_eval(ctx, term_era());
}

static void wl_known(TinyHVM *ctx) {
    {
        rec_mark("known.conv");
        f32 xdat[] = {1, 2, 3, 4, 5, 6, 7, 8, 9}, wdat[] = {1, 0, 0, 1}, bdat[] = {1};
        Tensor x = tensor_from_f32(ctx, xdat, SHAPE(1, 1, 3, 3));
        Tensor w = tensor_from_f32(ctx, wdat, SHAPE(1, 1, 2, 2));
        Tensor b = tensor_from_f32(ctx, bdat, SHAPE(1));
        u32 st[] = {1, 1}, pd[] = {0, 0, 0, 0};
        tensor_to_host_f32(tensor_realize(tensor_conv2d(x, w, &b, 1, st, pd)));
    }
    {
        rec_mark("known.pool");
        f32 xdat[] = {1, 2, 3, 4};
        Tensor x = tensor_from_f32(ctx, xdat, SHAPE(1, 1, 2, 2));
        thvm_set_requires_grad(ctx, x.term);
        u32 k[] = {2, 2}, st[] = {1, 1};
        tensor_to_host_f32(tensor_realize(tensor_maxpool2d(x, k, st)));
    }
    {
        rec_mark("known.bn_eval");
        f32 xdat[] = {1, 2, 3, 4}, gdat[] = {1}, bdat[] = {0}, mdat[] = {0}, vdat[] = {1};
        Tensor x = tensor_from_f32(ctx, xdat, SHAPE(1, 1, 2, 2));
        Tensor g = tensor_from_f32(ctx, gdat, SHAPE(1));
        Tensor b = tensor_from_f32(ctx, bdat, SHAPE(1));
        Tensor m = tensor_from_f32(ctx, mdat, SHAPE(1));
        Tensor v = tensor_from_f32(ctx, vdat, SHAPE(1));
        tensor_to_host_f32(tensor_realize(tensor_batchnorm(x, g, b, m, v, 1, 1, 2, 2, 0)));
    }
    {
        rec_mark("known.relu_linear");
        f32 x_d[] = {1, 2, 3, 4, 5, 6}, w_d[] = {0.1f, -0.2f, 0.3f, 0.4f, -0.5f, 0.6f}, b_d[] = {-0.1f, 0.2f};
        Tensor x = tensor_from_f32(ctx, x_d, SHAPE(2, 3));
        Tensor w = tensor_from_f32(ctx, w_d, SHAPE(3, 2));
        Tensor b = tensor_from_f32(ctx, b_d, SHAPE(1, 2));
        Linear lin = {.weight = w, .bias = b, .has_bias = 1};
        tensor_to_host_f32(tensor_realize(tensor_relu(linear_forward(&lin, x))));
    }
    {
        rec_mark("known.multiview");
        f32 x[] = {1, 2, 3, 4, 5, 6, 7, 8, 9};
        Term tx = thvm_tensor(ctx, x, SHAPE(1, 1, 3, 3));
        Term pooled = thvm_pool(ctx, tx, (u32[]){2, 2}, (u32[]){1, 1}, 2);
        Term x_rs = thvm_reshape(ctx, pooled, shape_of((u32[]){1, 1, 1, 1, 2, 2, 2, 2}, 8));
        Term doubled = thvm_op(ctx, UOP_ADD, x_rs, x_rs);
        Term total = thvm_sum_axes(ctx, doubled, (u32[]){0, 1, 2, 3, 4, 5, 6, 7}, 8);
        total = thvm_reshape(ctx, total, SHAPE(1));
        Term out = thvm_eval(ctx, total);
        if (term_tag(out) != TAG_TEN) out = thvm_force_tensor_term(ctx, out);
        u32 dt = DTYPE_F32;
        Shape os = SHAPE(1);
        (void)thvm_to_host_raw(ctx, out, &dt, &os);   /* the tensor's host_ptr: thvm_free frees it */
    }
    {
        rec_mark("known.fused_reduce");
        u32 an = 4 * 32 * 12 * 12 * 3 * 3, bn = 32 * 3 * 3;
        f32 *ad = malloc(an * 4), *bd = malloc(bn * 4);
        for (u32 i = 0; i < an; i++) ad[i] = 1.f;
        for (u32 i = 0; i < bn; i++) bd[i] = 1.f;
        Term a = thvm_tensor(ctx, ad, shape_of((u32[]){4, 1, 32, 12, 12, 1, 3, 3}, 8));
        Term b = thvm_tensor(ctx, bd, shape_of((u32[]){1, 1, 32, 1, 1, 1, 3, 3}, 8));
        free(ad);
        free(bd);
        Term summed = thvm_sum_axes(ctx, thvm_op(ctx, UOP_MUL, a, b), (u32[]){0, 3, 4}, 3);
        Term out = thvm_reshape(ctx, summed, shape_of((u32[]){1, 1, 32, 1, 1, 1, 3, 3}, 8));
        Term total = thvm_reshape(ctx, thvm_sum_axes(ctx, out, (u32[]){0, 1, 2, 3, 4, 5, 6, 7}, 8), SHAPE(1));
        f32 z = 0;
        Term dst = thvm_tensor(ctx, &z, SHAPE(1));
        known_assign_eval(ctx, dst, total);
        thvm_to_host(ctx, dst);
    }
    {
        rec_mark("known.mul_sum");
        f32 a[] = {1, 2, 3, 4, 5, 6}, b[] = {2, 3, 4, 5, 6, 7};
        Term ta = thvm_tensor(ctx, a, SHAPE(2, 3));
        Term tb = thvm_tensor(ctx, b, SHAPE(2, 3));
        Term out = thvm_reshape(ctx, thvm_sum_axes(ctx, thvm_op(ctx, UOP_MUL, ta, tb), (u32[]){1}, 1), SHAPE(2));
        f32 z[2] = {0};
        Term dst = thvm_tensor(ctx, z, SHAPE(2));
        known_assign_eval(ctx, dst, out);
        thvm_to_host(ctx, dst);
    }
    {
        rec_mark("known.mm_dup");
        f32 xd[] = {1.0f, 0.5f, 0.1f, -1.0f}, wd[] = {0.1f, 0.2f, 0.3f, 0.05f, 0.1f, -0.2f};
        Term x = thvm_tensor(ctx, xd, SHAPE(2, 2));
        Term W = thvm_tensor(ctx, wd, SHAPE(2, 3));
        thvm_set_requires_grad(ctx, W);
        Term logits = thvm_mm(ctx, x, W);
        Term l0, l1;
        thvm_dup(ctx, thvm_fresh_label(ctx), logits, &l0, &l1);
        Term loss = thvm_op(ctx, UOP_ADD, thvm_sum_axes(ctx, l0, (u32[]){0, 1}, 2),
                            thvm_sum_axes(ctx, l1, (u32[]){0, 1}, 2));
        thvm_to_host(ctx, thvm_eval(ctx, thvm_grad(ctx, loss, W)));
    }
    {
        rec_mark("known.dup_chain");
        f32 wd[4] = {1.0f, -2.0f, 3.5f, -0.5f};
        Term w = thvm_tensor(ctx, wd, SHAPE(4));
        thvm_set_requires_grad(ctx, w);
        Term p_fwd, w1, p_grad, w2, p_sgd, w3, p_assign, w4, p_next, p_done;
        thvm_dup(ctx, thvm_fresh_label(ctx), w, &p_fwd, &w1);
        thvm_dup(ctx, thvm_fresh_label(ctx), w1, &p_grad, &w2);
        thvm_dup(ctx, thvm_fresh_label(ctx), w2, &p_sgd, &w3);
        thvm_dup(ctx, thvm_fresh_label(ctx), w3, &p_assign, &w4);
        thvm_dup(ctx, thvm_fresh_label(ctx), w4, &p_next, &p_done);
        Term s[5];
        Term arms[5] = {p_fwd, p_grad, p_sgd, p_assign, p_next};
        for (int i = 0; i < 5; i++) s[i] = thvm_sum_axes(ctx, arms[i], (u32[]){0}, 1);
        Term loss = thvm_op(ctx, UOP_ADD, s[0],
                            thvm_op(ctx, UOP_ADD, s[1], thvm_op(ctx, UOP_ADD, s[2], thvm_op(ctx, UOP_ADD, s[3], s[4]))));
        thvm_spawn_detached_era(ctx, thvm_ctr(ctx, (Term[]){p_done}, 1));
        thvm_to_host(ctx, thvm_eval(ctx, thvm_grad(ctx, loss, w)));
    }
    {
        rec_mark("known.readme_grad");
        f32 xd[] = {1, 2, 3, 4, 5, 6}, wd[] = {0.1f, 0.2f, 0.3f};
        Tensor x = tensor_from_f32(ctx, xd, SHAPE(2, 3));
        Tensor w = tensor_from_f32(ctx, wd, SHAPE(3));
        thvm_set_requires_grad(ctx, w.term);
        Tensor loss = tensor_sum_axes(tensor_relu(tensor_mul(x, w)), (u32[]){0, 1}, 2);
        Tensor bundle = tensor_realize(tensor_backward_keep(loss, w));
        tensor_to_host_f32(tensor_bundle_get(bundle, 0));
    }
    {
        f32 xf[] = {1.9f, -2.1f, 3.0f};
        Term x = thvm_tensor(ctx, xf, SHAPE(3));
        rec_mark("known.dtype_cast_i32");
        thvm_to_host_i32(ctx, thvm_cast(ctx, x, DTYPE_I32));
        rec_mark("known.dtype_cast_f32");
        i32 iv[] = {3, -4};
        thvm_to_host(ctx, thvm_cast(ctx, thvm_tensor_i32(ctx, iv, SHAPE(2)), DTYPE_F32));
        rec_mark("known.dtype_add_i32");
        i32 aa[] = {10, -20}, bb[] = {-3, 4};
        Term ta = thvm_tensor_i32(ctx, aa, SHAPE(2)), tb = thvm_tensor_i32(ctx, bb, SHAPE(2));
        thvm_to_host_i32(ctx, thvm_eval(ctx, thvm_op(ctx, UOP_ADD, ta, tb)));
        rec_mark("known.dtype_sum_i32");
        i32 cc[] = {1, 2, 3};
        Term tc = thvm_tensor_i32(ctx, cc, SHAPE(3));
        thvm_to_host_i32(ctx, thvm_eval(ctx, thvm_sum_axes(ctx, tc, (u32[]){0}, 1)));
        rec_mark("known.dtype_cast_add_i32");
        i32 ones[] = {1, 1, 1};
        Term tones = thvm_tensor_i32(ctx, ones, SHAPE(3));
        thvm_to_host_i32(ctx, thvm_eval(ctx, thvm_op(ctx, UOP_ADD, thvm_cast(ctx, x, DTYPE_I32), tones)));
        rec_mark("known.dtype_where_i32");
        i32 condv[] = {0, 1, 0}, thenv[] = {10, 20, 30}, elsev[] = {1, 2, 3};
        thvm_to_host_i32(ctx, thvm_where(ctx, thvm_tensor_i32(ctx, condv, SHAPE(3)),
                                         thvm_tensor_i32(ctx, thenv, SHAPE(3)), thvm_tensor_i32(ctx, elsev, SHAPE(3))));
        rec_mark("known.dtype_argmax");
        i32 logitsv[] = {1, 9, 2, 8, 7, 3};
        thvm_to_host_u32(ctx, thvm_argmax(ctx, thvm_tensor_i32(ctx, logitsv, SHAPE(2, 3)), 2, 3));
        rec_mark("known.end");
    }
}

/* ASSIGN from strided views, the engine's use of contiguify
 * (src/interact/tensor_ops.c:113-120): a transpose, a broadcast, a zero-padded
 * (masked) view, a 3-D permute of i32 and a transpose of f16. Each case runs
 * twice: without a contiguify slot (the engine's host round trip gives the
 * golden bytes) and with it (the recorded call). */
typedef Term (*ViewFn)(TinyHVM *ctx, Term src);
/* Views are made eagerly (an aliasing tensor with a strided view, as
 * no_grad_alloc = 0 gives): ASSIGN waits for a tensor source, and a lazy
 * movement term is left to a scheduler pass that never comes for it. */
static Term eager_view(TinyHVM *ctx, Term t, int kind) {
    u8 saved = ctx->no_grad_alloc;
    ctx->no_grad_alloc = 0;
    Term v = kind == 0 ? thvm_permute(ctx, t, (u32[]){1, 0}, 2)
           : kind == 1 ? thvm_expand(ctx, t, SHAPE(4, 7))
           : kind == 2 ? thvm_pad(ctx, t, (u32[]){1, 1, 2, 0}, 2)
                       : thvm_permute(ctx, t, (u32[]){2, 0, 1}, 3);
    ctx->no_grad_alloc = saved;
    return v;
}
static Term v_transpose(TinyHVM *ctx, Term t) { return eager_view(ctx, t, 0); }
static Term v_bcast(TinyHVM *ctx, Term t) { return eager_view(ctx, t, 1); }
static Term v_pad(TinyHVM *ctx, Term t) { return eager_view(ctx, t, 2); }
static Term v_perm3(TinyHVM *ctx, Term t) { return eager_view(ctx, t, 3); }

static void assign_case(TinyHVM *ctx, const char *name, Shape ss, Shape ds, u32 dtype, ViewFn vf, u64 seed) {
    char mk[64];
    snprintf(mk, sizeof mk, "assign.%s", name);
    rec_mark(mk);
    u32 dist = dtype == DTYPE_F32 || dtype == DTYPE_F16 ? TRC_GEN_NORMAL : TRC_GEN_INT;
    f32 p0 = dist == TRC_GEN_INT ? -1000.f : 0.f, p1 = dist == TRC_GEN_INT ? 1000.f : 1.f;
    Term src = gen_tensor(ctx, ss, dtype, dist, seed, p0, p1);
    Term dst_host = gen_tensor(ctx, ds, dtype, TRC_GEN_CONST, seed + 1, 0.f, 0.f);
    Term dst_dev = gen_tensor(ctx, ds, dtype, TRC_GEN_CONST, seed + 2, 0.f, 0.f);
    u32 hid = ctx->tensors[(u32)term_val(dst_host)].buf_id;
    u64 nb = cpu_pool.sizes[hid];
    /* pass 1: no contiguify slot, the engine's host path */
    cpu_backend.contiguify = NULL;
    thvm_eval(ctx, thvm_assign(ctx, dst_host, vf(ctx, src)));
    g_contig_expect = malloc(nb);
    g_contig_expect_n = nb;
    memcpy(g_contig_expect, cpu_pool.bufs[hid], nb);
    /* pass 2: the recorded contiguify call */
    cpu_backend.contiguify = cap_contiguify;
    thvm_eval(ctx, thvm_assign(ctx, dst_dev, vf(ctx, src)));
    free(g_contig_expect);
    g_contig_expect = NULL;
    readback(ctx, dst_dev);
}

static void wl_assign(TinyHVM *ctx) {
    assign_case(ctx, "transpose_f32", SHAPE(5, 7), SHAPE(7, 5), DTYPE_F32, v_transpose, 6001);
    assign_case(ctx, "broadcast_f32", SHAPE(1, 7), SHAPE(4, 7), DTYPE_F32, v_bcast, 6011);
    assign_case(ctx, "pad_f32", SHAPE(5, 7), SHAPE(7, 9), DTYPE_F32, v_pad, 6021);
    assign_case(ctx, "permute3_i32", shape_of((u32[]){3, 4, 2}, 3), shape_of((u32[]){2, 3, 4}, 3), DTYPE_I32,
                v_perm3, 6031);
    assign_case(ctx, "transpose_f16", SHAPE(6, 3), SHAPE(3, 6), DTYPE_F16, v_transpose, 6041);
}

/* The legacy per-op slots, called directly on the recorded backend with the
 * argument shapes the materialize path produces: strided, broadcast and
 * transposed views, mixed storage dtypes, every unary/binary ALU op the CPU
 * backend implements (src/backend/cpu/ops.c:16-60), a strided matmul
 * (:80-113) and SUM/RMAX over the innermost dim (:115-130). */
static u32 gen_buf(u32 n, u32 dtype, u32 dist, u64 seed, f32 p0, f32 p1) {
    u64 bytes = (u64)n * dtype_size(dtype);
    u32 id = cpu_backend.buf_alloc(bytes);
    void *data = NULL;
    if (g_exec) {
        data = malloc((size_t)n * 4 + 4);
        thvm_gen_fill(data, dtype, dist, seed, p0, p1, 0, n);
    }
    g_gen.active = 1; g_gen.dist = dist; g_gen.dtype = dtype; g_gen.seed = seed;
    g_gen.p0 = p0; g_gen.p1 = p1;
    cpu_backend.buf_write(id, data, bytes);
    g_gen.active = 0;
    free(data);
    return id;
}

static View mkview(u32 rank, const u32 *dims, const i32 *strides, i32 offset) {
    View v;
    memset(&v, 0, sizeof v);
    v.shape.rank = rank;
    u32 n = 1, contig = offset == 0;
    i32 expect = 1;
    for (i32 d = (i32)rank - 1; d >= 0; d--) {
        v.shape.dims[d] = dims[d];
        v.strides[d] = strides[d];
        n *= dims[d];
        if (dims[d] != 1 && strides[d] != expect) contig = 0;
        expect *= (i32)dims[d];
    }
    v.offset = offset;
    v.numel = n;
    v.contiguous = contig;
    return v;
}

static void wl_legacy(void) {
    Backend *be = &cpu_backend;
    /* unary: every op on a contiguous f32 vector; a transposed source into f16
     * and i32 destinations; an op id the CPU treats as a plain copy */
    rec_mark("legacy.unary");
    {
        u32 n = 37;
        View v1 = mkview(1, (u32[]){n}, (i32[]){1}, 0);
        u32 x = gen_buf(n, DTYPE_F32, TRC_GEN_NORMAL, 7001, 0.f, 2.f);
        u32 xp = gen_buf(n, DTYPE_F32, TRC_GEN_UNIFORM, 7002, 0.01f, 9.f);
        u32 ops[5] = {UOP_NEG, UOP_RELU, UOP_EXP, UOP_LOG, UOP_SQRT};
        for (u32 i = 0; i < 5; i++) {
            u32 out = be->buf_alloc(n * 4);
            u32 src = (ops[i] == UOP_LOG || ops[i] == UOP_SQRT) ? xp : x;
            be->op_unary(ops[i], out, &v1, DTYPE_F32, src, &v1, DTYPE_F32);
        }
        /* LOG and SQRT of negative inputs: NaN */
        u32 o1 = be->buf_alloc(n * 4), o2 = be->buf_alloc(n * 4);
        be->op_unary(UOP_LOG, o1, &v1, DTYPE_F32, x, &v1, DTYPE_F32);
        be->op_unary(UOP_SQRT, o2, &v1, DTYPE_F32, x, &v1, DTYPE_F32);
        u32 a = gen_buf(35, DTYPE_F32, TRC_GEN_NORMAL, 7003, 0.f, 100.f);
        View dv = mkview(2, (u32[]){7, 5}, (i32[]){5, 1}, 0);
        View tv = mkview(2, (u32[]){7, 5}, (i32[]){1, 7}, 0);
        u32 h = be->buf_alloc(35 * 2), i32b = be->buf_alloc(35 * 4);
        be->op_unary(UOP_RELU, h, &dv, DTYPE_F16, a, &tv, DTYPE_F32);
        be->op_unary(UOP_NEG, i32b, &dv, DTYPE_I32, a, &tv, DTYPE_F32);
        u32 cpy = be->buf_alloc(35 * 4);
        be->op_unary(UOP_ADD, cpy, &dv, DTYPE_U32, a, &tv, DTYPE_F32);
    }
    /* binary: every op, b broadcast along rows (stride 0), b with zeros for
     * DIV, mixed source dtypes */
    rec_mark("legacy.binary");
    {
        u32 R = 6, Cn = 9;
        View dv = mkview(2, (u32[]){R, Cn}, (i32[]){(i32)Cn, 1}, 0);
        View row = mkview(2, (u32[]){R, Cn}, (i32[]){0, 1}, 0);
        u32 a = gen_buf(R * Cn, DTYPE_F32, TRC_GEN_NORMAL, 7011, 0.f, 1.f);
        u32 b = gen_buf(Cn, DTYPE_F32, TRC_GEN_INT, 7012, -2.f, 3.f);   /* integers: zeros for DIV */
        u32 ops[6] = {UOP_ADD, UOP_SUB, UOP_MUL, UOP_DIV, UOP_MAX, UOP_CMP};
        for (u32 i = 0; i < 6; i++) {
            u32 out = be->buf_alloc(R * Cn * 4);
            be->op_binary(ops[i], out, &dv, DTYPE_F32, a, &dv, DTYPE_F32, b, &row, DTYPE_F32);
        }
        u32 ai = gen_buf(R * Cn, DTYPE_I32, TRC_GEN_INT, 7013, -50.f, 50.f);
        u32 bh = gen_buf(R * Cn, DTYPE_F16, TRC_GEN_NORMAL, 7014, 0.f, 4.f);
        View tv = mkview(2, (u32[]){R, Cn}, (i32[]){1, (i32)R}, 0);
        u32 o = be->buf_alloc(R * Cn * 4), oh = be->buf_alloc(R * Cn * 2);
        be->op_binary(UOP_MUL, o, &dv, DTYPE_F32, ai, &dv, DTYPE_I32, bh, &tv, DTYPE_F16);
        be->op_binary(UOP_ADD, oh, &dv, DTYPE_F16, a, &tv, DTYPE_F32, ai, &dv, DTYPE_I32);
    }
    /* matmul: contiguous f32; A as a transposed view; f16 B into f16 */
    rec_mark("legacy.mm");
    {
        u32 M = 13, K = 17, N = 11;
        View av = mkview(2, (u32[]){M, K}, (i32[]){(i32)K, 1}, 0);
        View bv = mkview(2, (u32[]){K, N}, (i32[]){(i32)N, 1}, 0);
        View at = mkview(2, (u32[]){M, K}, (i32[]){1, (i32)M}, 0);
        u32 A = gen_buf(M * K, DTYPE_F32, TRC_GEN_UNIFORM, 7021, -1.f, 1.f);
        u32 B = gen_buf(K * N, DTYPE_F32, TRC_GEN_UNIFORM, 7022, -1.f, 1.f);
        u32 Bh = gen_buf(K * N, DTYPE_F16, TRC_GEN_UNIFORM, 7023, -1.f, 1.f);
        u32 o1 = be->buf_alloc(M * N * 4), o2 = be->buf_alloc(M * N * 4), o3 = be->buf_alloc(M * N * 2);
        be->op_mm(o1, DTYPE_F32, A, &av, DTYPE_F32, B, &bv, DTYPE_F32, M, K, N);
        be->op_mm(o2, DTYPE_F32, A, &at, DTYPE_F32, B, &bv, DTYPE_F32, M, K, N);
        be->op_mm(o3, DTYPE_F16, A, &av, DTYPE_F32, Bh, &bv, DTYPE_F16, M, K, N);
    }
    /* reduce: SUM and RMAX over the innermost dim, f32 and i32 sources */
    rec_mark("legacy.reduce");
    {
        u32 O = 9, Rn = 33;
        u32 x = gen_buf(O * Rn, DTYPE_F32, TRC_GEN_NORMAL, 7031, 0.f, 1.f);
        u32 xi = gen_buf(O * Rn, DTYPE_I32, TRC_GEN_INT, 7032, -1000.f, 1000.f);
        u32 s1 = be->buf_alloc(O * 4), s2 = be->buf_alloc(O * 4), s3 = be->buf_alloc(O * 4);
        be->op_reduce(UOP_SUM, s1, O, DTYPE_F32, x, O * Rn, DTYPE_F32, Rn);
        be->op_reduce(UOP_RMAX, s2, O, DTYPE_F32, x, O * Rn, DTYPE_F32, Rn);
        be->op_reduce(UOP_SUM, s3, O, DTYPE_I32, xi, O * Rn, DTYPE_I32, Rn);
    }
}

/* Reductions with few outputs over long axes (a row sum and row max of
 * [R, C], and a per-channel sum over [B, Ch, H, W] axes 0, 2, 3), the shape of
 * batchnorm statistics and bias gradients. */
static void wl_longreduce(TinyHVM *ctx, u32 R, u32 Cn) {
    Term x = gen_tensor(ctx, SHAPE(R, Cn), DTYPE_F32, TRC_GEN_NORMAL, 8001, 0.f, 1.f);
    rec_mark("longreduce.sum");
    readback(ctx, realize_as(ctx, thvm_sum_axes(ctx, binary(ctx, UOP_MUL, x, scalar_t(ctx, 0.5f)), (u32[]){1}, 1),
                             SHAPE(R)));
    rec_mark("longreduce.max");
    readback(ctx, realize_as(ctx, thvm_rmax_axes(ctx, x, (u32[]){1}, 1), SHAPE(R)));
    Term g = gen_tensor(ctx, shape_of((u32[]){8, 3, 40, 40}, 4), DTYPE_F32, TRC_GEN_UNIFORM, 8002, -1.f, 1.f);
    rec_mark("longreduce.chansum");
    readback(ctx, chansum(ctx, g, 3));
}

/* Storage dtypes and casts (the operations of the engine's own dtype test,
 * test/archive/test_dtype_cast.m, at edge values): f32 -> i32/u32/f16 casts
 * (truncation, out-of-range, negative, NaN, f16 ties and overflow), i32/u32
 * arithmetic and sums, f16 tensors in arithmetic and reductions. */
static void wl_dtypes(TinyHVM *ctx) {
    f32 xf[16] = {1.9f, -2.1f, 3.0f, 2147483648.0f, -3e9f, 1e19f, -1.0f, 4e9f,
                  2049.0f, 65520.0f, 1e-6f, -0.0f, 0.5f, 1.00048828125f, 3.0e-5f, 0.0f};
    xf[15] = nanf("");
    Term x = thvm_tensor(ctx, xf, SHAPE(16));
    rec_mark("dtypes.cast_i32");
    readback(ctx, realize(ctx, thvm_cast(ctx, x, DTYPE_I32)));
    rec_mark("dtypes.cast_u32");
    readback(ctx, realize(ctx, thvm_cast(ctx, x, DTYPE_U32)));
    rec_mark("dtypes.cast_f16");
    readback(ctx, realize(ctx, thvm_cast(ctx, x, DTYPE_F16)));
    i32 iv[4] = {3, -4, 100000, -7};
    Term ti = thvm_tensor_i32(ctx, iv, SHAPE(4));
    rec_mark("dtypes.i32");
    readback(ctx, realize(ctx, thvm_cast(ctx, ti, DTYPE_F32)));
    i32 bb[4] = {-3, 4, 5, 9};
    Term tb = thvm_tensor_i32(ctx, bb, SHAPE(4));
    readback(ctx, realize(ctx, binary(ctx, UOP_ADD, ti, tb)));
    readback(ctx, realize(ctx, thvm_sum_axes(ctx, ti, (u32[]){0}, 1)));
    i32 ones[16];
    for (int i = 0; i < 16; i++) ones[i] = 1;
    Term tones = thvm_tensor_i32(ctx, ones, SHAPE(16));
    readback(ctx, realize(ctx, binary(ctx, UOP_ADD, thvm_cast(ctx, x, DTYPE_I32), tones)));
    rec_mark("dtypes.u32");
    u32 uv[4] = {7, 4000000000u, 0, 123};
    Term tu = thvm_tensor_u32(ctx, uv, SHAPE(4));
    readback(ctx, realize(ctx, binary(ctx, UOP_MUL, tu, scalar_t(ctx, 2.0f))));
    readback(ctx, realize(ctx, thvm_sum_axes(ctx, tu, (u32[]){0}, 1)));
    rec_mark("dtypes.f16");
    u16 hv[300];
    for (int i = 0; i < 300; i++) hv[i] = f32_to_f16_bits(0.01f * (f32)(i - 150));
    Term th = thvm_tensor_typed(ctx, hv, SHAPE(300), DTYPE_F16);
    readback(ctx, realize(ctx, binary(ctx, UOP_MUL, th, scalar_t(ctx, 3.0f))));
    readback(ctx, realize(ctx, thvm_sum_axes(ctx, th, (u32[]){0}, 1)));
    readback(ctx, realize(ctx, thvm_rmax_axes(ctx, th, (u32[]){0}, 1)));
    readback(ctx, realize(ctx, thvm_cast(ctx, th, DTYPE_F32)));
    Term seed = thvm_scalar_typed(ctx, 1.0f, DTYPE_F16);
    readback(ctx, seed);
}

#ifndef CAPTURE_NO_MAIN
int main(int argc, char **argv) {
    int ai = 1;
    while (ai < argc && argv[ai][0] == '-') {
        if (strcmp(argv[ai], "-n") == 0) g_exec = 0;
        else if (strcmp(argv[ai], "-r") == 0) g_read_data = 1;
        ai++;
    }
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
    } else if (strcmp(wl, "mlp") == 0) {
        wl_mlp(ctx, nsz > 0 ? sz[0] : 64, nsz > 1 ? sz[1] : 784, nsz > 2 ? sz[2] : 128, nsz > 3 ? sz[3] : 10);
    } else if (strcmp(wl, "lenet") == 0) {
        wl_lenet(ctx, nsz > 0 ? sz[0] : 256, nsz > 1 ? (int)sz[1] : 1);
    } else if (strcmp(wl, "convblock") == 0) {
        wl_convblock(ctx, nsz > 0 ? sz[0] : 64, nsz > 1 ? sz[1] : 64, nsz > 2 ? sz[2] : 56);
    } else if (strcmp(wl, "pooltie") == 0) {
        wl_pooltie(ctx, nsz > 0 ? sz[0] : 2, nsz > 1 ? sz[1] : 4, nsz > 2 ? sz[2] : 16);
    } else if (strcmp(wl, "dtypes") == 0) {
        wl_dtypes(ctx);
    } else if (strcmp(wl, "assign") == 0) {
        wl_assign(ctx);
    } else if (strcmp(wl, "known") == 0) {
        wl_known(ctx);
    } else if (strcmp(wl, "adam") == 0) {
        wl_adam(ctx);
    } else if (strcmp(wl, "legacy") == 0) {
        wl_legacy();
    } else if (strcmp(wl, "longreduce") == 0) {
        wl_longreduce(ctx, nsz > 0 ? sz[0] : 4, nsz > 1 ? sz[1] : 20000);
    } else if (strcmp(wl, "linear") == 0) {
        wl_linear(ctx, nsz > 0 ? sz[0] : 64, nsz > 1 ? sz[1] : 64, nsz > 2 ? sz[2] : 64, 1);
    } else {
        fprintf(stderr, "unknown workload %s\n", wl);
        return 2;
    }
    fclose(g_out);
    return 0;
}
#endif /* CAPTURE_NO_MAIN */
