/*
 * backend.c - the HIP Backend vtable (drop-in for cpu_backend / metal_backend,
 * src/backend/cpu/_.c:21-35, src/backend/metal/_.m:30-57) and its dispatch.
 *
 * Everything runs on one device and one in-order HIP stream; the only calls
 * that block the host are buf_read (the engine's sync point), large pageable
 * buf_writes, and pool_reset when device memory must be returned.
 *
 * dispatch_uop_kernel: dense recognizers first (matmul / conv / pooling
 * shapes routed to hand-written kernels), else the hipRTC-generated kernel
 * for the KOp program, compiled once per program and cached.
 */
#include <stdlib.h>
#include <time.h>
#include <string.h>

#include "hipb.h"
#include "thvm_hip.h"
#include "kargs.h"
#include "noalloc.h"

HipbState hipb;

/* Workspace of split group reductions: grown on demand and reused by every
 * dispatch (the stream orders the users). */
static Scratch red_ws;

/* ASSIGN's buf_copy calls are queued and issued together as one batched copy
 * kernel: an SGD step copies every updated parameter back, one copy after
 * each update kernel, and none of those kernels touches an earlier copy's
 * buffers. Anything that does touch a queued buffer (a dispatch reading or
 * writing it, a host read or write, a free) issues the queue first, so the
 * stream still sees every copy before any later use of its buffers. */
static struct {
    CopyBatch b;
    u32 dst_id[COPY_BATCH_MAX], src_id[COPY_BATCH_MAX];
} CQ;

static void copyq_flush(void) {
    if (CQ.b.n == 0) return;
    hipFunction_t fn = rtc_static_fn("thvm_copy_batch");
    if (fn) {
        u64 mx = 0;
        for (u32 i = 0; i < CQ.b.n; i++) if (CQ.b.bytes[i] > mx) mx = CQ.b.bytes[i];
        u64 gx = (mx + 4095) / 4096;
        if (gx < 1) gx = 1;
        if (gx > 256) gx = 256;
        void *params[] = {&CQ.b};
        hipb_launch(fn, (u32)gx, CQ.b.n, 1, 256, params);
    } else {
        for (u32 i = 0; i < CQ.b.n; i++)
            HIPB_CHECK(hipMemcpyAsync((void *)(uintptr_t)CQ.b.dst[i], (const void *)(uintptr_t)CQ.b.src[i],
                                      CQ.b.bytes[i], hipMemcpyDeviceToDevice, hipb.stream));
    }
    CQ.b.n = 0;
}

static int copyq_uses(u32 id) {
    for (u32 i = 0; i < CQ.b.n; i++)
        if (CQ.dst_id[i] == id || CQ.src_id[i] == id) return 1;
    return 0;
}

/* issue the queue if buffer id takes part in it */
static void copyq_guard(u32 id) {
    if (CQ.b.n && id && copyq_uses(id)) copyq_flush();
}

static void copyq_guard_dispatch(u32 out, const u32 *leaves, u32 n) {
    if (!CQ.b.n) return;
    copyq_guard(out);
    for (u32 i = 0; i < n && CQ.b.n; i++) copyq_guard(leaves[i]);
}

/* Batched launches (co-launch). A generated kernel's launch of at most
 * HB_MAX_BLOCKS workgroups is held back instead of issued; while the next
 * dispatches are such launches too and touch no memory a held one writes
 * (and write none a held one reads), they join it. The held launches then go
 * out as one launch of a batch kernel that hands each one its own range of
 * workgroups and calls its module's device function (CoForm) with its own
 * block coordinates, so that independent kernels of a step run side by side
 * instead of one after another: a layer's weight, bias and input gradients,
 * a step's SGD updates. The batch kernel is compiled once per sequence of
 * programs and grid sizes. Any other work put on the stream issues the held
 * launches first (hipb_before_stream), so the stream still sees everything in
 * program order; launches in one batch are independent by construction.
 * A batch's workgroups have the largest size among its programs (a smaller
 * program's surplus waves end at once; a wave that has ended no longer takes
 * part in the workgroup's barriers). The batch kernel holds every program's
 * static LDS, at most HB_MAX_LDS in all; a batch with a program whose
 * workgroups wait for each other fits on the GPU at once, and each program
 * that combines partials through the combine area has its own slice of it. */
/* Sequences. Launches of a few workgroups each (the softmax and loss of a
 * training step: row maxima, exponentials, sums, logarithms on [batch, 10])
 * that depend on each other are held too: each one that touches memory an
 * earlier held launch writes (or writes what one reads) starts a new step,
 * and they go out as one launch of a sequence kernel whose single workgroup
 * runs the programs in order, each program's workgroups side by side on
 * their own waves, a workgroup barrier after each program (which also makes
 * the global writes before it visible to the whole workgroup). Every
 * program's code is its own device function, so the results are those of
 * separate launches bit for bit; the launches saved are what a step of tiny
 * dependent kernels pays for. A sequence holds only programs of at most
 * HB_SEQ_MAX_BLOCKS workgroups of at most HB_SEQ_THREADS lanes, without
 * workgroup barriers or LDS of their own, none resident or held alone; if
 * one no longer qualifies when the sequence goes out (a fusion grew it), the
 * held launches go out one by one in order. */
#define HB_SEQ_MAX_BLOCKS 4u
#define HB_SEQ_THREADS 256u
#define HB_MAX 16
#define HB_MAX_BLOCKS 512
#define HB_MAX_LDS 65536u
#define HB_ARG_BYTES (CO_MAX_PARAMS * 8)
typedef struct {
    CoForm co;             /* a copy (its strings live until shutdown) */
    hipFunction_t fn;
    u32 gx, gy;
    u8 args[HB_ARG_BYTES];
    HbMem m;
    int resident;
    u64 fz_key;            /* a contraction an elementwise consumer may fuse into (0: none) */
    u32 fz_serial, fz_out; /* ... its dense entry and its output buffer */
    int solo;              /* held only for a fused epilogue: joins no batch */
    const ChainInfo *ch;   /* a program an elementwise consumer may fuse after (chain.c; NULL: none) */
    u32 ch_bufs[1 + FUSE_MAX_LEAVES]; /* ... its buffers (output, leaves) */
    u64 ch_seq;            /* ... the pool's host-write clock when it was held */
    u32 ch_nb;
    u32 wg;                /* a run-sum group later sums and consumers may join (1 + index into HB.wg; 0: none) */
    const void *wmax;      /* a window max a run sum over its output may take in (window.c entry; NULL: none) */
    u32 wmax_bufs[2];      /* ... its output and input */
    u64 hid;               /* identifies the held launch while it is held */
    int seq_start;         /* reads or writes what an earlier held launch touches: starts a new step of
                              the held sequence */
} HbEnt;
static struct {
    HbEnt ent[HB_MAX];
    WinGroup wg[HB_MAX];
    u8 wg_used[HB_MAX];
    u64 next_hid;
    u32 n;
    u64 comb_used;         /* combine-area words given to the held launches */
    int flushing;
    int seq;               /* the held launches are a sequence of dependent steps (hb_seq_*) */
    struct { u64 key; hipModule_t mod; hipFunction_t fn; u32 cap; } cache[64];
    u32 ncache;
} HB;

static int hb_seq_eligible(const HbEnt *h);

static int hb_overlap(u64 a0, u64 a1, u64 b0, u64 b1) { return a0 < b1 && b0 < a1; }

void hbm_add(HbMem *m, const void *p, u64 bytes, int write) {
    if (!p || !bytes) return;
    if (m->n >= HB_RANGES) {
        /* out of slots: widen the last range to cover this one too */
        u64 lo = (u64)(uintptr_t)p, hi = lo + bytes;
        if (lo < m->lo[m->n - 1]) m->lo[m->n - 1] = lo;
        if (hi > m->hi[m->n - 1]) m->hi[m->n - 1] = hi;
        m->wr[m->n - 1] |= (u8)(write != 0);
        return;
    }
    m->lo[m->n] = (u64)(uintptr_t)p;
    m->hi[m->n] = m->lo[m->n] + bytes;
    m->wr[m->n] = (u8)(write != 0);
    m->n++;
}

static int hbm_clash(const HbMem *a, const HbMem *b) {
    for (u32 i = 0; i < a->n; i++)
        for (u32 j = 0; j < b->n; j++)
            if ((a->wr[i] || b->wr[j]) && hb_overlap(a->lo[i], a->hi[i], b->lo[j], b->hi[j])) return 1;
    return 0;
}

static u32 hb_arg_off(u32 off, u32 sz) { return (off + sz - 1u) & ~(sz - 1u); }

/* the launch parameters of one held launch, in its kernel's order */
static u32 hb_params(HbEnt *h, void **pv) {
    u32 off = 0;
    for (u32 j = 0; j < h->co.np; j++) {
        off = hb_arg_off(off, h->co.psz[j]);
        pv[j] = h->args + off;
        off += h->co.psz[j];
    }
    return h->co.np;
}

static u64 hb_mix(u64 h, u64 v) {
    h ^= v + 0x9E3779B97F4A7C15ull + (h << 6) + (h >> 2);
    h *= 0xFF51AFD7ED558CCDull;
    return h ^ (h >> 33);
}

static u32 hb_threads(void) {
    u32 t = 0;
    for (u32 i = 0; i < HB.n; i++) if (HB.ent[i].co.threads > t) t = HB.ent[i].co.threads;
    return t;
}

/* appends a parameter list's names (or "type name"s with `decl`), each
 * prefixed q<i>_ */
static size_t hb_put_params(char *src, size_t w, size_t cap, const char *params, u32 i, int decl, int first) {
    const char *p = params;
    while (*p) {
        const char *e = strstr(p, ", ");
        size_t len = e ? (size_t)(e - p) : strlen(p);
        const char *sp = p + len;
        while (sp > p && sp[-1] != ' ' && sp[-1] != '*') sp--;
        w += (size_t)snprintf(src + w, cap - w, "%s%.*sq%u_%.*s", first ? "" : ", ", decl ? (int)(sp - p) : 0, p, i,
                              (int)(len - (size_t)(sp - p)), sp);
        first = 0;
        p = e ? e + 2 : p + len;
    }
    return w;
}

/* Source of the batch kernel `name` for launches ents[0..n) in order, with
 * T lanes per workgroup: each program's module once, and an entry that hands
 * workgroup ranges to their device functions. */
/* Lanes of the sequence kernel of n held launches: the most any one program
 * takes with all its workgroups side by side (at most 1024). */
static u32 hb_seq_threads(const HbEnt *ents, u32 n) {
    u32 T = 64;
    for (u32 i = 0; i < n; i++) {
        const u32 t = ents[i].gx * ents[i].gy * ents[i].co.threads;
        if (t > T) T = t;
    }
    return T;
}

/* The sequence kernel of n held launches: one workgroup of T lanes runs the
 * programs in order, workgroup b of a program of W waves on waves
 * [b W, (b + 1) W), a barrier after each program (see Sequences above). */
static char *hb_seq_source(const HbEnt *ents, u32 n, u32 T, const char *name) {
    size_t cap = strlen(kgen_prelude()) + 4096;
    for (u32 i = 0; i < n; i++) cap += strlen(ents[i].co.src) + 4 * strlen(ents[i].co.params) + 512;
    char *src = malloc(cap);
    if (!src) return NULL;
    size_t w = (size_t)snprintf(src, cap, "%s\n", kgen_prelude());
    for (u32 i = 0; i < n; i++) {
        int seen = 0;
        for (u32 j = 0; j < i; j++) seen |= ents[j].co.id == ents[i].co.id;
        if (!seen) w += (size_t)snprintf(src + w, cap - w, "%s\n", ents[i].co.src);
    }
    w += (size_t)snprintf(src + w, cap - w, "extern \"C\" __global__ __launch_bounds__(%u) void %s(", T, name);
    for (u32 i = 0; i < n; i++) w = hb_put_params(src, w, cap, ents[i].co.params, i, 1, i == 0);
    w += (size_t)snprintf(src + w, cap - w,
                          ") {\n  const u32 wv_ = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);\n  (void)wv_;\n");
    for (u32 i = 0; i < n; i++) {
        const HbEnt *h = &ents[i];
        const u32 W = h->co.threads / 64u, G = h->gx * h->gy;
        w += (size_t)snprintf(src + w, cap - w, "  ");
        if (G * W * 64u < T) w += (size_t)snprintf(src + w, cap - w, "if (wv_ < %uu) ", G * W);
        w += (size_t)snprintf(src + w, cap - w,
                              "{\n    const u32 b_ = wv_ / %uu;\n    co_%u::%s(b_ %% %uu, b_ / %uu, %uu, %uu, "
                              "threadIdx.x - b_ * %uu",
                              W, h->co.id, h->co.name, h->gx, h->gx, h->gx, h->gy, h->co.threads);
        w = hb_put_params(src, w, cap, h->co.params, i, 0, 0);
        w += (size_t)snprintf(src + w, cap - w, ");\n  }\n  __syncthreads();\n");
    }
    snprintf(src + w, cap - w, "}\n");
    return src;
}

static char *hb_batch_source(const HbEnt *ents, u32 n, u32 T, const char *name) {
    size_t cap = strlen(kgen_prelude()) + 4096;
    for (u32 i = 0; i < n; i++) cap += strlen(ents[i].co.src) + 4 * strlen(ents[i].co.params) + 512;
    char *src = malloc(cap);
    if (!src) return NULL;
    size_t w = (size_t)snprintf(src, cap, "%s\n", kgen_prelude());
    for (u32 i = 0; i < n; i++) {
        int seen = 0;
        for (u32 j = 0; j < i; j++) seen |= ents[j].co.id == ents[i].co.id;
        if (!seen) w += (size_t)snprintf(src + w, cap - w, "%s\n", ents[i].co.src);
    }
    w += (size_t)snprintf(src + w, cap - w, "extern \"C\" __global__ __launch_bounds__(%u) void %s(", T, name);
    for (u32 i = 0; i < n; i++) w = hb_put_params(src, w, cap, ents[i].co.params, i, 1, i == 0);
    w += (size_t)snprintf(src + w, cap - w,
                          ") {\n  u32 b_ = blockIdx.x;\n"
                          "  const u32 wv_ = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);\n  (void)wv_;\n");
    for (u32 i = 0; i < n; i++) {
        const HbEnt *h = &ents[i];
        w += (size_t)snprintf(src + w, cap - w, "  if (b_ < %uu) {", h->gx * h->gy);
        if (h->co.threads < T) w += (size_t)snprintf(src + w, cap - w, " if (wv_ >= %uu) return;", h->co.threads / 64u);
        w += (size_t)snprintf(src + w, cap - w, " co_%u::%s(b_ %% %uu, b_ / %uu, %uu, %uu, threadIdx.x", h->co.id,
                              h->co.name, h->gx, h->gx, h->gx, h->gy);
        w = hb_put_params(src, w, cap, h->co.params, i, 0, 0);
        w += (size_t)snprintf(src + w, cap - w, "); return; }\n  b_ -= %uu;\n", h->gx * h->gy);
    }
    snprintf(src + w, cap - w, "}\n");
    return src;
}

/* The batch kernel for the held sequence (compiled once per key) and the
 * workgroups of it the GPU holds at once (*cap). */
static hipFunction_t hb_batch_fn(u64 key, u32 T, u32 *cap, int seq) {
    *cap = 0;
    for (u32 i = 0; i < HB.ncache; i++)
        if (HB.cache[i].key == key) {
            *cap = HB.cache[i].cap;
            return HB.cache[i].fn;
        }
    if (HB.ncache >= sizeof HB.cache / sizeof HB.cache[0]) return NULL;
    char name[48];
    snprintf(name, sizeof name, "thvm_%s_%016llx", seq ? "seq" : "batch", (unsigned long long)key);
    char *src = seq ? hb_seq_source(HB.ent, HB.n, T, name) : hb_batch_source(HB.ent, HB.n, T, name);
    if (!src) return NULL;
    if (hipb.verbose) {
        fprintf(stderr, "tinyhvm-hip: %s (%u lanes):", name, T);
        for (u32 i = 0; i < HB.n; i++)
            fprintf(stderr, " %s[%ux%u]", HB.ent[i].co.name, HB.ent[i].gx, HB.ent[i].gy);
        fprintf(stderr, "\n");
    }
    if (hipb.dump_src) fprintf(stderr, "---- batch kernel ----\n%s\n", src);
    char err[256] = {0};
    hipModule_t mod;
    hipFunction_t fn = NULL;
    if (rtc_build_module(src, &mod, err, sizeof err)) {
        if (hipModuleGetFunction(&fn, mod, name) == hipSuccess) {
            HB.cache[HB.ncache].key = key;
            HB.cache[HB.ncache].mod = mod;
            HB.cache[HB.ncache].fn = fn;
            HB.cache[HB.ncache].cap = *cap = rtc_capacity(fn, T);
            HB.ncache++;
            hipb.n_compile++;
        } else {
            HIPB_CHECK(hipModuleUnload(mod));
            fn = NULL;
        }
    } else {
        fprintf(stderr, "tinyhvm-hip: batch kernel build failed: %s\n", err);
    }
    free(src);
    return fn;
}

/* Device-free check of the co-launch forms: the batch kernel of n generated
 * modules (their sources, main kernel names, workgroup sizes and grids as gx,
 * gy pairs), compiled for gfx950 without loading. Returns the code-object
 * size, or -1 with the reason in errbuf. */
int thvm_hip_batch_compile_check(const char *const *srcs, const char *const *names, const u32 *threads,
                                 const u32 *grid, u32 n, char *errbuf, u64 errlen) {
    if (!srcs || !names || !threads || !grid || n == 0 || n > HB_MAX || !errbuf || errlen == 0) return -1;
    HbEnt *ents = calloc(n, sizeof(HbEnt));
    if (!ents) return -1;
    u32 T = 0, ok = 1;
    for (u32 i = 0; i < n && ok; i++) {
        if (!co_form_make(&ents[i].co, srcs[i], names[i], threads[i], NULL)) {
            snprintf(errbuf, errlen, "no co-launch form for %s", names[i]);
            ok = 0;
            break;
        }
        ents[i].gx = grid[2 * i];
        ents[i].gy = grid[2 * i + 1];
        if (threads[i] > T) T = threads[i];
    }
    long r = -1;
    char *src = ok ? hb_batch_source(ents, n, T, "thvm_batch_check") : NULL;
    if (src) r = rtc_compile_only(src, errbuf, (size_t)errlen);
    free(src);
    for (u32 i = 0; i < n; i++) co_form_free(&ents[i].co);
    free(ents);
    return (int)r;
}

/* Device-free check of the sequence kernel of n generated modules (as for
 * thvm_hip_batch_compile_check; the programs run in order by one
 * workgroup, each program's workgroups side by side). */
int thvm_hip_seq_compile_check(const char *const *srcs, const char *const *names, const u32 *threads,
                               const u32 *grid, u32 n, char *errbuf, u64 errlen) {
    if (!srcs || !names || !threads || !grid || n == 0 || n > HB_MAX || !errbuf || errlen == 0) return -1;
    HbEnt *ents = calloc(n, sizeof(HbEnt));
    if (!ents) return -1;
    u32 ok = 1;
    for (u32 i = 0; i < n && ok; i++) {
        if (!co_form_make(&ents[i].co, srcs[i], names[i], threads[i], NULL)) {
            snprintf(errbuf, errlen, "no co-launch form for %s", names[i]);
            ok = 0;
            break;
        }
        ents[i].gx = grid[2 * i];
        ents[i].gy = grid[2 * i + 1];
        if (!hb_seq_eligible(&ents[i])) {
            snprintf(errbuf, errlen, "%s cannot be a step of a sequence", names[i]);
            ok = 0;
        }
    }
    long r = -1;
    char *src = ok ? hb_seq_source(ents, n, hb_seq_threads(ents, n), "thvm_seq_check") : NULL;
    if (src) r = rtc_compile_only(src, errbuf, (size_t)errlen);
    free(src);
    for (u32 i = 0; i < n; i++) co_form_free(&ents[i].co);
    free(ents);
    return (int)r;
}

/* Issues the held launches: one alone as itself, several as their batch
 * kernel (or one by one if it cannot be built). */
static void hb_flush(void) {
    if (!HB.n || HB.flushing) return;
    HB.flushing = 1;
    int seq_ok = HB.seq && HB.n > 1;
    for (u32 i = 0; i < HB.n && seq_ok; i++) seq_ok = hb_seq_eligible(&HB.ent[i]);
    if (HB.n == 1) {
        void *pv[CO_MAX_PARAMS];
        hb_params(&HB.ent[0], pv);
        hipb_launch(HB.ent[0].fn, HB.ent[0].gx, HB.ent[0].gy, 1, HB.ent[0].co.threads, pv);
    } else if (HB.seq) {
        /* dependent steps: the sequence kernel, or each launch alone in order */
        const u32 T = hb_seq_threads(HB.ent, HB.n);
        u64 key = hb_mix(0x73657175656e6365ull, T);
        for (u32 i = 0; i < HB.n; i++)
            key = hb_mix(hb_mix(hb_mix(key, HB.ent[i].co.id), HB.ent[i].gx), HB.ent[i].gy);
        u32 cap = 0;
        hipFunction_t fn = seq_ok ? hb_batch_fn(key, T, &cap, 1) : NULL;
        if (fn) {
            void *pv[HB_MAX * CO_MAX_PARAMS];
            u32 np = 0;
            for (u32 i = 0; i < HB.n; i++) np += hb_params(&HB.ent[i], pv + np);
            hipb_launch(fn, 1, 1, 1, T, pv);
            hipb.n_batched += HB.n;
            hipb.n_seq += HB.n;
        } else {
            for (u32 i = 0; i < HB.n; i++) {
                void *pv[CO_MAX_PARAMS];
                hb_params(&HB.ent[i], pv);
                hipb_launch(HB.ent[i].fn, HB.ent[i].gx, HB.ent[i].gy, 1, HB.ent[i].co.threads, pv);
            }
        }
    } else {
        const u32 T = hb_threads();
        u64 key = hb_mix(0x626174636822ull, T);
        u32 total = 0, np = 0, cap = 0;
        int resident = 0;
        for (u32 i = 0; i < HB.n; i++) {
            key = hb_mix(hb_mix(hb_mix(key, HB.ent[i].co.id), HB.ent[i].gx), HB.ent[i].gy);
            total += HB.ent[i].gx * HB.ent[i].gy;
            resident |= HB.ent[i].resident;
        }
        hipFunction_t fn = hb_batch_fn(key, T, &cap, 0);
        /* a program whose workgroups wait for each other goes in a batch only
         * if the batch kernel's whole grid is on the GPU at once, with the
         * batch kernel's own occupancy (its summed LDS, its registers);
         * otherwise each launch goes out alone, as it was admitted */
        if (fn && resident && total > cap) {
            if (hipb.verbose)
                fprintf(stderr, "tinyhvm-hip: batch of %u launches: %u workgroups exceed what the GPU holds at once "
                        "(%u): launched one by one\n", HB.n, total, cap);
            fn = NULL;
        }
        if (fn) {
            void *pv[HB_MAX * CO_MAX_PARAMS];
            for (u32 i = 0; i < HB.n; i++) np += hb_params(&HB.ent[i], pv + np);
            hipb_launch(fn, total, 1, 1, T, pv);
            hipb.n_batched += HB.n;
        } else {
            for (u32 i = 0; i < HB.n; i++) {
                void *pv[CO_MAX_PARAMS];
                hb_params(&HB.ent[i], pv);
                hipb_launch(HB.ent[i].fn, HB.ent[i].gx, HB.ent[i].gy, 1, HB.ent[i].co.threads, pv);
            }
        }
    }
    HB.n = 0;
    HB.seq = 0;
    HB.comb_used = 0;
    memset(HB.wg_used, 0, sizeof HB.wg_used);
    HB.flushing = 0;
    pool_release_deferred();
}

int hipb_holding(void) { return HB.n > 0; }

int hipb_held_buffer(u32 id) {
    for (u32 i = 0; i < HB.n; i++) {
        const HbEnt *h = &HB.ent[i];
        if (h->ch)
            for (u32 b = 0; b < h->ch_nb; b++)
                if (h->ch_bufs[b] == id) return 1;
        if (h->wg && window_group_uses(&HB.wg[h->wg - 1], id, 0)) return 1;
        if (h->wmax && (h->wmax_bufs[0] == id || h->wmax_bufs[1] == id)) return 1;
    }
    return 0;
}

void hipb_before_stream(void) {
    if (HB.n && !HB.flushing) hb_flush();
}

void hipb_before_copy(const void *dst, u64 bytes) {
    if (!HB.n || HB.flushing) return;
    HbMem m;
    m.n = 0;
    hbm_add(&m, dst, bytes, 1);
    for (u32 i = 0; i < HB.n; i++)
        if (hbm_clash(&m, &HB.ent[i].m)) {
            hb_flush();
            return;
        }
}

/* whether a held launch may be a step of a held sequence */
static int hb_seq_eligible(const HbEnt *h) {
    if (hipb.no_seq || h->solo || h->resident || !h->co.src || h->gx * h->gy > HB_SEQ_MAX_BLOCKS ||
        h->co.threads == 0 || h->co.threads > HB_SEQ_THREADS || h->co.threads % 64u)
        return 0;
    /* no workgroup barriers or LDS of its own: then the sequence's barriers
     * are the only ones, and every wave reaches each of them (a wave whose
     * lanes leave a program early goes on to the barrier after it) */
    return h->co.no_sync;
}

/* whether h may follow the held launches as a new step of a sequence */
static int hb_seq_join(const HbEnt *h) {
    if (HB.n == 0 || HB.n >= HB_MAX || !hb_seq_eligible(h)) return 0;
    u32 lds = h->co.lds;
    for (u32 i = 0; i < HB.n; i++) {
        const HbEnt *o = &HB.ent[i];
        if (!hb_seq_eligible(o)) return 0;
        int seen = o->co.id == h->co.id;
        for (u32 j = 0; j < i && !seen; j++) seen = HB.ent[j].co.id == o->co.id;
        if (!seen) lds += o->co.lds;
    }
    return lds <= HB_MAX_LDS;
}

/* why h cannot join the held launches as they are (NULL: it can) */
static const char *hb_joins(const HbEnt *h) {
    if (HB.n >= HB_MAX) return "batch full";
    if (h->solo || (HB.n && HB.ent[0].solo)) return "held alone";
    u32 T = h->co.threads, lds = h->co.lds, blocks = h->gx * h->gy;
    int resident = h->resident;
    /* the batch kernel holds no more waves at once than its most demanding
     * program's kernel does (the exact count is checked when it is built) */
    u32 cap = h->co.cap_waves ? h->co.cap_waves : hipb_resident_waves();
    for (u32 i = 0; i < HB.n; i++) {
        const HbEnt *o = &HB.ent[i];
        if (hbm_clash(&h->m, &o->m)) return "memory";
        if (o->co.threads > T) T = o->co.threads;
        lds += o->co.lds;
        blocks += o->gx * o->gy;
        resident |= o->resident;
        const u32 c = o->co.cap_waves ? o->co.cap_waves : hipb_resident_waves();
        if (c < cap) cap = c;
    }
    if (lds > HB_MAX_LDS) return "LDS";
    if ((u64)blocks * T >= (1ull << 32)) return "grid size";
    if (resident && (u64)blocks * (T / 64u) > cap) return "residency";
    return NULL;
}

static int hb_hold(const CoForm *cf, hipFunction_t fn, u32 gx, u32 gy, void *const *params, const HbMem *m,
                   int resident, int comb_param, u64 comb_words, int solo);

int hipb_hold(const CoForm *cf, hipFunction_t fn, u32 gx, u32 gy, void *const *params, const HbMem *m,
              int resident, int comb_param, u64 comb_words) {
    return hb_hold(cf, fn, gx, gy, params, m, resident, comb_param, comb_words, 0);
}

int hipb_hold_solo(const CoForm *cf, hipFunction_t fn, u32 gx, u32 gy, void *const *params, const HbMem *m) {
    if (hipb.no_fuse) return 0;
    return hb_hold(cf, fn, gx, gy, params, m, 0, -1, 0, 1);
}

/* A chainable generated program (chain.c) of any grid size: held (and batched like
 * the small ones) so that a consumer of its output can fuse after it. */
static int hb_hold_large(const CoForm *cf, hipFunction_t fn, u32 gx, u32 gy, void *const *params, const HbMem *m) {
    if (hipb.no_fuse) return 0;
    return hb_hold(cf, fn, gx, gy, params, m, 0, -1, 0, 2);
}

int hipb_hold_large(const CoForm *cf, hipFunction_t fn, u32 gx, u32 gy, void *const *params, const HbMem *m,
                    int resident, int comb_param, u64 comb_words) {
    if (hipb.no_fuse) return 0;
    return hb_hold(cf, fn, gx, gy, params, m, resident, comb_param, comb_words, 2);
}

static int hb_hold(const CoForm *cf, hipFunction_t fn, u32 gx, u32 gy, void *const *params, const HbMem *m,
                   int resident, int comb_param, u64 comb_words, int solo) {
    if (!cf || !cf->src || hipb.no_batch || hipb.noalloc || hipb.sync_each || HB.flushing) return 0;
    if (gx == 0 || gy == 0 || (!solo && (u64)gx * gy > HB_MAX_BLOCKS) || (u64)gx * gy >= (1ull << 31) ||
        cf->threads == 0 || cf->threads % 64u ||
        cf->threads > 1024u || comb_words > COMB_SLOTS || (comb_param >= 0 && ((u32)comb_param >= cf->np ||
        cf->psz[comb_param] != 8)))
        return 0;
    HbEnt tmp, *h = &tmp;
    h->co = *cf;
    h->fz_key = 0;
    h->fz_serial = h->fz_out = 0;
    h->solo = solo == 1;
    h->ch = NULL;
    h->ch_nb = 0;
    h->wg = 0;
    h->wmax = NULL;
    h->hid = ++HB.next_hid;
    h->fn = fn;
    h->gx = gx;
    h->gy = gy;
    h->m = *m;
    h->resident = resident;
    u32 off = 0;
    for (u32 j = 0; j < cf->np; j++) {
        off = hb_arg_off(off, cf->psz[j]);
        if (off + cf->psz[j] > HB_ARG_BYTES) return 0;
        memcpy(h->args + off, params[j], cf->psz[j]);
        off += cf->psz[j];
    }
    h->seq_start = 0;
    const char *why = hb_joins(h);
    if (!why && HB.comb_used + comb_words > COMB_SLOTS) why = "combine area";
    if (!why && HB.seq && !hb_seq_join(h)) why = "sequence";
    if (why && strcmp(why, "memory") == 0 && comb_param < 0 && hb_seq_join(h)) {
        /* depends on a held launch: the next step of a held sequence */
        h->seq_start = 1;
        HB.seq = 1;
        why = NULL;
    }
    if (why) {
        if (hipb.verbose && HB.n)
            fprintf(stderr, "tinyhvm-hip: %s does not join %u held launches: %s\n", cf->name, HB.n, why);
        hb_flush();
    }
    if (comb_param >= 0) {
        /* its own slice of the combine area: after the held launches' slices */
        u32 o = 0;
        for (u32 j = 0; j < (u32)comb_param; j++) o = hb_arg_off(o, cf->psz[j]) + cf->psz[j];
        o = hb_arg_off(o, 8);
        unsigned long long *base;
        memcpy(&base, h->args + o, 8);
        base += HB.comb_used;
        memcpy(h->args + o, &base, 8);
        HB.comb_used += comb_words;
    }
    HB.ent[HB.n++] = *h;
    return 1;
}

void hipb_hold_tag(u64 key, u32 serial, u32 out_buf) {
    if (!HB.n) return;
    HbEnt *h = &HB.ent[HB.n - 1];
    h->fz_key = key;
    h->fz_serial = serial;
    h->fz_out = out_buf;
}

/* Marks the launch just held as the chainable program ch over buffers
 * (out_buf, leaf_bufs) that the next elementwise dispatch may fuse after. */
static void hb_hold_chain(const ChainInfo *ch, u32 out_buf, const u32 *leaf_bufs, u32 n_leaves) {
    if (!HB.n || !ch || n_leaves < ch->n_leaves) return;
    HbEnt *h = &HB.ent[HB.n - 1];
    h->ch = ch;
    h->ch_nb = ch->n_leaves + 1;
    h->ch_bufs[0] = out_buf;
    memcpy(h->ch_bufs + 1, leaf_bufs, ch->n_leaves * sizeof(u32));
    h->ch_seq = pool_write_clock();
}

/* The upload kernel: 16 bytes per lane from device-readable host memory,
 * the tail bytes by the first workgroup's lanes. Compiled once. */
static struct { hipModule_t mod; hipFunction_t fn; CoForm co; } UPK;

static const char UPLOAD_SRC[] =
    "extern \"C\" __global__ __launch_bounds__(256) void thvm_upload(char* dst, const char* src, u32 n16, u32 n) {\n"
    "  const u32 i = blockIdx.x * 256u + threadIdx.x;\n"
    "  if (i < n16) ((uint4*)dst)[i] = ((const uint4*)src)[i];\n"
    "  if (blockIdx.x == 0u && threadIdx.x < (n & 15u)) dst[n16 * 16u + threadIdx.x] = src[n16 * 16u + threadIdx.x];\n"
    "}\n";

/* prelude + the upload kernel (malloc'd) */
static char *upload_source(void) {
    const char *pre = kgen_prelude();
    char *src = malloc(strlen(pre) + sizeof UPLOAD_SRC + 2);
    if (src) sprintf(src, "%s\n%s", pre, UPLOAD_SRC);
    return src;
}

int hipb_hold_upload(void *dst, u64 dst_bytes, const void *src_dev, u64 bytes) {
    if (hipb.no_batch || hipb.noalloc || hipb.sync_each || HB.flushing || !hipb.initialized || !dst || !src_dev ||
        bytes == 0 || bytes > dst_bytes || bytes > 0xFFFFFFFFull || ((uintptr_t)dst & 15u) || ((uintptr_t)src_dev & 15u))
        return 0;
    /* a launch held for a fused epilogue joins no batch: the copy then goes on
     * the stream ahead of it, as before */
    if ((HB.n && HB.ent[0].solo) || !UPK.fn) return 0;
    const u32 n16 = (u32)(bytes / 16u), n = (u32)bytes;
    u32 gx = (n16 + 255u) / 256u;
    if (gx == 0) gx = 1;
    void *d = dst;
    const void *sp = src_dev;
    u32 a = n16, b = n;
    void *params[] = {&d, &sp, &a, &b};
    HbMem m;
    m.n = 0;
    hbm_add(&m, dst, dst_bytes, 1);
    if (!hipb_hold(&UPK.co, UPK.fn, gx, 1, params, &m, 0, -1, 0)) return 0;
    hipb.n_upload_held++;
    return 1;
}

/* at backend init (a module cannot be set up inside a graph capture);
 * without it uploads are copies */
static void upload_prepare(void) {
    if (UPK.fn || hipb.no_batch || hipb.rtc_fail) return;
    char *src = upload_source();
    char err[256] = {0};
    if (!src) return;
    /* backend machinery, not a dispatched program: not in the compile count */
    const u64 n_compile = hipb.n_compile;
    const int built = rtc_build_module(src, &UPK.mod, err, sizeof err);
    hipb.n_compile = n_compile;
    if (built) {
        if (hipModuleGetFunction(&UPK.fn, UPK.mod, "thvm_upload") != hipSuccess ||
            !co_form_make(&UPK.co, src, "thvm_upload", 256, UPK.fn)) {
            (void)hipGetLastError();
            HIPB_CHECK(hipModuleUnload(UPK.mod));
            co_form_free(&UPK.co);
            UPK.fn = NULL;
        }
    } else if (hipb.verbose) {
        fprintf(stderr, "tinyhvm-hip: no upload kernel: %s\n", err);
    }
    free(src);
}

static void upload_release(void) {
    if (UPK.fn) HIPB_CHECK(hipModuleUnload(UPK.mod));
    co_form_free(&UPK.co);
    memset(&UPK, 0, sizeof UPK);
}

/* Marks the launch just held as a run sum: a group of one that run sums of
 * the same shape and consumers of its output may join (hb_try_group). */
void hipb_hold_tag_sum(const void *we, u32 out_buf, const u32 *leaf_bufs, u32 n_leaves) {
    if (!HB.n || hipb.no_fuse) return;
    HbEnt *h = &HB.ent[HB.n - 1];
    for (u32 i = 0; i < HB_MAX; i++) {
        if (HB.wg_used[i]) continue;
        if (window_group_of_sum(&HB.wg[i], we, out_buf, leaf_bufs, n_leaves)) {
            HB.wg_used[i] = 1;
            h->wg = i + 1;
        }
        return;
    }
}

/* Marks the launch just held as a window max that a run sum over its output
 * may take in. */
void hipb_hold_tag_wmax(const void *we, u32 out_buf, u32 in_buf) {
    if (!HB.n || hipb.no_fuse) return;
    HbEnt *h = &HB.ent[HB.n - 1];
    h->wmax = we;
    h->wmax_bufs[0] = out_buf;
    h->wmax_bufs[1] = in_buf;
    h->ch_seq = pool_write_clock();
}

static i32 hb_find(u64 hid) {
    for (u32 i = 0; i < HB.n; i++)
        if (HB.ent[i].hid == hid) return (i32)i;
    return -1;
}

/* Points held launch h at kernel fn (form cf) with these parameters, in
 * place: its own slice of the combine area after the others'. Returns 0 if
 * they do not fit (h unchanged). */
static int hb_set_launch(HbEnt *h, const CoForm *cf, hipFunction_t fn, u32 gx, u32 gy, void *const *params,
                         int resident, int comb_param, u64 comb_words) {
    if (!cf || !cf->src || gx == 0 || gy == 0 || cf->np == 0 || comb_words > COMB_SLOTS ||
        HB.comb_used + comb_words > COMB_SLOTS || (comb_param >= 0 && ((u32)comb_param >= cf->np ||
        cf->psz[comb_param] != 8)))
        return 0;
    u8 args[HB_ARG_BYTES];
    u32 off = 0;
    for (u32 j = 0; j < cf->np; j++) {
        off = hb_arg_off(off, cf->psz[j]);
        if (off + cf->psz[j] > HB_ARG_BYTES) return 0;
        memcpy(args + off, params[j], cf->psz[j]);
        if ((i32)j == comb_param) {
            unsigned long long *base;
            memcpy(&base, args + off, 8);
            base += HB.comb_used;
            memcpy(args + off, &base, 8);
        }
        off += cf->psz[j];
    }
    if (comb_param >= 0) HB.comb_used += comb_words;
    memcpy(h->args, args, sizeof args);
    h->co = *cf;
    h->fn = fn;
    h->gx = gx;
    h->gy = gy;
    h->resident = resident;
    h->solo = 0;
    return 1;
}

/* Run-sum groups (window.c): a run sum that has the shape of a held group's
 * sums joins it, or takes in the held elementwise program or window max
 * whose output it reads; an elementwise consumer of a held group's output
 * becomes one of its tails. The held launch is rebuilt in place as the
 * group's kernel. Only when the new program's memory meets no other held
 * launch, and a taken-in producer's buffers are unwritten by the host since
 * it was held. Returns 1 when the dispatch joined. */
static int hb_try_group(u32 out_buf, const u32 *leaf_bufs, u32 n_leaves, const UOpKernel *k) {
    static WinGroup g;
    if (!HB.n || hipb.no_fuse || hipb.no_window || hipb.noalloc || hipb.sync_each || HB.flushing || !k ||
        k->n_leaves == 0 || k->n_leaves > n_leaves || k->n_leaves > WG_MAX_LEAVES || !pool_ptr(out_buf))
        return 0;
    int loop = 0;
    for (u32 i = 0; i < k->n_ops && !loop; i++) loop = k->ops[i].type == KOP_RANGE;
    i32 at = -1;
    if (!loop) {
        for (u32 i = HB.n; i-- > 0 && at < 0;) {
            if (!HB.ent[i].wg) continue;
            g = HB.wg[HB.ent[i].wg - 1];
            if (window_group_add_tail(&g, k, out_buf, leaf_bufs, n_leaves)) at = (i32)i;
        }
    } else {
        const void *we = window_sum_entry(k);
        if (!we) return 0;
        for (u32 i = HB.n; i-- > 0 && at < 0;) {
            if (!HB.ent[i].wg) continue;
            g = HB.wg[HB.ent[i].wg - 1];
            if (window_group_add_sum(&g, we, out_buf, leaf_bufs, n_leaves)) at = (i32)i;
        }
        for (u32 i = HB.n; i-- > 0 && at < 0;) {
            const HbEnt *h = &HB.ent[i];
            int fresh = 1;
            if (h->ch) {
                for (u32 b = 0; b < h->ch_nb; b++) {
                    const HipbBuf *pb = h->ch_bufs[b] ? pool_get(h->ch_bufs[b]) : NULL;
                    if (h->ch_bufs[b] && (!pb || !pb->ptr || pb->wseq > h->ch_seq)) fresh = 0;
                }
                if (fresh && window_group_of_chain(&g, h->ch, h->ch_bufs) &&
                    window_group_add_sum(&g, we, out_buf, leaf_bufs, n_leaves))
                    at = (i32)i;
            } else if (h->wmax) {
                for (u32 b = 0; b < 2; b++) {
                    const HipbBuf *pb = pool_get(h->wmax_bufs[b]);
                    if (!pb || !pb->ptr || pb->wseq > h->ch_seq) fresh = 0;
                }
                if (fresh && window_group_of_wmax(&g, h->wmax, h->wmax_bufs[0], h->wmax_bufs[1]) &&
                    window_group_add_sum(&g, we, out_buf, leaf_bufs, n_leaves))
                    at = (i32)i;
            }
        }
    }
    if (at < 0 || !window_group_build(&g)) return 0;
    HbMem m;
    window_group_mem(&g, &m);
    for (u32 i = 0; i < HB.n; i++)
        if ((i32)i != at && hbm_clash(&m, &HB.ent[i].m)) return 0;
    /* the new program's inputs current on the device (a copy that meets a
     * held launch issues the held launches, and then nothing joins) */
    const u64 hid = HB.ent[at].hid;
    if (loop) {
        for (u32 j = 0; j < k->n_leaves; j++) pool_sync_device(leaf_bufs[j]);
    } else {
        const u64 reads = window_group_tail_reads(&g, g.n_tail - 1);
        for (u32 j = 0; j < k->n_leaves; j++)
            if (j >= 64 || ((reads >> j) & 1u)) pool_sync_device(leaf_bufs[j]);
    }
    at = hb_find(hid);
    if (at < 0) return 0;
    HbEnt *h = &HB.ent[at];
    WgArgs a;
    void *params[CO_MAX_PARAMS + 8];
    const u32 np = window_group_params(&g, &a, params);
    if (np != g.co->np || !hb_set_launch(h, g.co, g.fn, g.grid, 1, params, g.resident, g.resident ? (int)np - 1 : -1,
                                         g.comb_words))
        return 0;
    h->m = m;
    h->ch = NULL;
    h->ch_nb = 0;
    h->wmax = NULL;
    h->fz_key = 0;
    if (!h->wg) {
        for (u32 i = 0; i < HB_MAX && !h->wg; i++)
            if (!HB.wg_used[i]) {
                HB.wg_used[i] = 1;
                h->wg = i + 1;
            }
    }
    if (h->wg) HB.wg[h->wg - 1] = g;
    hipb.n_fused++;
    return 1;
}

static u32 elem_count(u32 id, u32 dtype);

/* An elementwise dispatch that reads the output of a held contraction runs
 * as that launch's fused epilogue (dense_epilogue) instead of a launch of
 * its own: its buffers are appended to the held launch's parameters and its
 * memory to the launch's. Only when it touches nothing another held launch
 * writes or reads, except the contraction's output, which it reads at its
 * own index only; writes neither that output nor its own inputs. Returns 1
 * when it was fused. */
static int hb_try_epilogue(u32 out_buf, const u32 *leaf_bufs, u32 n_leaves, const UOpKernel *k) {
    if (!HB.n || hipb.no_fuse || hipb.noalloc || hipb.sync_each || HB.flushing || !k ||
        k->n_leaves > FUSE_MAX_LEAVES || n_leaves < k->n_leaves)
        return 0;
    HbEnt *e = NULL;
    u32 o_leaf = 0;
    for (u32 i = HB.n; i-- > 0 && !e;) {
        if (!HB.ent[i].fz_key) continue;
        for (u32 j = 0; j < k->n_leaves; j++)
            if (leaf_bufs[j] == HB.ent[i].fz_out) {
                e = &HB.ent[i];
                o_leaf = j + 1;
                break;
            }
    }
    if (!e || out_buf == e->fz_out || !pool_ptr(out_buf)) return 0;
    for (u32 j = 0; j < k->n_leaves; j++)
        if (leaf_bufs[j] == out_buf || (leaf_bufs[j] && !pool_ptr(leaf_bufs[j]))) return 0;
    const u64 fz = e->fz_key;
    const u32 fzs = e->fz_serial, fzo = e->fz_out;
    hipFunction_t fn;
    CoForm co;
    KGenScalars sc;
    if (!dense_epilogue(fz, fzs, k, o_leaf, &fn, &co, &sc)) return 0;
    /* loads at a constant index of host-held leaves take their value as an
     * argument (sm bit j set); a leaf read only that way is not uploaded */
    u32 sm = 0;
    float sv[KGEN_MAX_SCALARS];
    for (u32 j = 0; j < sc.n; j++) {
        const u32 id = leaf_bufs[sc.leaf[j]];
        sv[j] = 0.0f;
        if (id && id != out_buf && pool_host_value(id, k->leaf_dtypes[sc.leaf[j]], sc.index[j], &sv[j])) sm |= 1u << j;
    }
    /* its other inputs current on the device (the epilogue reads them from
     * memory): pending host writes are copied on the stream ahead of the
     * held launches, which do not read them (if one does, it goes out first
     * and nothing fuses) */
    for (u32 j = 0; j < k->n_leaves; j++) {
        if (leaf_bufs[j] == fzo) continue;
        int inline_only = 0, other = 0;
        for (u32 q = 0; q < k->n_ops; q++)
            if (k->ops[q].type == KOP_LOAD && k->ops[q].imm.u == j + 1) {
                int hit = 0;
                for (u32 t = 0; t < sc.n; t++)
                    hit |= sc.leaf[t] == j && ((sm >> t) & 1u) && k->ops[k->ops[q].arg[0]].imm.u == sc.index[t] &&
                           k->ops[k->ops[q].arg[0]].type == KOP_CONST_U;
                if (hit) inline_only = 1;
                else other = 1;
            }
        if (!inline_only || other) pool_sync_device(leaf_bufs[j]);
    }
    e = NULL;
    for (u32 i = 0; i < HB.n && !e; i++)
        if (HB.ent[i].fz_key == fz && HB.ent[i].fz_serial == fzs && HB.ent[i].fz_out == fzo) e = &HB.ent[i];
    if (!e) return 0;
    HbMem m;
    m.n = 0;
    hbm_add(&m, pool_ptr(out_buf), pool_bytes(out_buf), 1);
    for (u32 j = 0; j < k->n_leaves; j++)
        if (leaf_bufs[j] != e->fz_out) hbm_add(&m, pool_ptr(leaf_bufs[j]), pool_bytes(leaf_bufs[j]), 0);
    for (u32 i = 0; i < HB.n; i++)
        if (hbm_clash(&m, &HB.ent[i].m)) return 0;
    /* the consumer's buffers (the generated kernel's p<b>, c<b>) after the
     * contraction's parameters */
    u32 off = 0;
    for (u32 j = 0; j < e->co.np; j++) off = hb_arg_off(off, e->co.psz[j]) + e->co.psz[j];
    const u32 nb = k->n_leaves + 1;
    if (hb_arg_off(off, 8) + 8u * nb + 4u * nb + (sc.n ? 4u + 4u * sc.n : 0u) > HB_ARG_BYTES) return 0;
    for (u32 b = 0; b < nb; b++) {
        void *p = b == 0 ? pool_ptr(out_buf) : leaf_bufs[b - 1] ? pool_ptr(leaf_bufs[b - 1]) : hipb.dummy;
        off = hb_arg_off(off, 8);
        memcpy(e->args + off, &p, 8);
        off += 8;
    }
    for (u32 b = 0; b < nb; b++) {
        const u32 c = b == 0 ? elem_count(out_buf, k->out_dtype)
                             : leaf_bufs[b - 1] ? elem_count(leaf_bufs[b - 1], k->leaf_dtypes[b - 1]) : 0u;
        off = hb_arg_off(off, 4);
        memcpy(e->args + off, &c, 4);
        off += 4;
    }
    if (sc.n) {
        off = hb_arg_off(off, 4);
        memcpy(e->args + off, &sm, 4);
        off += 4;
        for (u32 j = 0; j < sc.n; j++) {
            memcpy(e->args + off, &sv[j], 4);
            off += 4;
        }
    }
    e->fn = fn;
    e->co = co;
    for (u32 r = 0; r < m.n; r++) {
        void *lo = (void *)(uintptr_t)m.lo[r];
        hbm_add(&e->m, lo, m.hi[r] - m.lo[r], m.wr[r]);
    }
    e->fz_key = 0;
    hipb.n_fused++;
    return 1;
}

static void hb_release(void) {
    HB.n = 0;
    HB.seq = 0;
    for (u32 i = 0; i < HB.ncache; i++) HIPB_CHECK(hipModuleUnload(HB.cache[i].mod));
    HB.ncache = 0;
}

static int env_flag(const char *name) {
    const char *v = getenv(name);
    return v && v[0] && strcmp(v, "0") != 0;
}

/* Matrix-core routing knobs (read at init, or before the first device-free
 * analysis call). */
static void read_dense_env(void) {
    hipb.dense_force = env_flag("THVM_HIP_DENSE_FORCE");
    hipb.dense_nosep = env_flag("THVM_HIP_DENSE_NOSEP");
    hipb.dense_nokperm = env_flag("THVM_HIP_DENSE_NOKPERM");
    hipb.dense_novec = env_flag("THVM_HIP_DENSE_NOVEC");
    hipb.dense_noswap = env_flag("THVM_HIP_DENSE_NOSWAP");
    hipb.dense_nopack = env_flag("THVM_HIP_DENSE_NOPACK");
    hipb.dense_noskinny = env_flag("THVM_HIP_DENSE_NOSKINNY");
    hipb.dense_noskinny_blocks = env_flag("THVM_HIP_DENSE_NOSKBLK");
    hipb.dense_nored = env_flag("THVM_HIP_DENSE_NORED");
    hipb.dense_nocomb = env_flag("THVM_HIP_DENSE_NOCOMB");
    hipb.dense_nowave = env_flag("THVM_HIP_DENSE_NOWAVE");
    hipb.dense_notail = env_flag("THVM_HIP_DENSE_NOTAIL");
    {
        const char *ts = getenv("THVM_HIP_WAVE_TAIL_S");
        const long v = ts ? strtol(ts, NULL, 10) : 0;
        hipb.wave_tail_s = (v == 2 || v == 4 || v == 8) ? (u32)v : 0u;
    }
    hipb.no_fuse = env_flag("THVM_HIP_NO_FUSE");
    hipb.host_profile = env_flag("THVM_HIP_HOST_PROFILE");
    hipb.dense_pack = env_flag("THVM_HIP_DENSE_PACK");
    const char *e = getenv("THVM_HIP_DENSE_SPLITS");
    hipb.dense_splits = e ? (u32)atoi(e) : 0;
    e = getenv("THVM_HIP_GEMM_PAD");
    hipb.gemm_pad_k = e ? (u32)atoi(e) : 0;
    hipb.gemm_pad_k_set = e && hipb.gemm_pad_k <= 8;
    e = getenv("THVM_HIP_GEMM_BK");
    hipb.gemm_bk = e ? (u32)atoi(e) : 0;
    if (hipb.gemm_bk != 16 && hipb.gemm_bk != 32 && hipb.gemm_bk != 64) hipb.gemm_bk = 0;
    e = getenv("THVM_HIP_DIRECT_WAVES");
    hipb.direct_waves = e ? (u32)atoi(e) : 0;
    if (hipb.direct_waves != 4 && hipb.direct_waves != 8 && hipb.direct_waves != 16) hipb.direct_waves = 0;
    e = getenv("THVM_HIP_DIRECT_MIN_CHUNK");
    hipb.direct_min_chunk = e ? (u32)atoi(e) : 0;
    if (hipb.direct_min_chunk > 65536) hipb.direct_min_chunk = 0;
    e = getenv("THVM_HIP_GEMM_PRIO");
    hipb.gemm_prio = e ? (u32)atoi(e) : 0;
    if (hipb.gemm_prio > 2) hipb.gemm_prio = 0;
    e = getenv("THVM_HIP_GEMM_DEPTH");
    hipb.gemm_depth = e ? (u32)atoi(e) : 0;
    if (hipb.gemm_depth > 2) hipb.gemm_depth = 0;
    e = getenv("THVM_HIP_DENSE_TILE");
    hipb.dense_tile = e ? (u32)atoi(e) : 0;
    if (hipb.dense_tile > 11) hipb.dense_tile = 0;
}

u32 hipb_resident_waves(void) { return hipb.resident_waves ? hipb.resident_waves : 256u * SINGLE_PASS_WAVES_PER_CU; }

/* After a wait on the stream: a single-pass combine that gave up waiting
 * for a partial (its output took a NaN) set the give-up word. It is
 * counted, printed, and reported by the next thvm_hip_synchronize; the
 * combine area is cleared again, since a partial published after its
 * taker gave up would otherwise be taken by a later launch. */
static void comb_check(void) {
    if (!hipb.comb_err_host || !*(volatile u32 *)hipb.comb_err_host) return;
    *(volatile u32 *)hipb.comb_err_host = 0;
    hipb.n_comb_gaveup++;
    hipb.comb_gaveup_pending = 1;
    fprintf(stderr, "tinyhvm-hip: a single-pass combine gave up waiting for a partial sum; "
                    "its output holds a NaN\n");
    hipFunction_t fill = rtc_static_fn("thvm_fill_u32");
    if (fill && hipb.comb_slots) {
        u32 n1 = COMB_SLOTS * 2, zero = 0;
        void *a1[] = {&hipb.comb_slots, &n1, &zero};
        hipb_launch(fill, (n1 + 255) / 256, 1, 1, 256, a1);
    }
}

hipError_t hipb_stream_wait(void) {
    hipb_before_stream();
    hipb.n_stream_sync++;
    const hipError_t e = hipStreamSynchronize(hipb.stream);
    if (e == hipSuccess) comb_check();
    return e;
}

static void hb_shutdown(void);
static void graphs_release_all(void);

/* Process exit without a shutdown call (an engine program that never calls
 * thvm_free, a script that just ends): the backend's stream, modules, graphs
 * and memory are released here, while the HIP runtime is still up. The
 * handler is registered after the runtime initialised, so it runs before the
 * runtime's own exit-time teardown. */
static void hb_atexit(void) {
    if (hipb.initialized) hb_shutdown();
}

static int hb_init(void) {
    static int atexit_done = 0;
    if (hipb.initialized) return 0;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        fprintf(stderr, "tinyhvm-hip: no HIP device\n");
        return -1;
    }
    memset(&hipb, 0, sizeof(hipb));
    kgen_prelude_reset();
    const char *dev = getenv("THVM_HIP_DEVICE");
    hipb.device = dev ? atoi(dev) : 0;
    if (hipSetDevice(hipb.device) != hipSuccess) {
        fprintf(stderr, "tinyhvm-hip: hipSetDevice(%d) failed\n", hipb.device);
        return -1;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, hipb.device) == hipSuccess) {
        if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
            fprintf(stderr, "tinyhvm-hip: device is %s; kernels are built for gfx950\n", prop.gcnArchName);
            return -1;
        }
        if (prop.multiProcessorCount > 0) {
            hipb.resident_waves = (u32)prop.multiProcessorCount * SINGLE_PASS_WAVES_PER_CU;
            hipb.n_cu = (u32)prop.multiProcessorCount;
        }
    }
    if (hipStreamCreateWithFlags(&hipb.stream, hipStreamNonBlocking) != hipSuccess) return -1;
    if (hipStreamCreateWithFlags(&hipb.setup_stream, hipStreamNonBlocking) != hipSuccess) return -1;
    hipb.sync_each = env_flag("THVM_HIP_SYNC");
    hipb.no_batch = env_flag("THVM_HIP_NO_BATCH");
    hipb.no_seq = env_flag("THVM_HIP_NO_SEQ");
    hipb.dump_src = env_flag("THVM_HIP_DUMP");
    hipb.no_dense = env_flag("THVM_HIP_NO_DENSE");
    hipb.no_window = env_flag("THVM_HIP_NO_WINDOW");
    hipb.verbose = env_flag("THVM_HIP_VERBOSE");
    hipb.force_interp = env_flag("THVM_HIP_INTERP");
    hipb.rtc_fail = env_flag("THVM_HIP_RTC_FAIL");
    read_dense_env();
    if (pool_init() != 0) return -1;
    hipb.dummy = pool_block_get(256, &hipb.dummy_cap);
    if (!hipb.dummy || hipMemset(hipb.dummy, 0, 256) != hipSuccess) return -1;
    /* the word a single-pass combine sets when it gives up waiting: host
     * memory the GPU writes, read after each wait on the stream */
    if (hipHostMalloc((void **)&hipb.comb_err_host, 256, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess ||
        hipHostGetDevicePointer((void **)&hipb.comb_err_dev, hipb.comb_err_host, 0) != hipSuccess) {
        (void)hipGetLastError();
        fprintf(stderr, "tinyhvm-hip: no host-mapped word for combine reports\n");
        if (hipb.comb_err_host) HIPB_CHECK(hipHostFree(hipb.comb_err_host));
        hipb.comb_err_host = NULL;
        hipb.comb_err_dev = NULL;
    } else {
        *(volatile u32 *)hipb.comb_err_host = 0;
    }
    if (rtc_init() != 0) return -1;
    /* the single-pass combine area, zeroed once by a kernel */
    {
        u64 c1 = 0;
        hipb.comb_slots = pool_block_get((u64)COMB_SLOTS * 8, &c1);
        hipFunction_t fill = rtc_static_fn("thvm_fill_u32");
        if (!hipb.comb_slots || !fill) return -1;
        u32 n1 = COMB_SLOTS * 2, zero = 0;
        void *a1[] = {&hipb.comb_slots, &n1, &zero};
        hipb_launch(fill, (n1 + 255) / 256, 1, 1, 256, a1);
        if (hipb_stream_wait() != hipSuccess) return -1;
    }
    upload_prepare();
    /* the static workspace of the no-allocation entry point, on this device */
    if (thvm_noalloc_scratch_init(hipb.device) == 0) hipb.noalloc_scratch = thvm_noalloc_scratch_ptr(hipb.device);
    else fprintf(stderr, "tinyhvm-hip: static workspace unavailable; dispatch without allocation is off\n");
    hipb.initialized = 1;
    if (!atexit_done) {
        atexit(hb_atexit);
        atexit_done = 1;
    }
    return 0;
}

/* Idempotent: every graph, module, workspace and buffer goes, then the
 * stream. */
static void hb_shutdown(void) {
    if (!hipb.initialized) return;
    copyq_flush();
    HIPB_CHECK(hipb_stream_wait());
    graphs_release_all();
    dense_shutdown();
    window_shutdown();
    hb_release();
    upload_release();
    rtc_shutdown();
    scratch_release(&red_ws);
    pool_block_put(hipb.comb_slots, (u64)COMB_SLOTS * 8);
    hipb.comb_slots = NULL;
    pool_block_put(hipb.dummy, hipb.dummy_cap);
    hipb.dummy = NULL;
    if (hipb.comb_err_host) HIPB_CHECK(hipHostFree(hipb.comb_err_host));
    hipb.comb_err_host = NULL;
    hipb.comb_err_dev = NULL;
    pool_shutdown();
    HIPB_CHECK(hipStreamDestroy(hipb.stream));
    HIPB_CHECK(hipStreamDestroy(hipb.setup_stream));
    hipb.initialized = 0;
}

u64 hipb_hp_now(void) {
    if (!hipb.host_profile) return 0;
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (u64)t.tv_sec * 1000000000ull + (u64)t.tv_nsec;
}

void hipb_hp_add(int cat, u64 t0) {
    if (!hipb.host_profile || cat < 0 || cat >= HP_N) return;
    hipb.hp_ns[cat] += hipb_hp_now() - t0;
    hipb.hp_calls[cat]++;
}

static u32 hb_buf_alloc(u64 bytes) {
    const u64 t0 = hipb_hp_now();
    const u32 id = pool_alloc(bytes);
    hipb_hp_add(HP_POOL, t0);
    return id;
}
static void hb_buf_free(u32 id) {
    const u64 t0 = hipb_hp_now();
    copyq_guard(id);
    pool_free(id);
    hipb_hp_add(HP_POOL, t0);
}
static void hb_buf_incref(u32 id) {
    const u64 t0 = hipb_hp_now();
    pool_incref(id);
    hipb_hp_add(HP_POOL, t0);
}
static void hb_buf_decref(u32 id) {
    const u64 t0 = hipb_hp_now();
    copyq_guard(id);
    pool_decref(id);
    hipb_hp_add(HP_POOL, t0);
}
static void hb_buf_write(u32 id, const void *data, u64 bytes) {
    const u64 t0 = hipb_hp_now();
    copyq_guard(id);
    pool_write(id, data, bytes);
    hipb_hp_add(HP_WRITE, t0);
}
static void hb_buf_read(u32 id, void *out, u64 bytes) { copyq_guard(id); pool_read(id, out, bytes, 0); }
static void hb_buf_read_nosync(u32 id, void *out, u64 bytes) { copyq_guard(id); pool_read(id, out, bytes, 1); }
static void hb_mem_checkpoint(u32 *ids, u32 n) { (void)ids; (void)n; }
static void hb_buf_mark_use(u32 id) { (void)id; }
static void hb_pool_reset(u32 keep) { copyq_flush(); hipb_before_stream(); pool_reset(keep); }
static void hb_pool_set_persistent(u32 max_buf) { pool_set_persistent(max_buf); }
static void hb_begin_batch(void) {}
static void hb_end_batch(void) {}

static u32 dtype_bytes(u32 dt) { return dt == DTYPE_F16 ? 2u : 4u; }

static u32 elem_count(u32 id, u32 dt) {
    u64 b = pool_bytes(id);
    u64 n = b / dtype_bytes(dt);
    return n > 0xFFFFFFFFull ? 0xFFFFFFFFu : (u32)n;
}

int hipb_launch(hipFunction_t fn, u32 gx, u32 gy, u32 gz, u32 bx, void **params) {
    hipb_before_stream();
    const u64 t0 = hipb_hp_now();
    hipError_t e = hipModuleLaunchKernel(fn, gx, gy, gz, bx, 1, 1, 0, hipb.stream, params, NULL);
    hipb_hp_add(HP_LAUNCH, t0);
    if (e != hipSuccess) {
        fprintf(stderr, "tinyhvm-hip: launch failed: %s\n", hipGetErrorString(e));
        return 0;
    }
    if (hipb.sync_each && !hipb.capturing) {
        e = hipStreamSynchronize(hipb.stream);
        if (e != hipSuccess) {
            fprintf(stderr, "tinyhvm-hip: kernel failed: %s\n", hipGetErrorString(e));
            return 0;
        }
    }
    return 1;
}

int hipb_launch_grid(hipFunction_t fn, u32 gx, u32 gy, u32 bx, void **params) {
    if ((u64)gx * bx >= (1ull << 32)) {
        fprintf(stderr, "tinyhvm-hip: grid of %u groups exceeds the launch limit\n", gx);
        return 0;
    }
    return hipb_launch(fn, gx, gy, 1, bx, params);
}

/* Grid for `blocks` workgroups of `bx` lanes: x holds up to 2^16 groups when
 * the work-item count would not fit 32 bits; the kernels fold y back in. */
static void grid_for(u64 blocks, u32 bx, u32 *gx, u32 *gy) {
    if (blocks * bx < (1ull << 32)) {
        *gx = (u32)blocks;
        *gy = 1;
    } else {
        *gx = 65536;
        *gy = (u32)((blocks + 65535) / 65536);
    }
}

static float *reduce_workspace(u64 bytes) { return scratch_reserve(&red_ws, bytes); }

static int kop_is_float(u32 t) {
    return t == KOP_CONST_F || t == KOP_LOAD || t == KOP_ALU || t == KOP_ACC_INIT || t == KOP_MASK;
}

/* The KOp interpreter (static kernel thvm_kop): the engine's CPU semantics,
 * one lane per gid, for a program that could not be compiled. A program
 * whose loops do not nest runs nothing, as on the reference
 * (src/backend/cpu/uop.c:118-155). */
static void interp_dispatch(u32 out_buf, const u32 *leaf_bufs, u32 n_leaves, const UOpKernel *k) {
    hipFunction_t fn = rtc_static_fn("thvm_kop");
    HipbBuf *ob = pool_get(out_buf);
    if (!fn || !ob || k->n_ops > KOP_MAX) return;
    for (u32 i = 0; i < n_leaves && i < FUSE_MAX_LEAVES; i++) pool_sync_device(leaf_bufs[i]);
    KopParams *P = calloc(1, sizeof *P);
    if (!P) return;
    u32 stack[KOP_MAX], sp = 0;
    for (u32 i = 0; i < k->n_ops; i++) {
        P->ops[i] = k->ops[i];
        P->ftype[i] = (u8)kop_is_float(k->ops[i].type);
        if (k->ops[i].type == KOP_RANGE) stack[sp++] = i;
        else if (k->ops[i].type == KOP_ENDRANGE) {
            if (sp == 0) { free(P); return; }
            u32 r = stack[--sp];
            P->pair[r] = (u16)i;
            P->pair[i] = (u16)r;
        }
    }
    if (sp != 0) { free(P); return; }
    P->n_ops = k->n_ops;
    P->out_ptr = (u64)(uintptr_t)ob->ptr;
    P->out_n = elem_count(out_buf, k->out_dtype);
    P->out_dtype = k->out_dtype;
    u32 nl = n_leaves < k->n_leaves ? n_leaves : k->n_leaves;
    if (nl > FUSE_MAX_LEAVES) nl = FUSE_MAX_LEAVES;
    P->n_leaves = nl;
    for (u32 i = 0; i < nl; i++) {
        void *lp = pool_ptr(leaf_bufs[i]);
        P->leaf_ptr[i] = (u64)(uintptr_t)lp;
        P->leaf_dtype[i] = k->leaf_dtypes[i];
        P->leaf_n[i] = lp ? elem_count(leaf_bufs[i], k->leaf_dtypes[i]) : 0u;
    }
    /* launch total as the reference counts it (u32 arithmetic) */
    P->total = k->local_size > 0 ? k->grid[0] : k->grid[0] * k->grid[1] * k->grid[2];
    u64 pcap = 0;
    void *dp = pool_block_get(sizeof *P, &pcap);
    if (!dp) { free(P); return; }
    pool_upload(dp, P, sizeof *P);
    const u32 chunk = 1u << 26;   /* gids per launch: 2^20 workgroups of 64 */
    for (u64 base = 0; base < P->total; base += chunk) {
        u32 b32 = (u32)base;
        u64 n = P->total - base < chunk ? P->total - base : chunk;
        void *params[] = {&dp, &b32};
        hipb_launch(fn, (u32)((n + 63) / 64), 1, 1, 64, params);
    }
    pool_block_put(dp, pcap);   /* stream order keeps the block alive for the launches above */
    pool_mark_device_write(out_buf);
    hipb.n_fallback++;
    free(P);
}

static void hb_dispatch_uop_kernel_(u32 out_buf, const u32 *leaf_bufs, u32 n_leaves, const UOpKernel *k);
static void hb_run_generated(KCacheEntry *e, u32 out_buf, const u32 *leaf_bufs, u32 n_leaves, const UOpKernel *k);
static u64 hb_inline_scalars(const KCacheEntry *e, u32 out_buf, const u32 *leaf_bufs, u32 n_leaves,
                             const UOpKernel *k, u32 *sm_out, float *sv);

/* A loop-free dispatch that reads the output of a held chainable program P
 * at its own gid runs fused after it (chain.c): P's held launch is taken
 * back and the merged program is dispatched in its place, which writes
 * both outputs. Only when every buffer of P is still live and unwritten by
 * the host since P was held (P's launch would have read the old contents),
 * and each output read is at least one launch long. The merged program
 * goes through the usual hold, so it waits behind held launches it
 * touches memory of and may take further consumers. Returns 1 when fused. */
static int hb_try_chain(u32 out_buf, const u32 *leaf_bufs, u32 n_leaves, const UOpKernel *k) {
    static UOpKernel M;
    static u32 mb[1 + FUSE_MAX_LEAVES];
    if (!HB.n || hipb.no_fuse || hipb.noalloc || hipb.sync_each || HB.flushing || !k || k->n_leaves > n_leaves ||
        k->n_leaves == 0 || k->n_leaves > FUSE_MAX_LEAVES)
        return 0;
    i32 at = -1;
    for (u32 i = HB.n; i-- > 0 && at < 0;) {
        const HbEnt *h = &HB.ent[i];
        if (!h->ch) continue;
        for (u32 s = 0; s < h->ch->n_st && at < 0; s++)
            for (u32 j = 0; j < k->n_leaves; j++)
                if (leaf_bufs[j] == h->ch_bufs[h->ch->st_slot[s]]) { at = (i32)i; break; }
    }
    if (at < 0) return 0;
    HbEnt *h = &HB.ent[at];
    const ChainInfo *ch = h->ch;
    for (u32 b = 0; b < h->ch_nb; b++) {
        const HipbBuf *pb = h->ch_bufs[b] ? pool_get(h->ch_bufs[b]) : NULL;
        if (h->ch_bufs[b] && (!pb || !pb->ptr || pb->wseq > h->ch_seq)) return 0;
    }
    for (u32 s = 0; s < ch->n_st; s++)
        if (elem_count(h->ch_bufs[ch->st_slot[s]], DTYPE_F32) < ch->total) return 0;
    if (!pool_ptr(out_buf) || !chain_merge(ch, h->ch_bufs, k, out_buf, leaf_bufs, n_leaves, &M, mb)) return 0;
    static u64 refused[64];   /* merged programs the generator or hipRTC refused */
    static u32 n_refused;
    const u64 key = uop_signature(&M);
    for (u32 i = 0; i < n_refused && i < 64; i++)
        if (refused[i] == key) return 0;
    KCacheEntry *e = rtc_lookup(key, &M);
    if (e) hipb.n_cache_hit++;
    else {
        e = rtc_compile_uop(key, &M);
        if (e && hipb.verbose)
            fprintf(stderr, "tinyhvm-hip: %s = %s + thvm_ew_%08x\n", e->name, h->co.name,
                    (u32)(uop_signature(k) & 0xFFFFFFFFu));
    }
    if (!e || e->splits > 1 || e->mode == KG_MODE_GROUP) {
        refused[n_refused++ % 64] = key;
        return 0;
    }
    /* the consumer's own inputs current on the device first: a copy that
     * overlaps a held launch issues it, and then nothing fuses (leaves the
     * merged program reads only as inline scalars need no copy) */
    const u32 tag[2] = {h->ch_bufs[0], (u32)h->ch_seq};
    {
        u32 sm;
        float sv[KGEN_MAX_SCALARS];
        const u64 only = hb_inline_scalars(e, mb[0], mb + 1, M.n_leaves, &M, &sm, sv);
        for (u32 j = 0; j < k->n_leaves; j++) {
            int skip = 0;
            for (u32 s2 = 0; s2 < M.n_leaves && s2 < 32; s2++)
                if (mb[1 + s2] == leaf_bufs[j] && ((only >> s2) & 1u)) skip = 1;
            if (!skip) pool_sync_device(leaf_bufs[j]);
        }
    }
    at = -1;
    for (u32 i = 0; i < HB.n && at < 0; i++)
        if (HB.ent[i].ch == ch && HB.ent[i].ch_bufs[0] == tag[0] && (u32)HB.ent[i].ch_seq == tag[1]) at = (i32)i;
    if (at < 0) return 0;
    if (HB.ent[at].wg) HB.wg_used[HB.ent[at].wg - 1] = 0;
    memmove(&HB.ent[at], &HB.ent[at + 1], (HB.n - (u32)at - 1) * sizeof(HbEnt));
    HB.n--;
    hb_run_generated(e, mb[0], mb + 1, M.n_leaves, &M);
    if (!HB.n) pool_release_deferred();   /* the merged launch went out at once */
    hipb.n_fused++;
    return 1;
}

int thvm_hip_chain_merge(const UOpKernel *p, const u32 *pb, const UOpKernel *c, u32 c_out, const u32 *c_leaves,
                         UOpKernel *m, u32 *mb) {
    if (!p || !pb || !c || !c_leaves || !m || !mb) return 0;
    ChainInfo *ci = chain_info_make(p, p->ops);
    if (!ci) return 0;
    const int r = chain_merge(ci, pb, c, c_out, c_leaves, c->n_leaves, m, mb);
    free(ci);
    return r;
}

/* A program that ran fused into another launch (an epilogue or a merged
 * chain) still gets the cache entries its own dispatch would leave: the
 * recognizers' negative entries and its compiled kernel. The dispatch
 * without allocation, which never compiles, then runs it on its own. */
static void hb_prepare_standalone(const UOpKernel *k) {
    static u64 refused[64];   /* programs the generator or hipRTC refused on their own */
    static u32 n_refused;
    const u64 key = uop_signature(k);
    if (rtc_lookup(key, k)) return;
    for (u32 i = 0; i < n_refused && i < 64; i++)
        if (refused[i] == key) return;
    if (!hipb.no_dense) dense_note_plain(k);
    if (!hipb.no_window) window_note_plain(k);
    if (!rtc_compile_uop(key, k)) refused[n_refused++ % 64] = key;
}

/* Loads of two leaf slots that name the same buffer (of one dtype, neither
 * stored into) read it through the first slot, so that the generated code
 * loads each element once: the engine passes a tensor once per use in an
 * expression (the pooling backward's input and its comparison operand).
 * Returns k itself when no slots repeat. */
static const UOpKernel *hb_dedup_slots(const UOpKernel *k, const u32 *leaf_bufs, u32 n_leaves) {
    static UOpKernel dk;
    const u32 n = k->n_leaves < n_leaves ? k->n_leaves : n_leaves;
    if (n < 2 || n >= 64) return k;
    const u64 stored = chain_store_slots(k);
    u8 map[64];
    int any = 0;
    for (u32 s = 1; s <= n; s++) {
        map[s] = (u8)s;
        if (!leaf_bufs[s - 1] || ((stored >> s) & 1u)) continue;
        for (u32 t = 1; t < s; t++)
            if (leaf_bufs[t - 1] == leaf_bufs[s - 1] && !((stored >> t) & 1u) &&
                k->leaf_dtypes[t - 1] == k->leaf_dtypes[s - 1]) {
                map[s] = (u8)t;
                any = 1;
                break;
            }
    }
    if (!any) return k;
    memcpy(&dk, k, sizeof dk);
    for (u32 i = 0; i < dk.n_ops; i++)
        if (dk.ops[i].type == KOP_LOAD && dk.ops[i].imm.u >= 1 && dk.ops[i].imm.u <= n)
            dk.ops[i].imm.u = map[dk.ops[i].imm.u];
    return &dk;
}

static void hb_dispatch_uop_kernel(u32 out_buf, const u32 *leaf_bufs, u32 n_leaves,
                                   const UOpKernel *k, u64 cache_key) {
    (void)cache_key;
    const u64 t0 = hipb_hp_now();
    if (k && leaf_bufs) k = hb_dedup_slots(k, leaf_bufs, n_leaves);
    /* the dispatched program's signature is computed once for the dispatch
     * (the lookups of every path ask for it); programs built during the
     * dispatch (merged, fused, copies) live elsewhere and are hashed anew */
    const UOpKernel *sk = hipb.sig_k;
    const u64 sh = hipb.sig_h;
    hipb.sig_k = k;
    hipb.sig_h = 0;
    hb_dispatch_uop_kernel_(out_buf, leaf_bufs, n_leaves, k);
    hipb.sig_k = sk;
    hipb.sig_h = sh;
    hipb_hp_add(HP_DISPATCH, t0);
}

static void hb_dispatch_uop_kernel_(u32 out_buf, const u32 *leaf_bufs, u32 n_leaves, const UOpKernel *k) {
    if (!hipb.initialized || !k) return;
    HipbBuf *ob = pool_get(out_buf);
    if (!ob) {
        fprintf(stderr, "tinyhvm-hip: dispatch into unknown buffer %u\n", out_buf);
        return;
    }
    hipb.n_dispatch++;
    copyq_guard_dispatch(out_buf, leaf_bufs, n_leaves < FUSE_MAX_LEAVES ? n_leaves : FUSE_MAX_LEAVES);
    pool_sync_device(out_buf);
    if (!hipb.force_interp && hb_try_group(out_buf, leaf_bufs, n_leaves, k)) {
        pool_mark_device_write(out_buf);
        int loop = 0;
        for (u32 i = 0; i < k->n_ops && !loop; i++) loop = k->ops[i].type == KOP_RANGE;
        if (!loop) hb_prepare_standalone(k);   /* a run sum's own kernel exists already */
        return;
    }
    if (!hipb.force_interp && hb_try_epilogue(out_buf, leaf_bufs, n_leaves, k)) {
        pool_mark_device_write(out_buf);
        hb_prepare_standalone(k);
        return;
    }
    if (!hipb.force_interp && hb_try_chain(out_buf, leaf_bufs, n_leaves, k)) {
        hb_prepare_standalone(k);
        return;
    }
    if (!hipb.no_dense && !hipb.force_interp && dense_try_dispatch(out_buf, leaf_bufs, n_leaves, k)) {
        pool_mark_device_write(out_buf);
        hipb.n_dense++;
        return;
    }
    if (hipb.noalloc && hipb.noalloc_err) return;
    if (!hipb.no_window && !hipb.force_interp && window_try_dispatch(out_buf, leaf_bufs, n_leaves, k)) {
        pool_mark_device_write(out_buf);
        hipb.n_window++;
        return;
    }
    if (hipb.noalloc && hipb.noalloc_err) return;
    if (hipb.noalloc && hipb.force_interp) {
        hipb.noalloc_err = THVM_HIP_ENOTREADY;
        return;
    }
    if (hipb.force_interp) {
        interp_dispatch(out_buf, leaf_bufs, n_leaves, k);
        return;
    }
    u64 key = uop_signature(k);
    KCacheEntry *e = rtc_lookup(key, k);
    if (e) hipb.n_cache_hit++;
    else if (hipb.noalloc) {
        hipb.noalloc_err = THVM_HIP_ENOTREADY;   /* never compiles without allocating */
        return;
    } else e = rtc_compile_uop(key, k);
    if (!e) {
        /* the generator or hipRTC refused the program: the interpreter runs
         * it, so the output is still written (counted in n_fallback) */
        interp_dispatch(out_buf, leaf_bufs, n_leaves, k);
        return;
    }

    hb_run_generated(e, out_buf, leaf_bufs, n_leaves, k);
}

/* The output and the leaf slots a generated program stores into hold
 * device-written contents. */
static void hb_mark_writes(const KCacheEntry *e, u32 out_buf, const u32 *leaf_bufs, u32 n_leaves) {
    pool_mark_device_write(out_buf);
    for (u32 i = 0; e->store_slots && i < n_leaves && i + 1 < 64; i++)
        if ((e->store_slots >> (i + 1)) & 1u) pool_mark_device_write(leaf_bufs[i]);
}

/* The inline scalars of compiled program e over these buffers: constant-
 * index loads of host-held leaves take their value from an argument (sm bit
 * j, value sv[j]). Returns the leaves read only that way (bit i: leaf i),
 * which need not be uploaded. */
static u64 hb_inline_scalars(const KCacheEntry *e, u32 out_buf, const u32 *leaf_bufs, u32 n_leaves,
                             const UOpKernel *k, u32 *sm_out, float *sv) {
    u32 sm = 0;
    for (u32 j = 0; j < e->n_scal; j++) {
        u32 leaf = e->scal_leaf[j];
        u32 id = leaf < n_leaves ? leaf_bufs[leaf] : 0;
        sv[j] = 0.0f;
        if (id && id != out_buf && pool_host_value(id, k->leaf_dtypes[leaf], e->scal_index[j], &sv[j]))
            sm |= 1u << j;
    }
    u64 only = 0;
    for (u32 i = 0; i < n_leaves && i < 32; i++) {
        int inline_only = (e->scal_only_leaves >> i) & 1u;
        for (u32 j = 0; j < e->n_scal && inline_only; j++)
            if (e->scal_leaf[j] == i && !((sm >> j) & 1u)) inline_only = 0;
        if (inline_only) only |= 1ull << i;
    }
    *sm_out = sm;
    return only;
}

/* Launches (or holds) compiled program e over its buffers. */
static void hb_run_generated(KCacheEntry *e, u32 out_buf, const u32 *leaf_bufs, u32 n_leaves, const UOpKernel *k) {
    HipbBuf *ob = pool_get(out_buf);
    if (!ob) return;
    /* constant-index loads of host-held leaves take their value inline; a
     * leaf read only that way is not uploaded */
    u32 sm = 0;
    float sv[KGEN_MAX_SCALARS];
    const u64 only = hb_inline_scalars(e, out_buf, leaf_bufs, n_leaves, k, &sm, sv);
    for (u32 i = 0; i < n_leaves && i < FUSE_MAX_LEAVES; i++)
        if (!((only >> i) & 1u)) pool_sync_device(leaf_bufs[i]);
    if (e->total == 0) return;

    /* kernel parameters: p0..pN (buffer pointers), c0..cN (element counts),
     * then sm_ and the inline scalars, then the split-reduce workspace */
    u32 nb = k->n_leaves + 1;
    void *ptrs[FUSE_MAX_LEAVES + 1];
    u32 counts[FUSE_MAX_LEAVES + 1];
    void *params[2 * (FUSE_MAX_LEAVES + 1) + 3 + KGEN_MAX_SCALARS];
    ptrs[0] = ob->ptr;
    counts[0] = elem_count(out_buf, k->out_dtype);
    for (u32 i = 0; i < k->n_leaves; i++) {
        void *lp = (i < n_leaves) ? pool_ptr(leaf_bufs[i]) : NULL;
        ptrs[i + 1] = lp ? lp : hipb.dummy;   /* loads index an absent buffer's element 0 */
        counts[i + 1] = lp ? elem_count(leaf_bufs[i], k->leaf_dtypes[i]) : 0u;
    }
    for (u32 b = 0; b < nb; b++) {
        params[b] = &ptrs[b];
        params[nb + b] = &counts[b];
    }
    u32 np = 2 * nb;
    if (e->n_scal) {
        params[np++] = &sm;
        for (u32 j = 0; j < e->n_scal; j++) params[np++] = &sv[j];
    }
    /* the memory it touches, for holding it for a batched launch */
    HbMem hm;
    hm.n = 0;
    hbm_add(&hm, ptrs[0], pool_bytes(out_buf), 1);
    for (u32 i = 0; i < n_leaves && i < FUSE_MAX_LEAVES; i++)
        hbm_add(&hm, pool_ptr(leaf_bufs[i]), pool_bytes(leaf_bufs[i]), i + 1 < 64 && ((e->store_slots >> (i + 1)) & 1u));
    u32 gx, gy;
    if (e->splits > 1 && !e->fn_fin) {
        /* split group reduce, partials combined by the last workgroup of each
         * output through the combine area */
        params[np] = &hipb.comb_slots;
        grid_for(e->total * e->splits, e->block, &gx, &gy);
        if (!hipb_hold(&e->co, e->fn, gx, gy, params, &hm, 1, (int)np, e->total * e->splits))
            hipb_launch(e->fn, gx, gy, 1, e->block, params);
        hb_mark_writes(e, out_buf, leaf_bufs, n_leaves);
        return;
    }
    if (e->splits > 1) {
        /* split group reduce: partials into the workspace, then the combine */
        float *ws = reduce_workspace((u64)e->total * e->splits * sizeof(float));
        if (!ws) return;
        params[np] = &ws;
        grid_for(e->total * e->splits, e->block, &gx, &gy);
        hipb_launch(e->fn, gx, gy, 1, e->block, params);
        void *p2[] = {&ptrs[0], &counts[0], &ws};
        hipb_launch(e->fn_fin, (u32)e->total, 1, 1, 256, p2);   /* a workgroup per output */
        hb_mark_writes(e, out_buf, leaf_bufs, n_leaves);
        return;
    }
    if (e->mode == KG_MODE_GROUP) grid_for(e->total, e->block, &gx, &gy);
    else grid_for((e->n_threads + e->block - 1) / e->block, e->block, &gx, &gy);
    /* a chainable program is held, alone if its grid is too large to
     * batch, so that a consumer of its output can fuse after it */
    if (hipb_hold(&e->co, e->fn, gx, gy, params, &hm, 0, -1, 0) ||
        (e->chain && hb_hold_large(&e->co, e->fn, gx, gy, params, &hm)))
        hb_hold_chain(e->chain, out_buf, leaf_bufs, n_leaves);
    else
        hipb_launch(e->fn, gx, gy, 1, e->block, params);
    hb_mark_writes(e, out_buf, leaf_bufs, n_leaves);
}

/* The same dispatch with its workspaces carved from the static array and no
 * compilation (see thvm_hip.h). */
int thvm_hip_dispatch_uop_kernel_noalloc(u32 out_buf, const u32 *leaf_bufs, u32 n_leaves,
                                         const UOpKernel *k) {
    if (!hipb.initialized || !k || !pool_get(out_buf)) return THVM_HIP_EINVAL;
    if (!hipb.noalloc_scratch) return THVM_HIP_ENOSCRATCH;
    hipb.noalloc = 1;
    hipb.noalloc_off = 0;
    hipb.noalloc_err = 0;
    hb_dispatch_uop_kernel(out_buf, leaf_bufs, n_leaves, k, 0);
    hipb.noalloc = 0;
    return hipb.noalloc_err;
}

/* ---- dispatch_kernel_rs: static interpreter ---- */
static void hb_dispatch_kernel_rs(u32 out_buf, u32 *leaf_bufs, const View **leaf_views,
                                  const ShapeTracker *const *leaf_sts, u32 n_leaves,
                                  FusedOp *ops, u32 n_ops, const Shape *full_shape,
                                  const ReduceSpec *reduce, u32 *side_bufs, const u32 *side_idx,
                                  u32 n_side, const u32 *leaf_dtypes, u32 out_dtype) {
    (void)side_bufs; (void)side_idx; (void)n_side;
    if (!hipb.initialized || !full_shape) return;
    HipbBuf *ob = pool_get(out_buf);
    if (!ob) return;
    copyq_guard_dispatch(out_buf, leaf_bufs, n_leaves < FUSE_MAX_LEAVES ? n_leaves : FUSE_MAX_LEAVES);
    pool_sync_device(out_buf);
    for (u32 i = 0; i < n_leaves && i < FUSE_MAX_LEAVES; i++) pool_sync_device(leaf_bufs[i]);
    if (n_leaves > FUSE_MAX_LEAVES || n_ops > FUSE_MAX_OPS || out_dtype >= DTYPE_COUNT) {
        fprintf(stderr, "tinyhvm-hip: dispatch_kernel_rs: unsupported kernel size\n");
        return;
    }
    u32 n_st = 0;
    for (u32 i = 0; i < n_leaves; i++)
        if (leaf_sts && leaf_sts[i] && leaf_sts[i]->n_views >= 2) n_st++;
    size_t psize = sizeof(RsParams) + (n_st ? (n_st - 1) : 0) * sizeof(ShapeTracker);
    RsParams *P = calloc(1, psize);
    if (!P) return;
    u32 rank = full_shape->rank ? full_shape->rank : 1;
    if (rank > MAX_DIM) rank = MAX_DIM;
    P->rank = rank;
    P->has_reduce = (reduce && reduce->reduce_type) ? 1u : 0u;
    P->reduce_type = P->has_reduce ? reduce->reduce_type : 0;
    P->post_start = P->has_reduce ? reduce->post_reduce_start : 0;
    P->n_post_leaves = P->has_reduce ? reduce->n_post_leaves : 0;
    u32 full_numel = 1, out_numel = 1, red_numel = 1;
    for (u32 d = 0; d < rank; d++) {
        P->dims[d] = full_shape->dims[d];
        P->is_reduce[d] = (P->has_reduce && reduce->is_reduce[d]) ? 1u : 0u;
        P->out_shape[d] = P->is_reduce[d] ? 1u : full_shape->dims[d];
        full_numel *= full_shape->dims[d];
        out_numel *= P->out_shape[d];
        if (P->is_reduce[d]) red_numel *= full_shape->dims[d];
    }
    P->full_numel = full_numel;
    P->out_numel = out_numel;
    P->reduce_numel = red_numel;
    P->n_leaves = n_leaves;
    P->n_ops = n_ops;
    P->out_dtype = out_dtype;
    P->out_n = elem_count(out_buf, out_dtype);
    P->out_ptr = (u64)(uintptr_t)ob->ptr;
    u32 si = 0;
    for (u32 i = 0; i < n_leaves; i++) {
        u32 dt = leaf_dtypes ? leaf_dtypes[i] : DTYPE_F32;
        if (dt >= DTYPE_COUNT) dt = DTYPE_F32;
        P->leaf_dtype[i] = dt;
        void *lp = pool_ptr(leaf_bufs[i]);
        P->leaf_ptr[i] = (u64)(uintptr_t)lp;
        P->leaf_n[i] = lp ? elem_count(leaf_bufs[i], dt) : 0;
        if (leaf_views && leaf_views[i]) P->views[i] = *leaf_views[i];
        if (leaf_sts && leaf_sts[i] && leaf_sts[i]->n_views >= 2) {
            P->sts[si] = *leaf_sts[i];
            P->leaf_st[i] = si++;
        } else {
            P->leaf_st[i] = 0xFFFFFFFFu;
        }
    }
    for (u32 i = 0; i < n_ops; i++) P->ops[i] = ops[i];

    hipFunction_t fn = rtc_static_fn("thvm_rs");
    u64 pcap = 0;
    void *dp = fn ? pool_block_get(psize, &pcap) : NULL;
    if (!dp) {
        free(P);
        return;
    }
    pool_upload(dp, P, psize);
    u32 threads = P->has_reduce ? out_numel : full_numel;
    u32 phase0 = 0, phase1 = 1;
    void *a0[] = {&dp, &phase0};
    void *a1[] = {&dp, &phase1};
    if (threads) hipb_launch(fn, (threads + 63) / 64, 1, 1, 64, a0);
    if (P->has_reduce && P->post_start && P->post_start < n_ops && out_numel)
        hipb_launch(fn, (out_numel + 63) / 64, 1, 1, 64, a1);
    pool_block_put(dp, pcap);   /* stream order keeps the block alive for the kernels above */
    pool_mark_device_write(out_buf);
    free(P);
    hipb.n_dispatch++;
}

static void hb_contiguify(u32 dst_buf, u32 numel, u32 src_buf, const View *src_view) {
    if (!hipb.initialized || !src_view || numel == 0) return;
    HipbBuf *d = pool_get(dst_buf), *s = pool_get(src_buf);
    if (!d) return;
    copyq_guard(dst_buf);
    copyq_guard(src_buf);
    pool_sync_device(dst_buf);
    pool_sync_device(src_buf);
    hipFunction_t fn = rtc_static_fn("thvm_contiguify");
    if (!fn) return;
    /* The engine calls this only when source and destination dtypes agree
     * (src/interact/tensor_ops.c:113-116) and allocates numel * dtype size
     * bytes, so the element size is the destination's bytes per element. */
    ContigArgs a;
    memset(&a, 0, sizeof a);
    a.esize = d->bytes == (u64)numel * 2 ? 2u : 4u;
    a.dst = (u64)(uintptr_t)d->ptr;
    a.dst_n = (u32)(d->bytes / a.esize);
    a.src = s ? (u64)(uintptr_t)s->ptr : 0;
    a.src_n = s ? (u32)(s->bytes / a.esize) : 0;
    a.v = *src_view;
    a.numel = numel;
    void *params[] = {&a};
    hipb_launch(fn, (numel + 255) / 256, 1, 1, 256, params);
    pool_mark_device_write(dst_buf);
}

/* ---- legacy per-op slots (src/tinyhvm.h:1004-1016) ----
 * Reached only from the engine's ENSURE/materialize path
 * (src/fuse/materialize.c:195,672,683,700). One lane per output in the CPU
 * backend's order (src/backend/cpu/ops.c), so results are bit-identical. */
static u32 elems_of(const HipbBuf *b, u32 dt) { return b ? (u32)(b->bytes / (dt == DTYPE_F16 ? 2u : 4u)) : 0u; }

static void legacy_guard(u32 dst, u32 a, u32 b) {
    copyq_guard(dst);
    copyq_guard(a);
    copyq_guard(b);
}

static void legacy_launch(const char *name, LegacyArgs *a, u32 dst) {
    hipFunction_t fn = rtc_static_fn(name);
    if (fn && a->n) {
        void *params[] = {a};
        hipb_launch(fn, (a->n + 255u) / 256u, 1, 1, 256, params);
    }
    pool_mark_device_write(dst);
}

static void hb_op_unary(u32 uop, u32 dst, const View *dv, u32 dd, u32 src, const View *sv, u32 sd) {
    HipbBuf *d = pool_get(dst), *s = pool_get(src);
    if (!hipb.initialized || !d || !dv || !sv) return;
    legacy_guard(dst, src, 0);
    pool_sync_device(dst);
    pool_sync_device(src);
    LegacyArgs a;
    memset(&a, 0, sizeof a);
    a.dst = (u64)(uintptr_t)d->ptr; a.dst_n = elems_of(d, dd); a.dd = dd;
    a.a = s ? (u64)(uintptr_t)s->ptr : 0; a.a_n = elems_of(s, sd); a.ad = sd; a.av = *sv;
    a.n = dv->numel; a.uop = uop; a.binary = 0;
    legacy_launch("thvm_op_ew", &a, dst);
}

static void hb_op_binary(u32 uop, u32 dst, const View *dv, u32 dd, u32 ab, const View *av, u32 ad, u32 bb,
                         const View *bv, u32 bd) {
    HipbBuf *d = pool_get(dst), *x = pool_get(ab), *y = pool_get(bb);
    if (!hipb.initialized || !d || !dv || !av || !bv) return;
    legacy_guard(dst, ab, bb);
    pool_sync_device(dst);
    pool_sync_device(ab);
    pool_sync_device(bb);
    LegacyArgs a;
    memset(&a, 0, sizeof a);
    a.dst = (u64)(uintptr_t)d->ptr; a.dst_n = elems_of(d, dd); a.dd = dd;
    a.a = x ? (u64)(uintptr_t)x->ptr : 0; a.a_n = elems_of(x, ad); a.ad = ad; a.av = *av;
    a.b = y ? (u64)(uintptr_t)y->ptr : 0; a.b_n = elems_of(y, bd); a.bd = bd; a.bv = *bv;
    a.n = dv->numel; a.uop = uop; a.binary = 1;
    legacy_launch("thvm_op_ew", &a, dst);
}

static void hb_op_mm(u32 dst, u32 dd, u32 ab, const View *av, u32 ad, u32 bb, const View *bv, u32 bd, u32 M,
                     u32 K, u32 N) {
    HipbBuf *d = pool_get(dst), *x = pool_get(ab), *y = pool_get(bb);
    if (!hipb.initialized || !d || !av || !bv) return;
    if ((u64)M * N > 0xFFFFFFFFull) {
        fprintf(stderr, "tinyhvm-hip: op_mm %ux%u output exceeds u32 indexing\n", M, N);
        return;
    }
    legacy_guard(dst, ab, bb);
    pool_sync_device(dst);
    pool_sync_device(ab);
    pool_sync_device(bb);
    LegacyArgs a;
    memset(&a, 0, sizeof a);
    a.dst = (u64)(uintptr_t)d->ptr; a.dst_n = elems_of(d, dd); a.dd = dd;
    a.a = x ? (u64)(uintptr_t)x->ptr : 0; a.a_n = elems_of(x, ad); a.ad = ad; a.av = *av;
    a.b = y ? (u64)(uintptr_t)y->ptr : 0; a.b_n = elems_of(y, bd); a.bd = bd; a.bv = *bv;
    a.M = M; a.K = K; a.N = N; a.n = M * N;
    legacy_launch("thvm_op_mm", &a, dst);
}

static void hb_op_reduce(u32 uop, u32 dst, u32 dn, u32 dd, u32 src, u32 sn, u32 sd, u32 rdim) {
    HipbBuf *d = pool_get(dst), *s = pool_get(src);
    (void)sn;
    if (!hipb.initialized || !d) return;
    legacy_guard(dst, src, 0);
    pool_sync_device(dst);
    pool_sync_device(src);
    LegacyArgs a;
    memset(&a, 0, sizeof a);
    a.dst = (u64)(uintptr_t)d->ptr; a.dst_n = elems_of(d, dd); a.dd = dd;
    a.a = s ? (u64)(uintptr_t)s->ptr : 0; a.a_n = elems_of(s, sd); a.ad = sd;
    a.n = dn; a.uop = uop; a.K = rdim;
    legacy_launch("thvm_op_reduce", &a, dst);
}

/* adam_step (src/tinyhvm.h:1033-1035; the engine calls it from
 * adam_step_direct, src/nn/adam.c:103-118): one fused pass, in place, with
 * the engine's lazy-update arithmetic. Buffers shorter than n elements make
 * the call a no-op, as a missing slot is. */
static void hb_adam_step(u32 param, u32 grad, u32 m, u32 v, f32 lr, f32 beta1, f32 beta2, f32 eps, f32 bc1,
                         f32 bc2, u32 n) {
    HipbBuf *bp = pool_get(param), *bg = pool_get(grad), *bm = pool_get(m), *bv = pool_get(v);
    const u64 need = (u64)n * 4;
    if (!hipb.initialized || !bp || !bg || !bm || !bv || n == 0) return;
    if (pool_bytes(param) < need || pool_bytes(grad) < need || pool_bytes(m) < need || pool_bytes(v) < need) {
        fprintf(stderr, "tinyhvm-hip: adam_step: buffers shorter than %u elements\n", n);
        return;
    }
    legacy_guard(param, grad, m);
    copyq_guard(v);
    pool_sync_device(param);
    pool_sync_device(grad);
    pool_sync_device(m);
    pool_sync_device(v);
    AdamArgs a;
    memset(&a, 0, sizeof a);
    a.p = (u64)(uintptr_t)bp->ptr; a.g = (u64)(uintptr_t)bg->ptr;
    a.m = (u64)(uintptr_t)bm->ptr; a.v = (u64)(uintptr_t)bv->ptr;
    a.lr = lr; a.beta1 = beta1; a.beta2 = beta2; a.eps = eps; a.bc1 = bc1; a.bc2 = bc2;
    a.n = n;
    a.vec = ((a.p | a.g | a.m | a.v) & 15u) == 0;
    hipFunction_t fn = rtc_static_fn("thvm_adam");
    if (fn) {
        void *params[] = {&a};
        u64 groups = ((u64)n + 3) / 4;
        hipb_launch(fn, (u32)((groups + 255) / 256), 1, 1, 256, params);
    }
    pool_mark_device_write(param);
    pool_mark_device_write(m);
    pool_mark_device_write(v);
}

/* A copy of the whole f32 output of a held chainable program as one more
 * consumer of it: the copy program (one load at gid, one store) merged into
 * the producer (hb_try_chain), so that the producer's launch writes both
 * buffers. ASSIGN copies each updated parameter or running statistic back
 * right after the kernel that computed it. Returns 1 when merged. */
static int hb_copy_as_chain(u32 dst_buf, u32 src_buf, u64 nbytes) {
    static UOpKernel ck;
    if (!HB.n || hipb.no_fuse || nbytes % 4 || nbytes / 4 == 0 || nbytes / 4 > 0xFFFFFFFFull ||
        pool_bytes(src_buf) < nbytes || pool_bytes(dst_buf) < nbytes || dst_buf == src_buf)
        return 0;
    int held = 0;
    for (u32 i = 0; i < HB.n && !held; i++)
        if (HB.ent[i].ch)
            for (u32 st = 0; st < HB.ent[i].ch->n_st; st++)
                held |= HB.ent[i].ch_bufs[HB.ent[i].ch->st_slot[st]] == src_buf &&
                        HB.ent[i].ch->total == (u32)(nbytes / 4) && HB.ent[i].ch->st_f32[st];
    if (!held) return 0;
    memset(&ck, 0, offsetof(UOpKernel, leaf_views));
    ck.ops[0].type = KOP_GID;
    ck.ops[1].type = KOP_LOAD;
    ck.ops[1].arg[0] = 0;
    ck.ops[1].imm.u = 1;
    ck.ops[2].type = KOP_STORE;
    ck.ops[2].arg[0] = 0;
    ck.ops[2].arg[1] = 1;
    ck.ops[2].imm.u = 0;
    ck.n_ops = 3;
    ck.n_leaves = 1;
    ck.n_bufs = 2;
    ck.leaf_dtypes[0] = DTYPE_F32;
    ck.out_dtype = DTYPE_F32;
    ck.grid[0] = (u32)(nbytes / 4);
    ck.grid[1] = ck.grid[2] = 1;
    ck.local_size = 0;
    if (!hb_try_chain(dst_buf, &src_buf, 1, &ck)) return 0;
    pool_mark_device_write(dst_buf);
    return 1;
}

static void hb_buf_copy(u32 dst_buf, u32 src_buf, u64 nbytes) {
    HipbBuf *d = pool_get(dst_buf), *s = pool_get(src_buf);
    if (!d || !s || nbytes == 0) return;
    /* the whole output of a held elementwise program: written by its launch */
    if (!copyq_uses(dst_buf) && !copyq_uses(src_buf) && !d->dev_stale && nbytes <= d->cap &&
        hb_copy_as_chain(dst_buf, src_buf, nbytes)) {
        hipb.n_copy_fused++;
        return;
    }
    /* a queued copy that writes this copy's source or touches its
     * destination must land first */
    for (u32 i = 0; i < CQ.b.n; i++)
        if (CQ.dst_id[i] == src_buf || CQ.dst_id[i] == dst_buf || CQ.src_id[i] == dst_buf) {
            copyq_flush();
            break;
        }
    pool_sync_device(dst_buf);
    pool_sync_device(src_buf);
    u64 n = nbytes;
    if (n > d->cap) n = d->cap;
    if (n > s->cap) n = s->cap;
    if (CQ.b.n == COPY_BATCH_MAX) copyq_flush();
    u32 q = CQ.b.n++;
    CQ.b.dst[q] = (u64)(uintptr_t)d->ptr;
    CQ.b.src[q] = (u64)(uintptr_t)s->ptr;
    CQ.b.bytes[q] = n;
    CQ.dst_id[q] = dst_buf;
    CQ.src_id[q] = src_buf;
    pool_mark_device_write(dst_buf);
}

static void hb_profile_report(void) {
    u64 live, cached, mallocs;
    pool_stats(&live, &cached, &mallocs);
    fprintf(stderr,
            "tinyhvm-hip: dispatches=%llu dense=%llu compiled=%llu cache_hits=%llu "
            "interpreted=%llu host_waits=%llu live=%.1fMB cached=%.1fMB hipMalloc=%llu\n",
            (unsigned long long)hipb.n_dispatch, (unsigned long long)hipb.n_dense,
            (unsigned long long)hipb.n_compile, (unsigned long long)hipb.n_cache_hit,
            (unsigned long long)hipb.n_fallback, (unsigned long long)hipb.n_stream_sync,
            live / 1e6, cached / 1e6, (unsigned long long)mallocs);
    if (hipb.host_profile) {
        static const char *nm[HP_N] = {"dispatch_uop_kernel", "kernel launches", "program signatures",
                                       "alloc/free/incref/decref", "buf_write"};
        for (int c = 0; c < HP_N; c++)
            fprintf(stderr, "tinyhvm-hip: host %-26s %10llu calls %10.3f ms %8.3f us/call\n", nm[c],
                    (unsigned long long)hipb.hp_calls[c], hipb.hp_ns[c] / 1e6,
                    hipb.hp_calls[c] ? hipb.hp_ns[c] / 1e3 / hipb.hp_calls[c] : 0.0);
    }
}

static void hb_profile_reset(void) {
    hipb.n_dispatch = hipb.n_compile = hipb.n_cache_hit = hipb.n_dense = 0;
    hipb.n_fallback = hipb.n_stream_sync = hipb.n_window = 0;
    memset(hipb.hp_ns, 0, sizeof hipb.hp_ns);
    memset(hipb.hp_calls, 0, sizeof hipb.hp_calls);
}

Backend hip_backend = {
    .init = hb_init,
    .shutdown = hb_shutdown,
    .buf_alloc = hb_buf_alloc,
    .buf_free = hb_buf_free,
    .buf_incref = hb_buf_incref,
    .buf_decref = hb_buf_decref,
    .mem_checkpoint = hb_mem_checkpoint,
    .buf_mark_use = hb_buf_mark_use,
    .buf_write = hb_buf_write,
    .buf_read = hb_buf_read,
    .op_unary = hb_op_unary,
    .op_binary = hb_op_binary,
    .op_mm = hb_op_mm,
    .op_reduce = hb_op_reduce,
    .dispatch_kernel_rs = hb_dispatch_kernel_rs,
    .dispatch_uop_kernel = hb_dispatch_uop_kernel,
    .contiguify = hb_contiguify,
    .buf_copy = hb_buf_copy,
    .buf_read_nosync = hb_buf_read_nosync,
    .adam_step = hb_adam_step,
    .pool_reset = hb_pool_reset,
    .pool_set_persistent = hb_pool_set_persistent,
    .begin_batch = hb_begin_batch,
    .end_batch = hb_end_batch,
    .profile_report = hb_profile_report,
    .profile_reset = hb_profile_reset,
};

/* ---- flat C entry points (same behaviour as the vtable slots) ---- */
int  thvm_hip_init(void) { return hb_init(); }
void thvm_hip_op_unary(u32 uop, u32 dst, const View *dv, u32 dd, u32 src, const View *sv, u32 sd) {
    hb_op_unary(uop, dst, dv, dd, src, sv, sd);
}
void thvm_hip_op_binary(u32 uop, u32 dst, const View *dv, u32 dd, u32 a, const View *av, u32 ad, u32 b,
                        const View *bv, u32 bd) {
    hb_op_binary(uop, dst, dv, dd, a, av, ad, b, bv, bd);
}
void thvm_hip_op_mm(u32 dst, u32 dd, u32 a, const View *av, u32 ad, u32 b, const View *bv, u32 bd, u32 M, u32 K,
                    u32 N) {
    hb_op_mm(dst, dd, a, av, ad, b, bv, bd, M, K, N);
}
void thvm_hip_op_reduce(u32 uop, u32 dst, u32 dn, u32 dd, u32 src, u32 sn, u32 sd, u32 rdim) {
    hb_op_reduce(uop, dst, dn, dd, src, sn, sd, rdim);
}
void thvm_hip_adam_step(u32 param, u32 grad, u32 m, u32 v, f32 lr, f32 beta1, f32 beta2, f32 eps, f32 bc1,
                        f32 bc2, u32 n) {
    hb_adam_step(param, grad, m, v, lr, beta1, beta2, eps, bc1, bc2, n);
}
void thvm_hip_shutdown(void) { hb_shutdown(); }
u32  thvm_hip_buf_alloc(u64 bytes) { return hb_buf_alloc(bytes); }
void thvm_hip_buf_free(u32 id) { hb_buf_free(id); }
void thvm_hip_buf_incref(u32 id) { hb_buf_incref(id); }
void thvm_hip_buf_decref(u32 id) { hb_buf_decref(id); }
void thvm_hip_buf_write(u32 id, const void *data, u64 bytes) { hb_buf_write(id, data, bytes); }
void thvm_hip_buf_read(u32 id, void *out, u64 bytes) { hb_buf_read(id, out, bytes); }
void thvm_hip_buf_read_nosync(u32 id, void *out, u64 bytes) { hb_buf_read_nosync(id, out, bytes); }
void thvm_hip_dispatch_uop_kernel(u32 out_buf, const u32 *leaf_bufs, u32 n_leaves,
                                  const UOpKernel *k, u64 cache_key) {
    hb_dispatch_uop_kernel(out_buf, leaf_bufs, n_leaves, k, cache_key);
}
void thvm_hip_dispatch_kernel_rs(u32 out_buf, u32 *leaf_bufs, const View **leaf_views,
                                 const ShapeTracker *const *leaf_sts, u32 n_leaves,
                                 FusedOp *ops, u32 n_ops, const Shape *full_shape,
                                 const ReduceSpec *reduce, u32 *side_bufs, const u32 *side_idx,
                                 u32 n_side, const u32 *leaf_dtypes, u32 out_dtype) {
    hb_dispatch_kernel_rs(out_buf, leaf_bufs, leaf_views, leaf_sts, n_leaves, ops, n_ops, full_shape,
                          reduce, side_bufs, side_idx, n_side, leaf_dtypes, out_dtype);
}
void thvm_hip_contiguify(u32 dst, u32 numel, u32 src, const View *v) { hb_contiguify(dst, numel, src, v); }
void thvm_hip_buf_copy(u32 dst, u32 src, u64 n) { hb_buf_copy(dst, src, n); }
void thvm_hip_pool_reset(u32 keep) { hb_pool_reset(keep); }
void thvm_hip_pool_set_persistent(u32 max_buf) { hb_pool_set_persistent(max_buf); }
void thvm_hip_profile_report(void) { hb_profile_report(); }
void thvm_hip_profile_reset(void) { hb_profile_reset(); }

int thvm_hip_counters(u64 *out, u32 n) {
    u64 live = 0, cached = 0, mallocs = 0;
    u32 pinned = 0, limbo = 0;
    pool_stats(&live, &cached, &mallocs);
    pool_pin_stats(&pinned, &limbo);
    u64 v[16] = {hipb.n_dispatch, hipb.n_dense, hipb.n_compile, hipb.n_cache_hit, hipb.n_fallback,
                 hipb.n_stream_sync, live, mallocs, pinned, limbo, hipb.n_window, hipb.n_batched, hipb.n_fused,
                 hipb.n_comb_gaveup, hipb.n_upload_held, hipb.n_seq};
    for (u32 i = 0; out && i < n && i < 16; i++) out[i] = v[i];
    return 16;
}

int thvm_hip_synchronize(void) {
    if (!hipb.initialized) return -1;
    if (pool_capture_forbids("a synchronize")) return -1;
    copyq_flush();
    hipError_t e = hipb_stream_wait();
    if (e != hipSuccess) {
        fprintf(stderr, "tinyhvm-hip: stream error: %s\n", hipGetErrorString(e));
        return -1;
    }
    if (hipb.comb_gaveup_pending) {
        hipb.comb_gaveup_pending = 0;
        return -1;
    }
    return 0;
}

void *thvm_hip_stream(void) { return hipb.initialized ? (void *)hipb.stream : NULL; }
void thvm_hip_flush(void) {
    if (!hipb.initialized) return;
    copyq_flush();
    hipb_before_stream();
}
void *thvm_hip_buf_device_ptr(u32 id) { return pool_ptr(id); }

const Backend *thvm_hip_backend(void) { return &hip_backend; }

int thvm_hip_abi_sizes(u32 *out, u32 n) {
    u32 v[4] = {(u32)sizeof(View), (u32)sizeof(ShapeTracker), (u32)sizeof(UOpKernel), (u32)sizeof(Backend)};
    for (u32 i = 0; i < n && i < 4; i++) out[i] = v[i];
    return 4;
}

int thvm_hip_kernel_source(const UOpKernel *k, char *buf, u64 buflen, u32 *mode, u32 *vec) {
    char err[256] = {0};
    KGenResult g;
    if (!kgen_uop(k, &g, err, sizeof err)) {
        if (buf && buflen) snprintf(buf, buflen, "error: %s", err);
        return -1;
    }
    size_t n = strlen(g.src);
    if (buf && buflen) {
        size_t c = n < buflen - 1 ? n : buflen - 1;
        memcpy(buf, g.src, c);
        buf[c] = 0;
    }
    if (mode) *mode = (u32)g.mode;
    if (vec) *vec = g.vec;
    kgen_free(&g);
    return (int)n;
}

int thvm_hip_kernel_lanes(const UOpKernel *k, u32 *lanes, u32 n_words, u32 *mode, u32 *vec) {
    char err[256] = {0};
    KGenResult g;
    if (!k || !lanes || n_words < 7u * k->n_ops) return -1;
    if (!kgen_uop_lanes(k, &g, lanes, err, sizeof err)) return -1;
    if (mode) *mode = (u32)g.mode;
    if (vec) *vec = g.vec;
    kgen_free(&g);
    return (int)k->n_ops;
}

int rtc_compile_check(const UOpKernel *k, size_t *code_len, char *err, size_t errlen);

/* The device-free entry points read the routing and tuning knobs once, as
 * init would. */
static void ensure_env(void) {
    static int env_read = 0;
    if (!hipb.initialized && !env_read) {
        read_dense_env();
        env_read = 1;
    }
}

int thvm_hip_window_analyze(const UOpKernel *k, u32 *kind, u32 *splits) {
    ensure_env();
    return window_analyze(k, kind, splits);
}

int thvm_hip_window_source(const UOpKernel *k, char *buf, u64 buflen) {
    char *src = window_source(k);
    if (!src) {
        if (buf && buflen) snprintf(buf, buflen, "not a window-max or run-sum program");
        return -1;
    }
    size_t n = strlen(src);
    if (buf && buflen) snprintf(buf, buflen, "%s", src);
    free(src);
    return (int)n;
}

int thvm_hip_epilogue_compile_check(const UOpKernel *producer, const UOpKernel *consumer, u32 o_leaf, char *errbuf,
                                    u64 errlen) {
    ensure_env();
    char err[256] = {0};
    char *src = producer && consumer ? dense_epilogue_source(producer, consumer, o_leaf, err, sizeof err) : NULL;
    if (!src) {
        if (errbuf && errlen) snprintf(errbuf, errlen, "%s", err[0] ? err : "no fused epilogue");
        return -1;
    }
    long n = rtc_compile_only(src, err, sizeof err);
    free(src);
    if (n < 0 && errbuf && errlen) snprintf(errbuf, errlen, "%s", err);
    return (int)n;
}

int thvm_hip_time_contraction(void *ev_begin, void *ev_end) {
    if (!hipb.initialized) return -1;
    const int fired = hipb.time_fired;
    hipb.time_fired = 0;
    hipb.time_ev[0] = ev_begin && ev_end ? ev_begin : NULL;
    hipb.time_ev[1] = ev_begin && ev_end ? ev_end : NULL;
    return fired;
}

int thvm_hip_upload_source(char *buf, u64 buflen) {
    ensure_env();
    char *src = upload_source();
    if (!src) return -1;
    const size_t len = strlen(src);
    if (buf && buflen) snprintf(buf, buflen, "%s", src);
    free(src);
    return (int)len;
}

int thvm_hip_group_source(const UOpKernel *const *ks, const u32 *const *bufs, u32 n, int producer, char *buf,
                          u64 buflen) {
    ensure_env();
    char err[256] = {0};
    char *src = window_group_source(ks, bufs, n, producer, err, sizeof err);
    if (!src) {
        if (buf && buflen) snprintf(buf, buflen, "%s", err[0] ? err : "no group");
        return -1;
    }
    const size_t len = strlen(src);
    if (buf && buflen) snprintf(buf, buflen, "%s", src);
    free(src);
    return (int)len;
}

int thvm_hip_group_compile_check(const UOpKernel *const *ks, const u32 *const *bufs, u32 n, int producer,
                                 char *errbuf, u64 errlen) {
    ensure_env();
    char err[256] = {0};
    char *src = window_group_source(ks, bufs, n, producer, err, sizeof err);
    if (!src) {
        if (errbuf && errlen) snprintf(errbuf, errlen, "%s", err[0] ? err : "no group");
        return -1;
    }
    long r = rtc_compile_only(src, err, sizeof err);
    free(src);
    if (r < 0 && errbuf && errlen) snprintf(errbuf, errlen, "%s", err);
    return (int)r;
}

int thvm_hip_window_compile_check(const UOpKernel *k, char *errbuf, u64 errlen) {
    char *src = window_source(k);
    if (!src) {
        if (errbuf && errlen) snprintf(errbuf, errlen, "not a window-max or run-sum program");
        return -1;
    }
    char err[256] = {0};
    long n = rtc_compile_only(src, err, sizeof err);
    free(src);
    if (n < 0 && errbuf && errlen) snprintf(errbuf, errlen, "%s", err);
    return (int)n;
}

int thvm_hip_dense_analyze(const UOpKernel *k, u32 *M, u32 *N, u32 *K, u32 *splits) {
    ensure_env();
    return dense_analyze(k, M, N, K, splits);
}

int thvm_hip_dense_source(const UOpKernel *k, char *buf, u64 buflen) {
    ensure_env();
    char *src = dense_source(k);
    if (!src) {
        if (buf && buflen) snprintf(buf, buflen, "not a matrix-core contraction");
        return -1;
    }
    size_t n = strlen(src);
    if (buf && buflen) snprintf(buf, buflen, "%s", src);
    free(src);
    return (int)n;
}

int thvm_hip_dense_compile_check(const UOpKernel *k, char *errbuf, u64 errlen) {
    ensure_env();
    char *src = dense_source(k);
    if (!src) {
        if (errbuf && errlen) snprintf(errbuf, errlen, "not a matrix-core contraction");
        return -1;
    }
    char err[256] = {0};
    long n = rtc_compile_only(src, err, sizeof err);
    free(src);
    if (n < 0 && errbuf && errlen) snprintf(errbuf, errlen, "%s", err);
    return (int)n;
}

int thvm_hip_compile_check(const UOpKernel *k, char *errbuf, u64 errlen) {
    size_t cl = 0;
    char err[256] = {0};
    int ok = rtc_compile_check(k, &cl, err, sizeof err);
    if (!ok && errbuf && errlen) snprintf(errbuf, errlen, "%s", err);
    return ok ? (int)cl : -1;
}

/* ---- HIP graphs of recorded work ----
 * A stretch of backend calls (one training step replayed from a kernel trace,
 * say) is captured from the stream into a HIP graph and launched again as one
 * submission. Kernels keep the arguments they were captured with (buffer
 * pointers, inline scalars), uploads read the graph's own pinned arena, and
 * the graph writes the same buffers at every launch, so a launch repeats the
 * captured step on the current contents of its persistent buffers. Capture
 * runs nothing on the device: host writes still pending are uploaded before
 * it starts, and the host's record of what the device holds stays
 * conservative (a buffer a captured kernel writes is read back from the
 * device; a host write made during the capture is uploaded again for eager
 * use). Every device block the captured work touches is pinned
 * to the graph (pool.c): while the graph lives, such a block never returns
 * to the free lists, even when its buffer id is freed or a workspace grows,
 * so no later allocation can alias memory the graph writes. Work a graph
 * cannot repeat (a host read, a synchronize, a large synchronous write)
 * abandons the capture: graph_end then returns NULL. No memset is ever
 * recorded (the dispatch path clears with kernels). */
#define GRAPH_ARENA_BYTES (4u << 20)

typedef struct HipbGraph {
    hipGraph_t graph;
    hipGraphExec_t exec;
    u8 *arena;
    PoolPins pins;           /* device blocks the captured work references */
    struct HipbGraph *next;  /* live graphs, released at shutdown */
    int released;
} HipbGraph;

static HipbGraph *g_capture;
static HipbGraph *g_live;

/* device-side resources of a graph; the handle itself stays until destroy */
static void graph_release(HipbGraph *g) {
    if (g->released) return;
    if (g->exec) HIPB_CHECK(hipGraphExecDestroy(g->exec));
    if (g->graph) HIPB_CHECK(hipGraphDestroy(g->graph));
    if (g->arena) HIPB_CHECK(hipHostFree(g->arena));
    g->exec = NULL;
    g->graph = NULL;
    g->arena = NULL;
    pool_pins_release(&g->pins);
    g->released = 1;
}

static void graphs_release_all(void) {
    for (HipbGraph *g = g_live; g; g = g->next) graph_release(g);
}

int thvm_hip_graph_begin(void) {
    if (!hipb.initialized || hipb.capturing) return -1;
    copyq_flush();
    /* pending host writes reach the device now, not inside the graph */
    pool_sync_all_device();
    HipbGraph *g = calloc(1, sizeof *g);
    if (!g) return -1;
    /* coherent: upload kernels in the graph read it directly */
    if (hipHostMalloc((void **)&g->arena, GRAPH_ARENA_BYTES, hipHostMallocMapped | hipHostMallocCoherent) !=
        hipSuccess) {
        (void)hipGetLastError();
        free(g);
        return -1;
    }
    hipb_before_stream();
    if (hipStreamBeginCapture(hipb.stream, hipStreamCaptureModeRelaxed) != hipSuccess) {
        (void)hipGetLastError();
        HIPB_CHECK(hipHostFree(g->arena));
        free(g);
        return -1;
    }
    hipb.capturing = 1;
    hipb.capture_bad = 0;
    pool_capture_begin(g->arena, GRAPH_ARENA_BYTES, &g->pins);
    g_capture = g;
    return 0;
}

void *thvm_hip_graph_end(void) {
    if (!hipb.capturing || !g_capture) return NULL;
    copyq_flush();
    hipb_before_stream();
    HipbGraph *g = g_capture;
    g_capture = NULL;
    hipError_t e = hipStreamEndCapture(hipb.stream, &g->graph);
    hipb.capturing = 0;
    pool_capture_end();
    if (e == hipSuccess && !hipb.capture_bad && g->graph)
        e = hipGraphInstantiate(&g->exec, g->graph, NULL, NULL, 0);
    if (e != hipSuccess || hipb.capture_bad || !g->exec) {
        if (e != hipSuccess) {
            (void)hipGetLastError();
            fprintf(stderr, "tinyhvm-hip: graph capture failed: %s\n", hipGetErrorString(e));
        }
        graph_release(g);
        free(g);
        hipb.capture_bad = 0;
        return NULL;
    }
    g->next = g_live;
    g_live = g;
    return g;
}

int thvm_hip_graph_launch(void *handle) {
    HipbGraph *g = handle;
    if (!hipb.initialized || hipb.capturing || !g || g->released || !g->exec) return -1;
    copyq_flush();
    /* host writes since the capture reach the buffers the graph reads, and
     * the host's copies of whatever it writes are no longer current */
    pool_device_wrote_all();
    hipb_before_stream();
    hipError_t e = hipGraphLaunch(g->exec, hipb.stream);
    if (e != hipSuccess) {
        fprintf(stderr, "tinyhvm-hip: graph launch failed: %s\n", hipGetErrorString(e));
        return -1;
    }
    return 0;
}

void thvm_hip_graph_destroy(void *handle) {
    HipbGraph *g = handle;
    if (!g) return;
    if (!g->released) {
        if (hipb.initialized) HIPB_CHECK(hipb_stream_wait());
        graph_release(g);
    }
    for (HipbGraph **pp = &g_live; *pp; pp = &(*pp)->next)
        if (*pp == g) {
            *pp = g->next;
            break;
        }
    free(g);
}
