/*
 * engine_live.c - the TinyHVM engine driving the HIP backend live.
 *
 * TEST INFRASTRUCTURE. Built by `make -C oracle ref` into oracle/_ref/ from
 * the engine's sources where they lie and the workloads of
 * tests/golden/capture.c; run by tests/test_gpu_live.py.
 *
 * Usage: engine_live <libthvm_hip.so> <workload> [sizes...]
 *
 * Runs one workload twice in one process, each time through the engine's own
 * scheduler, lowering and dispatch (thvm_eval, src/schedule/_.c:2268-2411):
 *   run 0  on the engine's CPU backend, under capture.c's recorder in exec
 *          mode (which runs kernels whose masked loads leave their buffer over
 *          zero-guarded leaves, so the interpreter does not fault);
 *   run 1  on a context made by thvm_init("hip"): the engine's thvm_init
 *          with the branch a maintainer adds for "hip" (tests/live/hip_init.h;
 *          src/ctx/init.c:23-37 does the same for Metal), which registers
 *          `hip_backend` as the default device; thvm_free then shuts it
 *          down, which the run checks (the library no longer synchronizes).
 * Every buffer the workload reads back (Backend.buf_read) is kept from both
 * runs and compared: same sequence and sizes, values within 1e-3 normwise
 * (max |gpu - cpu| / max |cpu| per read, as float32), NaNs in the same places.
 * Prints one JSON line and exits 0 when every read agrees.
 *
 * Timing mode: engine_live <libthvm_hip.so | -> time <lenet|mlp> <steps> [sizes...]
 * runs the workload's training steps through thvm_eval with hip_backend as
 * the default device: two steps to warm up (kernel compilation), then
 * <steps> timed steps, each from its "<workload>.step" mark to the next (the
 * engine's own host work, the dispatches, and the step's read-backs of its
 * loss and parameters or gradients). Every backend slot is wrapped to count
 * the host's waits on the stream inside it (thvm_hip_counters): a wait may
 * happen only inside buf_read, the engine's sync point; any other slot that
 * waits is reported. The same steps then run on the engine's CPU backend
 * (one LeNet step or three MLP steps, nothing to warm up), each buffer in a
 * zero-filled guard region (tm_guard_alloc) so that its interpreter runs the
 * zero-padded convolutions itself. Prints one JSON line. With "-" for the
 * library only the CPU leg runs (its GPU fields read 0).
 */
#define CAPTURE_NO_MAIN
#include "../golden/capture.c"

/* the engine's thvm_init, compiled as thvm_init_engine, with the "hip" branch */
#undef thvm_init
#include "hip_init.h"

#include <time.h>

#define LIVE_MAX_READS 4096
typedef struct { u64 n; u8 *data; } LiveRead;
static LiveRead g_reads[2][LIVE_MAX_READS];
static u32 g_nreads[2];
static int g_run;
static void (*g_inner_read)(u32, void *, u64);

static void live_read(u32 id, void *out, u64 bytes) {
    g_inner_read(id, out, bytes);
    u32 i = g_nreads[g_run];
    if (i >= LIVE_MAX_READS) return;
    g_reads[g_run][i].n = bytes;
    g_reads[g_run][i].data = malloc(bytes ? bytes : 1);
    if (g_reads[g_run][i].data) memcpy(g_reads[g_run][i].data, out, bytes);
    g_nreads[g_run] = i + 1;
}

static double now_s(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return t.tv_sec + t.tv_nsec * 1e-9;
}

static int run_workload(TinyHVM *ctx, const char *wl, const u32 *sz, u32 nsz) {
    if (strcmp(wl, "fused") == 0) wl_fused(ctx, nsz > 0 ? sz[0] : 64, nsz > 1 ? sz[1] : 256, 1, 1);
    else if (strcmp(wl, "mlp") == 0)
        wl_mlp(ctx, nsz > 0 ? sz[0] : 64, nsz > 1 ? sz[1] : 784, nsz > 2 ? sz[2] : 128, nsz > 3 ? sz[3] : 10);
    else if (strcmp(wl, "lenet") == 0) wl_lenet(ctx, nsz > 0 ? sz[0] : 8, nsz > 1 ? (int)sz[1] : 1);
    else if (strcmp(wl, "convblock") == 0)
        wl_convblock(ctx, nsz > 0 ? sz[0] : 2, nsz > 1 ? sz[1] : 4, nsz > 2 ? sz[2] : 8);
    else if (strcmp(wl, "linear") == 0)
        wl_linear(ctx, nsz > 0 ? sz[0] : 64, nsz > 1 ? sz[1] : 64, nsz > 2 ? sz[2] : 64, 1);
    else if (strcmp(wl, "adam") == 0) wl_adam(ctx);
    else if (strcmp(wl, "known") == 0) wl_known(ctx);
    else return 0;
    return 1;
}

/* ---- timing mode ---- */
#define TM_MAX_STEPS 1024
static int (*g_counters)(u64 *, u32);
static const char *g_step_mark;
static u32 g_nsteps;
static double g_step_t[TM_MAX_STEPS + 1];
static u64 g_step_waits[TM_MAX_STEPS + 1], g_step_reads[TM_MAX_STEPS + 1], g_step_disp[TM_MAX_STEPS + 1];
static u64 g_reads_total, g_disp_total, g_waits_outside;
/* host seconds inside the backend's slots: buf_read/buf_read_nosync (which
 * wait for the GPU), and every other slot */
static double g_bk_s, g_rd_s, g_step_bk[TM_MAX_STEPS + 1], g_step_rd[TM_MAX_STEPS + 1];
static char g_waits_outside_slot[64];
static Backend g_tm_inner;

static u64 host_waits(void) {
    u64 c[11] = {0};
    if (g_counters) g_counters(c, 11);
    return c[5];
}

static void tm_mark(const char *text) {
    if (!g_step_mark || strcmp(text, g_step_mark) != 0 || g_nsteps >= TM_MAX_STEPS) return;
    g_step_t[g_nsteps] = now_s();
    g_step_waits[g_nsteps] = host_waits();
    g_step_reads[g_nsteps] = g_reads_total;
    g_step_disp[g_nsteps] = g_disp_total;
    g_step_bk[g_nsteps] = g_bk_s;
    g_step_rd[g_nsteps] = g_rd_s;
    g_nsteps++;
}

static void tm_outside(const char *slot, u64 w0) {
    if (host_waits() != w0) {
        g_waits_outside++;
        snprintf(g_waits_outside_slot, sizeof g_waits_outside_slot, "%s", slot);
    }
}
#define TM_WRAP(slot, ...) do { u64 w0_ = host_waits(); double t0_ = now_s(); g_tm_inner.slot(__VA_ARGS__); \
                                   g_bk_s += now_s() - t0_; tm_outside(#slot, w0_); } while (0)
static u32 tm_alloc(u64 b) {
    u64 w0 = host_waits();
    double t0 = now_s();
    u32 id = g_tm_inner.buf_alloc(b);
    g_bk_s += now_s() - t0;
    tm_outside("buf_alloc", w0);
    return id;
}
static void tm_free(u32 id) { TM_WRAP(buf_free, id); }
static void tm_incref(u32 id) { TM_WRAP(buf_incref, id); }
static void tm_decref(u32 id) { TM_WRAP(buf_decref, id); }
static void tm_write(u32 id, const void *d, u64 b) { TM_WRAP(buf_write, id, d, b); }
static void tm_read(u32 id, void *o, u64 b) {
    g_reads_total++;
    double t0 = now_s();
    g_tm_inner.buf_read(id, o, b);
    g_rd_s += now_s() - t0;
}
static void tm_read_nosync(u32 id, void *o, u64 b) {
    g_reads_total++;
    double t0 = now_s();
    g_tm_inner.buf_read_nosync(id, o, b);
    g_rd_s += now_s() - t0;
}
static void tm_uop(u32 out, const u32 *l, u32 n, const UOpKernel *k, u64 key) {
    g_disp_total++;
    TM_WRAP(dispatch_uop_kernel, out, l, n, k, key);
}
static void tm_rs(u32 out, u32 *l, const View **v, const ShapeTracker *const *st, u32 n, FusedOp *ops, u32 nops,
                  const Shape *full, const ReduceSpec *red, u32 *sb, const u32 *si, u32 ns, const u32 *dts, u32 odt) {
    g_disp_total++;
    TM_WRAP(dispatch_kernel_rs, out, l, v, st, n, ops, nops, full, red, sb, si, ns, dts, odt);
}
static void tm_copy(u32 d, u32 s_, u64 b) { TM_WRAP(buf_copy, d, s_, b); }
static void tm_contig(u32 d, u32 n, u32 s_, const View *v) { TM_WRAP(contiguify, d, n, s_, v); }
static void tm_reset(u32 keep) { TM_WRAP(pool_reset, keep); }
static void tm_persist(u32 m) { TM_WRAP(pool_set_persistent, m); }

/* The CPU leg's buffers: each at the start of its own zero-filled, lazily
 * mapped region spanning every u32 element index of a 4-byte type (GUARD_SPAN),
 * placed at allocation. The engine's interpreter loads a leaf element before
 * the mask that discards it (src/backend/cpu/uop.c:55-72); over these regions
 * the stray loads of a zero-padded view read zeros, and the engine's CPU
 * backend runs every kernel itself with nothing added per dispatch. */
static u32 (*g_cpu_alloc)(u64);
static u32 tm_guard_alloc(u64 b) {
    u32 id = g_cpu_alloc(b);
    void *m = mmap(NULL, GUARD_SPAN, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
    if (m == MAP_FAILED) {
        fprintf(stderr, "engine_live: guard mapping failed for buffer %u\n", id);
        exit(1);
    }
    free(cpu_pool.bufs[id]);
    cpu_pool.bufs[id] = m;
    return id;
}
static void tm_guard_release(u32 id) {
    if (id < MAX_BUFS && cpu_pool.bufs[id]) munmap(cpu_pool.bufs[id], GUARD_SPAN);
    if (id < MAX_BUFS) cpu_pool.bufs[id] = NULL;
}
static void tm_guard_free(u32 id) { tm_guard_release(id); }
static void tm_guard_reset(u32 keep) {
    for (u32 i = keep + 1; i < cpu_pool.count; i++) tm_guard_release(i);
    cpu_pool.count = keep + 1;
}
static void tm_guard_shutdown(void) {
    for (u32 i = 1; i < cpu_pool.count; i++) tm_guard_release(i);
    memset(&cpu_pool, 0, sizeof cpu_pool);
}

static void tm_run(TinyHVM *ctx, const char *wl, u32 B, int steps) {
    if (strcmp(wl, "lenet") == 0) wl_lenet(ctx, B, steps);
    else wl_mlp_steps(ctx, B, 784, 128, 10, steps);
}

/* one timed run: returns the median step in seconds (0 when no step closed) */
static double g_last_bk, g_last_rd;   /* the last tm_steps: backend-slot and read seconds per step */
static double tm_steps(TinyHVM *ctx, const char *wl, u32 B, int steps, double *mean, double *waits, double *reads,
                       double *disp) {
    g_nsteps = 0;
    tm_run(ctx, wl, B, steps);
    if (g_nsteps >= TM_MAX_STEPS) return 0.0;
    g_step_t[g_nsteps] = now_s();   /* the last step ends when the workload returns */
    g_step_waits[g_nsteps] = host_waits();
    g_step_reads[g_nsteps] = g_reads_total;
    g_step_disp[g_nsteps] = g_disp_total;
    g_step_bk[g_nsteps] = g_bk_s;
    g_step_rd[g_nsteps] = g_rd_s;
    u32 n = g_nsteps;
    if (n == 0) return 0.0;
    g_last_bk = (g_step_bk[n] - g_step_bk[0]) / n;
    g_last_rd = (g_step_rd[n] - g_step_rd[0]) / n;
    double d[TM_MAX_STEPS], sum = 0.0;
    for (u32 i = 0; i < n; i++) {
        d[i] = g_step_t[i + 1] - g_step_t[i];
        sum += d[i];
    }
    for (u32 i = 1; i < n; i++)
        for (u32 j = i; j > 0 && d[j - 1] > d[j]; j--) { double t = d[j]; d[j] = d[j - 1]; d[j - 1] = t; }
    *mean = sum / n;
    *waits = (double)(g_step_waits[n] - g_step_waits[0]) / n;
    *reads = (double)(g_step_reads[n] - g_step_reads[0]) / n;
    *disp = (double)(g_step_disp[n] - g_step_disp[0]) / n;
    return d[n / 2];
}

static double g_hip_bk, g_hip_rd;
/* the hip_backend leg: returns the median step in seconds, -1 when the
 * backend cannot be loaded or initialised */
static double tm_hip_leg(const char *lib, const char *wl, u32 B, int steps, double *mean, double *waits,
                         double *reads, double *disp) {
    if (hip_backend_load(lib, 0) != 0) return -1;
    Backend *hb = g_hip_backend;
    g_counters = (int (*)(u64 *, u32))dlsym(g_hip_lib, "thvm_hip_counters");
    if (!g_counters) return -1;
    g_tm_inner = *hb;
    static Backend tm;
    tm = *hb;
    tm.buf_alloc = tm_alloc; tm.buf_free = tm_free; tm.buf_incref = tm_incref; tm.buf_decref = tm_decref;
    tm.buf_write = tm_write; tm.buf_read = tm_read; tm.buf_read_nosync = tm_read_nosync;
    tm.dispatch_uop_kernel = tm_uop; tm.dispatch_kernel_rs = tm_rs; tm.buf_copy = tm_copy;
    tm.contiguify = tm_contig; tm.pool_reset = tm_reset; tm.pool_set_persistent = tm_persist;
    g_hip_backend = &tm;   /* thvm_init("hip") registers the counting wrapper */
    TinyHVM *ctx = thvm_init("hip");
    if (!ctx || ctx->default_device != THVM_DEV_HIP) {
        fprintf(stderr, "engine_live: thvm_init(\"hip\") did not register hip_backend\n");
        return -1;
    }
    tm_steps(ctx, wl, B, 2, mean, waits, reads, disp);          /* warm-up: compiles every kernel */
    g_waits_outside = 0;
    g_waits_outside_slot[0] = 0;
    double med = tm_steps(ctx, wl, B, steps, mean, waits, reads, disp);
    g_hip_bk = g_last_bk;
    g_hip_rd = g_last_rd;
    thvm_free(ctx);
    return med;
}

static int time_mode(const char *lib, const char *wl, int steps, const u32 *sz, u32 nsz) {
    if (strcmp(wl, "lenet") != 0 && strcmp(wl, "mlp") != 0) return 2;
    u32 B = nsz > 0 ? sz[0] : (strcmp(wl, "lenet") == 0 ? 256 : 64);
    if (steps < 1 || steps > TM_MAX_STEPS - 2) return 2;
    g_step_mark = strcmp(wl, "lenet") == 0 ? "lenet.step" : "mlp.step";
    g_out = fopen("/dev/null", "wb");
    if (!g_out) return 1;
    g_mark_hook = tm_mark;
    double mean = 0, waits = 0, reads = 0, disp = 0, med = 0;
    int cpu_only = strcmp(lib, "-") == 0;   /* "-": the CPU leg alone */
    if (!cpu_only) {
        med = tm_hip_leg(lib, wl, B, steps, &mean, &waits, &reads, &disp);
        if (med < 0) return 1;
    }
    /* the engine's CPU backend, the same steps (no compilation to warm up),
     * its buffers in guard regions */
    g_cpu_alloc = cpu_backend.buf_alloc;
    cpu_backend.buf_alloc = tm_guard_alloc;
    cpu_backend.buf_free = tm_guard_free;
    cpu_backend.pool_reset = tm_guard_reset;
    cpu_backend.shutdown = tm_guard_shutdown;
    TinyHVM *cpu = thvm_init("cpu");
    double cmean = 0, cw = 0, cr = 0, cd = 0;
    /* the MLP marks its steps only when it runs more than one (its fixture
     * recording is a single unmarked step), so its CPU sample is 3 steps */
    double cmed = tm_steps(cpu, wl, B, strcmp(wl, "mlp") == 0 ? 3 : 1, &cmean, &cw, &cr, &cd);
    printf("{\"workload\": \"%s\", \"batch\": %u, \"steps\": %d, \"gpu\": {\"median_ms\": %.4f, "
           "\"mean_ms\": %.4f, \"steps_per_s\": %.2f, \"host_waits_per_step\": %.2f, \"reads_per_step\": %.2f, "
           "\"dispatches_per_step\": %.2f, \"waits_outside_reads\": %llu, \"wait_slot\": \"%s\", "
           "\"backend_slots_ms_per_step\": %.4f, \"read_ms_per_step\": %.4f}, "
           "\"cpu\": {\"seconds_per_step\": %.4f, \"steps_per_s\": %.5f}}\n",
           wl, B, steps, med * 1e3, mean * 1e3, med > 0 ? 1.0 / med : 0.0, waits, reads, disp,
           (unsigned long long)g_waits_outside, g_waits_outside_slot, g_hip_bk * 1e3, g_hip_rd * 1e3, cmed,
           cmed > 0 ? 1.0 / cmed : 0.0);
    fflush(stdout);
    return (cpu_only || med > 0) && cmed > 0 ? 0 : 1;
}

/* ---- capture and replay of an engine-driven training step ----
 * engine_live <libthvm_hip.so> jit <lenet|mlp> <steps> [batch]
 *
 * The Metal backend's JIT (src/backend/metal/jit.m:24-631, declared at
 * src/tinyhvm.h:1294-1299, driven by test/archive/test_jit_dense.m:95-157)
 * records the dispatches of one training step that thvm_eval issues and
 * replays them for later steps without the engine; between replays the
 * caller writes the next batch into the same persistent tensors. Here the
 * same with the backend's HIP graphs: on a context made by thvm_init("hip"),
 *   eager  2 warm-up steps (compilation), the parameters restored, then
 *          <steps> training steps through thvm_eval, each after writing its
 *          labels into the persistent one-hot tensor, each loss read from the
 *          persistent tensor the step assigns it to;
 *   graph  the parameters restored, one step through thvm_eval captured
 *          between thvm_hip_graph_begin and thvm_hip_graph_end (nothing
 *          runs), then <steps> launches of that graph, each after writing the
 *          same labels as the eager step of that index, each loss read.
 * Every loss and, at the end, every parameter must be the same bit for bit
 * (the same kernels with the same arguments in the same order). Both legs
 * are timed on the host clock, label write and loss read included. Prints
 * one JSON line; exits 0 when both agree. The step (LeNet-5 as
 * tests/golden/capture.c composes it; the 2-layer MLP with SGD on W1, b1,
 * W2, b2) reads its labels from the one-hot tensor and assigns its loss, so
 * a replay needs no engine work at all. */
typedef struct {
    int lenet;
    u32 B, n_params, keep;
    Term x, onehot, loss_out, params[10];
} JNet;

static void jnet_init(TinyHVM *ctx, JNet *n, int lenet, u32 B) {
    memset(n, 0, sizeof *n);
    n->lenet = lenet;
    n->B = B;
    if (lenet) {
        n->x = lenet_params(ctx, B, n->params);
        n->n_params = 10;
    } else {
        n->x = gen_tensor(ctx, SHAPE(B, 784), DTYPE_F32, TRC_GEN_NORMAL, 1001, 0.f, 1.f);
        n->params[0] = kaiming_u(ctx, SHAPE(784, 128), 784, 1002);
        n->params[1] = zeros(ctx, SHAPE(128), 1003);
        n->params[2] = kaiming_u(ctx, SHAPE(128, 10), 128, 1004);
        n->params[3] = zeros(ctx, SHAPE(10), 1005);
        n->n_params = 4;
    }
    f32 *z = calloc((size_t)B * 10, sizeof(f32));
    n->onehot = thvm_tensor(ctx, z, SHAPE(B, 10));
    free(z);
    f32 zero = 0.0f;
    n->loss_out = thvm_tensor(ctx, &zero, SHAPE(1, 1));
    n->keep = ctx->tensor_count;
}

/* the 2-layer MLP's training step, SGD (lr 0.01) on W1, b1, W2, b2 */
static void mlp_train_step(TinyHVM *ctx, JNet *n) {
    const u32 B = n->B;
    Term *p = n->params;
    Term h = dense(ctx, n->x, p[0], p[1], 1, B, 128);
    Term logits = dense(ctx, h, p[2], p[3], 0, B, 10);
    Term loss = ce_loss_onehot(ctx, logits, n->onehot, B, 10);
    Term d2 = ce_grad(ctx, logits, n->onehot, B, 10);
    DenseGrads g2 = dense_bwd(ctx, h, p[2], d2, B, 128, 10, 1);
    Term dz1 = realize_as(ctx, binary(ctx, UOP_MUL, g2.dx, binary(ctx, UOP_CMP, h, scalar_t(ctx, 0.0f))),
                          SHAPE(B, 128));
    DenseGrads g1 = dense_bwd(ctx, n->x, p[0], dz1, B, 784, 128, 0);
    Term grads[4] = {g1.dW, g1.db, g2.dW, g2.db};
    sgd_keep_loss(ctx, p, grads, 4, 0.01f, n->loss_out, loss);
}

static void jnet_step(TinyHVM *ctx, JNet *n) {
    if (n->lenet) lenet_step(ctx, n->B, n->x, n->params, n->onehot, NULL, n->loss_out);
    else mlp_train_step(ctx, n);
}

static TensorMeta *jmeta(TinyHVM *ctx, Term t) { return &ctx->tensors[(u32)term_val(t)]; }

/* host data into a persistent tensor through its backend, its buffer's epoch
 * bumped as an ASSIGN bumps it (src/interact/tensor_ops.c:142-146), so that
 * no cached kernel result that read the old contents is reused */
static void jwrite(TinyHVM *ctx, Term t, const void *data, u64 bytes) {
    TensorMeta *m = jmeta(ctx, t);
    m->backend->buf_write(m->buf_id, data, bytes);
    if (m->buf_id < MAX_BUF_EPOCHS) buf_epoch[m->buf_id]++;
}

static u64 jbytes(TinyHVM *ctx, Term t) { return (u64)jmeta(ctx, t)->view.numel * 4; }

/* step t's labels (uniform integers in [0,10), seed 7000 + t) as one-hot rows */
static void jnet_labels(TinyHVM *ctx, JNet *n, u32 t) {
    u8 *lab = labels_u8(n->B, 7000 + t);
    f32 *oh = calloc((size_t)n->B * 10, sizeof(f32));
    for (u32 i = 0; i < n->B; i++) oh[i * 10 + lab[i]] = 1.0f;
    jwrite(ctx, n->onehot, oh, (u64)n->B * 10 * sizeof(f32));
    free(oh);
    free(lab);
}

static f32 jloss(TinyHVM *ctx, JNet *n) {
    f32 v = 0.0f;
    TensorMeta *m = jmeta(ctx, n->loss_out);
    m->backend->buf_read(m->buf_id, &v, sizeof v);
    return v;
}

static void jparams_read(TinyHVM *ctx, JNet *n, u8 **out) {
    for (u32 i = 0; i < n->n_params; i++) {
        TensorMeta *m = jmeta(ctx, n->params[i]);
        out[i] = malloc(jbytes(ctx, n->params[i]));
        m->backend->buf_read(m->buf_id, out[i], jbytes(ctx, n->params[i]));
    }
}

static void jparams_write(TinyHVM *ctx, JNet *n, u8 *const *in) {
    for (u32 i = 0; i < n->n_params; i++) jwrite(ctx, n->params[i], in[i], jbytes(ctx, n->params[i]));
}

static int jit_mode(const char *lib, const char *wl, int steps, u32 B) {
    const int lenet = strcmp(wl, "lenet") == 0;
    if ((!lenet && strcmp(wl, "mlp") != 0) || steps < 1 || steps > 100000) return 2;
    if (B == 0) B = lenet ? 256 : 64;
    g_out = fopen("/dev/null", "wb");
    if (!g_out || hip_backend_load(lib, 0) != 0) return 1;
    int (*graph_begin)(void) = (int (*)(void))dlsym(g_hip_lib, "thvm_hip_graph_begin");
    void *(*graph_end)(void) = (void *(*)(void))dlsym(g_hip_lib, "thvm_hip_graph_end");
    int (*graph_launch)(void *) = (int (*)(void *))dlsym(g_hip_lib, "thvm_hip_graph_launch");
    void (*graph_destroy)(void *) = (void (*)(void *))dlsym(g_hip_lib, "thvm_hip_graph_destroy");
    if (!graph_begin || !graph_end || !graph_launch || !graph_destroy) return 1;
    TinyHVM *ctx = thvm_init("hip");
    if (!ctx || ctx->default_device != THVM_DEV_HIP) {
        fprintf(stderr, "engine_live: thvm_init(\"hip\") did not register hip_backend\n");
        return 1;
    }
    JNet n;
    jnet_init(ctx, &n, lenet, B);
    u8 *p0[10], *pe[10], *pg[10];
    jparams_read(ctx, &n, p0);
    f32 *le = calloc((size_t)steps, sizeof(f32)), *lg = calloc((size_t)steps, sizeof(f32));
    if (!le || !lg) return 1;
    /* warm-up: every kernel compiled, every workspace sized */
    for (u32 w = 0; w < 2; w++) {
        jnet_labels(ctx, &n, w);
        jnet_step(ctx, &n);
        (void)jloss(ctx, &n);
        thvm_reset(ctx, n.keep);
    }
    /* eager leg */
    jparams_write(ctx, &n, p0);
    double t0 = now_s();
    for (int t = 0; t < steps; t++) {
        jnet_labels(ctx, &n, (u32)t);
        jnet_step(ctx, &n);
        le[t] = jloss(ctx, &n);
        thvm_reset(ctx, n.keep);
    }
    const double t_eager = now_s() - t0;
    jparams_read(ctx, &n, pe);
    /* graph leg: one engine step captured, then replayed */
    jparams_write(ctx, &n, p0);
    jnet_labels(ctx, &n, 0);
    if (graph_begin() != 0) {
        fprintf(stderr, "engine_live: graph capture could not start\n");
        return 1;
    }
    jnet_step(ctx, &n);
    void *g = graph_end();
    thvm_reset(ctx, n.keep);
    if (!g) {
        fprintf(stderr, "engine_live: the engine's step could not be captured\n");
        return 1;
    }
    t0 = now_s();
    int launch_err = 0;
    for (int t = 0; t < steps; t++) {
        jnet_labels(ctx, &n, (u32)t);
        launch_err |= graph_launch(g) != 0;
        lg[t] = jloss(ctx, &n);
    }
    const double t_graph = now_s() - t0;
    jparams_read(ctx, &n, pg);
    int losses_equal = memcmp(le, lg, (size_t)steps * sizeof(f32)) == 0, params_equal = 1, moved = 0;
    for (u32 i = 0; i < n.n_params; i++) {
        const u64 nb = jbytes(ctx, n.params[i]);
        params_equal &= memcmp(pe[i], pg[i], nb) == 0;
        moved |= memcmp(pe[i], p0[i], nb) != 0;
    }
    int finite = 1;
    for (int t = 0; t < steps; t++) finite &= isfinite(le[t]) != 0;
    graph_destroy(g);
    thvm_free(ctx);
    const int ok = losses_equal && params_equal && moved && finite && !launch_err;
    printf("{\"workload\": \"%s\", \"batch\": %u, \"steps\": %d, \"eager\": {\"ms_per_step\": %.4f, "
           "\"steps_per_s\": %.2f}, \"graph\": {\"ms_per_step\": %.4f, \"steps_per_s\": %.2f}, "
           "\"losses_equal\": %s, \"params_equal\": %s, \"params_moved\": %s, \"loss_first\": %.6f, "
           "\"loss_last\": %.6f, \"ok\": %s}\n",
           wl, B, steps, t_eager * 1e3 / steps, steps / t_eager, t_graph * 1e3 / steps, steps / t_graph,
           losses_equal ? "true" : "false", params_equal ? "true" : "false", moved ? "true" : "false", le[0],
           le[steps - 1], ok ? "true" : "false");
    fflush(stdout);
    return ok ? 0 : 1;
}

int main(int argc, char **argv) {
    if (argc >= 5 && strcmp(argv[2], "jit") == 0)
        return jit_mode(argv[1], argv[3], atoi(argv[4]), argc >= 6 ? (u32)strtoul(argv[5], NULL, 10) : 0);
    if (argc >= 5 && strcmp(argv[2], "time") == 0) {
        u32 tsz[8] = {0}, tn = 0;
        for (int i = 5; i < argc && tn < 8; i++) tsz[tn++] = (u32)strtoul(argv[i], NULL, 10);
        return time_mode(argv[1], argv[3], atoi(argv[4]), tsz, tn);
    }
    if (argc < 3) {
        fprintf(stderr, "usage: engine_live <libthvm_hip.so> <workload> [sizes...]\n");
        return 2;
    }
    u32 sz[8] = {0}, nsz = 0;
    for (int i = 3; i < argc && nsz < 8; i++) sz[nsz++] = (u32)strtoul(argv[i], NULL, 10);

    /* run 0: the engine's CPU backend */
    g_out = fopen("/dev/null", "wb");
    if (!g_out) return 1;
    install_recorder();
    g_inner_read = cpu_backend.buf_read;
    cpu_backend.buf_read = live_read;
    g_run = 0;
    TinyHVM *cpu_ctx = thvm_init("cpu");
    double t0 = now_s();
    if (!run_workload(cpu_ctx, argv[2], sz, nsz)) {
        fprintf(stderr, "unknown workload %s\n", argv[2]);
        return 2;
    }
    double t_cpu = now_s() - t0;

    /* run 1: thvm_init("hip") registers hip_backend as the default device */
    if (hip_backend_load(argv[1], 0) != 0) return 1;
    Backend *hb = g_hip_backend;
    static Backend live_hip;
    live_hip = *hb;
    g_inner_read = hb->buf_read;
    live_hip.buf_read = live_read;
    g_hip_backend = &live_hip;
    g_run = 1;
    TinyHVM *ctx = thvm_init("hip");
    if (!ctx || ctx->default_device != THVM_DEV_HIP) {
        fprintf(stderr, "engine_live: thvm_init(\"hip\") did not register hip_backend\n");
        return 1;
    }
    t0 = now_s();
    run_workload(ctx, argv[2], sz, nsz);
    double t_gpu = now_s() - t0;
    /* thvm_free shuts every registered backend down (src/ctx/init.c:65-77) */
    thvm_free(ctx);
    int (*sync)(void) = (int (*)(void))dlsym(g_hip_lib, "thvm_hip_synchronize");
    const int shut_down = sync && sync() == -1;

    int ok = g_nreads[0] == g_nreads[1] && g_nreads[0] > 0;
    double worst = 0.0;
    printf("{\"workload\": \"%s\", \"reads\": [%u, %u], \"cpu_seconds\": %.4f, \"gpu_seconds\": %.4f, \"results\": [",
           argv[2], g_nreads[0], g_nreads[1], t_cpu, t_gpu);
    u32 n = g_nreads[0] < g_nreads[1] ? g_nreads[0] : g_nreads[1];
    for (u32 i = 0; i < n; i++) {
        const LiveRead *a = &g_reads[0][i], *b = &g_reads[1][i];
        double err = 0.0, mx = 0.0;
        int same = a->n == b->n;
        if (same) {
            const f32 *x = (const f32 *)b->data, *y = (const f32 *)a->data;
            for (u64 j = 0; j < a->n / 4; j++) {
                if (isnan(x[j]) || isnan(y[j])) {
                    if (isnan(x[j]) != isnan(y[j])) same = 0;
                    continue;
                }
                double d = fabs((double)x[j] - (double)y[j]);
                if (d > err) err = d;
                if (fabs((double)y[j]) > mx) mx = fabs((double)y[j]);
            }
            err = mx > 0 ? err / mx : err;
        }
        if (!same) err = 1e30;
        if (err > worst) worst = err;
        printf("%s[%llu, %.3e]", i ? ", " : "", (unsigned long long)a->n, err);
    }
    ok = ok && worst <= 1e-3 && shut_down;
    printf("], \"worst\": %.3e, \"registered_by_thvm_init\": true, \"shut_down_by_thvm_free\": %s, "
           "\"ok\": %s}\n", worst, shut_down ? "true" : "false", ok ? "true" : "false");
    fflush(stdout);
    return ok ? 0 : 1;
}
