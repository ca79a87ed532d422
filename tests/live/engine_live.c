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
 *   run 1  with `hip_backend` registered as the engine's default device, as
 *          the thvm_init branch for "hip" registers it (the engine's
 *          src/ctx/init.c:23-37 does the same for Metal).
 * Every buffer the workload reads back (Backend.buf_read) is kept from both
 * runs and compared: same sequence and sizes, values within 1e-3 normwise
 * (max |gpu - cpu| / max |cpu| per read, as float32), NaNs in the same places.
 * Prints one JSON line and exits 0 when every read agrees.
 */
#define CAPTURE_NO_MAIN
#include "../golden/capture.c"

#include <dlfcn.h>
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

int main(int argc, char **argv) {
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

    /* run 1: hip_backend as the engine's default device */
    void *h = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
    if (!h) {
        fprintf(stderr, "engine_live: %s\n", dlerror());
        return 1;
    }
    Backend *hb = (Backend *)dlsym(h, "hip_backend");
    if (!hb || !hb->init || hb->init() != 0) {
        fprintf(stderr, "engine_live: hip_backend unavailable\n");
        return 1;
    }
    static Backend live_hip;
    live_hip = *hb;
    g_inner_read = hb->buf_read;
    live_hip.buf_read = live_read;
    g_run = 1;
    TinyHVM *ctx = thvm_init("cpu");
    ctx->backends[2] = &live_hip;
    if (ctx->n_backends < 3) ctx->n_backends = 3;
    ctx->default_device = 2;
    t0 = now_s();
    run_workload(ctx, argv[2], sz, nsz);
    double t_gpu = now_s() - t0;

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
    ok = ok && worst <= 1e-3;
    printf("], \"worst\": %.3e, \"ok\": %s}\n", worst, ok ? "true" : "false");
    fflush(stdout);
    hb->shutdown();
    return ok ? 0 : 1;
}
