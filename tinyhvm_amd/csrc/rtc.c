/*
 * rtc.c - hipRTC compilation of generated kernels and the module cache.
 *
 * Cache identity: the fields the generated code depends on (op list, leaf
 * count and dtypes, output dtype, grid, local_size). That is what the engine's
 * thvm_uop_kernel_signature covers (src/tinyhvm.h:878-906) minus the leaf
 * views, which the KOp program already encodes; the engine's own cache_key
 * (KernelEntry signature, src/tinyhvm.h:866-876) omits dtypes and is not used.
 * A hit is confirmed by comparing the stored op list, so a hash collision
 * compiles a new kernel instead of running the wrong one.
 *
 * Compile options: gfx950, -O3, no FP contraction (a*b+c stays two rounded
 * ops, as in the x86 reference build), packed FP32 instructions disabled.
 */
#include <stdlib.h>
#include <string.h>
#include <hip/hiprtc.h>

#include "hipb.h"

extern const unsigned char thvm_static_kernels_co[];
extern const unsigned long thvm_static_kernels_co_len;

static struct {
    KCacheEntry *tab;
    u32 cap, n;
    int static_loaded;
} R;

static const char *RTC_OPTS[] = {
    "--offload-arch=gfx950", "-O3", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
};

static u64 mix(u64 h, u64 v) {
    h ^= v + 0x9E3779B97F4A7C15ull + (h << 6) + (h >> 2);
    h *= 0xFF51AFD7ED558CCDull;
    return h ^ (h >> 33);
}

u64 uop_signature(const UOpKernel *k) {
    u64 h = 0x746876686970ull;
    h = mix(h, k->n_ops);
    h = mix(h, k->n_leaves);
    h = mix(h, k->out_dtype);
    h = mix(h, k->local_size);
    for (int i = 0; i < 3; i++) h = mix(h, k->grid[i]);
    for (u32 i = 0; i < k->n_leaves && i < FUSE_MAX_LEAVES; i++) h = mix(h, k->leaf_dtypes[i]);
    u32 n = k->n_ops < KOP_MAX ? k->n_ops : KOP_MAX;
    for (u32 i = 0; i < n; i++) {
        const KOp *op = &k->ops[i];
        h = mix(h, ((u64)op->type << 32) ^ op->imm.u);
        h = mix(h, ((u64)op->arg[0] << 32) ^ op->arg[1]);
        h = mix(h, op->arg[2]);
    }
    return h ? h : 1;
}

static void program_meta(const UOpKernel *k, u32 *m) {
    memset(m, 0, (5 + FUSE_MAX_LEAVES) * sizeof(u32));
    m[0] = k->grid[0]; m[1] = k->grid[1]; m[2] = k->grid[2];
    m[3] = k->local_size; m[4] = k->out_dtype;
    for (u32 i = 0; i < k->n_leaves && i < FUSE_MAX_LEAVES; i++) m[5 + i] = k->leaf_dtypes[i];
}

static int same_program(const KCacheEntry *e, const UOpKernel *k) {
    if (e->n_ops != k->n_ops || e->n_leaves != k->n_leaves || !e->ops) return 0;
    u32 m[5 + FUSE_MAX_LEAVES];
    program_meta(k, m);
    if (memcmp(m, e->meta, sizeof m) != 0) return 0;
    return memcmp(e->ops, k->ops, (size_t)k->n_ops * sizeof(KOp)) == 0;
}

int rtc_init(void) {
    R.cap = 1024;
    R.n = 0;
    R.tab = calloc(R.cap, sizeof(KCacheEntry));
    if (!R.tab) return -1;
    hipError_t e = hipModuleLoadData(&hipb.static_mod, thvm_static_kernels_co);
    if (e != hipSuccess) {
        fprintf(stderr, "tinyhvm-hip: loading the static kernel module failed: %s\n",
                hipGetErrorString(e));
        return -1;
    }
    R.static_loaded = 1;
    return 0;
}

void rtc_shutdown(void) {
    if (R.tab) {
        for (u32 i = 0; i < R.cap; i++) {
            if (R.tab[i].key) {
                HIPB_CHECK(hipModuleUnload(R.tab[i].mod));
                free(R.tab[i].ops);
                free(R.tab[i].bsrc);
                free(R.tab[i].bparams);
            }
        }
        free(R.tab);
    }
    if (R.static_loaded) HIPB_CHECK(hipModuleUnload(hipb.static_mod));
    memset(&R, 0, sizeof(R));
}

hipFunction_t rtc_static_fn(const char *name) {
    hipFunction_t f = NULL;
    if (!R.static_loaded) return NULL;
    if (hipModuleGetFunction(&f, hipb.static_mod, name) != hipSuccess) {
        fprintf(stderr, "tinyhvm-hip: static kernel %s not found\n", name);
        return NULL;
    }
    return f;
}

KCacheEntry *rtc_lookup(u64 key, const UOpKernel *k) {
    if (!R.tab) return NULL;
    u32 m = R.cap - 1;
    for (u32 p = (u32)key & m, probes = 0; probes < R.cap; p = (p + 1) & m, probes++) {
        KCacheEntry *e = &R.tab[p];
        if (!e->key) return NULL;
        if (e->key == key && same_program(e, k)) return e;
    }
    return NULL;
}

static KCacheEntry *insert_slot(u64 key) {
    if ((R.n + 1) * 2 > R.cap) {
        u32 nc = R.cap * 2;
        KCacheEntry *nt = calloc(nc, sizeof(KCacheEntry));
        if (!nt) return NULL;
        for (u32 i = 0; i < R.cap; i++) {
            if (!R.tab[i].key) continue;
            u32 p = (u32)R.tab[i].key & (nc - 1);
            while (nt[p].key) p = (p + 1) & (nc - 1);
            nt[p] = R.tab[i];
        }
        free(R.tab);
        R.tab = nt;
        R.cap = nc;
    }
    u32 m = R.cap - 1;
    u32 p = (u32)key & m;
    while (R.tab[p].key) p = (p + 1) & m;
    R.n++;
    return &R.tab[p];
}

/* Compile HIP source to a gfx950 code object. Returns malloc'd code. */
static char *compile_source(const char *src, size_t *code_len, char *err, size_t errlen) {
    hiprtcProgram prog;
    if (hiprtcCreateProgram(&prog, src, "thvm_kernel.hip", 0, NULL, NULL) != HIPRTC_SUCCESS) {
        snprintf(err, errlen, "hiprtcCreateProgram failed");
        return NULL;
    }
    hiprtcResult rc = hiprtcCompileProgram(prog, (int)(sizeof RTC_OPTS / sizeof RTC_OPTS[0]), RTC_OPTS);
    if (rc != HIPRTC_SUCCESS) {
        size_t ls = 0;
        hiprtcGetProgramLogSize(prog, &ls);
        char *log = malloc(ls + 1);
        if (log) {
            hiprtcGetProgramLog(prog, log);
            log[ls] = 0;
            fprintf(stderr, "tinyhvm-hip: hipRTC compile failed:\n%s\n", log);
            free(log);
        }
        snprintf(err, errlen, "hipRTC compile failed (%s)", hiprtcGetErrorString(rc));
        hiprtcDestroyProgram(&prog);
        return NULL;
    }
    size_t cs = 0;
    hiprtcGetCodeSize(prog, &cs);
    char *code = malloc(cs);
    if (code) hiprtcGetCode(prog, code);
    hiprtcDestroyProgram(&prog);
    *code_len = cs;
    return code;
}

int rtc_build_module(const char *src, hipModule_t *mod, char *err, size_t errlen) {
    size_t cs = 0;
    char *code = compile_source(src, &cs, err, errlen);
    if (!code) return 0;
    hipError_t he = hipModuleLoadData(mod, code);
    free(code);
    if (he != hipSuccess) {
        snprintf(err, errlen, "hipModuleLoadData: %s", hipGetErrorString(he));
        return 0;
    }
    hipb.n_compile++;
    return 1;
}

long rtc_compile_only(const char *src, char *err, size_t errlen) {
    size_t cs = 0;
    char *code = compile_source(src, &cs, err, errlen);
    if (!code) return -1;
    free(code);
    return (long)cs;
}

/* Generate and compile without loading: usable without a GPU. */
int rtc_compile_check(const UOpKernel *k, size_t *code_len, char *err, size_t errlen) {
    KGenResult g;
    if (!kgen_uop(k, &g, err, errlen)) return 0;
    char *code = compile_source(g.src, code_len, err, errlen);
    kgen_free(&g);
    if (!code) return 0;
    free(code);
    return 1;
}

/* The batch form of a serial 256-lane kernel (see KCacheEntry): its
 * parameter list, and its text with the entry line made a device function
 * that takes the workgroup index as bk_. Only when the kernel reads its
 * workgroup index in the one place the generator emits it. */
static void make_batch_form(KCacheEntry *e, const char *src, const char *name) {
    char head[96];
    snprintf(head, sizeof head, "extern \"C\" __global__ __launch_bounds__(256) void %s(", name);
    const char *h = strstr(src, head);
    if (!h) return;
    const char *ps = h + strlen(head);
    const char *pe = strstr(ps, ") {\n");
    if (!pe) return;
    static const char tpat[] = "((unsigned long long)blockIdx.y * gridDim.x + blockIdx.x)";
    const char *t = strstr(pe, tpat);
    if (!t || strstr(t + strlen(tpat), "blockIdx") || strstr(t + strlen(tpat), "gridDim") ||
        strstr(pe, "__shared__") || strstr(pe, "__syncthreads"))
        return;
    size_t np = (size_t)(pe - ps), nb1 = (size_t)(t - (pe + 4)), nrest = strlen(t + strlen(tpat));
    char *params = malloc(np + 1);
    size_t cap = strlen(name) + np + nb1 + nrest + 128;
    char *b = malloc(cap);
    if (!params || !b) {
        free(params);
        free(b);
        return;
    }
    memcpy(params, ps, np);
    params[np] = 0;
    int w = snprintf(b, cap, "__device__ __forceinline__ void %s_b(u32 bk_, %s) {\n", name, params);
    memcpy(b + w, pe + 4, nb1);
    w += (int)nb1;
    w += snprintf(b + w, cap - (size_t)w, "((unsigned long long)bk_)");
    memcpy(b + w, t + strlen(tpat), nrest + 1);
    e->bparams = params;
    e->bsrc = b;
}

KCacheEntry *rtc_compile_uop(u64 key, const UOpKernel *k) {
    char err[256] = {0};
    KGenResult g;
    if (hipb.rtc_fail) return NULL;   /* test knob: every compile fails */
    if (!kgen_uop(k, &g, err, sizeof err)) {
        fprintf(stderr, "tinyhvm-hip: kernel rejected: %s\n", err);
        return NULL;
    }
    if (hipb.dump_src) fprintf(stderr, "---- generated kernel %016llx ----\n%s\n", (unsigned long long)key, g.src);
    size_t cs = 0;
    char *code = compile_source(g.src, &cs, err, sizeof err);
    if (!code) {
        kgen_free(&g);
        return NULL;
    }
    hipModule_t mod;
    hipError_t he = hipModuleLoadData(&mod, code);
    free(code);
    if (he != hipSuccess) {
        fprintf(stderr, "tinyhvm-hip: hipModuleLoadData failed: %s\n", hipGetErrorString(he));
        kgen_free(&g);
        return NULL;
    }
    hipFunction_t fn, fn_fin = NULL;
    char fin_name[48];
    snprintf(fin_name, sizeof fin_name, "%s_fin", g.name);
    if (hipModuleGetFunction(&fn, mod, g.name) != hipSuccess ||
        (g.combine_launch && hipModuleGetFunction(&fn_fin, mod, fin_name) != hipSuccess)) {
        fprintf(stderr, "tinyhvm-hip: kernel symbol missing\n");
        HIPB_CHECK(hipModuleUnload(mod));
        kgen_free(&g);
        return NULL;
    }
    KCacheEntry *e = insert_slot(key);
    if (!e) {
        HIPB_CHECK(hipModuleUnload(mod));
        kgen_free(&g);
        return NULL;
    }
    e->key = key;
    e->mod = mod;
    e->fn = fn;
    e->fn_fin = fn_fin;
    e->splits = g.splits > 1 ? g.splits : 1;
    e->n_scal = g.n_scal;
    memcpy(e->scal_leaf, g.scal_leaf, sizeof e->scal_leaf);
    memcpy(e->scal_index, g.scal_index, sizeof e->scal_index);
    e->scal_only_leaves = g.scal_only_leaves;
    e->mode = g.mode;
    e->vec = g.vec;
    e->block = g.block;
    e->total = g.total;
    e->n_threads = g.n_threads;
    e->n_ops = k->n_ops;
    e->n_leaves = k->n_leaves;
    program_meta(k, e->meta);
    e->ops = malloc((size_t)k->n_ops * sizeof(KOp));
    if (e->ops) memcpy(e->ops, k->ops, (size_t)k->n_ops * sizeof(KOp));
    snprintf(e->name, sizeof e->name, "%s", g.name);
    e->bsrc = e->bparams = NULL;
    if (g.mode == KG_MODE_SERIAL && g.splits <= 1 && g.block == 256) make_batch_form(e, g.src, g.name);
    hipb.n_compile++;
    kgen_free(&g);
    return e;
}
