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
#include <pthread.h>
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

static u64 uop_signature_(const UOpKernel *k);

u64 uop_signature(const UOpKernel *k) {
    if (k && k == hipb.sig_k && hipb.sig_h) return hipb.sig_h;
    const u64 t0 = hipb_hp_now();
    const u64 h = uop_signature_(k);
    hipb_hp_add(HP_SIGNATURE, t0);
    if (k && k == hipb.sig_k) hipb.sig_h = h;
    return h;
}

static u64 uop_signature_(const UOpKernel *k) {
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
                free(R.tab[i].chain);
                co_form_free(&R.tab[i].co);
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

/* Code objects compiled in this process, by source text: a backend that is
 * shut down and initialised again (tests, a serving process that restarts
 * its context) loads them instead of compiling again. The whole text is
 * compared on a hit; at most CODE_CACHE_BYTES are kept. */
#define CODE_CACHE_BYTES (256ull << 20)
typedef struct CodeEnt {
    u64 h;
    char *src;
    char *code;
    size_t len;
    struct CodeEnt *next;
} CodeEnt;
static struct {
    CodeEnt *bucket[1024];
    u64 bytes;
    pthread_mutex_t mu;
} CC = {.mu = PTHREAD_MUTEX_INITIALIZER};

static u64 text_hash(const char *s) {
    u64 h = 0xcbf29ce484222325ull;
    for (; *s; s++) h = (h ^ (u8)*s) * 0x100000001b3ull;
    return h;
}

static char *code_cache_get(const char *src, u64 h, size_t *len) {
    char *out = NULL;
    pthread_mutex_lock(&CC.mu);
    for (CodeEnt *e = CC.bucket[h & 1023]; e; e = e->next)
        if (e->h == h && strcmp(e->src, src) == 0) {
            out = malloc(e->len);
            if (out) {
                memcpy(out, e->code, e->len);
                *len = e->len;
            }
            break;
        }
    pthread_mutex_unlock(&CC.mu);
    return out;
}

static void code_cache_put(const char *src, u64 h, const char *code, size_t len) {
    const size_t sl = strlen(src) + 1;
    pthread_mutex_lock(&CC.mu);
    if (CC.bytes + sl + len <= CODE_CACHE_BYTES) {
        CodeEnt *e = malloc(sizeof *e);
        char *s2 = e ? malloc(sl) : NULL, *c2 = s2 ? malloc(len) : NULL;
        if (c2) {
            memcpy(s2, src, sl);
            memcpy(c2, code, len);
            e->h = h;
            e->src = s2;
            e->code = c2;
            e->len = len;
            e->next = CC.bucket[h & 1023];
            CC.bucket[h & 1023] = e;
            CC.bytes += sl + len;
        } else {
            free(s2);
            free(e);
        }
    }
    pthread_mutex_unlock(&CC.mu);
}

/* Compile HIP source to a gfx950 code object. Returns malloc'd code. */
static char *compile_source(const char *src, size_t *code_len, char *err, size_t errlen) {
    const u64 h = text_hash(src);
    char *hit = code_cache_get(src, h, code_len);
    if (hit) return hit;
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
    if (code) code_cache_put(src, h, code, cs);
    return code;
}

/* A loaded module's pointer to the combine give-up word (thvm_comb_err_, in
 * the prelude) is set to the backend's word, by a copy on a stream of its
 * own: a module first built while the main stream is captured into a graph
 * (a batch of launches first seen there) is set up the same way. */
static void module_setup(hipModule_t mod) {
    if (!hipb.comb_err_dev) return;
    hipDeviceptr_t p = 0;
    size_t n = 0;
    if (hipModuleGetGlobal(&p, &n, mod, "thvm_comb_err_") != hipSuccess || n != sizeof(void *)) {
        (void)hipGetLastError();   /* the module has no combine: nothing to set */
        return;
    }
    HIPB_CHECK(hipMemcpyHtoDAsync(p, &hipb.comb_err_dev, sizeof(void *), hipb.setup_stream));
    HIPB_CHECK(hipStreamSynchronize(hipb.setup_stream));
}

u32 rtc_capacity(hipFunction_t fn, u32 block) {
    int nb = 0;
    if (!fn || block == 0 || hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, (int)block, 0) != hipSuccess ||
        nb <= 0) {
        (void)hipGetLastError();
        return 0;
    }
    return (u32)nb * (hipb.n_cu ? hipb.n_cu : 256u);
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
    module_setup(*mod);
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

/* Co-launch form of a generated module (see CoForm): the source after the
 * shared prelude inside namespace co_<id>, every `extern "C" __global__`
 * kernel turned into a __device__ function whose block coordinates, grid
 * size and lane are its first arguments (blockIdx.x/.y, gridDim.x/.y and
 * threadIdx.x read them), so that a caller may run several of its workgroups
 * side by side in one larger workgroup. The prelude's block-wide helpers,
 * which read blockDim, become their forms with the program's wave count
 * fixed. Modules that use a third grid or thread dimension, blockDim,
 * dynamic LDS or includes keep cf->src NULL and launch on their own. */
static u32 co_next_id;

static int co_param_sizes(CoForm *cf) {
    const char *p = cf->params;
    cf->np = 0;
    while (*p) {
        while (*p == ' ' || *p == ',') p++;
        if (!*p) break;
        const char *e = strchr(p, ',');
        size_t len = e ? (size_t)(e - p) : strlen(p);
        if (cf->np >= CO_MAX_PARAMS) return 0;
        int ptr = memchr(p, '*', len) != NULL;
        int ll = 0;
        for (size_t t = 0; t + 9 <= len; t++) ll |= memcmp(p + t, "long long", 9) == 0;
        cf->psz[cf->np++] = (u8)((ptr || ll) ? 8 : 4);
        p += len;
    }
    return cf->np > 0;
}

int co_form_make(CoForm *cf, const char *src, const char *name, u32 threads, hipFunction_t fn) {
    memset(cf, 0, sizeof *cf);
    const char *pre = kgen_prelude();
    const size_t pl = strlen(pre);
    if (!src || strncmp(src, pre, pl) != 0 || strlen(name) >= sizeof cf->name) return 0;
    const char *body = src + pl;
    if (strstr(body, "blockIdx.z") || strstr(body, "gridDim.z") || strstr(body, "blockDim") ||
        strstr(body, "threadIdx.y") || strstr(body, "threadIdx.z") ||
        strstr(body, "extern __shared__") || strstr(body, "#include"))
        return 0;
    /* the main kernel's parameter list */
    char head[96];
    snprintf(head, sizeof head, " void %s(", name);
    const char *h = strstr(body, head);
    if (!h) return 0;
    const char *ps = h + strlen(head), *pe = strstr(ps, ") {");
    if (!pe) return 0;
    cf->params = malloc((size_t)(pe - ps) + 1);
    if (!cf->params) return 0;
    memcpy(cf->params, ps, (size_t)(pe - ps));
    cf->params[pe - ps] = 0;
    if (!co_param_sizes(cf)) goto fail;
    /* the transformed module */
    static const char kg[] = "extern \"C\" __global__ ", lb[] = "__launch_bounds__(";
    size_t cap = strlen(body) * 2 + 256;
    char *o = malloc(cap);
    if (!o) goto fail;
    cf->id = ++co_next_id;
    size_t w = (size_t)snprintf(o, cap, "namespace co_%u {\n", cf->id);
    const char *q = body;
    while (*q) {
        if (w + 128 >= cap) {
            char *n2 = realloc(o, cap * 2);
            if (!n2) { free(o); goto fail; }
            o = n2;
            cap *= 2;
        }
        if (strncmp(q, kg, sizeof kg - 1) == 0) {
            q += sizeof kg - 1;
            if (strncmp(q, lb, sizeof lb - 1) == 0) {
                const char *r = strchr(q, ')');
                if (!r) { free(o); goto fail; }
                q = r + 1;
                while (*q == ' ') q++;
            }
            /* a kernel attribute (waves per SIMD) does not apply to a device function */
            if (strncmp(q, "__attribute__((", 15) == 0) {
                int depth = 0;
                const char *r = q + 13;
                do {
                    if (*r == '(') depth++;
                    else if (*r == ')') depth--;
                    r++;
                } while (*r && depth > 0);
                if (depth != 0) { free(o); goto fail; }
                q = r;
                while (*q == ' ') q++;
            }
            if (strncmp(q, "void ", 5) != 0) { free(o); goto fail; }
            const char *par = strchr(q, '(');
            if (!par) { free(o); goto fail; }
            w += (size_t)snprintf(o + w, cap - w, "__device__ __forceinline__ %.*su32 bx_, u32 by_, u32 gx_, u32 gy_, u32 tx_, ",
                                  (int)(par + 1 - q), q);
            q = par + 1;
        } else if (strncmp(q, "bsum(", 5) == 0 || strncmp(q, "bmax(", 5) == 0) {
            /* the block-wide helpers with the program's own wave count */
            w += (size_t)snprintf(o + w, cap - w, "%.4s_n<%uu>(", q, threads / 64u);
            q += 5;
        } else if (strncmp(q, "threadIdx.x", 11) == 0) {
            /* the lane within the program's own workgroup */
            w += (size_t)snprintf(o + w, cap - w, "tx_");
            q += 11;
        } else if (strncmp(q, "blockIdx.x", 10) == 0 || strncmp(q, "blockIdx.y", 10) == 0) {
            w += (size_t)snprintf(o + w, cap - w, "b%c_", q[9]);
            q += 10;
        } else if (strncmp(q, "gridDim.x", 9) == 0 || strncmp(q, "gridDim.y", 9) == 0) {
            w += (size_t)snprintf(o + w, cap - w, "g%c_", q[8]);
            q += 9;
        } else {
            o[w++] = *q++;
        }
    }
    o[w] = 0;
    if (strstr(o, "__global__") || w + 8 >= cap) { free(o); goto fail; }
    snprintf(o + w, cap - w, "}\n");
    cf->src = o;
    snprintf(cf->name, sizeof cf->name, "%s", name);
    cf->threads = threads;
    cf->no_sync = !strstr(o, "__syncthreads") && !strstr(o, "bsum_n<") && !strstr(o, "bmax_n<") &&
                  !strstr(o, "__shared__");
    if (fn) {   /* NULL: a device-free check */
        int v = 0;
        if (hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, fn) != hipSuccess || v < 0) goto fail_src;
        cf->lds = (u32)v;
        cf->cap_waves = rtc_capacity(fn, threads) * (threads / 64u);
    }
    return 1;
fail_src:
    free(cf->src);
fail:
    free(cf->params);
    memset(cf, 0, sizeof *cf);
    return 0;
}

void co_form_free(CoForm *cf) {
    free(cf->src);
    free(cf->params);
    memset(cf, 0, sizeof *cf);
}

KCacheEntry *rtc_compile_uop(u64 key, const UOpKernel *k) {
    char err[256] = {0};
    KGenResult g;
    if (hipb.rtc_fail) return NULL;   /* test knob: every compile fails */
    int comb_launch = 0;
again:
    hipb.force_combine_launch = comb_launch;
    const int gen_ok = kgen_uop(k, &g, err, sizeof err);
    hipb.force_combine_launch = 0;
    if (!gen_ok) {
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
    module_setup(mod);
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
    /* one pass only if the whole grid is on the GPU at once with this
     * kernel's own occupancy (registers, LDS); else the combine kernel */
    if (g.splits > 1 && !g.combine_launch && !comb_launch &&
        (u64)g.total * g.splits > rtc_capacity(fn, g.block)) {
        if (hipb.verbose)
            fprintf(stderr, "tinyhvm-hip: %s: %llu workgroups exceed what the GPU holds at once (%u): combine kernel\n",
                    g.name, (unsigned long long)g.total * g.splits, rtc_capacity(fn, g.block));
        HIPB_CHECK(hipModuleUnload(mod));
        kgen_free(&g);
        comb_launch = 1;
        goto again;
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
    /* split reductions with a combine kernel are two launches: not co-launched */
    if (!g.combine_launch) co_form_make(&e->co, g.src, g.name, g.block, fn);
    e->store_slots = chain_store_slots(k);
    e->chain = (e->ops && g.mode != KG_MODE_GROUP && g.splits <= 1) ? chain_info_make(k, e->ops) : NULL;
    hipb.n_compile++;
    kgen_free(&g);
    return e;
}
