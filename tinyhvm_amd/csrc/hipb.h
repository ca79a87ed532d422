/*
 * hipb.h - internal interfaces of the HIP backend (plain C, HIP runtime C API).
 *
 * Components:
 *   pool.c     device buffer pool: u32 ids -> device blocks, size classes,
 *              refcounts, persistent floor, pinned staging for host copies
 *   kgen.c     KOp program analysis and HIP source generation
 *   rtc.c      hipRTC compilation and the module cache
 *   dense.c    recognizers that route dense UOpKernels to hand-written kernels
 *   backend.c  the Backend vtable (hip_backend) and dispatch
 *   replay.c   kernel-trace replay
 */
#ifndef HIPB_H
#define HIPB_H

#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <hip/hip_runtime_api.h>

#include "thvm_abi.h"
#include "affine.h"

#define HIPB_CHECK(expr)                                                         \
    do {                                                                         \
        hipError_t e_ = (expr);                                                  \
        if (e_ != hipSuccess) {                                                  \
            fprintf(stderr, "tinyhvm-hip: %s failed: %s (%s:%d)\n", #expr,      \
                    hipGetErrorString(e_), __FILE__, __LINE__);                  \
        }                                                                        \
    } while (0)

/* ---------------- global state ---------------- */

/* host-time categories of THVM_HIP_HOST_PROFILE */
enum { HP_DISPATCH = 0, HP_LAUNCH, HP_SIGNATURE, HP_POOL, HP_WRITE, HP_N };
typedef struct {
    int initialized;
    int device;
    hipStream_t stream;
    hipStream_t setup_stream; /* module set-up copies (legal while the main stream is captured) */
    int sync_each;           /* THVM_HIP_SYNC: synchronize after every dispatch */
    int dump_src;            /* THVM_HIP_DUMP: print generated HIP source */
    int no_dense;            /* THVM_HIP_NO_DENSE: skip dense recognizers */
    int no_window;           /* THVM_HIP_NO_WINDOW: skip the window-max and run-sum kernels */
    int verbose;             /* THVM_HIP_VERBOSE */
    int dense_force;         /* THVM_HIP_DENSE_FORCE: matrix cores for every contraction */
    u32 dense_splits;        /* THVM_HIP_DENSE_SPLITS: fixed split-K factor (0: chosen) */
    void *dummy;             /* 256 zero bytes: the pointer argument of an absent buffer */
    u64 dummy_cap;
    u32 gemm_pad_k;          /* THVM_HIP_GEMM_PAD: LDS row padding for k-major operand stages */
    int gemm_pad_k_set;      /* ... when set (else chosen per store layout) */
    u32 gemm_bk;             /* THVM_HIP_GEMM_BK: K per stage of the LDS tiles (0: the tile's own) */
    u32 gemm_depth;          /* THVM_HIP_GEMM_DEPTH: stages of loads in flight, 1 or 2 (0: chosen) */
    u32 gemm_prio;           /* THVM_HIP_GEMM_PRIO: a wave's priority raised over its stage's math on
                                the LDS tiles: 0 = chosen (the long-K weight gradients), 1 = on every
                                tile, 2 = on none */
    u32 direct_waves;        /* THVM_HIP_DIRECT_WAVES: waves per direct-kernel block, 4, 8 or 16 (0: chosen) */
    int dense_nosep;         /* THVM_HIP_DENSE_NOSEP: evaluate every operand through its program */
    int dense_nokperm;       /* THVM_HIP_DENSE_NOKPERM: no K-reordered affine loaders */
    int dense_novec;         /* THVM_HIP_DENSE_NOVEC: no 16-byte operand loads */
    int dense_noswap;        /* THVM_HIP_DENSE_NOSWAP: lanes along n in every GEMM epilogue */
    int dense_nopack;        /* THVM_HIP_DENSE_NOPACK: never pack a GEMM's B side */
    int dense_noskinny;      /* THVM_HIP_DENSE_NOSKINNY: no row-per-lane kernel for N <= 16 */
    int dense_noskinny_blocks; /* THVM_HIP_DENSE_NOSKBLK: the row-per-lane kernel walks K per k */
    int dense_nored;         /* THVM_HIP_DENSE_NORED: no outer-product reduction kernel */
    int dense_nocomb;        /* THVM_HIP_DENSE_NOCOMB: split-K partials always through a sum kernel */
    int dense_nowave;        /* THVM_HIP_DENSE_NOWAVE: no LDS-free wave-tile kernel for 64-column contractions */
    int dense_notail;        /* THVM_HIP_DENSE_NOTAIL: the wave tile's last tiles are not split */
    u32 wave_tail_s;         /* THVM_HIP_WAVE_TAIL_S: waves per workgroup of the split (2, 4, 8; 0 = 4) */
    int no_fuse;             /* THVM_HIP_NO_FUSE: no elementwise consumer fused into a contraction's epilogue */
    u32 direct_min_chunk;    /* THVM_HIP_DIRECT_MIN_CHUNK: shortest K chunk of a direct-kernel split (0: chosen) */
    int dense_pack;          /* THVM_HIP_DENSE_PACK: pack wherever the layout allows (tests) */
    u32 dense_tile;          /* THVM_HIP_DENSE_TILE: 0 chosen, 1 128x128, 2 64x64, 3 256x32, 4 32x256, 5 direct,
                                6 256x64, 7 128x64, 8 skinny (where N <= 16), 9 outer-product reduction
                                (where it applies), 10 128x64 of 4 waves x 32x64, 11 wave tile (where it
                                applies) */
    int force_interp;        /* THVM_HIP_INTERP: run generated-kernel programs on the KOp interpreter */
    int rtc_fail;            /* THVM_HIP_RTC_FAIL: treat every program compile as failed (tests) */
    u64 n_dispatch, n_compile, n_cache_hit, n_dense;
    u64 n_fallback;          /* dispatches run on the KOp interpreter */
    u64 n_window;            /* dispatches run on the window-max and run-sum kernels */
    u64 n_batched;           /* dispatches issued inside a batched launch */
    u64 n_fused;             /* elementwise dispatches run as a contraction's fused epilogue */
    u64 n_copy_fused;        /* buffer copies written by the launch of the program that produced them */
    u64 n_upload_held;       /* host uploads copied by a held upload kernel */
    u64 n_seq;               /* dispatches issued as steps of a sequence kernel */
    int host_profile;        /* THVM_HIP_HOST_PROFILE: host time per category, printed by profile_report */
    u64 hp_ns[HP_N], hp_calls[HP_N];
    int no_batch;            /* THVM_HIP_NO_BATCH: launch every dispatch on its own */
    int no_seq;              /* THVM_HIP_NO_SEQ: no sequence kernels for dependent small launches */
    u64 n_stream_sync;       /* host waits on the stream (buf_read, synchronize, ...) */
    hipModule_t static_mod;  /* precompiled kernels */
    unsigned long long *comb_slots; /* single-pass combines: partial words (cleared after each use) */
    u32 resident_waves;      /* waves the device holds at once for a single-pass grid */
    u32 n_cu;                /* compute units (256 on MI355X; assumed where no device is open) */
    void *noalloc_scratch;   /* device address of the static workspace (noalloc.hip), or NULL */
    int noalloc;             /* a no-allocation dispatch is running: workspaces come from it */
    void *time_ev[2];        /* events to record around the next contraction's main kernel, or NULL */
    const UOpKernel *sig_k;  /* the program being dispatched, and its signature once computed (0: not yet) */
    u64 sig_h;
    int time_fired;          /* they were recorded */
    u64 noalloc_off;         /* bytes of the static workspace handed out in that dispatch */
    int noalloc_err;         /* why that dispatch could not run (THVM_HIP_E*), or 0 */
    u32 *comb_err_host;      /* host-mapped word a single-pass combine sets when it gave up waiting */
    u32 *comb_err_dev;       /* ... its device address, written into every loaded module */
    u64 n_comb_gaveup;       /* waits after which such a word was found set */
    int comb_gaveup_pending; /* ... since the last thvm_hip_synchronize */
    int force_combine_launch; /* generate split reductions with a combine kernel (the grid does not fit at once) */
    int capturing;           /* a graph capture is open on the stream */
    int capture_bad;         /* the open capture met work a graph cannot replay */
} HipbState;

extern HipbState hipb;

/* ---------------- pool ---------------- */
/* While a graph is captured, host-to-device uploads stage through a pinned
 * arena that the graph owns (a captured copy reads its source at every
 * replay, and the staging ring is reused); anything that would synchronize
 * the host marks the capture unusable instead. */
void pool_sync_all_device(void);
void pool_device_wrote_all(void);
/* the device blocks one graph references (each holds one pin) */
typedef struct { void **ptr; u32 n, cap; } PoolPins;
void pool_capture_begin(u8 *arena, u64 bytes, PoolPins *pins);
void pool_capture_end(void);
int  pool_capture_forbids(const char *what);
void pool_pins_release(PoolPins *pins);
void pool_pin_stats(u32 *pinned, u32 *limbo);
/* hipStreamSynchronize on the backend's stream, counted */
hipError_t hipb_stream_wait(void);
/* Host clock for THVM_HIP_HOST_PROFILE (0 when it is off). */
u64 hipb_hp_now(void);
void hipb_hp_add(int cat, u64 t0);
/* Issues the dispatches held for a batched launch; every operation put on
 * the stream calls it first, so the stream sees work in program order. */
void hipb_before_stream(void);
/* The same for a host-to-device copy into [dst, dst + bytes): only if a held
 * dispatch touches that memory (the copy may go ahead of independent ones). */
void hipb_before_copy(const void *dst, u64 bytes);
/* Holds a copy of `bytes` from device-readable host memory src_dev into the
 * device buffer at dst (dst_bytes long) as a launch of the upload kernel, so
 * that it goes out with independent held launches. Returns 0 when it is not
 * held (the caller copies with hipMemcpyAsync). */
int  hipb_hold_upload(void *dst, u64 dst_bytes, const void *src_dev, u64 bytes);
/* Whether a held launch that a consumer may still fuse after names buffer
 * id (its free then waits: pool_release_deferred after the launch). */
int  hipb_held_buffer(u32 id);
/* launches are held (not yet issued) */
int  hipb_holding(void);
void pool_release_deferred(void);
typedef struct {
    void *ptr;        /* device pointer, NULL if free */
    u64 bytes;        /* requested bytes */
    u64 cap;          /* capacity of the block (size class) */
    u32 refcount;
    u8  live;
    u8  host_valid;   /* host mirror holds the current contents */
    u8  dev_stale;    /* the mirror has not been copied to the device yet */
    u32 mirror_bytes; /* bytes of the mirror that were written */
    void *host_mirror;
    u32 write_capture; /* the graph capture during which the host last wrote it (0: none) */
    u64 wseq;          /* pool_write_clock() just after its last host write */
} HipbBuf;

int   pool_init(void);
void  pool_shutdown(void);
u32   pool_alloc(u64 bytes);
/* device blocks outside the engine's id space */
typedef struct { void *ptr; u64 cap; } Scratch;
void *pool_block_get(u64 bytes, u64 *cap_out);
void  pool_block_put(void *ptr, u64 cap);
void *scratch_reserve(Scratch *sc, u64 bytes);
void  scratch_release(Scratch *sc);
void  pool_upload(void *dst, const void *src, u64 bytes);
void  pool_free(u32 id);
void  pool_incref(u32 id);
void  pool_decref(u32 id);
void  pool_reset(u32 keep);
void  pool_set_persistent(u32 max_buf);
HipbBuf *pool_get(u32 id);
void *pool_ptr(u32 id);
u64   pool_bytes(u32 id);
void  pool_mark_device_write(u32 id);
void  pool_sync_device(u32 id);
int   pool_host_value(u32 id, u32 dtype, u32 idx, float *out);
void  pool_write(u32 id, const void *data, u64 bytes);
/* counts host writes (buf_write) into any buffer */
u64   pool_write_clock(void);
void  pool_read(u32 id, void *out, u64 bytes, int nosync);
void  pool_stats(u64 *live_bytes, u64 *cached_bytes, u64 *n_mallocs);

/* ---------------- code generation ---------------- */
enum { KG_MODE_SERIAL = 0, KG_MODE_GROUP = 1 };
#define KGEN_MAX_SCALARS 16

typedef struct {
    char *src;            /* generated HIP source (malloc'd) */
    char name[32];        /* entry symbol */
    int mode;             /* KG_MODE_* */
    u32 vec;              /* elements per thread-vector (1 or 4) */
    u32 block;            /* threads per workgroup */
    u64 total;            /* serial: gids; group: outputs */
    u64 n_threads;        /* serial: number of vector lanes (ceil(total/vec)) */
    u32 splits;           /* group: workgroups per output (> 1: partials combined in one pass) */
    int combine_launch;   /* ... or, with splits > 1, by a separate <name>_fin kernel */
    u32 n_scal;           /* constant-index leaf loads that take an inline value (sm_, sv*) */
    u32 scal_leaf[KGEN_MAX_SCALARS], scal_index[KGEN_MAX_SCALARS];
    u32 scal_only_leaves; /* bit b: every load of leaf b is such a load */
} KGenResult;

int  kgen_uop(const UOpKernel *k, KGenResult *out, char *err, size_t errlen);
/* As kgen_uop; lanes (7 words per op, if not NULL) receives the vector-lane
 * classification: kind (0 invariant, 1 lane-offset, 2 varying, 3 float),
 * off[4], the divisor of the lane-0 value (0: the value is 0) and the bound. */
int  kgen_uop_lanes(const UOpKernel *k, KGenResult *out, u32 *lanes, char *err, size_t errlen);
void kgen_free(KGenResult *r);
int  kgen_validate(const UOpKernel *k, char *err, size_t errlen);
const char *kgen_prelude(void);
/* rebuilt with the current knobs on the next kgen_prelude() (backend init) */
void kgen_prelude_reset(void);
int  kgen_alu_expr(u32 uop, u32 aux, const char *a, const char *b, char *out, size_t n);
/* An elementwise program's inline scalars: its loads of leaf[j] at index[j]
 * (constant) take argument sv<j> when bit j of sm_ is set. */
typedef struct { u32 n, leaf[KGEN_MAX_SCALARS], index[KGEN_MAX_SCALARS]; } KGenScalars;
int  kgen_epilogue(const UOpKernel *k, u32 o_leaf, char *out, size_t outlen, KGenScalars *sc);
/* the same as a device function named fname that returns the value it stores */
int  kgen_epilogue_fn(const UOpKernel *k, u32 o_leaf, const char *fname, char *out, size_t outlen,
                      KGenScalars *sc);
/* A loop-free program as a device function fname(gid_, st_, r0_.., p0.., c0..)
 * that computes it for gid_, stores its STOREs when st_ is set and returns
 * STORE j's value in *r<j>_. */
int  kgen_producer_fn(const UOpKernel *k, const char *fname, char *out, size_t outlen, KGenScalars *sc);
/* the same for gids X0..X0+3 (X0 a multiple of 4, `total` gids in all) in the
 * serial generator's vector form: fname(X0, st_, r0_.., ...), float4 values */
int  kgen_producer4_fn(const UOpKernel *k, u32 total, const char *fname, char *out, size_t outlen,
                       KGenScalars *sc);
int  kgen_emit_cone(const UOpKernel *k, const u8 *cone, const char *gid_expr, const char *r_expr,
                    char *out, size_t outlen);

/* Single-pass combine area: one partial word per workgroup, zeroed at init;
 * every kernel that uses it leaves it zeroed again. */
#define COMB_SLOTS (1u << 19)
/* A grid combines its partials in one pass only if it fits on the GPU at
 * once (a combining workgroup waits for the others of its output): at most
 * 16 waves per compute unit, hipb.resident_waves in all (4096 on MI355X's
 * 256 CUs; the device's own count once initialised). */
#define SINGLE_PASS_WAVES_PER_CU 16u
u32 hipb_resident_waves(void);

/* ---------------- co-launch ---------------- */
/* A generated module as device functions, so that independent dispatches can
 * go out together in one launch of a batch kernel: the module after the
 * shared prelude, inside namespace co_<id>, each kernel a __device__ function
 * taking its block coordinates, grid size and lane within its own workgroup
 * (bx_, by_, gx_, gy_, tx_) first. */
#define CO_MAX_PARAMS 48
typedef struct {
    char *src;             /* NULL: the kernel is launched on its own */
    char *params;          /* the main kernel's parameter list */
    char name[48];         /* the main kernel's name */
    u32 id;                /* namespace co_<id>, unique in the process */
    u32 threads;           /* its workgroup size */
    u32 lds;               /* its static LDS bytes */
    u32 cap_waves;         /* its waves the GPU holds at once (0: not known) */
    u32 np;
    u8 psz[CO_MAX_PARAMS]; /* its parameters' sizes in bytes */
    u8 no_sync;            /* no workgroup barrier or LDS of its own */
} CoForm;
int  co_form_make(CoForm *cf, const char *src, const char *name, u32 threads, hipFunction_t fn);
void co_form_free(CoForm *cf);

/* Memory a held dispatch touches, as address ranges (write: written, maybe
 * also read). */
#define HB_RANGES (FUSE_MAX_LEAVES + 4)
typedef struct {
    u32 n;
    u64 lo[HB_RANGES], hi[HB_RANGES];
    u8 wr[HB_RANGES];
} HbMem;
void hbm_add(HbMem *m, const void *p, u64 bytes, int write);
/* Holds a launch of cf's kernel (returns 1) for a batch with the next
 * independent dispatches, or returns 0: the caller launches it now.
 * `resident`: the kernel's workgroups wait for each other (the batch must fit
 * on the GPU at once). A kernel that combines partials through the combine
 * area names the parameter that points there (comb_param, else -1) and the
 * words it uses from there (comb_words): each kernel of a batch gets its own
 * slice of the area. */
int  hipb_hold(const CoForm *cf, hipFunction_t fn, u32 gx, u32 gy, void *const *params, const HbMem *m,
               int resident, int comb_param, u64 comb_words);
/* hipb_hold for a launch of any grid size that a later dispatch may join
 * (a run sum, a window max: run-sum groups); only while fusion is on. */
int  hipb_hold_large(const CoForm *cf, hipFunction_t fn, u32 gx, u32 gy, void *const *params, const HbMem *m,
                     int resident, int comb_param, u64 comb_words);
/* Holds a launch (of any grid size) only so that the next dispatch can fuse
 * into it (hipb_hold_tag); it joins no batch. Returns 1 if held. */
int  hipb_hold_solo(const CoForm *cf, hipFunction_t fn, u32 gx, u32 gy, void *const *params, const HbMem *m);
/* Marks the launch just held as a contraction (dense entry key, serial)
 * writing buffer out_buf that an elementwise consumer may fuse into. */
void hipb_hold_tag(u64 key, u32 serial, u32 out_buf);
/* dense.c: the contraction (key, serial) with the elementwise program c,
 * which reads its output as leaf buffer o_leaf, fused into its epilogue */
int  dense_epilogue(u64 key, u32 serial, const UOpKernel *c, u32 o_leaf, hipFunction_t *fn, CoForm *co,
                    KGenScalars *sc);
char *dense_epilogue_source(const UOpKernel *k, const UOpKernel *c, u32 o_leaf, char *err, size_t errlen);

/* ---------------- chain.c: elementwise programs fused in sequence ---------------- */
#define CHAIN_MAX_OPS 256     /* the generator vectorises programs up to this size */
#define CHAIN_MAX_STORES 8
typedef struct {
    const KOp *ops;           /* the compiled program's copy (owned by the kernel cache) */
    u32 n_ops, n_leaves, total, out_dtype;
    u32 grid[3];
    u32 leaf_dtypes[FUSE_MAX_LEAVES];
    u32 n_st, st_slot[CHAIN_MAX_STORES], st_val[CHAIN_MAX_STORES];  /* its STOREs: buffer slot, value op */
    u8 st_f32[CHAIN_MAX_STORES];
    u64 gid_loads;            /* bit s: every load of leaf slot s is at gid (a lane reads only its own element) */
} ChainInfo;
/* A program with no loop or one top-level loop, whose STOREs all follow
 * the loop and write at gid (so a consumer that reads one of its outputs at
 * gid can take the stored value), or NULL. */
ChainInfo *chain_info_make(const UOpKernel *k, const KOp *ops);
/* The program M = P then C, C's loads of P's outputs taking P's stored
 * values and C's STORE going to a new leaf slot; pb/mb are the buffer ids
 * (output, leaves) of P and of M. Returns 0 when the pair does not fuse. */
int chain_merge(const ChainInfo *p, const u32 *pb, const UOpKernel *c, u32 c_out, const u32 *c_leaves,
                u32 c_nl, UOpKernel *m, u32 *mb);
/* bit s set: the program STOREs into leaf slot s (s >= 1) */
u64 chain_store_slots(const UOpKernel *k);

/* ---------------- rtc / cache ---------------- */
typedef struct {
    u64 key;
    hipModule_t mod;
    hipFunction_t fn;
    hipFunction_t fn_fin;  /* split group reduce: combine kernel */
    u32 splits;
    u32 n_scal, scal_leaf[KGEN_MAX_SCALARS], scal_index[KGEN_MAX_SCALARS], scal_only_leaves;
    int mode;
    u32 vec, block;
    u64 total, n_threads;
    u32 n_ops, n_leaves;
    KOp *ops;             /* copy for collision checks */
    u32 meta[5 + FUSE_MAX_LEAVES]; /* grid, local_size, out_dtype, leaf dtypes */
    char name[32];        /* the kernel's symbol */
    CoForm co;            /* its co-launch form */
    ChainInfo *chain;     /* set when a consumer may fuse after it */
    u64 store_slots;      /* leaf slots it writes (chain_store_slots) */
} KCacheEntry;

int  rtc_init(void);
void rtc_shutdown(void);
KCacheEntry *rtc_lookup(u64 key, const UOpKernel *k);
KCacheEntry *rtc_compile_uop(u64 key, const UOpKernel *k);
hipFunction_t rtc_static_fn(const char *name);
/* Compile HIP source and load it; returns the module (0 on failure). */
int  rtc_build_module(const char *src, hipModule_t *mod, char *err, size_t errlen);
/* Workgroups of `block` lanes of fn that the GPU holds at once (its
 * occupancy per compute unit times the compute units), or 0. */
u32  rtc_capacity(hipFunction_t fn, u32 block);
/* Compile only (no device needed); returns the code size or -1. */
long rtc_compile_only(const char *src, char *err, size_t errlen);
u64  uop_signature(const UOpKernel *k);

/* ---------------- dense paths ---------------- */
int  dense_try_dispatch(u32 out_buf, const u32 *leaf_bufs, u32 n_leaves, const UOpKernel *k);
int  dense_analyze(const UOpKernel *k, u32 *M, u32 *N, u32 *K, u32 *splits);
char *dense_source(const UOpKernel *k);
void dense_reset_stats(void);
/* a program that is not a contraction gets its (negative) entry without a dispatch */
void dense_note_plain(const UOpKernel *k);
void dense_shutdown(void);

/* ---------------- pooling windows and run sums ---------------- */
int  window_try_dispatch(u32 out_buf, const u32 *leaf_bufs, u32 n_leaves, const UOpKernel *k);
/* kind: 0 none, 1 window max, 2 run sum; splits: workgroups per output */
int  window_analyze(const UOpKernel *k, u32 *kind, u32 *splits);
char *window_source(const UOpKernel *k);
void window_shutdown(void);
/* a program that is neither gets its (negative) entry without a dispatch */
void window_note_plain(const UOpKernel *k);

/* Run-sum groups (window.c): one launch that computes several run sums of
 * the same shape (outputs, loop, runs, splits) over what they read, with
 * optionally
 *   - the producer of a tensor they read taken in: an elementwise program
 *     or a window max, computed where the sums load the tensor and stored
 *     there by the same lane (the sums read every element of it once), and
 *   - elementwise consumers of the sums' outputs ("tails"), applied by the
 *     workgroup that combines each output to the value it stores.
 * Every value is computed by the same operations in the same order as in
 * the separate launches, so the results are theirs bit for bit. */
#define WG_MAX_SUMS 4
#define WG_MAX_TAILS 4
#define WG_MAX_LEAVES 16
typedef struct { u32 id, cnt; void *ptr; u64 bytes; } WgBuf;
typedef struct { u32 nb; WgBuf b[1 + WG_MAX_LEAVES]; } WgBufs;   /* output, then the leaves */
typedef struct {
    u32 n_sum, n_tail;
    const void *sum[WG_MAX_SUMS];        /* the run sums (window.c cache entries) */
    WgBufs sb[WG_MAX_SUMS];
    int8_t sub[WG_MAX_SUMS][1 + WG_MAX_LEAVES]; /* per leaf slot: the producer STORE it reads (-1: memory) */
    int pkind;                           /* producer: 0 none, 1 elementwise program, 2 window max */
    const ChainInfo *pc;                 /* pkind 1 */
    const void *pw;                      /* pkind 2: the window max (window.c cache entry) */
    u64 psig;                            /* the producer's program signature */
    WgBufs pb;
    int has_canon;                       /* the index the sums read the producer's tensor at */
    Aff canon;
    const UOpKernel *tail[WG_MAX_TAILS]; /* window.c's copies of the consumers' programs */
    u64 tsig[WG_MAX_TAILS];
    WgBufs tb[WG_MAX_TAILS];
    u32 tleaf[WG_MAX_TAILS];             /* the leaf slot (1 + leaf) that takes the value */
    u8 tsrc[WG_MAX_TAILS];               /* that value: sum s (s < WG_MAX_SUMS) or tail WG_MAX_SUMS + t */
    /* set by window_group_build */
    hipFunction_t fn;
    const CoForm *co;
    const KGenScalars *psc, *tsc;        /* the producer's and the tails' inline scalars */
    u32 grid, comb_words;
    int resident;
} WinGroup;
/* a held run sum (window_try_dispatch) as a group of one */
int  window_group_of_sum(WinGroup *g, const void *we, u32 out_buf, const u32 *leaf_bufs, u32 n_leaves);
/* an empty group around a held producer (its buffers: output, leaves) */
int  window_group_of_chain(WinGroup *g, const ChainInfo *pc, const u32 *bufs);
int  window_group_of_wmax(WinGroup *g, const void *we, u32 out_buf, u32 in_buf);
/* the run-sum program's single-launch entry (compiled), or NULL */
const void *window_sum_entry(const UOpKernel *k);
/* g extended by run sum k / elementwise consumer k; 0: it does not join */
int  window_group_add_sum(WinGroup *g, const void *we, u32 out_buf, const u32 *leaf_bufs, u32 n_leaves);
int  window_group_add_tail(WinGroup *g, const UOpKernel *k, u32 out_buf, const u32 *leaf_bufs, u32 n_leaves);
/* whether the group reads or writes buffer id (writes only: `writes`) */
int  window_group_uses(const WinGroup *g, u32 id, int writes);
/* the group's kernel (compiled once per shape): fn, co, grid, comb_words */
int  window_group_build(WinGroup *g);
/* its launch parameters (into the caller's storage), their count */
typedef struct { void *ptr[160]; u32 cnt[160]; u32 sm[1 + WG_MAX_TAILS]; float sv[(1 + WG_MAX_TAILS) * KGEN_MAX_SCALARS]; } WgArgs;
u32  window_group_params(const WinGroup *g, WgArgs *a, void **params);
void window_group_mem(const WinGroup *g, HbMem *m);
/* the leaves of tail t (bit i: leaf i) that are read from memory (must be current on the device) */
u64  window_group_tail_reads(const WinGroup *g, u32 t);
/* device-free: the group kernel of programs ks[0..n) over buffer ids (bufs[i]: output, leaves),
 * the first a producer when `producer` is set; NULL with the reason in err */
char *window_group_source(const UOpKernel *const *ks, const u32 *const *bufs, u32 n, int producer, char *err,
                          size_t errlen);
/* backend.c: the launch just held is a run sum (a group of one) or a window max a run sum may take in */
void hipb_hold_tag_sum(const void *we, u32 out_buf, const u32 *leaf_bufs, u32 n_leaves);
void hipb_hold_tag_wmax(const void *we, u32 out_buf, u32 in_buf);

/* ---------------- launch helpers ---------------- */
int  hipb_launch(hipFunction_t fn, u32 gx, u32 gy, u32 gz, u32 bx, void **params);
/* gx*gy workgroups of bx lanes; gx may exceed the 32-bit work-item limit */
int  hipb_launch_grid(hipFunction_t fn, u32 gx, u32 gy, u32 bx, void **params);

#endif /* HIPB_H */
