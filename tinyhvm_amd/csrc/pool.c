/*
 * pool.c - device buffer pool behind the Backend buffer slots.
 *
 * Contract (src/tinyhvm.h:992-1000, CPU pool src/backend/cpu/pool.c:6-26,
 * Metal pool src/backend/metal/pool.m:46-223):
 *   - ids are nonzero u32, handed out in increasing order; 0 means failure;
 *   - buf_free may be called repeatedly for the same id (views alias ids);
 *   - pool_reset(keep) releases ids >= keep+1 and restarts numbering there;
 *   - decref on an id at or below the persistent floor is ignored.
 *
 * Device memory: every block comes from hipMalloc in a size class (256 B,
 * then quarter-power-of-two steps) and returns to its class free list when
 * its id dies. All device work is ordered on one stream, so a block freed
 * by the host may be handed to a later dispatch without waiting: the stream
 * orders the old readers before the new writer.
 *
 * HIP graphs: a captured graph keeps the raw device addresses of every block
 * its work touched, and writes them again at each launch. Such a block is
 * pinned: every block resolved while a capture is open (buffers named by the
 * captured calls, kernel workspaces, parameter blocks) is entered in a pin
 * table with one count per graph holding it. A pinned block that is released
 * (its id freed or reset, a workspace outgrown) waits in limbo instead of the
 * free list, so no later allocation can receive memory a graph still writes;
 * when its last graph is destroyed it returns to the free list.
 *
 * Ids stop below 16384: the engine tracks buffer epochs for its kernel result
 * cache only for ids under MAX_BUF_EPOCHS (src/tinyhvm.h:720), and its CPU
 * and Metal pools hold MAX_BUFS = 16384 ids (src/backend/cpu/pool.c:4,
 * src/backend/metal/pool.m:50). Past that, buf_alloc fails (returns 0) until
 * a pool_reset recycles ids.
 *
 * Host copies: writes of at most 4 KiB are kept in a host mirror and reach
 * the device only when something on the device first needs the buffer (a
 * dispatch reading or writing it, a copy, a synchronous read): the engine
 * writes many small metadata buffers (shape and axis tensors, scalars) that
 * no kernel reads. Larger writes up to one staging segment go through a
 * pinned ring (memcpy, then an async copy on the stream), so buf_write
 * returns as soon as the caller's memory has been consumed and never blocks
 * unless the ring wraps onto a segment still in flight.
 */
#include <stdlib.h>
#include <string.h>

#include "hipb.h"
#include "thvm_hip.h"

#define POOL_MIN_CLASS_BYTES 256ull
#define POOL_N_CLASSES 256
#define POOL_MIRROR_MAX 16384ull
#define STAGE_SEGMENTS 4
#define STAGE_SEG_BYTES (16ull << 20)
/* Host writes of more than UP_EAGER_MIN and at most POOL_MIRROR_MAX bytes
 * are copied by a kernel that reads them from pinned, coherent host memory
 * (an upload ring of UP_SEGMENTS segments), so that the copy can go out in
 * one launch with independent held work. */
#define UP_SEGMENTS 2
#define UP_SEG_BYTES (2ull << 20)
#define UP_MAX (64ull << 10)
#define UP_EAGER_MIN 256ull
#define POOL_MAX_IDS 16384u

typedef struct {
    void **ptrs;
    u32 n, cap;
} FreeList;

/* pin table entry: a block some graph references, and how many graphs do */
typedef struct {
    void *ptr;
    u64 cap;
    u32 pins;
    u32 seq;       /* the capture that pinned it last (one count per capture) */
} PinEnt;

static struct {
    HipbBuf *bufs;
    u64 wclock;           /* host writes so far */
    u32 cap;
    u32 count;            /* next id */
    u32 persistent_floor;
    FreeList free[POOL_N_CLASSES];
    u64 live_bytes, cached_bytes, n_mallocs;
    /* pinned staging ring */
    u8 *stage;
    hipEvent_t seg_done[STAGE_SEGMENTS];
    u8 seg_pending[STAGE_SEGMENTS];
    u32 seg;
    u64 seg_off;
    /* upload ring (host pointer, device pointer) */
    u8 *up, *up_dev;
    hipEvent_t up_done[UP_SEGMENTS];
    u8 up_pending[UP_SEGMENTS];
    u32 up_seg;
    i32 up_closing;       /* segment whose event waits for the held launches to go out, or -1 */
    u64 up_off;
    /* graph capture: uploads go to the capturing graph's arena */
    u8 *arena, *arena_dev;
    u64 arena_cap, arena_off;
    u32 capture_seq;      /* numbers the captures; buffers record the one they were written in */
    PoolPins *capture_pins; /* blocks the open capture references */
    /* pinned blocks (open addressing on the address) and released pinned blocks */
    PinEnt *pin;
    u32 pin_cap, pin_n;
    void **limbo;
    u64 *limbo_cap;
    u32 limbo_n, limbo_max;
} P;

static u32 pin_slot(const void *p) {
    return (u32)((((uintptr_t)p >> 8) * 0x9E3779B97F4A7C15ull) >> 32) & (P.pin_cap - 1);
}

static PinEnt *pin_find(const void *p) {
    if (!P.pin_cap || !p) return NULL;
    for (u32 i = pin_slot(p);; i = (i + 1) & (P.pin_cap - 1)) {
        if (!P.pin[i].ptr) return NULL;
        if (P.pin[i].ptr == p) return &P.pin[i];
    }
}

static int pin_grow(void) {
    u32 nc = P.pin_cap ? P.pin_cap * 2 : 256;
    PinEnt *old = P.pin, *nt = calloc(nc, sizeof(PinEnt));
    u32 oc = P.pin_cap;
    if (!nt) return 0;
    P.pin = nt;
    P.pin_cap = nc;
    for (u32 i = 0; i < oc; i++) {
        if (!old[i].ptr) continue;
        u32 j = pin_slot(old[i].ptr);
        while (P.pin[j].ptr) j = (j + 1) & (nc - 1);
        P.pin[j] = old[i];
    }
    free(old);
    return 1;
}

/* Removes slot i, shifting later entries of its probe run back into place. */
static void pin_erase(u32 i) {
    u32 mask = P.pin_cap - 1, j = i;
    for (;;) {
        j = (j + 1) & mask;
        if (!P.pin[j].ptr) break;
        u32 k = pin_slot(P.pin[j].ptr);
        /* entry j may move to i unless its home slot k lies cyclically in (i, j] */
        int stays = (i <= j) ? (k > i && k <= j) : (k > i || k <= j);
        if (!stays) {
            P.pin[i] = P.pin[j];
            i = j;
        }
    }
    memset(&P.pin[i], 0, sizeof(PinEnt));
    P.pin_n--;
}

/* Records that the open capture references a block (once per capture). */
static void capture_pin(void *ptr, u64 cap) {
    if (!hipb.capturing || !ptr || !P.capture_pins) return;
    PinEnt *e = pin_find(ptr);
    if (e && e->seq == P.capture_seq) return;
    PoolPins *pp = P.capture_pins;
    if (pp->n == pp->cap) {
        u32 nc = pp->cap ? pp->cap * 2 : 64;
        void **np = realloc(pp->ptr, nc * sizeof(void *));
        if (!np) {
            pool_capture_forbids("pin bookkeeping out of host memory");
            return;
        }
        pp->ptr = np;
        pp->cap = nc;
    }
    if (!e) {
        if ((P.pin_n + 1) * 2 > P.pin_cap && !pin_grow()) {
            pool_capture_forbids("pin bookkeeping out of host memory");
            return;
        }
        u32 j = pin_slot(ptr);
        while (P.pin[j].ptr) j = (j + 1) & (P.pin_cap - 1);
        e = &P.pin[j];
        e->ptr = ptr;
        e->cap = cap;
        e->pins = 0;
        P.pin_n++;
    }
    e->pins++;
    e->seq = P.capture_seq;
    pp->ptr[pp->n++] = ptr;
}

void pool_capture_begin(u8 *arena, u64 bytes, PoolPins *pins) {
    P.capture_seq++;
    P.arena = arena;
    P.arena_dev = NULL;
    if (arena && hipHostGetDevicePointer((void **)&P.arena_dev, arena, 0) != hipSuccess) {
        (void)hipGetLastError();
        P.arena_dev = NULL;
    }
    P.arena_cap = bytes;
    P.arena_off = 0;
    P.capture_pins = pins;
    /* the fill block of absent buffers and the combine area are in every
     * graph's kernels */
    capture_pin(hipb.dummy, hipb.dummy_cap);
    capture_pin(hipb.comb_slots, (u64)COMB_SLOTS * 8);
}

void pool_capture_end(void) {
    /* the captured uploads did not run: mirrors written during the capture
     * are still to be copied for eager use */
    for (u32 i = 1; i < P.count; i++) {
        HipbBuf *b = &P.bufs[i];
        if (b->live && b->host_valid && b->host_mirror && b->write_capture == P.capture_seq) b->dev_stale = 1;
    }
    P.arena = P.arena_dev = NULL;
    P.arena_cap = P.arena_off = 0;
    P.capture_pins = NULL;
}

int pool_capture_forbids(const char *what) {
    if (!hipb.capturing) return 0;
    if (!hipb.capture_bad && hipb.verbose) fprintf(stderr, "tinyhvm-hip: graph capture abandoned: %s\n", what);
    hipb.capture_bad = 1;
    return 1;
}

/* Size class of a byte count: 256 B minimum, then 4 classes per octave. */
static u32 size_class(u64 bytes, u64 *cap_out) {
    if (bytes <= POOL_MIN_CLASS_BYTES) {
        *cap_out = POOL_MIN_CLASS_BYTES;
        return 0;
    }
    u32 lg = 63 - (u32)__builtin_clzll(bytes - 1);   /* 2^lg < bytes <= 2^(lg+1) */
    u64 base = 1ull << lg;
    u64 quarter = base >> 2;
    u32 sub = (u32)((bytes - base + quarter - 1) / quarter); /* 1..4 */
    *cap_out = base + (u64)sub * quarter;
    u32 c = (lg - 8) * 4 + sub;
    return c < POOL_N_CLASSES ? c : POOL_N_CLASSES - 1;
}

static int fl_push(FreeList *f, void *p) {
    if (f->n == f->cap) {
        u32 nc = f->cap ? f->cap * 2 : 16;
        void **np = realloc(f->ptrs, nc * sizeof(void *));
        if (!np) return 0;
        f->ptrs = np;
        f->cap = nc;
    }
    f->ptrs[f->n++] = p;
    return 1;
}

/* A piece of the static workspace for the running no-allocation dispatch
 * (256-byte aligned), or NULL with the error recorded when it is full. */
static void *noalloc_carve(u64 bytes) {
    u64 off = (hipb.noalloc_off + 255) & ~255ull;
    if (!hipb.noalloc_scratch) {
        hipb.noalloc_err = THVM_HIP_ENOSCRATCH;
        return NULL;
    }
    if (bytes > THVM_HIP_NOALLOC_SCRATCH_BYTES || off + bytes > THVM_HIP_NOALLOC_SCRATCH_BYTES) {
        fprintf(stderr, "tinyhvm-hip: dispatch without allocation needs %llu bytes of workspace; "
                "the static workspace holds %llu\n", (unsigned long long)(off + bytes),
                (unsigned long long)THVM_HIP_NOALLOC_SCRATCH_BYTES);
        hipb.noalloc_err = THVM_HIP_ESCRATCH;
        return NULL;
    }
    hipb.noalloc_off = off + bytes;
    return (u8 *)hipb.noalloc_scratch + off;
}

static int in_static_scratch(const void *p) {
    const u8 *s = hipb.noalloc_scratch;
    return s && (const u8 *)p >= s && (const u8 *)p < s + THVM_HIP_NOALLOC_SCRATCH_BYTES;
}

/* A released block: to limbo while a graph references it, else to its
 * class's free list (or back to HIP if the list cannot grow). */
static void block_release(void *ptr, u64 cap) {
    if (!ptr || in_static_scratch(ptr)) return;
    if (pin_find(ptr)) {
        if (P.limbo_n == P.limbo_max) {
            u32 nc = P.limbo_max ? P.limbo_max * 2 : 64;
            void **np = realloc(P.limbo, nc * sizeof(void *));
            u64 *nq = realloc(P.limbo_cap, nc * sizeof(u64));
            if (np) P.limbo = np;
            if (nq) P.limbo_cap = nq;
            if (!np || !nq) {
                /* cannot track it: leak the block rather than reuse it */
                fprintf(stderr, "tinyhvm-hip: out of host memory; a graph-held block is leaked\n");
                return;
            }
            P.limbo_max = nc;
        }
        P.limbo[P.limbo_n] = ptr;
        P.limbo_cap[P.limbo_n] = cap;
        P.limbo_n++;
        return;
    }
    u64 c2 = 0;
    u32 c = size_class(cap, &c2);
    if (fl_push(&P.free[c], ptr)) P.cached_bytes += c2;
    else if (!pool_capture_forbids("a block free")) {
        HIPB_CHECK(hipb_stream_wait());
        HIPB_CHECK(hipFree(ptr));
    }
}

/* A graph is gone: its blocks lose one pin each; released blocks no graph
 * holds any more leave limbo for the free lists. */
void pool_pins_release(PoolPins *pp) {
    if (!pp) return;
    for (u32 i = 0; i < pp->n; i++) {
        PinEnt *e = pin_find(pp->ptr[i]);
        if (!e) continue;
        if (e->pins > 1) {
            e->pins--;
            continue;
        }
        void *ptr = e->ptr;
        pin_erase((u32)(e - P.pin));
        for (u32 j = 0; j < P.limbo_n; j++) {
            if (P.limbo[j] != ptr) continue;
            u64 cap = P.limbo_cap[j];
            P.limbo_n--;
            P.limbo[j] = P.limbo[P.limbo_n];
            P.limbo_cap[j] = P.limbo_cap[P.limbo_n];
            block_release(ptr, cap);
            break;
        }
    }
    free(pp->ptr);
    memset(pp, 0, sizeof *pp);
}

void pool_pin_stats(u32 *pinned, u32 *limbo) {
    if (pinned) *pinned = P.pin_n;
    if (limbo) *limbo = P.limbo_n;
}

static void release_cache(void) {
    if (pool_capture_forbids("device memory exhausted")) return;
    HIPB_CHECK(hipb_stream_wait());
    for (u32 c = 0; c < POOL_N_CLASSES; c++) {
        for (u32 i = 0; i < P.free[c].n; i++) HIPB_CHECK(hipFree(P.free[c].ptrs[i]));
        P.free[c].n = 0;
    }
    P.cached_bytes = 0;
}

int pool_init(void) {
    memset(&P, 0, sizeof(P));
    P.cap = 1024;
    P.bufs = calloc(P.cap, sizeof(HipbBuf));
    if (!P.bufs) return -1;
    P.count = 1;
    if (hipHostMalloc((void **)&P.stage, STAGE_SEGMENTS * STAGE_SEG_BYTES, 0) != hipSuccess) {
        fprintf(stderr, "tinyhvm-hip: pinned staging allocation failed\n");
        P.stage = NULL;
        return -1;
    }
    for (u32 s = 0; s < STAGE_SEGMENTS; s++) {
        if (hipEventCreateWithFlags(&P.seg_done[s], hipEventDisableTiming) != hipSuccess) return -1;
    }
    /* the upload ring: optional (uploads fall back to copies without it) */
    P.up_closing = -1;
    if (hipHostMalloc((void **)&P.up, UP_SEGMENTS * UP_SEG_BYTES, hipHostMallocMapped | hipHostMallocCoherent) !=
            hipSuccess ||
        hipHostGetDevicePointer((void **)&P.up_dev, P.up, 0) != hipSuccess) {
        (void)hipGetLastError();
        if (P.up) HIPB_CHECK(hipHostFree(P.up));
        P.up = P.up_dev = NULL;
    }
    for (u32 s = 0; s < UP_SEGMENTS && P.up; s++)
        if (hipEventCreateWithFlags(&P.up_done[s], hipEventDisableTiming) != hipSuccess) return -1;
    return 0;
}

void pool_shutdown(void) {
    if (!P.bufs) return;
    HIPB_CHECK(hipb_stream_wait());
    for (u32 i = 1; i < P.count; i++) {
        if (P.bufs[i].live && P.bufs[i].ptr) HIPB_CHECK(hipFree(P.bufs[i].ptr));
        free(P.bufs[i].host_mirror);
    }
    release_cache();
    for (u32 j = 0; j < P.limbo_n; j++) HIPB_CHECK(hipFree(P.limbo[j]));
    free(P.limbo);
    free(P.limbo_cap);
    free(P.pin);
    for (u32 c = 0; c < POOL_N_CLASSES; c++) free(P.free[c].ptrs);
    for (u32 s = 0; s < STAGE_SEGMENTS; s++) HIPB_CHECK(hipEventDestroy(P.seg_done[s]));
    if (P.stage) HIPB_CHECK(hipHostFree(P.stage));
    if (P.up) {
        for (u32 s = 0; s < UP_SEGMENTS; s++) HIPB_CHECK(hipEventDestroy(P.up_done[s]));
        HIPB_CHECK(hipHostFree(P.up));
    }
    free(P.bufs);
    memset(&P, 0, sizeof(P));
}

static int ensure_cap(u32 id) {
    if (id < P.cap) return 1;
    u32 nc = P.cap;
    while (nc <= id) nc *= 2;
    HipbBuf *nb = realloc(P.bufs, (size_t)nc * sizeof(HipbBuf));
    if (!nb) return 0;
    memset(nb + P.cap, 0, (size_t)(nc - P.cap) * sizeof(HipbBuf));
    P.bufs = nb;
    P.cap = nc;
    return 1;
}

/* A device block of at least `bytes` from its size class's free list, or
 * hipMalloc (after releasing the cached blocks on failure). */
void *pool_block_get(u64 bytes, u64 *cap_out) {
    if (hipb.noalloc) {
        *cap_out = bytes;
        return noalloc_carve(bytes);
    }
    u64 cap = 0;
    u32 c = size_class(bytes ? bytes : 4, &cap);
    void *ptr = NULL;
    if (P.free[c].n > 0) {
        ptr = P.free[c].ptrs[--P.free[c].n];
        P.cached_bytes -= cap;
    } else {
        if (hipMalloc(&ptr, cap) != hipSuccess) {
            (void)hipGetLastError();
            release_cache();
            if (hipMalloc(&ptr, cap) != hipSuccess) {
                (void)hipGetLastError();
                fprintf(stderr, "tinyhvm-hip: out of device memory (%llu bytes)\n",
                        (unsigned long long)cap);
                return NULL;
            }
        }
        P.n_mallocs++;
    }
    *cap_out = cap;
    capture_pin(ptr, cap);
    return ptr;
}

/* Returns a block to its free list (to limbo while a graph holds it). The
 * stream orders its last users before any later owner's work. */
void pool_block_put(void *ptr, u64 cap) { block_release(ptr, cap); }

/* Device scratch outside the engine's buffer ids (kernel workspaces): grown
 * on demand, kept until released. Engine ids are never used for it, so
 * pool_reset cannot free it and the engine's id numbering is untouched. */
void *scratch_reserve(Scratch *sc, u64 bytes) {
    if (hipb.noalloc) return noalloc_carve(bytes);   /* the workspace it keeps stays as it is */
    if (bytes <= sc->cap && sc->ptr) {
        capture_pin(sc->ptr, sc->cap);
        return sc->ptr;
    }
    pool_block_put(sc->ptr, sc->cap);
    sc->ptr = pool_block_get(bytes, &sc->cap);
    if (!sc->ptr) sc->cap = 0;
    return sc->ptr;
}

void scratch_release(Scratch *sc) {
    pool_block_put(sc->ptr, sc->cap);
    sc->ptr = NULL;
    sc->cap = 0;
}

u32 pool_alloc(u64 bytes) {
    if (!hipb.initialized) return 0;
    if (P.count >= POOL_MAX_IDS) {
        fprintf(stderr, "tinyhvm-hip: buffer ids exhausted (%u ids; pool_reset recycles them)\n",
                POOL_MAX_IDS - 1);
        return 0;
    }
    u64 cap = 0;
    void *ptr = pool_block_get(bytes, &cap);
    if (!ptr) return 0;
    u32 id = P.count;
    if (!ensure_cap(id)) {
        pool_block_put(ptr, cap);
        return 0;
    }
    P.count++;
    HipbBuf *b = &P.bufs[id];
    free(b->host_mirror);
    memset(b, 0, sizeof(*b));
    b->ptr = ptr;
    b->bytes = bytes;
    b->cap = cap;
    b->refcount = 1;
    b->live = 1;
    b->dev_stale = 0;
    b->mirror_bytes = 0;
    P.live_bytes += cap;
    return id;
}

static void release_block(HipbBuf *b) {
    block_release(b->ptr, b->cap);
    P.live_bytes -= b->cap;
    b->ptr = NULL;
    b->live = 0;
    b->refcount = 0;
    b->host_valid = 0;
    b->dev_stale = 0;
    free(b->host_mirror);
    b->host_mirror = NULL;
}

/* Frees of buffers that a held launch may still be merged with (its
 * buffers are looked up again by id when a consumer fuses after it) wait
 * until the held launches have been issued. */
#define POOL_DEFER_MAX 64
static struct { u32 id[POOL_DEFER_MAX]; u32 n; } DF;

static int defer_free(u32 id) {
    for (u32 i = 0; i < DF.n; i++)
        if (DF.id[i] == id) return 1;
    if (DF.n >= POOL_DEFER_MAX || !hipb_held_buffer(id)) return 0;
    DF.id[DF.n++] = id;
    return 1;
}

void pool_release_deferred(void) {
    if (P.up_closing >= 0) {   /* the held launches are out: the segment left before is done after them */
        HIPB_CHECK(hipEventRecord(P.up_done[P.up_closing], hipb.stream));
        P.up_pending[P.up_closing] = 1;
        P.up_closing = -1;
    }
    const u32 n = DF.n;
    DF.n = 0;
    for (u32 i = 0; i < n; i++) {
        const u32 id = DF.id[i];
        if (id < P.count && P.bufs[id].live) release_block(&P.bufs[id]);
    }
}

void pool_free(u32 id) {
    if (id == 0 || id >= P.count || !P.bufs[id].live) return;
    if (defer_free(id)) return;
    release_block(&P.bufs[id]);
}

void pool_incref(u32 id) {
    if (id == 0 || id >= P.count || !P.bufs[id].live) return;
    P.bufs[id].refcount++;
}

void pool_decref(u32 id) {
    if (id == 0 || id >= P.count || !P.bufs[id].live) return;
    if (id <= P.persistent_floor) return;
    if (P.bufs[id].refcount > 0) P.bufs[id].refcount--;
    if (P.bufs[id].refcount == 0 && !defer_free(id)) release_block(&P.bufs[id]);
}

void pool_reset(u32 keep) {
    hipb_before_stream();   /* held launches out, deferred frees done: ids are reused from here */
    pool_release_deferred();
    u32 first = keep + 1;
    if (first < 1) first = 1;
    for (u32 i = first; i < P.count; i++)
        if (P.bufs[i].live) release_block(&P.bufs[i]);
    if (first < P.count) P.count = first;
}

void pool_set_persistent(u32 max_buf) { P.persistent_floor = max_buf; }

HipbBuf *pool_get(u32 id) {
    if (id == 0 || id >= P.count || !P.bufs[id].live) return NULL;
    HipbBuf *b = &P.bufs[id];
    capture_pin(b->ptr, b->cap);
    return b;
}

u64 pool_write_clock(void) { return P.wclock; }

void *pool_ptr(u32 id) {
    HipbBuf *b = pool_get(id);
    return b ? b->ptr : NULL;
}

u64 pool_bytes(u32 id) {
    HipbBuf *b = pool_get(id);
    return b ? b->bytes : 0;
}

/* Element idx of a buffer from its host mirror, as the device loads read it
 * (f16 widened exactly, integers converted to float; past the end reads 0).
 * Returns 0 when the host does not hold the buffer's current contents. */
int pool_host_value(u32 id, u32 dtype, u32 idx, float *out) {
    HipbBuf *b = pool_get(id);
    if (!b || !b->host_valid || !b->host_mirror) return 0;
    /* a graph keeps an inline value for good: only for contents the captured
     * calls wrote themselves, which every launch repeats */
    if (hipb.capturing && b->write_capture != P.capture_seq) return 0;
    u64 es = dtype == DTYPE_F16 ? 2 : 4;
    if ((u64)idx * es + es > b->bytes) { *out = 0.0f; return 1; }
    if ((u64)idx * es + es > b->mirror_bytes) return 0;
    const u8 *p = (const u8 *)b->host_mirror + (u64)idx * es;
    switch (dtype) {
    case DTYPE_F16: {
        u16 h;
        memcpy(&h, p, 2);
        u32 sign = ((u32)h & 0x8000u) << 16, ex = ((u32)h >> 10) & 0x1Fu, man = (u32)h & 0x3FFu, bits;
        if (ex == 0) {
            if (man == 0) bits = sign;
            else {
                ex = 1;
                while (!(man & 0x400u)) { man <<= 1; ex -= 1; }
                bits = sign | ((ex + 112u) << 23) | ((man & 0x3FFu) << 13);
            }
        } else if (ex == 0x1Fu) bits = sign | 0x7F800000u | (man << 13);
        else bits = sign | ((ex + 112u) << 23) | (man << 13);
        memcpy(out, &bits, 4);
        return 1;
    }
    case DTYPE_I32: { i32 v; memcpy(&v, p, 4); *out = (float)v; return 1; }
    case DTYPE_U32: { u32 v; memcpy(&v, p, 4); *out = (float)v; return 1; }
    default: memcpy(out, p, 4); return 1;
    }
}

void pool_mark_device_write(u32 id) {
    HipbBuf *b = pool_get(id);
    if (b) b->host_valid = 0;
}

static u8 *stage_reserve(u64 n);

/* n bytes of device-readable pinned memory for an upload kernel to read:
 * the capturing graph's arena, else the upload ring (a segment is reused once
 * the work issued before it moved on has finished). NULL if there is none. */
static u8 *up_reserve(u64 n, u8 **dev) {
    if (hipb.capturing) {
        if (!P.arena_dev) return NULL;
        u8 *h = stage_reserve(n);
        if (!h) return NULL;
        *dev = P.arena_dev + (h - P.arena);
        return h;
    }
    if (!P.up || n > UP_MAX) return NULL;
    if (P.up_off + n > UP_SEG_BYTES) {
        /* the segment left is done once the work issued after its last
         * upload has finished: its event is recorded now, or, while launches
         * (upload kernels reading it among them) are held, once they go out,
         * so that the ring never decides which launches go out together */
        const u32 next = (P.up_seg + 1) % UP_SEGMENTS;
        if (P.up_closing == (i32)next) hipb_before_stream();   /* records it */
        if (hipb_holding()) {
            P.up_closing = (i32)P.up_seg;
        } else {
            HIPB_CHECK(hipEventRecord(P.up_done[P.up_seg], hipb.stream));
            P.up_pending[P.up_seg] = 1;
        }
        P.up_seg = next;
        if (P.up_pending[P.up_seg]) {
            hipb.n_stream_sync++;
            HIPB_CHECK(hipEventSynchronize(P.up_done[P.up_seg]));
            P.up_pending[P.up_seg] = 0;
        }
        P.up_off = 0;
    }
    const u64 o = (u64)P.up_seg * UP_SEG_BYTES + P.up_off;
    P.up_off += (n + 255) & ~255ull;
    *dev = P.up_dev + o;
    return P.up + o;
}

/* A host write of the whole buffer, just taken into the mirror, held as an
 * upload kernel: it goes out in one launch with the independent launches
 * held now, instead of as a copy of its own when a consumer needs it (that
 * copy would precede the consumer's launch and split no batch, but costs a
 * copy per write). Stays pending if it cannot be held. */
static void up_eager(u32 id, HipbBuf *b) {
    u8 *dev = NULL, *h = up_reserve(b->mirror_bytes, &dev);
    if (!h) return;
    memcpy(h, b->host_mirror, b->mirror_bytes);
    if (hipb_hold_upload(b->ptr, pool_bytes(id), dev, b->mirror_bytes)) b->dev_stale = 0;
}

/* Copy a pending host mirror to the device (stream ordered; ahead of held
 * launches that do not touch the buffer). */
void pool_sync_device(u32 id) {
    HipbBuf *b = pool_get(id);
    if (!b || !b->dev_stale) return;
    hipb_before_copy(b->ptr, b->cap);
    u8 *st = stage_reserve(b->mirror_bytes);
    memcpy(st, b->host_mirror, b->mirror_bytes);
    HIPB_CHECK(hipMemcpyAsync(b->ptr, st, b->mirror_bytes, hipMemcpyHostToDevice, hipb.stream));
    b->dev_stale = 0;
}

/* Every pending host mirror to the device: before work that reads buffers
 * without a dispatch naming them (a graph launch). */
void pool_sync_all_device(void) {
    for (u32 i = 1; i < P.count; i++)
        if (P.bufs[i].live && P.bufs[i].dev_stale) pool_sync_device(i);
}

/* No host mirror is current any more: after work that may write any buffer
 * without a dispatch naming it (a graph launch). Pending uploads first. */
void pool_device_wrote_all(void) {
    pool_sync_all_device();
    for (u32 i = 1; i < P.count; i++)
        if (P.bufs[i].live) P.bufs[i].host_valid = 0;
}

/* Reserve n bytes of pinned staging; waits only if the ring wraps onto a
 * segment whose copies are still in flight. */
static u8 *stage_reserve(u64 n) {
    if (hipb.capturing) {
        u64 need = (n + 255) & ~255ull;
        if (P.arena && P.arena_off + need <= P.arena_cap) {
            u8 *p = P.arena + P.arena_off;
            P.arena_off += need;
            return p;
        }
        pool_capture_forbids("uploads beyond the graph's staging arena");
    }
    if (P.seg_off + n > STAGE_SEG_BYTES) {
        HIPB_CHECK(hipEventRecord(P.seg_done[P.seg], hipb.stream));
        P.seg_pending[P.seg] = 1;
        P.seg = (P.seg + 1) % STAGE_SEGMENTS;
        if (P.seg_pending[P.seg]) {
            hipb.n_stream_sync++;
            HIPB_CHECK(hipEventSynchronize(P.seg_done[P.seg]));
            P.seg_pending[P.seg] = 0;
        }
        P.seg_off = 0;
    }
    u8 *p = P.stage + (u64)P.seg * STAGE_SEG_BYTES + P.seg_off;
    P.seg_off += (n + 255) & ~255ull;
    return p;
}

void pool_write(u32 id, const void *data, u64 bytes) {
    HipbBuf *b = pool_get(id);
    if (!b || !data || bytes == 0) return;
    b->write_capture = hipb.capturing ? P.capture_seq : 0;
    b->wseq = ++P.wclock;
    if (bytes > b->cap) {
        fprintf(stderr, "tinyhvm-hip: buf_write of %llu bytes into buffer %u of %llu bytes; truncated\n",
                (unsigned long long)bytes, id, (unsigned long long)b->cap);
        bytes = b->cap;
    }
    /* Defer small writes when the mirror then holds the whole buffer: a full
     * overwrite, or a partial one over contents the mirror already holds. */
    if (bytes <= POOL_MIRROR_MAX && (bytes >= b->bytes || b->host_valid)) {
        if (!b->host_mirror) b->host_mirror = malloc(POOL_MIRROR_MAX);
        if (b->host_mirror) {
            memcpy(b->host_mirror, data, bytes);
            if (bytes >= b->bytes) b->mirror_bytes = (u32)bytes;
            b->host_valid = 1;
            b->dev_stale = 1;
            /* small buffers (scalars, shapes) stay pending: their readers
             * often take them inline, and then they are never uploaded */
            if (bytes >= b->bytes && bytes > UP_EAGER_MIN) up_eager(id, b);
            return;
        }
    }
    pool_sync_device(id);
    hipb_before_copy(b->ptr, b->cap);
    b->dev_stale = 0;
    b->host_valid = 0;
    if (bytes <= STAGE_SEG_BYTES) {
        u8 *s = stage_reserve(bytes);
        memcpy(s, data, bytes);
        HIPB_CHECK(hipMemcpyAsync(b->ptr, s, bytes, hipMemcpyHostToDevice, hipb.stream));
    } else if (!pool_capture_forbids("a write larger than the staging segment")) {
        HIPB_CHECK(hipMemcpyAsync(b->ptr, data, bytes, hipMemcpyHostToDevice, hipb.stream));
        HIPB_CHECK(hipb_stream_wait());
    }
}

/* Host bytes to device memory on the stream (through the staging ring, so
 * the caller's memory may be reused on return). */
void pool_upload(void *dst, const void *src, u64 bytes) {
    if (!dst || !src || bytes == 0) return;
    hipb_before_copy(dst, bytes);
    if (bytes <= STAGE_SEG_BYTES) {
        u8 *s = stage_reserve(bytes);
        memcpy(s, src, bytes);
        HIPB_CHECK(hipMemcpyAsync(dst, s, bytes, hipMemcpyHostToDevice, hipb.stream));
    } else if (!pool_capture_forbids("an upload larger than the staging segment")) {
        HIPB_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, hipb.stream));
        HIPB_CHECK(hipb_stream_wait());
    }
}

void pool_read(u32 id, void *out, u64 bytes, int nosync) {
    HipbBuf *b = pool_get(id);
    if (!out || bytes == 0) return;
    if (!b) {
        memset(out, 0, bytes);
        return;
    }
    u64 n = bytes < b->bytes ? bytes : b->bytes;
    (void)nosync;
    if (!(b->host_valid && n <= b->mirror_bytes)) hipb_before_stream();
    if (b->host_valid && n <= b->mirror_bytes) {
        /* no device write since the host wrote it: the mirror is current */
        memcpy(out, b->host_mirror, n);
    } else if (pool_capture_forbids("a read back to the host")) {
        memset(out, 0, n);
    } else if (n <= STAGE_SEG_BYTES) {
        pool_sync_device(id);
        u8 *s = stage_reserve(n);
        HIPB_CHECK(hipMemcpyAsync(s, b->ptr, n, hipMemcpyDeviceToHost, hipb.stream));
        HIPB_CHECK(hipb_stream_wait());
        memcpy(out, s, n);
    } else {
        pool_sync_device(id);
        HIPB_CHECK(hipMemcpyAsync(out, b->ptr, n, hipMemcpyDeviceToHost, hipb.stream));
        HIPB_CHECK(hipb_stream_wait());
    }
    if (n < bytes) memset((u8 *)out + n, 0, bytes - n);
}

void pool_stats(u64 *live_bytes, u64 *cached_bytes, u64 *n_mallocs) {
    if (live_bytes) *live_bytes = P.live_bytes;
    if (cached_bytes) *cached_bytes = P.cached_bytes;
    if (n_mallocs) *n_mallocs = P.n_mallocs;
}
