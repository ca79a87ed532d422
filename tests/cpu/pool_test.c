/*
 * pool_test.c - the buffer pool (tinyhvm_amd/csrc/pool.c) against the
 * engine's buffer contract, on the CPU with tests/cpu/fake_hip.c:
 *   - ids are nonzero and increasing, 0 means failure (src/tinyhvm.h:994);
 *   - ids stop below MAX_BUF_EPOCHS = 16384 (src/tinyhvm.h:720), as the CPU
 *     and Metal pools' MAX_BUFS (src/backend/cpu/pool.c:4,
 *     src/backend/metal/pool.m:50), until pool_reset recycles them;
 *   - buf_free is idempotent (views alias ids);
 *   - pool_reset(keep) releases ids > keep and numbering restarts at keep+1
 *     (src/backend/cpu/pool.c:19-26);
 *   - decref at or below the persistent floor is ignored;
 *   - out of device memory: cached blocks are returned and the allocation
 *     retried; if it still fails, buf_alloc returns 0;
 *   - blocks a HIP graph references never return to the free lists while the
 *     graph lives (freed ids, outgrown workspaces), and do once it is gone;
 *   - writes and reads round-trip through the host mirror and the staging ring.
 * Prints "pool_test: N checks passed" and exits 0, or names the failed check.
 */
#include <stdlib.h>
#include <string.h>

#include "hipb.h"

HipbState hipb;
hipError_t hipb_stream_wait(void) {
    hipb.n_stream_sync++;
    return hipStreamSynchronize(hipb.stream);
}
/* the backend's held dispatches (none here: the pool alone is under test) */
void hipb_before_stream(void) {}
void hipb_before_copy(const void *dst, u64 bytes) { (void)dst; (void)bytes; }
int hipb_held_buffer(u32 id) { (void)id; return 0; }
int hipb_holding(void) { return 0; }
/* an upload kernel run at once, on every other upload (the others take the
 * copy path) */
static u64 uploads_held;
int hipb_hold_upload(void *dst, u64 dst_bytes, const void *src_dev, u64 bytes) {
    static int turn;
    if (bytes > dst_bytes || (turn++ & 1)) return 0;
    memmove(dst, src_dev, bytes);
    uploads_held++;
    return 1;
}

extern size_t fake_hip_limit, fake_hip_live;
extern unsigned long fake_hip_mallocs, fake_hip_frees;

static int checks = 0;
#define CHECK(c)                                                              \
    do {                                                                      \
        checks++;                                                             \
        if (!(c)) {                                                           \
            fprintf(stderr, "pool_test: FAILED %s (line %d)\n", #c, __LINE__); \
            exit(1);                                                          \
        }                                                                     \
    } while (0)

static void test_ids(void) {
    u32 a = pool_alloc(100), b = pool_alloc(100);
    CHECK(a == 1 && b == 2);
    for (u32 i = 3; i < 16384; i++) CHECK(pool_alloc(4) == i);
    CHECK(pool_alloc(4) == 0);          /* the 16384th id does not exist */
    CHECK(pool_alloc(4) == 0);
    pool_reset(0);
    CHECK(pool_get(1) == NULL && pool_get(16383) == NULL);
    CHECK(pool_alloc(8) == 1);
    pool_reset(0);
}

static void test_free_reset_floor(void) {
    u32 a = pool_alloc(1024), b = pool_alloc(1024), c = pool_alloc(1024);
    CHECK(a && b && c);
    pool_free(b);
    pool_free(b);                       /* idempotent */
    pool_free(0);
    pool_free(999999);
    CHECK(pool_get(b) == NULL && pool_get(a) != NULL && pool_get(c) != NULL);
    pool_reset(a);                      /* keeps ids <= a */
    CHECK(pool_get(a) != NULL && pool_get(c) == NULL);
    CHECK(pool_alloc(16) == a + 1);
    /* persistent floor: decref at or below it is ignored */
    u32 d = pool_alloc(64);
    pool_set_persistent(d);
    pool_decref(d);
    CHECK(pool_get(d) != NULL);
    u32 e = pool_alloc(64);
    pool_incref(e);                     /* refcount 2 */
    pool_decref(e);
    CHECK(pool_get(e) != NULL);
    pool_decref(e);
    CHECK(pool_get(e) == NULL);
    pool_set_persistent(0);
    pool_reset(0);
}

static void test_oom(void) {
    pool_reset(0);
    u64 live = 0, cached = 0, mallocs = 0;
    pool_stats(&live, &cached, &mallocs);
    size_t base = fake_hip_live - cached;     /* what stays allocated once the cache is released */
    fake_hip_limit = base + (8u << 20);       /* 8 MiB more of "device memory" */
    u32 a = pool_alloc(3u << 20), b = pool_alloc(3u << 20);
    CHECK(a && b);
    CHECK(pool_alloc(3u << 20) == 0);          /* does not fit: failure, not a crash */
    pool_free(a);                              /* cached in the free list */
    u32 c = pool_alloc(3u << 20);              /* reuses the cached block */
    CHECK(c != 0 && pool_ptr(c) != NULL);
    pool_free(b);
    pool_free(c);
    /* a different size class: the cached blocks must be released for it */
    u32 d = pool_alloc(6u << 20);
    CHECK(d != 0);
    pool_free(d);
    fake_hip_limit = (size_t)1 << 40;
    pool_reset(0);
}

static void test_graph_pins(void) {
    pool_reset(0);
    u32 x = pool_alloc(4096), y = pool_alloc(4096), z = pool_alloc(4096);
    void *px = pool_ptr(x), *py = pool_ptr(y), *pz = pool_ptr(z);
    Scratch ws = {0};
    void *w0 = scratch_reserve(&ws, 4096);
    CHECK(px && py && pz && w0);
    pool_free(z);                              /* free before the capture: ordinary reuse */
    /* capture: x and y are used, a temporary t is made and freed, ws is used */
    PoolPins pins = {0};
    u8 *arena = malloc(1 << 16);
    hipb.capturing = 1;
    pool_capture_begin(arena, 1 << 16, &pins);
    CHECK(pool_get(x) && pool_get(y));
    u32 t = pool_alloc(4096);
    void *pt = pool_ptr(t);
    CHECK(pt != NULL && pt == pz);             /* z's block, not pinned before the capture */
    CHECK(scratch_reserve(&ws, 1024) == w0);
    pool_free(t);                              /* freed inside the capture: held for the graph */
    u32 t2 = pool_alloc(4096);
    CHECK(pool_ptr(t2) != pt);
    pool_capture_end();
    hipb.capturing = 0;
    u32 pinned = 0, limbo = 0;
    pool_pin_stats(&pinned, &limbo);
    CHECK(pinned >= 4 && limbo == 1);
    /* after the capture: frees and growth must not recycle the graph's blocks */
    pool_free(y);
    void *w1 = scratch_reserve(&ws, 1 << 20);  /* outgrown: w0 waits for the graph */
    CHECK(w1 != w0);
    int clash = 0;
    u32 fresh[8];
    for (int i = 0; i < 8; i++) {
        fresh[i] = pool_alloc(4096);
        void *p = pool_ptr(fresh[i]);
        if (p == px || p == py || p == pt || p == w0) clash = 1;
    }
    CHECK(!clash);
    pool_pin_stats(&pinned, &limbo);
    CHECK(limbo == 3);                         /* t, y and the old workspace */
    /* the graph is destroyed: its released blocks are reusable again */
    pool_pins_release(&pins);
    pool_pin_stats(&pinned, &limbo);
    CHECK(pinned == 0 && limbo == 0);
    int reused = 0;
    for (int i = 0; i < 4; i++) {
        void *p = pool_ptr(pool_alloc(4096));
        if (p == py || p == pt) reused++;
    }
    CHECK(reused == 2);
    scratch_release(&ws);
    free(arena);
    pool_reset(0);
}

static void test_write_read(void) {
    pool_reset(0);
    u32 a = pool_alloc(64), b = pool_alloc(1u << 20);
    u8 small[64], big[1u << 16], out[1u << 16];
    for (int i = 0; i < 64; i++) small[i] = (u8)(i * 7);
    for (u32 i = 0; i < sizeof big; i++) big[i] = (u8)(i * 13 + 1);
    pool_write(a, small, sizeof small);        /* held in the host mirror */
    memset(out, 0, sizeof out);
    pool_read(a, out, 80, 0);                  /* reading past the buffer zero-fills */
    CHECK(memcmp(out, small, 64) == 0 && out[64] == 0 && out[79] == 0);
    pool_sync_device(a);
    CHECK(memcmp(pool_ptr(a), small, 64) == 0);
    pool_write(b, big, sizeof big);            /* through the staging ring */
    pool_read(b, out, sizeof big, 0);
    CHECK(memcmp(out, big, sizeof big) == 0);
    u64 before = hipb.n_stream_sync;
    pool_read(b, out, 16, 0);
    CHECK(hipb.n_stream_sync == before + 1);   /* a device read waits for the stream */
    pool_reset(0);
}

/* Small writes reach the device through the upload ring: held as upload
 * kernels or copied, across several wraps of the ring's segments. */
static void test_uploads(void) {
    pool_reset(0);
    u32 a = pool_alloc(16384), b = pool_alloc(100);
    u8 src[16384];
    const u64 held0 = uploads_held;
    for (u32 r = 0; r < 600; r++) {
        for (u32 i = 0; i < sizeof src; i++) src[i] = (u8)(i * 31 + r);
        const u32 n = r % 3 == 0 ? 16384 : 4096 + r;
        pool_write(a, src, n);
        pool_sync_device(a);
        CHECK(memcmp(pool_ptr(a), src, n) == 0);
        pool_write(b, src + r, 100);
        pool_sync_device(b);
        CHECK(memcmp(pool_ptr(b), src + r, 100) == 0);
    }
    CHECK(uploads_held > held0);
    pool_reset(0);
}

int main(void) {
    memset(&hipb, 0, sizeof hipb);
    if (pool_init() != 0) {
        fprintf(stderr, "pool_test: pool_init failed\n");
        return 1;
    }
    hipb.dummy = pool_block_get(256, &hipb.dummy_cap);
    hipb.initialized = 1;
    test_ids();
    test_free_reset_floor();
    test_oom();
    test_graph_pins();
    test_write_read();
    test_uploads();
    pool_block_put(hipb.dummy, hipb.dummy_cap);
    pool_shutdown();
    CHECK(fake_hip_live == 0);                 /* everything went back */
    printf("pool_test: %d checks passed\n", checks);
    return 0;
}
