/*
 * ref_replay.c - times the engine's own CPU backend (src/backend/cpu/) on a
 * kernel trace: the CPU baseline next to the GPU numbers.
 *
 * Built only where the engine sources are present (oracle/Makefile, target
 * `ref`); the binary lands in oracle/_ref/. It replays records [0, setup_end)
 * once, then times `reps` replays of [lo, hi) on the calling thread.
 *
 * Usage: ref_replay <trace> <mark_lo> <mark_hi or -> <reps> [--check] [--guard]
 * Prints one JSON line: {"seconds": total, "reps": n, "dispatches": d, "per_rep": s}.
 * --check replays the whole trace once, comparing each SNAPSHOT with the live
 * buffer at that point (bit-exact), and prints the mismatches.
 * --guard places every buffer at the start of its own zero-filled, lazily
 * mapped region spanning every u32 element index of a 4-byte type. The
 * interpreter loads a leaf element before the mask that discards it
 * (src/backend/cpu/uop.c:55-72), so a zero-padded view (a convolution's pad,
 * whose negative offset wraps to a large u32 index) reads outside its buffer
 * and faults on plain heap blocks; over these regions the stray loads read
 * zeros that the masks discard, and every kernel runs unchanged on the
 * engine's own interpreter. The regions are placed at allocation, outside the
 * per-dispatch work, so the timed replays run the interpreter and nothing else.
 */
#include "backend/cpu/_.c"
#include "thvm_replay.h"

#include <sys/mman.h>
#include <time.h>

#define GUARD_SPAN (((u64)1 << 34) + 65536)

static u32 guard_alloc(u64 b) {
    u32 id = cpu_buf_alloc(b);
    void *m = mmap(NULL, GUARD_SPAN, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
    if (m == MAP_FAILED) {
        fprintf(stderr, "ref_replay: guard mapping failed for buffer %u\n", id);
        exit(1);
    }
    free(cpu_pool.bufs[id]);
    cpu_pool.bufs[id] = m;
    return id;
}

static void guard_release(u32 id) {
    if (cpu_pool.bufs[id]) munmap(cpu_pool.bufs[id], GUARD_SPAN);
    cpu_pool.bufs[id] = NULL;
}

static void guard_free(u32 id) { guard_release(id); }

/* The engine's CPU backend has no buf_copy slot: ASSIGN of a contiguous
 * source reads it to the host and writes it back (thvm_to_host_raw, then
 * buf_write; src/interact/tensor_ops.c:121-136), which moves the same bytes
 * as this. (contiguify and adam_step records, which only the assign and adam
 * fixtures hold, are not replayed on this backend.) */
static void host_copy(u32 dst, u32 src, u64 nbytes) {
    if (!cpu_pool.bufs[dst] || !cpu_pool.bufs[src]) return;
    u64 n = nbytes;
    if (n > cpu_pool.sizes[dst]) n = cpu_pool.sizes[dst];
    if (n > cpu_pool.sizes[src]) n = cpu_pool.sizes[src];
    memmove(cpu_pool.bufs[dst], cpu_pool.bufs[src], n);
}

static void guard_reset(u32 keep) {
    for (u32 i = keep + 1; i < cpu_pool.count; i++) guard_release(i);
    cpu_pool.count = keep + 1;
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec * 1e-9;
}

int main(int argc, char **argv) {
    if (argc < 5) {
        fprintf(stderr, "usage: ref_replay <trace> <mark_lo> <mark_hi|-> <reps> [--check]\n");
        return 2;
    }
    ThvmTrace *t = thvm_trace_load(argv[1]);
    if (!t) { fprintf(stderr, "cannot load %s\n", argv[1]); return 1; }
    int check = 0, guard = 0;
    for (int a = 5; a < argc; a++) {
        check |= strcmp(argv[a], "--check") == 0;
        guard |= strcmp(argv[a], "--guard") == 0;
    }
    Backend be = cpu_backend;
    be.buf_copy = host_copy;
    if (guard) {
        be.buf_alloc = guard_alloc;
        be.buf_free = guard_free;
        be.pool_reset = guard_reset;
    }
    be.init();
    u32 n = thvm_trace_count(t);
    if (check) {
        int bad = 0;
        for (u32 i = 0; i < n; i++) {
            if (thvm_trace_tag(t, i) != 13) {
                thvm_trace_replay(t, &be, i, i + 1, 0);
                continue;
            }
            u32 live = thvm_trace_live_id(t, thvm_trace_rec_id(t, i));
            u64 b = thvm_trace_rec_bytes(t, i);
            if (!live || !cpu_pool.bufs[live] || memcmp(cpu_pool.bufs[live], thvm_trace_rec_data(t, i), b) != 0) {
                u64 nd = 0;
                for (u64 j = 0; live && cpu_pool.bufs[live] && j + 4 <= b; j += 4)
                    nd += memcmp((u8 *)cpu_pool.bufs[live] + j, (const u8 *)thvm_trace_rec_data(t, i) + j, 4) != 0;
                printf("snapshot %u differs (after a record of tag %u): %llu of %llu words\n", i,
                       i ? thvm_trace_tag(t, i - 1) : 0, (unsigned long long)nd, (unsigned long long)(b / 4));
                bad++;
            }
        }
        printf("{\"check_mismatches\": %d}\n", bad);
        return bad ? 1 : 0;
    }
    int lo = thvm_trace_find_mark(t, argv[2], 0);
    if (lo < 0) { fprintf(stderr, "mark %s not found\n", argv[2]); return 1; }
    int hi = strcmp(argv[3], "-") == 0 ? (int)n : thvm_trace_find_mark(t, argv[3], (u32)lo);
    if (hi < 0) hi = (int)n;
    int reps = atoi(argv[4]);
    thvm_trace_replay(t, &be, 0, (u32)lo, 0);
    int disp = 0;
    double t0 = now_s();
    for (int r = 0; r < reps; r++) disp += thvm_trace_replay(t, &be, (u32)lo, (u32)hi, THVM_REPLAY_SKIP_READS);
    double dt = now_s() - t0;
    printf("{\"seconds\": %.6f, \"reps\": %d, \"dispatches\": %d, \"per_rep\": %.6f}\n", dt, reps, disp,
           reps ? dt / reps : 0.0);
    return 0;
}
