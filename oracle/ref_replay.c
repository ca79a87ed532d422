/*
 * ref_replay.c - times the engine's own CPU backend (src/backend/cpu/) on a
 * kernel trace: the CPU baseline next to the GPU numbers.
 *
 * Built only where the engine sources are present (oracle/Makefile, target
 * `ref`); the binary lands in oracle/_ref/. It replays records [0, setup_end)
 * once, then times `reps` replays of [lo, hi) on the calling thread.
 *
 * Usage: ref_replay <trace> <mark_lo> <mark_hi or -> <reps> [--check]
 * Prints one JSON line: {"seconds": total, "reps": n, "dispatches": d, "per_rep": s}.
 * --check compares each SNAPSHOT with the live buffer after replaying the
 * whole trace once (bit-exact), printing mismatches.
 */
#include "backend/cpu/_.c"
#include "thvm_replay.h"

#include <time.h>

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
    int check = argc > 5 && strcmp(argv[5], "--check") == 0;
    cpu_backend.init();
    u32 n = thvm_trace_count(t);
    if (check) {
        thvm_trace_replay(t, &cpu_backend, 0, n, 0);
        int bad = 0;
        for (u32 i = 0; i < n; i++) {
            if (thvm_trace_tag(t, i) != 13) continue;
            u32 live = thvm_trace_live_id(t, thvm_trace_rec_id(t, i));
            u64 b = thvm_trace_rec_bytes(t, i);
            if (!live || !cpu_pool.bufs[live] || memcmp(cpu_pool.bufs[live], thvm_trace_rec_data(t, i), b) != 0) {
                printf("snapshot %u differs\n", i);
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
    thvm_trace_replay(t, &cpu_backend, 0, (u32)lo, 0);
    int disp = 0;
    double t0 = now_s();
    for (int r = 0; r < reps; r++) disp += thvm_trace_replay(t, &cpu_backend, (u32)lo, (u32)hi, THVM_REPLAY_SKIP_READS);
    double dt = now_s() - t0;
    printf("{\"seconds\": %.6f, \"reps\": %d, \"dispatches\": %d, \"per_rep\": %.6f}\n", dt, reps, disp,
           reps ? dt / reps : 0.0);
    return 0;
}
