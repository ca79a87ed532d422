/*
 * ora_replay.c - times the oracle (this directory's CPU restatement of the
 * engine's interpreter) on a kernel trace, on the calling thread. It is the
 * CPU baseline where the engine's own CPU backend cannot run a workload
 * (padded convolutions fault in its interpreter).
 *
 * Usage: ora_replay <trace> <mark_lo> <mark_hi or -> <reps>
 * Prints {"seconds": total, "reps": n, "dispatches": d, "per_rep": s}.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "thvm_abi.h"
#include "thvm_replay.h"

extern Backend oracle_backend;

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec * 1e-9;
}

int main(int argc, char **argv) {
    if (argc < 5) {
        fprintf(stderr, "usage: ora_replay <trace> <mark_lo> <mark_hi|-> <reps>\n");
        return 2;
    }
    ThvmTrace *t = thvm_trace_load(argv[1]);
    if (!t) { fprintf(stderr, "cannot load %s\n", argv[1]); return 1; }
    oracle_backend.init();
    u32 n = thvm_trace_count(t);
    int lo = thvm_trace_find_mark(t, argv[2], 0);
    if (lo < 0) { fprintf(stderr, "mark %s not found\n", argv[2]); return 1; }
    int hi = strcmp(argv[3], "-") == 0 ? (int)n : thvm_trace_find_mark(t, argv[3], (u32)lo);
    if (hi < 0) hi = (int)n;
    int reps = atoi(argv[4]);
    thvm_trace_replay(t, &oracle_backend, 0, (u32)lo, 0);
    int disp = 0;
    double t0 = now_s();
    for (int r = 0; r < reps; r++) disp += thvm_trace_replay(t, &oracle_backend, (u32)lo, (u32)hi, THVM_REPLAY_SKIP_READS);
    double dt = now_s() - t0;
    printf("{\"seconds\": %.6f, \"reps\": %d, \"dispatches\": %d, \"per_rep\": %.6f}\n", dt, reps, disp,
           reps ? dt / reps : 0.0);
    return 0;
}
