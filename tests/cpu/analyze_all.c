/*
 * analyze_all.c - runs the backend's device-free program analysis over every
 * lowered kernel of the given kernel traces: the kernel generator
 * (thvm_hip_kernel_source, thvm_hip_kernel_lanes), the matrix-core
 * recognizer (thvm_hip_dense_analyze, thvm_hip_dense_source) and the
 * pooling-window / run-sum recognizer (thvm_hip_window_analyze,
 * thvm_hip_window_source). Built with
 * AddressSanitizer and UndefinedBehaviorSanitizer, it checks that parsing
 * the engine-supplied programs neither reads nor writes out of bounds nor
 * hits undefined arithmetic. No GPU is used. Also feeds each program with
 * its op count cut short, and with out-of-range op arguments, which the
 * analyses must reject or handle without a fault.
 * Prints "analyze_all: N kernels" and exits 0 when no sanitizer fired.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "thvm_abi.h"
#include "thvm_hip.h"
#include "thvm_replay.h"

static char src[1 << 20];
static u32 lanes[7 * KOP_MAX];

static void analyze(const UOpKernel *k) {
    u32 mode = 0, vec = 0, M, N, K, S, kind;
    thvm_hip_kernel_source(k, src, sizeof src, &mode, &vec);
    thvm_hip_kernel_lanes(k, lanes, 7 * KOP_MAX, &mode, &vec);
    if (thvm_hip_dense_analyze(k, &M, &N, &K, &S)) thvm_hip_dense_source(k, src, sizeof src);
    if (thvm_hip_window_analyze(k, &kind, &S)) thvm_hip_window_source(k, src, sizeof src);
}

int main(int argc, char **argv) {
    unsigned long n = 0;
    UOpKernel *k = malloc(sizeof *k);
    for (int a = 1; a < argc; a++) {
        ThvmTrace *t = thvm_trace_load(argv[a]);
        if (!t) {
            fprintf(stderr, "analyze_all: cannot load %s\n", argv[a]);
            return 1;
        }
        for (u32 i = 0; i < thvm_trace_count(t); i++) {
            const UOpKernel *rk = thvm_trace_rec_kernel(t, i);
            if (!rk) continue;
            analyze(rk);
            n++;
            /* truncated programs: every prefix length at a few points */
            memcpy(k, rk, sizeof *k);
            for (u32 cut = 1; cut < rk->n_ops; cut += 1 + rk->n_ops / 7) {
                k->n_ops = cut;
                analyze(k);
            }
            /* dangling operands: every argument of one op pointed past the program */
            memcpy(k, rk, sizeof *k);
            if (k->n_ops > 2) {
                u32 j = k->n_ops / 2;
                k->ops[j].arg[0] = k->ops[j].arg[1] = k->ops[j].arg[2] = 0xFFFFFFF0u;
                analyze(k);
            }
            /* an op count past the array */
            memcpy(k, rk, sizeof *k);
            k->n_ops = KOP_MAX + 5;
            analyze(k);
        }
        thvm_trace_free(t);
    }
    free(k);
    printf("analyze_all: %lu kernels\n", n);
    return 0;
}
