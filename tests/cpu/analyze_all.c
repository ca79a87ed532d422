/*
 * analyze_all.c - runs the backend's device-free program analysis over every
 * lowered kernel of the given kernel traces: the kernel generator
 * (thvm_hip_kernel_source, thvm_hip_kernel_lanes), the matrix-core
 * recognizer (thvm_hip_dense_analyze, thvm_hip_dense_source) and the
 * pooling-window / run-sum recognizer (thvm_hip_window_analyze,
 * thvm_hip_window_source), and the merge of two consecutive programs
 * (thvm_hip_chain_merge, the second reading the first's output as its
 * first leaf; a merged program is analysed in turn). Built with
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

/* p followed by c, c's first leaf standing for p's output */
static unsigned long merge_pair(const UOpKernel *p, const UOpKernel *c, UOpKernel *m) {
    u32 pb[1 + FUSE_MAX_LEAVES], cl[FUSE_MAX_LEAVES], mb[1 + FUSE_MAX_LEAVES];
    pb[0] = 1000;
    for (u32 j = 0; j < FUSE_MAX_LEAVES; j++) {
        pb[1 + j] = 1 + j;
        cl[j] = j == 0 ? 1000 : 2000 + j;
    }
    if (!thvm_hip_chain_merge(p, pb, c, 3000, cl, m, mb)) return 0;
    analyze(m);
    return 1;
}

int main(int argc, char **argv) {
    unsigned long n = 0, merged = 0;
    UOpKernel *k = malloc(sizeof *k), *m = malloc(sizeof *m);
    for (int a = 1; a < argc; a++) {
        ThvmTrace *t = thvm_trace_load(argv[a]);
        if (!t) {
            fprintf(stderr, "analyze_all: cannot load %s\n", argv[a]);
            return 1;
        }
        const UOpKernel *prev = NULL;
        for (u32 i = 0; i < thvm_trace_count(t); i++) {
            const UOpKernel *rk = thvm_trace_rec_kernel(t, i);
            if (!rk) continue;
            analyze(rk);
            n++;
            if (prev) merged += merge_pair(prev, rk, m);
            prev = rk;
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
            merge_pair(k, rk, m);
            merge_pair(rk, k, m);
        }
        thvm_trace_free(t);
    }
    free(k);
    free(m);
    printf("analyze_all: %lu kernels, %lu merged pairs\n", n, merged);
    return 0;
}
