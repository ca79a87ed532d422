/*
 * thvm_replay.h - kernel-trace loading and replay against a Backend vtable.
 *
 * Replays the engine calls recorded in a trace (format: thvm_trace.h), the
 * vtable-level analogue of the Metal backend's capture/replay
 * (src/backend/metal/jit.m:24-631). No counterpart exists in the engine's C
 * API; the entry points are for benchmarks, tests and record/replay callers.
 */
#ifndef THVM_REPLAY_H
#define THVM_REPLAY_H

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ThvmTrace ThvmTrace;

enum {
    THVM_REPLAY_SKIP_READS = 1,   /* do not issue buf_read records */
    THVM_REPLAY_SKIP_WRITES = 2   /* do not issue buf_write records */
};

ThvmTrace *thvm_trace_load(const char *path);
void thvm_trace_free(ThvmTrace *t);
u32  thvm_trace_count(const ThvmTrace *t);
u32  thvm_trace_tag(const ThvmTrace *t, u32 index);
u32  thvm_trace_rec_id(const ThvmTrace *t, u32 index);
u64  thvm_trace_rec_bytes(const ThvmTrace *t, u32 index);
const void *thvm_trace_rec_data(const ThvmTrace *t, u32 index);
const UOpKernel *thvm_trace_rec_kernel(const ThvmTrace *t, u32 index);
/* Index of the first MARK record with this text at or after `from`, or -1. */
int  thvm_trace_find_mark(const ThvmTrace *t, const char *text, u32 from);
/* Replays records [lo, hi) against `be`; returns the number of dispatches, -1 on error. */
int  thvm_trace_replay(ThvmTrace *t, const Backend *be, u32 lo, u32 hi, u32 flags);
/* Backend buffer id currently bound to a trace buffer id (0 if none). */
u32  thvm_trace_live_id(const ThvmTrace *t, u32 trace_id);
/* Frees every buffer the replay allocated. */
void thvm_trace_release(ThvmTrace *t, const Backend *be);
/* Frees the host copies of generated inputs. */
void thvm_trace_drop_gen_cache(ThvmTrace *t);
/* Fills n 4-byte elements with the shared generator (thvm_gen.h) on `threads` threads (0 = auto). */
void thvm_gen_fill_parallel(void *dst, u32 dtype, u32 dist, u64 seed, f32 p0, f32 p1, u64 n, u32 threads);

#ifdef __cplusplus
}
#endif

#endif
