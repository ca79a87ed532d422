/*
 * thvm_hip.h - C ABI of the MI355X (gfx950) HIP backend for TinyHVM.
 *
 * The drop-in is the vtable `hip_backend`, a `Backend` exactly like the
 * engine's `cpu_backend` (src/backend/cpu/_.c:21) and `metal_backend`
 * (src/backend/metal/_.m:30); the engine registers it from thvm_init
 * (src/ctx/init.c:17-35). The flat thvm_hip_* functions below are the same
 * slots under plain names, for FFI callers (ctypes) that do not walk a vtable.
 *
 * All calls come from one host thread in dependency order (the engine's
 * contract, src/schedule/_.c:2005-2043). Work is enqueued on one HIP stream;
 * only buf_read (and large buf_writes) block.
 */
#ifndef THVM_HIP_H
#define THVM_HIP_H

#include "thvm_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The vtable. Replaces cpu_backend / metal_backend (src/tinyhvm.h:988-1046). */
extern Backend hip_backend;

/* Backend.init / .shutdown (src/tinyhvm.h:990-991). init returns 0 on success
 * and -1 without a usable gfx950 device (the engine then stays on the CPU,
 * src/ctx/init.c:26-33). */
int  thvm_hip_init(void);
void thvm_hip_shutdown(void);

/* Backend.buf_alloc (src/tinyhvm.h:994): nonzero id, 0 on failure. */
u32  thvm_hip_buf_alloc(u64 bytes);
/* Backend.buf_free (src/tinyhvm.h:995): idempotent. */
void thvm_hip_buf_free(u32 id);
/* Backend.buf_incref / buf_decref (src/tinyhvm.h:996-997). */
void thvm_hip_buf_incref(u32 id);
void thvm_hip_buf_decref(u32 id);
/* Backend.buf_write (src/tinyhvm.h:1000): the host buffer may be reused on return. */
void thvm_hip_buf_write(u32 id, const void *data, u64 bytes);
/* Backend.buf_read (src/tinyhvm.h:1001): waits for all enqueued work. */
void thvm_hip_buf_read(u32 id, void *out, u64 bytes);
/* Backend.buf_read_nosync (src/tinyhvm.h:1032): serves host-written metadata
 * without a device sync when no kernel has written the buffer since. */
void thvm_hip_buf_read_nosync(u32 id, void *out, u64 bytes);

/* Backend.dispatch_uop_kernel (src/tinyhvm.h:1027-1029), called from
 * thvm_sched_dispatch_kernel (src/schedule/_.c:2370-2371). */
void thvm_hip_dispatch_uop_kernel(u32 out_buf, const u32 *leaf_bufs, u32 n_leaves,
                                  const UOpKernel *kernel, u64 cache_key);
/* Backend.dispatch_kernel_rs (src/tinyhvm.h:1020-1026), the fallback the
 * scheduler uses when lowering fails (src/schedule/_.c:2372-2379). */
void thvm_hip_dispatch_kernel_rs(u32 out_buf, u32 *leaf_bufs, const View **leaf_views,
                                 const ShapeTracker *const *leaf_sts, u32 n_leaves,
                                 FusedOp *ops, u32 n_ops, const Shape *full_shape,
                                 const ReduceSpec *reduce, u32 *side_bufs,
                                 const u32 *side_op_indices, u32 n_side_outputs,
                                 const u32 *leaf_dtypes, u32 out_dtype);
/* Backend.contiguify / buf_copy (src/tinyhvm.h:1030-1031), used by ASSIGN
 * (src/interact/tensor_ops.c:113-120). */
void thvm_hip_contiguify(u32 dst_buf, u32 numel, u32 src_buf, const View *src_view);
void thvm_hip_buf_copy(u32 dst_buf, u32 src_buf, u64 nbytes);
/* Backend.pool_reset / pool_set_persistent (src/tinyhvm.h:1039-1040). */
void thvm_hip_pool_reset(u32 keep);
void thvm_hip_pool_set_persistent(u32 max_buf);
/* Backend.op_unary / op_binary / op_mm / op_reduce (src/tinyhvm.h:1004-1016),
 * the legacy per-op slots of the ENSURE/materialize path
 * (src/fuse/materialize.c:195,672,683,700); semantics of
 * src/backend/cpu/ops.c. */
void thvm_hip_op_unary(u32 uop, u32 dst, const View *dst_view, u32 dst_dtype, u32 src,
                       const View *src_view, u32 src_dtype);
void thvm_hip_op_binary(u32 uop, u32 dst, const View *dst_view, u32 dst_dtype, u32 a, const View *a_view,
                        u32 a_dtype, u32 b, const View *b_view, u32 b_dtype);
void thvm_hip_op_mm(u32 dst, u32 dst_dtype, u32 a, const View *a_view, u32 a_dtype, u32 b,
                    const View *b_view, u32 b_dtype, u32 M, u32 K, u32 N);
void thvm_hip_op_reduce(u32 uop, u32 dst, u32 dst_numel, u32 dst_dtype, u32 src, u32 src_numel,
                        u32 src_dtype, u32 reduce_dim);
/* Backend.adam_step (src/tinyhvm.h:1033-1035), as adam_step_direct calls it
 * (src/nn/adam.c:103-118): param, m and v updated in place over n f32
 * elements with the arithmetic of the engine's lazy update (src/nn/adam.c:
 * 75-88): m' = beta1*m + (1-beta1)*g, v' = beta2*v + (1-beta2)*(g*g),
 * p' = p - lr*((m'/bc1)/(sqrt(v'/bc2)+eps)). A buffer shorter than n elements
 * makes the call a no-op. */
void thvm_hip_adam_step(u32 param, u32 grad, u32 m, u32 v, f32 lr, f32 beta1, f32 beta2, f32 eps, f32 bc1,
                        f32 bc2, u32 n);
/* Backend.profile_report / profile_reset (src/tinyhvm.h:1044-1045). */
void thvm_hip_profile_report(void);
void thvm_hip_profile_reset(void);

/* ---- additions with no counterpart in the engine ---- */
/* HIP graphs of recorded work, for callers that repeat a fixed stretch of
 * backend calls (a training step replayed from a kernel trace): the kernel
 * trace replay of the Metal backend's JIT record/replay role
 * (src/backend/metal/jit.m:24-631) taken one step further.
 *   thvm_hip_graph_begin    start capturing the stream (0, or -1)
 *   thvm_hip_graph_end      stop; the graph, or NULL when the captured calls
 *                           included work a graph cannot repeat (a host read
 *                           or synchronize, a write over 16 MiB)
 *   thvm_hip_graph_launch   run the captured work again (0, or -1)
 *   thvm_hip_graph_destroy  release it (waits for the stream)
 * Capture runs nothing on the device. A launch repeats the captured kernels
 * with their captured arguments and uploads on the current contents of the
 * device memory they touch. That memory stays reserved for the graph until
 * it is destroyed: buffers freed during or after the capture, and outgrown
 * workspaces, are not handed to later allocations while a graph holds them.
 * thvm_hip_shutdown releases every graph's device resources; a handle is
 * still destroyed with thvm_hip_graph_destroy afterwards. */
int   thvm_hip_graph_begin(void);
void *thvm_hip_graph_end(void);
int   thvm_hip_graph_launch(void *graph);
void  thvm_hip_graph_destroy(void *graph);

/* Dispatch without allocation. No counterpart in the reference: it is for
 * callers that cannot allocate device memory while they dispatch (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The same work as thvm_hip_dispatch_uop_kernel, with the same kernels in the
 * same order (so the same bits), except that every workspace its kernels use
 * (split-K partial sums, split reduction partials, packed GEMM operands) comes
 * from a static device array of THVM_HIP_NOALLOC_SCRATCH_BYTES per GPU,
 * reserved when the library initialises, and that it never compiles: the
 * program must have run once through thvm_hip_dispatch_uop_kernel (also
 * when it ran there fused into another dispatch's launch). It calls
 * no hipMalloc or hipFree. All calls on one GPU share the array; calls are
 * ordered on the backend's single stream, so consecutive calls are safe,
 * but calls that overlap on one GPU (from other streams or threads) race.
 * Returns THVM_HIP_OK, or:
 *   THVM_HIP_EINVAL     not initialised, no kernel, or an unknown output buffer
 *   THVM_HIP_ENOTREADY  the program has not been compiled yet (or runs only on
 *                       the KOp interpreter, which is not offered here)
 *   THVM_HIP_ESCRATCH   its workspaces need more than THVM_HIP_NOALLOC_SCRATCH_BYTES
 *   THVM_HIP_ENOSCRATCH the static array is not available on this device
 * On an error nothing is launched and the output is not written. */
#define THVM_HIP_NOALLOC_SCRATCH_BYTES (32ull << 20)
#define THVM_HIP_OK 0
#define THVM_HIP_EINVAL (-1)
#define THVM_HIP_ENOTREADY (-2)
#define THVM_HIP_ESCRATCH (-3)
#define THVM_HIP_ENOSCRATCH (-4)
int  thvm_hip_dispatch_uop_kernel_noalloc(u32 out_buf, const u32 *leaf_bufs, u32 n_leaves,
                                          const UOpKernel *kernel);

/* Counters, for tests and the engine-driven timing (no counterpart in the
 * reference): out[0..15] = dispatches, matrix-core dispatches, compiled
 * programs, program cache hits, dispatches run on the KOp interpreter
 * (programs the generator or hipRTC refused; their outputs are still
 * written), host waits on the stream, live device bytes, hipMalloc calls,
 * device blocks pinned by HIP graphs, released blocks held for graphs,
 * dispatches run on the window-max and run-sum kernels, dispatches issued
 * inside a batched launch, elementwise dispatches run as the fused epilogue
 * of the contraction whose output they read, host waits after which a
 * single-pass combine was found to have given up waiting for a partial sum,
 * host uploads copied by an upload kernel held with other launches,
 * dispatches issued as steps of a sequence kernel (dependent small launches
 * run in order by one workgroup). Returns the number of counters (16). */
int  thvm_hip_counters(u64 *out, u32 n);
/* Wait for all enqueued work; returns 0, or -1 on a device error or when a
 * kernel that combines its workgroups' partial sums in one pass gave up
 * waiting for one of them since the last call (its output then holds a
 * NaN; buf_read reports the same on stderr and in the counters). */
int  thvm_hip_synchronize(void);
/* The hipStream_t all work is ordered on (for timing with events). */
void *thvm_hip_stream(void);
/* Issues the launches the backend holds back (independent dispatches it
 * batches, queued copies), without waiting: a caller that puts work of its
 * own on thvm_hip_stream() (a timing event) calls it first so that the
 * stream has every earlier dispatch ahead of that work. No counterpart in
 * the reference (its backends issue every dispatch at once). */
void thvm_hip_flush(void);
/* Device address of a buffer (for tests and timing harnesses). */
void *thvm_hip_buf_device_ptr(u32 id);
/* The vtable, for callers that cannot read exported data symbols. */
const Backend *thvm_hip_backend(void);
/* sizeof(View), sizeof(ShapeTracker), sizeof(UOpKernel), sizeof(Backend). */
int  thvm_hip_abi_sizes(u32 *out, u32 n);
/* Generated HIP source for a kernel (no device needed). Returns its length,
 * or -1 with the reason in buf. mode: 0 serial, 1 group; vec: lanes per thread. */
int  thvm_hip_kernel_source(const UOpKernel *kernel, char *buf, u64 buflen, u32 *mode, u32 *vec);
/* The generator's vector-lane classification of a kernel's ops (no device
 * needed), 7 words per op: kind (0 the same on every lane of a thread-vector,
 * 1 lane v = lane 0 + off[v], 2 varying, 3 float valued), off[0..3], a divisor
 * of the lane-0 value (0: that value is 0) and an upper bound of the value.
 * Returns the number of ops, or -1. A diagnostic with no counterpart in the
 * reference: it lets tests check the index analysis against the op semantics. */
int  thvm_hip_kernel_lanes(const UOpKernel *kernel, u32 *lanes, u32 n_words, u32 *mode, u32 *vec);
/* Generate and compile with hipRTC for gfx950, without loading (no device
 * needed). Returns the code-object size, or -1 with the reason in errbuf. */
int  thvm_hip_compile_check(const UOpKernel *kernel, char *errbuf, u64 errlen);

/* Whether a kernel is a contraction the backend runs on matrix cores, and its
 * GEMM shape (no device needed). Reads THVM_HIP_DENSE_FORCE /
 * THVM_HIP_DENSE_SPLITS before init. Returns 1 if so, else 0. */
int  thvm_hip_dense_analyze(const UOpKernel *kernel, u32 *M, u32 *N, u32 *K, u32 *splits);
/* Generated HIP source of that matrix-core kernel (no device needed); returns
 * its length, or -1 with the reason in buf. */
int  thvm_hip_dense_source(const UOpKernel *kernel, char *buf, u64 buflen);
/* Generate and compile that matrix-core kernel without loading it; returns the
 * code-object size, or -1 with the reason in errbuf. */
int  thvm_hip_dense_compile_check(const UOpKernel *kernel, char *errbuf, u64 errlen);

/* Whether a kernel is a window max (the RMAX over a pooling window that
 * thvm_maxpool2d lowers to, src/nn/conv.c:484-514) or a run sum (a long SUM
 * over contiguous runs into few outputs: batchnorm's per-channel statistics,
 * src/nn/batchnorm.c:35-111, bias gradients, loss sums) that the backend runs
 * on its dedicated kernels (no device needed). kind: 0 neither, 1 window max,
 * 2 run sum; splits: workgroups per output. Returns 1 if so, else 0. */
int  thvm_hip_window_analyze(const UOpKernel *kernel, u32 *kind, u32 *splits);
/* Its generated HIP source; returns the length, or -1 with the reason in buf. */
int  thvm_hip_window_source(const UOpKernel *kernel, char *buf, u64 buflen);
/* Generate and compile it without loading; the code-object size, or -1. */
int  thvm_hip_window_compile_check(const UOpKernel *kernel, char *errbuf, u64 errlen);

/* An elementwise dispatch that reads a matrix-core contraction's output at
 * its own index runs in that contraction's epilogue (no launch of its own)
 * when the contraction's launch is still held: the fused module of producer
 * and consumer (which reads the producer's output as leaf buffer o_leaf, 1 +
 * leaf), compiled without loading (no device needed). Returns the
 * code-object size, or -1 with the reason in errbuf (also when the pair does
 * not fuse). A diagnostic with no counterpart in the reference. */
int  thvm_hip_epilogue_compile_check(const UOpKernel *producer, const UOpKernel *consumer, u32 o_leaf,
                                     char *errbuf, u64 errlen);

/* A loop-free dispatch that reads a held loop-free program's output at its
 * own gid runs fused after it, as one program over both programs' buffers
 * that writes both outputs (its STOREs name their buffer in imm.u, like the
 * engine's KOp STORE, src/tinyhvm.h:683). The merged program of producer p
 * (buffer ids pb: output, then leaves) and consumer c (output c_out, leaves
 * c_leaves), as the backend builds it, without a device: returns 1 with m
 * and its buffer ids mb (output, then m->n_leaves leaves) filled, 0 when
 * the pair does not fuse. A diagnostic with no counterpart in the
 * reference. */
int  thvm_hip_chain_merge(const UOpKernel *p, const u32 *pb, const UOpKernel *c, u32 c_out, const u32 *c_leaves,
                          UOpKernel *m, u32 *mb);

/* Run sums of one shape that follow each other (batchnorm's sums over one
 * tensor, src/nn/batchnorm.c:35-111) run as one launch that reads what they
 * share once; a held elementwise program or window max whose output they
 * read is computed inside it (and still stored), and elementwise programs
 * over their outputs (the mean, the variance, the inverse deviation) run in
 * the workgroup that combines each output. The group kernel of programs
 * ks[0..n) over buffer ids bufs[i] (output, then leaves), the first the
 * producer when `producer` is set, generated and compiled without loading
 * (no device needed). Returns the code-object size, or -1 with the reason in
 * errbuf (also when a program does not join). A diagnostic with no
 * counterpart in the reference. */
int  thvm_hip_group_compile_check(const UOpKernel *const *ks, const u32 *const *bufs, u32 n, int producer,
                                  char *errbuf, u64 errlen);
/* Its source (length, or -1 with the reason in buf). */
int  thvm_hip_group_source(const UOpKernel *const *ks, const u32 *const *bufs, u32 n, int producer, char *buf,
                           u64 buflen);

/* Timing of one matrix-core kernel: with two hipEvent_t, the next
 * contraction dispatch records ev_begin on the backend stream right before
 * its main kernel and ev_end right after it (the kernel then goes out on its
 * own instead of in a batch; a pack or split-K sum kernel of the same
 * dispatch stays outside the pair). NULL, NULL disarms. Returns 1 if the
 * previous pair was recorded, 0 if not, -1 before thvm_hip_init. For
 * benchmarks (the rocprof kernel statistics name the same kernel); no
 * counterpart in the reference. */
int  thvm_hip_time_contraction(void *ev_begin, void *ev_end);

/* Source of the upload kernel (main kernel thvm_upload, 256 lanes): host
 * writes of at most 64 KiB reach the device through it, read from pinned
 * coherent host memory, and it joins a batch launch with independent held
 * work. Length, or -1. A diagnostic with no counterpart in the reference. */
int  thvm_hip_upload_source(char *buf, u64 buflen);

/* Independent dispatches held back and issued as one launch: the batch
 * kernel of n generated modules (srcs[i] as the generators above return it,
 * names[i] its main kernel, threads[i] its workgroup size, grid[2i], grid[2i+1]
 * its grid), compiled without loading (no device needed). Returns the
 * code-object size, or -1 with the reason in errbuf. A diagnostic with no
 * counterpart in the reference: it checks the generated modules' device-
 * function forms that batched launches compile. */
int  thvm_hip_batch_compile_check(const char *const *srcs, const char *const *names, const u32 *threads,
                                  const u32 *grid, u32 n, char *errbuf, u64 errlen);
/* The same for the sequence kernel of dependent small launches (the programs
 * run in order by one 256-lane workgroup); -1 also when a program cannot be
 * a step of a sequence (more than 4 workgroups, more than 256 lanes, or
 * workgroup barriers or LDS of its own). A diagnostic with no counterpart in
 * the reference. */
int  thvm_hip_seq_compile_check(const char *const *srcs, const char *const *names, const u32 *threads,
                                const u32 *grid, u32 n, char *errbuf, u64 errlen);

#ifdef __cplusplus
}
#endif

#endif /* THVM_HIP_H */
