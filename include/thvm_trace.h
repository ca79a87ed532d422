/*
 * thvm_trace.h - the kernel-trace format: a recorded sequence of Backend
 * vtable calls that can be replayed against any backend.
 *
 * It plays the role of the Metal backend's capture/replay command list
 * (src/backend/metal/jit.m:24-631): one training step, or one kernel, is
 * captured once from the engine and replayed without the engine.
 *
 * File layout (little-endian):
 *   8-byte magic "THVMTRC1", then records.
 *   Each record: u32 tag, u32 flags (0), u64 payload_len, payload bytes.
 *
 * Serialized sub-objects (all fields u32 unless noted):
 *   VIEW (56 words): rank, dims[8], strides[8] (i32), offset (i32), numel,
 *        contiguous, has_mask, mask_begin[8], mask_end[8], n_compound,
 *        2 x {dim_a, dim_b, stride_a (i32), begin, end}, mod_size[8]
 *   SHAPE (9 words): rank, dims[8]
 *   ST: n_views, then n_views x VIEW
 *   KOP (5 words): type, arg0, arg1, arg2, imm (raw bits)
 *   REDUCESPEC (21 words): is_reduce[8], reduce_type, post_reduce_start,
 *        n_post_leaves, reduce2_type, reduce2_start, is_reduce2[8]
 *
 * Record payloads:
 *   ALLOC     id, pad, u64 bytes
 *   FREE      id
 *   INCREF    id
 *   DECREF    id
 *   WRITE     id, enc, u64 bytes, then enc==RAW: bytes of data;
 *             enc==GEN: dist, dtype, u64 seed, f32 p0, f32 p1
 *   READ      id, has_data, u64 bytes, [data if has_data]
 *   UOP       out, n_leaves, leaf_bufs[n_leaves], u64 cache_key,
 *             n_ops, n_bufs, rank, SHAPE full, grid[3], tg[3], local_size,
 *             reduce_numel, out_dtype, coord_uop[8], KOP[n_ops],
 *             VIEW[n_leaves], leaf_dtypes[n_leaves]
 *   RS        out, n_leaves, leaf_bufs[n], VIEW[n], has_st[n], ST for each
 *             leaf with has_st, n_ops, FusedOp[n_ops] (4 words), SHAPE full,
 *             has_reduce, REDUCESPEC (if has_reduce), n_side,
 *             side_bufs[n_side], side_idx[n_side], has_dtypes,
 *             leaf_dtypes[n] (if has_dtypes), out_dtype
 *   COPY      dst, src, u64 bytes
 *   CONTIG    dst, numel, src, VIEW
 *   RESET     keep
 *   PERSIST   max_buf
 *   SNAPSHOT  id, source, u64 bytes, data   (buffer contents after the
 *             preceding dispatch: source 0 = produced by the engine's CPU
 *             backend; 2 = produced by the engine's CPU backend with its
 *             leaves in zero-filled guard memory, because its interpreter
 *             loads masked elements outside the buffer before discarding
 *             them; 1 = produced by the oracle, where neither could run)
 *   MARK      n, n bytes of text (annotation: phase names, config)
 *   OPUN      uop, dst, dst_dtype, VIEW dst_view, src, src_dtype, VIEW src_view
 *   OPBIN     uop, dst, dst_dtype, VIEW dst_view, a, a_dtype, VIEW a_view,
 *             b, b_dtype, VIEW b_view
 *   OPMM      dst, dst_dtype, a, a_dtype, VIEW a_view, b, b_dtype, VIEW b_view,
 *             M, K, N
 *   OPRED     uop, dst, dst_numel, dst_dtype, src, src_numel, src_dtype,
 *             reduce_dim
 *   (the OP* records are the legacy per-op slots op_unary, op_binary, op_mm,
 *   op_reduce, src/tinyhvm.h:1004-1016)
 *   ADAM      param, grad, m, v, f32 lr, f32 beta1, f32 beta2, f32 eps,
 *             f32 bc1, f32 bc2, n   (the adam_step slot, src/tinyhvm.h:1033-1035,
 *             as src/nn/adam.c:103-118 calls it)
 */
#ifndef THVM_TRACE_H
#define THVM_TRACE_H

#define THVM_TRACE_MAGIC "THVMTRC1"

enum {
    TRC_ALLOC = 1,
    TRC_FREE = 2,
    TRC_INCREF = 3,
    TRC_DECREF = 4,
    TRC_WRITE = 5,
    TRC_READ = 6,
    TRC_UOP = 7,
    TRC_RS = 8,
    TRC_COPY = 9,
    TRC_CONTIG = 10,
    TRC_RESET = 11,
    TRC_PERSIST = 12,
    TRC_SNAPSHOT = 13,
    TRC_MARK = 14,
    TRC_OPUN = 15,
    TRC_OPBIN = 16,
    TRC_OPMM = 17,
    TRC_OPRED = 18,
    TRC_ADAM = 19
};

enum { TRC_ENC_RAW = 0, TRC_ENC_GEN = 1 };

/* Synthetic input distributions for WRITE/GEN (generator: SplitMix64). */
enum {
    TRC_GEN_UNIFORM = 1,   /* U(p0, p1) */
    TRC_GEN_NORMAL = 2,    /* N(p0, p1^2), Box-Muller in f64 */
    TRC_GEN_INT = 3,       /* uniform integer in [p0, p1) */
    TRC_GEN_CONST = 4      /* every element = p0 */
};

#define TRC_VIEW_WORDS 56u
#define TRC_SHAPE_WORDS 9u
#define TRC_KOP_WORDS 5u
#define TRC_REDUCE_WORDS 21u

#endif /* THVM_TRACE_H */
