/*
 * kargs.h - parameter blocks shared by the host (gcc) and the precompiled
 * kernels (hipcc), so both sides see one layout.
 */
#ifndef THVM_KARGS_H
#define THVM_KARGS_H

#include "thvm_abi.h"

/* dispatch_kernel_rs interpreter: copied to device memory per dispatch. */
typedef struct {
    u32 rank;
    u32 dims[MAX_DIM];
    u32 out_shape[MAX_DIM];
    u32 is_reduce[MAX_DIM];
    u32 has_reduce, reduce_type, post_start, n_post_leaves;
    u32 n_leaves, n_ops, out_dtype;
    u32 full_numel, out_numel, reduce_numel;
    u32 out_n;
    u32 leaf_dtype[FUSE_MAX_LEAVES];
    u32 leaf_n[FUSE_MAX_LEAVES];
    u32 leaf_st[FUSE_MAX_LEAVES];     /* index into sts, or 0xFFFFFFFF */
    u64 leaf_ptr[FUSE_MAX_LEAVES];
    u64 out_ptr;
    FusedOp ops[FUSE_MAX_OPS];
    View views[FUSE_MAX_LEAVES];
    ShapeTracker sts[1];              /* one per leaf with a stacked tracker */
} RsParams;

/* contiguify: passed by value as the kernel's only argument. dst_n/src_n
 * are capacities in elements of esize (2 or 4) bytes. */
typedef struct {
    u64 dst;
    u64 src;
    u32 dst_n;
    u32 src_n;
    u32 numel;
    u32 esize;
    View v;
} ContigArgs;

/* legacy per-op slots (op_unary / op_binary / op_mm / op_reduce): passed by
 * value. Capacities are in elements of each buffer's dtype. */
typedef struct {
    u64 dst, a, b;
    u32 dst_n, a_n, b_n;
    u32 n;                 /* outputs: dst numel, or M*N for mm */
    u32 uop, binary;
    u32 dd, ad, bd;        /* dtypes */
    u32 M, K, N;           /* mm; K doubles as reduce_dim for reduce */
    u32 pad;
    View av, bv;
} LegacyArgs;

/* batched buffer-to-buffer copies: passed by value */
#define COPY_BATCH_MAX 32
typedef struct {
    u32 n, pad;
    u64 dst[COPY_BATCH_MAX], src[COPY_BATCH_MAX], bytes[COPY_BATCH_MAX];
} CopyBatch;

/* adam_step (src/tinyhvm.h:1033-1035): parameter, gradient and moment
 * buffers of n f32 each; vec = 1 when all four are 16-byte aligned. */
typedef struct {
    u64 p, g, m, v;
    f32 lr, beta1, beta2, eps, bc1, bc2;
    u32 n, vec;
} AdamArgs;

/* KOp interpreter (the dispatch_uop_kernel fallback when a program cannot be
 * compiled): the program plus its loop pairing and the buffers, copied to
 * device memory per dispatch. pair[i] of a RANGE is its ENDRANGE and of an
 * ENDRANGE its RANGE; ftype[i] = 1 for ops whose value is a float. */
typedef struct {
    u64 out_ptr;
    u32 out_n, out_dtype;
    u64 leaf_ptr[FUSE_MAX_LEAVES];
    u32 leaf_n[FUSE_MAX_LEAVES];
    u32 leaf_dtype[FUSE_MAX_LEAVES];
    u32 n_ops, n_leaves, total, pad;
    u16 pair[KOP_MAX];
    u8 ftype[KOP_MAX];
    KOp ops[KOP_MAX];
} KopParams;

#endif
