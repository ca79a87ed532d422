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

/* contiguify: passed by value as the kernel's only argument. */
typedef struct {
    u64 dst;
    u64 src;
    u32 dst_n;
    u32 src_n;
    u32 numel;
    u32 pad;
    View v;
} ContigArgs;

#endif
