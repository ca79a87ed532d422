/*
 * thvm_abi.h - the data types that cross TinyHVM's backend boundary.
 *
 * A backend receives these structs from the engine by pointer, so every
 * layout below must be byte-identical to the engine's own definitions in
 * src/tinyhvm.h (cited per type). The layout test in tests/ compiles a probe
 * against the engine header and compares sizeof/offsetof for every field.
 *
 * Conventions kept from the engine:
 *   - all compute is f32; storage dtypes are f32/f16/i32/u32;
 *   - element indices are u32 and wrap modulo 2^32;
 *   - buffers are named by nonzero u32 ids (0 is the null buffer).
 */
#ifndef THVM_ABI_H
#define THVM_ABI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint8_t  u8;
typedef uint16_t u16;
typedef uint32_t u32;
typedef uint64_t u64;
typedef int32_t  i32;
typedef float    f32;

/* UOp codes used inside kernels (src/tinyhvm.h:112-137). */
enum {
    UOP_NEG = 3, UOP_EXP = 4, UOP_LOG = 5, UOP_RELU = 6, UOP_CAST = 7,
    UOP_SQRT = 8, UOP_ADD = 9, UOP_MUL = 10, UOP_DIV = 11, UOP_MAX = 12,
    UOP_CMP = 13, UOP_SUB = 14, UOP_SUM = 15, UOP_RMAX = 16, UOP_MM = 17
};

/* Storage dtypes (src/tinyhvm.h:419-423). */
enum { DTYPE_F32 = 0, DTYPE_F16 = 1, DTYPE_I32 = 2, DTYPE_U32 = 3, DTYPE_COUNT = 4 };

#define MAX_DIM          8   /* src/tinyhvm.h:528 */
#define ST_MAX_VIEWS     4   /* src/tinyhvm.h:574 */
#define FUSE_MAX_OPS    64   /* src/tinyhvm.h:656 */
#define FUSE_MAX_LEAVES 64   /* src/tinyhvm.h:657 */
#define KOP_MAX        512   /* src/tinyhvm.h:674 */

/* Shape: src/tinyhvm.h:532-535. */
typedef struct {
    u32 dims[MAX_DIM];
    u32 rank;
} Shape;

/* Strided, optionally masked view of a buffer: src/tinyhvm.h:547-565.
 * Element (c0..c{r-1}) lives at offset + sum(c_d * strides[d]). A view with
 * has_mask reads 0 outside mask_begin[d] <= c_d < mask_end[d] and outside each
 * compound mask begin <= c[dim_a]*stride_a + c[dim_b] < end. */
typedef struct {
    u8  dim_a, dim_b;
    i32 stride_a;
    u32 begin, end;
} ViewCompoundMask;

typedef struct {
    Shape shape;
    i32   strides[MAX_DIM];
    i32   offset;
    u32   numel;
    u8    contiguous;
    u8    has_mask;
    u32   mask_begin[MAX_DIM];
    u32   mask_end[MAX_DIM];
    u8    n_compound_masks;
    ViewCompoundMask compound_masks[2];
    u32   mod_size[MAX_DIM];
} View;

/* Stack of views composed right-to-left: src/tinyhvm.h:572-577. */
typedef struct {
    View views[ST_MAX_VIEWS];
    u8   n_views;
} ShapeTracker;

/* Fused elementwise op; arg indices < n_leaves name leaves, the rest name
 * earlier ops (n_leaves + op index): src/tinyhvm.h:659. */
typedef struct { u32 uop; u32 arg_a; u32 arg_b; u32 aux; } FusedOp;

/* Reduction spec: src/tinyhvm.h:660-672. */
typedef struct {
    u8  is_reduce[MAX_DIM];
    u32 reduce_type;
    u32 post_reduce_start;
    u32 n_post_leaves;
    u32 reduce2_type;
    u32 reduce2_start;
    u8  is_reduce2[MAX_DIM];
} ReduceSpec;

/* Linear kernel program ops: src/tinyhvm.h:675-691. */
typedef enum {
    KOP_NOOP = 0,
    KOP_GID,       /* flat output position (imm.u = axis, always 0 in practice) */
    KOP_CONST_F,   /* imm.f */
    KOP_CONST_U,   /* imm.u */
    KOP_RANGE,     /* reduce loop over [0, imm.u) */
    KOP_ENDRANGE,  /* closes the loop opened by op arg[0] */
    KOP_LOAD,      /* buffer imm.u (0 = output, 1+i = leaf i) at index arg[0] */
    KOP_STORE,     /* output[arg[0]] = arg[1] */
    KOP_ALU,       /* UOp imm.u on arg[0], arg[1]; arg[2] = aux (CAST dtype) */
    KOP_ACC_INIT,  /* accumulator, initial value imm.f */
    KOP_ACC,       /* acc(arg[0]) <- reduce imm.u (SUM/RMAX) with arg[1] */
    KOP_IDX,       /* arg[0] * imm.u + arg[1] */
    KOP_MOD,       /* arg[0] % imm.u */
    KOP_DIV,       /* arg[0] / imm.u */
    KOP_MASK       /* arg[0] != 0 ? arg[1] : 0.0f */
} KOpType;

typedef struct {
    KOpType type;
    u32     arg[3];
    union { f32 f; u32 u; } imm;
} KOp;

/* Lowered kernel handed to dispatch_uop_kernel: src/tinyhvm.h:701-717. */
typedef struct {
    KOp   ops[KOP_MAX];
    u32   n_ops;
    u32   n_bufs;
    u32   n_leaves;
    View  leaf_views[FUSE_MAX_LEAVES];
    u32   leaf_dtypes[FUSE_MAX_LEAVES];
    u32   coord_uop[MAX_DIM];
    u32   rank;
    Shape full_shape;
    u32   grid[3];
    u32   tg[3];
    u32   local_size;
    u32   reduce_numel;
    u32   out_dtype;
} UOpKernel;

/* Backend vtable: src/tinyhvm.h:988-1046. Slot order is the ABI. */
typedef struct Backend Backend;
struct Backend {
    int   (*init)(void);
    void  (*shutdown)(void);
    u32   (*buf_alloc)(u64 bytes);
    void  (*buf_free)(u32 id);
    void  (*buf_incref)(u32 id);
    void  (*buf_decref)(u32 id);
    void  (*mem_checkpoint)(u32 *leaf_buf_ids, u32 n_leaves);
    void  (*buf_mark_use)(u32 id);
    void  (*buf_write)(u32 id, const void *data, u64 bytes);
    void  (*buf_read)(u32 id, void *out, u64 bytes);
    void  (*op_unary)(u32 uop, u32 dst, const View *dv, u32 dst_dtype,
                      u32 src, const View *sv, u32 src_dtype);
    void  (*op_binary)(u32 uop, u32 dst, const View *dv, u32 dst_dtype,
                       u32 a, const View *av, u32 a_dtype,
                       u32 b, const View *bv, u32 b_dtype);
    void  (*op_mm)(u32 dst, u32 dst_dtype,
                   u32 a, const View *av, u32 a_dtype, u32 b, const View *bv, u32 b_dtype,
                   u32 M, u32 K, u32 N);
    void  (*op_reduce)(u32 uop, u32 dst, u32 dst_numel, u32 dst_dtype,
                       u32 src, u32 src_numel, u32 src_dtype, u32 reduce_dim);
    void  (*dispatch_kernel_rs)(u32 out_buf,
                                u32 *leaf_bufs, const View **leaf_views,
                                const ShapeTracker *const *leaf_sts, u32 n_leaves,
                                FusedOp *ops, u32 n_ops,
                                const Shape *full_shape, const ReduceSpec *reduce,
                                u32 *side_bufs, const u32 *side_op_indices, u32 n_side_outputs,
                                const u32 *leaf_dtypes, u32 out_dtype);
    void  (*dispatch_uop_kernel)(u32 out_buf, const u32 *leaf_bufs, u32 n_leaves,
                                 const UOpKernel *kernel, u64 cache_key);
    void  (*contiguify)(u32 dst_buf, u32 numel, u32 src_buf, const View *src_view);
    void  (*buf_copy)(u32 dst_buf, u32 src_buf, u64 nbytes);
    void  (*buf_read_nosync)(u32 id, void *out, u64 bytes);
    void  (*adam_step)(u32 param, u32 grad, u32 m, u32 v,
                       f32 lr, f32 beta1, f32 beta2, f32 eps,
                       f32 bc1, f32 bc2, u32 n);
    void  (*pool_reset)(u32 keep);
    void  (*pool_set_persistent)(u32 max_buf);
    void  (*begin_batch)(void);
    void  (*end_batch)(void);
    void  (*profile_report)(void);
    void  (*profile_reset)(void);
};

/* Layout constants checked at compile time and against the engine header. */
#define THVM_ABI_SIZEOF_VIEW          212u
#define THVM_ABI_SIZEOF_SHAPETRACKER  852u
#define THVM_ABI_SIZEOF_UOPKERNEL   24184u
#define THVM_ABI_SIZEOF_BACKEND       208u

#ifdef __cplusplus
}
#endif

#endif /* THVM_ABI_H */
