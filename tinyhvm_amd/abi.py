"""ctypes mirrors of the backend-boundary structs declared in include/thvm_abi.h.

Layouts follow the engine header src/tinyhvm.h (Shape :532, View :547,
ShapeTracker :572, FusedOp :659, ReduceSpec :660, KOp :693, UOpKernel :701,
Backend :988). Sizes are asserted at import.
"""
import ctypes as C

MAX_DIM = 8
ST_MAX_VIEWS = 4
FUSE_MAX_OPS = 64
FUSE_MAX_LEAVES = 64
KOP_MAX = 512

# UOp codes (src/tinyhvm.h:112-137)
UOP_NEG, UOP_EXP, UOP_LOG, UOP_RELU, UOP_CAST, UOP_SQRT = 3, 4, 5, 6, 7, 8
UOP_ADD, UOP_MUL, UOP_DIV, UOP_MAX, UOP_CMP, UOP_SUB = 9, 10, 11, 12, 13, 14
UOP_SUM, UOP_RMAX, UOP_MM = 15, 16, 17
UNARY_UOPS = {UOP_NEG, UOP_EXP, UOP_LOG, UOP_RELU, UOP_CAST, UOP_SQRT}

DTYPE_F32, DTYPE_F16, DTYPE_I32, DTYPE_U32 = 0, 1, 2, 3
DTYPE_SIZE = {0: 4, 1: 2, 2: 4, 3: 4}

(KOP_NOOP, KOP_GID, KOP_CONST_F, KOP_CONST_U, KOP_RANGE, KOP_ENDRANGE, KOP_LOAD,
 KOP_STORE, KOP_ALU, KOP_ACC_INIT, KOP_ACC, KOP_IDX, KOP_MOD, KOP_DIV, KOP_MASK) = range(15)
KOP_NAMES = ["NOOP", "GID", "CONST_F", "CONST_U", "RANGE", "ENDRANGE", "LOAD", "STORE",
             "ALU", "ACC_INIT", "ACC", "IDX", "MOD", "DIV", "MASK"]


class Shape(C.Structure):
    _fields_ = [("dims", C.c_uint32 * MAX_DIM), ("rank", C.c_uint32)]


class ViewCompoundMask(C.Structure):
    _fields_ = [("dim_a", C.c_uint8), ("dim_b", C.c_uint8), ("stride_a", C.c_int32),
                ("begin", C.c_uint32), ("end", C.c_uint32)]


class View(C.Structure):
    _fields_ = [("shape", Shape), ("strides", C.c_int32 * MAX_DIM), ("offset", C.c_int32),
                ("numel", C.c_uint32), ("contiguous", C.c_uint8), ("has_mask", C.c_uint8),
                ("mask_begin", C.c_uint32 * MAX_DIM), ("mask_end", C.c_uint32 * MAX_DIM),
                ("n_compound_masks", C.c_uint8), ("compound_masks", ViewCompoundMask * 2),
                ("mod_size", C.c_uint32 * MAX_DIM)]


class ShapeTracker(C.Structure):
    _fields_ = [("views", View * ST_MAX_VIEWS), ("n_views", C.c_uint8)]


class FusedOp(C.Structure):
    _fields_ = [("uop", C.c_uint32), ("arg_a", C.c_uint32), ("arg_b", C.c_uint32),
                ("aux", C.c_uint32)]


class ReduceSpec(C.Structure):
    _fields_ = [("is_reduce", C.c_uint8 * MAX_DIM), ("reduce_type", C.c_uint32),
                ("post_reduce_start", C.c_uint32), ("n_post_leaves", C.c_uint32),
                ("reduce2_type", C.c_uint32), ("reduce2_start", C.c_uint32),
                ("is_reduce2", C.c_uint8 * MAX_DIM)]


class KOpImm(C.Union):
    _fields_ = [("f", C.c_float), ("u", C.c_uint32)]


class KOp(C.Structure):
    _fields_ = [("type", C.c_int), ("arg", C.c_uint32 * 3), ("imm", KOpImm)]


class UOpKernel(C.Structure):
    _fields_ = [("ops", KOp * KOP_MAX), ("n_ops", C.c_uint32), ("n_bufs", C.c_uint32),
                ("n_leaves", C.c_uint32), ("leaf_views", View * FUSE_MAX_LEAVES),
                ("leaf_dtypes", C.c_uint32 * FUSE_MAX_LEAVES),
                ("coord_uop", C.c_uint32 * MAX_DIM), ("rank", C.c_uint32),
                ("full_shape", Shape), ("grid", C.c_uint32 * 3), ("tg", C.c_uint32 * 3),
                ("local_size", C.c_uint32), ("reduce_numel", C.c_uint32),
                ("out_dtype", C.c_uint32)]


_FP = C.CFUNCTYPE
_u32, _u64, _f32, _vp = C.c_uint32, C.c_uint64, C.c_float, C.c_void_p
_PView = C.POINTER(View)


class Backend(C.Structure):
    _fields_ = [
        ("init", _FP(C.c_int)),
        ("shutdown", _FP(None)),
        ("buf_alloc", _FP(_u32, _u64)),
        ("buf_free", _FP(None, _u32)),
        ("buf_incref", _FP(None, _u32)),
        ("buf_decref", _FP(None, _u32)),
        ("mem_checkpoint", _FP(None, C.POINTER(_u32), _u32)),
        ("buf_mark_use", _FP(None, _u32)),
        ("buf_write", _FP(None, _u32, _vp, _u64)),
        ("buf_read", _FP(None, _u32, _vp, _u64)),
        ("op_unary", _FP(None, _u32, _u32, _PView, _u32, _u32, _PView, _u32)),
        ("op_binary", _FP(None, _u32, _u32, _PView, _u32, _u32, _PView, _u32, _u32, _PView, _u32)),
        ("op_mm", _FP(None, _u32, _u32, _u32, _PView, _u32, _u32, _PView, _u32, _u32, _u32, _u32)),
        ("op_reduce", _FP(None, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32)),
        ("dispatch_kernel_rs", _FP(None, _u32, C.POINTER(_u32), C.POINTER(_PView),
                                   C.POINTER(C.POINTER(ShapeTracker)), _u32,
                                   C.POINTER(FusedOp), _u32, C.POINTER(Shape),
                                   C.POINTER(ReduceSpec), C.POINTER(_u32), C.POINTER(_u32),
                                   _u32, C.POINTER(_u32), _u32)),
        ("dispatch_uop_kernel", _FP(None, _u32, C.POINTER(_u32), _u32, C.POINTER(UOpKernel),
                                    _u64)),
        ("contiguify", _FP(None, _u32, _u32, _u32, _PView)),
        ("buf_copy", _FP(None, _u32, _u32, _u64)),
        ("buf_read_nosync", _FP(None, _u32, _vp, _u64)),
        ("adam_step", _FP(None, _u32, _u32, _u32, _u32, _f32, _f32, _f32, _f32, _f32, _f32,
                          _u32)),
        ("pool_reset", _FP(None, _u32)),
        ("pool_set_persistent", _FP(None, _u32)),
        ("begin_batch", _FP(None)),
        ("end_batch", _FP(None)),
        ("profile_report", _FP(None)),
        ("profile_reset", _FP(None)),
    ]


assert C.sizeof(View) == 212
assert C.sizeof(ShapeTracker) == 852
assert C.sizeof(ReduceSpec) == 36
assert C.sizeof(KOp) == 20
assert C.sizeof(UOpKernel) == 24184
assert C.sizeof(Backend) == 208
