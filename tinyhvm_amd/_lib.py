"""ctypes binding of libthvm_hip.so (include/thvm_hip.h, include/thvm_replay.h).

Loading fails loudly when the library has not been built: there is no CPU
fallback behind these entry points.
"""
import ctypes as C
import os

from . import abi

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libthvm_hip.so")

_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError("libthvm_hip.so is not built (run __graft_entry__.build() "
                           "or python -m tinyhvm_amd.build)")
    L = C.CDLL(LIB_PATH)
    u32, u64, f32, vp, cp = C.c_uint32, C.c_uint64, C.c_float, C.c_void_p, C.c_char_p
    PU32 = C.POINTER(u32)
    sigs = {
        "thvm_hip_init": (C.c_int, []),
        "thvm_hip_shutdown": (None, []),
        "thvm_hip_buf_alloc": (u32, [u64]),
        "thvm_hip_buf_free": (None, [u32]),
        "thvm_hip_buf_incref": (None, [u32]),
        "thvm_hip_buf_decref": (None, [u32]),
        "thvm_hip_buf_write": (None, [u32, vp, u64]),
        "thvm_hip_buf_read": (None, [u32, vp, u64]),
        "thvm_hip_buf_read_nosync": (None, [u32, vp, u64]),
        "thvm_hip_dispatch_uop_kernel": (None, [u32, PU32, u32, C.POINTER(abi.UOpKernel), u64]),
        "thvm_hip_dispatch_kernel_rs": (None, [u32, PU32, C.POINTER(C.POINTER(abi.View)),
                                               C.POINTER(C.POINTER(abi.ShapeTracker)), u32,
                                               C.POINTER(abi.FusedOp), u32, C.POINTER(abi.Shape),
                                               C.POINTER(abi.ReduceSpec), PU32, PU32, u32, PU32,
                                               u32]),
        "thvm_hip_contiguify": (None, [u32, u32, u32, C.POINTER(abi.View)]),
        "thvm_hip_op_unary": (None, [u32, u32, C.POINTER(abi.View), u32, u32, C.POINTER(abi.View), u32]),
        "thvm_hip_op_binary": (None, [u32, u32, C.POINTER(abi.View), u32, u32, C.POINTER(abi.View), u32, u32,
                                      C.POINTER(abi.View), u32]),
        "thvm_hip_op_mm": (None, [u32, u32, u32, C.POINTER(abi.View), u32, u32, C.POINTER(abi.View), u32, u32,
                                  u32, u32]),
        "thvm_hip_op_reduce": (None, [u32, u32, u32, u32, u32, u32, u32, u32]),
        "thvm_hip_adam_step": (None, [u32, u32, u32, u32, f32, f32, f32, f32, f32, f32, u32]),
        "thvm_hip_graph_begin": (C.c_int, []),
        "thvm_hip_graph_end": (vp, []),
        "thvm_hip_graph_launch": (C.c_int, [vp]),
        "thvm_hip_graph_destroy": (None, [vp]),
        "thvm_hip_buf_copy": (None, [u32, u32, u64]),
        "thvm_hip_pool_reset": (None, [u32]),
        "thvm_hip_pool_set_persistent": (None, [u32]),
        "thvm_hip_profile_report": (None, []),
        "thvm_hip_profile_reset": (None, []),
        "thvm_hip_synchronize": (C.c_int, []),
        "thvm_hip_counters": (C.c_int, [C.POINTER(u64), u32]),
        "thvm_hip_dispatch_uop_kernel_noalloc": (C.c_int, [u32, PU32, u32, C.POINTER(abi.UOpKernel)]),
        "thvm_hip_stream": (vp, []),
        "thvm_hip_buf_device_ptr": (vp, [u32]),
        "thvm_hip_backend": (C.POINTER(abi.Backend), []),
        "thvm_hip_abi_sizes": (C.c_int, [PU32, u32]),
        "thvm_hip_kernel_source": (C.c_int, [C.POINTER(abi.UOpKernel), cp, u64, PU32, PU32]),
        "thvm_hip_kernel_lanes": (C.c_int, [C.POINTER(abi.UOpKernel), PU32, u32, PU32, PU32]),
        "thvm_hip_compile_check": (C.c_int, [C.POINTER(abi.UOpKernel), cp, u64]),
        "thvm_hip_dense_analyze": (C.c_int, [C.POINTER(abi.UOpKernel), PU32, PU32, PU32, PU32]),
        "thvm_hip_dense_compile_check": (C.c_int, [C.POINTER(abi.UOpKernel), cp, u64]),
        "thvm_hip_dense_source": (C.c_int, [C.POINTER(abi.UOpKernel), cp, u64]),
        "thvm_hip_window_analyze": (C.c_int, [C.POINTER(abi.UOpKernel), PU32, PU32]),
        "thvm_hip_window_source": (C.c_int, [C.POINTER(abi.UOpKernel), cp, u64]),
        "thvm_hip_window_compile_check": (C.c_int, [C.POINTER(abi.UOpKernel), cp, u64]),
        "thvm_hip_flush": (None, []),
        "thvm_hip_chain_merge": (C.c_int, [C.POINTER(abi.UOpKernel), PU32, C.POINTER(abi.UOpKernel), u32,
                                           PU32, C.POINTER(abi.UOpKernel), PU32]),
        "thvm_hip_epilogue_compile_check": (C.c_int, [C.POINTER(abi.UOpKernel), C.POINTER(abi.UOpKernel), u32, cp,
                                                      u64]),
        "thvm_hip_batch_compile_check": (C.c_int, [C.POINTER(C.c_char_p), C.POINTER(C.c_char_p), PU32, PU32, u32,
                                                   cp, u64]),
        "thvm_hip_seq_compile_check": (C.c_int, [C.POINTER(C.c_char_p), C.POINTER(C.c_char_p), PU32, PU32, u32,
                                                 cp, u64]),
        "thvm_hip_group_compile_check": (C.c_int, [C.POINTER(C.POINTER(abi.UOpKernel)), C.POINTER(PU32), u32,
                                                   C.c_int, cp, u64]),
        "thvm_hip_time_contraction": (C.c_int, [vp, vp]),
        "thvm_hip_upload_source": (C.c_int, [cp, u64]),
        "thvm_hip_group_source": (C.c_int, [C.POINTER(C.POINTER(abi.UOpKernel)), C.POINTER(PU32), u32, C.c_int,
                                            cp, u64]),
        "thvm_trace_load": (vp, [cp]),
        "thvm_trace_free": (None, [vp]),
        "thvm_trace_count": (u32, [vp]),
        "thvm_trace_tag": (u32, [vp, u32]),
        "thvm_trace_rec_id": (u32, [vp, u32]),
        "thvm_trace_rec_bytes": (u64, [vp, u32]),
        "thvm_trace_rec_data": (vp, [vp, u32]),
        "thvm_trace_rec_kernel": (C.POINTER(abi.UOpKernel), [vp, u32]),
        "thvm_trace_find_mark": (C.c_int, [vp, cp, u32]),
        "thvm_trace_replay": (C.c_int, [vp, C.POINTER(abi.Backend), u32, u32, u32]),
        "thvm_trace_live_id": (u32, [vp, u32]),
        "thvm_trace_release": (None, [vp, C.POINTER(abi.Backend)]),
        "thvm_trace_drop_gen_cache": (None, [vp]),
        "thvm_gen_fill_parallel": (None, [vp, u32, u32, u64, f32, f32, u64, u32]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


EXPORTED = ["hip_backend"] + [
    "thvm_hip_init", "thvm_hip_shutdown", "thvm_hip_buf_alloc", "thvm_hip_buf_free",
    "thvm_hip_buf_incref", "thvm_hip_buf_decref", "thvm_hip_buf_write", "thvm_hip_buf_read",
    "thvm_hip_buf_read_nosync", "thvm_hip_dispatch_uop_kernel", "thvm_hip_dispatch_kernel_rs",
    "thvm_hip_contiguify", "thvm_hip_op_unary", "thvm_hip_op_binary", "thvm_hip_op_mm",
    "thvm_hip_op_reduce", "thvm_hip_adam_step", "thvm_hip_graph_begin", "thvm_hip_graph_end",
    "thvm_hip_graph_launch", "thvm_hip_graph_destroy", "thvm_hip_buf_copy", "thvm_hip_pool_reset",
    "thvm_hip_pool_set_persistent", "thvm_hip_profile_report", "thvm_hip_profile_reset",
    "thvm_hip_synchronize", "thvm_hip_counters", "thvm_hip_dispatch_uop_kernel_noalloc", "thvm_hip_stream", "thvm_hip_buf_device_ptr", "thvm_hip_backend",
    "thvm_hip_abi_sizes", "thvm_hip_kernel_source", "thvm_hip_kernel_lanes", "thvm_hip_compile_check",
    "thvm_hip_dense_analyze", "thvm_hip_dense_compile_check", "thvm_hip_dense_source",
    "thvm_hip_window_analyze", "thvm_hip_window_source", "thvm_hip_window_compile_check",
    "thvm_hip_batch_compile_check", "thvm_hip_flush", "thvm_hip_epilogue_compile_check", "thvm_hip_chain_merge",
    "thvm_hip_group_compile_check", "thvm_hip_group_source", "thvm_hip_upload_source", "thvm_hip_time_contraction",
    "thvm_hip_seq_compile_check",
    "thvm_trace_load", "thvm_trace_free", "thvm_trace_count", "thvm_trace_tag",
    "thvm_trace_rec_id", "thvm_trace_rec_bytes", "thvm_trace_rec_data", "thvm_trace_rec_kernel",
    "thvm_trace_find_mark", "thvm_trace_replay", "thvm_trace_live_id", "thvm_trace_release",
    "thvm_trace_drop_gen_cache", "thvm_gen_fill_parallel",
]


def gen_bytes(dist, dtype, seed, p0, p1, nbytes):
    n = nbytes // (2 if dtype == abi.DTYPE_F16 else 4)
    buf = (C.c_uint8 * max(nbytes, 4))()
    lib().thvm_gen_fill_parallel(C.cast(buf, C.c_void_p), dtype, dist, seed, p0, p1, n, 0)
    return bytes(buf)[:nbytes]


def kernel_source(k: abi.UOpKernel):
    buf = C.create_string_buffer(1 << 20)
    mode, vec = C.c_uint32(), C.c_uint32()
    n = lib().thvm_hip_kernel_source(C.byref(k), buf, len(buf), C.byref(mode), C.byref(vec))
    text = buf.value.decode()
    if n < 0:
        raise ValueError(text)
    return text, mode.value, vec.value


def batch_compile_check(items):
    """Compile the batch kernel of generated modules without a device; items
    are (source, main kernel name, workgroup size, gx, gy). Returns the
    code-object size; raises ValueError with the compiler's reason."""
    n = len(items)
    srcs = (C.c_char_p * n)(*[it[0].encode() for it in items])
    names = (C.c_char_p * n)(*[it[1].encode() for it in items])
    threads = (C.c_uint32 * n)(*[it[2] for it in items])
    grid = (C.c_uint32 * (2 * n))(*[v for it in items for v in (it[3], it[4])])
    err = C.create_string_buffer(4096)
    r = lib().thvm_hip_batch_compile_check(srcs, names, threads, grid, n, err, len(err))
    if r < 0:
        raise ValueError(err.value.decode())
    return r


def seq_compile_check(items):
    """Compile the sequence kernel of generated modules without a device
    (items as for batch_compile_check). Returns the code-object size; raises
    ValueError with the reason."""
    n = len(items)
    srcs = (C.c_char_p * n)(*[it[0].encode() for it in items])
    names = (C.c_char_p * n)(*[it[1].encode() for it in items])
    threads = (C.c_uint32 * n)(*[it[2] for it in items])
    grid = (C.c_uint32 * (2 * n))(*[v for it in items for v in (it[3], it[4])])
    err = C.create_string_buffer(4096)
    r = lib().thvm_hip_seq_compile_check(srcs, names, threads, grid, n, err, len(err))
    if r < 0:
        raise ValueError(err.value.decode())
    return r


def chain_merge(p: abi.UOpKernel, pb, c: abi.UOpKernel, c_out: int, c_leaves):
    """The merged program of loop-free p (buffer ids pb: output, leaves)
    followed by c (output c_out, leaves c_leaves): (m, mb), or None when
    the pair does not fuse."""
    W = C.c_uint32 * (1 + abi.FUSE_MAX_LEAVES)
    m = abi.UOpKernel()
    mb, pbv, clv = W(), W(*pb), W(*c_leaves)
    if not lib().thvm_hip_chain_merge(C.byref(p), pbv, C.byref(c), c_out, clv, C.byref(m), mb):
        return None
    return m, list(mb[:1 + m.n_leaves])


def epilogue_compile_check(producer: abi.UOpKernel, consumer: abi.UOpKernel, o_leaf: int):
    """Code-object size of the fused module of a contraction and the
    elementwise consumer of its output; raises ValueError with the reason
    when the pair does not fuse or does not compile."""
    err = C.create_string_buffer(4096)
    r = lib().thvm_hip_epilogue_compile_check(C.byref(producer), C.byref(consumer), o_leaf, err, len(err))
    if r < 0:
        raise ValueError(err.value.decode())
    return r


def _group_args(kernels, bufs):
    n = len(kernels)
    ks = (C.POINTER(abi.UOpKernel) * n)(*[C.pointer(k) for k in kernels])
    arrs = [(C.c_uint32 * len(b))(*b) for b in bufs]
    pu = C.POINTER(C.c_uint32)
    bp = (pu * n)(*[C.cast(a, pu) for a in arrs])
    return ks, bp, arrs


def group_source(kernels, bufs, producer=False):
    """Source of the run-sum group kernel of `kernels` (the first the taken-in
    producer when `producer`) over buffer ids `bufs` (per program: output,
    then leaves); raises ValueError with the reason when they do not group."""
    ks, bp, _keep = _group_args(kernels, bufs)
    buf = C.create_string_buffer(1 << 20)
    n = lib().thvm_hip_group_source(ks, bp, len(kernels), int(producer), buf, len(buf))
    if n < 0:
        raise ValueError(buf.value.decode())
    return buf.value.decode()


def upload_source():
    buf = C.create_string_buffer(1 << 20)
    if lib().thvm_hip_upload_source(buf, len(buf)) < 0:
        raise ValueError("no upload kernel source")
    return buf.value.decode()


def group_compile_check(kernels, bufs, producer=False):
    """Code-object size of that kernel (compiled without a device)."""
    ks, bp, _keep = _group_args(kernels, bufs)
    err = C.create_string_buffer(4096)
    r = lib().thvm_hip_group_compile_check(ks, bp, len(kernels), int(producer), err, len(err))
    if r < 0:
        raise ValueError(err.value.decode())
    return r


def dense_analyze(k: abi.UOpKernel):
    """(M, N, K, splits) if the backend runs this kernel on matrix cores, else None."""
    M, N, K, S = C.c_uint32(), C.c_uint32(), C.c_uint32(), C.c_uint32()
    if lib().thvm_hip_dense_analyze(C.byref(k), C.byref(M), C.byref(N), C.byref(K), C.byref(S)):
        return M.value, N.value, K.value, S.value
    return None


def dense_source(k: abi.UOpKernel):
    buf = C.create_string_buffer(1 << 20)
    n = lib().thvm_hip_dense_source(C.byref(k), buf, len(buf))
    if n < 0:
        raise ValueError(buf.value.decode())
    return buf.value.decode()


def dense_compile_check(k: abi.UOpKernel):
    err = C.create_string_buffer(512)
    n = lib().thvm_hip_dense_compile_check(C.byref(k), err, len(err))
    if n < 0:
        raise RuntimeError(err.value.decode())
    return n


def compile_check(k: abi.UOpKernel):
    err = C.create_string_buffer(512)
    n = lib().thvm_hip_compile_check(C.byref(k), err, len(err))
    if n < 0:
        raise RuntimeError(err.value.decode())
    return n


def kernel_lanes(k: abi.UOpKernel):
    """The generator's vector-lane classification: (mode, vec, rows), one row
    per op (kind, off0..off3, divisor, bound); see thvm_hip_kernel_lanes."""
    n = 7 * max(int(k.n_ops), 1)
    buf = (C.c_uint32 * n)()
    mode, vec = C.c_uint32(), C.c_uint32()
    r = lib().thvm_hip_kernel_lanes(C.byref(k), buf, n, C.byref(mode), C.byref(vec))
    if r < 0:
        raise ValueError("kernel generation failed")
    rows = [tuple(buf[7 * i:7 * i + 7]) for i in range(r)]
    return mode.value, vec.value, rows


def window_analyze(k: abi.UOpKernel):
    """(kind, splits) if the backend runs this kernel on its window-max (1) or
    run-sum (2) kernels, else None."""
    kind, S = C.c_uint32(), C.c_uint32()
    if lib().thvm_hip_window_analyze(C.byref(k), C.byref(kind), C.byref(S)):
        return kind.value, S.value
    return None


def window_compile_check(k: abi.UOpKernel):
    err = C.create_string_buffer(512)
    n = lib().thvm_hip_window_compile_check(C.byref(k), err, len(err))
    if n < 0:
        raise RuntimeError(err.value.decode())
    return n


def window_source(k: abi.UOpKernel):
    buf = C.create_string_buffer(1 << 20)
    n = lib().thvm_hip_window_source(C.byref(k), buf, len(buf))
    if n < 0:
        raise ValueError(buf.value.decode())
    return buf.value.decode()
