// static_kernels.hip - precompiled gfx950 kernels loaded once at init:
//   thvm_rs          FusedOp/ReduceSpec interpreter (dispatch_kernel_rs fallback)
//   thvm_contiguify  strided, masked view -> dense copy (2- or 4-byte elements),
//                    as the engine's host read src/ops/_.c:338-357
//   thvm_op_ew / thvm_op_mm / thvm_op_reduce
//                    the legacy per-op slots (src/backend/cpu/ops.c)
//   thvm_copy_batch  several buffer-to-buffer copies in one launch
//   thvm_fill_u32    fill a buffer with a 32-bit pattern (graph-safe clear)
//   thvm_adam        the adam_step slot: one fused pass over parameter,
//                    gradient and both moments
//   thvm_kop         KOp program interpreter: the dispatch_uop_kernel path
//                    for a program hipRTC could not compile; one lane per gid,
//                    the reference interpreter's semantics
//                    (src/backend/cpu/uop.c:29-155)
//
// The rs interpreter restates the engine's CPU fallback
// (src/backend/cpu/dispatch.c:23-282): leaves are read through their view
// (mask and compound masks checked before the read, broadcast by coord %
// dim, negative index reads 0) or through a multi-view ShapeTracker; the
// FusedOp DAG is evaluated with the engine ALU; SUM/RMAX accumulate in the
// output's storage dtype in flat iteration order. Each thread owns one output
// element and walks its reduce sub-domain in the same row-major order as the
// CPU's flat loop, so results are bit-identical, f16 rounding included.
#include <hip/hip_runtime.h>
#include "thvm_abi.h"

#include "kargs.h"

__device__ __forceinline__ float h2f(u32 h) {
    u32 sign = (h & 0x8000u) << 16, ex = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    if (ex == 0u) {
        if (man == 0u) bits = sign;
        else {
            ex = 1u;
            while ((man & 0x400u) == 0u) { man <<= 1; ex -= 1u; }
            man &= 0x3FFu;
            bits = sign | ((ex + 112u) << 23) | (man << 13);
        }
    } else if (ex == 0x1Fu) bits = sign | 0x7F800000u | (man << 13);
    else bits = sign | ((ex + 112u) << 23) | (man << 13);
    return __uint_as_float(bits);
}

__device__ __forceinline__ u32 f2h(float f) {
    u32 x = __float_as_uint(f), sign = (x >> 16) & 0x8000u, man = x & 0x7FFFFFu;
    int ex = (int)((x >> 23) & 0xFFu) - 112;
    if (ex <= 0) {
        if (ex < -10) return sign;
        man = (man | 0x800000u) >> (1 - ex);
        if (man & 0x1000u) man += 0x2000u;
        return sign | (man >> 13);
    }
    if (ex >= 31) return sign | 0x7C00u | (man ? 0x200u : 0u);
    if (man & 0x1000u) {
        man += 0x2000u;
        if (man & 0x800000u) { man = 0u; ex += 1; if (ex >= 31) return sign | 0x7C00u; }
    }
    return sign | ((u32)ex << 10) | (man >> 13);
}

__device__ __forceinline__ u32 f2u(float f) {
    if (!(fabsf(f) < 9.2233720368547758e18f)) return 0u;
    return (u32)(unsigned long long)(long long)f;
}
__device__ __forceinline__ int f2i(float f) {
    if (!(f >= -2147483648.0f && f < 2147483648.0f)) return (int)0x80000000u;
    return (int)f;
}
__device__ __forceinline__ float cast_f(float v, u32 dt) {
    if (dt == DTYPE_F16) return h2f(f2h(v));
    if (dt == DTYPE_I32) return (float)f2i(v);
    if (dt == DTYPE_U32) return (float)f2u(v);
    return v;
}

__device__ __forceinline__ float load_as_f32(const void *p, u32 dt, u32 n, u32 i) {
    if (!p || i >= n) return 0.0f;
    switch (dt) {
    case DTYPE_F16: return h2f(((const unsigned short *)p)[i]);
    case DTYPE_I32: return (float)((const int *)p)[i];
    case DTYPE_U32: return (float)((const u32 *)p)[i];
    default: return ((const float *)p)[i];
    }
}

__device__ __forceinline__ void store_from_f32(void *p, u32 dt, u32 n, u32 i, float v) {
    if (!p || i >= n) return;
    switch (dt) {
    case DTYPE_F16: ((unsigned short *)p)[i] = (unsigned short)f2h(v); break;
    case DTYPE_I32: ((int *)p)[i] = f2i(v); break;
    case DTYPE_U32: ((u32 *)p)[i] = f2u(v); break;
    default: ((float *)p)[i] = v; break;
    }
}

__device__ __forceinline__ float alu(u32 uop, u32 aux, float a, float b) {
    switch (uop) {
    case UOP_ADD: return a + b;
    case UOP_MUL: return a * b;
    case UOP_DIV: return b != 0.0f ? a / b : 0.0f;
    case UOP_SUB: return a - b;
    case UOP_MAX: return a > b ? a : b;
    case UOP_CMP: return a > b ? 1.0f : 0.0f;
    case UOP_NEG: return -a;
    case UOP_RELU: return a > 0.0f ? a : 0.0f;
    case UOP_EXP: return expf(a);
    case UOP_LOG: return logf(a);
    case UOP_SQRT: return sqrtf(a);
    case UOP_CAST: return cast_f(a, aux);
    default: return a;
    }
}

// Read through one view; coords are in the iteration domain.
__device__ float view_read(const void *buf, u32 dt, u32 n, const View *v, const u32 *coords, u32 rank) {
    if (v->has_mask) {
        for (u32 d = 0; d < rank && d < v->shape.rank; d++)
            if (coords[d] < v->mask_begin[d] || coords[d] >= v->mask_end[d]) return 0.0f;
        for (u32 cm = 0; cm < v->n_compound_masks; cm++) {
            u32 da = v->compound_masks[cm].dim_a, db = v->compound_masks[cm].dim_b;
            if (da >= MAX_DIM || db >= MAX_DIM) return 0.0f;
            int composed = (int)coords[da] * v->compound_masks[cm].stride_a + (int)coords[db];
            if (composed < (int)v->compound_masks[cm].begin || composed >= (int)v->compound_masks[cm].end)
                return 0.0f;
        }
    }
    int idx = v->offset;
    for (u32 d = 0; d < rank && d < v->shape.rank; d++) {
        u32 dim = v->shape.dims[d];
        u32 c = dim ? coords[d] % dim : 0u;
        idx = (int)((u32)idx + c * (u32)v->strides[d]);
    }
    if (idx < 0) return 0.0f;
    return load_as_f32(buf, dt, n, (u32)idx);
}

// Read through a stacked ShapeTracker (src/backend/cpu/dispatch.c:26-83).
__device__ float st_read(const void *buf, u32 dt, u32 n, const ShapeTracker *st, const u32 *coords,
                         u32 rank, const u32 *full_dims) {
    if (st->n_views <= 1) return 0.0f;
    u32 si = 0;
    {
        u32 stride = 1;
        for (int d = (int)rank - 1; d >= 0; d--) {
            si += coords[d] * stride;
            stride *= full_dims[d];
        }
    }
    for (int vi = (int)st->n_views - 2; vi >= 0; vi--) {
        const View *vw = &st->views[vi];
        const View *outer = &st->views[vi + 1];
        u32 outer_flat = 0;
        {
            u32 udiv = 1;
            u32 ostr[MAX_DIM];
            u32 orank = outer->shape.rank < MAX_DIM ? outer->shape.rank : MAX_DIM;
            if (orank > 0) {
                ostr[orank - 1] = 1;
                for (int d = (int)orank - 2; d >= 0; d--) ostr[d] = ostr[d + 1] * outer->shape.dims[d + 1];
            }
            for (int d = (int)orank - 1; d >= 0; d--) {
                u32 dim = outer->shape.dims[d];
                if (dim <= 1) { udiv *= dim; continue; }
                u32 c = udiv ? (si / udiv) % dim : 0u;
                outer_flat += c * ostr[d];
                udiv *= dim;
            }
        }
        int idx = vw->offset;
        {
            u32 rem = outer_flat;
            u32 istr[MAX_DIM];
            u32 irank = vw->shape.rank < MAX_DIM ? vw->shape.rank : MAX_DIM;
            if (irank > 0) {
                istr[irank - 1] = 1;
                for (int d = (int)irank - 2; d >= 0; d--) istr[d] = istr[d + 1] * vw->shape.dims[d + 1];
            }
            for (u32 d = 0; d < irank; d++) {
                u32 c = istr[d] ? rem / istr[d] : 0u;
                rem = istr[d] ? rem % istr[d] : rem;
                if (vw->has_mask && (c < vw->mask_begin[d] || c >= vw->mask_end[d])) return 0.0f;
                if (vw->strides[d] != 0) idx = (int)((u32)idx + c * (u32)vw->strides[d]);
            }
        }
        if (idx < 0) return 0.0f;
        si = (u32)idx;
    }
    return load_as_f32(buf, dt, n, si);
}

__device__ float read_leaf(const RsParams *P, u32 i, const u32 *coords, u32 rank, const u32 *full_dims) {
    const void *p = (const void *)(uintptr_t)P->leaf_ptr[i];
    if (P->leaf_st[i] != 0xFFFFFFFFu)
        return st_read(p, P->leaf_dtype[i], P->leaf_n[i], &P->sts[P->leaf_st[i]], coords, rank, full_dims);
    return view_read(p, P->leaf_dtype[i], P->leaf_n[i], &P->views[i], coords, rank);
}

// Evaluates ops [lo, hi) over vals; returns 0 if an arg is out of range
// (the CPU stops evaluating at that op).
__device__ void eval_ops(const RsParams *P, float *vals, u32 lo, u32 hi, u32 limit) {
    for (u32 i = lo; i < hi; i++) {
        u32 aa = P->ops[i].arg_a, bb = P->ops[i].arg_b;
        if (aa >= limit || bb >= limit) break;
        vals[P->n_leaves + i] = alu(P->ops[i].uop, P->ops[i].aux, vals[aa], vals[bb]);
    }
}

extern "C" __global__ __launch_bounds__(64) void thvm_rs(const RsParams *P, u32 phase) {
    const u32 t = blockIdx.x * 64u + threadIdx.x;
    const u32 rank = P->rank;
    float vals[FUSE_MAX_LEAVES + FUSE_MAX_OPS];
    u32 coords[MAX_DIM];
    u32 n_ops = P->n_ops, n_leaves = P->n_leaves;
    void *out = (void *)(uintptr_t)P->out_ptr;
    if (phase == 0) {
        if (!P->has_reduce) {
            if (t >= P->full_numel) return;
            u32 rem = t;
            for (int d = (int)rank - 1; d >= 0; d--) {
                coords[d] = P->dims[d] ? rem % P->dims[d] : 0u;
                rem = P->dims[d] ? rem / P->dims[d] : 0u;
            }
            for (u32 i = 0; i < n_leaves; i++) vals[i] = read_leaf(P, i, coords, rank, P->dims);
            eval_ops(P, vals, 0, n_ops, n_leaves + n_ops);
            float result = n_ops > 0 ? vals[n_leaves + n_ops - 1] : vals[0];
            store_from_f32(out, P->out_dtype, P->out_n, t, result);
            return;
        }
        if (t >= P->out_numel) return;
        // output coords from t over out_shape
        u32 rem = t;
        for (int d = (int)rank - 1; d >= 0; d--) {
            u32 od = P->out_shape[d];
            coords[d] = od ? rem % od : 0u;
            rem = od ? rem / od : 0u;
        }
        u32 eval_n = P->post_start ? P->post_start : n_ops;
        float acc = cast_f(P->reduce_type == UOP_RMAX ? -1e30f : 0.0f, P->out_dtype);
        for (u32 r = 0; r < P->reduce_numel; r++) {
            u32 rr = r;
            for (int d = (int)rank - 1; d >= 0; d--) {
                if (!P->is_reduce[d]) continue;
                coords[d] = P->dims[d] ? rr % P->dims[d] : 0u;
                rr = P->dims[d] ? rr / P->dims[d] : 0u;
            }
            for (u32 i = 0; i < n_leaves; i++) vals[i] = read_leaf(P, i, coords, rank, P->dims);
            eval_ops(P, vals, 0, eval_n, n_leaves + eval_n);
            float result = eval_n > 0 ? vals[n_leaves + eval_n - 1] : vals[0];
            if (P->reduce_type == UOP_SUM) acc = cast_f(acc + result, P->out_dtype);
            else if (P->reduce_type == UOP_RMAX) acc = cast_f(result > acc ? result : acc, P->out_dtype);
        }
        store_from_f32(out, P->out_dtype, P->out_n, t, acc);
        return;
    }
    // phase 1: post-reduce ops over the reduced output
    if (t >= P->out_numel) return;
    u32 rem = t;
    for (int d = (int)rank - 1; d >= 0; d--) {
        u32 od = P->out_shape[d];
        coords[d] = od ? rem % od : 0u;
        rem = od ? rem / od : 0u;
    }
    float reduce_result = load_as_f32(out, P->out_dtype, P->out_n, t);
    u32 n_pre = n_leaves - P->n_post_leaves;
    u32 zero_dims[MAX_DIM] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (u32 i = 0; i < n_leaves; i++)
        vals[i] = i < n_pre ? 0.0f : read_leaf(P, i, coords, rank, zero_dims);
    u32 ps = P->post_start;
    const u32 LIM = FUSE_MAX_LEAVES + FUSE_MAX_OPS;
    if (ps > 0 && n_leaves + ps - 1 < LIM) vals[n_leaves + ps - 1] = reduce_result;
    for (u32 i = ps; i < n_ops; i++) {
        u32 aa = P->ops[i].arg_a, bb = P->ops[i].arg_b;
        float a = aa < LIM ? vals[aa] : 0.0f, b = bb < LIM ? vals[bb] : 0.0f;
        vals[n_leaves + i] = alu(P->ops[i].uop, P->ops[i].aux, a, b);
    }
    store_from_f32(out, P->out_dtype, P->out_n, t, vals[n_leaves + n_ops - 1]);
}

// Dense copy of a strided, masked view of 4-byte elements.
extern "C" __global__ __launch_bounds__(256) void thvm_contiguify(ContigArgs A) {
    const u32 t = blockIdx.x * 256u + threadIdx.x;
    const View &v = A.v;
    if (t >= A.numel || t >= A.dst_n) return;
    u32 rem = t;
    int idx = v.offset;
    int masked = 0;
    for (int d = (int)v.shape.rank - 1; d >= 0; d--) {
        const u32 dim = v.shape.dims[d];
        const u32 c = dim ? rem % dim : 0u;
        rem = dim ? rem / dim : 0u;
        if (v.has_mask && (c < v.mask_begin[d] || c >= v.mask_end[d])) masked = 1;
        idx += (int)c * (v.strides[d] > 0 ? v.strides[d] : 0);
    }
    const int ok = !masked && idx >= 0 && (u32)idx < A.src_n;
    if (A.esize == 2u) {
        const unsigned short *src = (const unsigned short *)(uintptr_t)A.src;
        ((unsigned short *)(uintptr_t)A.dst)[t] = ok ? src[(u32)idx] : (unsigned short)0;
    } else {
        const u32 *src = (const u32 *)(uintptr_t)A.src;
        ((u32 *)(uintptr_t)A.dst)[t] = ok ? src[(u32)idx] : 0u;
    }
}

// ---- legacy per-op slots (src/backend/cpu/ops.c) ----
// One lane per output, each in the CPU's order of operations, so results are
// bit-identical (EXP/LOG aside). Index arithmetic is strided_index
// (src/backend/cpu/ops.c:3-13): u32, no masks; loads out of range read 0.
__device__ __forceinline__ u32 strided_index(u32 flat, const View &v) {
    u32 idx = (u32)v.offset, rem = flat;
    for (int d = (int)v.shape.rank - 1; d >= 0; d--) {
        const u32 dim = v.shape.dims[d];
        const u32 c = dim ? rem % dim : 0u;
        rem = dim ? rem / dim : 0u;
        idx += c * (u32)v.strides[d];
    }
    return idx;
}

extern "C" __global__ __launch_bounds__(256) void thvm_op_ew(LegacyArgs A) {
    const u32 t = blockIdx.x * 256u + threadIdx.x;
    if (t >= A.n) return;
    const float va = load_as_f32((const void *)(uintptr_t)A.a, A.ad, A.a_n, strided_index(t, A.av));
    float vr = va;
    if (A.binary) {
        const float vb = load_as_f32((const void *)(uintptr_t)A.b, A.bd, A.b_n, strided_index(t, A.bv));
        switch (A.uop) {
        case UOP_ADD: vr = va + vb; break;
        case UOP_MUL: vr = va * vb; break;
        case UOP_DIV: vr = vb != 0.0f ? va / vb : 0.0f; break;
        case UOP_SUB: vr = va - vb; break;
        case UOP_MAX: vr = va > vb ? va : vb; break;
        case UOP_CMP: vr = va > vb ? 1.0f : 0.0f; break;
        default: break;
        }
    } else {
        switch (A.uop) {
        case UOP_NEG: vr = -va; break;
        case UOP_RELU: vr = va > 0.0f ? va : 0.0f; break;
        case UOP_EXP: vr = expf(va); break;
        case UOP_LOG: vr = logf(va); break;
        case UOP_SQRT: vr = sqrtf(va); break;
        default: break;
        }
    }
    store_from_f32((void *)(uintptr_t)A.dst, A.dd, A.dst_n, t, vr);
}

// C[i][j] = sum_k A[i*K+k] * B[k*N+j] through the operand views, k in order
// (src/backend/cpu/ops.c:80-113, the path without BLAS).
extern "C" __global__ __launch_bounds__(256) void thvm_op_mm(LegacyArgs A) {
    const u32 t = blockIdx.x * 256u + threadIdx.x;
    if (t >= A.n) return;
    const u32 i = t / A.N, j = t % A.N;
    const void *pa = (const void *)(uintptr_t)A.a, *pb = (const void *)(uintptr_t)A.b;
    float acc = 0.0f;
    for (u32 k = 0; k < A.K; k++) {
        const float va = load_as_f32(pa, A.ad, A.a_n, strided_index(i * A.K + k, A.av));
        const float vb = load_as_f32(pb, A.bd, A.b_n, strided_index(k * A.N + j, A.bv));
        acc = acc + va * vb;
    }
    store_from_f32((void *)(uintptr_t)A.dst, A.dd, A.dst_n, i * A.N + j, acc);
}

// out[o] = SUM / RMAX of src[o*R .. o*R+R) in order (src/backend/cpu/ops.c:115-130); R = A.K.
extern "C" __global__ __launch_bounds__(256) void thvm_op_reduce(LegacyArgs A) {
    const u32 o = blockIdx.x * 256u + threadIdx.x;
    if (o >= A.n) return;
    const void *ps = (const void *)(uintptr_t)A.a;
    float acc = A.uop == UOP_RMAX ? -1e30f : 0.0f;
    for (u32 r = 0; r < A.K; r++) {
        const float v = load_as_f32(ps, A.ad, A.a_n, o * A.K + r);
        if (A.uop == UOP_SUM) acc = acc + v;
        else if (A.uop == UOP_RMAX) acc = v > acc ? v : acc;
    }
    store_from_f32((void *)(uintptr_t)A.dst, A.dd, A.dst_n, o, acc);
}

// Batched device copies (ASSIGN's buf_copy): blockIdx.y picks the copy; the
// blocks of a row stride over it in 16-byte words, then the byte tail.
extern "C" __global__ __launch_bounds__(256) void thvm_copy_batch(CopyBatch B) {
    const u32 c = blockIdx.y;
    if (c >= B.n) return;
    char *d = (char *)(uintptr_t)B.dst[c];
    const char *s = (const char *)(uintptr_t)B.src[c];
    const unsigned long long nb = B.bytes[c], n16 = nb / 16u;
    const unsigned long long t0 = (unsigned long long)blockIdx.x * 256u + threadIdx.x;
    const unsigned long long step = (unsigned long long)gridDim.x * 256u;
    if (((uintptr_t)d % 16u) == 0u && ((uintptr_t)s % 16u) == 0u) {
        for (unsigned long long i = t0; i < n16; i += step) ((uint4 *)d)[i] = ((const uint4 *)s)[i];
        for (unsigned long long i = n16 * 16u + t0; i < nb; i += step) d[i] = s[i];
    } else {
        for (unsigned long long i = t0; i < nb; i += step) d[i] = s[i];
    }
}

extern "C" __global__ __launch_bounds__(256) void thvm_fill_u32(u32 *dst, u32 n, u32 value) {
    const u32 t = blockIdx.x * 256u + threadIdx.x;
    if (t < n) dst[t] = value;
}

// adam_step with the arithmetic of the engine's lazy update, the CPU
// backend's result (src/nn/adam.c:75-88): each product, quotient and sum is
// one f32 rounding in the composition's order (no contraction: the file is
// built with -ffp-contract=off), DIV guarded as the engine's ALU guards it.
// One pass: reads p, g, m, v and writes p, m, v (28 bytes per element);
// each lane owns 4 consecutive elements, with 128-bit accesses when aligned.
__device__ __forceinline__ float adam_div(float a, float b) { return b != 0.0f ? a / b : 0.0f; }

__device__ __forceinline__ void adam_one(const AdamArgs &a, float &p, float g, float &m, float &v) {
    const float mi = a.beta1 * m + (1.0f - a.beta1) * g;
    const float vi = a.beta2 * v + (1.0f - a.beta2) * (g * g);
    const float m_hat = adam_div(mi, a.bc1);
    const float v_hat = adam_div(vi, a.bc2);
    const float denom = sqrtf(v_hat) + a.eps;
    const float step = a.lr * adam_div(m_hat, denom);
    m = mi;
    v = vi;
    p = p - step;
}

extern "C" __global__ __launch_bounds__(256) void thvm_adam(AdamArgs a) {
    float *P = (float *)(uintptr_t)a.p, *M = (float *)(uintptr_t)a.m, *V = (float *)(uintptr_t)a.v;
    const float *G = (const float *)(uintptr_t)a.g;
    const unsigned long long i0 = ((unsigned long long)blockIdx.x * 256u + threadIdx.x) * 4u;
    if (i0 >= a.n) return;
    if (a.vec && i0 + 4u <= a.n) {
        float4 p = *(float4 *)(P + i0), m = *(float4 *)(M + i0), v = *(float4 *)(V + i0);
        const float4 g = *(const float4 *)(G + i0);
        adam_one(a, p.x, g.x, m.x, v.x);
        adam_one(a, p.y, g.y, m.y, v.y);
        adam_one(a, p.z, g.z, m.z, v.z);
        adam_one(a, p.w, g.w, m.w, v.w);
        *(float4 *)(P + i0) = p;
        *(float4 *)(M + i0) = m;
        *(float4 *)(V + i0) = v;
        return;
    }
    for (unsigned long long i = i0; i < i0 + 4u && i < a.n; i++) {
        float p = P[i], m = M[i], v = V[i];
        adam_one(a, p, G[i], m, v);
        P[i] = p;
        M[i] = m;
        V[i] = v;
    }
}

// KOp interpreter (src/backend/cpu/uop.c:29-155): lane = one gid of the
// launch, running the whole program with its reduce loops in order, so
// results are those of the engine's CPU backend (libm EXP/LOG aside). Like
// the reference, each op has an unsigned slot and a float slot, zeroed per
// gid; ftype says which one an op's value lives in. Loops: RANGE sets its
// counter to 0 (a loop of trip 0 jumps past its ENDRANGE and leaves the
// counter as it was); ENDRANGE steps the counter of its RANGE and jumps back
// while it is below the trip, so after the loop the counter holds trip - 1,
// as the reference's leaves it. The host checks that loops nest.
__device__ __forceinline__ u32 kop_u(const KopParams *P, const u32 *uv, const float *fv, u32 id) {
    if (id >= P->n_ops) return 0u;
    return P->ftype[id] ? f2u(fv[id]) : uv[id];
}
__device__ __forceinline__ float kop_f(const KopParams *P, const u32 *uv, const float *fv, u32 id) {
    if (id >= P->n_ops) return 0.0f;
    return P->ftype[id] ? fv[id] : (float)uv[id];
}

extern "C" __global__ __launch_bounds__(64) void thvm_kop(const KopParams *P, u32 base) {
    const u32 gid = base + blockIdx.x * 64u + threadIdx.x;
    if (gid >= P->total || gid < base) return;
    u32 uv[KOP_MAX];
    float fv[KOP_MAX];
    const u32 n = P->n_ops;
    for (u32 i = 0; i < n; i++) {
        uv[i] = 0u;
        fv[i] = 0.0f;
    }
#define KU(id) kop_u(P, uv, fv, (id))
#define KF(id) kop_f(P, uv, fv, (id))
    u32 i = 0;
    while (i < n) {
        const KOp op = P->ops[i];
        switch (op.type) {
        case KOP_GID: uv[i] = gid; break;
        case KOP_CONST_U: uv[i] = op.imm.u; break;
        case KOP_CONST_F: fv[i] = op.imm.f; break;
        case KOP_MOD: uv[i] = op.imm.u ? KU(op.arg[0]) % op.imm.u : 0u; break;
        case KOP_DIV: uv[i] = op.imm.u ? KU(op.arg[0]) / op.imm.u : 0u; break;
        case KOP_IDX: uv[i] = KU(op.arg[0]) * op.imm.u + KU(op.arg[1]); break;
        case KOP_LOAD: {
            const u32 bi = op.imm.u, idx = KU(op.arg[0]);
            float x = 0.0f;
            if (bi == 0u) x = load_as_f32((const void *)P->out_ptr, P->out_dtype, P->out_n, idx);
            else if (bi - 1u < P->n_leaves)
                x = load_as_f32((const void *)P->leaf_ptr[bi - 1u], P->leaf_dtype[bi - 1u], P->leaf_n[bi - 1u], idx);
            fv[i] = x;
            break;
        }
        case KOP_MASK: fv[i] = KF(op.arg[0]) != 0.0f ? KF(op.arg[1]) : 0.0f; break;
        case KOP_ALU: fv[i] = alu(op.imm.u, op.arg[2], KF(op.arg[0]), KF(op.arg[1])); break;
        case KOP_ACC_INIT: fv[i] = op.imm.f; break;
        case KOP_ACC: {
            const u32 a = op.arg[0];
            if (a >= n) break;
            const float x = KF(op.arg[1]);
            fv[a] = op.imm.u == UOP_RMAX ? (fv[a] > x ? fv[a] : x) : fv[a] + x;
            break;
        }
        case KOP_RANGE:
            if (op.imm.u == 0u) {
                i = (u32)P->pair[i] + 1u;
                continue;
            }
            uv[i] = 0u;
            break;
        case KOP_ENDRANGE: {
            const u32 s = P->pair[i];
            const u32 r = uv[s] + 1u;
            if (r < P->ops[s].imm.u) {
                uv[s] = r;
                i = s + 1u;
                continue;
            }
            break;
        }
        case KOP_STORE:
            store_from_f32((void *)P->out_ptr, P->out_dtype, P->out_n, KU(op.arg[0]), KF(op.arg[1]));
            break;
        default: break;
        }
        i++;
    }
#undef KU
#undef KF
}
