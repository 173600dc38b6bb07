// ggml_backend.hip -- the op hooks of ane's ggml backend (reference
// src/ggml-backend/ggml-ane.cpp:109-277, 287-299, 363-393): GGML_OP_MUL_MAT
// on the Q8_0 kernels of q8_0.hip and the Q4_0 GEMV of qformats.hip; ADD,
// MUL, SCALE and CPY/CONT/DUP as fp32 row kernels here; RMS_NORM, SOFT_MAX,
// ROPE and SILU in the reference handlers' arithmetic (decode_ref.hip).
// Each op is claimed only where this file computes ggml's semantics for it
// (include/ggml-ane-hip.h lists the conditions).
//
// MUL_MAT:
// dst[i3][i2][i1][i0] = sum_k src0[i3/r3][i2/r2][i0][k] * src1[i3][i2][i1][k]
// with r2 = ne12/ne02, r3 = ne13/ne03 (ggml's broadcast of the weights over
// the activation batches).  Every token row i1 < ne11 is computed.
//
// Launch plan per node:
//  * weights shared by all batches (ne02 == ne03 == 1) and activation/output
//    rows uniformly strided across batches -> one call over all rows;
//  * otherwise one call per (i2, i3) batch.
// Activation rows whose stride is not K floats are gathered into the
// backend's workspace first; output rows whose stride is not N floats are
// computed there and scattered.
#include <hip/hip_runtime.h>

#include <cstring>

#include "../../include/ane_decode.h"
#include "../../include/ggml-ane-hip.h"
#include "common.hpp"
#include "ggml_rows.hpp"

struct ane_ggml_backend {
    hipStream_t stream;
    int q8_mode;
    void* ws;
    size_t wsb;
};

namespace ane {
namespace {

// rows x cols fp32, source rows `stride` bytes apart -> contiguous dst.
__global__ void __launch_bounds__(256)
k_gather_rows(const uint8_t* __restrict__ src, uint64_t stride, uint32_t rows, uint32_t cols,
              float* __restrict__ dst) {
    const uint64_t n = (uint64_t)rows * cols;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256) {
        const uint64_t r = i / cols, c = i - r * cols;
        dst[i] = reinterpret_cast<const float*>(src + r * stride)[c];
    }
}

__global__ void __launch_bounds__(256)
k_scatter_rows(const float* __restrict__ src, uint32_t rows, uint32_t cols, uint8_t* __restrict__ dst,
               uint64_t stride) {
    const uint64_t n = (uint64_t)rows * cols;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256) {
        const uint64_t r = i / cols, c = i - r * cols;
        reinterpret_cast<float*>(dst + r * stride)[c] = src[i];
    }
}

uint32_t grid_for(uint64_t n) {
    uint64_t g = (n + 255) / 256;
    if (g > 65536) g = 65536;
    return (uint32_t)(g ? g : 1);
}

const ane_ggml_tensor* src_of(const ane_ggml_tensor* t, int i) { return t ? t->src[i] : nullptr; }

bool mul_mat_supported(const ane_ggml_tensor* d) {
    const ane_ggml_tensor* a = src_of(d, 0);
    const ane_ggml_tensor* b = src_of(d, 1);
    if (!a || !b || d->type != ANE_GGML_TYPE_F32 ||
        (a->type != ANE_GGML_TYPE_Q8_0 && a->type != ANE_GGML_TYPE_Q4_0) || b->type != ANE_GGML_TYPE_F32)
        return false;
    const size_t bb = a->type == ANE_GGML_TYPE_Q8_0 ? 34 : 18;  // bytes per 32-weight block
    for (int i = 0; i < 4; i++)
        if (d->ne[i] < 0 || a->ne[i] < 0 || b->ne[i] < 0) return false;
    const int64_t K = a->ne[0];
    if (K % 32 != 0 || b->ne[0] != K || d->ne[0] != a->ne[1] || d->ne[1] != b->ne[1] ||
        d->ne[2] != b->ne[2] || d->ne[3] != b->ne[3])
        return false;
    if (a->ne[2] == 0 || a->ne[3] == 0 || b->ne[2] % a->ne[2] != 0 || b->ne[3] % a->ne[3] != 0)
        return false;
    // innermost strides: one block / one float; weight rows packed
    if (a->nb[0] != bb || a->nb[1] != (size_t)(K / 32) * bb || b->nb[0] != 4 || d->nb[0] != 4)
        return false;
    if (d->ne[0] > 0xffffffffLL || K > 0xffffffffLL) return false;
    return true;
}

bool ensure_ws(ane_ggml_backend* be, size_t bytes) {
    if (bytes <= be->wsb) return true;
    if (be->ws) {
        if (hipStreamSynchronize(be->stream) != hipSuccess) return false;
        (void)hipFree(be->ws);
        be->ws = nullptr;
        be->wsb = 0;
    }
    size_t sz = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
    if (hipMalloc(&be->ws, sz) != hipSuccess) {
        be->ws = nullptr;
        return false;
    }
    be->wsb = sz;
    return true;
}

// One weight matrix over T rows: x rows `xs` bytes apart, y rows `ys` bytes
// apart.  Q8_0 in the backend's mode; Q4_0 with the reference's q4_0_gemv
// arithmetic (its only one) for every row.
int mul_mat_rows(ane_ggml_backend* be, int type, uint32_t N, uint32_t K, uint32_t T, const void* W,
                 const uint8_t* x, uint64_t xs, uint8_t* y, uint64_t ys) {
    if (T == 0 || N == 0) return ANE_OK;
    const bool xc = xs == (uint64_t)K * 4, yc = ys == (uint64_t)N * 4;
    const bool g = type == ANE_GGML_TYPE_Q8_0 && be->q8_mode == ANE_GGML_Q8_G;
    const size_t qws = g ? ane_hip_q8_0_mul_mat_workspace_size_n(N, K, T) : 0;
    const size_t xoff = ceil_to(qws, 256);
    const size_t xbytes = xc ? 0 : ceil_to((uint64_t)T * K * 4, 256);
    const size_t yoff = xoff + xbytes;
    const size_t ybytes = yc ? 0 : ceil_to((uint64_t)T * N * 4, 256);
    if (!ensure_ws(be, yoff + ybytes + 256)) return ANE_ERR_HIP;
    uint8_t* ws = static_cast<uint8_t*>(be->ws);
    const float* xp = reinterpret_cast<const float*>(x);
    if (!xc) {
        float* xg = reinterpret_cast<float*>(ws + xoff);
        hipLaunchKernelGGL(k_gather_rows, dim3(grid_for((uint64_t)T * K)), dim3(256), 0, be->stream, x, xs,
                           T, K, xg);
        xp = xg;
    }
    float* yp = yc ? reinterpret_cast<float*>(y) : reinterpret_cast<float*>(ws + yoff);
    int st = ANE_OK;
    if (g) {
        st = ane_hip_q8_0_mul_mat(N, K, T, xp, W, yp, ws, qws, be->stream);
    } else {
        const auto gemv = type == ANE_GGML_TYPE_Q8_0 ? ane_hip_q8_0_gemv : ane_hip_q4_0_gemv;
        for (uint32_t t = 0; t < T && st == ANE_OK; t++)
            st = gemv(N, K, xp + (uint64_t)t * K, W, yp + (uint64_t)t * N, be->stream);
    }
    if (st != ANE_OK) return st;
    if (!yc) {
        hipLaunchKernelGGL(k_scatter_rows, dim3(grid_for((uint64_t)T * N)), dim3(256), 0, be->stream, yp, T,
                           N, y, ys);
    }
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

int mul_mat(ane_ggml_backend* be, const ane_ggml_tensor* d) {
    const ane_ggml_tensor* a = d->src[0];
    const ane_ggml_tensor* b = d->src[1];
    const uint32_t K = (uint32_t)a->ne[0], N = (uint32_t)a->ne[1];
    const int64_t T = b->ne[1], B2 = b->ne[2], B3 = b->ne[3];
    if (T == 0 || B2 == 0 || B3 == 0 || N == 0) return ANE_OK;
    if (!a->data || !b->data || !d->data) return ANE_ERR_BAD_POINTER;
    const int64_t r2 = B2 / a->ne[2], r3 = B3 / a->ne[3];
    const uint8_t* x0 = static_cast<const uint8_t*>(b->data);
    uint8_t* y0 = static_cast<uint8_t*>(d->data);
    // all (i1, i2, i3) rows as one uniform sequence?
    const bool w_shared = a->ne[2] == 1 && a->ne[3] == 1;
    const bool x_uniform = (B2 == 1 || b->nb[2] == (size_t)T * b->nb[1]) &&
                           (B3 == 1 || b->nb[3] == (size_t)(T * B2) * b->nb[1]);
    const bool y_uniform = (B2 == 1 || d->nb[2] == (size_t)T * d->nb[1]) &&
                           (B3 == 1 || d->nb[3] == (size_t)(T * B2) * d->nb[1]);
    const int64_t rows = T * B2 * B3;
    if (w_shared && x_uniform && y_uniform && rows <= 0xffffffffLL)
        return mul_mat_rows(be, a->type, N, K, (uint32_t)rows, a->data, x0, b->nb[1], y0, d->nb[1]);
    if (T > 0xffffffffLL) return ANE_ERR_INVALID_ARG;
    for (int64_t i3 = 0; i3 < B3; i3++) {
        for (int64_t i2 = 0; i2 < B2; i2++) {
            const uint8_t* W = static_cast<const uint8_t*>(a->data) + (i2 / r2) * a->nb[2] + (i3 / r3) * a->nb[3];
            const int st = mul_mat_rows(be, a->type, N, K, (uint32_t)T, W, x0 + i2 * b->nb[2] + i3 * b->nb[3],
                                        b->nb[1], y0 + i2 * d->nb[2] + i3 * d->nb[3], d->nb[1]);
            if (st != ANE_OK) return st;
        }
    }
    return ANE_OK;
}

bool is_empty(const ane_ggml_tensor* t) {
    for (int i = 0; i < 4; i++)
        if (t->ne[i] == 0) return true;
    return false;
}

// ------------------------------------------------------------ fp32 nodes
float param_f32(const ane_ggml_tensor* t, int i) {
    float f;
    std::memcpy(&f, &t->op_params[i], 4);
    return f;
}

// F32, no negative extent, strides whole floats; unit innermost stride
// unless `any_inner`.
bool f32_layout(const ane_ggml_tensor* t, bool any_inner = false) {
    if (!t || t->type != ANE_GGML_TYPE_F32) return false;
    for (int i = 0; i < 4; i++)
        if (t->ne[i] < 0 || t->nb[i] % 4 != 0) return false;
    return any_inner || t->nb[0] == 4;
}

bool same_shape(const ane_ggml_tensor* a, const ane_ggml_tensor* b) {
    for (int i = 0; i < 4; i++)
        if (a->ne[i] != b->ne[i]) return false;
    return true;
}

// b repeats over d as ggml broadcasts (each extent of b divides d's).
bool repeats_over(const ane_ggml_tensor* b, const ane_ggml_tensor* d) {
    for (int i = 0; i < 4; i++) {
        if (b->ne[i] == 0) return d->ne[i] == 0;
        if (d->ne[i] % b->ne[i] != 0) return false;
    }
    return true;
}

// ggml_is_contiguous: dimensions of extent 1 place no condition.
bool contiguous(const ane_ggml_tensor* t) {
    uint64_t want = 4;
    for (int i = 0; i < 4; i++) {
        if (t->ne[i] != 1 && t->nb[i] != want) return false;
        want *= (uint64_t)t->ne[i];
    }
    return true;
}

uint64_t n_elements(const ane_ggml_tensor* t) {
    return (uint64_t)t->ne[0] * (uint64_t)t->ne[1] * (uint64_t)t->ne[2] * (uint64_t)t->ne[3];
}

uint64_t n_rows(const ane_ggml_tensor* t) { return (uint64_t)t->ne[1] * (uint64_t)t->ne[2] * (uint64_t)t->ne[3]; }

NodeRows rows_of(const ane_ggml_tensor* t) {
    return NodeRows{(uint64_t)t->ne[1], (uint64_t)t->ne[2], (uint64_t)t->ne[3], t->nb[1], t->nb[2], t->nb[3]};
}

bool aligned4(const void* p) { return ((uintptr_t)p & 3) == 0; }

bool binary_supported(const ane_ggml_tensor* d) {
    const ane_ggml_tensor* a = src_of(d, 0);
    const ane_ggml_tensor* b = src_of(d, 1);
    return f32_layout(d) && f32_layout(a) && f32_layout(b) && same_shape(a, d) && repeats_over(b, d);
}

bool scale_supported(const ane_ggml_tensor* d) {
    const ane_ggml_tensor* a = src_of(d, 0);
    return f32_layout(d) && f32_layout(a) && same_shape(a, d) && param_f32(d, 1) == 0.0f;
}

bool rms_norm_supported(const ane_ggml_tensor* d) {
    const ane_ggml_tensor* a = src_of(d, 0);
    return f32_layout(d) && f32_layout(a) && same_shape(a, d) && d->ne[0] % 16 == 0 && d->ne[0] <= 0x7fffffffLL;
}

bool soft_max_supported(const ane_ggml_tensor* d) {
    const ane_ggml_tensor* a = src_of(d, 0);
    const ane_ggml_tensor* m = src_of(d, 1);
    if (!f32_layout(d) || !f32_layout(a) || !same_shape(a, d) || d->ne[0] > 0x7fffffffLL) return false;
    if (param_f32(d, 1) != 0.0f || src_of(d, 2)) return false;  // ALiBi max_bias, attention sinks
    if (!m) return true;
    if (!f32_layout(m) || m->ne[0] != d->ne[0] || m->ne[1] < d->ne[1]) return false;
    return m->ne[2] > 0 && m->ne[3] > 0 && d->ne[2] % m->ne[2] == 0 && d->ne[3] % m->ne[3] == 0;
}

bool silu_supported(const ane_ggml_tensor* d) {
    const ane_ggml_tensor* a = src_of(d, 0);
    return f32_layout(d) && f32_layout(a) && same_shape(a, d) && contiguous(a) && contiguous(d);
}

bool rope_supported(const ane_ggml_tensor* d) {
    const ane_ggml_tensor* a = src_of(d, 0);
    const ane_ggml_tensor* p = src_of(d, 1);
    if (!f32_layout(d) || !f32_layout(a) || !same_shape(a, d) || !p || src_of(d, 2)) return false;
    if (p->type != ANE_GGML_TYPE_I32 || p->nb[0] != 4 || p->ne[0] != d->ne[2] || p->ne[1] != 1 ||
        p->ne[2] != 1 || p->ne[3] != 1)
        return false;
    const int64_t n_dims = d->op_params[1], mode = d->op_params[2];
    return n_dims == d->ne[0] && n_dims % 2 == 0 && n_dims > 0 && n_dims <= 0x7fffffffLL && mode == 0 &&
           param_f32(d, 6) == 1.0f && param_f32(d, 7) == 0.0f && param_f32(d, 8) == 1.0f;
}

bool cpy_supported(const ane_ggml_tensor* d) {
    const ane_ggml_tensor* a = src_of(d, 0);
    return f32_layout(d, true) && f32_layout(a, true) && n_elements(a) == n_elements(d);
}

// dst = src0 (op) src1 per element over rows of ne0; src1 repeated over
// dst (its row from row_offset, its element i % bne0).  OP: 0 add, 1 mul,
// 2 scale by s, 3 copy.  Grid: x over ne0, y grid-stride over rows.
template <int OP>
__global__ void __launch_bounds__(256)
k_rows_ew(uint64_t ne0, uint64_t rows, NodeRows d, NodeRows a, NodeRows b, uint64_t bne0, uint8_t* dst,
          const uint8_t* src0, const uint8_t* src1, float s) {
    for (uint64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const RowIdx i = row_index(d, r);
        float* o = reinterpret_cast<float*>(dst + row_offset(d, i));
        const float* x = reinterpret_cast<const float*>(src0 + row_offset(a, i));
        const float* y = OP < 2 ? reinterpret_cast<const float*>(src1 + row_offset(b, i)) : nullptr;
        for (uint64_t e = (uint64_t)blockIdx.x * 256 + threadIdx.x; e < ne0; e += (uint64_t)gridDim.x * 256) {
            float v = x[e];
            if (OP == 0) v = __fadd_rn(v, y[bne0 == ne0 ? e : e % bne0]);
            if (OP == 1) v = __fmul_rn(v, y[bne0 == ne0 ? e : e % bne0]);
            if (OP == 2) v = __fmul_rn(v, s);
            o[e] = v;
        }
    }
}

struct Shape4 {
    uint64_t ne[4];
    uint64_t nb[4];
};

Shape4 shape_of(const ane_ggml_tensor* t) {
    Shape4 s;
    for (int i = 0; i < 4; i++) {
        s.ne[i] = (uint64_t)t->ne[i];
        s.nb[i] = t->nb[i];
    }
    return s;
}

__device__ __forceinline__ uint64_t offset_of(const Shape4& s, uint64_t n) {
    uint64_t off = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint64_t q = n / s.ne[k];
        off += (n - q * s.ne[k]) * s.nb[k];
        n = q;
    }
    return off;
}

// Element n of src (row-major over its shape) to element n of dst, any
// strides: ggml's dup of tensors with equal element counts.
__global__ void __launch_bounds__(256)
k_copy_any(uint64_t n, Shape4 sd, uint8_t* dst, Shape4 ss, const uint8_t* src) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256)
        *reinterpret_cast<float*>(dst + offset_of(sd, i)) = *reinterpret_cast<const float*>(src + offset_of(ss, i));
}

template <int OP>
int rows_ew(ane_ggml_backend* be, const ane_ggml_tensor* d, const ane_ggml_tensor* a, const ane_ggml_tensor* b,
            float s) {
    const uint64_t ne0 = (uint64_t)d->ne[0], rows = n_rows(d);
    uint64_t gx = (ne0 + 255) / 256;
    if (gx > 64) gx = 64;
    const uint64_t gy = rows < 65535 ? rows : 65535;
    const NodeRows bd = b ? rows_of(b) : rows_of(a);
    hipLaunchKernelGGL(k_rows_ew<OP>, dim3((uint32_t)gx, (uint32_t)gy), dim3(256), 0, be->stream, ne0, rows,
                       rows_of(d), rows_of(a), bd, b ? (uint64_t)b->ne[0] : ne0, static_cast<uint8_t*>(d->data),
                       static_cast<const uint8_t*>(a->data), b ? static_cast<const uint8_t*>(b->data) : nullptr, s);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

bool data_ok(const ane_ggml_tensor* t) { return t && t->data && aligned4(t->data); }

int fp32_node(ane_ggml_backend* be, const ane_ggml_tensor* d) {
    const ane_ggml_tensor* a = d->src[0];
    const ane_ggml_tensor* b = d->src[1];
    if (!data_ok(d) || !data_ok(a)) return ANE_ERR_BAD_POINTER;
    const hipStream_t s = be->stream;
    switch (d->op) {
        case ANE_GGML_OP_ADD:
        case ANE_GGML_OP_MUL:
            if (!data_ok(b)) return ANE_ERR_BAD_POINTER;
            return d->op == ANE_GGML_OP_ADD ? rows_ew<0>(be, d, a, b, 0.0f) : rows_ew<1>(be, d, a, b, 0.0f);
        case ANE_GGML_OP_SCALE:
            return rows_ew<2>(be, d, a, nullptr, param_f32(d, 0));
        case ANE_GGML_OP_RMS_NORM:
            return rms_norm_node_launch((uint32_t)d->ne[0], n_rows(d), param_f32(d, 0),
                                        static_cast<const uint8_t*>(a->data), rows_of(a),
                                        static_cast<uint8_t*>(d->data), rows_of(d), s);
        case ANE_GGML_OP_SOFT_MAX: {
            if (b && !data_ok(b)) return ANE_ERR_BAD_POINTER;
            const NodeRows none{1, 1, 1, 0, 0, 0};
            return softmax_node_launch((uint32_t)d->ne[0], n_rows(d), param_f32(d, 0),
                                       static_cast<const uint8_t*>(a->data), rows_of(a),
                                       b ? static_cast<const uint8_t*>(b->data) : nullptr, b ? rows_of(b) : none,
                                       static_cast<uint8_t*>(d->data), rows_of(d), s);
        }
        case ANE_GGML_OP_SILU:
            return ane_hip_silu_fp32(n_elements(d), static_cast<const float*>(a->data),
                                     static_cast<float*>(d->data), s);
        case ANE_GGML_OP_ROPE:
            if (!data_ok(b)) return ANE_ERR_BAD_POINTER;
            return rope_node_launch((uint32_t)d->ne[0], n_rows(d), param_f32(d, 5),
                                    static_cast<const int32_t*>(b->data), static_cast<const uint8_t*>(a->data),
                                    rows_of(a), static_cast<uint8_t*>(d->data), rows_of(d), s);
        case ANE_GGML_OP_CPY: {
            const uint64_t n = n_elements(d);
            if (contiguous(a) && contiguous(d)) {
                if (d->data == a->data) return ANE_OK;
                return hipMemcpyAsync(d->data, a->data, n * 4, hipMemcpyDeviceToDevice, s) == hipSuccess
                           ? ANE_OK
                           : ANE_ERR_HIP;
            }
            if (same_shape(a, d) && a->nb[0] == 4 && d->nb[0] == 4) return rows_ew<3>(be, d, a, nullptr, 0.0f);
            uint64_t g = (n + 255) / 256;
            if (g > 65536) g = 65536;
            hipLaunchKernelGGL(k_copy_any, dim3((uint32_t)g), dim3(256), 0, s, n, shape_of(d),
                               static_cast<uint8_t*>(d->data), shape_of(a), static_cast<const uint8_t*>(a->data));
            ANE_HIP_CHECK_LAUNCH();
            return ANE_OK;
        }
        default:
            return ANE_ERR_INVALID_ARG;
    }
}

bool node_supported(const ane_ggml_tensor* d) {
    switch (d->op) {
        case ANE_GGML_OP_MUL_MAT: return mul_mat_supported(d);
        case ANE_GGML_OP_ADD:
        case ANE_GGML_OP_MUL: return binary_supported(d);
        case ANE_GGML_OP_SCALE: return scale_supported(d);
        case ANE_GGML_OP_RMS_NORM: return rms_norm_supported(d);
        case ANE_GGML_OP_SOFT_MAX: return soft_max_supported(d);
        case ANE_GGML_OP_SILU: return silu_supported(d);
        case ANE_GGML_OP_ROPE: return rope_supported(d);
        case ANE_GGML_OP_CPY: return cpy_supported(d);
        default: return false;
    }
}

}  // namespace
}  // namespace ane

using namespace ane;

extern "C" const char* ane_ggml_backend_name(void) { return "ANE"; }
extern "C" const char* ane_ggml_device_name(void) { return "ANE0"; }

extern "C" ane_ggml_backend_t ane_ggml_backend_init(void* stream) {
    auto* be = new (std::nothrow) ane_ggml_backend{(hipStream_t)stream, ANE_GGML_Q8_G, nullptr, 0};
    return be;
}

extern "C" void ane_ggml_backend_free(ane_ggml_backend_t be) {
    if (!be) return;
    if (be->ws) {
        (void)hipStreamSynchronize(be->stream);
        (void)hipFree(be->ws);
    }
    delete be;
}

extern "C" void* ane_ggml_backend_get_stream(ane_ggml_backend_t be) { return be ? (void*)be->stream : nullptr; }

extern "C" void ane_ggml_backend_set_stream(ane_ggml_backend_t be, void* stream) {
    if (be) be->stream = (hipStream_t)stream;
}

extern "C" void ane_ggml_backend_set_q8_mode(ane_ggml_backend_t be, int mode) {
    if (be) be->q8_mode = mode == ANE_GGML_Q8_R ? ANE_GGML_Q8_R : ANE_GGML_Q8_G;
}

extern "C" int ane_ggml_supports_op(const ane_ggml_tensor* node) {
    if (!node) return 0;
    return node_supported(node) ? 1 : 0;
}

extern "C" int ane_ggml_compute_forward(ane_ggml_backend_t be, const ane_ggml_tensor* node) {
    if (!be || !node) return ANE_ERR_BAD_POINTER;
    if (node->op == ANE_GGML_OP_NONE || is_empty(node)) return ANE_OK;
    if (!node_supported(node)) return ANE_ERR_INVALID_ARG;
    return node->op == ANE_GGML_OP_MUL_MAT ? mul_mat(be, node) : fp32_node(be, node);
}

extern "C" int ane_ggml_graph_compute(ane_ggml_backend_t be, ane_ggml_tensor* const* nodes, int n_nodes) {
    if (!be || (n_nodes > 0 && !nodes)) return ANE_ERR_BAD_POINTER;
    for (int i = 0; i < n_nodes; i++) {
        const int st = ane_ggml_compute_forward(be, nodes[i]);
        if (st != ANE_OK) return st;
    }
    return hipStreamSynchronize(be->stream) == hipSuccess ? ANE_OK : ANE_ERR_HIP;
}
