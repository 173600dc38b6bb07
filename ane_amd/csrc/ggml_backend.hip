// ggml_backend.hip -- the GGML_OP_MUL_MAT hook of ane's ggml backend
// (reference src/ggml-backend/ggml-ane.cpp:109-154, 287-299, 363-368) on the
// Q8_0 kernels of q8_0.hip and the Q4_0 GEMV of qformats.hip.
//
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

#include "../../include/ggml-ane-hip.h"
#include "common.hpp"

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
    if (node->op == ANE_GGML_OP_MUL_MAT) return mul_mat_supported(node) ? 1 : 0;
    return 0;
}

extern "C" int ane_ggml_compute_forward(ane_ggml_backend_t be, const ane_ggml_tensor* node) {
    if (!be || !node) return ANE_ERR_BAD_POINTER;
    if (node->op == ANE_GGML_OP_NONE || is_empty(node)) return ANE_OK;
    if (node->op != ANE_GGML_OP_MUL_MAT || !mul_mat_supported(node)) return ANE_ERR_INVALID_ARG;
    return mul_mat(be, node);
}

extern "C" int ane_ggml_graph_compute(ane_ggml_backend_t be, ane_ggml_tensor* const* nodes, int n_nodes) {
    if (!be || (n_nodes > 0 && !nodes)) return ANE_ERR_BAD_POINTER;
    for (int i = 0; i < n_nodes; i++) {
        const int st = ane_ggml_compute_forward(be, nodes[i]);
        if (st != ANE_OK) return st;
    }
    return hipStreamSynchronize(be->stream) == hipSuccess ? ANE_OK : ANE_ERR_HIP;
}
