// q8_0.hip -- Q8_0 matrix-vector kernels (ggml block layout: fp16 d followed
// by 32 int8 quants, 34 bytes per 32 weights, rows of K/32 blocks).
//
//   R mode  = the reference's q8_0_gemv (0x57, bytecode_interpreter.s:7010-7063):
//             fp32 x, 16 fma lanes per row, FADDV tree; reproduced bit-exactly.
//   G mode  = x quantized to Q8_0 per 32-block (0x19 arithmetic, fp32 scale),
//             v_dot4 int8 block dots, 16 fp32 partials (block b -> partial
//             b % 16, fmaf((float)isum, d_w*d_x, p)) combined by the same
//             FADDV tree.  Serves GGML_OP_MUL_MAT for every token.
#include "common.hpp"

namespace ane {

constexpr int kRowsPerBlock = 16;  // 16 lanes per row, 256 threads

__device__ __forceinline__ float faddv16(float v) {
    // xor-butterfly over 16 lanes with offsets 1, 2, 4, 8: every lane ends
    // with ((((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)))+(...)), the FADDV order.
    v = v + __shfl_xor(v, 1, kWave);
    v = v + __shfl_xor(v, 2, kWave);
    v = v + __shfl_xor(v, 4, kWave);
    v = v + __shfl_xor(v, 8, kWave);
    return v;
}

__global__ void __launch_bounds__(256)
k_q8_0_gemv_r(uint32_t M, uint32_t nb, const float* __restrict__ x,
              const uint8_t* __restrict__ W, float* __restrict__ y) {
    const uint32_t l = threadIdx.x & 15;
    const uint64_t m = (uint64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 4);
    const bool live = m < M;
    float acc = 0.0f;
    if (live) {
        const uint8_t* row = W + m * nb * 34;
        for (uint32_t b = 0; b < nb; b++) {
            const uint8_t* blk = row + (uint64_t)b * 34;
            const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(blk));
            const float w0 = __fmul_rn((float)(int8_t)blk[2 + l], d);
            acc = __builtin_fmaf(w0, x[32 * b + l], acc);
            const float w1 = __fmul_rn((float)(int8_t)blk[18 + l], d);
            acc = __builtin_fmaf(w1, x[32 * b + 16 + l], acc);
        }
    }
    acc = faddv16(acc);
    if (live && l == 0) y[m] = acc;
}

// Activation quantizer: one thread per 32-element block of x.
// Token t's row of x starts at x + t*K (K need not be a multiple of 32; the
// trailing K%32 values are ignored like the reference's nb = K >> 5).
__global__ void __launch_bounds__(256)
k_q8_0_quantize_x(uint64_t nblocks, uint32_t nb, uint32_t K, const float* __restrict__ x,
                  int8_t* __restrict__ qx, float* __restrict__ dx) {
    const uint64_t b = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblocks) return;
    const float* s = x + (b / nb) * K + (b % nb) * 32;
    uint32_t m = 0;
    for (int i = 0; i < 32; i++) {
        uint32_t a = abs_key(s[i]);
        m = m > a ? m : a;
    }
    float scale, inv;
    quant_params(__uint_as_float(m), scale, inv);
    dx[b] = scale;
    uint32_t* q = reinterpret_cast<uint32_t*>(qx + b * 32);
    for (int w = 0; w < 8; w++) {
        q[w] = (uint32_t)(quant1(s[4 * w], inv) & 0xff) |
               ((uint32_t)(quant1(s[4 * w + 1], inv) & 0xff) << 8) |
               ((uint32_t)(quant1(s[4 * w + 2], inv) & 0xff) << 16) |
               ((uint32_t)(quant1(s[4 * w + 3], inv) & 0xff) << 24);
    }
}

constexpr int kTokChunk = 4;

__global__ void __launch_bounds__(256)
k_q8_0_mul_mat_g(uint32_t N, uint32_t nb, uint32_t T, const int8_t* __restrict__ qx,
                 const float* __restrict__ dx, const uint8_t* __restrict__ W,
                 float* __restrict__ y) {
    const uint32_t l = threadIdx.x & 15;
    const uint64_t m = (uint64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 4);
    const bool live = m < N;
    const uint8_t* row = W + (live ? m : 0) * nb * 34;
    for (uint32_t t0 = 0; t0 < T; t0 += kTokChunk) {
        float p[kTokChunk];
#pragma unroll
        for (int t = 0; t < kTokChunk; t++) p[t] = 0.0f;
        if (live) {
            for (uint32_t b = l; b < nb; b += 16) {
                const uint8_t* blk = row + (uint64_t)b * 34;
                const uint16_t* h = reinterpret_cast<const uint16_t*>(blk);
                const float dw = half_bits_to_float(h[0]);
                int wq[8];
#pragma unroll
                for (int q = 0; q < 8; q++) wq[q] = (int)((uint32_t)h[1 + 2 * q] | ((uint32_t)h[2 + 2 * q] << 16));
#pragma unroll
                for (int t = 0; t < kTokChunk; t++) {
                    if (t0 + t < T) {
                        const uint64_t xb = (uint64_t)(t0 + t) * nb + b;
                        const int* xq = reinterpret_cast<const int*>(qx + xb * 32);
                        int isum = 0;
#pragma unroll
                        for (int q = 0; q < 8; q++) isum = __builtin_amdgcn_sdot4(wq[q], xq[q], isum, false);
                        const float dd = __fmul_rn(dw, dx[xb]);
                        p[t] = __builtin_fmaf((float)isum, dd, p[t]);
                    }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < kTokChunk; t++) {
            const float v = faddv16(p[t]);
            if (live && l == 0 && t0 + t < T) y[(uint64_t)(t0 + t) * N + m] = v;
        }
    }
}

}  // namespace ane

using namespace ane;

extern "C" int ane_hip_q8_0_gemv(uint32_t M, uint32_t K, const float* x, const void* W, float* y,
                                 void* stream) {
    if (M == 0) return ANE_OK;
    if (!y || ((K >> 5) && (!x || !W))) return ANE_ERR_BAD_POINTER;
    if ((((uintptr_t)W) & 1) != 0) return ANE_ERR_INVALID_ARG;
    const uint32_t nb = K >> 5;
    const uint64_t grid = ((uint64_t)M + kRowsPerBlock - 1) / kRowsPerBlock;
    hipLaunchKernelGGL(k_q8_0_gemv_r, dim3((uint32_t)grid), dim3(256), 0, (hipStream_t)stream, M, nb,
                       x, (const uint8_t*)W, y);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

extern "C" size_t ane_hip_q8_0_mul_mat_workspace_size(uint32_t K, uint32_t T) {
    const uint64_t nb = K >> 5;
    return (size_t)(ceil_to((uint64_t)T * nb * 32, 256) + ceil_to((uint64_t)T * nb * 4, 256) + 256);
}

extern "C" int ane_hip_q8_0_mul_mat(uint32_t N, uint32_t K, uint32_t T, const float* x,
                                    const void* W, float* y, void* workspace,
                                    size_t workspace_bytes, void* stream) {
    if (N == 0 || T == 0) return ANE_OK;
    const uint32_t nb = K >> 5;
    if (!y || (nb && (!x || !W))) return ANE_ERR_BAD_POINTER;
    if ((((uintptr_t)W) & 1) != 0) return ANE_ERR_INVALID_ARG;
    if (!workspace || (((uintptr_t)workspace) & 255) ||
        workspace_bytes < ane_hip_q8_0_mul_mat_workspace_size(K, T))
        return ANE_ERR_WORKSPACE;
    hipStream_t s = (hipStream_t)stream;
    int8_t* qx = (int8_t*)workspace;
    float* dx = (float*)((uint8_t*)workspace + ceil_to((uint64_t)T * nb * 32, 256));
    const uint64_t nblocks = (uint64_t)T * nb;
    if (nblocks) {
        hipLaunchKernelGGL(k_q8_0_quantize_x, dim3((uint32_t)((nblocks + 255) / 256)), dim3(256), 0,
                           s, nblocks, nb, K, x, qx, dx);
    }
    const uint64_t grid = ((uint64_t)N + kRowsPerBlock - 1) / kRowsPerBlock;
    hipLaunchKernelGGL(k_q8_0_mul_mat_g, dim3((uint32_t)grid), dim3(256), 0, s, N, nb, T, qx, dx,
                       (const uint8_t*)W, y);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}
