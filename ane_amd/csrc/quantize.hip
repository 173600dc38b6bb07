// quantize.hip -- fp32 <-> int8 element-wise kernels of the ane opcode set:
// quantize_fp32_i8 (0x19), dequantize_i8_fp32 (0x1A),
// quantize_fp32_i8_channelwise (0x1C) and pack_b_i8 (0x1B).
//
// All of them are HBM-bound streaming passes: 16-byte global loads per lane,
// a grid sized to a few waves per CU, no LDS except block reductions.
#include "common.hpp"

namespace ane {

constexpr int kQThreads = 256;
constexpr uint32_t kMaxPartials = 2048;

static uint32_t stream_blocks(uint64_t n_vec4) {
    uint64_t b = (n_vec4 + kQThreads * 4 - 1) / (kQThreads * 4);
    if (b < 1) b = 1;
    if (b > kMaxPartials) b = kMaxPartials;
    return (uint32_t)b;
}

// Pass 1 of 0x19 (bytecode_interpreter.s:1893-1905): per-block max |x| keys.
__global__ void __launch_bounds__(kQThreads)
k_absmax_partial(const float* __restrict__ src, uint64_t n,
                 uint32_t* __restrict__ partials) {
    __shared__ uint32_t red[4];
    uint32_t m = 0;
    const uint64_t tid = (uint64_t)blockIdx.x * kQThreads + threadIdx.x;
    const uint64_t stride = (uint64_t)gridDim.x * kQThreads;
    uint64_t head = 0;
    if ((((uintptr_t)src) & 15) == 0) {
        const uint64_t n4 = n >> 2;
        const float4* s4 = reinterpret_cast<const float4*>(src);
        for (uint64_t i = tid; i < n4; i += stride) {
            float4 v = s4[i];
            uint32_t a = abs_key(v.x), b = abs_key(v.y), c = abs_key(v.z), d = abs_key(v.w);
            a = a > b ? a : b;
            c = c > d ? c : d;
            a = a > c ? a : c;
            m = m > a ? m : a;
        }
        head = n4 << 2;
    }
    for (uint64_t i = head + tid; i < n; i += stride) {
        uint32_t a = abs_key(src[i]);
        m = m > a ? m : a;
    }
    m = block_max_u32_256(m, red);
    if (threadIdx.x == 0) partials[blockIdx.x] = m;
}

// Pass 2 of 0x19 (bytecode_interpreter.s:1906-1950): every block folds the
// partial maxima, derives (scale, inv) and quantizes its grid-stride share.
__global__ void __launch_bounds__(kQThreads)
k_quantize(const float* __restrict__ src, uint64_t n, int8_t* __restrict__ dst,
           const uint32_t* __restrict__ partials, uint32_t np,
           float* __restrict__ scale_out) {
    __shared__ uint32_t red[4];
    uint32_t m = 0;
    for (uint32_t i = threadIdx.x; i < np; i += kQThreads) {
        uint32_t a = partials[i];
        m = m > a ? m : a;
    }
    m = block_max_u32_256(m, red);
    float scale, inv;
    quant_params(__uint_as_float(m), scale, inv);
    if (blockIdx.x == 0 && threadIdx.x == 0 && scale_out) *scale_out = scale;

    const uint64_t tid = (uint64_t)blockIdx.x * kQThreads + threadIdx.x;
    const uint64_t stride = (uint64_t)gridDim.x * kQThreads;
    uint64_t head = 0;
    if ((((uintptr_t)src) & 15) == 0 && (((uintptr_t)dst) & 3) == 0) {
        const uint64_t n4 = n >> 2;
        const float4* s4 = reinterpret_cast<const float4*>(src);
        uint32_t* d4 = reinterpret_cast<uint32_t*>(dst);
        // every value is one whose max |x| was just folded, so pack4_fast
        // (bit-identical, two VALU per value) applies whenever that max and
        // inv are finite
        if (fast_quant_ok(__uint_as_float(m), inv)) {
            for (uint64_t i = tid; i < n4; i += stride) {
                const float4 v = s4[i];
                d4[i] = pack4_fast(v.x, v.y, v.z, v.w, inv);
            }
        } else {
            for (uint64_t i = tid; i < n4; i += stride) {
                const float4 v = s4[i];
                d4[i] = pack4(v.x, v.y, v.z, v.w, inv);
            }
        }
        head = n4 << 2;
    }
    for (uint64_t i = head + tid; i < n; i += stride) dst[i] = (int8_t)quant1(src[i], inv);
}

// 0x1A (bytecode_interpreter.s:1951-1977): scvtf then fmul.
__global__ void __launch_bounds__(kQThreads)
k_dequantize(const int8_t* __restrict__ src, uint64_t n, float scale,
             float* __restrict__ dst) {
    const uint64_t tid = (uint64_t)blockIdx.x * kQThreads + threadIdx.x;
    const uint64_t stride = (uint64_t)gridDim.x * kQThreads;
    uint64_t head = 0;
    if ((((uintptr_t)src) & 3) == 0 && (((uintptr_t)dst) & 15) == 0) {
        const uint64_t n4 = n >> 2;
        const uint32_t* s4 = reinterpret_cast<const uint32_t*>(src);
        float4* d4 = reinterpret_cast<float4*>(dst);
        for (uint64_t i = tid; i < n4; i += stride) {
            uint32_t q = s4[i];
            float4 o;
            o.x = __fmul_rn((float)(int8_t)(q & 0xff), scale);
            o.y = __fmul_rn((float)(int8_t)((q >> 8) & 0xff), scale);
            o.z = __fmul_rn((float)(int8_t)((q >> 16) & 0xff), scale);
            o.w = __fmul_rn((float)(int8_t)(q >> 24), scale);
            d4[i] = o;
        }
        head = n4 << 2;
    }
    for (uint64_t i = head + tid; i < n; i += stride)
        dst[i] = __fmul_rn((float)src[i], scale);
}

// 0x1C (bytecode_interpreter.s:2591-2662): one block per row, two passes.
__global__ void __launch_bounds__(kQThreads)
k_quantize_channelwise(const float* __restrict__ src, uint32_t cpad,
                       int8_t* __restrict__ dst, float* __restrict__ scales) {
    __shared__ uint32_t red[4];
    const uint64_t row = blockIdx.x;
    const float* s = src + row * cpad;
    int8_t* d = dst + row * cpad;
    uint32_t m = 0;
    for (uint32_t i = threadIdx.x; i < cpad; i += kQThreads) {
        uint32_t a = abs_key(s[i]);
        m = m > a ? m : a;
    }
    m = block_max_u32_256(m, red);
    float scale, inv;
    quant_params(__uint_as_float(m), scale, inv);
    if (threadIdx.x == 0) scales[row] = scale;
    for (uint32_t i = threadIdx.x; i < cpad; i += kQThreads) d[i] = (int8_t)quant1(s[i], inv);
}

// 0x1B (bytecode_interpreter.s:2459-2582): each thread writes one 64-byte
// group of the SMOPA panel format, dst[(p*G+g)*64 + 4c + d] = B[4g+d][16p+c].
__global__ void __launch_bounds__(kQThreads)
k_pack_b(uint32_t K, uint32_t N, uint32_t G, uint32_t P,
         const int8_t* __restrict__ src, int8_t* __restrict__ dst) {
    const uint64_t idx = (uint64_t)blockIdx.x * kQThreads + threadIdx.x;  // p*G + g
    if (idx >= (uint64_t)P * G) return;
    const uint32_t p = (uint32_t)(idx / G), g = (uint32_t)(idx % G);
    uint32_t out[16];
#pragma unroll
    for (int c = 0; c < 16; c++) {
        uint32_t w = 0;
        const uint32_t col = 16 * p + c;
#pragma unroll
        for (int d = 0; d < 4; d++) {
            const uint32_t k = 4 * g + d;
            uint32_t b = (k < K && col < N) ? (uint8_t)src[(uint64_t)k * N + col] : 0u;
            w |= b << (8 * d);
        }
        out[c] = w;
    }
    uint4* o = reinterpret_cast<uint4*>(dst + idx * 64);
    if ((((uintptr_t)dst) & 15) == 0) {
#pragma unroll
        for (int q = 0; q < 4; q++)
            o[q] = make_uint4(out[4 * q], out[4 * q + 1], out[4 * q + 2], out[4 * q + 3]);
    } else {
        for (int c = 0; c < 16; c++)
            for (int d = 0; d < 4; d++) dst[idx * 64 + 4 * c + d] = (int8_t)(out[c] >> (8 * d));
    }
}

}  // namespace ane

using namespace ane;

extern "C" size_t ane_hip_quantize_workspace_size(uint64_t n) {
    (void)n;
    return kMaxPartials * sizeof(uint32_t);
}

extern "C" int ane_hip_quantize_fp32_i8(uint64_t count, int pad16, const float* src,
                                        int8_t* dst, float* scale_out, void* workspace,
                                        size_t workspace_bytes, void* stream) {
    uint64_t n = count;
    if (pad16) {
        n = ceil_to(count, 16);
        if (n == 0) n = 16;
    }
    if (!src || !dst) return ANE_ERR_BAD_POINTER;
    if (!workspace || workspace_bytes < ane_hip_quantize_workspace_size(n)) return ANE_ERR_WORKSPACE;
    hipStream_t s = (hipStream_t)stream;
    uint32_t* partials = (uint32_t*)workspace;
    const uint32_t nb = stream_blocks(n / 4 + 1);
    hipLaunchKernelGGL(k_absmax_partial, dim3(nb), dim3(kQThreads), 0, s, src, n, partials);
    hipLaunchKernelGGL(k_quantize, dim3(nb), dim3(kQThreads), 0, s, src, n, dst, partials, nb,
                       scale_out);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

extern "C" int ane_hip_dequantize_i8_fp32(uint64_t count, float scale, const int8_t* src,
                                          float* dst, void* stream) {
    const uint64_t n = ceil_to(count, 16);
    if (n == 0) return ANE_OK;
    if (!src || !dst) return ANE_ERR_BAD_POINTER;
    const uint32_t nb = stream_blocks(n / 4 + 1);
    hipLaunchKernelGGL(k_dequantize, dim3(nb), dim3(kQThreads), 0, (hipStream_t)stream, src, n,
                       scale, dst);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

extern "C" int ane_hip_quantize_channelwise(uint32_t rows, uint32_t cols, const float* src,
                                            int8_t* dst, float* scales, void* stream) {
    if (rows == 0) return ANE_OK;
    if (!src || !dst || !scales) return ANE_ERR_BAD_POINTER;
    uint64_t cpad = ceil_to(cols, 16);
    if (cpad == 0) cpad = 16;
    if (cpad > 0xffffffffull) return ANE_ERR_INVALID_ARG;
    hipLaunchKernelGGL(k_quantize_channelwise, dim3(rows), dim3(kQThreads), 0,
                       (hipStream_t)stream, src, (uint32_t)cpad, dst, scales);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

extern "C" size_t ane_hip_packed_b_size(uint32_t K, uint32_t N) {
    const uint64_t G = ceil_to(K, 4) / 4, P = ceil_to(N, 16) / 16;
    return (size_t)(P * G * 64);
}

extern "C" int ane_hip_pack_b_i8(uint32_t K, uint32_t N, const int8_t* src, int8_t* dst,
                                 void* stream) {
    const uint64_t G = ceil_to(K, 4) / 4, P = ceil_to(N, 16) / 16;
    if (G == 0 || P == 0) return ANE_OK;
    if (!src || !dst) return ANE_ERR_BAD_POINTER;
    const uint64_t groups = G * P;
    const uint64_t nb = (groups + kQThreads - 1) / kQThreads;
    if (nb > 0x7fffffffull) return ANE_ERR_INVALID_ARG;
    hipLaunchKernelGGL(k_pack_b, dim3((uint32_t)nb), dim3(kQThreads), 0, (hipStream_t)stream, K, N,
                       (uint32_t)G, (uint32_t)P, src, dst);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}
