// common.hpp -- shared device helpers for the gfx950 kernels of ane_amd.
//
// Numerics: every kernel file is compiled with -ffp-contract=off and fp32
// denormals kept, so the float expressions below round exactly once per
// operation, as the reference's SVE instructions do.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ane_hip.h"

namespace ane {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// AArch64 FMAX with a non-NaN second operand (the clamp constants and the
// ReLU floor): NaN a -> NaN, max(-0, +0) = +0, otherwise the larger.
__device__ __forceinline__ float fmax_a(float a, float lo) {
    if (a != a) return a;
    return a > lo ? a : lo;
}

// bytecode_interpreter.s:1906-1920: zero guard, then two correctly rounded
// divisions (HIP fp32 '/' is IEEE-exact unless fast-math is requested).
__device__ __forceinline__ void quant_params(float amax, float& scale, float& inv) {
    if (amax == 0.0f) {
        scale = 1.0f;
        inv = 127.0f;
    } else {
        scale = amax / 127.0f;
        inv = 127.0f / amax;
    }
}

// bytecode_interpreter.s:1932-1944: fmul, clamp to [-127, 127], frintn,
// fcvtzs (NaN -> 0).  Returns the int8 value sign-extended to int.
__device__ __forceinline__ int quant1(float x, float inv) {
    float t = __fmul_rn(x, inv);
    if (t != t) return 0;
    t = fminf(fmaxf(t, -127.0f), 127.0f);
    return (int)__builtin_rintf(t);
}

// |x| as an order-preserving uint32 key: non-negative floats order like
// their bit patterns, and every NaN sorts above +inf, so a uint max over
// keys is the NaN-propagating FMAX reduction of bytecode_interpreter.s:1900.
__device__ __forceinline__ uint32_t abs_key(float x) {
    return __float_as_uint(x) & 0x7fffffffu;
}

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    _Float16 f;
    uint16_t b = (uint16_t)h;
    __builtin_memcpy(&f, &b, 2);
    return (float)f;  // v_cvt_f32_f16: exact, half denormals kept
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        uint32_t o = (uint32_t)__shfl_xor((int)v, off, kWave);
        v = v > o ? v : o;
    }
    return v;
}

// Block-wide max for blockDim.x == 256 (4 waves); result in every thread.
__device__ __forceinline__ uint32_t block_max_u32_256(uint32_t v, uint32_t* red4) {
    v = wave_max_u32(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red4[w] = v;
    __syncthreads();
    uint32_t r = red4[0];
    r = r > red4[1] ? r : red4[1];
    r = r > red4[2] ? r : red4[2];
    r = r > red4[3] ? r : red4[3];
    __syncthreads();
    return r;
}

__host__ __device__ inline uint64_t ceil_to(uint64_t x, uint64_t m) {
    return (x + m - 1) / m * m;
}

}  // namespace ane

#define ANE_HIP_CHECK_LAUNCH()                                   \
    do {                                                         \
        hipError_t e__ = hipGetLastError();                      \
        if (e__ != hipSuccess) return ANE_ERR_HIP;               \
    } while (0)
