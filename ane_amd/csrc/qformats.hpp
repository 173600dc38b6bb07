// qformats.hpp -- the reference's other weight formats as lane decoders:
// each format's super-block size and acc(s, xs, l, acc), lane l's fmas over
// one staged super-block in the handler's order (bytecode_interpreter.s
// lines per format below).  Shared by k_qgemv (qformats.hip) and the
// streaming kernel (q8_0.hip).
#pragma once

#include "common.hpp"

namespace ane {
namespace qf {

__device__ __forceinline__ uint32_t lu8(const uint8_t* p) { return *p; }
__device__ __forceinline__ uint32_t lu16(const uint8_t* p) { return lu8(p) | (lu8(p + 1) << 8); }
__device__ __forceinline__ uint32_t lu32(const uint8_t* p) { return lu16(p) | (lu16(p + 2) << 16); }
__device__ __forceinline__ float lh(const uint8_t* p) { return half_bits_to_float(lu16(p)); }

// Q4_K / Q5_K 6-bit (scale, min) of sub-block j (bytecode_interpreter.s:11064-11089).
__device__ __forceinline__ void scale_min6(const uint8_t* s, int j, uint32_t& sc, uint32_t& m) {
    if (j < 4) {
        sc = lu8(s + j) & 63u;
        m = lu8(s + j + 4) & 63u;
    } else {
        sc = (lu8(s + j + 4) & 15u) | ((lu8(s + j - 4) >> 6) << 4);
        m = (lu8(s + j + 4) >> 4) | ((lu8(s + j) >> 6) << 4);
    }
}

// Each format: kBytes / kValues per super-block (a Q4_0 block counts as one),
// kStage super-blocks per stage, and acc(s, xs, l, acc): lane l's fmas over
// the super-block at LDS s with its inputs at LDS xs, in the handler's order.
struct Q40 {
    static constexpr uint32_t kBytes = 18, kValues = 32, kStage = 32;
    __device__ static void acc(const uint8_t* s, const float* xs, uint32_t l, float& a) {
        const float d = lh(s);
        const uint32_t b = lu8(s + 2 + l);
        // q - 8 without an int conversion: the float with bits 2^23 + q,
        // minus 2^23 + 8, is q - 8 exactly.  The high nibble stays in place
        // (16 (q - 8)) and meets d / 16, an exact scaling, so both products
        // equal the handler's fmul((float)(q - 8), d) bit for bit (they are
        // exact: 4- by 11-bit significands), infinities and NaNs included.
        const float lo = __fsub_rn(__uint_as_float((b & 15u) | 0x4B000000u), 8388616.0f);
        const float hi = __fsub_rn(__uint_as_float((b & 0xF0u) | 0x4B000000u), 8388736.0f);
        a = __builtin_fmaf(__fmul_rn(lo, d), xs[l], a);
        a = __builtin_fmaf(__fmul_rn(hi, __fmul_rn(d, 0.0625f)), xs[16 + l], a);
    }
};

struct Q4K {
    static constexpr uint32_t kBytes = 144, kValues = 256, kStage = 4;
    __device__ static void acc(const uint8_t* s, const float* xs, uint32_t l, float& a) {
        const float d = lh(s), nmin = -lh(s + 2);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint32_t sc, m;
            scale_min6(s + 4, j, sc, m);
            const float ds = __fmul_rn(d, (float)sc), dm = __fmul_rn(nmin, (float)m);
            const uint32_t b = lu8(s + 16 + 16 * j + l);
            a = __builtin_fmaf(__fadd_rn(__fmul_rn((float)(b & 15u), ds), dm), xs[32 * j + l], a);
            a = __builtin_fmaf(__fadd_rn(__fmul_rn((float)(b >> 4), ds), dm), xs[32 * j + 16 + l], a);
        }
    }
};

struct Q2K {
    static constexpr uint32_t kBytes = 84, kValues = 256, kStage = 4;
    __device__ static void acc(const uint8_t* s, const float* xs, uint32_t l, float& a) {
        const float d = lh(s + 80), nmin = -lh(s + 82);
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const uint32_t scb = lu8(s + j);
            const float ds = __fmul_rn(d, (float)(scb & 15u)), dm = __fmul_rn(nmin, (float)(scb >> 4));
            const uint32_t q = (lu32(s + 16 + 4 * j) >> (2 * l)) & 3u;
            a = __builtin_fmaf(__fadd_rn(__fmul_rn((float)q, ds), dm), xs[16 * j + l], a);
        }
    }
};

// The second half of each sub-block first shifts its qs word right by the bit
// pattern of the lane's first-half input (SVE LSR: amounts >= 32 give 0), as
// the handler does with the register its input load reused (:11323-11329).
struct Q3K {
    static constexpr uint32_t kBytes = 110, kValues = 256, kStage = 4;
    __device__ static void acc(const uint8_t* s, const float* xs, uint32_t l, float& a) {
        const float d = lh(s + 108);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t sc = j < 4 ? (lu8(s + 96 + j) & 63u)
                                      : ((lu8(s + 100 + j) & 15u) | ((lu8(s + 92 + j) >> 6) << 4));
            const float ds = __fmul_rn(d, (float)((int)sc - 32));
            const float xa = xs[32 * j + l];
            const uint32_t qa = lu32(s + 32 + 8 * j), ha = lu16(s + 4 * j);
            const int q0 = (int)(((qa >> (2 * l)) & 3u) | (((ha >> l) & 1u) << 2));
            a = __builtin_fmaf(__fmul_rn((float)(q0 - 4), ds), xa, a);
            const uint32_t sh = __float_as_uint(xa);
            const uint32_t qb = sh >= 32u ? 0u : lu32(s + 36 + 8 * j) >> sh;
            const uint32_t hb = lu16(s + 4 * j + 2);
            const int q1 = (int)(((qb >> (2 * l)) & 3u) | (((hb >> l) & 1u) << 2));
            a = __builtin_fmaf(__fmul_rn((float)(q1 - 4), ds), xs[32 * j + 16 + l], a);
        }
    }
};

struct Q5K {
    static constexpr uint32_t kBytes = 176, kValues = 256, kStage = 4;
    __device__ static void acc(const uint8_t* s, const float* xs, uint32_t l, float& a) {
        const float d = lh(s), nmin = -lh(s + 2);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint32_t sc, m;
            scale_min6(s + 4, j, sc, m);
            const float ds = __fmul_rn(d, (float)sc), dm = __fmul_rn(nmin, (float)m);
            const uint32_t b = lu8(s + 48 + 16 * j + l), h = lu32(s + 16 + 4 * j);
            const uint32_t q0 = (b & 15u) | ((((h & 0xffffu) >> l) & 1u) << 4);
            const uint32_t q1 = (b >> 4) | ((((h >> 16) >> l) & 1u) << 4);
            a = __builtin_fmaf(__fadd_rn(__fmul_rn((float)q0, ds), dm), xs[32 * j + l], a);
            a = __builtin_fmaf(__fadd_rn(__fmul_rn((float)q1, ds), dm), xs[32 * j + 16 + l], a);
        }
    }
};

struct Q6K {
    static constexpr uint32_t kBytes = 210, kValues = 256, kStage = 4;
    __device__ static void acc(const uint8_t* s, const float* xs, uint32_t l, float& a) {
        const float d = lh(s + 208);
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const float ds = __fmul_rn(d, (float)(int8_t)lu8(s + 192 + j));
            const uint32_t byte = lu8(s + 8 * j + (l >> 1));
            const uint32_t nib = (l & 1) ? (byte >> 4) : (byte & 15u);
            const int q = (int)(nib | (((lu32(s + 128 + 4 * j) >> (2 * l)) & 3u) << 4));
            a = __builtin_fmaf(__fmul_rn((float)(q - 32), ds), xs[16 * j + l], a);
        }
    }
};

}  // namespace qf
}  // namespace ane
