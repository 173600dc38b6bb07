// qformats.hpp -- the reference's other weight formats as lane decoders:
// each format's super-block size and acc(s, xs, l, acc), lane l's fmas over
// one staged super-block in the handler's order (bytecode_interpreter.s
// lines per format below).  Shared by k_qgemv (qformats.hip) and the
// streaming kernel (q8_0.hip).
#pragma once

#include "common.hpp"

#include <type_traits>

namespace ane {
namespace qf {

__device__ __forceinline__ uint32_t lu8(const uint8_t* p) { return *p; }
__device__ __forceinline__ uint32_t lu16(const uint8_t* p) { return lu8(p) | (lu8(p + 1) << 8); }
__device__ __forceinline__ uint32_t lu32(const uint8_t* p) { return lu16(p) | (lu16(p + 2) << 16); }
__device__ __forceinline__ float lh(const uint8_t* p) { return half_bits_to_float(lu16(p)); }

// Multi-byte fields of a super-block in LDS whose base is A-byte aligned.
// A = 1 (k_qgemv, whose rows sit at any byte offset): composed from bytes.
// A = 2, 4 or 16 (the streaming kernel: super-blocks laid out from 16-byte
// aligned rows): single typed 16- or 32-bit reads of the aligned fields.  A
// load the compiler composes from bytes loses its alias information, and
// before such an LDS load it waits for every outstanding copy to LDS, the
// ring's next items included; the typed reads keep it.
template <int A>
__device__ __forceinline__ uint32_t fld16(const uint8_t* p) {
    if constexpr (A >= 2) return *reinterpret_cast<const uint16_t*>(p);
    else return lu16(p);
}
template <int A>
__device__ __forceinline__ uint32_t fld32(const uint8_t* p) {
    if constexpr (A >= 4) {
        return *reinterpret_cast<const uint32_t*>(p);
    } else if constexpr (A == 2) {
        return (uint32_t)*reinterpret_cast<const uint16_t*>(p) |
               ((uint32_t)*reinterpret_cast<const uint16_t*>(p + 2) << 16);
    } else {
        return lu32(p);
    }
}
template <int A>
__device__ __forceinline__ float fldh(const uint8_t* p) { return half_bits_to_float(fld16<A>(p)); }

// v of lane J of this lane's 16-lane row (DPP row_newbcast).  The 16 lanes
// of a weight row form one DPP row in every caller, and all of them are
// active where the decoders run, so a sub-block's scales can be decoded by
// one lane and shared: the values are the same fp32 numbers every lane
// would have computed.
template <int J>
__device__ __forceinline__ float row_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + J, 0xf, 0xf, false));
}

template <int J>
__device__ __forceinline__ uint32_t row_bcast_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x150 + J, 0xf, 0xf, false);
}

// f(integral_constant<int, J>) for J = 0 .. N-1, in order.
template <int N, int J = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (J < N) {
        f(std::integral_constant<int, J>{});
        static_for<N, J + 1>(f);
    }
}

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
    template <int A = 1>
    __device__ static void acc(const uint8_t* s, const float* xs, uint32_t l, float& a) {
        // lane l decodes sub-block l % 8's fl(d * sc) and fl(-dmin * m)
        const float d = fldh<A>(s), nmin = -fldh<A>(s + 2);
        uint32_t scl, ml;
        scale_min6(s + 4, (int)(l & 7), scl, ml);
        const float dsl = __fmul_rn(d, (float)scl), dml = __fmul_rn(nmin, (float)ml);
        static_for<8>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            const float ds = row_bcast<j>(dsl), dm = row_bcast<j>(dml);
            const uint32_t b = lu8(s + 16 + 16 * j + l);
            a = __builtin_fmaf(__fadd_rn(__fmul_rn((float)(b & 15u), ds), dm), xs[32 * j + l], a);
            a = __builtin_fmaf(__fadd_rn(__fmul_rn((float)(b >> 4), ds), dm), xs[32 * j + 16 + l], a);
        });
    }
};

struct Q2K {
    static constexpr uint32_t kBytes = 84, kValues = 256, kStage = 4;
    template <int A = 1>
    __device__ static void acc(const uint8_t* s, const float* xs, uint32_t l, float& a) {
        // lane l decodes sub-block l's fl(d * sc) and fl(-dmin * m)
        const float d = fldh<A>(s + 80), nmin = -fldh<A>(s + 82);
        // (the qs words stay per-lane LDS reads: broadcasting them as well
        // measured slower for this format)
        const uint32_t scb = lu8(s + l);
        const float dsl = __fmul_rn(d, (float)(scb & 15u)), dml = __fmul_rn(nmin, (float)(scb >> 4));
        static_for<16>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            const float ds = row_bcast<j>(dsl), dm = row_bcast<j>(dml);
            const uint32_t q = (fld32<A>(s + 16 + 4 * j) >> (2 * l)) & 3u;
            a = __builtin_fmaf(__fadd_rn(__fmul_rn((float)q, ds), dm), xs[16 * j + l], a);
        });
    }
};

// The second half of each sub-block first shifts its qs word right by the bit
// pattern of the lane's first-half input (SVE LSR: amounts >= 32 give 0), as
// the handler does with the register its input load reused (:11323-11329).
struct Q3K {
    static constexpr uint32_t kBytes = 110, kValues = 256, kStage = 4;
    template <int A = 1>
    __device__ static void acc(const uint8_t* s, const float* xs, uint32_t l, float& a) {
        // lane l decodes sub-block l % 8's fl(d * (sc - 32))
        const float d = fldh<A>(s + 108);
        const uint32_t jl = l & 7;
        const uint32_t scl = jl < 4 ? (lu8(s + 96 + jl) & 63u)
                                    : ((lu8(s + 100 + jl) & 15u) | ((lu8(s + 92 + jl) >> 6) << 4));
        const float dsl = __fmul_rn(d, (float)((int)scl - 32));
        // dword l of qs and dword l % 8 of hmask, which every lane of the row reads
        const uint32_t qsl = fld32<A>(s + 32 + 4 * l), hml = fld32<A>(s + 4 * jl);
        static_for<8>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            const float ds = row_bcast<j>(dsl);
            const float xa = xs[32 * j + l];
            const uint32_t hm = row_bcast_u32<j>(hml);
            const uint32_t qa = row_bcast_u32<2 * j>(qsl), ha = hm & 0xffffu;
            const int q0 = (int)(((qa >> (2 * l)) & 3u) | (((ha >> l) & 1u) << 2));
            a = __builtin_fmaf(__fmul_rn((float)(q0 - 4), ds), xa, a);
            const uint32_t sh = __float_as_uint(xa);
            const uint32_t qbw = row_bcast_u32<2 * j + 1>(qsl);
            const uint32_t qb = sh >= 32u ? 0u : qbw >> sh;
            const uint32_t hb = hm >> 16;
            const int q1 = (int)(((qb >> (2 * l)) & 3u) | (((hb >> l) & 1u) << 2));
            a = __builtin_fmaf(__fmul_rn((float)(q1 - 4), ds), xs[32 * j + 16 + l], a);
        });
    }
};

struct Q5K {
    static constexpr uint32_t kBytes = 176, kValues = 256, kStage = 4;
    template <int A = 1>
    __device__ static void acc(const uint8_t* s, const float* xs, uint32_t l, float& a) {
        // lane l decodes sub-block l % 8's fl(d * sc) and fl(-dmin * m)
        const float d = fldh<A>(s), nmin = -fldh<A>(s + 2);
        uint32_t scl, ml;
        scale_min6(s + 4, (int)(l & 7), scl, ml);
        const float dsl = __fmul_rn(d, (float)scl), dml = __fmul_rn(nmin, (float)ml);
        static_for<8>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            const float ds = row_bcast<j>(dsl), dm = row_bcast<j>(dml);
            // (qh stays a per-lane LDS read: broadcasting it measured slower)
            const uint32_t b = lu8(s + 48 + 16 * j + l), h = fld32<A>(s + 16 + 4 * j);
            const uint32_t q0 = (b & 15u) | ((((h & 0xffffu) >> l) & 1u) << 4);
            const uint32_t q1 = (b >> 4) | ((((h >> 16) >> l) & 1u) << 4);
            a = __builtin_fmaf(__fadd_rn(__fmul_rn((float)q0, ds), dm), xs[32 * j + l], a);
            a = __builtin_fmaf(__fadd_rn(__fmul_rn((float)q1, ds), dm), xs[32 * j + 16 + l], a);
        });
    }
};

struct Q6K {
    static constexpr uint32_t kBytes = 210, kValues = 256, kStage = 4;
    __device__ static void acc(const uint8_t* s, const float* xs, uint32_t l, float& a) {
        // lane l decodes sub-block l's fl(d * sc)
        const float d = lh(s + 208);
        const float dsl = __fmul_rn(d, (float)(int8_t)lu8(s + 192 + l));
        const uint32_t qhl = lu32(s + 128 + 4 * l);  // dword l of qh, read by every lane
        static_for<16>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            const float ds = row_bcast<j>(dsl);
            const uint32_t byte = lu8(s + 8 * j + (l >> 1));
            const uint32_t nib = (l & 1) ? (byte >> 4) : (byte & 15u);
            const int q = (int)(nib | (((row_bcast_u32<j>(qhl) >> (2 * l)) & 3u) << 4));
            a = __builtin_fmaf(__fmul_rn((float)(q - 32), ds), xs[16 * j + l], a);
        });
    }
};

}  // namespace qf
}  // namespace ane
