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
typedef unsigned v4u __attribute__((ext_vector_type(4)));
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

// ------------------------------------------------- DPP row permutations
// v_mov_b32 with a DPP control: every lane reads the named lane of its own
// 16-lane row (all rows and banks enabled, so every source is valid).
enum : int {
    kDppQuadXor1 = 0xB1,    // quad_perm [1,0,3,2]: lane ^ 1
    kDppQuadXor2 = 0x4E,    // quad_perm [2,3,0,1]: lane ^ 2
    kDppHalfMirror = 0x141, // lane i <-> 7-i within each 8 lanes
    kDppRowMirror = 0x140,  // lane i <-> 15-i within each 16 lanes
};

template <int ctrl>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, ctrl, 0xf, 0xf, false);
}
template <int ctrl>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xf, 0xf, false));
}

// SVE FADDV over 16 lanes (bytecode_interpreter.s:7059): the pairwise tree
// ((((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)))+(((a8+a9)+...))).  Each step adds
// the partner group's partial; after step k all lanes of a 2^k-group hold
// bit-identical values (fp32 addition is commutative), so pairing lane i
// with its mirror instead of i ^ 4 / i ^ 8 forms the same sums.  Every lane
// of the 16-lane row ends with the full sum.
__device__ __forceinline__ float faddv16(float v) {
    v = v + dpp_f32<kDppQuadXor1>(v);
    v = v + dpp_f32<kDppQuadXor2>(v);
    v = v + dpp_f32<kDppHalfMirror>(v);
    v = v + dpp_f32<kDppRowMirror>(v);
    return v;
}

// max over each aligned group of 8 lanes.
__device__ __forceinline__ uint32_t max8_u32(uint32_t m) {
    uint32_t o = dpp_u32<kDppQuadXor1>(m);
    m = m > o ? m : o;
    o = dpp_u32<kDppQuadXor2>(m);
    m = m > o ? m : o;
    o = dpp_u32<kDppHalfMirror>(m);
    return m > o ? m : o;
}

// SiLU(g) * u = (g / (1 + e^-g)) * u, the one definition every fused and
// unfused SiLU step uses (bytecode_interpreter.s:6617 computes the sigmoid
// with an exp approximation; fp32 expf here).
__device__ __forceinline__ float silu_mul1(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

// The canonical sum of squares of RMSNorm over K = 32 * nb values, the same
// bits whatever the workgroup shape that computes it:
//   q(b, p) = (x0^2 + x1^2) + (x2^2 + x3^2) for part p (values 4p..4p+3) of
//             32-block b, in fp64 (every square is exact);
//   s(b)    = ((q0 + q1) + (q2 + q3)) + ((q4 + q5) + (q6 + q7));
//   c(l)    = s(l) + s(l + 64) + s(l + 128) + ... in increasing b, l < 64;
//   ss      = the pairwise tree over c(0..63), adjacent pairs first.
// Lanes 8k..8k+7 of a wave hold the eight parts of one block.
__device__ __forceinline__ double sumsq4_f64(float4 f) {
    return ((double)f.x * f.x + (double)f.y * f.y) + ((double)f.z * f.z + (double)f.w * f.w);
}
__device__ __forceinline__ double sum8_f64(double v) {
    v += __shfl_xor(v, 1, 64);
    v += __shfl_xor(v, 2, 64);
    v += __shfl_xor(v, 4, 64);
    return v;
}
__device__ __forceinline__ double tree64_f64(double v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
    return v;
}
// c(l) then the tree, by one whole wave over the block sums s[0..nb).
__device__ __forceinline__ double canon_total_f64(const double* s, uint32_t nb) {
    const uint32_t lane = threadIdx.x & 63;
    double c = 0.0;
    for (uint32_t b = lane; b < nb; b += 64) c += s[b];
    return tree64_f64(c);
}

// RMSNorm's scale from the canonical sum of squares: 1 / sqrt(fl(fl(ss/K) + eps)).
__device__ __forceinline__ float rms_inv(double ss, uint32_t K, float eps) {
    const float ms = (float)(ss / (double)K);
    return 1.0f / sqrtf(ms + eps);
}

// Four quantized values packed little-endian into one dword.
__device__ __forceinline__ uint32_t pack4(float a, float b, float c, float d, float inv) {
    return (uint32_t)(quant1(a, inv) & 0xff) | ((uint32_t)(quant1(b, inv) & 0xff) << 8) |
           ((uint32_t)(quant1(c, inv) & 0xff) << 16) | ((uint32_t)(quant1(d, inv) & 0xff) << 24);
}

// pack4 for the values of a tensor whose quantization steps stay finite:
// amax = max |x| over the tensor and inv = fl(127 / amax) both finite
// (fast_quant_ok), and every x one of that tensor's values.  Then
//   t = fl(x * inv) is finite and |t| <= 127 (1 + 2^-24)^2 < 127.5 (inv is
//       a correctly rounded quotient, |x| <= amax), so the clamp of quant1
//       to [-127, 127] cannot bind once t is rounded to an integer;
//   t + 1.5 * 2^23 is a float in [2^23, 2^24), whose ulp is 1: the addition
//       rounds t half-to-even to an integer (frintn), and the low byte of
//       the sum's bits is that integer's two's-complement int8.
// Each addition is a v_add_f32 in SDWA form that writes only that low byte,
// into byte k of the packed result (the first one zero-fills the other
// bytes): two VALU instructions per value, against about ten for pack4.
// Bit-identical to pack4 under that condition; callers check it once per
// tensor.
__device__ __forceinline__ uint32_t pack4_fast(float a, float b, float c, float d, float inv) {
    const float magic = 12582912.0f;  // 1.5 * 2^23
    const float ta = __fmul_rn(a, inv), tb = __fmul_rn(b, inv), tc = __fmul_rn(c, inv), td = __fmul_rn(d, inv);
    uint32_t r;
    asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:DWORD"
        : "=v"(r) : "v"(ta), "v"(magic));
    asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
        : "+v"(r) : "v"(tb), "v"(magic));
    asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
        : "+v"(r) : "v"(tc), "v"(magic));
    asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
        : "+v"(r) : "v"(td), "v"(magic));
    return r;
}
// The condition of pack4_fast: amax (the NaN-propagating max of |x|) and
// inv = 127 / amax (or 127 when amax == 0) both finite.
__device__ __forceinline__ bool fast_quant_ok(float amax, float inv) {
    return __builtin_isfinite(amax) && __builtin_isfinite(inv);
}

// ----------------------------------------------------------- LDS copy helpers
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Raw buffer resource over [base, base + bytes): loads past `bytes` return
// zeros (checked per dword) without touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// One buffer_load_dwordx4 ... lds: lane l's 16 bytes at `voffset` land at
// LDS dst + 16*l (dst must be wave-uniform).
__device__ __forceinline__ void copy16_to_lds(__amdgpu_buffer_rsrc_t r, void* dst, uint32_t voffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)dst, 16, voffset, 0, 0, 0);
}

// The same copy with the non-temporal cache hint (the gfx940+ "nt" bit of
// the buffer instruction's cache-policy field): for weight streams read once
// per launch, measured 3-8 % faster on the Q8_0 matvecs.
constexpr int kCpolNt = 2;
// The gfx940+ "sc1" bit (agent scope) on a store: the line is written
// through the XCD's L2 to the memory side instead of being left dirty there,
// so a kernel that writes its output last does not end with a write-back
// burst of its L2s (the operand quantizer: 1.5 us of a 30 us launch, and
// the contraction reading its output next is no slower).
constexpr int kCpolSc1 = 16;
__device__ __forceinline__ void copy16_to_lds_nt(__amdgpu_buffer_rsrc_t r, void* dst, uint32_t voffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)dst, 16, voffset, 0, 0, kCpolNt);
}

// One buffer_load_dword ... lds: lane l's dword at `voffset` lands at LDS
// dst + 4*l.
__device__ __forceinline__ void copy4_to_lds(__amdgpu_buffer_rsrc_t r, void* dst, uint32_t voffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)dst, 4, voffset, 0, 0, 0);
}

// s_waitcnt with vmcnt = n and the LDS/export counters left unconstrained;
// the "memory" clobber keeps the compiler from moving LDS reads across it.
// Vector-memory loads (including copies to LDS) complete in issue order.
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(n >= 0 && n < 64, "vmcnt out of range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory");
}

// Workgroup barrier without the release fence of __syncthreads(), which
// would wait for every outstanding vector-memory operation (vmcnt(0)) and
// so drain copies that are meant to stay in flight.  LDS is coherent within
// the workgroup: a wave's completed copies (its vmcnt wait) or LDS writes
// (its lgkmcnt wait) plus s_barrier make them visible to the others.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

// s_waitcnt lgkmcnt(0) only (LDS and scalar memory), leaving stores in flight.
__device__ __forceinline__ void wait_lgkmcnt0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// LDS loads of bytes whose copies to LDS the caller has already waited for
// (its ring wait and barrier).  Before an ordinary load from LDS the
// compiler's wait insertion cannot always tell that no outstanding
// buffer_load ... lds writes those bytes, and then waits for every
// outstanding copy (vmcnt(0)); in a copy ring that includes the stage issued
// just before, so each stage's math would start only once the next stage has
// landed.  These loads wait for their own data only (lgkmcnt(0)).  The
// "memory" clobber keeps them after the caller's wait and barrier.
__device__ __forceinline__ uint32_t lds_offset(const void* p) { return (uint32_t)(uintptr_t)p; }
__device__ __forceinline__ float4 lds_load_settled_f4(const void* p) {
    float4 v;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_offset(p)) : "memory");
    return v;
}
__device__ __forceinline__ float lds_load_settled_f32(const void* p) {
    float v;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_offset(p)) : "memory");
    return v;
}
// N settled float4 loads at p, p + 64, ..., p + 64 (N - 1) bytes with one
// wait for all of them.
template <int N>
__device__ __forceinline__ void lds_load_settled_f4x(const void* p, float4 (&o)[N]) {
    static_assert(N == 1 || N == 2 || N == 4, "1, 2 or 4 loads");
    v4u u[N];
    if constexpr (N == 1) {
        asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(u[0]) : "v"(lds_offset(p)) : "memory");
    } else if constexpr (N == 2) {
        asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:64\n\ts_waitcnt lgkmcnt(0)"
                     : "=&v"(u[0]), "=&v"(u[1])
                     : "v"(lds_offset(p))
                     : "memory");
    } else {
        asm volatile(
            "ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:64\n\tds_read_b128 %2, %4 offset:128\n\t"
            "ds_read_b128 %3, %4 offset:192\n\ts_waitcnt lgkmcnt(0)"
            : "=&v"(u[0]), "=&v"(u[1]), "=&v"(u[2]), "=&v"(u[3])
            : "v"(lds_offset(p))
            : "memory");
    }
#pragma unroll
    for (int i = 0; i < N; i++)
        o[i] = make_float4(__uint_as_float(u[i].x), __uint_as_float(u[i].y), __uint_as_float(u[i].z),
                           __uint_as_float(u[i].w));
}

// The store counterpart, for LDS bytes no outstanding copy targets: an
// ordinary LDS store may otherwise wait for every outstanding copy first.
__device__ __forceinline__ void lds_store_settled_f4(void* p, float4 v) {
    const v4u u = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)};
    asm volatile("ds_write_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" ::"v"(lds_offset(p)), "v"(u) : "memory");
}

}  // namespace ane

namespace ane {
// Set (on the calling host thread) while ane_decode_token checks that every
// step of a layer can launch: the launch helpers then make all their checks
// and return ANE_OK just before launching anything.
extern thread_local bool t_plan_only;
}  // namespace ane

#define ANE_HIP_CHECK_LAUNCH()                                   \
    do {                                                         \
        hipError_t e__ = hipGetLastError();                      \
        if (e__ != hipSuccess) return ANE_ERR_HIP;               \
    } while (0)
