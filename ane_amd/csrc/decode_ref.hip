// decode_ref.hip -- the reference's decode-step handlers on gfx950, in their
// exact fp32 operation sequence, and the steps of the reference-arithmetic
// decode mode built from them.
//
// Handlers (src/bytecode_interpreter.s):
//   0x51 rms_norm_fp32  :6508-6565   16 fmla lanes over x^2, FADDV, fdiv by
//        (float)dim, fadd eps, frsqrte + two frsqrts steps, fl(fl(x*r)*w)
//   0x54 silu_fp32      :6617-6713   exp(-x) by a floor range reduction, a
//        degree-4 Horner polynomial and exponent-bit injection; 1/(1+e) by
//        frecpe + two frecps steps; fl(x * r)
//   0x55 rope_fp32      :6714-6912   ratio = theta^(2/dim) from a log/exp
//        polynomial chain; per pair pos / power, range reduction by rint of
//        x/pi, sin/cos Horner polynomials (fmad), rotation by fmul + fmls/fmla
//   0x56 softmax_fp32   :6913-7009   fmax, the same exp polynomial, 16 fadd
//        lanes, FADDV, fdiv 1/sum, fmul
// The estimate instructions follow the Arm ARM pseudocode (FPRSqrtEstimate /
// RecipSqrtEstimate, FPRecipEstimate / RecipEstimate, FPCR.AH = 0); FRSQRTS
// and FRECPS are fused: (3 - a*b)/2 and 2 - a*b.  Every fmla / fmls / fmad is
// an fmaf here, every other operation one correctly rounded fp32 operation
// (the file is compiled with -ffp-contract=off and denormals kept).
//
// A "lane" of the handlers is a 16-wide SVE vector lane: sums and dot
// products run in 16 sequential chains (element i in chain i mod 16) that
// meet in the FADDV tree, and the kernels below keep exactly those chains.
#include "../../include/ane_decode.h"
#include "common.hpp"
#include "ggml_rows.hpp"

namespace ane {
namespace {

constexpr uint32_t kLog2e = 0x3FB8AA3Bu, kC4 = 0x3C1D955Au, kC3 = 0x3D635847u, kC2 = 0x3E75FDF0u,
                   kLn2 = 0x3F317218u;

__device__ __forceinline__ float f_of(uint32_t u) { return __uint_as_float(u); }

// RecipSqrtEstimate(a), a in [128, 512).  The Arm ARM steps b up from 512
// while a' * (b+1)^2 < 2^28 (a' = 2a+1, or the even part of a plus one,
// doubled), then returns (b+1)/2: so b+1 is the least m >= 513 with
// a' * m^2 >= 2^28.  Here m comes from a double-precision sqrt and one
// integer correction each way, which gives the loop's result for all 384
// inputs (m is within one of ceil(sqrt(2^28 / a'))), instead of up to ~500
// serial iterations.
__device__ uint32_t recip_sqrt_estimate(uint32_t a) {
    if (a < 256) a = a * 2 + 1;
    else a = (((a >> 1) << 1) + 1) * 2;
    uint32_t m = (uint32_t)ceil(sqrt(268435456.0 / (double)a));
    if (m < 513) m = 513;
    if ((uint64_t)a * m * m < (1ull << 28)) m++;
    if (m > 513 && (uint64_t)a * (m - 1) * (m - 1) >= (1ull << 28)) m--;
    return m / 2;
}

__device__ float frsqrte_a(float x) {
    const uint32_t u = __float_as_uint(x), sign = u >> 31, ex = (u >> 23) & 0xff, fr = u & 0x7fffff;
    if (ex == 0xff && fr) return f_of(u | 0x00400000u);
    if (ex == 0 && fr == 0) return f_of((sign << 31) | 0x7f800000u);
    if (sign) return f_of(0x7fc00000u);
    if (ex == 0xff) return 0.0f;
    uint64_t f52 = (uint64_t)fr << 29;
    int e = (int)ex;
    if (e == 0) {  // normalise a denormal: its leading one to bit 51, then dropped
        const int sh = __builtin_clzll(f52) - 12;
        f52 <<= sh;
        e -= sh;
        f52 = (f52 << 1) & ((1ull << 52) - 1);
    }
    const uint32_t scaled = (e & 1) == 0 ? 256u + (uint32_t)(f52 >> 44) : 128u + (uint32_t)(f52 >> 45);
    const int rexp = (380 - e) / 2;
    const uint32_t est = recip_sqrt_estimate(scaled);
    return f_of(((uint32_t)(rexp & 0xff) << 23) | ((est & 0xff) << 15));
}

__device__ __forceinline__ float frecpe_a(float x) {
    const uint32_t u = __float_as_uint(x), sign = u >> 31, ex = (u >> 23) & 0xff, fr = u & 0x7fffff;
    if (ex == 0xff && fr) return f_of(u | 0x00400000u);
    if (ex == 0xff) return f_of(sign << 31);
    if (ex == 0 && fr < (1u << 21)) return f_of((sign << 31) | 0x7f800000u);  // zero or |x| < 2^-128
    uint64_t f52 = (uint64_t)fr << 29;
    int e = (int)ex;
    if (e == 0) {
        if (!(f52 & (1ull << 51))) {
            e = -1;
            f52 = (f52 << 2) & ((1ull << 52) - 1);
        } else {
            f52 = (f52 << 1) & ((1ull << 52) - 1);
        }
    }
    const uint32_t scaled = 256u + (uint32_t)(f52 >> 44);
    int rexp = 253 - e;
    const uint32_t est = ((1u << 19) / (scaled * 2 + 1) + 1) / 2;
    uint64_t frac = (uint64_t)(est & 0xff) << 44;
    if (rexp == 0) {
        frac = (1ull << 51) | (frac >> 1);
    } else if (rexp == -1) {
        frac = (1ull << 50) | (frac >> 2);
        rexp = 0;
    }
    return f_of((sign << 31) | ((uint32_t)(rexp & 0xff) << 23) | (uint32_t)(frac >> 29));
}

__device__ __forceinline__ bool inf_times_zero(float a, float b) {
    return (__builtin_isinf(a) && b == 0.0f) || (a == 0.0f && __builtin_isinf(b));
}
__device__ __forceinline__ float frsqrts_a(float a, float b) {
    return inf_times_zero(a, b) ? 1.5f : __fmul_rn(__builtin_fmaf(-a, b, 3.0f), 0.5f);
}
__device__ __forceinline__ float frecps_a(float a, float b) {
    return inf_times_zero(a, b) ? 2.0f : __builtin_fmaf(-a, b, 2.0f);
}

// fcvtzs to int32: truncation, saturating, NaN -> 0.
__device__ __forceinline__ int32_t cvtzs_a(float x) {
    if (x != x) return 0;
    if (x >= 2147483648.0f) return 0x7fffffff;
    if (x <= -2147483648.0f) return (int32_t)0x80000000u;
    return (int32_t)x;
}

// The handlers' exp approximation (:6627-6665, :6965-6989): 2^n injected as
// exponent bits (n + 127) << 23, n clamped below at -127 when `clamp`.
__device__ __forceinline__ float exp_poly_a(float x, bool clamp) {
    const float t = __fmul_rn(x, f_of(kLog2e));
    const float n = floorf(t);
    const float f = __fsub_rn(t, n);
    float p = __fmul_rn(f_of(kC4), f);
    p = __fadd_rn(p, f_of(kC3));
    p = __fmul_rn(p, f);
    p = __fadd_rn(p, f_of(kC2));
    p = __fmul_rn(p, f);
    p = __fadd_rn(p, f_of(kLn2));
    p = __fmul_rn(p, f);
    p = __fadd_rn(p, 1.0f);
    int32_t ni = cvtzs_a(n);
    if (clamp && ni < -127) ni = -127;
    return __fmul_rn(p, f_of(((uint32_t)ni + 127u) << 23));
}

__device__ __forceinline__ float silu_a(float x) {
    const float e = exp_poly_a(-x, true);
    const float d = __fadd_rn(e, 1.0f);
    float r = frecpe_a(d);
    r = __fmul_rn(r, frecps_a(d, r));
    r = __fmul_rn(r, frecps_a(d, r));
    return __fmul_rn(x, r);
}

// rope_fp32's theta^(2/dim) (:6725-6783).
__device__ float rope_ratio_a(uint32_t dim, float theta) {
    const uint32_t tb = __float_as_uint(theta);
    const int32_t e = (int32_t)((tb >> 23) & 0xff) - 127;
    const float fe = (float)e;
    const float m = f_of((tb & ~(0xffu << 23)) | (127u << 23));
    const float t = __fsub_rn(m, 1.0f);
    float l = __fmul_rn(f_of(0x3E943014u), t);
    l = __fadd_rn(l, f_of(0xBEFBD464u));
    l = __fmul_rn(l, t);
    l = __fadd_rn(l, f_of(0x3F7FF972u));
    l = __fmul_rn(l, t);
    float lt = __fmul_rn(fe, f_of(kLn2));
    lt = __fadd_rn(lt, l);
    float step = __fdiv_rn(2.0f, (float)dim);
    step = __fmul_rn(step, lt);
    return exp_poly_a(step, false);
}

// The rotation of pair p (:6827-6905): power = ratio^(p mod 16) by
// sequential products, times ratio^16 once per earlier 16-pair chunk.
__device__ __forceinline__ float2 rope_pair_a(float a, float b, uint32_t p, float ratio, float posf) {
    float power = 1.0f, r16 = 1.0f;
    for (uint32_t k = 0; k < 16; k++) {
        if (k == (p & 15)) power = r16;
        r16 = __fmul_rn(r16, ratio);
    }
    for (uint32_t c = 0; c < (p >> 4); c++) power = __fmul_rn(power, r16);
    const float freq = __fdiv_rn(posf, power);
    const float nq = __builtin_rintf(__fmul_rn(freq, f_of(0x3EA2F983u)));
    const uint32_t odd = ((uint32_t)cvtzs_a(nq) & 1u) << 31;
    const float r = __builtin_fmaf(-nq, f_of(0x40490FDBu), freq);
    const float r2 = __fmul_rn(r, r);
    float sn = f_of(0xB9500D01u);
    sn = __builtin_fmaf(sn, r2, f_of(0x3C088889u));
    sn = __builtin_fmaf(sn, r2, f_of(0xBE2AAAABu));
    sn = __builtin_fmaf(sn, r2, 1.0f);
    sn = __fmul_rn(sn, r);
    float cs = f_of(0xBAB60B61u);
    cs = __builtin_fmaf(cs, r2, f_of(0x3D2AAAABu));
    cs = __builtin_fmaf(cs, r2, -0.5f);
    cs = __builtin_fmaf(cs, r2, 1.0f);
    sn = f_of(__float_as_uint(sn) ^ odd);
    cs = f_of(__float_as_uint(cs) ^ odd);
    float oe = __fmul_rn(a, cs);
    oe = __builtin_fmaf(-b, sn, oe);
    float oo = __fmul_rn(b, cs);
    oo = __builtin_fmaf(a, sn, oo);
    return make_float2(oe, oo);
}

// NaN-propagating FMAX (AArch64, not FMAXNM): max(+0, -0) = +0.
__device__ __forceinline__ float fmax_nan(float a, float b) {
    if (a != a) return a;
    if (b != b) return b;
    if (a == b) return __float_as_uint(a) >> 31 ? b : a;
    return a > b ? a : b;
}

constexpr uint32_t kStageFloats = 8192;  // rows up to this long are held in registers and LDS

// chain l of a 16-lane accumulation over v[0..n): acc = op(v[i], acc) for
// i = l, l + 16, ... in order; 8 values are loaded ahead of each 8 steps.
// (Rows longer than kStageFloats, read from global memory.)
template <bool FMA_SQ>
__device__ __forceinline__ float chain16(const float* v, uint32_t n, uint32_t l) {
    float acc = 0.0f;
    uint32_t i = l;
    for (; i + 7 * 16 < n; i += 8 * 16) {
        float t[8];
#pragma unroll
        for (int k = 0; k < 8; k++) t[k] = v[i + 16 * k];
#pragma unroll
        for (int k = 0; k < 8; k++) acc = FMA_SQ ? __builtin_fmaf(t[k], t[k], acc) : __fadd_rn(acc, t[k]);
    }
    for (; i < n; i += 16) acc = FMA_SQ ? __builtin_fmaf(v[i], v[i], acc) : __fadd_rn(acc, v[i]);
    return acc;
}

// A row of up to kStageFloats values held by a workgroup of 256 threads:
// thread t keeps elements t + 256u (u < kItems) in registers, and the row
// is also written to LDS transposed by chain, element i at
// ct[(i % 16) * kChainStride + i / 16], so chain l reads its elements in
// order with 16-byte loads.  Slots from the row's end to the next multiple
// of 64 hold +0, which adds nothing to a chain (every chain's partial is
// +0 or positive: sums of squares, sums of exponentials).  kChainStride is 4
// mod 64 words, so the 16 chains' rows start in distinct 4-bank groups.
constexpr uint32_t kItems = kStageFloats / 256;
constexpr uint32_t kChainStride = kStageFloats / 16 + 4;

__device__ __forceinline__ void stage_chains(float* ct, uint32_t dim, const float (&v)[kItems]) {
    const uint32_t nz = (dim + 63) & ~63u;
#pragma unroll
    for (uint32_t u = 0; u < kItems; u++) {
        const uint32_t i = threadIdx.x + 256 * u;
        if (i < nz) ct[(i & 15) * kChainStride + (i >> 4)] = i < dim ? v[u] : 0.0f;
    }
}

template <bool FMA_SQ>
__device__ __forceinline__ float chain16_staged(const float* ct, uint32_t dim, uint32_t l) {
    const float4* c = reinterpret_cast<const float4*>(ct + l * kChainStride);
    const uint32_t n4 = (dim + 63) / 64;  // 4-element groups per chain, zero tail included
    float acc = 0.0f;
    auto step = [&](float t) { acc = FMA_SQ ? __builtin_fmaf(t, t, acc) : __fadd_rn(acc, t); };
    uint32_t q = 0;
    for (; q + 4 <= n4; q += 4) {
        float4 t[4];
#pragma unroll
        for (int k = 0; k < 4; k++) t[k] = c[q + k];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            step(t[k].x);
            step(t[k].y);
            step(t[k].z);
            step(t[k].w);
        }
    }
    for (; q < n4; q++) {
        const float4 t = c[q];
        step(t.x);
        step(t.y);
        step(t.z);
        step(t.w);
    }
    return acc;
}

// 1/sqrt(mean + eps) as 0x51 computes it from the FADDV of the chains.
__device__ __forceinline__ float rms_factor(float acc, uint32_t dim, float eps) {
    const float ss = faddv16(acc);
    const float mean = __fdiv_rn(ss, (float)dim);
    const float t = __fadd_rn(mean, eps);
    float r = frsqrte_a(t);
    float s = __fmul_rn(r, r);
    s = frsqrts_a(t, s);
    r = __fmul_rn(r, s);
    s = __fmul_rn(r, r);
    s = frsqrts_a(t, s);
    return __fmul_rn(r, s);
}

// f(u) for the items u of a staged row, in groups of 8 whose condition
// (the group holds an element of the row) is the same for the whole
// workgroup.  f loads element min(t + 256u, dim - 1) with no condition, so
// a group's loads are all in flight before the first is used.
template <class F>
__device__ __forceinline__ void for_item_groups(uint32_t dim, F&& f) {
#pragma unroll
    for (uint32_t g = 0; g < kItems / 8; g++) {
        if (g * 2048 < dim) {
#pragma unroll
            for (uint32_t k = 0; k < 8; k++) f(g * 8 + k);
        }
    }
}

__device__ __forceinline__ uint32_t item_index(uint32_t u, uint32_t dim) {
    const uint32_t i = threadIdx.x + 256 * u;
    return i < dim ? i : dim - 1;
}

// 0x51 over one row, by one workgroup (256 threads).  Every lane of wave 0
// runs chain lane & 15 (four copies of the 16 chains), so the FADDV tree
// reads only active DPP rows.  HAS_W: weights w (else 1.0f, unit weights).
// HAS_Y: the row is fl(x + y) (a residual add), written back to xsum.  o
// may alias x.
template <bool HAS_W, bool HAS_Y>
__device__ __forceinline__ void rms_norm_row(uint32_t dim, float eps, const float* x, const float* w, float* o,
                                             const float* y, float* xsum) {
    __shared__ float rs;
    __shared__ __attribute__((aligned(16))) float ct[16 * kChainStride];
    const uint32_t t = threadIdx.x;
    if (dim <= kStageFloats) {
        float v[kItems], wv[kItems], yv[kItems];
#pragma unroll
        for (uint32_t u = 0; u < kItems; u++) v[u] = wv[u] = yv[u] = 0.0f;
        for_item_groups(dim, [&](uint32_t u) {
            const uint32_t i = item_index(u, dim);
            v[u] = x[i];
            if (HAS_W) wv[u] = w[i];
            if (HAS_Y) yv[u] = y[i];
        });
        if (HAS_Y) {
#pragma unroll
            for (uint32_t u = 0; u < kItems; u++) v[u] = __fadd_rn(v[u], yv[u]);
        }
        stage_chains(ct, dim, v);
        __syncthreads();
        if (t < 64) {
            const float r = rms_factor(chain16_staged<true>(ct, dim, t & 15), dim, eps);
            if (t == 0) rs = r;
        }
        __syncthreads();
        const float r = rs;
#pragma unroll
        for (uint32_t u = 0; u < kItems; u++) {
            const uint32_t i = t + 256 * u;
            if (i < dim) {
                o[i] = __fmul_rn(__fmul_rn(v[u], r), HAS_W ? wv[u] : 1.0f);
                if (HAS_Y) xsum[i] = v[u];
            }
        }
        return;
    }
    // longer rows: chains over global memory (the sum, if any, written first)
    if (HAS_Y) {
        for (uint32_t i = t; i < dim; i += 256) xsum[i] = __fadd_rn(x[i], y[i]);
        __threadfence_block();
        __syncthreads();
        x = xsum;
    }
    if (t < 64) {
        const float r = rms_factor(chain16<true>(x, dim, t & 15), dim, eps);
        if (t == 0) rs = r;
    }
    __syncthreads();
    const float r = rs;
    for (uint32_t i = t; i < dim; i += 256) o[i] = __fmul_rn(__fmul_rn(x[i], r), HAS_W ? w[i] : 1.0f);
}

__global__ void __launch_bounds__(256)
k_rms_norm_ref(uint32_t dim, float eps, const float* in, const float* __restrict__ w, float* out, uint64_t stride) {
    rms_norm_row<true, false>(dim, eps, in + blockIdx.x * stride, w, out + blockIdx.x * stride, nullptr, nullptr);
}

// x = fl(x + y), xn = 0x51(x) with weights w: one row (the residual add of
// the reference-arithmetic decode, then its norm).
__global__ void __launch_bounds__(256)
k_add_rms_norm_ref(uint32_t dim, float eps, float* x, const float* __restrict__ y, const float* __restrict__ w,
                   float* __restrict__ xn) {
    rms_norm_row<true, true>(dim, eps, x, w, xn, y, x);
}

__global__ void __launch_bounds__(256) k_silu_ref(uint64_t n, const float* __restrict__ in, float* __restrict__ out) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = silu_a(in[i]);
}

// 0x55 over `rows` rows of dim floats (row stride `stride` floats), one
// thread per pair.
__global__ void __launch_bounds__(256)
k_rope_ref(uint32_t rows, uint32_t dim, uint32_t pos, float theta, const float* __restrict__ in,
           float* __restrict__ out, uint64_t stride) {
    const uint32_t pairs = dim / 2;
    const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= (uint64_t)rows * pairs) return;
    const uint32_t row = (uint32_t)(t / pairs), p = (uint32_t)(t - (uint64_t)row * pairs);
    const float ratio = rope_ratio_a(dim, theta);
    const float* x = in + row * stride;
    const float2 v = rope_pair_a(x[2 * p], x[2 * p + 1], p, ratio, (float)pos);
    float* o = out + row * stride;
    o[2 * p] = v.x;
    o[2 * p + 1] = v.y;
}

// 0x56 over one row, by one workgroup: the max (any order: max is exact),
// e = exp(x - max), the 16 fadd chains (in wave 0, four copies), FADDV,
// 1/sum, fl(e * inv).  A dim that is not a multiple of 16 leaves the last
// chains shorter.  o may alias x.  NODE (ggml's SOFT_MAX): the values are
// fl(fl(x * scale) + m) (m from mrow, or no add when mrow is null), and an
// element whose x - max is -inf gives e = 0 (the polynomial would give NaN
// there: floor(-inf) - -inf).
template <bool NODE>
__device__ __forceinline__ void softmax_row(uint32_t dim, const float* x, float* o, float scale, const float* mrow) {
    __shared__ float red[4];
    __shared__ float sinv;
    __shared__ __attribute__((aligned(16))) float ct[16 * kChainStride];
    const uint32_t t = threadIdx.x;
    auto val = [&](uint32_t i) {
        if (!NODE) return x[i];
        const float v = __fmul_rn(x[i], scale);
        return mrow ? __fadd_rn(v, mrow[i]) : v;
    };
    auto expd = [&](float v, float m) {
        const float d = __fsub_rn(v, m);
        return NODE && d == -__builtin_inff() ? 0.0f : exp_poly_a(d, true);
    };
    auto max_of = [&](float m) {
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) m = fmax_nan(m, __shfl_xor(m, off, 64));
        if ((t & 63) == 0) red[t >> 6] = m;
        __syncthreads();
        return fmax_nan(fmax_nan(red[0], red[1]), fmax_nan(red[2], red[3]));
    };
    auto inv_of = [&](float acc) {
        if (t < 64) {
            const float inv = __fdiv_rn(1.0f, faddv16(acc));
            if (t == 0) sinv = inv;
        }
        __syncthreads();
        return sinv;
    };
    if (dim <= kStageFloats) {
        float v[kItems];
        float m = -__builtin_inff();
#pragma unroll
        for (uint32_t u = 0; u < kItems; u++) v[u] = 0.0f;
        for_item_groups(dim, [&](uint32_t u) { v[u] = val(item_index(u, dim)); });
#pragma unroll
        for (uint32_t u = 0; u < kItems; u++)
            if (t + 256 * u < dim) m = fmax_nan(m, v[u]);
        m = max_of(m);
#pragma unroll
        for (uint32_t u = 0; u < kItems; u++)
            if (t + 256 * u < dim) v[u] = expd(v[u], m);
        stage_chains(ct, dim, v);
        __syncthreads();
        const float inv = inv_of(t < 64 ? chain16_staged<false>(ct, dim, t & 15) : 0.0f);
#pragma unroll
        for (uint32_t u = 0; u < kItems; u++)
            if (t + 256 * u < dim) o[t + 256 * u] = __fmul_rn(v[u], inv);
        return;
    }
    // longer rows: e through o in global memory
    float m = -__builtin_inff();
    for (uint32_t i = t; i < dim; i += 256) m = fmax_nan(m, val(i));
    m = max_of(m);
    for (uint32_t i = t; i < dim; i += 256) o[i] = expd(val(i), m);
    __threadfence_block();
    __syncthreads();
    const float inv = inv_of(t < 64 ? chain16<false>(o, dim, t & 15) : 0.0f);
    for (uint32_t i = t; i < dim; i += 256) o[i] = __fmul_rn(o[i], inv);
}

__global__ void __launch_bounds__(256) k_softmax_ref(uint32_t dim, const float* in, float* out, uint64_t stride) {
    softmax_row<false>(dim, in + blockIdx.x * stride, out + blockIdx.x * stride, 1.0f, nullptr);
}

// ------------------------------------------------------ ggml node forms
// One workgroup per row of the node (ggml_rows.hpp); the rows' operands
// may sit anywhere their strides put them.
__global__ void __launch_bounds__(256)
k_rms_norm_node(uint32_t dim, float eps, const uint8_t* in, NodeRows src, uint8_t* out, NodeRows dst) {
    const RowIdx i = row_index(dst, blockIdx.x);
    rms_norm_row<false, false>(dim, eps, reinterpret_cast<const float*>(in + row_offset(src, i)), nullptr,
                               reinterpret_cast<float*>(out + row_offset(dst, i)), nullptr, nullptr);
}

__global__ void __launch_bounds__(256)
k_softmax_node(uint32_t dim, float scale, const uint8_t* in, NodeRows src, const uint8_t* mask, NodeRows msk,
               uint8_t* out, NodeRows dst) {
    const RowIdx i = row_index(dst, blockIdx.x);
    softmax_row<true>(dim, reinterpret_cast<const float*>(in + row_offset(src, i)),
                      reinterpret_cast<float*>(out + row_offset(dst, i)), scale,
                      mask ? reinterpret_cast<const float*>(mask + row_offset(msk, i)) : nullptr);
}

// One thread per pair, grid-stride over rows * dim/2 pairs.  Both values of
// a pair are read before either is written, so out may alias in.
__global__ void __launch_bounds__(256)
k_rope_node(uint32_t dim, uint64_t total, float theta, const int32_t* __restrict__ pos, const uint8_t* in,
            NodeRows src, uint8_t* out, NodeRows dst) {
    const uint32_t pairs = dim / 2;
    const float ratio = rope_ratio_a(dim, theta);
    for (uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += (uint64_t)gridDim.x * 256) {
        const uint64_t row = t / pairs;
        const uint32_t p = (uint32_t)(t - row * pairs);
        const RowIdx i = row_index(dst, row);
        const float* x = reinterpret_cast<const float*>(in + row_offset(src, i));
        float* o = reinterpret_cast<float*>(out + row_offset(dst, i));
        const float2 v = rope_pair_a(x[2 * p], x[2 * p + 1], p, ratio, (float)pos[i.i2]);
        o[2 * p] = v.x;
        o[2 * p + 1] = v.y;
    }
}

__device__ __forceinline__ uint16_t f16_bits(float f) {
    const _Float16 h = (_Float16)f;  // v_cvt_f16_f32, round to nearest even
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

// ---------------------------------------------------- decode steps (reference mode)
// RoPE (0x55 arithmetic, dim 128) of the q and k heads of the qkv vector at
// pos: q rotated in place, k rotated and appended to the fp16 cache, v
// appended.  One thread per pair (q and k heads) or per v element.
__global__ void __launch_bounds__(256)
k_rope_ref_kv(float* __restrict__ qkv, uint32_t n_heads, uint32_t n_kv, uint32_t pos, uint32_t ctx, float theta,
              uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache) {
    const uint32_t t = blockIdx.x * 256 + threadIdx.x;
    const uint32_t nrot = (n_heads + n_kv) * 64, nv = n_kv * 128;
    if (t < nrot) {
        const uint32_t head = t / 64, p = t % 64;
        float* x = qkv + head * 128;
        const float2 v = rope_pair_a(x[2 * p], x[2 * p + 1], p, rope_ratio_a(128, theta), (float)pos);
        if (head < n_heads) {
            x[2 * p] = v.x;
            x[2 * p + 1] = v.y;
        } else {
            uint16_t* kc = k_cache + ((uint64_t)(head - n_heads) * ctx + pos) * 128;
            kc[2 * p] = f16_bits(v.x);
            kc[2 * p + 1] = f16_bits(v.y);
        }
    } else if (t < nrot + nv) {
        const uint32_t i = t - nrot, g = i / 128, d = i % 128;
        v_cache[((uint64_t)g * ctx + pos) * 128 + d] = f16_bits(qkv[(n_heads + n_kv) * 128 + i]);
    }
}

__device__ __forceinline__ float h2f(uint16_t h) { return half_bits_to_float(h); }

// s[h][j] = fl(dot16(q_h, k_j) * fl(1/sqrt(128))): 16 chains of 8 fmas
// (chain l over elements l, l + 16, ... in order), then the FADDV tree in
// registers.  One workgroup per (kv head g, block of kScRows positions):
// the block's K rows are copied global -> LDS (row r's 16-byte piece c at
// slot c ^ (r mod 16), so the 16 rows a ds_read_b128 serves sit in distinct
// banks) with the group's q rows; thread t takes position j0 + t % kScRows
// for the group's query heads 2(t / kScRows) and 2(t / kScRows) + 1,
// holding its K row in registers.
constexpr uint32_t kScRows = 128, kScHeads = 4;
__global__ void __launch_bounds__(256)
k_attn_scores_ref(uint32_t len, uint32_t ctx, const float* __restrict__ q, const uint16_t* __restrict__ k_cache,
                  float* __restrict__ s) {
    __shared__ __attribute__((aligned(16))) uint16_t ks[kScRows * 128];  // 32 KB
    __shared__ __attribute__((aligned(16))) float qs[kScHeads * 128];     // 2 KB
    const uint32_t nblk = (len + kScRows - 1) / kScRows;
    const uint32_t g = blockIdx.x / nblk, j0 = (blockIdx.x % nblk) * kScRows;
    const uint32_t t = threadIdx.x;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
    const uint32_t nrows = len - j0 < kScRows ? len - j0 : kScRows;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(k_cache + ((uint64_t)g * ctx + j0) * 128, nrows * 256);
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(q + (uint64_t)g * kScHeads * 128, kScHeads * 128 * 4);
#pragma unroll
    for (uint32_t i = wave; i < kScRows / 4; i += 4) {  // 4 rows per wave-instruction; rows past len -> zeros
        const uint32_t r = 4 * i + lane / 16, c = (lane & 15) ^ (r & 15);
        copy16_to_lds(rk, reinterpret_cast<int8_t*>(ks) + 1024 * i, r * 256 + c * 16);
    }
#pragma unroll
    for (uint32_t i = wave; i < kScHeads * 128 / 64; i += 4) copy4_to_lds(rq, qs + 64 * i, (64 * i + lane) * 4);
    wait_vmcnt<0>();
    __syncthreads();
    const uint32_t r = t % kScRows, hp = t / kScRows, j = j0 + r;
    v4i kr[16];  // this row's 128 halves, piece c = elements 8c .. 8c + 7
#pragma unroll
    for (uint32_t c = 0; c < 16; c++) kr[c] = *reinterpret_cast<const v4i*>(ks + r * 128 + ((c ^ (r & 15)) * 8));
    auto kv = [&](uint32_t e) {  // element e of the row, as fp32
        const uint32_t w = (uint32_t)kr[e / 8][(e % 8) / 2];
        return h2f((uint16_t)((e & 1) ? (w >> 16) : (w & 0xffff)));
    };
#pragma unroll
    for (uint32_t hh = 2 * hp; hh < 2 * hp + 2; hh++) {
        const float* qh = qs + hh * 128;
        float acc[16];
#pragma unroll
        for (int l = 0; l < 16; l++) acc[l] = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < 8; i++) {
            float4 qv[4];
#pragma unroll
            for (int k = 0; k < 4; k++) qv[k] = *reinterpret_cast<const float4*>(qh + 16 * i + 4 * k);
#pragma unroll
            for (uint32_t l = 0; l < 16; l++) {
                const float4& v = qv[l / 4];
                const float qe = (l % 4) == 0 ? v.x : (l % 4) == 1 ? v.y : (l % 4) == 2 ? v.z : v.w;
                acc[l] = __builtin_fmaf(qe, kv(16 * i + l), acc[l]);
            }
        }
        float t8[8], t4[4];
#pragma unroll
        for (int l = 0; l < 8; l++) t8[l] = __fadd_rn(acc[2 * l], acc[2 * l + 1]);
#pragma unroll
        for (int l = 0; l < 4; l++) t4[l] = __fadd_rn(t8[2 * l], t8[2 * l + 1]);
        const float dot = __fadd_rn(__fadd_rn(t4[0], t4[1]), __fadd_rn(t4[2], t4[3]));
        if (j < len) s[(uint64_t)(g * kScHeads + hh) * len + j] = __fmul_rn(dot, f_of(0x3DB504F3u));
    }
}

// out[h][d] = FADDV over 16 chains, chain l = fma(p_j, v_j[d], acc) for
// j = l mod 16 in increasing j.  One workgroup per (kv head g, block of 16
// dimensions, query head hq of the group): thread t runs chain l = t / 16
// of dimension d = t % 16.  Positions pass through LDS in chunks of up to
// kPvChunk (4096: the whole context of config 5 in one chunk), the V rows'
// 32-byte slices as 16-byte pieces and the P row as dwords, copied global
// -> LDS directly (positions at or past len read as zeros and are never
// folded); one wait and one barrier per chunk.  Each chain folds its
// positions in batches of 8, the next batch's LDS reads in flight during the
// current batch's fmas (two register sets in turn).  The 16 chains of a
// dimension meet through LDS for the FADDV tree.
// SOFTMAX (len <= kPvChunk): p holds the raw scores and the workgroup
// turns its head's row into probabilities in LDS first, exactly as 0x56
// does (softmax_row: any-order max, e = exp(s - max), 16 fadd chains in
// wave 0, FADDV, 1/sum, fl(e * inv)); every workgroup of the head computes
// the same row.
constexpr uint32_t kPvHeads = 4, kPvChunk = 4096, kPvBatch = 8;
template <bool SOFTMAX>
__global__ void __launch_bounds__(256)
k_attn_pv_ref(uint32_t len, uint32_t ctx, const float* __restrict__ p, const uint16_t* __restrict__ v_cache,
              float* __restrict__ out) {
    __shared__ __attribute__((aligned(16))) uint16_t vs[kPvChunk * 16];  // 128 KB
    __shared__ __attribute__((aligned(16))) float ps[kPvChunk];          // 16 KB
    __shared__ float red[256];
    const uint32_t hq = blockIdx.x % kPvHeads, db = (blockIdx.x / kPvHeads) & 7, g = blockIdx.x / (kPvHeads * 8);
    const uint32_t t = threadIdx.x, l = t >> 4, d = t & 15;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
    const uint16_t* vg = v_cache + (uint64_t)g * ctx * 128 + db * 16;
    const float* pg = p + (uint64_t)(g * kPvHeads + hq) * len;
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vg, len * 256);
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(pg, len * 4);
    const uint32_t nch = (len + kPvChunk - 1) / kPvChunk;
    float acc = 0.0f;
    for (uint32_t c = 0; c < nch; c++) {
        const uint32_t j0 = c * kPvChunk, nj = min(kPvChunk, len - j0);
        if (c > 0) __syncthreads();  // everyone is done with the previous chunk
        // P first (the softmax needs it before the V rows): 64 positions per
        // wave-instruction.  V: piece q of the chunk = row q / 2, half q % 2;
        // 64 pieces (1 KB of LDS) per wave-instruction.
        for (uint32_t i = wave; i < (nj + 63) / 64; i += 4) {
            const uint32_t j = j0 + 64 * i + lane;
            copy4_to_lds(rp, ps + 64 * i, j < len ? j * 4 : 0x80000000u);
        }
        if (SOFTMAX) {  // the row is needed first; V lands while it is computed
            wait_vmcnt<0>();
            __syncthreads();
        }
        for (uint32_t i = wave; i < (nj * 2 + 63) / 64; i += 4) {
            const uint32_t q = 64 * i + lane, j = j0 + (q >> 1);
            copy16_to_lds(rv, reinterpret_cast<int8_t*>(vs) + 1024 * i,
                          j < len ? j * 256 + (q & 1) * 16 : 0x80000000u);
        }
        if (SOFTMAX) {
            float m = -__builtin_inff();
            for (uint32_t j = t; j < nj; j += 256) m = fmax_nan(m, ps[j]);
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) m = fmax_nan(m, __shfl_xor(m, off, 64));
            if (lane == 0) red[wave] = m;
            wait_lgkmcnt0();  // LDS-only barriers here: the V copies stay in flight
            lds_barrier();
            m = fmax_nan(fmax_nan(red[0], red[1]), fmax_nan(red[2], red[3]));
            for (uint32_t j = t; j < nj; j += 256) ps[j] = exp_poly_a(__fsub_rn(ps[j], m), true);
            wait_lgkmcnt0();
            lds_barrier();
            if (t < 64) {
                const float inv = __fdiv_rn(1.0f, faddv16(chain16<false>(ps, nj, t & 15)));
                if (t == 0) red[4] = inv;
            }
            wait_lgkmcnt0();
            lds_barrier();
            const float inv = red[4];
            for (uint32_t j = t; j < nj; j += 256) ps[j] = __fmul_rn(ps[j], inv);
        }
        wait_vmcnt<0>();  // this wave's copies landed
        __syncthreads();  // everyone's did
        auto ld = [&](float (&pq)[kPvBatch], uint16_t (&vq)[kPvBatch], uint32_t k0) {
#pragma unroll
            for (uint32_t u = 0; u < kPvBatch; u++) {
                pq[u] = ps[k0 + 16 * u];
                vq[u] = vs[(k0 + 16 * u) * 16 + d];
            }
        };
        auto fold = [&](const float (&pq)[kPvBatch], const uint16_t (&vq)[kPvBatch]) {
#pragma unroll
            for (uint32_t u = 0; u < kPvBatch; u++) acc = __builtin_fmaf(pq[u], h2f(vq[u]), acc);
        };
        // chain l holds positions l + 16 m, m < cnt; nb full batches of 8
        const uint32_t cnt = l < nj ? (nj - l + 15) / 16 : 0, nb = cnt / kPvBatch;
        float pa[kPvBatch], pb[kPvBatch];
        uint16_t va[kPvBatch], vb[kPvBatch];
        if (nb > 0) ld(pa, va, l);
        for (uint32_t bt = 0; bt < nb; bt += 2) {
            if (bt + 1 < nb) ld(pb, vb, l + 16 * kPvBatch * (bt + 1));
            fold(pa, va);
            if (bt + 2 < nb) ld(pa, va, l + 16 * kPvBatch * (bt + 2));
            if (bt + 1 < nb) fold(pb, vb);
        }
        for (uint32_t k = l + 16 * kPvBatch * nb; k < nj; k += 16) acc = __builtin_fmaf(ps[k], h2f(vs[k * 16 + d]), acc);
    }
    __syncthreads();  // red's softmax slots are read before the chains' partials overwrite them
    red[d * 16 + l] = acc;
    __syncthreads();
    const float v = faddv16(red[t]);  // lanes t..t+15 hold the 16 chains of dimension t / 16
    if ((t & 15) == 0) out[(uint64_t)(g * kPvHeads + hq) * 128 + db * 16 + (t >> 4)] = v;
}

// h[i] = fl(silu_fp32(g_i) * u_i) on gate|up interleaved in 32-row groups.
__global__ void __launch_bounds__(256)
k_silu_mul_ref_il(uint32_t F, const float* __restrict__ gu, float* __restrict__ h) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= F) return;
    const uint32_t b = 64 * (i / 32) + (i % 32);
    h[i] = __fmul_rn(silu_a(gu[b]), gu[b + 32]);
}

}  // namespace

// ------------------------------------------------------------- launchers
int rms_norm_ref_launch(uint32_t rows, uint32_t dim, float eps, const float* in, const float* w, float* out,
                        uint64_t stride, hipStream_t s) {
    if (rows == 0 || dim == 0) return ANE_OK;
    if (rows > 0x7fffffffu) return ANE_ERR_INVALID_ARG;
    hipLaunchKernelGGL(k_rms_norm_ref, dim3(rows), dim3(256), 0, s, dim, eps, in, w, out, stride);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

// x = fl(x + y) (written back), xn = rms_norm_fp32(x) with weights w: one
// row of dim values.
int add_rms_norm_ref_launch(uint32_t dim, float eps, float* x, const float* y, const float* w, float* xn,
                            hipStream_t s) {
    if (dim == 0) return ANE_OK;
    hipLaunchKernelGGL(k_add_rms_norm_ref, dim3(1), dim3(256), 0, s, dim, eps, x, y, w, xn);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

int softmax_ref_launch(uint32_t rows, uint32_t dim, const float* in, float* out, uint64_t stride, hipStream_t s) {
    if (rows == 0 || dim == 0) return ANE_OK;
    if (rows > 0x7fffffffu) return ANE_ERR_INVALID_ARG;
    hipLaunchKernelGGL(k_softmax_ref, dim3(rows), dim3(256), 0, s, dim, in, out, stride);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

int rope_ref_kv_launch(float* qkv, uint32_t n_heads, uint32_t n_kv, uint32_t pos, uint32_t ctx, float theta,
                       uint16_t* kc, uint16_t* vc, hipStream_t s) {
    const uint32_t n = (n_heads + n_kv) * 64 + n_kv * 128;
    hipLaunchKernelGGL(k_rope_ref_kv, dim3((n + 255) / 256), dim3(256), 0, s, qkv, n_heads, n_kv, pos, ctx, theta,
                       kc, vc);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

// Reference-mode attention over positions 0..len-1: scores, softmax_fp32
// per head, then P.V.  ws holds n_heads * len floats of scores and as many
// of probabilities.
int attention_ref_launch(uint32_t n_heads, uint32_t n_kv, uint32_t len, uint32_t ctx, const float* q,
                         const uint16_t* kc, const uint16_t* vc, float* out, float* ws, hipStream_t s) {
    const uint32_t group = n_heads / n_kv;
    if (group != kPvHeads || group != kScHeads || n_heads != group * n_kv) return ANE_ERR_INVALID_ARG;
    float* sc = ws;
    float* pr = ws + (uint64_t)n_heads * len;
    hipLaunchKernelGGL(k_attn_scores_ref, dim3(n_kv * ((len + kScRows - 1) / kScRows)), dim3(256), 0, s, len, ctx,
                       q, kc, sc);
    if (len <= kPvChunk) {  // the softmax inside the P.V workgroups
        hipLaunchKernelGGL(k_attn_pv_ref<true>, dim3(n_kv * 8 * kPvHeads), dim3(256), 0, s, len, ctx, sc, vc, out);
    } else {
        hipLaunchKernelGGL(k_softmax_ref, dim3(n_heads), dim3(256), 0, s, len, sc, pr, (uint64_t)len);
        hipLaunchKernelGGL(k_attn_pv_ref<false>, dim3(n_kv * 8 * kPvHeads), dim3(256), 0, s, len, ctx, pr, vc, out);
    }
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

int rms_norm_node_launch(uint32_t dim, uint64_t rows, float eps, const uint8_t* in, const NodeRows& src,
                         uint8_t* out, const NodeRows& dst, hipStream_t s) {
    if (rows == 0 || dim == 0) return ANE_OK;
    if (rows > 0x7fffffffu) return ANE_ERR_INVALID_ARG;
    hipLaunchKernelGGL(k_rms_norm_node, dim3((uint32_t)rows), dim3(256), 0, s, dim, eps, in, src, out, dst);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

int softmax_node_launch(uint32_t dim, uint64_t rows, float scale, const uint8_t* in, const NodeRows& src,
                        const uint8_t* mask, const NodeRows& msk, uint8_t* out, const NodeRows& dst, hipStream_t s) {
    if (rows == 0 || dim == 0) return ANE_OK;
    if (rows > 0x7fffffffu) return ANE_ERR_INVALID_ARG;
    hipLaunchKernelGGL(k_softmax_node, dim3((uint32_t)rows), dim3(256), 0, s, dim, scale, in, src, mask, msk, out,
                       dst);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

int rope_node_launch(uint32_t dim, uint64_t rows, float theta, const int32_t* pos, const uint8_t* in,
                     const NodeRows& src, uint8_t* out, const NodeRows& dst, hipStream_t s) {
    const uint64_t total = rows * (dim / 2);
    if (total == 0) return ANE_OK;
    uint64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_rope_node, dim3((uint32_t)blocks), dim3(256), 0, s, dim, total, theta, pos, in, src, out,
                       dst);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

int silu_mul_ref_il_launch(uint32_t F, const float* gu, float* h, hipStream_t s) {
    hipLaunchKernelGGL(k_silu_mul_ref_il, dim3((F + 255) / 256), dim3(256), 0, s, F, gu, h);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

}  // namespace ane

using namespace ane;

extern "C" int ane_hip_rms_norm_fp32(uint32_t rows, uint32_t dim, float eps, const float* in, const float* w,
                                     float* out, void* stream) {
    if (rows == 0 || dim == 0) return ANE_OK;
    if (!in || !w || !out) return ANE_ERR_BAD_POINTER;
    return rms_norm_ref_launch(rows, dim, eps, in, w, out, dim, (hipStream_t)stream);
}

extern "C" int ane_hip_silu_fp32(uint64_t count, const float* in, float* out, void* stream) {
    if (count == 0) return ANE_OK;
    if (!in || !out) return ANE_ERR_BAD_POINTER;
    const uint64_t blocks = (count + 255) / 256;
    if (blocks > 0x7fffffffull) return ANE_ERR_INVALID_ARG;
    hipLaunchKernelGGL(k_silu_ref, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, count, in, out);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

extern "C" int ane_hip_rope_fp32(uint32_t rows, uint32_t dim, uint32_t pos, float theta, const float* in, float* out,
                                 void* stream) {
    const uint64_t n = (uint64_t)rows * (dim / 2);
    if (n == 0) return ANE_OK;
    if (!in || !out) return ANE_ERR_BAD_POINTER;
    if ((n + 255) / 256 > 0x7fffffffull) return ANE_ERR_INVALID_ARG;
    hipLaunchKernelGGL(k_rope_ref, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, rows, dim,
                       pos, theta, in, out, (uint64_t)dim);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

extern "C" int ane_hip_softmax_fp32(uint32_t rows, uint32_t dim, const float* in, float* out, void* stream) {
    if (rows == 0 || dim == 0) return ANE_OK;
    if (!in || !out) return ANE_ERR_BAD_POINTER;
    return softmax_ref_launch(rows, dim, in, out, dim, (hipStream_t)stream);
}
