// decode.hip -- single-token decode of a Llama-shaped model: the steps
// around the Q8_0 matrix products (RoPE + KV append, GQA attention over the
// fp16 cache, SiLU * up) and the per-token driver ane_decode_token.
//
// Matrix products run on the Q8_0 streaming kernel of q8_0.hip with the
// steps around them fused in, so a layer is six launches:
//   qkv       RMSNorm in the activation prologue
//   attention partial: RoPE of q and k and the fp16 KV append fused
//   attention merge, which also writes the output's Q8 activation form
//   o         on that Q8 form, residual add in the epilogue
//   gate|up   RMSNorm prologue, SiLU * up quantized to the Q8 form in the
//             epilogue (gate and up rows interleaved in 32-row groups)
//   down      on that Q8 form, residual add in the epilogue
//
// Attention is split over the context in chunks of ANE_ATTN_CHUNK positions
// (flash-decoding): one workgroup per (kv head, chunk) reads that chunk's K
// and V rows once for all G = n_heads / n_kv_heads query heads of the group,
// keeps per-head max / sum / output, and the merge kernel combines the
// chunks with the usual exp(m_c - M) rescaling.
#include <hip/hip_runtime.h>
#include <math.h>

#include "../../include/ane_decode.h"
#include "../../include/ggml-ane-hip.h"
#include "common.hpp"

namespace ane {
namespace {

constexpr int kHD = 128;     // head_dim
#ifndef ANE_ATTN_CHUNK
#define ANE_ATTN_CHUNK 64
#endif
constexpr int kChunk = ANE_ATTN_CHUNK;  // context positions per attention workgroup
static_assert(kChunk % 16 == 0 && kChunk <= 128, "chunk: a multiple of 16 positions, at most 128");
constexpr int kGroup = 4;    // query heads per kv head (one wave each in the softmax)

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    const _Float16 h = (_Float16)f;  // v_cvt_f16_f32, round to nearest even
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

// Threads [0, nq*64) rotate q pairs in place, [nq*64, (nq+nkv)*64) rotate k
// pairs into the k cache, the next nkv*128 copy v into the v cache.
__global__ void __launch_bounds__(256)
k_rope_kv_append(float* __restrict__ qkv, uint32_t nq, uint32_t nkv, const float* __restrict__ cs,
                 uint32_t pos, uint32_t ctx, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    const uint32_t qpairs = nq * (kHD / 2), kpairs = nkv * (kHD / 2), vel = nkv * kHD;
    if (i < qpairs + kpairs) {
        const bool isq = i < qpairs;
        const uint32_t pi = isq ? i : i - qpairs;
        const uint32_t head = pi / (kHD / 2), pr = pi % (kHD / 2);
        float* src = qkv + (isq ? 0 : nq * kHD) + head * kHD + 2 * pr;
        const float c = cs[2 * pr], s = cs[2 * pr + 1];
        const float a = src[0], b = src[1];
        const float o0 = __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, s));
        const float o1 = __fadd_rn(__fmul_rn(a, s), __fmul_rn(b, c));
        if (isq) {
            src[0] = o0;
            src[1] = o1;
        } else {
            uint16_t* dst = kc + ((uint64_t)head * ctx + pos) * kHD + 2 * pr;
            dst[0] = f32_to_f16_bits(o0);
            dst[1] = f32_to_f16_bits(o1);
        }
    } else if (i < qpairs + kpairs + vel) {
        const uint32_t vi = i - qpairs - kpairs;
        const uint32_t head = vi / kHD, d = vi % kHD;
        vc[((uint64_t)head * ctx + pos) * kHD + d] = f32_to_f16_bits(qkv[(nq + nkv) * kHD + vi]);
    }
}

// Wave-wide max / sum: DPP within each 16-lane row, then the four row
// results read out with v_readlane (no LDS round trips).
__device__ __forceinline__ float wave_max_f32(float v) {
    v = fmaxf(v, dpp_f32<kDppQuadXor1>(v));
    v = fmaxf(v, dpp_f32<kDppQuadXor2>(v));
    v = fmaxf(v, dpp_f32<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_f32<kDppRowMirror>(v));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
__device__ __forceinline__ float wave_sum_f32(float v) {
    v = faddv16(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

// One workgroup (4 waves) per (kv head g, chunk c of kChunk positions).
//  loads: the small operands first (q slices, RoPE row, this token's k and v
//         slices), then every K and V row of the chunk (positions past `len`
//         read a clamped valid row; their probability and value are zeroed),
//         all unconditional, so scores start once K has landed while V is
//         still in flight;
//  scores: 16 lanes per position (8 dims each, one 16-byte K load), 4
//          positions per wave per step, all 4 query heads of the group;
//  softmax: wave w takes head w over the chunk's positions;
//  values: lane owns dims 2l, 2l+1; wave w sums a quarter of the positions;
//          the four waves' partial outputs are added in LDS;
//  output: (max, sum, unnormalised output) of the chunk per head, merged by
//          k_attn_combine with exp(m_c - M) rescaling.
// ROPE: q and k come unrotated from qkv and are rotated here with the table
// row of `pos` (the same fp32 operations as k_rope_kv_append); position pos
// = len-1 uses this token's k and v (rounded to fp16, as the cache holds
// them), which the workgroup holding pos also writes to the caches.
__device__ __forceinline__ void rope_pair(float a, float b, float c, float s, float& o0, float& o1) {
    o0 = __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, s));
    o1 = __fadd_rn(__fmul_rn(a, s), __fmul_rn(b, c));
}

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    return (uint32_t)f32_to_f16_bits(a) | ((uint32_t)f32_to_f16_bits(b) << 16);
}

template <bool ROPE>
__global__ void __launch_bounds__(256)
k_attention(const float* __restrict__ q, const float* __restrict__ cs, uint16_t* kc, uint16_t* vc,
            uint32_t len, uint32_t ctx, uint32_t nq, uint32_t nkv, uint32_t nch, float scale,
            float* __restrict__ po, float* __restrict__ pml) {
    __shared__ float sc[kGroup][kChunk];
    __shared__ float red[4][kGroup][kHD];
    const uint32_t g = blockIdx.x, c = blockIdx.y;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, sub = lane & 15;
    const uint32_t j0 = c * kChunk;
    const uint32_t pos = len - 1;

    // ---- small operands
    float4 qa[kGroup], qb[kGroup];
#pragma unroll
    for (int h = 0; h < kGroup; h++) {
        const float* qh = q + (g * kGroup + h) * kHD + sub * 8;
        qa[h] = *reinterpret_cast<const float4*>(qh);
        qb[h] = *reinterpret_cast<const float4*>(qh + 4);
    }
    float4 csa = make_float4(0, 0, 0, 0), csb = csa, ka = csa, kb = csa;
    float2 vv = make_float2(0, 0);
    if (ROPE) {
        csa = *reinterpret_cast<const float4*>(cs + 8 * sub);      // (cos, sin) of pairs 4sub, 4sub+1
        csb = *reinterpret_cast<const float4*>(cs + 8 * sub + 4);  // pairs 4sub+2, 4sub+3
        const float* kh = q + nq * kHD + g * kHD + sub * 8;
        ka = *reinterpret_cast<const float4*>(kh);
        kb = *reinterpret_cast<const float4*>(kh + 4);
        vv = *reinterpret_cast<const float2*>(q + (nq + nkv) * kHD + g * kHD + 2 * lane);
    }

    // ---- every K and V row of the chunk (non-temporal loads: the cache is
    // streamed once per token).  The loads stay in this order (small
    // operands, K, V): vector-memory loads complete in order, so a score
    // waits only for its K row and the loads before it, while V lands
    // during the scores and the softmax; left free, the scheduler put V
    // (and part of q) ahead of K.
    __builtin_amdgcn_sched_barrier(0);
    uint4 kraw[kChunk / 16];
#pragma unroll
    for (uint32_t st = 0; st < kChunk / 16; st++) {
        const uint32_t j = j0 + st * 16 + wave * 4 + (lane >> 4);
        const uint32_t jc = j < len ? j : len - 1;
        const v4i t = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(kc + ((uint64_t)g * ctx + jc) * kHD + sub * 8));
        kraw[st] = make_uint4((uint32_t)t.x, (uint32_t)t.y, (uint32_t)t.z, (uint32_t)t.w);
    }
    __builtin_amdgcn_sched_barrier(0);
    uint32_t vraw[kChunk / 4];
#pragma unroll
    for (uint32_t jj = 0; jj < kChunk / 4; jj++) {
        const uint32_t j = j0 + wave * (kChunk / 4) + jj;
        const uint32_t jc = j < len ? j : len - 1;
        vraw[jj] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(vc + ((uint64_t)g * ctx + jc) * kHD + 2 * lane));
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- q (rotated), and this token's k and v as fp16
    float qv[kGroup][8];
#pragma unroll
    for (int h = 0; h < kGroup; h++) {
        const float in[8] = {qa[h].x, qa[h].y, qa[h].z, qa[h].w, qb[h].x, qb[h].y, qb[h].z, qb[h].w};
        if (ROPE) {
            rope_pair(in[0], in[1], csa.x, csa.y, qv[h][0], qv[h][1]);
            rope_pair(in[2], in[3], csa.z, csa.w, qv[h][2], qv[h][3]);
            rope_pair(in[4], in[5], csb.x, csb.y, qv[h][4], qv[h][5]);
            rope_pair(in[6], in[7], csb.z, csb.w, qv[h][6], qv[h][7]);
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) qv[h][e] = in[e];
        }
    }
    uint4 kpos = make_uint4(0, 0, 0, 0);
    uint32_t vpos = 0;
    if (ROPE) {
        float k[8];
        rope_pair(ka.x, ka.y, csa.x, csa.y, k[0], k[1]);
        rope_pair(ka.z, ka.w, csa.z, csa.w, k[2], k[3]);
        rope_pair(kb.x, kb.y, csb.x, csb.y, k[4], k[5]);
        rope_pair(kb.z, kb.w, csb.z, csb.w, k[6], k[7]);
        kpos = make_uint4(pack_f16x2(k[0], k[1]), pack_f16x2(k[2], k[3]), pack_f16x2(k[4], k[5]),
                          pack_f16x2(k[6], k[7]));
        vpos = pack_f16x2(vv.x, vv.y);
    }

    // ---- scores
#pragma unroll
    for (uint32_t st = 0; st < kChunk / 16; st++) {
        const uint32_t jl = st * 16 + wave * 4 + (lane >> 4);
        const uint32_t j = j0 + jl;
        const bool here = ROPE && j == pos;
        const uint4 raw = here ? kpos : kraw[st];
        if (here) *reinterpret_cast<uint4*>(kc + ((uint64_t)g * ctx + pos) * kHD + sub * 8) = kpos;
        const uint32_t wd[4] = {raw.x, raw.y, raw.z, raw.w};
        float kf[8];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            kf[2 * e] = half_bits_to_float(wd[e] & 0xffffu);
            kf[2 * e + 1] = half_bits_to_float(wd[e] >> 16);
        }
#pragma unroll
        for (int h = 0; h < kGroup; h++) {
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) d = __builtin_fmaf(qv[h][e], kf[e], d);
            d = faddv16(d);
            if (sub == 0) sc[h][jl] = j < len ? d * scale : -INFINITY;
        }
    }
    __syncthreads();
    {
        const uint32_t h = wave;
        const float a = lane < kChunk ? sc[h][lane] : -INFINITY;
        const float b = lane + 64 < kChunk ? sc[h][lane + 64] : -INFINITY;
        const float m = wave_max_f32(fmaxf(a, b));  // finite: position j0 < len
        const float pa = expf(a - m), pb = expf(b - m);
        const float l = wave_sum_f32(pa + pb);
        if (lane < kChunk) sc[h][lane] = pa;
        if (lane + 64 < kChunk) sc[h][lane + 64] = pb;
        if (lane == 0) {
            pml[((g * kGroup + h) * nch + c) * 2] = m;
            pml[((g * kGroup + h) * nch + c) * 2 + 1] = l;
        }
    }
    __syncthreads();

    // ---- values
    float o[kGroup][2];
#pragma unroll
    for (int h = 0; h < kGroup; h++) o[h][0] = o[h][1] = 0.0f;
#pragma unroll
    for (uint32_t jj = 0; jj < kChunk / 4; jj++) {
        const uint32_t jl = wave * (kChunk / 4) + jj, j = j0 + jl;
        const bool here = ROPE && j == pos;
        const uint32_t raw = here ? vpos : vraw[jj];
        if (here) *reinterpret_cast<uint32_t*>(vc + ((uint64_t)g * ctx + pos) * kHD + 2 * lane) = vpos;
        // past len: value 0 as well (the clamped row may hold non-finite fp16)
        const bool live = j < len;
        const float v0 = live ? half_bits_to_float(raw & 0xffffu) : 0.0f;
        const float v1 = live ? half_bits_to_float(raw >> 16) : 0.0f;
#pragma unroll
        for (int h = 0; h < kGroup; h++) {
            const float p = sc[h][jl];
            o[h][0] = __builtin_fmaf(p, v0, o[h][0]);
            o[h][1] = __builtin_fmaf(p, v1, o[h][1]);
        }
    }
#pragma unroll
    for (int h = 0; h < kGroup; h++) {
        red[wave][h][2 * lane] = o[h][0];
        red[wave][h][2 * lane + 1] = o[h][1];
    }
    __syncthreads();
    {
        const uint32_t h = wave;
        float2 r;
        r.x = red[0][h][2 * lane] + red[1][h][2 * lane] + red[2][h][2 * lane] + red[3][h][2 * lane];
        r.y = red[0][h][2 * lane + 1] + red[1][h][2 * lane + 1] + red[2][h][2 * lane + 1] + red[3][h][2 * lane + 1];
        *reinterpret_cast<float2*>(po + ((g * kGroup + h) * nch + c) * kHD + 2 * lane) = r;
    }
}

// One workgroup per query head merges the chunks in one round trip: every
// thread issues the loads of its dimension for up to 64 chunks before the
// (max, sum) pairs are read; both waves reduce the pairs (M, then
// L = sum l_c e^(m_c - M)) on their own, and wave 0 publishes the weights
// e^(m_c - M) in LDS.
__global__ void __launch_bounds__(kHD)
k_attn_combine(const float* __restrict__ po, const float* __restrict__ pml, uint32_t nch,
               float* __restrict__ out, uint8_t* __restrict__ q8, uint32_t nq) {
    extern __shared__ float wsh[];  // [nch rounded up to 64]
    const uint32_t h = blockIdx.x, d = threadIdx.x, lane = d & 63;
    const float* ml = pml + (uint64_t)h * nch * 2;
    const float* pd = po + (uint64_t)h * nch * kHD + d;
    float v[64];  // chunks past nch read chunk nch-1 (finite) and get weight 0
#pragma unroll
    for (int k = 0; k < 64; k++) v[k] = pd[(uint64_t)min((uint32_t)k, nch - 1) * kHD];
    float M = -INFINITY;
    for (uint32_t c = lane; c < nch; c += 64) M = fmaxf(M, ml[2 * c]);
    M = wave_max_f32(M);
    float L = 0.0f;
    for (uint32_t c = lane; c < nch; c += 64) {
        const float w = expf(ml[2 * c] - M);
        L = __builtin_fmaf(ml[2 * c + 1], w, L);
        if (d < 64) wsh[c] = w;
    }
    const uint32_t nch64 = (nch + 63) & ~63u;  // wsh is sized in whole batches of 64; the tail weighs 0
    if (d < 64 && nch + lane < nch64) wsh[nch + lane] = 0.0f;
    L = wave_sum_f32(L);
    __syncthreads();
    float O = 0.0f;
#pragma unroll
    for (int k = 0; k < 64; k++) O = __builtin_fmaf(v[k], wsh[k], O);
    for (uint32_t c0 = 64; c0 < nch; c0 += 64) {  // contexts past 64 chunks
#pragma unroll
        for (int k = 0; k < 64; k++) v[k] = pd[(uint64_t)min(c0 + k, nch - 1) * kHD];
#pragma unroll
        for (int k = 0; k < 64; k++) O = __builtin_fmaf(v[k], wsh[c0 + k], O);
    }
    const float r = O / L;
    out[h * kHD + d] = r;
    if (q8) {  // the 32-blocks of the output, quantized as the G-mode staging would
        uint32_t m = abs_key(r);
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) {
            const uint32_t o = __shfl_xor(m, off, kWave);
            m = m > o ? m : o;
        }
        float bs, inv;
        quant_params(__uint_as_float(m), bs, inv);
        const uint32_t i = h * kHD + d;
        q8[i] = (uint8_t)quant1(r, inv);
        if ((d & 31) == 0) reinterpret_cast<float*>(q8 + nq)[i >> 5] = bs;
    }
}

__global__ void __launch_bounds__(256)
k_silu_mul(uint32_t n, const float* __restrict__ gu, float* __restrict__ h) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    h[i] = silu_mul1(gu[i], gu[n + i]);
}

// h = silu(g) * u quantized to Q8 activation blocks: 8 lanes per 32-block,
// a float4 each (the arithmetic of the G-mode staging).  xq: qx [nb][32],
// then dx [nb] fp32.
__global__ void __launch_bounds__(256)
k_silu_mul_quant(uint32_t nb, const float* __restrict__ gu, uint8_t* __restrict__ xq) {
    const uint32_t t = blockIdx.x * 256 + threadIdx.x, blk = t >> 3, part = t & 7;
    const uint32_t n = nb * 32;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(gu, 2 * n * 4);
    const uint32_t o = blk < nb ? (blk * 32 + part * 4) * 4 : 0x80000000u;  // whole 8-lane groups stay active
    float h[4];
#pragma unroll
    for (int e = 0; e < 4; e++)
        h[e] = silu_mul1(__uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, o + 4 * e, 0, 0)),
                         __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, o + 4 * e + n * 4, 0, 0)));
    const uint32_t m = max8_u32(max(max(abs_key(h[0]), abs_key(h[1])), max(abs_key(h[2]), abs_key(h[3]))));
    float bs, inv;
    quant_params(__uint_as_float(m), bs, inv);
    if (blk < nb) {
        reinterpret_cast<uint32_t*>(xq)[blk * 8 + part] = pack4(h[0], h[1], h[2], h[3], inv);
        if (part == 0) reinterpret_cast<float*>(xq + n)[blk] = bs;
    }
}

// The build's RMSNorm of one row, with an optional residual add first:
// x' = y ? fl(x + y) : x, written to xsum when y is given (xsum may alias x:
// every element is read and written by the same thread); out =
// fl(fl(x' * inv) * w).  The sum of squares takes the canonical order of
// common.hpp, so the result is bit-identical to the norm the fused products
// apply in their prologue.  One workgroup of 256 threads; in pass p, thread
// t holds 4 values of block 32p + t/8 (x and y 16-byte aligned).  A batch of
// kNormBatch passes (K <= 16384 in one batch) is loaded before its first
// reduction, and kept in registers for the output when one batch holds the
// row.  Dynamic LDS: K/32 doubles of block sums.
constexpr uint32_t kNormBatch = 16;
__global__ void __launch_bounds__(256)
k_rms_norm_build(uint32_t K, float eps, const float* x, const float* __restrict__ y, const float* __restrict__ w,
                 float* xsum, float* __restrict__ out) {
    extern __shared__ double sums[];
    __shared__ double tot;
    const uint32_t nb = K / 32, part = threadIdx.x & 7, npass = (nb + 31) / 32;
    auto load = [&](uint32_t p) {
        const uint32_t b = 32 * p + (threadIdx.x >> 3);
        float4 f = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (b < nb) {
            f = *reinterpret_cast<const float4*>(x + b * 32 + part * 4);
            if (y) {
                const float4 r = *reinterpret_cast<const float4*>(y + b * 32 + part * 4);
                f = make_float4(__fadd_rn(f.x, r.x), __fadd_rn(f.y, r.y), __fadd_rn(f.z, r.z), __fadd_rn(f.w, r.w));
            }
        }
        return f;
    };
    float4 f[kNormBatch];
    for (uint32_t p0 = 0; p0 < npass; p0 += kNormBatch) {
#pragma unroll
        for (uint32_t k = 0; k < kNormBatch; k++)
            if (p0 + k < npass) f[k] = load(p0 + k);
#pragma unroll
        for (uint32_t k = 0; k < kNormBatch; k++) {
            if (p0 + k < npass) {  // uniform: whole 8-lane groups take the same passes
                const uint32_t b = 32 * (p0 + k) + (threadIdx.x >> 3);
                const double sb = sum8_f64(sumsq4_f64(f[k]));
                if (part == 0 && b < nb) sums[b] = sb;
            }
        }
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const double t = canon_total_f64(sums, nb);
        if (threadIdx.x == 0) tot = t;
    }
    __syncthreads();
    const float inv = rms_inv(tot, K, eps);
    for (uint32_t p0 = 0; p0 < npass; p0 += kNormBatch) {
        if (npass > kNormBatch) {
#pragma unroll
            for (uint32_t k = 0; k < kNormBatch; k++)
                if (p0 + k < npass) f[k] = load(p0 + k);  // the same bits again
        }
#pragma unroll
        for (uint32_t k = 0; k < kNormBatch; k++) {
            const uint32_t b = 32 * (p0 + k) + (threadIdx.x >> 3);
            if (p0 + k < npass && b < nb) {
                const uint32_t i = b * 32 + part * 4;
                const float v[4] = {f[k].x, f[k].y, f[k].z, f[k].w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    if (y) xsum[i + e] = v[e];
                    out[i + e] = __fmul_rn(__fmul_rn(v[e], inv), w[i + e]);
                }
            }
        }
    }
}

__global__ void __launch_bounds__(256)
k_add(uint32_t n, const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ out) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = __fadd_rn(a[i], b[i]);
}

// h[i] = silu(g_i) * u_i (silu_mul1) on gate|up interleaved in 32-row groups.
__global__ void __launch_bounds__(256)
k_silu_mul_il(uint32_t F, const float* __restrict__ gu, float* __restrict__ h) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= F) return;
    const uint32_t b = 64 * (i / 32) + (i % 32);
    h[i] = silu_mul1(gu[b], gu[b + 32]);
}

bool cfg_ok(const ane_decode_config* c) {
    return c && c->head_dim == kHD && c->n_kv_heads > 0 && c->n_heads == kGroup * c->n_kv_heads &&
           c->hidden > 0 && c->ffn > 0 && c->ctx > 0 && c->ctx <= (1u << 20) && c->hidden % 256 == 0 &&
           c->ffn % 256 == 0 &&
           (uint64_t)c->n_heads * kHD % 32 == 0;
}

uint32_t n_chunks(uint32_t len) { return (len + kChunk - 1) / kChunk; }

// Attention workspace: partial outputs [n_heads][nch][head_dim], then
// (max, sum) [n_heads][nch][2].
struct AttnWs {
    float* po;
    float* pml;
};

size_t attn_layout(const ane_decode_config* cfg, void* base, AttnWs* w) {
    const uint64_t nch = n_chunks(cfg->ctx);
    const size_t a = ceil_to((uint64_t)cfg->n_heads * nch * kHD * 4, 256);
    const size_t b = ceil_to((uint64_t)cfg->n_heads * nch * 8, 256);
    if (w && base) {
        uint8_t* p = static_cast<uint8_t*>(base);
        *w = AttnWs{reinterpret_cast<float*>(p), reinterpret_cast<float*>(p + a)};
    }
    return a + b;
}

int attention_launch(const ane_decode_config* cfg, bool rope, const float* q, const float* table_row,
                     uint16_t* k_cache, uint16_t* v_cache, uint32_t len, float* out, void* out_q8,
                     void* workspace, size_t workspace_bytes, void* stream) {
    if (out_q8 && (((uintptr_t)out_q8) & 15)) return ANE_ERR_INVALID_ARG;
    if (!workspace || (((uintptr_t)workspace) & 255) || workspace_bytes < attn_layout(cfg, nullptr, nullptr))
        return ANE_ERR_WORKSPACE;
    if (t_plan_only) return ANE_OK;
    AttnWs w;
    attn_layout(cfg, workspace, &w);
    const uint32_t nch = n_chunks(len);
    const float scale = 1.0f / sqrtf((float)kHD);
    hipStream_t s = (hipStream_t)stream;
    if (rope)
        hipLaunchKernelGGL(k_attention<true>, dim3(cfg->n_kv_heads, nch), dim3(256), 0, s, q, table_row, k_cache,
                           v_cache, len, cfg->ctx, cfg->n_heads, cfg->n_kv_heads, nch, scale, w.po, w.pml);
    else
        hipLaunchKernelGGL(k_attention<false>, dim3(cfg->n_kv_heads, nch), dim3(256), 0, s, q, table_row, k_cache,
                           v_cache, len, cfg->ctx, cfg->n_heads, cfg->n_kv_heads, nch, scale, w.po, w.pml);
    hipLaunchKernelGGL(k_attn_combine, dim3(cfg->n_heads), dim3(kHD), ((nch + 63) & ~63u) * 4, s, w.po, w.pml, nch, out,
                       static_cast<uint8_t*>(out_q8), cfg->n_heads * kHD);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

struct DecodeWs {
    float *qkv, *attn;
    uint8_t *attn_q8, *h_q8;  // Q8 activation blocks: qx [nb][32], then dx [nb]
    void* att;
    size_t attb;
};

size_t layout(const ane_decode_config* c, uint8_t* base, DecodeWs* w) {
    const uint64_t nqkv = (uint64_t)(c->n_heads + 2 * c->n_kv_heads) * kHD;
    size_t off = 0;
    auto take = [&](uint64_t bytes) {
        const size_t o = off;
        off += ceil_to(bytes, 256);
        return base ? base + o : nullptr;
    };
    float* qkv = reinterpret_cast<float*>(take(nqkv * 4));
    float* attn = reinterpret_cast<float*>(take((uint64_t)c->n_heads * kHD * 4));
    uint8_t* attn_q8 = take((uint64_t)c->n_heads * kHD / 32 * 36);
    uint8_t* h_q8 = take((uint64_t)c->ffn / 32 * 36);
    const size_t attb = ane_hip_attention_workspace_size(c);
    void* att = take(attb);
    if (w) *w = DecodeWs{qkv, attn, attn_q8, h_q8, att, attb};
    return off;
}

// The ggml route's workspace: the norm output, qkv, the attention output,
// a product output, gate|up, h, then the attention scratch (the build's
// chunk partials or the reference mode's scores and probabilities).
struct GgmlWs {
    float *xn, *qkv, *attn, *y, *gu, *h;
    void* att;
    size_t attb;
};

size_t ggml_layout(const ane_decode_config* c, uint8_t* base, GgmlWs* w) {
    const uint64_t nqkv = (uint64_t)(c->n_heads + 2 * c->n_kv_heads) * kHD, nq = (uint64_t)c->n_heads * kHD;
    size_t off = 0;
    auto take = [&](uint64_t bytes) {
        const size_t o = off;
        off += ceil_to(bytes, 256);
        return base ? base + o : nullptr;
    };
    float* xn = reinterpret_cast<float*>(take((uint64_t)c->hidden * 4));
    float* qkv = reinterpret_cast<float*>(take(nqkv * 4));
    float* attn = reinterpret_cast<float*>(take(nq * 4));
    float* y = reinterpret_cast<float*>(take((uint64_t)c->hidden * 4));
    float* gu = reinterpret_cast<float*>(take((uint64_t)c->ffn * 8));
    float* h = reinterpret_cast<float*>(take((uint64_t)c->ffn * 4));
    size_t attb = ane_hip_attention_workspace_size(c);
    const size_t refb = (size_t)c->n_heads * c->ctx * 8;
    if (refb > attb) attb = refb;
    void* att = take(attb);
    if (w) *w = GgmlWs{xn, qkv, attn, y, gu, h, att, attb};
    return off;
}

// One GGML_OP_MUL_MAT node: Q8_0 weights W (N rows of K values) times one
// fp32 column x, into y -- ggml's shapes: src0 ne = {K, N}, src1 ne = {K, 1},
// dst ne = {N, 1}, contiguous strides.
struct MulMatNode {
    ane_ggml_tensor w, a, d;
    MulMatNode(const void* W, uint32_t N, uint32_t K, const float* x, float* y) : w(), a(), d() {
        const size_t rb = (size_t)(K / 32) * 34;
        w.type = ANE_GGML_TYPE_Q8_0;
        w.ne[0] = K, w.ne[1] = N, w.ne[2] = w.ne[3] = 1;
        w.nb[0] = 34, w.nb[1] = rb, w.nb[2] = w.nb[3] = rb * N;
        w.data = const_cast<void*>(W);
        a.type = ANE_GGML_TYPE_F32;
        a.ne[0] = K, a.ne[1] = a.ne[2] = a.ne[3] = 1;
        a.nb[0] = 4, a.nb[1] = a.nb[2] = a.nb[3] = (size_t)K * 4;
        a.data = const_cast<float*>(x);
        d.type = ANE_GGML_TYPE_F32;
        d.op = ANE_GGML_OP_MUL_MAT;
        d.ne[0] = N, d.ne[1] = d.ne[2] = d.ne[3] = 1;
        d.nb[0] = 4, d.nb[1] = d.nb[2] = d.nb[3] = (size_t)N * 4;
        d.src[0] = &w;
        d.src[1] = &a;
        d.data = y;
    }
};

}  // namespace

int rms_norm_ref_launch(uint32_t rows, uint32_t dim, float eps, const float* in, const float* w, float* out,
                        uint64_t stride, hipStream_t s);
int add_rms_norm_ref_launch(uint32_t dim, float eps, float* x, const float* y, const float* w, float* xn,
                            hipStream_t s);
int rope_ref_kv_launch(float* qkv, uint32_t n_heads, uint32_t n_kv, uint32_t pos, uint32_t ctx, float theta,
                       uint16_t* kc, uint16_t* vc, hipStream_t s);
int attention_ref_launch(uint32_t n_heads, uint32_t n_kv, uint32_t len, uint32_t ctx, const float* q,
                         const uint16_t* kc, const uint16_t* vc, float* out, float* ws, hipStream_t s);
int silu_mul_ref_il_launch(uint32_t F, const float* gu, float* h, hipStream_t s);

}  // namespace ane

using namespace ane;

extern "C" int ane_hip_rope_kv_append(const ane_decode_config* cfg, float* qkv, const float* rope_table,
                                      uint32_t pos, uint16_t* k_cache, uint16_t* v_cache, void* stream) {
    if (!cfg_ok(cfg)) return ANE_ERR_INVALID_ARG;
    if (!qkv || !rope_table || !k_cache || !v_cache) return ANE_ERR_BAD_POINTER;
    if (pos >= cfg->ctx) return ANE_ERR_INVALID_ARG;
    const uint64_t n = (uint64_t)(cfg->n_heads + cfg->n_kv_heads) * (kHD / 2) + (uint64_t)cfg->n_kv_heads * kHD;
    hipLaunchKernelGGL(k_rope_kv_append, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       qkv, cfg->n_heads, cfg->n_kv_heads, rope_table + (uint64_t)pos * kHD, pos, cfg->ctx,
                       k_cache, v_cache);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

extern "C" size_t ane_hip_attention_workspace_size(const ane_decode_config* cfg) {
    if (!cfg_ok(cfg)) return 0;
    return attn_layout(cfg, nullptr, nullptr);
}

extern "C" int ane_hip_attention_decode(const ane_decode_config* cfg, const float* q, const uint16_t* k_cache,
                                        const uint16_t* v_cache, uint32_t len, float* out, void* workspace,
                                        size_t workspace_bytes, void* stream) {
    if (!cfg_ok(cfg)) return ANE_ERR_INVALID_ARG;
    if (!q || !k_cache || !v_cache || !out) return ANE_ERR_BAD_POINTER;
    if (len == 0 || len > cfg->ctx) return ANE_ERR_INVALID_ARG;
    return attention_launch(cfg, false, q, nullptr, const_cast<uint16_t*>(k_cache), const_cast<uint16_t*>(v_cache),
                            len, out, nullptr, workspace, workspace_bytes, stream);
}

extern "C" int ane_hip_attention_decode_rope(const ane_decode_config* cfg, const float* qkv, const float* rope_table,
                                             uint32_t pos, uint16_t* k_cache, uint16_t* v_cache, float* out,
                                             void* out_q8, void* workspace, size_t workspace_bytes, void* stream) {
    if (!cfg_ok(cfg)) return ANE_ERR_INVALID_ARG;
    if (!qkv || !rope_table || !k_cache || !v_cache || !out) return ANE_ERR_BAD_POINTER;
    if (pos >= cfg->ctx) return ANE_ERR_INVALID_ARG;
    return attention_launch(cfg, true, qkv, rope_table + (uint64_t)pos * kHD, k_cache, v_cache, pos + 1, out,
                            out_q8, workspace, workspace_bytes, stream);
}

extern "C" int ane_hip_silu_mul(uint32_t n, const float* gu, float* h, void* stream) {
    if (n == 0) return ANE_OK;
    if (!gu || !h) return ANE_ERR_BAD_POINTER;
    hipLaunchKernelGGL(k_silu_mul, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, n, gu, h);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

extern "C" int ane_hip_silu_mul_quant(uint32_t n, const float* gu, void* xq, void* stream) {
    if (n == 0) return ANE_OK;
    if (!gu || !xq) return ANE_ERR_BAD_POINTER;
    if ((n & 31) || (((uintptr_t)xq) & 15)) return ANE_ERR_INVALID_ARG;
    const uint32_t nb = n >> 5;
    hipLaunchKernelGGL(k_silu_mul_quant, dim3((nb * 8 + 255) / 256), dim3(256), 0, (hipStream_t)stream, nb, gu,
                       static_cast<uint8_t*>(xq));
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

extern "C" size_t ane_decode_workspace_size(const ane_decode_config* cfg) {
    if (!cfg_ok(cfg)) return 0;
    return layout(cfg, nullptr, nullptr);
}

extern "C" int ane_decode_token(const ane_decode_config* cfg, const ane_decode_layer* layers,
                                const float* rope_table, uint32_t pos, float* x, void* workspace,
                                size_t workspace_bytes, void* stream) {
    if (!cfg_ok(cfg)) return ANE_ERR_INVALID_ARG;
    if (!layers || !rope_table || !x) return ANE_ERR_BAD_POINTER;
    if (pos >= cfg->ctx) return ANE_ERR_INVALID_ARG;
    if (!workspace || (((uintptr_t)workspace) & 255) || workspace_bytes < layout(cfg, nullptr, nullptr))
        return ANE_ERR_WORKSPACE;
    DecodeWs w;
    layout(cfg, static_cast<uint8_t*>(workspace), &w);
    const uint32_t H = cfg->hidden, F = cfg->ffn;
    const uint32_t nq = cfg->n_heads * kHD;
    const uint32_t nqkv = (cfg->n_heads + 2 * cfg->n_kv_heads) * kHD;
    auto run_layer = [&](const ane_decode_layer& L) -> int {
        int st;
        if ((st = ane_hip_q8_0_matvec_fused(nqkv, H, x, L.attn_norm, cfg->eps, L.w_qkv, nullptr, w.qkv, stream)))
            return st;
        if ((st = ane_hip_attention_decode_rope(cfg, w.qkv, rope_table, pos, L.k_cache, L.v_cache, w.attn,
                                                w.attn_q8, w.att, w.attb, stream)))
            return st;
        if ((st = ane_hip_q8_0_matvec_q8(H, nq, w.attn_q8, L.w_o, x, x, stream))) return st;
        if ((st = ane_hip_q8_0_gate_up_silu_quant(F, H, x, L.ffn_norm, cfg->eps, L.w_gate_up, w.h_q8, stream)))
            return st;
        return ane_hip_q8_0_matvec_q8(H, F, w.h_q8, L.w_down, x, x, stream);
    };
    for (uint32_t l = 0; l < cfg->n_layers; l++) {
        const ane_decode_layer& L = layers[l];
        if (!L.w_qkv || !L.w_o || !L.w_gate_up || !L.w_down || !L.attn_norm || !L.ffn_norm || !L.k_cache ||
            !L.v_cache)
            return ANE_ERR_BAD_POINTER;
        // the streaming products take 16-byte aligned weights
        if (((uintptr_t)L.w_qkv | (uintptr_t)L.w_o | (uintptr_t)L.w_gate_up | (uintptr_t)L.w_down) & 15)
            return ANE_ERR_INVALID_ARG;
    }
    // Every step's preconditions (shapes, alignment, LDS fit, rows per wave)
    // are checked on layer 0 before anything is launched (the layers share
    // their shapes), so a configuration that cannot run fails with x and
    // the KV caches untouched.
    if (cfg->n_layers > 0) {
        t_plan_only = true;
        const int st = run_layer(layers[0]);
        t_plan_only = false;
        if (st) return st;
    }
    for (uint32_t l = 0; l < cfg->n_layers; l++) {
        const int st = run_layer(layers[l]);
        if (st) return st;
    }
    return ANE_OK;
}

extern "C" int ane_hip_rms_norm(uint32_t K, const float* x, const float* w, float eps, float* out, void* stream) {
    if (K == 0) return ANE_OK;
    if (!x || !w || !out) return ANE_ERR_BAD_POINTER;
    // K/32 doubles of block sums in LDS: at most 128 KB
    if ((K & 31) || (((uintptr_t)x) & 15) || K > (1u << 19)) return ANE_ERR_INVALID_ARG;
    hipLaunchKernelGGL(k_rms_norm_build, dim3(1), dim3(256), (K / 32) * 8, (hipStream_t)stream, K, eps, x,
                       (const float*)nullptr, w, (float*)nullptr, out);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

extern "C" int ane_hip_add_fp32(uint32_t n, const float* a, const float* b, float* out, void* stream) {
    if (n == 0) return ANE_OK;
    if (!a || !b || !out) return ANE_ERR_BAD_POINTER;
    hipLaunchKernelGGL(k_add, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, n, a, b, out);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

extern "C" size_t ane_decode_ggml_workspace_size(const ane_decode_config* cfg) {
    if (!cfg_ok(cfg)) return 0;
    return ggml_layout(cfg, nullptr, nullptr);
}

extern "C" int ane_decode_token_ggml(const ane_decode_config* cfg, const ane_decode_layer* layers,
                                     const float* rope_table, float rope_theta, uint32_t pos, float* x,
                                     void* workspace, size_t workspace_bytes, ane_ggml_backend_t backend,
                                     int arith) {
    if (!cfg_ok(cfg) || (arith != ANE_DECODE_ARITH_BUILD && arith != ANE_DECODE_ARITH_REFERENCE))
        return ANE_ERR_INVALID_ARG;
    if (!layers || !x || !backend || (arith == ANE_DECODE_ARITH_BUILD && !rope_table)) return ANE_ERR_BAD_POINTER;
    // the norms keep hidden/32 doubles of block sums in LDS
    if (pos >= cfg->ctx || (((uintptr_t)x) & 15) || cfg->hidden > (1u << 19)) return ANE_ERR_INVALID_ARG;
    if (!workspace || (((uintptr_t)workspace) & 255) || workspace_bytes < ggml_layout(cfg, nullptr, nullptr))
        return ANE_ERR_WORKSPACE;
    GgmlWs w;
    ggml_layout(cfg, static_cast<uint8_t*>(workspace), &w);
    const uint32_t H = cfg->hidden, F = cfg->ffn;
    const uint32_t nq = cfg->n_heads * kHD, nqkv = (cfg->n_heads + 2 * cfg->n_kv_heads) * kHD;
    for (uint32_t l = 0; l < cfg->n_layers; l++) {
        const ane_decode_layer& L = layers[l];
        if (!L.w_qkv || !L.w_o || !L.w_gate_up || !L.w_down || !L.attn_norm || !L.ffn_norm || !L.k_cache ||
            !L.v_cache)
            return ANE_ERR_BAD_POINTER;
    }
    // every product must be a node the hook computes before anything runs
    if (cfg->n_layers > 0) {
        const ane_decode_layer& L = layers[0];
        const MulMatNode n1(L.w_qkv, nqkv, H, w.xn, w.qkv), n2(L.w_o, H, nq, w.attn, w.y),
            n3(L.w_gate_up, 2 * F, H, w.xn, w.gu), n4(L.w_down, H, F, w.h, w.y);
        if (!ane_ggml_supports_op(&n1.d) || !ane_ggml_supports_op(&n2.d) || !ane_ggml_supports_op(&n3.d) ||
            !ane_ggml_supports_op(&n4.d))
            return ANE_ERR_INVALID_ARG;
    }
    hipStream_t s = (hipStream_t)ane_ggml_backend_get_stream(backend);
    const bool ref = arith == ANE_DECODE_ARITH_REFERENCE;
    // the products' arithmetic goes with the mode: G (int8 dots) for the
    // build's, R (opcode 0x57, what the reference's hook runs) for the reference's
    ane_ggml_backend_set_q8_mode(backend, ref ? ANE_GGML_Q8_R : ANE_GGML_Q8_G);
    const uint32_t gA = (H + 255) / 256;
    int st;
#define ANE_TRY(e)             \
    do {                       \
        if ((st = (e))) return st; \
    } while (0)
    // the build's residual adds ride on the norm that follows them:
    // x = fl(x + y), xn = norm(x) in one launch
    auto add_norm = [&](const float* y, const float* nw) {
        hipLaunchKernelGGL(k_rms_norm_build, dim3(1), dim3(256), (H / 32) * 8, s, H, cfg->eps, (const float*)x, y,
                           nw, x, w.xn);
    };
    for (uint32_t l = 0; l < cfg->n_layers; l++) {
        const ane_decode_layer& L = layers[l];
        if (l == 0) {
            if (ref) ANE_TRY(rms_norm_ref_launch(1, H, cfg->eps, x, L.attn_norm, w.xn, H, s));
            else ANE_TRY(ane_hip_rms_norm(H, x, L.attn_norm, cfg->eps, w.xn, s));
        }
        {
            const MulMatNode n(L.w_qkv, nqkv, H, w.xn, w.qkv);
            ANE_TRY(ane_ggml_compute_forward(backend, &n.d));
        }
        if (ref) {
            ANE_TRY(rope_ref_kv_launch(w.qkv, cfg->n_heads, cfg->n_kv_heads, pos, cfg->ctx, rope_theta, L.k_cache,
                                       L.v_cache, s));
            ANE_TRY(attention_ref_launch(cfg->n_heads, cfg->n_kv_heads, pos + 1, cfg->ctx, w.qkv, L.k_cache,
                                         L.v_cache, w.attn, static_cast<float*>(w.att), s));
        } else {
            ANE_TRY(ane_hip_attention_decode_rope(cfg, w.qkv, rope_table, pos, L.k_cache, L.v_cache, w.attn, nullptr,
                                                  w.att, w.attb, s));
        }
        {
            const MulMatNode n(L.w_o, H, nq, w.attn, w.y);
            ANE_TRY(ane_ggml_compute_forward(backend, &n.d));
        }
        if (ref) {
            ANE_TRY(add_rms_norm_ref_launch(H, cfg->eps, x, w.y, L.ffn_norm, w.xn, s));
        } else {
            add_norm(w.y, L.ffn_norm);
        }
        {
            const MulMatNode n(L.w_gate_up, 2 * F, H, w.xn, w.gu);
            ANE_TRY(ane_ggml_compute_forward(backend, &n.d));
        }
        if (ref) ANE_TRY(silu_mul_ref_il_launch(F, w.gu, w.h, s));
        else hipLaunchKernelGGL(k_silu_mul_il, dim3((F + 255) / 256), dim3(256), 0, s, F, w.gu, w.h);
        {
            const MulMatNode n(L.w_down, H, F, w.h, w.y);
            ANE_TRY(ane_ggml_compute_forward(backend, &n.d));
        }
        // the residual add rides on the next layer's norm (the same fl(x + y)
        // then the norm of the sum, in one launch)
        if (l + 1 < cfg->n_layers) {
            if (ref) ANE_TRY(add_rms_norm_ref_launch(H, cfg->eps, x, w.y, layers[l + 1].attn_norm, w.xn, s));
            else add_norm(w.y, layers[l + 1].attn_norm);
        } else {
            hipLaunchKernelGGL(k_add, dim3(gA), dim3(256), 0, s, H, x, w.y, x);
        }
        ANE_HIP_CHECK_LAUNCH();
    }
#undef ANE_TRY
    return ANE_OK;
}
