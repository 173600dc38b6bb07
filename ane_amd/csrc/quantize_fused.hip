// quantize_fused.hip -- operand preparation of dense_fused_i8 (README.md:84-97):
// per-tensor absmax quantization of fp32 A (M x K) and B (K x N) with the
// arithmetic of quantize_fp32_i8 (bytecode_interpreter.s:1885-1950), writing
//   qA  : M x Kp int8, row-major (K contiguous), zeros for k >= K;
//   qBt : N x Kp int8, B transposed (K contiguous per column), zeros for k >= K;
//   scales[0..1] = {sa, sb}.
// Two HBM-bound launches: a max-|x| pass over both tensors (per-block
// partial maxima), then one quantize pass in which every block first folds
// its tensor's partials.  The second read of A and B mostly hits the 256 MB
// Infinity Cache.
#include "gemm_i8.hpp"

namespace ane {
namespace {

constexpr int kT = 256;

__device__ __forceinline__ uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint32_t absmax4(float4 v) {
    return umax(umax(abs_key(v.x), abs_key(v.y)), umax(abs_key(v.z), abs_key(v.w)));
}

// Pass 1: blocks [0, nbA) reduce A, [nbA, nbA+nbB) reduce B.  Each block
// reads one contiguous range of its tensor's float4s (contiguous ranges per
// workgroup measured faster on this HBM than a grid-stride interleave),
// four 16-byte loads in flight per thread.
__global__ void __launch_bounds__(kT)
k_absmax_two(const float* __restrict__ A, uint64_t nA, uint32_t nbA, const float* __restrict__ B,
             uint64_t nB, uint32_t nbB, uint32_t* __restrict__ partials) {
    __shared__ uint32_t red[4];
    const bool isA = blockIdx.x < nbA;
    const float* src = isA ? A : B;
    const uint64_t n = isA ? nA : nB;
    const uint32_t b = isA ? blockIdx.x : blockIdx.x - nbA;
    const uint32_t nblk = isA ? nbA : nbB;
    uint32_t m = 0;
    uint64_t head = 0;
    if ((((uintptr_t)src) & 15) == 0) {
        const uint64_t n4 = n >> 2;
        const uint64_t per = (n4 + nblk - 1) / nblk;
        const uint64_t c0 = (uint64_t)b * per, c1 = c0 + per < n4 ? c0 + per : n4;
        const float4* s4 = reinterpret_cast<const float4*>(src);
        uint64_t i = c0 + threadIdx.x;
        for (; i + 3 * kT < c1; i += 4 * kT) {
            const float4 v0 = s4[i], v1 = s4[i + kT], v2 = s4[i + 2 * kT], v3 = s4[i + 3 * kT];
            m = umax(m, umax(umax(absmax4(v0), absmax4(v1)), umax(absmax4(v2), absmax4(v3))));
        }
        for (; i < c1; i += kT) m = umax(m, absmax4(s4[i]));
        head = n4 << 2;
    }
    // the tail past the last whole float4 (or everything, unaligned), grid-stride
    const uint64_t stride = (uint64_t)nblk * kT;
    for (uint64_t j = head + (uint64_t)b * kT + threadIdx.x; j < n; j += stride) m = umax(m, abs_key(src[j]));
    m = block_max_u32_256(m, red);
    if (threadIdx.x == 0) partials[blockIdx.x] = m;
}

__device__ __forceinline__ float fold_partials(const uint32_t* partials, uint32_t n, uint32_t* red) {
    uint32_t m = 0;
    for (uint32_t i = threadIdx.x; i < n; i += kT) m = umax(m, partials[i]);
    return __uint_as_float(block_max_u32_256(m, red));
}

// B tiles: 128 k x 64 n per block.
constexpr int kBTK = 128, kBTN = 64;
constexpr int kTileRowDw = kBTK / 4 + 1;  // dwords per transposed row (+1 pad)

// Pass 2.  Blocks [0, nqA) quantize A row-major into qA (16 elements per
// thread per step, one contiguous range of A per block); blocks [nqA, ...)
// quantize one 128 x 64 tile of B each: thread t loads rows 4(t/16)+{0..3}
// (and +64) x columns 4(t%16)+{0..3} as float4s, transposes each 4 x 4 byte
// block in registers, stages the tile as qBt rows in LDS and writes 128-byte
// row segments.
__global__ void __launch_bounds__(kT)
k_quantize_two(const float* __restrict__ A, const float* __restrict__ B, uint32_t M, uint32_t N,
               uint32_t K, uint32_t Kp, const uint32_t* __restrict__ partials, uint32_t nbA,
               uint32_t nbB, uint32_t nqA, int8_t* __restrict__ qA, int8_t* __restrict__ qBt,
               float* __restrict__ scales) {
    __shared__ uint32_t red[4];
    __shared__ uint32_t tileT[kBTN * kTileRowDw];
    const bool isA = blockIdx.x < nqA;
    const float amax = isA ? fold_partials(partials, nbA, red) : fold_partials(partials + nbA, nbB, red);
    float scale, inv;
    quant_params(amax, scale, inv);
    if (threadIdx.x == 0 && (blockIdx.x == 0 || blockIdx.x == nqA)) scales[isA ? 0 : 1] = scale;

    if (isA) {
        const uint64_t chunks_per_row = Kp / 16;
        const uint64_t total = (uint64_t)M * chunks_per_row;
        const bool vec = ((K & 3) == 0) && ((((uintptr_t)A) & 15) == 0);
        // one contiguous range of chunks per block
        const uint64_t per = (total + nqA - 1) / nqA;
        const uint64_t c0 = (uint64_t)blockIdx.x * per, c1 = c0 + per < total ? c0 + per : total;
        for (uint64_t c = c0 + threadIdx.x; c < c1; c += kT) {
            const uint64_t i = c / chunks_per_row;
            const uint32_t k = (uint32_t)(c % chunks_per_row) * 16;
            const float* src = A + i * K + k;
            uint32_t w[4] = {0, 0, 0, 0};
            if (vec && k + 16 <= K) {
                const float4 v0 = reinterpret_cast<const float4*>(src)[0];
                const float4 v1 = reinterpret_cast<const float4*>(src)[1];
                const float4 v2 = reinterpret_cast<const float4*>(src)[2];
                const float4 v3 = reinterpret_cast<const float4*>(src)[3];
                w[0] = pack4(v0.x, v0.y, v0.z, v0.w, inv);
                w[1] = pack4(v1.x, v1.y, v1.z, v1.w, inv);
                w[2] = pack4(v2.x, v2.y, v2.z, v2.w, inv);
                w[3] = pack4(v3.x, v3.y, v3.z, v3.w, inv);
            } else {
                for (int e = 0; e < 16; e++)
                    if (k + e < K) w[e >> 2] |= (uint32_t)(quant1(src[e], inv) & 0xff) << (8 * (e & 3));
            }
            *reinterpret_cast<uint4*>(qA + i * Kp + k) = make_uint4(w[0], w[1], w[2], w[3]);
        }
        return;
    }

    const uint32_t tb = blockIdx.x - nqA;
    const uint32_t ntn = (N + kBTN - 1) / kBTN;
    const uint32_t k0 = (tb / ntn) * kBTK, n0 = (tb % ntn) * kBTN;
    const uint32_t kq = threadIdx.x >> 4, nq = threadIdx.x & 15;
    const uint32_t gn = n0 + 4 * nq;
    const bool vec = ((N & 3) == 0) && ((((uintptr_t)B) & 15) == 0) && gn + 3 < N;
#pragma unroll
    for (int g = 0; g < 2; g++) {
        float v[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t gk = k0 + g * 64 + 4 * kq + i;
            if (gk < K && vec) {
                const float4 f = *reinterpret_cast<const float4*>(B + (uint64_t)gk * N + gn);
                v[i][0] = f.x; v[i][1] = f.y; v[i][2] = f.z; v[i][3] = f.w;
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    v[i][j] = (gk < K && gn + j < N) ? B[(uint64_t)gk * N + gn + j] : 0.0f;
            }
        }
        // column j of the 4 x 4 block = 4 consecutive k of output row n = gn + j
#pragma unroll
        for (int j = 0; j < 4; j++)
            tileT[(4 * nq + j) * kTileRowDw + g * 16 + kq] = pack4(v[0][j], v[1][j], v[2][j], v[3][j], inv);
    }
    __syncthreads();
    {
        const uint32_t n = threadIdx.x >> 2, part = threadIdx.x & 3;  // 32 bytes per thread
        if (n0 + n < N && k0 + part * 32 < Kp) {
            const uint32_t* row = tileT + n * kTileRowDw + part * 8;
            uint4 lo = make_uint4(row[0], row[1], row[2], row[3]);
            uint4 hi = make_uint4(row[4], row[5], row[6], row[7]);
            int8_t* dst = qBt + (uint64_t)(n0 + n) * Kp + k0 + part * 32;
            reinterpret_cast<uint4*>(dst)[0] = lo;
            reinterpret_cast<uint4*>(dst)[1] = hi;
        }
    }
}

uint32_t blocks_for(uint64_t n) {
    uint64_t b = (n / 4 + 4 * kT - 1) / (4 * kT);
    if (b < 1) b = 1;
    if (b > kFusedPartials) b = kFusedPartials;
    return (uint32_t)b;
}

}  // namespace

int launch_fused_quantize(const float* A, const float* B, uint32_t M, uint32_t N, uint32_t K,
                          uint32_t Kp, uint32_t* partials, int8_t* qA, int8_t* qBt, float* scales,
                          hipStream_t s) {
    const uint64_t nA = (uint64_t)M * K, nB = (uint64_t)K * N;
    const uint32_t nbA = blocks_for(nA), nbB = blocks_for(nB);
    hipLaunchKernelGGL(k_absmax_two, dim3(nbA + nbB), dim3(kT), 0, s, A, nA, nbA, B, nB, nbB, partials);
    uint64_t nqA = ((uint64_t)M * (Kp / 16) + 2 * kT - 1) / (2 * kT);
    if (nqA > 4096) nqA = 4096;
    if (nqA < 1) nqA = 1;
    const uint64_t nqB = Kp ? ((uint64_t)Kp / kBTK) * (((uint64_t)N + kBTN - 1) / kBTN) : 1;
    if (nqA + nqB > 0x7fffffffull) return ANE_ERR_INVALID_ARG;
    hipLaunchKernelGGL(k_quantize_two, dim3((uint32_t)(nqA + nqB)), dim3(kT), 0, s, A, B, M, N, K, Kp,
                       partials, nbA, nbB, (uint32_t)nqA, qA, qBt, scales);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

}  // namespace ane
