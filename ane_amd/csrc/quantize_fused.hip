// quantize_fused.hip -- operand preparation of dense_fused_i8 (README.md:84-97):
// per-tensor absmax quantization of fp32 A (M x K) and B (K x N) with the
// arithmetic of quantize_fp32_i8 (bytecode_interpreter.s:1885-1950), writing
//   qA  : M x Kp int8, row-major (K contiguous), zeros for k >= K;
//   qBt : N x Kp int8, B transposed (K contiguous per column), zeros for k >= K;
//   scales[0..1] = {sa, sb}.
// Two routes:
//  - resident (k_quantize_resident, one launch): one workgroup per CU reads
//    its share of A and B once, keeping B in VGPRs and up to 128 KB of A in
//    LDS, publishes its partial maxima, meets the other workgroups at a
//    grid-wide barrier, then quantizes from on-chip copies (re-reading only
//    the part of A that did not fit);
//  - two-pass (k_absmax_two + k_quantize_two): a max-|x| pass over both
//    tensors (per-block partial maxima), then one quantize pass in which
//    every block first folds its tensor's partials.  It takes the shapes
//    the resident route does not.
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>

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
               float* __restrict__ scales, uint32_t* __restrict__ wstatus) {
    __shared__ uint32_t red[4];
    __shared__ uint32_t tileT[kBTN * kTileRowDw];
    const bool isA = blockIdx.x < nqA;
    const float amax = isA ? fold_partials(partials, nbA, red) : fold_partials(partials + nbA, nbB, red);
    float scale, inv;
    quant_params(amax, scale, inv);
    if (threadIdx.x == 0 && (blockIdx.x == 0 || blockIdx.x == nqA)) scales[isA ? 0 : 1] = scale;
    if (threadIdx.x == 0 && blockIdx.x == 0) wstatus[0] = 0;  // no grid-wide wait on this route
    // the values quantized here are the tensor's own, whose max was just
    // folded: pack4_fast applies whenever that max and inv are finite
    const bool fast = fast_quant_ok(amax, inv);

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
                if (fast) {
                    w[0] = pack4_fast(v0.x, v0.y, v0.z, v0.w, inv);
                    w[1] = pack4_fast(v1.x, v1.y, v1.z, v1.w, inv);
                    w[2] = pack4_fast(v2.x, v2.y, v2.z, v2.w, inv);
                    w[3] = pack4_fast(v3.x, v3.y, v3.z, v3.w, inv);
                } else {
                    w[0] = pack4(v0.x, v0.y, v0.z, v0.w, inv);
                    w[1] = pack4(v1.x, v1.y, v1.z, v1.w, inv);
                    w[2] = pack4(v2.x, v2.y, v2.z, v2.w, inv);
                    w[3] = pack4(v3.x, v3.y, v3.z, v3.w, inv);
                }
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
            tileT[(4 * nq + j) * kTileRowDw + g * 16 + kq] =
                fast ? pack4_fast(v[0][j], v[1][j], v[2][j], v[3][j], inv) : pack4(v[0][j], v[1][j], v[2][j], v[3][j], inv);
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

// ------------------------------------------------------------ few-tile route
// dense_fused_i8 on small operands in two launches instead of three:
// k_absmax_two, then k_fused_small with one workgroup per 16 x 16 tile of C.
// The workgroup folds the partial maxima, quantizes its 16 rows of A and 16
// columns of B straight into LDS (pack4 / pack4_fast under the same
// condition as k_quantize_two, so the same bytes; zeros past M, N and K),
// and multiplies them with v_mfma_i32_16x16x64_i8: lane (g, c16) gives row
// c16 of A and column c16 of B the same 16 bytes of each 64-byte step, so
// the int32 sums are the exact dot products, and the four waves take every
// fourth step, their sums meeting in LDS (exact in any order).  The
// epilogue is the contraction kernels' fmaxA(fadd(fmul((float)acc, s), +0),
// lo) with s = (sa * sb) * smul.  qA and qBt are not written: nothing after
// the op reads them (the quantize entry point keeps the two-launch route).
constexpr uint32_t kSmallMaxK = 1024;
// Measured against the three-launch route (tiles, fp32 elements read by all
// workgroups, µs): 128 / 2M (128x128x1000) 15.7 -> 10.0, 256 / 8M
// (256x256x1024) 14.2 -> 10.0, 512 / 16M (256x512x1024) 14.5 -> 11.2; past
// one workgroup per CU and a half, slower: 1024 / 8M (512x512x256) 12.0 ->
// 13.7, 1024 / 32M (256x1024x1024) 15.0 -> 18.0.
constexpr uint64_t kSmallMaxReads = 16u << 20;
constexpr uint64_t kSmallMaxTiles = 512;
constexpr uint32_t kSmallStride = kSmallMaxK + 16;  // bytes per staged row; rows 4 banks apart

__global__ void __launch_bounds__(kT)
k_fused_small(const float* __restrict__ A, const float* __restrict__ B, uint32_t M, uint32_t N, uint32_t K,
              const uint32_t* __restrict__ partials, uint32_t nbA, uint32_t nbB, float smul, float lo,
              float* __restrict__ C, float* __restrict__ scales, uint32_t* __restrict__ wstatus) {
    __shared__ uint32_t red[4];
    __shared__ __attribute__((aligned(16))) int8_t qa[16 * kSmallStride];
    __shared__ __attribute__((aligned(16))) int8_t qb[16 * kSmallStride];
    __shared__ v4i part[4][64];
    const float amaxA = fold_partials(partials, nbA, red);
    const float amaxB = fold_partials(partials + nbA, nbB, red);
    float sa, ia, sb, ib;
    quant_params(amaxA, sa, ia);
    quant_params(amaxB, sb, ib);
    if (threadIdx.x == 0 && blockIdx.x == 0 && blockIdx.y == 0) {
        scales[0] = sa;
        scales[1] = sb;
        wstatus[0] = 0;  // no grid-wide wait on this route
    }
    const bool fa = fast_quant_ok(amaxA, ia), fb = fast_quant_ok(amaxB, ib);
    const uint32_t m0 = blockIdx.y * 16, n0 = blockIdx.x * 16;
    const uint32_t Kp = (K + 63) & ~63u;  // whole 64-byte steps
    const uint32_t kq = Kp / 4;

    // Every load is issued before any is quantized (one memory round trip):
    // range-checked buffer loads, an offset past the buffer reading zeros.
    // A: 16 rows x Kp, four consecutive k per thread and step.
    constexpr int kAIt = 16 * (kSmallMaxK / 4) / kT, kBIt = 4 * (kSmallMaxK / 4) / kT;
    constexpr uint32_t kNone = 0x80000000u;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, M * K * 4), rb = make_rsrc(B, K * N * 4);
    const bool va = (K & 3) == 0 && (((uintptr_t)A) & 15) == 0;  // whole float4s (uniform)
    float a4[kAIt][4];
#pragma unroll
    for (int it = 0; it < kAIt; it++) {
        const uint32_t c = threadIdx.x + it * kT, r = c / kq, k = (c - r * kq) * 4, m = m0 + r;
        const bool live = c < 16 * kq && m < M;
        if (va) {
            const float4 f = __builtin_bit_cast(
                float4, __builtin_amdgcn_raw_buffer_load_b128(ra, live && k < K ? (m * K + k) * 4 : kNone, 0, 0));
            a4[it][0] = f.x, a4[it][1] = f.y, a4[it][2] = f.z, a4[it][3] = f.w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                a4[it][e] = __uint_as_float(
                    __builtin_amdgcn_raw_buffer_load_b32(ra, live && k + e < K ? (m * K + k + e) * 4 : kNone, 0, 0));
        }
    }
    // B: 4 k x 4 columns per thread and step, transposed in registers so
    // each staged row is one column of B
    const bool vb = (N & 3) == 0 && (((uintptr_t)B) & 15) == 0;
    float b4[kBIt][4][4];  // [step][k + i][n + j]
#pragma unroll
    for (int it = 0; it < kBIt; it++) {
        const uint32_t c = threadIdx.x + it * kT, k = (c >> 2) * 4, n = n0 + (c & 3) * 4;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const bool live = c < 4 * kq && k + i < K;
            if (vb) {
                const float4 f = __builtin_bit_cast(
                    float4,
                    __builtin_amdgcn_raw_buffer_load_b128(rb, live && n < N ? ((k + i) * N + n) * 4 : kNone, 0, 0));
                b4[it][i][0] = f.x, b4[it][i][1] = f.y, b4[it][i][2] = f.z, b4[it][i][3] = f.w;
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    b4[it][i][j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                        rb, live && n + j < N ? ((k + i) * N + n + j) * 4 : kNone, 0, 0));
            }
        }
    }
#pragma unroll
    for (int it = 0; it < kAIt; it++) {
        const uint32_t c = threadIdx.x + it * kT, r = c / kq, k = (c - r * kq) * 4;
        if (c < 16 * kq)
            *reinterpret_cast<uint32_t*>(qa + r * kSmallStride + k) =
                fa ? pack4_fast(a4[it][0], a4[it][1], a4[it][2], a4[it][3], ia)
                   : pack4(a4[it][0], a4[it][1], a4[it][2], a4[it][3], ia);
    }
#pragma unroll
    for (int it = 0; it < kBIt; it++) {
        const uint32_t c = threadIdx.x + it * kT, k = (c >> 2) * 4, j4 = (c & 3) * 4;
        if (c < 4 * kq) {
#pragma unroll
            for (int j = 0; j < 4; j++)
                *reinterpret_cast<uint32_t*>(qb + (j4 + j) * kSmallStride + k) =
                    fb ? pack4_fast(b4[it][0][j], b4[it][1][j], b4[it][2][j], b4[it][3][j], ib)
                       : pack4(b4[it][0][j], b4[it][1][j], b4[it][2][j], b4[it][3][j], ib);
        }
    }
    __syncthreads();

    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4, c16 = lane & 15;
    v4i acc = {0, 0, 0, 0};
    for (uint32_t k0 = wave * 64; k0 < Kp; k0 += 256) {
        const v4i a = *reinterpret_cast<const v4i*>(qa + c16 * kSmallStride + k0 + 16 * g);
        const v4i b = *reinterpret_cast<const v4i*>(qb + c16 * kSmallStride + k0 + 16 * g);
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc, 0, 0, 0);
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
        const v4i t = part[0][lane] + part[1][lane] + part[2][lane] + part[3][lane];
        const float s = __fmul_rn(__fmul_rn(sa, sb), smul);
        const uint32_t n = n0 + c16;
#pragma unroll
        for (int i = 0; i < 4; i++) {  // D lane (g, c16), register i: row 4g + i, column c16
            const uint32_t m = m0 + 4 * g + i;
            if (m < M && n < N) C[(uint64_t)m * N + n] = fmax_a(__fadd_rn(__fmul_rn((float)t[i], s), 0.0f), lo);
        }
    }
}

// ------------------------------------------------------------ resident route
// Grid: one 512-thread workgroup per CU (its 158 KB of LDS allows no
// second), every workgroup resident at once, so the grid-wide barrier
// below always completes; its wait is bounded anyway (kSyncTimeoutTicks of
// the 100 MHz realtime counter), and a workgroup that gives up records it
// in the slot's error word.
//   B: tile tb = k-tile * (N/64) + n-tile covers k0 .. k0+127, n0 .. n0+63;
//      workgroup w holds tiles [w*perT, (w+1)*perT) (perT <= kRNT), thread t
//      rows k0 + 4*(t/16) + {0..3} x columns n0 + 4*(t%16) + {0..3} as four
//      float4 VGPRs per tile.
//   A: workgroup w holds float4s [w*perA4, (w+1)*perA4) of A (K % 128 == 0,
//      so the float4 j of A is the dword j of qA); the first kRLdsA4 of
//      them are copied into LDS, the next kRVA per thread are loaded into
//      VGPRs, and any rest is read for the maximum and read again to
//      quantize.  In phase 2 the B transposes are staged in A's LDS once
//      A's LDS part has been written out.
// Sync slot: one per device, zero at module load (layout and protocol at
// grid_arrive_wait).
constexpr int kRT = 512;
constexpr int kRNT = 8;
constexpr uint32_t kRLdsA4 = 10112;  // float4s of A in LDS (158 KB, a multiple of 64); B's transposes reuse it
constexpr uint32_t kRLdsSteps = (kRLdsA4 + kRT - 1) / kRT;
constexpr int kRVA = 10;             // float4s of A per thread in VGPRs (249 VGPRs in all, no spill)
constexpr uint64_t kROnChip4 = kRLdsA4 + (uint64_t)kRVA * kRT;  // 15,232 float4s (238 KB) of A on chip
constexpr int kRBatch = 8;           // float4 loads in flight per thread on the rest of A
static_assert(kRNT * 4 + kRVA + kRBatch < 64, "the loads issued after A's copies fit the vmcnt field");
constexpr uint32_t kTileDw = 64 * kTileRowDw;
static_assert(kRLdsA4 % kWave == 0, "the LDS part of A is copied in whole 64-slot runs");
static_assert(kRNT * kTileDw * 4 <= kRLdsA4 * 16, "the B transposes fit in A's LDS");
constexpr uint64_t kSyncTimeoutTicks = 200000000ull;  // 2 s at 100 MHz
constexpr uint64_t kResidentMinBytes = (uint64_t)12 << 20;

// Grid-wide exchange of the workgroup maxima, by thread 0 of each
// workgroup.  Every access is an agent-scope atomic (coherent across the
// XCDs' L2s without cache write-back or invalidation), and s_waitcnt
// vmcnt(0) orders each workgroup's partial stores before its arrival.
// Arrivals are counted in kSyncGroups groups (workgroup w in group
// w % kSyncGroups, each counter on its own 128-byte line) so no line takes
// more than ~G/kSyncGroups atomics; the last arrival of a group adds to the
// top counter, and the last group's last arrival writes every group's
// release word, which the waiting workgroups poll (each read its group's
// word before arriving, so the release cannot be missed).  The last
// arrivals reset the group and top counters to zero, so the slot is at rest
// between launches (a launch's resets complete before the kernel does).
//
// Every launch carries a nonzero 32-bit tag (the host numbers launches
// 1, 2, 3, ...), so that two launches sharing the slot at once (a replayed
// graph overlapping another call) cannot pass each other's workgroups
// silently:
//  * each arrival adds (tag << 32) | 1 to a 64-bit counter; a counter that
//    reaches its member count holds members * tag in its high half when all
//    its arrivals are one launch's, and a different sum when two launches'
//    arrivals mixed in it, unless their tags differ by a multiple of 2^27 (a
//    counter has at most 64 members): the arrival that completes it records
//    kSyncMixed in the error word;
//  * a release word is (epoch << 32) | tag of the releasing launch, and a
//    waiter passes only on a release carrying its own tag: one by another
//    launch is recorded (kSyncMixed) and the wait goes on for its own.
// The wait gives up after timeout_ticks of the 100 MHz realtime counter and
// records kSyncTimeout.  Returns this workgroup's view: 0, or the bits it
// recorded.  Two launches with the same tag (one captured graph replayed
// twice at once, on the same workspace) are not told apart.
constexpr uint32_t kSyncGroups = 16;
constexpr uint32_t kSyncLineDw = 32;                       // 128-byte lines
constexpr uint32_t kSyncSlotDw = (1 + 2 * kSyncGroups) * kSyncLineDw;
constexpr uint32_t kSyncTimeout = 1u, kSyncMixed = 2u;
__device__ __forceinline__ uint64_t* sync_top(uint32_t* sync) { return reinterpret_cast<uint64_t*>(sync); }
__device__ __forceinline__ uint32_t* sync_err(uint32_t* sync) { return sync + 2; }
__device__ __forceinline__ uint64_t* sync_gen(uint32_t* sync, uint32_t g) {
    return reinterpret_cast<uint64_t*>(sync + (1 + g) * kSyncLineDw);
}
__device__ __forceinline__ uint64_t* sync_sub(uint32_t* sync, uint32_t g) {
    return reinterpret_cast<uint64_t*>(sync + (1 + kSyncGroups + g) * kSyncLineDw);
}

__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_agent64(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent64(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t add_agent64(uint64_t* p, uint64_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void or_err(uint32_t* sync, uint32_t bits) {
    __hip_atomic_fetch_or(sync_err(sync), bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// True when a counter that has just reached `members` arrivals (old is its
// value before the last add of `tag`) holds only arrivals tagged `tag`.
__device__ __forceinline__ bool sync_tags_match(uint64_t old, uint32_t tag, uint32_t members) {
    return (uint32_t)(old >> 32) + tag == members * tag;
}

__device__ __forceinline__ uint32_t grid_arrive_wait(uint32_t* sync, uint32_t* partials, uint32_t ma,
                                                     uint32_t mb, uint32_t w, uint32_t G, uint32_t tag,
                                                     uint64_t timeout_ticks) {
    const uint32_t ng = G < kSyncGroups ? G : kSyncGroups;
    const uint32_t g = w % ng, members = (G - g + ng - 1) / ng;
    uint64_t* gen = sync_gen(sync, g);
    const uint64_t gen0 = ld_agent64(gen);
    st_agent(&partials[w], ma);
    st_agent(&partials[G + w], mb);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const uint64_t inc = ((uint64_t)tag << 32) | 1u;
    uint32_t bad = 0;
    const uint64_t old = add_agent64(sync_sub(sync, g), inc);
    if ((uint32_t)old == members - 1) {
        if (!sync_tags_match(old, tag, members)) bad = kSyncMixed;
        // the group's counter is reset after the top counter's add, so that
        // add does not queue behind the store
        const uint64_t top = add_agent64(sync_top(sync), inc);
        const bool last = (uint32_t)top == ng - 1;
        if (last && !sync_tags_match(top, tag, ng)) bad = kSyncMixed;
        if (bad) or_err(sync, bad);
        st_agent64(sync_sub(sync, g), 0u);
        if (last) {
            st_agent64(sync_top(sync), 0u);
            const uint64_t rel = (((gen0 >> 32) + 1) << 32) | tag;
            for (uint32_t i = 0; i < ng; i++) st_agent64(sync_gen(sync, i), rel);
            return bad;
        }
    }
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
        const uint64_t v = ld_agent64(gen);
        if (v != gen0) {
            if ((uint32_t)v == tag) break;  // this launch's release
            if (!(bad & kSyncMixed)) {
                bad |= kSyncMixed;          // another launch's release
                or_err(sync, kSyncMixed);
            }
        }
        __builtin_amdgcn_s_sleep(4);
        if (__builtin_amdgcn_s_memrealtime() - t0 > timeout_ticks) {
            or_err(sync, kSyncTimeout);
            bad |= kSyncTimeout;
            break;
        }
    }
    asm volatile("" ::: "memory");
    return bad;
}

// max over the 64 lanes, every lane gets it: DPP within each 16-lane row,
// then the four row maxima through readlane (no LDS round trips)
__device__ __forceinline__ uint32_t wave_max_dpp(uint32_t m) {
    m = umax(m, dpp_u32<kDppQuadXor1>(m));
    m = umax(m, dpp_u32<kDppQuadXor2>(m));
    m = umax(m, dpp_u32<kDppHalfMirror>(m));
    m = umax(m, dpp_u32<kDppRowMirror>(m));
    const uint32_t r0 = __builtin_amdgcn_readlane(m, 0), r1 = __builtin_amdgcn_readlane(m, 16);
    const uint32_t r2 = __builtin_amdgcn_readlane(m, 32), r3 = __builtin_amdgcn_readlane(m, 48);
    return umax(umax(r0, r1), umax(r2, r3));
}

// Range-checked buffer access (make_rsrc): a load past the resource's
// range returns zeros and a store past it is dropped (stores write through
// the L2, kCpolSc1), so the resident
// kernel's per-lane edge cases need no branches, and the compiler's
// s_waitcnt counts stay exact (a branch around a load makes it drain
// every load in flight at the join).  kOff is past every range.
constexpr uint32_t kOff = 0x80000000u;
__device__ __forceinline__ float4 load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 v = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void store1(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t v) {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, kCpolSc1);
}
__device__ __forceinline__ void store4(__amdgpu_buffer_rsrc_t r, uint32_t off, v4i v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, v), r, off, 0, kCpolSc1);
}
template <bool B_>
struct BoolTag {
    static constexpr bool value = B_;
};

__global__ void __launch_bounds__(kRT)
k_quantize_resident(const float* __restrict__ A, const float* __restrict__ B, uint32_t N, uint32_t K,
                    uint64_t nA4, uint64_t perA4, uint32_t nTiles, uint32_t perT,
                    uint32_t* __restrict__ partials, int8_t* __restrict__ qA, int8_t* __restrict__ qBt,
                    float* __restrict__ scales, uint32_t* __restrict__ sync, uint32_t tag,
                    uint64_t timeout_ticks, uint32_t* __restrict__ status) {
    __shared__ float4 As[kRLdsA4];
    __shared__ uint32_t red[2 * (kRT / kWave)];
    uint32_t* tileT = reinterpret_cast<uint32_t*>(As);  // phase 2, once A's LDS part is written out
    const uint32_t t = threadIdx.x, wv = t >> 6, lane = t & 63;
    const uint32_t G = gridDim.x, w = blockIdx.x;
    const uint32_t ntn = N / kBTN;
    // Share index: workgroups go to the eight XCDs round-robin (w % 8), and
    // shares that are contiguous per XCD (one block of A and one run of B's
    // tiles for each XCD) measured faster to read than shares interleaved
    // across the XCDs (4096^3: phase 1 about 3 us sooner).  Any order is
    // correct; this one is a permutation of 0 .. G-1.
    const uint32_t ws = G % 8 == 0 ? (w % 8) * (G / 8) + w / 8 : w;

    // ---- phase 1: every operand byte read once.  Vector-memory loads
    // complete in issue order, so the copies of A's LDS part go first: they
    // are waited for (by count) and reduced while the B tiles, A's VGPR part
    // and the first batch of A's rest are still in flight.
    //   A: share ws's nw float4s from a0.  The first kRLdsA4 are copied
    //      into LDS (a wave copies only whole 64-slot runs that start below
    //      nres, so no copy writes past As), the next kRVA per thread are
    //      loaded into VGPRs, and the rest is read for the maximum here and
    //      read again in phase 2.
    //   B: share ws's perT tiles into VGPRs (tiles past the last read as zeros).
    const uint64_t a0 = (uint64_t)ws * perA4;
    const uint32_t nw = a0 < nA4 ? (uint32_t)(a0 + perA4 < nA4 ? perA4 : nA4 - a0) : 0;
    const uint32_t nres = nw < kRLdsA4 ? nw : kRLdsA4;
    const __amdgpu_buffer_rsrc_t rsA = make_rsrc(A + 4 * a0, nw * 16u);
#pragma unroll
    for (uint32_t s = 0; s < kRLdsSteps; s++)
        if (s * kRT + wv * kWave < nres) copy16_to_lds(rsA, &As[s * kRT + wv * kWave], (s * kRT + t) * 16u);
    asm volatile("" ::: "memory");  // keeps the loads below after the copies

    const uint32_t tb0 = ws * perT;
    const uint32_t nt = nTiles > tb0 ? (nTiles - tb0 < perT ? nTiles - tb0 : perT) : 0;
    const uint32_t kq = t >> 4, nq = t & 15;
    const __amdgpu_buffer_rsrc_t rsB = make_rsrc(B, K * N * 4u);
    float4 bv[kRNT][4];
#pragma unroll
    for (int i = 0; i < kRNT; i++) {
        const uint32_t tile = tb0 + i;
        const uint32_t k0 = (tile / ntn) * kBTK, n0 = (tile % ntn) * kBTN;
        const uint32_t off = ((k0 + 4 * kq) * N + n0 + 4 * nq) * 4u;
#pragma unroll
        for (int r = 0; r < 4; r++) bv[i][r] = load4(rsB, (uint32_t)i < nt ? off + r * N * 4u : kOff);
    }
    float4 av[kRVA];
#pragma unroll
    for (int u = 0; u < kRVA; u++) av[u] = load4(rsA, (kRLdsA4 + u * kRT + t) * 16u);
    float4 rv[kRBatch];
#pragma unroll
    for (int u = 0; u < kRBatch; u++) rv[u] = load4(rsA, (kROnChip4 + u * kRT + t) * 16u);

    wait_vmcnt<kRNT * 4 + kRVA + kRBatch>();  // this wave's copies have landed
    lds_barrier();
    uint32_t mA = 0, mB = 0;
#pragma unroll
    for (uint32_t s = 0; s < kRLdsSteps; s++) {
        const uint32_t idx = s * kRT + t;
        const uint32_t m = absmax4(As[idx < kRLdsA4 ? idx : kRLdsA4 - 1]);
        mA = umax(mA, idx < nres ? m : 0u);
    }
#pragma unroll
    for (int i = 0; i < kRNT; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) mB = umax(mB, absmax4(bv[i][r]));
#pragma unroll
    for (int u = 0; u < kRVA; u++) mA = umax(mA, absmax4(av[u]));
#pragma unroll
    for (int u = 0; u < kRBatch; u++) mA = umax(mA, absmax4(rv[u]));
    for (uint32_t base = kROnChip4 + kRBatch * kRT; base < nw; base += kRBatch * kRT) {
#pragma unroll
        for (int u = 0; u < kRBatch; u++) rv[u] = load4(rsA, (base + u * kRT + t) * 16u);
#pragma unroll
        for (int u = 0; u < kRBatch; u++) mA = umax(mA, absmax4(rv[u]));
    }

    // ---- workgroup maxima, then the grid-wide wait
    mA = wave_max_dpp(mA);
    mB = wave_max_dpp(mB);
    if (lane == 0) {
        red[wv] = mA;
        red[kRT / kWave + wv] = mB;
    }
    __syncthreads();
    if (t == 0) {
        uint32_t ma = 0, mb = 0;
        for (int i = 0; i < kRT / kWave; i++) {
            ma = umax(ma, red[i]);
            mb = umax(mb, red[kRT / kWave + i]);
        }
        // this launch's record in the workspace: entry w = what workgroup w
        // saw at the wait, the count of entries at status[0] (written by
        // every launch, so no clearing is needed)
        const uint32_t bad = grid_arrive_wait(sync, partials, ma, mb, w, G, tag, timeout_ticks);
        st_agent(&status[1 + w], bad);
        if (w == 0) st_agent(&status[0], G);
    }
    __syncthreads();
    uint32_t pa = 0, pb = 0;
    for (uint32_t i = t; i < G; i += kRT) {
        pa = umax(pa, ld_agent(&partials[i]));
        pb = umax(pb, ld_agent(&partials[G + i]));
    }
    pa = wave_max_dpp(pa);
    pb = wave_max_dpp(pb);
    if (lane == 0) {
        red[wv] = pa;
        red[kRT / kWave + wv] = pb;
    }
    __syncthreads();
    pa = 0;
    pb = 0;
#pragma unroll
    for (int i = 0; i < kRT / kWave; i++) {
        pa = umax(pa, red[i]);
        pb = umax(pb, red[kRT / kWave + i]);
    }
    float scaleA, invA, scaleB, invB;
    quant_params(__uint_as_float(pa), scaleA, invA);
    quant_params(__uint_as_float(pb), scaleB, invB);
    if (w == 0 && t == 0) {
        scales[0] = scaleA;
        scales[1] = scaleB;
    }

    // ---- phase 2, straight-line for one quantizer (pack4_fast when both
    // tensors allow it, else the exact pack4 for both).  Order: A from VGPRs
    // (freeing them for the first batch of A's rest, whose loads then fly
    // under the stores that follow), A from LDS, then the B tiles (packed
    // and staged in A's freed LDS at i * kTileDw, one barrier, read back as
    // 128-byte qBt row segments), then A's rest.  K % 128 == 0, so float4 j
    // of A is dword j of qA.
    const __amdgpu_buffer_rsrc_t rsQ = make_rsrc(reinterpret_cast<uint32_t*>(qA) + a0, nw * 4u);
    const __amdgpu_buffer_rsrc_t rsQB = make_rsrc(qBt, K * N);
    auto phase2 = [&](auto tag, auto full_tag) {
        constexpr bool F = decltype(tag)::value;
        // U: A's LDS and VGPR parts are full here, so their stores need no
        // guard; otherwise workgroup-uniform guards skip the arithmetic on
        // zeros (workgroups holding little or no A)
        constexpr bool U = decltype(full_tag)::value;
        auto q4 = [&](float a, float b, float c, float d, float inv) {
            return F ? pack4_fast(a, b, c, d, inv) : pack4(a, b, c, d, inv);
        };
#pragma unroll
        for (int u = 0; u < kRVA; u++)
            if (U || kRLdsA4 + u * kRT < nw)
                store1(rsQ, (kRLdsA4 + u * kRT + t) * 4u, q4(av[u].x, av[u].y, av[u].z, av[u].w, invA));
        // the first batch of A's rest: loaded here on the fast path, after
        // the B tiles on the exact one (whose pack4 needs more registers)
        auto load_rest = [&] {
#pragma unroll
            for (int u = 0; u < kRVA; u++) av[u] = load4(rsA, (kROnChip4 + u * kRT + t) * 16u);
        };
        if (F) load_rest();
#pragma unroll
        for (uint32_t s = 0; s < kRLdsSteps; s++) {
            if (U || s * kRT < nres) {
                const uint32_t idx = s * kRT + t;
                const float4 v = As[idx < kRLdsA4 ? idx : kRLdsA4 - 1];
                store1(rsQ, idx < nres ? idx * 4u : kOff, q4(v.x, v.y, v.z, v.w, invA));
            }
        }
        wait_lgkmcnt0();  // every read of As is done: the B transposes reuse it
        lds_barrier();
#pragma unroll
        for (int i = 0; i < kRNT; i++) {
            uint32_t* buf = tileT + i * kTileDw;
            buf[(4 * nq + 0) * kTileRowDw + kq] = q4(bv[i][0].x, bv[i][1].x, bv[i][2].x, bv[i][3].x, invB);
            buf[(4 * nq + 1) * kTileRowDw + kq] = q4(bv[i][0].y, bv[i][1].y, bv[i][2].y, bv[i][3].y, invB);
            buf[(4 * nq + 2) * kTileRowDw + kq] = q4(bv[i][0].z, bv[i][1].z, bv[i][2].z, bv[i][3].z, invB);
            buf[(4 * nq + 3) * kTileRowDw + kq] = q4(bv[i][0].w, bv[i][1].w, bv[i][2].w, bv[i][3].w, invB);
        }
        wait_lgkmcnt0();
        lds_barrier();
        {
            const uint32_t n = t >> 3, part = t & 7;
#pragma unroll
            for (int i = 0; i < kRNT; i++) {
                const uint32_t* row = tileT + i * kTileDw + n * kTileRowDw + part * 4;
                const v4i v = {(int)row[0], (int)row[1], (int)row[2], (int)row[3]};
                const uint32_t tile = tb0 + i;
                const uint32_t k0 = (tile / ntn) * kBTK, n0 = (tile % ntn) * kBTN;
                store4(rsQB, (uint32_t)i < nt ? (n0 + n) * K + k0 + part * 16 : kOff, v);
            }
        }
        if (!F) load_rest();
#pragma unroll
        for (int u = 0; u < kRVA; u++)
            if (kROnChip4 + u * kRT < nw)
                store1(rsQ, (kROnChip4 + u * kRT + t) * 4u, q4(av[u].x, av[u].y, av[u].z, av[u].w, invA));
        for (uint32_t base = kROnChip4 + kRVA * kRT; base < nw; base += kRBatch * kRT) {
            float4 v[kRBatch];
#pragma unroll
            for (int u = 0; u < kRBatch; u++) v[u] = load4(rsA, (base + u * kRT + t) * 16u);
#pragma unroll
            for (int u = 0; u < kRBatch; u++)
                store1(rsQ, (base + u * kRT + t) * 4u, q4(v[u].x, v[u].y, v[u].z, v[u].w, invA));
        }
    };
    if (!fast_quant_ok(__uint_as_float(pa), invA) || !fast_quant_ok(__uint_as_float(pb), invB))
        phase2(BoolTag<false>{}, BoolTag<false>{});
    else if (nw >= kROnChip4)
        phase2(BoolTag<true>{}, BoolTag<true>{});
    else
        phase2(BoolTag<true>{}, BoolTag<false>{});
}

// ------------------------------------------------------------ strip route
// dense_fused_i8 with at most 16 rows of A, in one launch.  Workgroup w (one
// per CU, all resident, the grid-wide wait above) holds strip ws of B -- its
// 16 columns n0 = 16 ws .. n0 + 15 over all K rows -- in VGPRs, and a share
// of A for the maximum; after the wait it quantizes the strip into LDS as
// 16 qBt rows and all of A as 16 qA rows (zeros past M), with pack4 /
// pack4_fast under the resident route's condition (so the same bytes), and
// contracts them with v_mfma_i32_16x16x64_i8 as k_fused_small does (lane
// (g, c16) gives row c16 of qA and column c16 of the strip the same 16
// bytes of each 64-byte step; the eight waves take every eighth step and
// their int32 sums meet in LDS, exact in any order).  Then the contraction
// kernels' epilogue for C's 16 columns.  B is read once and qBt never goes
// through memory: against the resident quantizer plus a contraction launch
// this saves qBt's write and re-read and one launch.  qA and qBt are not
// written (the quantize entry point keeps the resident route).
//   B: thread (rq = t / 4, cq = t % 4) holds rows 512 i + 4 rq + j (j < 4)
//      x columns n0 + 4 cq .. +3, one float4 each: 4 consecutive k of a
//      column pack into one qBt dword.
//   A: rows m < M, float4 c = t and t + 512 of each row (K / 4 <= 1024);
//      rows 0-7 are loaded before the wait (into VGPRs beside the strip),
//      rows 8-15 once the strip is packed.
// Shapes: M <= 16, K % 512 == 0, K <= 4096, N % 16 == 0, N / 16 <= the
// grid, 16-byte aligned A and B, and K * N * 4 < 2^31.
constexpr uint32_t kSMaxK = 4096;
constexpr int kSNI = kSMaxK / 512;          // float4 row groups per thread of the strip
constexpr uint32_t kSStride = kSMaxK + 16;  // bytes per staged row: rows 4 banks apart
constexpr int kSPre = 4;                    // rows of A loaded before the wait: 2 x kSPre

__global__ void __launch_bounds__(kRT)
k_fused_strip(const float* __restrict__ A, const float* __restrict__ B, uint32_t M, uint32_t N, uint32_t K,
              uint32_t perA4, float smul, float lo, float* __restrict__ C, uint32_t* __restrict__ partials,
              float* __restrict__ scales, uint32_t* __restrict__ sync, uint32_t tag, uint64_t timeout_ticks,
              uint32_t* __restrict__ status) {
    __shared__ __attribute__((aligned(16))) int8_t qa[16 * kSStride];
    __shared__ __attribute__((aligned(16))) int8_t qb[16 * kSStride];
    __shared__ v4i part[kRT / kWave][kWave];
    __shared__ uint32_t red[2 * (kRT / kWave)];
    const uint32_t t = threadIdx.x, wv = t >> 6, lane = t & 63;
    const uint32_t G = gridDim.x, w = blockIdx.x;
    // strips contiguous per XCD, as the resident quantizer's shares
    const uint32_t ws = G % 8 == 0 ? (w % 8) * (G / 8) + w / 8 : w;
    const bool has = ws < N / 16;
    const uint32_t n0 = ws * 16, ni = K / 512, K4 = K / 4;

    // ---- phase 1: the strip, A's share (for the maximum) and A's first rows
    const uint32_t rq = t >> 2, cq = t & 3;
    const __amdgpu_buffer_rsrc_t rsB = make_rsrc(B, K * N * 4u);
    float4 bv[kSNI][4];
#pragma unroll
    for (int i = 0; i < kSNI; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            bv[i][j] = load4(rsB, has && (uint32_t)i < ni ? ((512 * i + 4 * rq + j) * N + n0 + 4 * cq) * 4u : kOff);
    const uint32_t nA4 = M * K4;
    const __amdgpu_buffer_rsrc_t rsA = make_rsrc(A, nA4 * 16u);
    const uint32_t a0 = w * perA4;
    const float4 ash = load4(rsA, t < perA4 && a0 + t < nA4 ? (a0 + t) * 16u : kOff);
    auto a_off = [&](uint32_t m, uint32_t h) {
        const uint32_t c = t + 512 * h;
        return m < M && c < K4 ? (m * K4 + c) * 16u : kOff;
    };
    float4 ap[kSPre][2], ab[4][2];
#pragma unroll
    for (int m = 0; m < kSPre; m++)
#pragma unroll
        for (int h = 0; h < 2; h++) ap[m][h] = load4(rsA, a_off(m, h));
#pragma unroll
    for (int m = 0; m < 4; m++)
#pragma unroll
        for (int h = 0; h < 2; h++) ab[m][h] = load4(rsA, a_off(kSPre + m, h));
    // qA rows past M read as zeros in the contraction
    for (uint32_t r = M; r < 16; r++)
#pragma unroll
        for (uint32_t h = 0; h < 2; h++)
            if (t + 512 * h < K4) *reinterpret_cast<uint32_t*>(qa + r * kSStride + 4 * (t + 512 * h)) = 0;

    uint32_t mA = absmax4(ash), mB = 0;
#pragma unroll
    for (int i = 0; i < kSNI; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) mB = umax(mB, absmax4(bv[i][j]));
    mA = wave_max_dpp(mA);
    mB = wave_max_dpp(mB);
    if (lane == 0) {
        red[wv] = mA;
        red[kRT / kWave + wv] = mB;
    }
    __syncthreads();
    if (t == 0) {
        uint32_t ma = 0, mb = 0;
        for (int i = 0; i < kRT / kWave; i++) {
            ma = umax(ma, red[i]);
            mb = umax(mb, red[kRT / kWave + i]);
        }
        const uint32_t bad = grid_arrive_wait(sync, partials, ma, mb, w, G, tag, timeout_ticks);
        st_agent(&status[1 + w], bad);
        if (w == 0) st_agent(&status[0], G);
    }
    __syncthreads();
    uint32_t pa = 0, pb = 0;
    for (uint32_t i = t; i < G; i += kRT) {
        pa = umax(pa, ld_agent(&partials[i]));
        pb = umax(pb, ld_agent(&partials[G + i]));
    }
    pa = wave_max_dpp(pa);
    pb = wave_max_dpp(pb);
    if (lane == 0) {
        red[wv] = pa;
        red[kRT / kWave + wv] = pb;
    }
    __syncthreads();
    pa = 0;
    pb = 0;
#pragma unroll
    for (int i = 0; i < kRT / kWave; i++) {
        pa = umax(pa, red[i]);
        pb = umax(pb, red[kRT / kWave + i]);
    }
    float sa, ia, sb, ib;
    quant_params(__uint_as_float(pa), sa, ia);
    quant_params(__uint_as_float(pb), sb, ib);
    if (w == 0 && t == 0) {
        scales[0] = sa;
        scales[1] = sb;
    }
    const bool fa = fast_quant_ok(__uint_as_float(pa), ia), fb = fast_quant_ok(__uint_as_float(pb), ib);

    // ---- phase 2: the strip and A packed into LDS, each tensor with pack4_fast
    // or pack4 (one instantiation each, chosen per tensor as the resident
    // route does: the same bytes either way)
    auto pack_b = [&](auto ftag) {
        constexpr bool F = decltype(ftag)::value;
#pragma unroll
        for (int i = 0; i < kSNI; i++) {
            if ((uint32_t)i < ni) {
                int8_t* dst = qb + 4 * cq * kSStride + 512 * i + 4 * rq;
                auto q4 = [&](float a, float b, float c, float d) {
                    return F ? pack4_fast(a, b, c, d, ib) : pack4(a, b, c, d, ib);
                };
                *reinterpret_cast<uint32_t*>(dst) = q4(bv[i][0].x, bv[i][1].x, bv[i][2].x, bv[i][3].x);
                *reinterpret_cast<uint32_t*>(dst + kSStride) = q4(bv[i][0].y, bv[i][1].y, bv[i][2].y, bv[i][3].y);
                *reinterpret_cast<uint32_t*>(dst + 2 * kSStride) =
                    q4(bv[i][0].z, bv[i][1].z, bv[i][2].z, bv[i][3].z);
                *reinterpret_cast<uint32_t*>(dst + 3 * kSStride) =
                    q4(bv[i][0].w, bv[i][1].w, bv[i][2].w, bv[i][3].w);
            }
        }
    };
    if (has) {
        if (fb)
            pack_b(BoolTag<true>{});
        else
            pack_b(BoolTag<false>{});
    }
    auto pack_a = [&](auto ftag) {
        constexpr bool F = decltype(ftag)::value;
        auto put = [&](uint32_t m, uint32_t h, float4 v) {
            const uint32_t c = t + 512 * h;
            if (m < M && c < K4)
                *reinterpret_cast<uint32_t*>(qa + m * kSStride + 4 * c) =
                    F ? pack4_fast(v.x, v.y, v.z, v.w, ia) : pack4(v.x, v.y, v.z, v.w, ia);
        };
#pragma unroll
        for (int m = 0; m < kSPre; m++)
#pragma unroll
            for (int h = 0; h < 2; h++) put(m, h, ap[m][h]);
        if (M > kSPre + 4) {
            float4 ar[8][2];
#pragma unroll
            for (int m = 0; m < 8; m++)
#pragma unroll
                for (int h = 0; h < 2; h++) ar[m][h] = load4(rsA, a_off(kSPre + 4 + m, h));
#pragma unroll
            for (int m = 0; m < 4; m++)
#pragma unroll
                for (int h = 0; h < 2; h++) put(kSPre + m, h, ab[m][h]);
#pragma unroll
            for (int m = 0; m < 8; m++)
#pragma unroll
                for (int h = 0; h < 2; h++) put(kSPre + 4 + m, h, ar[m][h]);
        } else {
#pragma unroll
            for (int m = 0; m < 4; m++)
#pragma unroll
                for (int h = 0; h < 2; h++) put(kSPre + m, h, ab[m][h]);
        }
    };
    if (fa)
        pack_a(BoolTag<true>{});
    else
        pack_a(BoolTag<false>{});
    __syncthreads();
    if (!has) return;

    // ---- the contraction: wave wv takes 64-byte steps wv, wv + 8, ... (at
    // most kSMaxK / 512 of them), every fragment read issued first
    const uint32_t g = lane >> 4, c16 = lane & 15;
    constexpr int kSSteps = kSMaxK / (64 * (kRT / kWave));
    v4i fa4[kSSteps], fb4[kSSteps];
#pragma unroll
    for (int u = 0; u < kSSteps; u++) {
        const uint32_t k0 = (wv + (kRT / kWave) * u) * 64;
        if (k0 < K) {
            fa4[u] = *reinterpret_cast<const v4i*>(qa + c16 * kSStride + k0 + 16 * g);
            fb4[u] = *reinterpret_cast<const v4i*>(qb + c16 * kSStride + k0 + 16 * g);
        }
    }
    v4i acc = {0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < kSSteps; u++)
        if ((wv + (kRT / kWave) * u) * 64 < K) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa4[u], fb4[u], acc, 0, 0, 0);
    part[wv][lane] = acc;
    __syncthreads();
    if (wv == 0) {
        v4i s4 = part[0][lane];
#pragma unroll
        for (int i = 1; i < kRT / kWave; i++) s4 += part[i][lane];
        const float s = __fmul_rn(__fmul_rn(sa, sb), smul);
        const uint32_t n = n0 + c16;
#pragma unroll
        for (int i = 0; i < 4; i++) {  // D lane (g, c16), register i: row 4g + i, column c16
            const uint32_t m = 4 * g + i;
            if (m < M) C[(uint64_t)m * N + n] = fmax_a(__fadd_rn(__fmul_rn((float)s4[i], s), 0.0f), lo);
        }
    }
}

// The wait's slot in device memory: zero when the code object loads, left
// with its counters at rest by every launch.  Launches that wait on it
// (k_quantize_resident, k_fused_strip) are ordered per device
// (launch_grid_wait), so one slot per device serves them all.
__device__ __align__(256) uint32_t resident_sync[kSyncSlotDw];

struct ResidentDevice {
    uint32_t* sync = nullptr;  // device address of resident_sync
    // CUs x resident workgroups per CU of each kernel that waits on the
    // slot (0: that route is unusable)
    uint32_t grid = 0;        // k_quantize_resident
    uint32_t grid_strip = 0;  // k_fused_strip
    bool probed = false;
    // The last grid-wide-wait launch made by a host call: two grids that
    // each need every CU must not run at once (their workgroups would split
    // the CUs and neither grid could pass its wait), so a launch on another
    // stream first waits for this event.
    hipEvent_t last = nullptr;
    hipStream_t last_stream = nullptr;
    bool last_valid = false;
    uint32_t tag = 0;  // the last launch's tag (launches are numbered from 1)
};
std::mutex g_res_mu;
ResidentDevice g_res_dev[64];
std::atomic<uint64_t> g_wait_limit{kSyncTimeoutTicks};

// ANE_COOPERATIVE=0 in the environment makes the uncaptured launches plain
// ones too (for tools that do not handle cooperative launches: rocprofv3's
// teardown has crashed after them); read once.
bool cooperative_launches() {
    static const bool on = [] {
        const char* e = std::getenv("ANE_COOPERATIVE");
        return !(e && std::strcmp(e, "0") == 0);
    }();
    return on;
}

// The device's slot and grids (probed once per device, with it current);
// null when the slot is unavailable (then the routes without a grid-wide
// wait run).  Called with g_res_mu held.
ResidentDevice* resident_device(hipStream_t s, int* dev_out) {
    if (s == hipStreamPerThread) return nullptr;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    ResidentDevice& d = g_res_dev[dev];
    if (!d.probed) {
        d.probed = true;
        void* p = nullptr;
        int cus = 0, occ = 0, occ_strip = 0;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(resident_sync)) != hipSuccess || !p ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k_quantize_resident, kRT, 0) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ_strip, k_fused_strip, kRT, 0) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        d.sync = (uint32_t*)p;
        if (cus > 0 && occ > 0 && (uint64_t)cus * occ <= kFusedPartials) d.grid = (uint32_t)(cus * occ);
        if (cus > 0 && occ_strip > 0 && (uint64_t)cus * occ_strip <= kFusedPartials)
            d.grid_strip = (uint32_t)(cus * occ_strip);
    }
    if (!d.sync) return nullptr;
    *dev_out = dev;
    return &d;
}

// What the grid-wide-wait launches share: the capture check, the ordering
// of such launches per device, the launch tag and the choice of a
// cooperative launch.  `fits(G)` checks the shape against the kernel's grid
// G (d.*grid_of); `go(G, sync, tag, limit, coop)` queues the kernel and
// returns the launch call's error.  Returns true when the kernel was queued
// (*status = ANE_ERR_HIP if it failed after that), false when the route
// cannot run (nothing queued: the caller takes another route).
template <class Fits, class Go>
bool launch_grid_wait(hipStream_t s, uint32_t ResidentDevice::*grid_of, Fits fits, Go go, int* status) {
    *status = ANE_OK;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cap) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    const bool capturing = cap != hipStreamCaptureStatusNone;
    std::lock_guard<std::mutex> lock(g_res_mu);
    int dev = 0;
    ResidentDevice* dp = resident_device(s, &dev);
    if (!dp) return false;
    ResidentDevice& d = *dp;
    const uint32_t G = d.*grid_of;
    if (!G || !fits(G)) return false;
    // Grid-wide-wait launches on one device are ordered: a launch on another
    // stream than the previous one waits for it.  A captured launch cannot
    // wait for work outside its graph, so under capture the route is taken
    // only on the stream of the previous launch (graph replays are ordered
    // by their caller).
    const bool other = d.last_valid && d.last_stream != s;
    if (capturing && other) return false;
    if (!capturing) {
        if (!d.last && hipEventCreateWithFlags(&d.last, hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            d.last = nullptr;
            return false;
        }
        if (other && hipStreamWaitEvent(s, d.last, 0) != hipSuccess) {
            (void)hipGetLastError();
            return false;
        }
    }
    // Outside capture the grid goes out as a cooperative launch: the runtime
    // then starts it only with every workgroup resident at once, or refuses
    // it (another route runs instead).  A captured launch is a plain one;
    // the ordering above and the bounded, tagged wait cover it.
    if (++d.tag == 0) d.tag = 1;
    const bool coop = !capturing && cooperative_launches();
    if (go(G, d.sync, d.tag, g_wait_limit.load(std::memory_order_relaxed), coop) != hipSuccess) {
        (void)hipGetLastError();
        if (coop) return false;  // refused before anything was queued
        *status = ANE_ERR_HIP;
        return true;
    }
    if (!capturing) {
        if (hipEventRecord(d.last, s) != hipSuccess) {
            (void)hipGetLastError();
            *status = ANE_ERR_HIP;
            return true;
        }
        d.last_stream = s;
        d.last_valid = true;
    }
    return true;
}

// The resident route, when the shape allows it: whole 128 x 64 B tiles
// (K % 128 == 0, N % 64 == 0), 16-byte aligned operands, and at most kRNT
// B tiles per workgroup.  Returns true when it launched.
bool launch_resident(const float* A, const float* B, uint32_t M, uint32_t N, uint32_t K,
                     uint32_t* partials, int8_t* qA, int8_t* qBt, float* scales, uint32_t* wstatus,
                     hipStream_t s, int* status) {
    *status = ANE_OK;
    if (K == 0 || M == 0 || N == 0 || (K % kBTK) || (N % kBTN)) return false;
    // below ~12 MiB of operands the two launches of the two-pass route are
    // faster than one grid-wide wait (measured: 1024^3 7.7 against 9.0 us,
    // 64 x 2048 x 2048 10.0 against 9.4 us)
    if (((uint64_t)M * K + (uint64_t)K * N) * 4 < kResidentMinBytes) return false;
    if ((((uintptr_t)A) | ((uintptr_t)B)) & 15) return false;
    const uint64_t nTiles = (uint64_t)(K / kBTK) * (N / kBTN);
    const uint64_t nA4 = (uint64_t)M * K / 4;
    uint32_t perT = 0;
    uint64_t perA4 = 0;
    auto fits = [&](uint32_t G) {
        if (nTiles > (uint64_t)kRNT * G) return false;
        perT = (uint32_t)((nTiles + G - 1) / G);
        perA4 = (nA4 + G - 1) / G;
        // the kernel's buffer offsets are 32-bit byte offsets below kOff
        return perA4 * 16 < kOff && (uint64_t)K * N * 4 < kOff;
    };
    auto go = [&](uint32_t G, uint32_t* sync, uint32_t tag, uint64_t limit, bool coop) {
        const float* kA = A;
        const float* kB = B;
        uint32_t kN = N, kK = K, kTiles = (uint32_t)nTiles, kPerT = perT, kTag = tag;
        uint64_t kNA4 = nA4, kPerA4 = perA4, kLimit = limit;
        uint32_t* kPartials = partials;
        int8_t* kQA = qA;
        int8_t* kQBt = qBt;
        float* kScales = scales;
        uint32_t* kSync = sync;
        uint32_t* kStatus = wstatus;
        if (coop) {
            void* args[] = {&kA, &kB, &kN, &kK, &kNA4, &kPerA4, &kTiles, &kPerT, &kPartials, &kQA, &kQBt,
                            &kScales, &kSync, &kTag, &kLimit, &kStatus};
            return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(k_quantize_resident), dim3(G),
                                              dim3(kRT), args, 0, s);
        }
        hipLaunchKernelGGL(k_quantize_resident, dim3(G), dim3(kRT), 0, s, kA, kB, kN, kK, kNA4, kPerA4, kTiles,
                           kPerT, kPartials, kQA, kQBt, kScales, kSync, kTag, kLimit, kStatus);
        return hipGetLastError();
    };
    return launch_grid_wait(s, &ResidentDevice::grid, fits, go, status);
}

// The current device's slot, if the resident route was ever set up on it.
uint32_t* resident_slot_of() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(g_res_mu);
    return g_res_dev[dev].sync;
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
                          uint32_t* wstatus, hipStream_t s) {
    int st = ANE_OK;
    if (Kp == K && launch_resident(A, B, M, N, K, partials, qA, qBt, scales, wstatus, s, &st)) return st;
    const uint64_t nA = (uint64_t)M * K, nB = (uint64_t)K * N;
    const uint32_t nbA = blocks_for(nA), nbB = blocks_for(nB);
    hipLaunchKernelGGL(k_absmax_two, dim3(nbA + nbB), dim3(kT), 0, s, A, nA, nbA, B, nB, nbB, partials);
    uint64_t nqA = ((uint64_t)M * (Kp / 16) + 2 * kT - 1) / (2 * kT);
    if (nqA > 4096) nqA = 4096;
    if (nqA < 1) nqA = 1;
    const uint64_t nqB = Kp ? ((uint64_t)Kp / kBTK) * (((uint64_t)N + kBTN - 1) / kBTN) : 1;
    if (nqA + nqB > 0x7fffffffull) return ANE_ERR_INVALID_ARG;
    hipLaunchKernelGGL(k_quantize_two, dim3((uint32_t)(nqA + nqB)), dim3(kT), 0, s, A, B, M, N, K, Kp,
                       partials, nbA, nbB, (uint32_t)nqA, qA, qBt, scales, wstatus);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

bool small_fused_eligible(uint32_t M, uint32_t N, uint32_t K) {
    if (M == 0 || N == 0 || K == 0 || K > kSmallMaxK) return false;
    // every workgroup reads its 16 rows of A and 16 columns of B whole: the
    // route is for few tiles and operands small enough that those re-reads
    // stay cheap
    const uint64_t tm = (M + 15) / 16, tn = (N + 15) / 16;
    return tm * tn <= kSmallMaxTiles && (uint64_t)M * K * tn + (uint64_t)K * N * tm <= kSmallMaxReads;
}

int launch_fused_small(const float* A, const float* B, uint32_t M, uint32_t N, uint32_t K, float smul, float lo,
                       float* C, uint32_t* partials, float* scales, uint32_t* wstatus, hipStream_t s) {
    if (!small_fused_eligible(M, N, K)) return ANE_ERR_INVALID_ARG;
    const uint64_t nA = (uint64_t)M * K, nB = (uint64_t)K * N;
    const uint32_t nbA = blocks_for(nA), nbB = blocks_for(nB);
    hipLaunchKernelGGL(k_absmax_two, dim3(nbA + nbB), dim3(kT), 0, s, A, nA, nbA, B, nB, nbB, partials);
    hipLaunchKernelGGL(k_fused_small, dim3((N + 15) / 16, (M + 15) / 16), dim3(kT), 0, s, A, B, M, N, K, partials,
                       nbA, nbB, smul, lo, C, scales, wstatus);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

bool strip_fused_eligible(uint32_t M, uint32_t N, uint32_t K, const float* A, const float* B) {
    if (M == 0 || M > 16 || N == 0 || N % 16 || K == 0 || K % 512 || K > kSMaxK) return false;
    if ((((uintptr_t)A) | ((uintptr_t)B)) & 15) return false;
    // as for the resident quantizer: below ~12 MiB of B the launches
    // without a grid-wide wait are the faster ones
    return (uint64_t)K * N * 4 >= kResidentMinBytes && (uint64_t)K * N * 4 < kOff;
}

bool launch_fused_strip(const float* A, const float* B, uint32_t M, uint32_t N, uint32_t K, float smul, float lo,
                        float* C, uint32_t* partials, float* scales, uint32_t* wstatus, hipStream_t s,
                        int* status) {
    *status = ANE_OK;
    if (!strip_fused_eligible(M, N, K, A, B)) return false;
    const uint64_t nA4 = (uint64_t)M * K / 4;
    uint32_t perA4 = 0;
    auto fits = [&](uint32_t G) {
        if (N / 16 > G) return false;  // one strip per workgroup
        perA4 = (uint32_t)((nA4 + G - 1) / G);
        return perA4 <= (uint32_t)kRT;  // one float4 of A's share per thread
    };
    auto go = [&](uint32_t G, uint32_t* sync, uint32_t tag, uint64_t limit, bool coop) {
        const float* kA = A;
        const float* kB = B;
        uint32_t kM = M, kN = N, kK = K, kPerA4 = perA4, kTag = tag;
        float kSmul = smul, kLo = lo;
        float* kC = C;
        uint32_t* kPartials = partials;
        float* kScales = scales;
        uint32_t* kSync = sync;
        uint64_t kLimit = limit;
        uint32_t* kStatus = wstatus;
        if (coop) {
            void* args[] = {&kA, &kB, &kM, &kN, &kK, &kPerA4, &kSmul, &kLo, &kC, &kPartials, &kScales,
                            &kSync, &kTag, &kLimit, &kStatus};
            return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(k_fused_strip), dim3(G), dim3(kRT),
                                              args, 0, s);
        }
        hipLaunchKernelGGL(k_fused_strip, dim3(G), dim3(kRT), 0, s, kA, kB, kM, kN, kK, kPerA4, kSmul, kLo, kC,
                           kPartials, kScales, kSync, kTag, kLimit, kStatus);
        return hipGetLastError();
    };
    return launch_grid_wait(s, &ResidentDevice::grid_strip, fits, go, status);
}

}  // namespace ane

extern "C" void ane_hip_set_grid_wait_limit(uint64_t ticks) {
    ane::g_wait_limit.store(ticks ? ticks : ane::kSyncTimeoutTicks, std::memory_order_relaxed);
}

namespace ane {

int resident_slot_check(uint32_t* bits) {
    *bits = 0;
    uint32_t* slot = resident_slot_of();
    if (!slot) return ANE_OK;
    uint32_t err = 0;
    if (hipMemcpy(&err, slot + 2, 4, hipMemcpyDeviceToHost) != hipSuccess) {
        (void)hipGetLastError();
        return ANE_ERR_HIP;
    }
    *bits = err;
    if (!err) return ANE_OK;
    // Back to rest: once every launch on the device has ended, the top and
    // group counters and the error word are zeroed (the generation words
    // keep counting).  Arrivals of two launches mixed in one counter can
    // leave it short of, or past, a whole launch's count.
    if (hipDeviceSynchronize() != hipSuccess) {
        (void)hipGetLastError();
        return ANE_ERR_HIP;
    }
    static const uint32_t zeros[4] = {0, 0, 0, 0};
    bool ok = hipMemcpy(slot, zeros, 3 * sizeof(uint32_t), hipMemcpyHostToDevice) == hipSuccess;
    for (uint32_t g = 0; g < kSyncGroups && ok; g++)
        ok = hipMemcpy(slot + (1 + kSyncGroups + g) * kSyncLineDw, zeros, 2 * sizeof(uint32_t),
                       hipMemcpyHostToDevice) == hipSuccess;
    if (!ok) {
        (void)hipGetLastError();
        return ANE_ERR_HIP;
    }
    return ANE_OK;
}

bool resident_mixed_bit(uint32_t bits) { return (bits & kSyncMixed) != 0; }

}  // namespace ane

extern "C" int ane_hip_grid_wait_status(void* stream) {
    if (hipStreamSynchronize((hipStream_t)stream) != hipSuccess) {
        (void)hipGetLastError();
        return ANE_ERR_HIP;
    }
    uint32_t bits = 0;
    const int st = ane::resident_slot_check(&bits);
    if (st != ANE_OK) return st;
    return bits ? ANE_ERR_GRID_WAIT : ANE_OK;
}
