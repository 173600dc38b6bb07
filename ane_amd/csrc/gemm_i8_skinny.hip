// gemm_i8_skinny.hip -- the int8 contraction for few rows (M <= 128): the
// small-M end of dense_fused_i8's M sweep and gemm_s8_i32.  Output tiles of
// 128 x 128 would give 4096 columns only 32 workgroups, so the operand that
// matters, Bt (N x Kp), would stream through 32 CUs.
//
// Design (gfx950):
//  * One workgroup per 16 output columns: ceil(N/16) workgroups of 4 waves
//    (256 for N = 4096).  The workgroup holds every output row (up to 8
//    16-row blocks, MB) of its columns.
//  * K advances in 128-byte steps; wave w takes steps w, w+4, w+8, ... (the
//    four waves together read each Bt row front to back).  A step is two
//    v_mfma_i32_16x16x64_i8 per row block: lane l loads the 32 contiguous
//    bytes of column n0 + l%16 (Bt row) and of row 16rb + l%16 (A row) at
//    k = 128s + 32(l/16), and gives the first 16 to one instruction and the
//    next 16 to the other (so a pair of loads covers whole 128-byte lines;
//    measured 7 % faster than 64-byte steps at M = 16).  A and B place the
//    same k in the same lane and byte, so the int32 sums are the exact dot
//    products whatever order the instructions add in.
//  * With 4+ row blocks, the workgroups start their walks over K at four
//    different phases (a rotation of the steps, which changes no sum), so
//    the workgroups of an XCD do not all read the same lines of A at once
//    (M = 128: 20.6 -> 19.7 us).
//  * Operands are read straight into VGPRs with range-checked 16-byte buffer
//    loads (rows past M or N and k past Kp read as zeros), two steps per
//    batch, the next batch in flight while the current one is multiplied.
//    Bt is read once (non-temporal); A is small and shared through L2.
//  * The four waves' int32 accumulators meet in LDS (exact), and the fused
//    epilogue fmaxA(fadd(fmul((float)acc, s), bias), lo) (one rounding per
//    operation, as in the other contraction kernels) or the raw int32 goes
//    out.  D lane l, register i of a 16 x 16 block is row 4(l/16) + i,
//    column l%16.
#include "gemm_i8.hpp"

namespace ane {
namespace {

template <int MB>
__global__ void __launch_bounds__(256) k_gemm_skinny(GemmParams p) {
    __shared__ v4i red[4][MB][64];
    const uint32_t lane = threadIdx.x & 63, c16 = lane & 15, g = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t n0 = blockIdx.x * 16;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A, (uint32_t)(p.rowsA * p.lda));
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.B, (uint32_t)(p.colsB * p.ldb));
    const uint32_t nsteps = (p.Kp + 127) / 128;  // the last step may be partial: k < Kp decides per chunk
    const uint32_t nj = (nsteps + 3) / 4;  // this wave's steps, rounded up (extra steps read zeros)
    // the rotation of this workgroup's walk (4+ row blocks)
    const uint32_t phase = MB >= 4 ? (blockIdx.x & 3) * (nsteps / 4) : 0;
    const uint32_t offB = (n0 + c16) * (uint32_t)p.ldb + 32 * g;
    uint32_t offA[MB];
#pragma unroll
    for (int r = 0; r < MB; r++) offA[r] = (16 * r + c16) * (uint32_t)p.lda + 32 * g;

    // step j of this wave: 16-byte chunks h = 0, 1 at k = 128 S + 32 g + 16 h
    auto load = [&](uint32_t j, v4i (&b)[2], v4i (&a)[2][MB]) {
        uint32_t S = wave + 4 * j;
        const bool in = S < nsteps;
        if (in) S = (S + phase) % nsteps;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const bool live = in && 128 * S + 32 * g + 16 * h < p.Kp;
            b[h] = __builtin_bit_cast(
                v4i, __builtin_amdgcn_raw_buffer_load_b128(rb, live ? offB + 128 * S + 16 * h : 0x80000000u, 0, kCpolNt));
#pragma unroll
            for (int r = 0; r < MB; r++)
                a[h][r] = __builtin_bit_cast(
                    v4i, __builtin_amdgcn_raw_buffer_load_b128(ra, live ? offA[r] + 128 * S + 16 * h : 0x80000000u, 0, 0));
        }
    };
    auto mma = [&](v4i (&acc)[MB], const v4i (&b)[2], const v4i (&a)[2][MB]) {
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int r = 0; r < MB; r++) acc[r] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[h][r], b[h], acc[r], 0, 0, 0);
    };

    v4i acc[MB];
#pragma unroll
    for (int r = 0; r < MB; r++) acc[r] = v4i{0, 0, 0, 0};
    v4i b0[2], b1[2], a0[2][MB], a1[2][MB];
    load(0, b0, a0);
    for (uint32_t j = 0; j < nj; j += 2) {
        load(j + 1, b1, a1);
        mma(acc, b0, a0);
        load(j + 2, b0, a0);
        mma(acc, b1, a1);
    }

#pragma unroll
    for (int r = 0; r < MB; r++) red[wave][r][lane] = acc[r];
    __syncthreads();

    float s = p.s;
    if (p.sdev) s = __fmul_rn(__fmul_rn(p.sdev[0], p.sdev[1]), p.smul);
    const uint32_t j = n0 + c16;
    const float bj = (p.bias && j < p.Nout) ? p.bias[j] : 0.0f;
    for (uint32_t r = wave; r < (uint32_t)MB; r += 4) {
        const v4i t = red[0][r][lane] + red[1][r][lane] + red[2][r][lane] + red[3][r][lane];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t row = 16 * r + 4 * g + i;
            if (row >= p.Mout || j >= p.Nout) continue;
            if (p.Craw) {
                p.Craw[(uint64_t)row * p.ldc + j] = t[i];
            } else {
                const float f = __fadd_rn(__fmul_rn((float)t[i], s), bj);
                p.C[(uint64_t)row * p.ldc + j] = fmax_a(f, p.lo);
            }
        }
    }
}

}  // namespace

bool skinny_eligible(const GemmParams& p) {
    if (p.Mout == 0 || p.Mout > 128 || p.Nout == 0) return false;
    if (p.Kp == 0 || (p.Kp & 15)) return false;
    if ((p.lda & 15) || (p.ldb & 15)) return false;
    if ((((uintptr_t)p.A) & 15) || (((uintptr_t)p.B) & 15)) return false;
    if (p.rowsA < p.Mout || p.colsB < p.Nout) return false;
    // 32-bit buffer offsets; 0x80000000 marks an empty load: every row a
    // workgroup may touch (up to 16 past the last column, 128 A rows) and
    // every step stay below it
    const uint64_t kspan = ceil_to(p.Kp, 256) + 128;
    if ((uint64_t)ceil_to(p.Nout, 16) * p.ldb + kspan >= (1ull << 31)) return false;
    if (128ull * p.lda + kspan >= (1ull << 31)) return false;
    if ((uint64_t)p.rowsA * p.lda >= (1ull << 31) || (uint64_t)p.colsB * p.ldb >= (1ull << 31)) return false;
    return true;
}

int launch_gemm_skinny(const GemmParams& p, hipStream_t s) {
    const uint32_t mb = (p.Mout + 15) / 16;
    const dim3 grid((p.Nout + 15) / 16);
    switch (mb) {
        case 1: hipLaunchKernelGGL(k_gemm_skinny<1>, grid, dim3(256), 0, s, p); break;
        case 2: hipLaunchKernelGGL(k_gemm_skinny<2>, grid, dim3(256), 0, s, p); break;
        case 3:
        case 4: hipLaunchKernelGGL(k_gemm_skinny<4>, grid, dim3(256), 0, s, p); break;
        default: hipLaunchKernelGGL(k_gemm_skinny<8>, grid, dim3(256), 0, s, p); break;
    }
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

}  // namespace ane
