// igemm.hip -- the strided integer GEMMs cblas_igemm / cblas_ugemm /
// cblas_usgemm (opcodes 0x61-0x63) on the int8 MFMA contraction.
//
// Reference: the CBLAS_INTEGER_GEMM macro, src/bytecode_interpreter.s:8328-9135,
// instantiated at :9137-9139 with smopa, umopa and usmopa.  What it computes
// for the outputs it stores (rows < M, columns < N of C, stride ldc):
//   acc  = seed + sum_{k < 64*floor(K/64)} a(i,k) * b(k,j)   (wrapping int32)
//   seed = 0 when the bits of beta are zero, else the BIT PATTERN of
//          fl(beta * C[i][j]) (:8402-8488: the scaled C is moved into the
//          int32 za tiles before the products are accumulated)
//   C    = fl(fl32(acc) * alpha)                              (:8962-8980)
//   a(i,k) = A[i*lda + k]; with transA the handler adds the k offset to
//            A + ti and steps rows by lda (:8513-8514, :8562-8575), so row i
//            reads A[(i%16)*lda + (i - i%16) + k]
//   b(k,j) = B[k*ldb + j], or B[j*ldb + k] with transB (:8768-8872)
// ANE_IGEMM_BLAS instead computes what the handler's header describes:
// op(A) = A^T with transA, and C = fl(fl(fl32(acc)*alpha) + fl(beta*C)),
// C not read when beta == 0.
//
// Design.  The MFMA instruction multiplies signed bytes, so each operand is
// first gathered into K-contiguous signed rows (the layout the contraction
// kernels stream): a pre-pass per operand walks 64 x 64 tiles through LDS,
// reading along whichever direction is contiguous in memory.  An unsigned
// byte u is stored as u ^ 0x80 = u - 128, and the epilogue adds back
//   128 * sum_k b'(k,j)   (A unsigned)
//   128 * sum_k a'(i,k)   (B unsigned)
//   16384 * Ke            (both)
// which is exact modulo 2^32, like the handler's own wrapping sums.  The row
// sums come from the same pre-pass (integer atomics: order-free and exact).
// Signed operands that are already K-contiguous rows (A without transA, B
// with transB) with 16-byte aligned rows skip the pre-pass: the contraction
// reads them in place (1024^3 transB: 15.8 -> 10.8 us, two launches fewer).
#include "gemm_i8.hpp"

namespace ane {
namespace {

constexpr uint32_t kT = 64;  // tile rows x tile k of the pre-pass

// dst[r][k] = byte at src + r*rs + (r%16)*r16 + k*ks, flipped to signed
// when `flip`, for r < R, k < Ke (Ke % 64 == 0); sums[r] += its signed bytes.
__global__ void __launch_bounds__(256)
k_igemm_gather(uint32_t R, uint32_t Ke, const uint8_t* __restrict__ src, int64_t rs, int64_t r16, int64_t ks,
               uint32_t flip, int8_t* __restrict__ dst, int32_t* __restrict__ sums) {
    __shared__ uint8_t tile[kT][kT + 4];
    const uint32_t r0 = blockIdx.y * kT, k0 = blockIdx.x * kT, t = threadIdx.x;
    auto addr = [&](uint32_t r, uint32_t k) {
        return src + (int64_t)r * rs + (int64_t)(r & 15) * r16 + (int64_t)k * ks;
    };
    if (ks == 1) {
        // rows contiguous in memory: 4 lanes per row, 16 bytes each
        const uint32_t r = t >> 2, kk = (t & 3) * 16;
        if (r0 + r < R) {
            const uint8_t* p = addr(r0 + r, k0 + kk);
#pragma unroll
            for (int e = 0; e < 16; e++) tile[r][kk + e] = p[e] ^ flip;
        }
    } else {
        // columns contiguous (or strided both ways): lanes along the rows
        const uint32_t r = t & 63, kq = t >> 6;
        if (r0 + r < R) {
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const uint32_t kk = kq + 4 * e;
                tile[r][kk] = *addr(r0 + r, k0 + kk) ^ flip;
            }
        }
    }
    __syncthreads();
    const uint32_t r = t >> 2, kk = (t & 3) * 16;
    if (r0 + r >= R) return;
    uint32_t w[4];
    int32_t s = 0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        uint32_t v = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint8_t b = tile[r][kk + 4 * q + e];
            v |= (uint32_t)b << (8 * e);
            s += (int32_t)(int8_t)b;
        }
        w[q] = v;
    }
    *reinterpret_cast<uint4*>(dst + (uint64_t)(r0 + r) * Ke + k0 + kk) = make_uint4(w[0], w[1], w[2], w[3]);
    if (sums) {
        // the 4 lanes of a row are adjacent: fold them, then one atomic per row and tile
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        if ((t & 3) == 0) atomicAdd(sums + r0 + r, s);
    }
}

__global__ void __launch_bounds__(256) k_fill_i32(uint32_t n, int32_t* __restrict__ p) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0;
}

// C[i*ldc + j] for i < M, j < N from the signed-operand accumulators and
// the unsigned corrections; SEM 0 = the handler's arithmetic, 1 = BLAS.
template <int SEM>
__global__ void __launch_bounds__(256)
k_igemm_epilogue(uint32_t M, uint32_t N, const int32_t* __restrict__ acc, const int32_t* __restrict__ rowsum,
                 const int32_t* __restrict__ colsum, uint32_t corr, float alpha, float beta,
                 float* __restrict__ C, uint64_t ldc) {
    const uint32_t j = blockIdx.x * 64 + (threadIdx.x & 63);
    const uint32_t i = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (i >= M || j >= N) return;
    uint32_t a = acc ? (uint32_t)acc[(uint64_t)i * N + j] : 0u;
    if (colsum) a += 128u * (uint32_t)colsum[j];
    if (rowsum) a += 128u * (uint32_t)rowsum[i];
    a += corr;
    float* c = C + (uint64_t)i * ldc + j;
    if (SEM == 0) {
        if (__float_as_uint(beta) != 0u) a += __float_as_uint(__fmul_rn(beta, *c));
        *c = __fmul_rn((float)(int32_t)a, alpha);
    } else {
        float v = __fmul_rn((float)(int32_t)a, alpha);
        if (beta != 0.0f) v = __fadd_rn(v, __fmul_rn(beta, *c));
        *c = v;
    }
}

struct IgemmWs {
    int8_t *a, *bt;
    int32_t *acc, *rowsum, *colsum;
};

size_t igemm_layout(uint32_t M, uint32_t N, uint32_t K, uint8_t* base, IgemmWs* w) {
    const uint64_t Ke = (uint64_t)(K / 64) * 64;
    size_t off = 0;
    auto take = [&](uint64_t bytes) {
        const size_t o = off;
        off += ceil_to(bytes, 256);
        return base ? base + o : nullptr;
    };
    int8_t* a = reinterpret_cast<int8_t*>(take((uint64_t)M * Ke));
    int8_t* bt = reinterpret_cast<int8_t*>(take((uint64_t)N * Ke));
    int32_t* acc = reinterpret_cast<int32_t*>(take(Ke ? (uint64_t)M * N * 4 : 0));
    int32_t* rowsum = reinterpret_cast<int32_t*>(take((uint64_t)M * 4));
    int32_t* colsum = reinterpret_cast<int32_t*>(take((uint64_t)N * 4));
    if (w) *w = IgemmWs{a, bt, acc, rowsum, colsum};
    return off;
}

int gather(uint32_t R, uint32_t Ke, const void* src, int64_t rs, int64_t r16, int64_t ks, bool flip, int8_t* dst,
           int32_t* sums, hipStream_t s) {
    if (sums) {
        hipLaunchKernelGGL(k_fill_i32, dim3((R + 255) / 256), dim3(256), 0, s, R, sums);
    }
    const dim3 grid(Ke / kT, (R + kT - 1) / kT);
    hipLaunchKernelGGL(k_igemm_gather, grid, dim3(256), 0, s, R, Ke, static_cast<const uint8_t*>(src), rs, r16, ks,
                       flip ? 0x80u : 0u, dst, sums);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

}  // namespace
}  // namespace ane

using namespace ane;

extern "C" size_t ane_hip_cblas_igemm_workspace_size(uint32_t M, uint32_t N, uint32_t K) {
    return igemm_layout(M, N, K, nullptr, nullptr) + 256;
}

extern "C" int ane_hip_cblas_igemm(int variant, int semantics, uint8_t flags, uint32_t M, uint32_t N, uint32_t K,
                                   uint32_t lda, uint32_t ldb, uint32_t ldc, float alpha, float beta, const void* A,
                                   const void* B, float* C, void* workspace, size_t workspace_bytes, void* stream) {
    if (variant < 0 || variant > 2 || semantics < 0 || semantics > 1) return ANE_ERR_INVALID_ARG;
    if (M == 0 || N == 0) return ANE_OK;
    const uint32_t Ke = K / 64 * 64;
    if (!C || (Ke && (!A || !B))) return ANE_ERR_BAD_POINTER;
    if (ldc < N) return ANE_ERR_INVALID_ARG;
    if (!workspace || (((uintptr_t)workspace) & 255) ||
        workspace_bytes < igemm_layout(M, N, K, nullptr, nullptr))
        return ANE_ERR_WORKSPACE;
    if ((uint64_t)M * N > 0xffffffffull || (N + 63) / 64 > 0x7fffffffu || (M + 3) / 4 > 65535u)
        return ANE_ERR_INVALID_ARG;
    const bool au = variant != 0, bu = variant == 1;
    const bool ta = flags & 1, tb = (flags >> 1) & 1;
    hipStream_t s = (hipStream_t)stream;
    IgemmWs w;
    igemm_layout(M, N, K, static_cast<uint8_t*>(workspace), &w);
    int st;
    if (Ke) {
        if ((uint64_t)M * Ke >= (1ull << 31) || (uint64_t)N * Ke >= (1ull << 31) || (M + kT - 1) / kT > 65535u ||
            (N + kT - 1) / kT > 65535u)
            return ANE_ERR_INVALID_ARG;
        // Signed operands already in the contraction's layout (A's rows, or
        // B's rows under transB, K contiguous with 16-byte aligned rows) are
        // read in place: no gather pass, no row sums needed (both signed).
        const bool a_direct = !au && !bu && !ta && (lda & 15) == 0 && lda >= Ke && (((uintptr_t)A) & 15) == 0;
        const bool b_direct = !au && !bu && tb && (ldb & 15) == 0 && ldb >= Ke && (((uintptr_t)B) & 15) == 0;
        if (!a_direct) {
            // A rows: plain, the handler's transA addressing, or A^T (BLAS)
            const int64_t rs = !ta ? (int64_t)lda : 1;
            const int64_t r16 = (ta && semantics == 0) ? (int64_t)lda - 1 : 0;
            const int64_t ksa = (ta && semantics == 1) ? (int64_t)lda : 1;
            if ((st = gather(M, Ke, A, rs, r16, ksa, au, w.a, bu ? w.rowsum : nullptr, s))) return st;
        }
        if (!b_direct) {
            // Bt rows: B^T of a K x N matrix, or B itself (transB)
            if ((st = gather(N, Ke, B, tb ? (int64_t)ldb : 1, 0, tb ? 1 : (int64_t)ldb, bu, w.bt,
                             au ? w.colsum : nullptr, s)))
                return st;
        }
        if ((st = ane_hip_gemm_s8_i32(M, N, Ke, a_direct ? static_cast<const int8_t*>(A) : w.a,
                                      a_direct ? lda : Ke, b_direct ? static_cast<const int8_t*>(B) : w.bt,
                                      b_direct ? ldb : Ke, w.acc, s)))
            return st;
    }
    const uint32_t corr = (au && bu) ? 16384u * Ke : 0u;
    const dim3 grid((N + 63) / 64, (M + 3) / 4);
    const int32_t* acc = Ke ? w.acc : nullptr;
    const int32_t* rows = (Ke && bu) ? w.rowsum : nullptr;
    const int32_t* cols = (Ke && au) ? w.colsum : nullptr;
    if (semantics == 0)
        hipLaunchKernelGGL(k_igemm_epilogue<0>, grid, dim3(256), 0, s, M, N, acc, rows, cols, corr, alpha, beta, C,
                           (uint64_t)ldc);
    else
        hipLaunchKernelGGL(k_igemm_epilogue<1>, grid, dim3(256), 0, s, M, N, acc, rows, cols, corr, alpha, beta, C,
                           (uint64_t)ldc);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}
