// gemm_i8.hip -- int8 x int8 -> int32 contraction on gfx950 MFMA with the
// fused dequant / scale / bias / ReLU epilogue of the ane dense opcodes:
//   dense_i8 (0x18) and dense_u8s8 (0x1E): B in the SMOPA panel format
//     (bytecode_interpreter.s:1978-2446, 2835-3300);
//   dense_fused_i8 (README.md:84-97): fp32 A and B quantized per tensor by
//     two streaming kernels, B written transposed (K contiguous per column)
//     so both MFMA operands load as 16-byte rows;
//   gemm_s8_i32: raw accumulators for tests.
//
// Tile: 128 x 128 output per 256-thread workgroup, K staged through LDS in
// 128-byte slices, four waves each owning a 64 x 64 block of 2 x 2
// v_mfma_i32_32x32x32_i8 tiles.  Both operand tiles sit in LDS as
// [row][128 bytes] with the 16-byte chunk index XOR-swizzled by
// (row ^ row>>3) & 7 so the ds_read_b128 of 16 consecutive rows (one LDS
// cycle: 64 banks x 4 bytes) hits 16 distinct bank groups.  Large shapes use the 256 x 256 kernel of
// gemm_i8_tile256.hip instead, and up to 128 rows the few-row kernel of
// gemm_i8_skinny.hip.
#include "gemm_i8.hpp"

#include <atomic>
#include <vector>

namespace ane {

constexpr int kBM = 128, kBN = 128, kBK = 128;
constexpr int kGThreads = 256;

enum BLayout : int { kBTransposed = 0, kBPanel = 1 };

__device__ __forceinline__ uint32_t swz(uint32_t row, uint32_t chunk) {
    return row * kBK + ((chunk ^ ((row ^ (row >> 3)) & 7)) << 4);
}

template <int BL, bool AU8>
__global__ void __launch_bounds__(kGThreads)
k_gemm_i8(GemmParams p) {
    __shared__ __attribute__((aligned(16))) int8_t sA[kBM * kBK];
    __shared__ __attribute__((aligned(16))) int8_t sB[kBN * kBK];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = tid >> 6;
    const uint32_t row0 = blockIdx.y * kBM;
    const uint32_t col0 = blockIdx.x * kBN;
    const uint32_t wr0 = (wave >> 1) * 64;
    const uint32_t wc0 = (wave & 1) * 64;

    v16i acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;
    int colsum[2] = {0, 0};  // AU8 only: sum_k B[k][j] for this lane's columns

    for (uint32_t k0 = 0; k0 < p.Kp; k0 += kBK) {
        // ---- A tile: 128 rows x 8 chunks of 16 bytes, 4 per thread
#pragma unroll
        for (int it = 0; it < 4; it++) {
            const uint32_t idx = it * kGThreads + tid;
            const uint32_t r = idx >> 3, c = idx & 7;
            const uint32_t gr = row0 + r, gk = k0 + c * 16;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (gr < p.rowsA && gk < p.Kp) {
                v = *reinterpret_cast<const uint4*>(p.A + (uint64_t)gr * p.lda + gk);
                if (AU8) {  // uint8 a -> int8 (a - 128); the bias is added back in the epilogue
                    v.x ^= 0x80808080u; v.y ^= 0x80808080u; v.z ^= 0x80808080u; v.w ^= 0x80808080u;
                }
            }
            *reinterpret_cast<uint4*>(sA + swz(r, c)) = v;
        }
        // ---- B tile
        if (BL == kBTransposed) {
#pragma unroll
            for (int it = 0; it < 4; it++) {
                const uint32_t idx = it * kGThreads + tid;
                const uint32_t r = idx >> 3, c = idx & 7;
                const uint32_t gc = col0 + r, gk = k0 + c * 16;
                uint4 v = make_uint4(0, 0, 0, 0);
                if (gc < p.colsB && gk < p.Kp)
                    v = *reinterpret_cast<const uint4*>(p.B + (uint64_t)gc * p.ldb + gk);
                *reinterpret_cast<uint4*>(sB + swz(r, c)) = v;
            }
        } else {
            // 8 panels of 16 columns; the k-slice of one panel is 32 groups
            // x 64 bytes, contiguous.  A 16-byte piece = 4 columns x 4 k.
#pragma unroll
            for (int it = 0; it < 4; it++) {
                const uint32_t idx = it * kGThreads + tid;
                const uint32_t pl = idx >> 7, ch = idx & 127;
                const uint32_t gl = ch >> 2, q = ch & 3;
                const uint32_t gp = (col0 >> 4) + pl, gg = (k0 >> 2) + gl;
                uint4 v = make_uint4(0, 0, 0, 0);
                if (gp * 16 < p.colsB && gg * 4 < p.Kp)
                    v = *reinterpret_cast<const uint4*>(p.B + ((uint64_t)gp * p.ldb + gg) * 64 + q * 16);
                const uint32_t cbase = pl * 16 + q * 4;
                const uint32_t chunk = gl >> 2, sub = (gl & 3) * 4;
                *reinterpret_cast<uint32_t*>(sB + swz(cbase + 0, chunk) + sub) = v.x;
                *reinterpret_cast<uint32_t*>(sB + swz(cbase + 1, chunk) + sub) = v.y;
                *reinterpret_cast<uint32_t*>(sB + swz(cbase + 2, chunk) + sub) = v.z;
                *reinterpret_cast<uint32_t*>(sB + swz(cbase + 3, chunk) + sub) = v.w;
            }
        }
        __syncthreads();

#pragma unroll
        for (int ks = 0; ks < kBK / 32; ks++) {
            const uint32_t chunk = ks * 2 + (lane >> 5);
            v4i a[2], b[2];
#pragma unroll
            for (int mi = 0; mi < 2; mi++)
                a[mi] = *reinterpret_cast<const v4i*>(sA + swz(wr0 + mi * 32 + (lane & 31), chunk));
#pragma unroll
            for (int ni = 0; ni < 2; ni++) {
                b[ni] = *reinterpret_cast<const v4i*>(sB + swz(wc0 + ni * 32 + (lane & 31), chunk));
                if (AU8) {
                    colsum[ni] = __builtin_amdgcn_sdot4(b[ni].x, 0x01010101, colsum[ni], false);
                    colsum[ni] = __builtin_amdgcn_sdot4(b[ni].y, 0x01010101, colsum[ni], false);
                    colsum[ni] = __builtin_amdgcn_sdot4(b[ni].z, 0x01010101, colsum[ni], false);
                    colsum[ni] = __builtin_amdgcn_sdot4(b[ni].w, 0x01010101, colsum[ni], false);
                }
            }
#pragma unroll
            for (int mi = 0; mi < 2; mi++)
#pragma unroll
                for (int ni = 0; ni < 2; ni++)
                    acc[mi][ni] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[mi], b[ni], acc[mi][ni], 0, 0, 0);
        }
        __syncthreads();
    }

    if (AU8) {
#pragma unroll
        for (int ni = 0; ni < 2; ni++) colsum[ni] += __shfl_xor(colsum[ni], 32, kWave);
    }

    // ---- epilogue: C = fmaxA(fadd(fmul((float)acc, s), bias[j]), lo)
    float s = p.s;
    if (p.sdev) s = __fmul_rn(__fmul_rn(p.sdev[0], p.sdev[1]), p.smul);
#pragma unroll
    for (int ni = 0; ni < 2; ni++) {
        const uint32_t j = col0 + wc0 + ni * 32 + (lane & 31);
        if (j >= p.Nout) continue;
        const float bj = p.bias ? p.bias[j] : 0.0f;
#pragma unroll
        for (int mi = 0; mi < 2; mi++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t i = row0 + wr0 + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (i >= p.Mout) continue;
                int32_t v = acc[mi][ni][r];
                if (AU8) v = (int32_t)((uint32_t)v + 128u * (uint32_t)colsum[ni]);
                if (p.Craw) {
                    p.Craw[(uint64_t)i * p.ldc + j] = v;
                } else {
                    float f = __fadd_rn(__fmul_rn((float)v, s), bj);
                    p.C[(uint64_t)i * p.ldc + j] = fmax_a(f, p.lo);
                }
            }
        }
    }
}

// The CU count of the current device (256-tiles are preferred from one per CU).
static uint64_t tile256_min_tiles() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (!n) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return (uint64_t)n;
}

template <int BL, bool AU8>
static int launch_gemm(const GemmParams& p, hipStream_t s) {
    if (p.Mout == 0 || p.Nout == 0) return ANE_OK;
    if (BL == kBTransposed && !AU8) {
        // 256-tiles while they fill every CU, few rows on the skinny kernel,
        // otherwise 128-tiles (four times the workgroups)
        const uint64_t tiles256 = (uint64_t)((p.Mout + 255) / 256) * ((p.Nout + 255) / 256);
        const bool e256 = tile256_eligible(p);
        if (e256 && tiles256 >= tile256_min_tiles()) return launch_gemm_tile256(p, s);
        if (skinny_eligible(p)) return launch_gemm_skinny(p, s);
        if (tile128_eligible(p)) {
            // one 128-tile per CU or fewer: the deeper ring; more: two per CU
            const uint64_t tiles128 = (uint64_t)((p.Mout + 127) / 128) * ((p.Nout + 127) / 128);
            if (tiles128 <= tile256_min_tiles() && tile128d_eligible(p)) return launch_gemm_tile128d(p, s);
            return launch_gemm_tile128(p, s);
        }
        if (e256) return launch_gemm_tile256(p, s);
    }
    dim3 grid((p.Nout + kBN - 1) / kBN, (p.Mout + kBM - 1) / kBM);
    if (grid.y > 65535) return ANE_ERR_INVALID_ARG;
    hipLaunchKernelGGL((k_gemm_i8<BL, AU8>), grid, dim3(kGThreads), 0, s, p);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

static bool aligned16(const void* ptr) { return (((uintptr_t)ptr) & 15) == 0; }

}  // namespace ane

using namespace ane;

extern "C" int ane_hip_dense_i8(uint32_t M, uint32_t N, uint32_t K, float sa, float sb,
                                uint8_t flags, const void* A, const int8_t* Bp,
                                const float* bias, float* C, int a_unsigned, void* stream) {
    const uint64_t Kp = ceil_to(K, 64);
    uint64_t Mp = ceil_to(M, 16);
    if (Mp == 0) Mp = 16;  // the reference's tile-row loop runs at least once
    if (N == 0) return ANE_OK;
    if (!A || !Bp || !bias || !C) return ANE_ERR_BAD_POINTER;
    if (!aligned16(A) || !aligned16(Bp)) return ANE_ERR_INVALID_ARG;
    if (Kp > 0x7fffffffull || Mp > 0xffffffffull) return ANE_ERR_INVALID_ARG;
    GemmParams p{};
    p.A = (const int8_t*)A;
    p.lda = Kp;
    p.B = Bp;
    p.ldb = Kp / 4;
    p.rowsA = (uint32_t)Mp;
    p.colsB = (uint32_t)ceil_to(N, 16);
    p.Kp = (uint32_t)Kp;
    p.Mout = (uint32_t)Mp;
    p.Nout = N;
    p.s = sa * sb;  // host fmul, IEEE single (bytecode_interpreter.s:2017)
    p.sdev = nullptr;
    p.bias = bias;
    p.lo = (flags & 1) ? 0.0f : -3.40282347e+38f;
    p.C = C;
    p.ldc = N;
    hipStream_t s = (hipStream_t)stream;
    return a_unsigned ? launch_gemm<kBPanel, true>(p, s) : launch_gemm<kBPanel, false>(p, s);
}

extern "C" int ane_hip_gemm_s8_i32(uint32_t M, uint32_t N, uint32_t K, const int8_t* A,
                                   uint32_t lda, const int8_t* Bt, uint32_t ldb, int32_t* acc,
                                   void* stream) {
    if (M == 0 || N == 0) return ANE_OK;
    if (!A || !Bt || !acc) return ANE_ERR_BAD_POINTER;
    if ((K & 15) || (lda & 15) || (ldb & 15) || !aligned16(A) || !aligned16(Bt) || lda < K ||
        ldb < K)
        return ANE_ERR_INVALID_ARG;
    GemmParams p{};
    p.A = A;
    p.lda = lda;
    p.B = Bt;
    p.ldb = ldb;
    p.rowsA = M;
    p.colsB = N;
    p.Kp = K;
    p.Mout = M;
    p.Nout = N;
    p.s = 1.0f;
    p.lo = 0.0f;
    p.Craw = acc;
    p.ldc = N;
    return launch_gemm<kBTransposed, false>(p, (hipStream_t)stream);
}

// The fused operands are laid out with K padded (zeros) to a multiple of 128
// so both contraction kernels run whole 128-byte K slices.
static uint64_t fused_kp(int32_t K) { return ceil_to((uint64_t)(K > 0 ? K : 0), 128); }

// Workspace layout: scales {sa, sb} at 0; at 256 the absmax partials
// (2 x kFusedPartials uint32) followed by the quantizer's wait record
// (1 + kFusedPartials uint32); then qA and qBt, each rounded up to 256
// bytes; then, for few rows, the split contraction's int32 planes.
static uint64_t fused_partials_bytes() { return ceil_to((uint64_t)(3 * kFusedPartials + 1) * 4, 256); }

// Few rows (kSplitMinRows .. 128): the contraction on 128 x 128 tiles with K
// split over up to kMaxSplit workgroups per tile, each writing an int32
// plane, then k_split_epilogue adds the planes (int32, exact in any order)
// and applies the epilogue.  A full-K workgroup per 16 columns
// (k_gemm_skinny) re-reads all of A for every 16 columns; here each
// workgroup reads A and Bt over its share of K only.  Measured whole op at
// N = K = 4096 (skinny / 4 splits / 8 splits): M = 64 31.7 / 32.9 / 32.0 us,
// M = 96 36.9 / 33.1 / 32.6, M = 128 39.4 / 33.2 / 33.3 (contraction alone
// at M = 128: 20.1 / 13.5 / 16.0).
constexpr uint32_t kSplitMinRows = 65;
constexpr uint32_t kMaxSplit = 4;
static uint64_t fused_split_bytes(int32_t M, int32_t N, int32_t K) {
    if (M < (int32_t)kSplitMinRows || M > 128 || N < 128 || K <= 0) return 0;
    return ceil_to((uint64_t)kMaxSplit * M * N * 4, 256);
}

extern "C" size_t ane_hip_dense_fused_i8_workspace_size(int32_t M, int32_t N, int32_t K) {
    if (M < 0 || N < 0 || K < 0) return 0;
    const uint64_t Kp = fused_kp(K);
    uint64_t bytes = 256;                                  // scales + alignment slack
    bytes += fused_partials_bytes();                      // absmax partials + wait record
    bytes += ceil_to((uint64_t)M * Kp, 256);               // qA
    bytes += ceil_to((uint64_t)N * Kp, 256);               // qBt
    bytes += fused_split_bytes(M, N, K);                   // split contraction planes
    return (size_t)bytes;
}


// C = fmaxA(fadd(fmul((float)acc, s), +0), lo) with acc the int32 sum
// (wrapping, exact in any order) of the ksplit planes and s = (sa*sb)*smul:
// the same operations as the contraction kernels' epilogue.  Four outputs
// per thread.
__global__ void __launch_bounds__(256)
k_split_epilogue(const int32_t* __restrict__ planes, uint32_t ksplit, uint64_t n, const float* __restrict__ sdev,
                 float smul, float lo, float* __restrict__ C) {
    const uint64_t i4 = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i4 >= n) return;
    const float s = __fmul_rn(__fmul_rn(sdev[0], sdev[1]), smul);
    auto epi = [&](uint32_t acc) { return fmax_a(__fadd_rn(__fmul_rn((float)(int32_t)acc, s), 0.0f), lo); };
    if ((n & 3) == 0 && (((uintptr_t)C) & 15) == 0) {
        uint4 acc = make_uint4(0, 0, 0, 0);
        for (uint32_t y = 0; y < ksplit; y++) {
            const uint4 v = *reinterpret_cast<const uint4*>(planes + y * n + i4);
            acc.x += v.x;
            acc.y += v.y;
            acc.z += v.z;
            acc.w += v.w;
        }
        *reinterpret_cast<float4*>(C + i4) = make_float4(epi(acc.x), epi(acc.y), epi(acc.z), epi(acc.w));
        return;
    }
    for (uint64_t i = i4; i < i4 + 4 && i < n; i++) {
        uint32_t acc = 0;
        for (uint32_t y = 0; y < ksplit; y++) acc += (uint32_t)planes[y * n + i];
        C[i] = epi(acc);
    }
}

struct FusedLayout {
    uint64_t Kp;
    float* scales;
    uint32_t* partials;
    uint32_t* wstatus;
    int8_t* qA;
    int8_t* qBt;
    int32_t* planes;  // split contraction (few rows), or null
};

static FusedLayout fused_layout(int32_t M, int32_t N, int32_t K, void* workspace) {
    FusedLayout L;
    L.Kp = fused_kp(K);
    uint8_t* ws = (uint8_t*)workspace;
    L.scales = (float*)ws;
    L.partials = (uint32_t*)(ws + 256);
    L.wstatus = L.partials + 2 * kFusedPartials;
    L.qA = (int8_t*)(ws + 256 + fused_partials_bytes());
    L.qBt = L.qA + ceil_to((uint64_t)M * L.Kp, 256);
    L.planes = fused_split_bytes(M, N, K) ? reinterpret_cast<int32_t*>(L.qBt + ceil_to((uint64_t)N * L.Kp, 256))
                                          : nullptr;
    return L;
}

static int fused_check(int32_t M, int32_t N, int32_t K, const void* workspace, size_t workspace_bytes) {
    if (M < 0 || N < 0 || K < 0) return ANE_ERR_INVALID_ARG;
    if (!workspace || !aligned16(workspace) ||
        workspace_bytes < ane_hip_dense_fused_i8_workspace_size(M, N, K))
        return ANE_ERR_WORKSPACE;
    return ANE_OK;
}

extern "C" int ane_hip_dense_fused_i8_quantize(int32_t M, int32_t N, int32_t K, const float* A,
                                               const float* B, float* scales_out, void* workspace,
                                               size_t workspace_bytes, void* stream) {
    int st = fused_check(M, N, K, workspace, workspace_bytes);
    if (st != ANE_OK) return st;
    if (M == 0 || N == 0) return ANE_OK;
    if (K > 0 && (!A || !B)) return ANE_ERR_BAD_POINTER;
    hipStream_t s = (hipStream_t)stream;
    const FusedLayout L = fused_layout(M, N, K, workspace);
    const uint64_t Kp = L.Kp;
    st = launch_fused_quantize(A, B, (uint32_t)M, (uint32_t)N, (uint32_t)K, (uint32_t)Kp, L.partials,
                               L.qA, L.qBt, L.scales, L.wstatus, s);
    if (st != ANE_OK) return st;
    if (scales_out) {
        hipError_t e = hipMemcpyAsync(scales_out, L.scales, 2 * sizeof(float), hipMemcpyDeviceToDevice, s);
        if (e != hipSuccess) return ANE_ERR_HIP;
    }
    return ANE_OK;
}

extern "C" int ane_hip_dense_fused_i8_gemm(int32_t M, int32_t N, int32_t K, float scale, int relu,
                                           float* C, const void* workspace, size_t workspace_bytes,
                                           void* stream) {
    int st = fused_check(M, N, K, workspace, workspace_bytes);
    if (st != ANE_OK) return st;
    if (M == 0 || N == 0) return ANE_OK;
    if (!C) return ANE_ERR_BAD_POINTER;
    const FusedLayout L = fused_layout(M, N, K, (void*)workspace);
    GemmParams p{};
    p.A = L.qA;
    p.lda = L.Kp;
    p.B = L.qBt;
    p.ldb = L.Kp;
    p.rowsA = (uint32_t)M;
    p.colsB = (uint32_t)N;
    p.Kp = (uint32_t)L.Kp;
    p.Mout = (uint32_t)M;
    p.Nout = (uint32_t)N;
    p.sdev = L.scales;
    p.smul = scale;
    p.bias = nullptr;
    p.lo = relu ? 0.0f : -3.40282347e+38f;
    p.C = C;
    p.ldc = (uint64_t)N;
    hipStream_t s = (hipStream_t)stream;
    if (L.planes) {
        // K split so that the tiles x splits fill the CUs, at least two
        // 128-byte slices per split
        const uint32_t tiles = (uint32_t)((N + 127) / 128), nk = (uint32_t)(L.Kp / 128);
        uint32_t ksplit = (uint32_t)(tile256_min_tiles() / tiles);
        if (ksplit > kMaxSplit) ksplit = kMaxSplit;
        if (ksplit > nk / 2) ksplit = nk / 2;
        GemmParams q = p;
        q.C = nullptr;
        q.Craw = L.planes;
        if (ksplit >= 2 && tile128_eligible(q, true)) {
            const int st = (uint64_t)tiles * ksplit <= tile256_min_tiles() && tile128d_eligible(q, true)
                               ? launch_gemm_tile128d(q, s, ksplit)
                               : launch_gemm_tile128(q, s, ksplit);
            if (st != ANE_OK) return st;
            const uint64_t n = (uint64_t)M * N;
            hipLaunchKernelGGL(k_split_epilogue, dim3((uint32_t)((n + 1023) / 1024)), dim3(256), 0, s, L.planes,
                               ksplit, n, L.scales, scale, p.lo, C);
            ANE_HIP_CHECK_LAUNCH();
            return ANE_OK;
        }
    }
    return launch_gemm<kBTransposed, false>(p, s);
}

extern "C" int ane_hip_dense_fused_i8(int32_t M, int32_t N, int32_t K, float scale, int relu,
                                      const float* A, const float* B, float* C,
                                      float* scales_out, void* workspace,
                                      size_t workspace_bytes, void* stream) {
    if (M > 0 && N > 0 && !C) return ANE_ERR_BAD_POINTER;
    if (M > 0 && N > 0 && K > 0 && small_fused_eligible((uint32_t)M, (uint32_t)N, (uint32_t)K)) {
        // small operands: the absmax pass and one quantize-and-contract launch
        int st = fused_check(M, N, K, workspace, workspace_bytes);
        if (st != ANE_OK) return st;
        if (!A || !B) return ANE_ERR_BAD_POINTER;
        hipStream_t s = (hipStream_t)stream;
        const FusedLayout L = fused_layout(M, N, K, workspace);
        st = launch_fused_small(A, B, (uint32_t)M, (uint32_t)N, (uint32_t)K, scale, relu ? 0.0f : -3.40282347e+38f, C,
                                L.partials, L.scales, L.wstatus, s);
        if (st != ANE_OK) return st;
        if (scales_out && hipMemcpyAsync(scales_out, L.scales, 2 * sizeof(float), hipMemcpyDeviceToDevice, s) !=
                              hipSuccess)
            return ANE_ERR_HIP;
        return ANE_OK;
    }
    if (M > 0 && N > 0 && K > 0 && strip_fused_eligible((uint32_t)M, (uint32_t)N, (uint32_t)K, A, B)) {
        // at most 16 rows: one launch holding a 16-column strip of B per CU
        // (when the device's grid has a workgroup for every strip)
        int st = fused_check(M, N, K, workspace, workspace_bytes);
        if (st != ANE_OK) return st;
        hipStream_t s = (hipStream_t)stream;
        const FusedLayout L = fused_layout(M, N, K, workspace);
        if (launch_fused_strip(A, B, (uint32_t)M, (uint32_t)N, (uint32_t)K, scale, relu ? 0.0f : -3.40282347e+38f,
                               C, L.partials, L.scales, L.wstatus, s, &st)) {
            if (st != ANE_OK) return st;
            if (scales_out && hipMemcpyAsync(scales_out, L.scales, 2 * sizeof(float), hipMemcpyDeviceToDevice,
                                             s) != hipSuccess)
                return ANE_ERR_HIP;
            return ANE_OK;
        }
    }
    int st = ane_hip_dense_fused_i8_quantize(M, N, K, A, B, scales_out, workspace, workspace_bytes,
                                             stream);
    if (st != ANE_OK) return st;
    return ane_hip_dense_fused_i8_gemm(M, N, K, scale, relu, C, workspace, workspace_bytes, stream);
}

extern "C" int ane_hip_dense_fused_i8_status(const void* workspace, void* stream) {
    if (!workspace || !aligned16(workspace)) return ANE_ERR_WORKSPACE;
    if (hipStreamSynchronize((hipStream_t)stream) != hipSuccess) {
        (void)hipGetLastError();
        return ANE_ERR_HIP;
    }
    const uint32_t* rec = (const uint32_t*)((const uint8_t*)workspace + 256) + 2 * kFusedPartials;
    uint32_t n = 0;
    if (hipMemcpy(&n, rec, 4, hipMemcpyDeviceToHost) != hipSuccess) {
        (void)hipGetLastError();
        return ANE_ERR_HIP;
    }
    if (n > kFusedPartials) return ANE_ERR_INVALID_ARG;  // no quantize call wrote this workspace
    uint32_t bits = 0;
    if (n) {
        std::vector<uint32_t> h(n);
        if (hipMemcpy(h.data(), rec + 1, (size_t)n * 4, hipMemcpyDeviceToHost) != hipSuccess) {
            (void)hipGetLastError();
            return ANE_ERR_HIP;
        }
        for (uint32_t v : h) bits |= v;
    }
    // A launch whose wait was completed by another launch's arrivals does
    // not see that itself: the arrival that completed it recorded it on the
    // device, so the device's record is read (and cleared) as well.
    uint32_t dev_bits = 0;
    const int st = resident_slot_check(&dev_bits);
    if (st != ANE_OK) return st;
    if (bits || resident_mixed_bit(dev_bits)) return ANE_ERR_GRID_WAIT;
    return ANE_OK;
}
