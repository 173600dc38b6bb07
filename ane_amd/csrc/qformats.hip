// qformats.hip -- the reference's other weight formats: Q4_0 and the K-quant
// GEMVs (R mode: fp32 x, the handler's 16 fma lanes per row and FADDV tree)
// and the Q8_0 / Q4_0 row gathers.
//
//   0x58 q4_0_gemv      bytecode_interpreter.s:7071-7126    18 B / 32 values
//   0x75 q4_k_gemv      :11024-11131                         144 B / 256
//   0x76 q2_k_gemv      :11146-11222                         84 B / 256
//   0x77 q3_k_gemv      :11236-11358                         110 B / 256
//   0x78 q5_k_gemv      :11372-11483                         176 B / 256
//   0x79 q6_k_gemv      :11498-11626                         210 B / 256
//   0x7C get_rows_q8_0  :12363-12408
//   0x7D get_rows_q4_0  :12419-12469
//
// GEMV layout on the GPU: a workgroup of RW*16 threads takes RW rows (16,
// 8 or 4, so that there are at least two workgroups per CU), one per
// 16-lane group, lane l of a row carrying the handler's lane l.  A group
// streams its row in stages of P super-blocks: 16-byte range-checked buffer
// loads (non-temporal: every weight byte is read once) of the
// 16-byte-aligned window around the stage (any row alignment: the window
// never leaves the pointer's 16-byte granule at the front and reads zeros
// past the matrix's last dword), two stages in flight in registers, each
// stage written to the group's own LDS window and decoded from there with
// byte reads.  x is staged in LDS in chunks of 4096 values shared by the
// workgroup's rows.
#include "../../include/ane_hip.h"
#include "common.hpp"
#include "qformats.hpp"

namespace ane {
namespace {

using namespace qf;

constexpr uint32_t kXChunk = 4096;  // x values staged per pass (16 KB of LDS: five workgroups per CU)

template <class F>
struct Stage {
    // 16-byte loads per lane covering a stage's window (<= 15 bytes of lead-in)
    static constexpr uint32_t kLoads = (F::kStage * F::kBytes + 15 + 255) / 256;
    static constexpr uint32_t kWindow = kLoads * 256;
};

// RW rows per workgroup (16, 8 or 4: RW 16-lane groups, RW * 16 threads).
template <class F, int RW>
__global__ void __launch_bounds__(RW * 16)
k_qgemv(uint32_t M, uint32_t nsb, uint32_t K, const float* __restrict__ x, const uint8_t* Wa, uint32_t off,
        uint32_t wbytes, float* __restrict__ y) {
    // K here is nsb * values: the x staging below never reads past it
    using St = Stage<F>;
    // windows 64 bytes apart beyond their length: the four rows of a wave
    // read their bytes from four different bank groups
    __shared__ __attribute__((aligned(16))) uint8_t win_all[RW][St::kWindow + 64];
    __shared__ __attribute__((aligned(16))) float xs[kXChunk];
    const uint32_t g = threadIdx.x >> 4, l = threadIdx.x & 15;
    const uint32_t r = blockIdx.x * RW + g;
    const bool live = r < M;
    uint8_t* win = win_all[g];
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(Wa, wbytes);
    const uint64_t rb = (uint64_t)nsb * F::kBytes;
    const uint64_t row0 = off + (live ? r : 0) * rb;  // byte of the row in the rsrc
    const uint32_t nst = (nsb + F::kStage - 1) / F::kStage;
    constexpr uint32_t kChunkSb = kXChunk / F::kValues;  // super-blocks per x chunk
    static_assert(kChunkSb % (2 * F::kStage) == 0, "x chunks start on the even stages the loop restages at");

    auto load = [&](uint4 (&v)[St::kLoads], uint32_t st) {
        const uint64_t b = row0 + (uint64_t)st * F::kStage * F::kBytes;
        const uint32_t w0 = (uint32_t)(b & ~(uint64_t)15);
#pragma unroll
        for (uint32_t i = 0; i < St::kLoads; i++) {
            const uint32_t o = (live && st < nst) ? w0 + 256 * i + 16 * l : 0x80000000u;
            v[i] = make_uint4(__builtin_amdgcn_raw_buffer_load_b32(wr, o, 0, kCpolNt),
                              __builtin_amdgcn_raw_buffer_load_b32(wr, o + 4, 0, kCpolNt),
                              __builtin_amdgcn_raw_buffer_load_b32(wr, o + 8, 0, kCpolNt),
                              __builtin_amdgcn_raw_buffer_load_b32(wr, o + 12, 0, kCpolNt));
        }
    };
    auto run = [&](const uint4 (&v)[St::kLoads], uint32_t st, float& acc) {
#pragma unroll
        for (uint32_t i = 0; i < St::kLoads; i++) *reinterpret_cast<uint4*>(win + 256 * i + 16 * l) = v[i];
        __builtin_amdgcn_wave_barrier();
        const uint32_t lead = (uint32_t)((row0 + (uint64_t)st * F::kStage * F::kBytes) & 15);
        const uint32_t sb0 = st * F::kStage;
#pragma unroll
        for (uint32_t p = 0; p < F::kStage; p++)
            if (sb0 + p < nsb) F::acc(win + lead + p * F::kBytes, xs + ((sb0 + p) % kChunkSb) * F::kValues, l, acc);
        __builtin_amdgcn_wave_barrier();
    };

    const bool xvec = (K & 3) == 0 && (((uintptr_t)x) & 15) == 0;
    float acc = 0.0f;
    uint4 va[St::kLoads], vb[St::kLoads];
    load(va, 0);
    load(vb, 1);
    for (uint32_t st = 0; st < nst; st += 2) {
        if ((st * F::kStage) % kChunkSb == 0) {  // next x chunk (every group is at the same stage)
            __syncthreads();
            const uint32_t k0 = st * F::kStage * F::kValues;
            if (xvec) {  // 16-byte loads (x 16-byte aligned, K % 4 == 0)
                for (uint32_t i = 4 * threadIdx.x; i < kXChunk; i += 4 * RW * 16)
                    *reinterpret_cast<float4*>(xs + i) = k0 + i < K ? *reinterpret_cast<const float4*>(x + k0 + i)
                                                                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            } else {
                for (uint32_t i = threadIdx.x; i < kXChunk; i += RW * 16) xs[i] = k0 + i < K ? x[k0 + i] : 0.0f;
            }
            __syncthreads();
        }
        run(va, st, acc);
        load(va, st + 2);
        if (st + 1 < nst) {
            run(vb, st + 1, acc);
            load(vb, st + 3);
        }
    }
    const float v = faddv16(acc);
    if (live && l == 0) y[r] = v;
}

// 8 lanes per 32-block, 4 outputs each, over a flat grid of every output
// row; rows whose index is past table_rows are written as zeros.
template <bool Q4>
__global__ void __launch_bounds__(256)
k_get_rows(uint32_t n_rows, uint32_t nb, const uint8_t* __restrict__ table, uint64_t table_rows,
           const uint32_t* __restrict__ idx, float* __restrict__ out) {
    const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    const uint64_t rb = (uint64_t)nb * 8;  // threads per output row
    if (t >= rb * n_rows) return;
    const uint32_t r = (uint32_t)(t / rb), blk = (uint32_t)(t - (uint64_t)r * rb) >> 3, part = t & 7;
    const uint32_t row = idx[r];
    float* o = out + ((uint64_t)r * nb + blk) * 32 + part * 4;
    if (row >= table_rows) {
        o[0] = o[1] = o[2] = o[3] = 0.0f;
        return;
    }
    constexpr uint32_t kB = Q4 ? 18 : 34;
    const uint8_t* b = table + ((uint64_t)row * nb + blk) * kB;
    const float d = half_bits_to_float((uint32_t)b[0] | ((uint32_t)b[1] << 8));
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const uint32_t i = part * 4 + e;  // element of the block
        float v;
        if (Q4) {
            const uint32_t q = b[2 + (i & 15)];
            v = __fmul_rn((float)((int)(i < 16 ? (q & 15u) : (q >> 4)) - 8), d);
        } else {
            v = __fmul_rn((float)(int8_t)b[2 + i], d);
        }
        o[e] = v;
    }
}

template <class F>
int qgemv_launch(uint32_t M, uint32_t K, const float* x, const void* W, float* y, void* stream) {
    if (M == 0) return ANE_OK;
    const uint32_t nsb = K / F::kValues;  // the handlers ignore a remainder (K >> 5 / K >> 8)
    if (!y || (nsb && (!x || !W))) return ANE_ERR_BAD_POINTER;
    const uintptr_t wp = reinterpret_cast<uintptr_t>(W);
    const uint32_t off = (uint32_t)(wp & 15);
    const uint64_t bytes = off + (uint64_t)M * nsb * F::kBytes + 512;  // + the last window's over-read
    if (bytes >= 0x80000000ull) return ANE_ERR_INVALID_ARG;
    // the range ends on a dword boundary: the range check drops a whole dword
    // that crosses its end, and the bytes up to the boundary share the last
    // byte's 4-byte granule (so its page)
    const uint32_t range = (uint32_t)((off + (uint64_t)M * nsb * F::kBytes + 3) & ~(uint64_t)3);
    // 16 rows per workgroup from one workgroup per CU up (4096 rows on 256
    // CUs: 8 rows per workgroup measured slower there, the x staging then
    // serving half as many rows), 8 or 4 below that so short matrices still
    // spread over the CUs
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return ANE_ERR_HIP;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return ANE_ERR_HIP;
    const uint8_t* base = reinterpret_cast<const uint8_t*>(wp - off);
    hipStream_t s = (hipStream_t)stream;
    // x is staged only up to the values the super-blocks consume: a
    // remainder of K past them is never read (the caller's x may end there)
    const uint32_t kx = nsb * F::kValues;
    if (M >= 16u * (uint32_t)cus)
        hipLaunchKernelGGL((k_qgemv<F, 16>), dim3((M + 15) / 16), dim3(256), 0, s, M, nsb, kx, x, base, off, range, y);
    else if (M >= 8u * (uint32_t)cus)
        hipLaunchKernelGGL((k_qgemv<F, 8>), dim3((M + 7) / 8), dim3(128), 0, s, M, nsb, kx, x, base, off, range, y);
    else
        hipLaunchKernelGGL((k_qgemv<F, 4>), dim3((M + 3) / 4), dim3(64), 0, s, M, nsb, kx, x, base, off, range, y);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

template <bool Q4>
int get_rows_launch(uint32_t n_rows, uint32_t dim, const void* table, uint64_t table_rows, const uint32_t* indices,
                    float* out, void* stream) {
    if (n_rows == 0 || dim < 32) return ANE_OK;
    if (!table || !indices || !out) return ANE_ERR_BAD_POINTER;
    if (dim & 31) return ANE_ERR_INVALID_ARG;
    const uint32_t nb = dim >> 5;
    const uint64_t blocks = ((uint64_t)n_rows * nb * 8 + 255) / 256;
    if (blocks > 0x7fffffffull) return ANE_ERR_INVALID_ARG;
    hipLaunchKernelGGL(k_get_rows<Q4>, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, n_rows, nb,
                       static_cast<const uint8_t*>(table), table_rows, indices, out);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

}  // namespace
}  // namespace ane

namespace ane {
// q8_0.hip: the same formats on the streaming kernel, -1 when a shape does not fit it
int q4_0_stream_gemv(uint32_t M, uint32_t K, const float* x, const void* W, float* y, hipStream_t s);
int qk_stream_gemv(int fmt, uint32_t M, uint32_t K, const float* x, const void* W, float* y, hipStream_t s);
}

using namespace ane;

// 16-byte aligned rows stream through the Q8_0 kernel's per-wave DMA rings
// (q8_0.hip, kModeR4 / kModeQ4K..kModeQ5K); any other alignment, and Q6_K,
// takes k_qgemv.  Both follow the handler's arithmetic bit for bit (the
// K-quants with the same qf:: decoders).
extern "C" int ane_hip_q4_0_gemv(uint32_t M, uint32_t K, const float* x, const void* W, float* y, void* stream) {
    if (M != 0 && (K >> 5) != 0 && x && W && y) {
        const int r = q4_0_stream_gemv(M, K, x, W, y, (hipStream_t)stream);
        if (r >= 0) return r;
    }
    return qgemv_launch<Q40>(M, K, x, W, y, stream);
}
extern "C" int ane_hip_q4_k_gemv(uint32_t M, uint32_t K, const float* x, const void* W, float* y, void* stream) {
    if (M != 0 && (K >> 8) != 0 && x && W && y) {
        const int r = qk_stream_gemv(1, M, K, x, W, y, (hipStream_t)stream);
        if (r >= 0) return r;
    }
    return qgemv_launch<Q4K>(M, K, x, W, y, stream);
}
extern "C" int ane_hip_q2_k_gemv(uint32_t M, uint32_t K, const float* x, const void* W, float* y, void* stream) {
    if (M != 0 && (K >> 8) != 0 && x && W && y) {
        const int r = qk_stream_gemv(2, M, K, x, W, y, (hipStream_t)stream);
        if (r >= 0) return r;
    }
    return qgemv_launch<Q2K>(M, K, x, W, y, stream);
}
extern "C" int ane_hip_q3_k_gemv(uint32_t M, uint32_t K, const float* x, const void* W, float* y, void* stream) {
    if (M != 0 && (K >> 8) != 0 && x && W && y) {
        const int r = qk_stream_gemv(3, M, K, x, W, y, (hipStream_t)stream);
        if (r >= 0) return r;
    }
    return qgemv_launch<Q3K>(M, K, x, W, y, stream);
}
extern "C" int ane_hip_q5_k_gemv(uint32_t M, uint32_t K, const float* x, const void* W, float* y, void* stream) {
    if (M != 0 && (K >> 8) != 0 && x && W && y) {
        const int r = qk_stream_gemv(4, M, K, x, W, y, (hipStream_t)stream);
        if (r >= 0) return r;
    }
    return qgemv_launch<Q5K>(M, K, x, W, y, stream);
}
extern "C" int ane_hip_q6_k_gemv(uint32_t M, uint32_t K, const float* x, const void* W, float* y, void* stream) {
    return qgemv_launch<Q6K>(M, K, x, W, y, stream);
}
extern "C" int ane_hip_get_rows_q8_0(uint32_t n_rows, uint32_t dim, const void* table, uint64_t table_rows,
                                     const uint32_t* indices, float* out, void* stream) {
    return get_rows_launch<false>(n_rows, dim, table, table_rows, indices, out, stream);
}
extern "C" int ane_hip_get_rows_q4_0(uint32_t n_rows, uint32_t dim, const void* table, uint64_t table_rows,
                                     const uint32_t* indices, float* out, void* stream) {
    return get_rows_launch<true>(n_rows, dim, table, table_rows, indices, out, stream);
}
