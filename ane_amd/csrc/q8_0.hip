// q8_0.hip -- Q8_0 matrix-vector kernels (ggml block layout: fp16 d followed
// by 32 int8 quants, 34 bytes per 32 weights, rows of K/32 blocks;
// API.md:598, bytecode_interpreter.s:7013, 7036-7056).
//
//   R mode  = the reference's q8_0_gemv (0x57, bytecode_interpreter.s:7010-7063):
//             fp32 x, 16 fma lanes per row (lane l takes elements l and 16+l
//             of every block in order), FADDV tree; reproduced bit-exactly.
//   G mode  = x quantized to Q8_0 per 32-block (0x19 arithmetic, fp32 scale),
//             v_dot4 int8 block dots, 16 fp32 partials (block b -> partial
//             b % 16, fmaf((float)isum, d_w*d_x, p)) combined by the same
//             FADDV tree.  Serves GGML_OP_MUL_MAT for every token.
//
// Implementations, bit-identical by construction:
//  * streaming kernels (k_q8_0_stream), R and G mode for up to 4 tokens,
//    used when every row starts 16-byte aligned (nb % 8 == 0, W 16-byte
//    aligned), the matrix is under 2 GB and the activations fit in LDS;
//  * the MFMA kernels (k_q8_0_mma, k_q8_0_mmt), G mode for 5+ tokens when
//    nb % 16 == 0;
//  * general kernels (k_q8_0_gemv_r, k_q8_0_quantize_x + k_q8_0_mul_mat_g)
//    for everything else.
#include "../../include/ane_decode.h"
#include "common.hpp"
#include "qformats.hpp"
#include "q8_0_mmv.hpp"

#include <atomic>
#include <map>
#include <mutex>

namespace ane {

thread_local bool t_plan_only = false;

namespace {

// ====================================================== general kernels
constexpr int kRowsPerBlock = 16;  // 16 lanes per row, 256 threads

__global__ void __launch_bounds__(256)
k_q8_0_gemv_r(uint32_t M, uint32_t nb, const float* __restrict__ x,
              const uint8_t* __restrict__ W, float* __restrict__ y) {
    const uint32_t l = threadIdx.x & 15;
    const uint64_t m = (uint64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 4);
    const bool live = m < M;
    float acc = 0.0f;
    if (live) {
        const uint8_t* row = W + m * nb * 34;
        for (uint32_t b = 0; b < nb; b++) {
            const uint8_t* blk = row + (uint64_t)b * 34;
            const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(blk));
            const float w0 = __fmul_rn((float)(int8_t)blk[2 + l], d);
            acc = __builtin_fmaf(w0, x[32 * b + l], acc);
            const float w1 = __fmul_rn((float)(int8_t)blk[18 + l], d);
            acc = __builtin_fmaf(w1, x[32 * b + 16 + l], acc);
        }
    }
    acc = faddv16(acc);
    if (live && l == 0) y[m] = acc;
}

// Activation quantizer: one thread per 32-element block of x.
// Token t's row of x starts at x + t*K (K need not be a multiple of 32; the
// trailing K%32 values are ignored like the reference's nb = K >> 5).
__global__ void __launch_bounds__(256)
k_q8_0_quantize_x(uint64_t nblocks, uint32_t nb, uint32_t K, const float* __restrict__ x,
                  int8_t* __restrict__ qx, float* __restrict__ dx) {
    const uint64_t b = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblocks) return;
    const float* s = x + (b / nb) * K + (b % nb) * 32;
    uint32_t m = 0;
    for (int i = 0; i < 32; i++) {
        uint32_t a = abs_key(s[i]);
        m = m > a ? m : a;
    }
    float scale, inv;
    quant_params(__uint_as_float(m), scale, inv);
    dx[b] = scale;
    uint32_t* q = reinterpret_cast<uint32_t*>(qx + b * 32);
    for (int w = 0; w < 8; w++) q[w] = pack4(s[4 * w], s[4 * w + 1], s[4 * w + 2], s[4 * w + 3], inv);
}

// Activation quantizer into the Q8 activation form (qx [T*nb][32] int8,
// then dx [T*nb] fp32 at byte T*nb*32): 8 lanes per 32-block, one float4
// each (coalesced), the 0x19 arithmetic of XStage::store, so a streaming
// kernel that copies this form (kFusePreQuant) computes exactly what its own
// prologue would.  Token t's row starts at x + t*K.
__global__ void __launch_bounds__(256)
k_q8_act_quantize(uint32_t nblocks, uint32_t nb, uint32_t K, const float* __restrict__ x,
                  uint8_t* __restrict__ xq) {
    const uint32_t t = blockIdx.x * 256 + threadIdx.x, blk = t >> 3, part = t & 7;
    const uint32_t tok = blk / nb, b = blk - tok * nb;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(x, (nblocks / nb) * K * 4);
    const uint32_t o = blk < nblocks ? (tok * K + b * 32 + part * 4) * 4 : 0x80000000u;  // whole 8-lane groups
    float f[4];
#pragma unroll
    for (int e = 0; e < 4; e++) f[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, o + 4 * e, 0, 0));
    const uint32_t m = max8_u32(max(max(abs_key(f[0]), abs_key(f[1])), max(abs_key(f[2]), abs_key(f[3]))));
    float scale, inv;
    quant_params(__uint_as_float(m), scale, inv);
    if (blk < nblocks) {
        reinterpret_cast<uint32_t*>(xq)[blk * 8 + part] = pack4(f[0], f[1], f[2], f[3], inv);
        if (part == 0) reinterpret_cast<float*>(xq + (uint64_t)nblocks * 32)[blk] = scale;
    }
}

constexpr int kTokChunk = 4;

__global__ void __launch_bounds__(256)
k_q8_0_mul_mat_g(uint32_t N, uint32_t nb, uint32_t T, const int8_t* __restrict__ qx,
                 const float* __restrict__ dx, const uint8_t* __restrict__ W,
                 float* __restrict__ y) {
    const uint32_t l = threadIdx.x & 15;
    const uint64_t m = (uint64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 4);
    const bool live = m < N;
    const uint8_t* row = W + (live ? m : 0) * nb * 34;
    for (uint32_t t0 = 0; t0 < T; t0 += kTokChunk) {
        float p[kTokChunk];
#pragma unroll
        for (int t = 0; t < kTokChunk; t++) p[t] = 0.0f;
        if (live) {
            for (uint32_t b = l; b < nb; b += 16) {
                const uint8_t* blk = row + (uint64_t)b * 34;
                const uint16_t* h = reinterpret_cast<const uint16_t*>(blk);
                const float dw = half_bits_to_float(h[0]);
                int wq[8];
#pragma unroll
                for (int q = 0; q < 8; q++) wq[q] = (int)((uint32_t)h[1 + 2 * q] | ((uint32_t)h[2 + 2 * q] << 16));
#pragma unroll
                for (int t = 0; t < kTokChunk; t++) {
                    if (t0 + t < T) {
                        const uint64_t xb = (uint64_t)(t0 + t) * nb + b;
                        const int* xq = reinterpret_cast<const int*>(qx + xb * 32);
                        int isum = 0;
#pragma unroll
                        for (int q = 0; q < 8; q++) isum = __builtin_amdgcn_sdot4(wq[q], xq[q], isum, false);
                        const float dd = __fmul_rn(dw, dx[xb]);
                        p[t] = __builtin_fmaf((float)isum, dd, p[t]);
                    }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < kTokChunk; t++) {
            const float v = faddv16(p[t]);
            if (live && l == 0 && t0 + t < T) y[(uint64_t)(t0 + t) * N + m] = v;
        }
    }
}

// ====================================================== streaming kernels
//  * Persistent grid: workgroups = CUs x occupancy, NW waves each.  Wave w
//    owns the contiguous row range [w*N/Wt, (w+1)*N/Wt) of the Wt waves, so
//    every wave streams the same number of bytes.
//  * A wave walks its rows 4 at a time ("unit": one row per 16-lane group;
//    in G mode lane l of a group owns blocks b = l mod 16, the partial order
//    of the definition) and each unit in segments of SB blocks ("item").
//    Items are copied global -> LDS with buffer_load_dwordx4 ... lds into a
//    ring of S stages private to the wave: each copy wave-instruction moves
//    1 KB of consecutive bytes of one or two rows, so HBM sees fully
//    coalesced reads, and no VGPRs or workgroup barriers are spent on
//    staging.  S items are issued before the activation prologue; after item
//    i is computed its stage is refilled with item i+S.  Items past the end
//    issue all-out-of-range copies so the s_waitcnt count is fixed.
//  * Staged rows sit SB*17/8 + pad chunks apart, 16 or 48 dwords mod 64, so
//    the four groups' block reads (dword offsets 17(l/2) + 8(l%2), distinct
//    mod 16) never share an LDS bank.
//  * A block b at byte 34b of its staged row is read as 9 aligned dwords
//    from 34b - 2(b%2); v_perm_b32 realigns the scale and the 8 quant
//    dwords (lanes of one parity share the selector, no branches).
//  * G mode: each workgroup first quantizes the T activation rows into LDS
//    (one 32-block per 8 lanes, 0x19 arithmetic); the halves of the 32-byte
//    qx blocks are swapped on odd (b/8) so 16 lanes reading 16 blocks hit 16
//    distinct bank quads.  R mode: x is copied to LDS as fp32.  The first
//    batch of activation loads is issued ahead of the ring's first copies
//    (vector-memory loads complete in issue order).
constexpr int kUnitRows = 4;       // rows per wave pass (one per 16-lane group)
constexpr uint32_t kXBatch = 8;    // activation float4 loads in flight per thread

// kModeR4: the R arithmetic of q4_0_gemv (0x58) over Q4_0 blocks (18 bytes).
// kModeQ4K .. kModeQ5K: the K-quant GEMVs (0x75-0x78) over their 256-value
// super-blocks, each lane decoding with the format's qf:: decoder.
enum { kModeR = 0, kModeG = 1, kModeR4 = 2, kModeQ4K = 3, kModeQ2K = 4, kModeQ3K = 5, kModeQ5K = 6 };

template <int MODE>
struct ModeFmt {
    using F = void;
};
template <> struct ModeFmt<kModeQ4K> { using F = qf::Q4K; };
template <> struct ModeFmt<kModeQ2K> { using F = qf::Q2K; };
template <> struct ModeFmt<kModeQ3K> { using F = qf::Q3K; };
template <> struct ModeFmt<kModeQ5K> { using F = qf::Q5K; };

template <int MODE>
constexpr bool kIsQK = MODE >= kModeQ4K;

// Bytes and values per block of the weight format a mode streams (a K-quant
// super-block counts as one block).
template <int MODE>
constexpr uint32_t block_bytes() {
    if constexpr (kIsQK<MODE>) return ModeFmt<MODE>::F::kBytes;
    else return MODE == kModeR4 ? 18 : 34;
}
template <int MODE>
constexpr uint32_t kBlockBytes = block_bytes<MODE>();
template <int MODE>
constexpr uint32_t kBlockValues = kIsQK<MODE> ? 256 : 32;
__host__ __device__ constexpr uint32_t mode_block_values(int mode) { return mode >= kModeQ4K ? 256 : 32; }

// LDS bytes of the activation region (G: qx then fp32 scales; R: fp32 x),
// rounded to 16; the fp64 reduction slots of the norm fusion follow it.
__host__ __device__ __forceinline__ uint32_t stream_x_bytes(int mode, uint32_t nb, uint32_t T) {
    const uint64_t xb = mode == kModeG ? ceil_to((uint64_t)T * nb * 32, 16) + (uint64_t)T * nb * 4
                                       : (uint64_t)nb * mode_block_values(mode) * 4;
    return (uint32_t)ceil_to(xb, 16);
}

// Pad chunks that put a staged row 16 or 48 dwords (mod 64) after the
// previous one, so the four rows of a unit sit in four bank groups.
__host__ __device__ constexpr uint32_t row_pad(uint32_t cpr) {
    uint32_t p = 0;
    while ((cpr + p) % 16 != 4 && (cpr + p) % 16 != 12) p++;
    return p;
}

template <int SB, uint32_t BB = 34>
struct Seg {
    static_assert(BB != 34 || SB % 16 == 0, "G mode: segment length a multiple of 16 blocks");
    static_assert((SB * BB) % 16 == 0, "a row segment is whole 16-byte chunks");
    static constexpr uint32_t kCpr = SB * BB / 16;             // 16-byte chunks per row segment
    static constexpr uint32_t kPad = BB == 34 ? (SB == 32 ? 0 : 4) : row_pad(kCpr);
    static constexpr uint32_t kRowChunks = kCpr + kPad;
    static constexpr uint32_t kStageChunks = kUnitRows * kRowChunks;
    static constexpr uint32_t kDma = (kStageChunks + 63) / 64;          // copy wave-instructions per item
    static constexpr uint32_t kLastLanes = kStageChunks - 64 * (kDma - 1);  // lanes of the last one
    static constexpr uint32_t kStageBytes = kStageChunks * 16;
};

// One copy wave-instruction j of an item: the last one runs only its first
// kLastLanes lanes, so a stage holds exactly kStageChunks chunks.  Weights
// are streamed once per launch: non-temporal copies.
template <int SB, uint32_t BB>
__device__ __forceinline__ void copy_chunk(__amdgpu_buffer_rsrc_t w, int8_t* stage, uint32_t j,
                                           uint32_t lane, uint32_t voffset) {
    using G = Seg<SB, BB>;
    if (G::kLastLanes == 64 || j + 1 < G::kDma || lane < G::kLastLanes)
        copy16_to_lds_nt(w, stage + j * 1024, voffset);
}

__device__ __forceinline__ uint32_t umax32(uint32_t a, uint32_t b) { return a > b ? a : b; }

// Per-lane byte offsets (relative to the item's first row) of the chunks a
// full-segment item copies; 0x80000000 marks pad chunks.  Chunk c = lane +
// 64 j is staged row c / kRowChunks, chunk c % kRowChunks.
template <int SB, uint32_t BB>
__device__ __forceinline__ void full_offsets(uint32_t lane, uint32_t rb, uint32_t (&off)[Seg<SB, BB>::kDma]) {
    using G = Seg<SB, BB>;
#pragma unroll
    for (uint32_t j = 0; j < G::kDma; j++) {
        const uint32_t c = j * 64 + lane;
        const uint32_t g = c / G::kRowChunks, cc = c - g * G::kRowChunks;
        off[j] = (g < kUnitRows && cc < G::kCpr) ? g * rb + cc * 16 : 0x80000000u;
    }
}

// Copies one full-segment item: rows_live rows from byte `base` of W.  A
// chunk is live iff its row is below rows_live, i.e. off < rows_live * rb
// (pad offsets exceed every such bound).
template <int SB, uint32_t BB>
__device__ __forceinline__ void issue_full(__amdgpu_buffer_rsrc_t w, int8_t* stage, uint32_t lane, uint32_t base,
                                           uint32_t rows_live, uint32_t rb,
                                           const uint32_t (&off)[Seg<SB, BB>::kDma]) {
    const uint32_t lim = rows_live * rb;
#pragma unroll
    for (uint32_t j = 0; j < Seg<SB, BB>::kDma; j++)
        copy_chunk<SB, BB>(w, stage, j, lane, off[j] < lim ? base + off[j] : 0x80000000u);
}

// The last, shorter segment of a row (nb % SB blocks, a multiple of 8):
// staged stride sbk*BB/16 + pad chunks, offsets computed per call.
template <int SB, uint32_t BB>
__device__ __forceinline__ void issue_partial(__amdgpu_buffer_rsrc_t w, int8_t* stage, uint32_t lane,
                                              uint32_t base, uint32_t rows_live, uint32_t rb,
                                              uint32_t sbk) {
    const uint32_t cpr = sbk * BB / 16;
    const uint32_t rc = cpr + Seg<SB, BB>::kPad;
#pragma unroll
    for (uint32_t j = 0; j < Seg<SB, BB>::kDma; j++) {
        const uint32_t c = j * 64 + lane;
        const uint32_t g = c / rc, cc = c - g * rc;
        const bool live = g < rows_live && cc < cpr;
        copy_chunk<SB, BB>(w, stage, j, lane, live ? base + g * rb + cc * 16 : 0x80000000u);
    }
}

// Activation staging, in passes of one float4 per thread.
//  G mode: pass p covers 32-blocks p*(THREADS/8) ... of the T x nb block
//  grid (8 lanes per block); the 8 lanes reduce max|x|, quantize with the
//  0x19 arithmetic and write 4 bytes each plus the fp32 scale.
//  R mode: pass p covers float4s p*THREADS ... of x, copied as is.
// Loads are four range-checked buffer_load_dword (any 4-byte alignment of
// x and K; lanes past the end read zeros), issued unconditionally so the
// loads of a batch and the ring copies after them are counted exactly by
// the compiler's s_waitcnt placement.
template <int MODE, int THREADS>
struct XStage {
    __amdgpu_buffer_rsrc_t xr;
    uint32_t K, nb, T, n;  // n = blocks (G) or float4s (R)
    int8_t* lds;
    float* dxs;

    static constexpr uint32_t kPerPass = MODE == kModeG ? THREADS / 8 : THREADS;

    __device__ __forceinline__ uint32_t passes() const { return (n + kPerPass - 1) / kPerPass; }

    // shift: extra bytes added to the offset (the up half of gate|up).
    __device__ __forceinline__ float4 load(uint32_t p, uint32_t shift = 0) const {
        uint32_t o = 0x80000000u;
        if (MODE == kModeG) {
            const uint32_t blk = p * kPerPass + (threadIdx.x >> 3);
            const uint32_t t = T == 1 ? 0 : blk / nb, b = blk - t * nb;
            if (blk < n) o = (t * K + b * 32 + (threadIdx.x & 7) * 4) * 4 + shift;
        } else {
            const uint32_t i = p * kPerPass + threadIdx.x;
            if (i < n) o = 16 * i + shift;
        }
        return make_float4(__uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xr, o, 0, 0)),
                           __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xr, o + 4, 0, 0)),
                           __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xr, o + 8, 0, 0)),
                           __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xr, o + 12, 0, 0)));
    }

    // G mode, one token: the norm weights at the same elements as load(p).
    __device__ __forceinline__ float4 load_w(uint32_t p, __amdgpu_buffer_rsrc_t wr) const {
        const uint32_t blk = p * kPerPass + (threadIdx.x >> 3);
        const uint32_t o = blk < n ? (blk * 32 + (threadIdx.x & 7) * 4) * 4 : 0x80000000u;
        return make_float4(__uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(wr, o, 0, 0)),
                           __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(wr, o + 4, 0, 0)),
                           __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(wr, o + 8, 0, 0)),
                           __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(wr, o + 12, 0, 0)));
    }

    __device__ __forceinline__ void store(uint32_t p, float4 f) const {
        if (MODE == kModeG) {
            const uint32_t blk = p * kPerPass + (threadIdx.x >> 3), part = threadIdx.x & 7;
            const uint32_t m =
                max8_u32(umax32(umax32(abs_key(f.x), abs_key(f.y)), umax32(abs_key(f.z), abs_key(f.w))));
            float scale, inv;
            quant_params(__uint_as_float(m), scale, inv);
            if (blk < n) {
                const uint32_t b = T == 1 ? blk : blk % nb;
                const uint32_t half = (part >> 2) ^ ((b >> 3) & 1);
                *reinterpret_cast<uint32_t*>(lds + (uint64_t)blk * 32 + 16 * half + 4 * (part & 3)) =
                    pack4(f.x, f.y, f.z, f.w, inv);
                if (part == 0) dxs[blk] = scale;
            }
        } else {
            const uint32_t i = p * kPerPass + threadIdx.x;
            if (i < n) reinterpret_cast<float4*>(lds)[i] = f;
        }
    }
};

// The staged block at rowp + 34b: its fp16 scale as fp32 and its 32 quants
// as 8 dwords (bytes realigned with v_perm_b32).
struct StagedBlock {
    float dw;
    int q[8];
};

__device__ __forceinline__ StagedBlock load_block(const int8_t* rowp, uint32_t b, uint32_t odd, uint32_t sel,
                                                  uint32_t ssel) {
    const uint32_t* a = reinterpret_cast<const uint32_t*>(rowp + 34 * b - 2 * odd);
    uint32_t D[9];
#pragma unroll
    for (int i = 0; i < 9; i++) D[i] = a[i];
    StagedBlock r;
    r.dw = half_bits_to_float(__builtin_amdgcn_perm(D[1], D[0], ssel));
#pragma unroll
    for (int i = 0; i < 8; i++) r.q[i] = (int)__builtin_amdgcn_perm(D[i + 1], D[i], sel);
    return r;
}

// isum of a staged block against the quantized activation block at xb32
// (32 bytes, halves swapped when h = 1).
__device__ __forceinline__ int block_isum(const StagedBlock& w, const int8_t* xb32, uint32_t h) {
    const v4i* xb = reinterpret_cast<const v4i*>(xb32);
    const v4i x0 = xb[h], x1 = xb[h ^ 1];
    int isum = 0;
    isum = __builtin_amdgcn_sdot4(w.q[0], x0.x, isum, false);
    isum = __builtin_amdgcn_sdot4(w.q[1], x0.y, isum, false);
    isum = __builtin_amdgcn_sdot4(w.q[2], x0.z, isum, false);
    isum = __builtin_amdgcn_sdot4(w.q[3], x0.w, isum, false);
    isum = __builtin_amdgcn_sdot4(w.q[4], x1.x, isum, false);
    isum = __builtin_amdgcn_sdot4(w.q[5], x1.y, isum, false);
    isum = __builtin_amdgcn_sdot4(w.q[6], x1.z, isum, false);
    isum = __builtin_amdgcn_sdot4(w.q[7], x1.w, isum, false);
    return isum;
}

// One G-mode block: isum of the staged block at rowp + 34b against each
// token's quantized block gb, folded into p[t] with one fma.
template <int TT>
__device__ __forceinline__ void block_g(const int8_t* rowp, uint32_t b, uint32_t odd, uint32_t sel,
                                        uint32_t ssel, uint32_t gb, const int8_t* qxs,
                                        const float* dxs, uint32_t nb, uint32_t T, float (&p)[TT]) {
    const StagedBlock w = load_block(rowp, b, odd, sel, ssel);
    const uint32_t h = (gb >> 3) & 1;
#pragma unroll
    for (int t = 0; t < TT; t++) {
        if (TT == 1 || t < (int)T) {
            const int isum = block_isum(w, qxs + ((uint64_t)t * nb + gb) * 32, h);
            const float dd = __fmul_rn(w.dw, dxs[t * nb + gb]);
            p[t] = __builtin_fmaf((float)isum, dd, p[t]);
        }
    }
}

// Blocks b = l, l+16, ... < sbk of one staged row, in increasing order.
template <int SB, int TT, bool Full>
__device__ __forceinline__ void compute_g(const int8_t* rowp, uint32_t l, uint32_t sbk, uint32_t gb0,
                                          const int8_t* qxs, const float* dxs, uint32_t nb,
                                          uint32_t T, float (&p)[TT]) {
    const uint32_t odd = l & 1;
    const uint32_t sel = odd ? 0x07060504u : 0x05040302u;   // quant dword i = bytes 2..5 / 4..7 of {D[i+1]:D[i]}
    const uint32_t ssel = odd ? 0x0c0c0302u : 0x0c0c0100u;  // fp16 scale = bytes 0,1 / 2,3 of D[0]
    if (Full) {
#pragma unroll
        for (uint32_t k = 0; k < SB / 16; k++)
            block_g<TT>(rowp, l + 16 * k, odd, sel, ssel, gb0 + l + 16 * k, qxs, dxs, nb, T, p);
    } else {
        for (uint32_t b = l; b < sbk; b += 16) block_g<TT>(rowp, b, odd, sel, ssel, gb0 + b, qxs, dxs, nb, T, p);
    }
}

// R mode: lane l takes bytes 2+l and 18+l of every block in order.
__device__ __forceinline__ float compute_r(const int8_t* rowp, uint32_t l, uint32_t sbk, uint32_t gb0,
                                           const float* xs, float acc) {
#pragma unroll 8
    for (uint32_t b = 0; b < sbk; b++) {
        const int8_t* blk = rowp + 34 * b;
        const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(blk));
        const float w0 = __fmul_rn((float)blk[2 + l], d);
        const float w1 = __fmul_rn((float)blk[18 + l], d);
        const float* xb = xs + (gb0 + b) * 32;
        acc = __builtin_fmaf(w0, xb[l], acc);
        acc = __builtin_fmaf(w1, xb[16 + l], acc);
    }
    return acc;
}

// R mode over Q4_0 blocks (q4_0_gemv, bytecode_interpreter.s:7071-7126):
// lane l takes the low and the high nibble of byte 2+l of every block in
// order, w = (q - 8) * d then fma with x.  q - 8 is formed without an int
// conversion (the float with bits 2^23 + q, minus 2^23 + 8); the high
// nibble stays in place (16 (q - 8)) and meets d / 16, an exact scaling, so
// both products equal fmul((float)(q - 8), d) bit for bit.
__device__ __forceinline__ float compute_r4(const int8_t* rowp, uint32_t l, uint32_t sbk, uint32_t gb0,
                                            const float* xs, float acc) {
#pragma unroll 8
    for (uint32_t b = 0; b < sbk; b++) {
        const uint8_t* blk = reinterpret_cast<const uint8_t*>(rowp) + 18 * b;
        const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(blk));
        const uint32_t q = blk[2 + l];
        const float lo = __fsub_rn(__uint_as_float((q & 15u) | 0x4B000000u), 8388616.0f);
        const float hi = __fsub_rn(__uint_as_float((q & 0xF0u) | 0x4B000000u), 8388736.0f);
        const float* xb = xs + (gb0 + b) * 32;
        acc = __builtin_fmaf(__fmul_rn(lo, d), xb[l], acc);
        acc = __builtin_fmaf(__fmul_rn(hi, __fmul_rn(d, 0.0625f)), xb[16 + l], acc);
    }
    return acc;
}

// K-quant GEMVs: lane l's fmas over each staged super-block in order, with
// the format's decoder (the same code as k_qgemv, so the same bits).
// The staged rows start 16-byte aligned, so super-block p sits at the
// alignment gcd(kBytes, 16) and the decoders read its fields with typed loads.
template <class F>
__device__ __forceinline__ float compute_qf(const int8_t* rowp, uint32_t l, uint32_t sbk, uint32_t gsb0,
                                            const float* xs, float acc) {
    constexpr int kAlign = F::kBytes % 16 == 0 ? 16 : F::kBytes % 4 == 0 ? 4 : F::kBytes % 2 == 0 ? 2 : 1;
    for (uint32_t p = 0; p < sbk; p++)
        F::template acc<kAlign>(reinterpret_cast<const uint8_t*>(rowp) + p * F::kBytes, xs + (gsb0 + p) * 256, l,
                                acc);
    return acc;
}

// Optional fusions of the G-mode single-token kernel (the decode step):
//  kFuseNorm: x' = fl(fl(x * inv) * w) with inv = 1 / sqrt(fl(fl(ss / K) + eps)),
//    ss = the sum of x^2 in fp64 in the canonical order of common.hpp
//    (sumsq4_f64 .. canon_total_f64), the same bits as the standalone
//    ane_hip_rms_norm and the oracle, then x' is quantized as usual;
//  kFuseResidual: y[n] = fl(FADDV(p) + r[n]) (r may alias y: each row is read
//    by the wave that owns it, into LDS, before that wave writes it).
//  kFuseSiluMul: the input is gate|up (2K floats) and the row quantized is
//    x[i] = (g / (1 + expf(-g))) * u with g = in[i], u = in[K + i].
//  kFusePreQuant: the input is already quantized (qx [nb][32] int8, then dx
//    [nb] fp32, as the staging would have produced it) and is copied into LDS.
//  kFuseSiluQuant: the rows are gate|up interleaved in 32-row groups (rows
//    64k..64k+31 = gate 32k.., rows 64k+32..64k+63 = up 32k..); a workgroup
//    owns one 64-row group, keeps its outputs in LDS and writes
//    q8(silu(gate) * up) for those 32 values: one block of the Q8 activation
//    form (qx at y, dx at y + N/2 bytes), as ane_hip_silu_mul_quant would.
enum { kFuseNorm = 1, kFuseResidual = 2, kFuseSiluMul = 4, kFusePreQuant = 8, kFuseSiluQuant = 16 };

struct StreamFuse {
    const float* norm_w;
    float eps;
    const float* residual;
};

// The prologue of the streaming kernels: copies the residual of rows
// r0 .. r1-1 (at most 64, one per lane) into this wave's LDS slot rres,
// issues the activation loads (and those of the norm weights or the up
// half), then ring_start() to put the first RING weight copies in flight
// behind them, applies the fusions, stores x into LDS and waits for every
// wave.
template <int MODE, int NW, int FUSE, int RING, int XB, class Start>
__device__ __forceinline__ void stream_prologue(const XStage<MODE, NW * 64>& xst, const StreamFuse& fz,
                                                uint32_t N, uint32_t r0, uint32_t r1, double* red, float* rres,
                                                Start&& ring_start) {
    static_assert(!(FUSE & kFusePreQuant) || !(FUSE & (kFuseNorm | kFuseSiluMul)),
                  "a pre-quantized input takes no activation fusion");
    const uint32_t npass = xst.passes();
    const uint32_t lane = threadIdx.x & 63;
    if (FUSE & kFuseResidual) {  // issued first: every later wait covers it
        const __amdgpu_buffer_rsrc_t rr = make_rsrc(fz.residual, N * 4);
        copy4_to_lds(rr, rres, r0 + lane < r1 ? (r0 + lane) * 4 : 0x80000000u);
    }
    if (FUSE & kFusePreQuant) {
        // 16-byte chunks: 2n of qx (n = T*nb blocks; the halves of token
        // block b swapped on odd b/8, as XStage::store writes them), then n/4
        // of dx
        const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const uint32_t nq = 2 * xst.n, nchunks = nq + xst.n / 4;
        for (uint32_t c0 = wave * 64; c0 < nchunks; c0 += NW * 64) {
            const uint32_t c = c0 + lane, blk = c >> 1, b = blk % xst.nb;
            const uint32_t src = c < nq ? (2 * blk + ((c & 1) ^ ((b >> 3) & 1))) * 16 : c * 16;
            if (c < nchunks) copy16_to_lds(xst.xr, xst.lds + c0 * 16, src);
        }
        ring_start();
        wait_vmcnt<RING>();  // the activation copies have landed (the ring's may be in flight)
        lds_barrier();
        return;
    }
    float4 xv[XB];
#pragma unroll
    for (uint32_t k = 0; k < XB; k++) xv[k] = xst.load(k);
    float4 wv[(FUSE & (kFuseNorm | kFuseSiluMul)) ? XB : 1];
    if (FUSE & kFuseNorm) {
        const __amdgpu_buffer_rsrc_t wr = make_rsrc(fz.norm_w, xst.K * 4);
#pragma unroll
        for (uint32_t k = 0; k < XB; k++) wv[k] = xst.load_w(k, wr);
    }
    if (FUSE & kFuseSiluMul) {
#pragma unroll
        for (uint32_t k = 0; k < XB; k++) wv[k] = xst.load(k, xst.K * 4);  // up
    }
    ring_start();
    if (FUSE & kFuseSiluMul) {
#pragma unroll
        for (uint32_t k = 0; k < XB; k++) {
            const float4 g = xv[k], u = wv[k];
            xv[k] = make_float4(silu_mul1(g.x, u.x), silu_mul1(g.y, u.y), silu_mul1(g.z, u.z), silu_mul1(g.w, u.w));
        }
    }
    if (FUSE & kFuseNorm) {  // the host guarantees npass <= XB for this fusion
        // the canonical order of common.hpp: block sums into the x staging
        // area (free until the quantized x is stored), then wave 0's tree
        double* sums = reinterpret_cast<double*>(xst.lds);
#pragma unroll
        for (uint32_t k = 0; k < XB; k++) {
            if (k < npass) {  // uniform: every lane takes the same passes
                const double sb = sum8_f64(sumsq4_f64(xv[k]));  // lanes past the end hold zeros
                const uint32_t blk = k * XStage<MODE, NW * 64>::kPerPass + (threadIdx.x >> 3);
                if ((threadIdx.x & 7) == 0 && blk < xst.n) sums[blk] = sb;
            }
        }
        wait_lgkmcnt0();
        lds_barrier();
        if (threadIdx.x < 64) {
            const double tot = canon_total_f64(sums, xst.n);
            if (threadIdx.x == 0) red[0] = tot;
        }
        // a second barrier: the quantized x is stored over the block sums
        wait_lgkmcnt0();
        lds_barrier();
        const double ss = red[0];
        const float inv = rms_inv(ss, xst.K, fz.eps);
#pragma unroll
        for (uint32_t k = 0; k < XB; k++) {
            const float4 f = xv[k], w4 = wv[k];
            xv[k] = make_float4(__fmul_rn(__fmul_rn(f.x, inv), w4.x), __fmul_rn(__fmul_rn(f.y, inv), w4.y),
                                __fmul_rn(__fmul_rn(f.z, inv), w4.z), __fmul_rn(__fmul_rn(f.w, inv), w4.w));
        }
    }
#pragma unroll
    for (uint32_t k = 0; k < XB; k++)
        if (k < npass) xst.store(k, xv[k]);
    for (uint32_t p0 = XB; p0 < npass; p0 += XB) {  // SiLU*up is elementwise: any K
#pragma unroll
        for (uint32_t k = 0; k < XB; k++) xv[k] = xst.load(p0 + k);
        if (FUSE & kFuseSiluMul) {
#pragma unroll
            for (uint32_t k = 0; k < XB; k++) wv[k] = xst.load(p0 + k, xst.K * 4);
#pragma unroll
            for (uint32_t k = 0; k < XB; k++) {
                const float4 g = xv[k], u = wv[k];
                xv[k] = make_float4(silu_mul1(g.x, u.x), silu_mul1(g.y, u.y), silu_mul1(g.z, u.z),
                                    silu_mul1(g.w, u.w));
            }
        }
#pragma unroll
        for (uint32_t k = 0; k < XB; k++)
            if (p0 + k < npass) xst.store(p0 + k, xv[k]);
    }
    wait_lgkmcnt0();
    lds_barrier();
}

template <int MODE, int NW, int SB, int S, int TT, int FUSE = 0, int XB = kXBatch>
__global__ void __launch_bounds__(NW * 64)
k_q8_0_stream(uint32_t N, uint32_t nb, uint32_t K, uint32_t T, const float* __restrict__ x,
              const uint8_t* __restrict__ W, float* y, uint32_t total_waves, StreamFuse fz) {
    constexpr uint32_t BB = kBlockBytes<MODE>;
    using G = Seg<SB, BB>;
    static_assert(FUSE == 0 || (MODE == kModeG && (TT == 1 || FUSE == kFusePreQuant)),
                  "fusions are for the G-mode decode step; a pre-quantized input takes any token count");
    static_assert(S * G::kDma < 64, "copies in flight exceed the vmcnt range");
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63, grp = lane >> 4, l = lane & 15;
    int8_t* ring = smem + wave * (S * G::kStageBytes);
    int8_t* xlds = smem + NW * S * G::kStageBytes;

    const uint32_t gw = blockIdx.x * NW + wave;
    static_assert(!(FUSE & kFuseSiluQuant) || (64 / NW) % kUnitRows == 0, "whole units per wave");
    const uint32_t r0 = (FUSE & kFuseSiluQuant) ? blockIdx.x * 64 + wave * (64 / NW)
                                                : (uint32_t)(((uint64_t)gw * N) / total_waves);
    const uint32_t r1 = (FUSE & kFuseSiluQuant) ? min(r0 + 64 / NW, N)
                                                : (uint32_t)(((uint64_t)(gw + 1) * N) / total_waves);
    const uint32_t nseg = (nb + SB - 1) / SB;
    const uint32_t nitems = (r1 - r0 + kUnitRows - 1) / kUnitRows * nseg;
    const uint32_t rb = nb * BB;
    const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(W, N * rb);
    uint32_t off[G::kDma];
    full_offsets<SB, BB>(lane, rb, off);

    auto issue = [&](uint32_t i) {
        const uint32_t u = i / nseg, s = i - u * nseg;
        const uint32_t row0 = r0 + kUnitRows * u;
        const uint32_t rows_live = i < nitems ? min((uint32_t)kUnitRows, r1 - row0) : 0u;
        const uint32_t sbk = min((uint32_t)SB, nb - s * SB);
        int8_t* stage = ring + (i % S) * G::kStageBytes;
        const uint32_t base = row0 * rb + s * (SB * BB);
        if (sbk == (uint32_t)SB) issue_full<SB, BB>(rsrc, stage, lane, base, rows_live, rb, off);
        else issue_partial<SB, BB>(rsrc, stage, lane, base, rows_live, rb, sbk);
    };

    const int8_t* qxs = xlds;
    float* dxs = reinterpret_cast<float*>(xlds + ceil_to((uint64_t)T * nb * 32, 16));
    const float* xs = reinterpret_cast<const float*>(xlds);
    const uint32_t xbytes = (FUSE & kFusePreQuant) ? T * nb * 36 : ((FUSE & kFuseSiluMul) ? 2 : 1) * T * K * 4;
    const XStage<MODE, NW * 64> xst{make_rsrc(x, xbytes), K, nb, T,
                                    MODE == kModeG ? nb * T : nb * (kBlockValues<MODE> / 4), xlds, dxs};
    const auto ring_start = [&] {
#pragma unroll
        for (int i = 0; i < S; i++) issue(i);
    };
    double* red = reinterpret_cast<double*>(xlds + stream_x_bytes(MODE, nb, T));
    float* rres = reinterpret_cast<float*>(red + NW) + wave * 64;
    float* hq = reinterpret_cast<float*>(red + NW) + NW * 64;  // the group's 64 outputs (kFuseSiluQuant)
    stream_prologue<MODE, NW, FUSE, S * G::kDma, XB>(xst, fz, N, r0, r1, red, rres, ring_start);

    float p[TT];
#pragma unroll
    for (int t = 0; t < TT; t++) p[t] = 0.0f;
    for (uint32_t i = 0; i < nitems; i++) {
        wait_vmcnt<(S - 1) * G::kDma>();  // item i has landed (items i+1 .. i+S-1 may be in flight)
        const uint32_t u = i / nseg, s = i - u * nseg;
        const uint32_t sbk = min((uint32_t)SB, nb - s * SB);
        const int8_t* rowp = ring + (i % S) * G::kStageBytes + grp * (sbk * BB / 16 + G::kPad) * 16;
        if (s == 0) {
#pragma unroll
            for (int t = 0; t < TT; t++) p[t] = 0.0f;
        }
        if constexpr (MODE == kModeG) {
            if (sbk == (uint32_t)SB) compute_g<SB, TT, true>(rowp, l, sbk, s * SB, qxs, dxs, nb, T, p);
            else compute_g<SB, TT, false>(rowp, l, sbk, s * SB, qxs, dxs, nb, T, p);
        } else if constexpr (kIsQK<MODE>) {
            p[0] = compute_qf<typename ModeFmt<MODE>::F>(rowp, l, sbk, s * SB, xs, p[0]);
        } else if (MODE == kModeR4) {
            p[0] = compute_r4(rowp, l, sbk, s * SB, xs, p[0]);
        } else {
            p[0] = compute_r(rowp, l, sbk, s * SB, xs, p[0]);
        }
        if (s == nseg - 1) {
            const uint32_t row = r0 + kUnitRows * u + grp;
#pragma unroll
            for (int t = 0; t < TT; t++) {
                float v = faddv16(p[t]);
                if (FUSE & kFuseResidual) v = v + rres[kUnitRows * u + grp];
                if (FUSE & kFuseSiluQuant) {
                    if (l == 0 && row < r1) hq[row - blockIdx.x * 64] = v;
                } else if (l == 0 && row < r1 && (TT == 1 || t < (int)T)) {
                    y[(uint64_t)t * N + row] = v;
                }
            }
        }
        wait_lgkmcnt0();  // this stage's LDS reads are done before it is refilled
        issue(i + S);
    }
    wait_vmcnt<0>();  // no copy may land in LDS after the workgroup ends
    if (FUSE & kFuseSiluQuant) {
        __syncthreads();
        if (wave == 0 && lane < 32) {  // 32 values of h, the 0x19 arithmetic over the block
            const float h = silu_mul1(hq[lane], hq[32 + lane]);
            uint32_t m = abs_key(h);
#pragma unroll
            for (int o = 16; o >= 1; o >>= 1) {
                const uint32_t q = __shfl_xor(m, o, kWave);
                m = m > q ? m : q;
            }
            float bs, inv;
            quant_params(__uint_as_float(m), bs, inv);
            uint8_t* out = reinterpret_cast<uint8_t*>(y);
            out[blockIdx.x * 32 + lane] = (uint8_t)quant1(h, inv);
            if (lane == 0) reinterpret_cast<float*>(out + N / 2)[blockIdx.x] = bs;
        }
    }
}

constexpr uint32_t kLdsLimit = 160 * 1024;

constexpr int kMaxStreamTokens = 4;

bool stream_eligible(uint32_t N, uint32_t nb, uint32_t K, uint32_t T, const void* W, uint32_t block_bytes = 34) {
    return nb > 0 && nb % 8 == 0 && (((uintptr_t)W) & 15) == 0 &&
           (uint64_t)N * nb * block_bytes < 0x80000000ull && (uint64_t)T * K * 4 < 0x80000000ull;
}

template <int MODE, int NW, int SB, int S>
uint64_t stream_lds(uint32_t nb, uint32_t T) {
    return (uint64_t)NW * S * Seg<SB, kBlockBytes<MODE>>::kStageBytes + stream_x_bytes(MODE, nb, T) + 8 * NW +
           256 * NW + 256;
}

int cu_count(int dev) {
    static std::atomic<int> cached[64];
    if (dev < 0 || dev >= 64) return 0;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (!n) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Host state of one streaming-kernel instantiation: its dynamic-LDS limit is
// raised to kLdsLimit once per device (so launches of any size up to that
// stay valid whichever thread set it), and its occupancy is cached per
// (device, LDS size).  A mutex makes both safe for concurrent host threads.
struct StreamLaunchCache {
    std::mutex mu;
    bool attr[64] = {};
    std::map<uint64_t, int> occ;
};

// The occupancy of fn at `lds` bytes of dynamic LDS, or a negative status.
int stream_occupancy(StreamLaunchCache& c, const void* fn, int dev, int threads, uint32_t lds) {
    std::lock_guard<std::mutex> lock(c.mu);
    if (!c.attr[dev]) {
        if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsLimit) != hipSuccess)
            return ANE_ERR_HIP;
        c.attr[dev] = true;
    }
    const uint64_t key = ((uint64_t)dev << 32) | lds;
    const auto it = c.occ.find(key);
    if (it != c.occ.end()) return it->second;
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, threads, lds) != hipSuccess || occ < 1)
        return ANE_ERR_HIP;
    c.occ[key] = occ;
    return occ;
}

// Launches one configuration if its LDS fits; returns -1 if it does not.
// Occupancy is queried once per (device, LDS size).
template <int MODE, int NW, int SB, int S, int TT, int FUSE = 0, int XB = kXBatch>
int try_stream(uint32_t N, uint32_t nb, uint32_t K, uint32_t T, const float* x, const void* W,
               float* y, hipStream_t s, StreamFuse fz = StreamFuse{nullptr, 0.0f, nullptr}) {
    const uint64_t lds64 = stream_lds<MODE, NW, SB, S>(nb, T);
    if (lds64 > kLdsLimit) return -1;
    const uint32_t lds = (uint32_t)lds64;
    auto fn = k_q8_0_stream<MODE, NW, SB, S, TT, FUSE, XB>;
    static StreamLaunchCache cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return ANE_ERR_HIP;
    const int occ = stream_occupancy(cache, reinterpret_cast<const void*>(fn), dev, NW * 64, lds);
    if (occ < 0) return occ;
    const int cus = cu_count(dev);
    if (cus <= 0) return ANE_ERR_HIP;
    const uint64_t units = ((uint64_t)N + kUnitRows - 1) / kUnitRows;
    uint64_t grid = (uint64_t)cus * occ;
    const uint64_t need = (units + NW - 1) / NW;
    if (grid > need) grid = need;
    if (grid < 1) grid = 1;
    // the residual fusion holds one row per lane: at most 64 rows per wave
    if ((FUSE & kFuseResidual) && ((uint64_t)N + grid * NW - 1) / (grid * NW) > 64) return -1;
    // the norm fusion holds all of x in registers until the sum of squares is known
    if ((FUSE & kFuseNorm) && (nb + NW * 8 - 1) / (NW * 8) > XB) return -1;
    if (t_plan_only) return ANE_OK;
    hipLaunchKernelGGL(fn, dim3((uint32_t)grid), dim3(NW * 64), lds, s, N, nb, K, T, x,
                       (const uint8_t*)W, y, (uint32_t)(grid * NW), fz);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

// Configuration choice (waves per workgroup, blocks per segment, ring
// stages).  A wave takes whole 4-row units, so a matrix with few units per
// CU runs the 4-wave configuration: the 8-wave one would
// leave CUs idle (4096 rows = 1024 units = 128 eight-wave workgroups).
// Otherwise the 8-wave configuration (two workgroups per CU).  The first
// configuration whose LDS fits is launched.
#ifndef ANE_Q8_SMALL_UNITS_PER_CU
#define ANE_Q8_SMALL_UNITS_PER_CU 12
#endif
#ifndef ANE_Q8_SMALL_CFG
#define ANE_Q8_SMALL_CFG 4, 32, 2
#endif
#ifndef ANE_Q8_LARGE_CFG
#define ANE_Q8_LARGE_CFG 8, 32, 2
#endif

template <int NW, int SB, int S>
struct SmallCfg {
    static constexpr int kNw = NW;
};
using Q8SmallCfg = SmallCfg<ANE_Q8_SMALL_CFG>;

template <int MODE, int TT, int FUSE = 0>
int stream_auto(uint32_t N, uint32_t nb, uint32_t K, uint32_t T, const float* x, const void* W, float* y,
                hipStream_t s, StreamFuse fz = StreamFuse{nullptr, 0.0f, nullptr}) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return ANE_ERR_HIP;
    const uint64_t units = ((uint64_t)N + kUnitRows - 1) / kUnitRows;
    int r = -1;
    if constexpr (MODE == kModeR && FUSE == 0 && TT == 1) {
        // R mode keeps x as fp32 in LDS (16 KB at K = 4096), so its workgroup
        // shapes differ (measured, 14336/4096 rows x 4096/14336): 16 waves of
        // 16-block stages for many rows (20.4 -> 18.9 us), 2 waves of 32-block
        // stages for few (10.2 -> 9.6 us, 27.1 -> 26.3 us)
        const bool few = units < (uint64_t)cu_count(dev) * ANE_Q8_SMALL_UNITS_PER_CU;
        r = few ? try_stream<MODE, 2, 32, 2, TT, FUSE>(N, nb, K, T, x, W, y, s, fz)
                : try_stream<MODE, 16, 16, 2, TT, FUSE>(N, nb, K, T, x, W, y, s, fz);
        if (r >= 0) return r;
    }
    if constexpr (MODE == kModeG && TT == kMaxStreamTokens && FUSE == kFusePreQuant) {
        // 2-4 pre-quantized tokens over many rows: 16-block stages leave
        // room for two workgroups per CU beside the activations (gate_up
        // 28672x4096 at T = 4: 31.3 -> 29.6 us; fewer rows measured best on
        // the shapes below)
        if (units >= (uint64_t)cu_count(dev) * ANE_Q8_SMALL_UNITS_PER_CU) {
            r = try_stream<MODE, 8, 16, 2, TT, FUSE>(N, nb, K, T, x, W, y, s, fz);
            if (r >= 0) return r;
        }
    }
    if (units < (uint64_t)cu_count(dev) * ANE_Q8_SMALL_UNITS_PER_CU) {
        // a plain single-token product whose activation needs 9-16 passes
        // loads all of it before the ring's copies (one batch of 16)
        constexpr int kSmallNw = Q8SmallCfg::kNw;
        const uint64_t per_pass = MODE == kModeG ? kSmallNw * 64 / 8 : kSmallNw * 64;
        const uint64_t npass =
            ((MODE == kModeG ? (uint64_t)nb * T : (uint64_t)nb * (kBlockValues<MODE> / 4)) + per_pass - 1) / per_pass;
        if (FUSE == 0 && TT == 1 && npass > kXBatch && npass <= 2 * kXBatch)
            r = try_stream<MODE, ANE_Q8_SMALL_CFG, TT, FUSE, 2 * kXBatch>(N, nb, K, T, x, W, y, s, fz);
        else
            r = try_stream<MODE, ANE_Q8_SMALL_CFG, TT, FUSE>(N, nb, K, T, x, W, y, s, fz);
    }
    if (r < 0) r = try_stream<MODE, ANE_Q8_LARGE_CFG, TT, FUSE>(N, nb, K, T, x, W, y, s, fz);
    if (r < 0) r = try_stream<MODE, 4, 32, 2, TT, FUSE>(N, nb, K, T, x, W, y, s, fz);
    return r;
}

// The gate|up product of the decode step with SiLU*up quantized in its
// epilogue: one workgroup per 64-row group; 8 waves of 2 units each with
// 2-stage rings measured fastest (4 waves x 4 stages, 16 waves and 3-stage
// rings were slower).
int gate_up_silu_quant(uint32_t N, uint32_t nb, uint32_t K, const float* x, const void* W, void* xq,
                       hipStream_t s, StreamFuse fz) {
#ifndef ANE_GU_CFG
#define ANE_GU_CFG 8, 32, 2
#endif
    constexpr int kCfg[3] = {ANE_GU_CFG};
    constexpr int kNw = kCfg[0], kSb = kCfg[1], kS = kCfg[2];
    constexpr int kFuse = kFuseNorm | kFuseSiluQuant;
    const uint64_t lds64 = stream_lds<kModeG, kNw, kSb, kS>(nb, 1);
    if (lds64 > kLdsLimit || (nb + kNw * 8 - 1) / (kNw * 8) > kXBatch) return -1;
    auto fn = k_q8_0_stream<kModeG, kNw, kSb, kS, 1, kFuse>;
    static StreamLaunchCache cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return ANE_ERR_HIP;
    const int occ = stream_occupancy(cache, reinterpret_cast<const void*>(fn), dev, kNw * 64, (uint32_t)lds64);
    if (occ < 0) return occ;
    if (t_plan_only) return ANE_OK;
    hipLaunchKernelGGL(fn, dim3(N / 64), dim3(kNw * 64), (uint32_t)lds64, s, N, nb, K, 1u, x, (const uint8_t*)W,
                       static_cast<float*>(xq), 0u, fz);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

// ====================================================== MFMA mul_mat (T > 4)
// G mode for 5+ tokens.  One v_mfma_i32_16x16x32_i8 is exactly one Q8_0
// block's isum for a tile of 16 weight rows x 16 tokens (K = 32 = one
// block), so the matrix cores produce the integer dots and the fp32 part
// stays the definition's: lane (g, t) holds the tile's rows 4g..4g+3 for
// token t, folds block b into p[b % 16][i] = fmaf((float)isum,
// fl(d_w * d_x), p[b % 16][i]) in increasing b, and the row result is the
// FADDV tree over the 16 partials.
//
// A workgroup of RT x TT x KS waves takes RT row tiles x TT token tiles.
// They share a ring of S stages in LDS; a stage is 16 blocks of the RT*16
// weight rows (34-byte blocks, rows 35 chunks apart), of the TT*16 tokens'
// quantized activations (rows 34 chunks apart) and of their fp32 scales,
// copied global -> LDS with buffer_load_dwordx4 ... lds.  The copy
// instructions of a stage are dealt round-robin to the waves; each stage
// ends with s_waitcnt + s_barrier.  With more than two stages a wave with
// fewer real copies issues zero-copies into its own trash slot, so every
// wave has the same count in flight and the s_waitcnt immediates stay
// exact; with two stages every wave waits for vmcnt(0) and issues none
// (the padding was measured at 7-17 % of the config-4 time: the copy
// instructions' issue, not their bytes, paces these kernels).
//
// KS > 1 splits the 16 blocks of a stage among KS waves of the same tile by
// residue: wave ks computes blocks b with (b % 16) / (16 / KS) == ks, so each
// of the 16 fp32 chains stays inside one wave in its own order, and the
// partials only meet, through LDS, for the final FADDV tree.
constexpr uint32_t kMmaSb = 16;                           // blocks per stage
constexpr uint32_t kMmaWRowChunks = kMmaSb * 17 / 8 + 1;  // 34 + 1 pad
constexpr uint32_t kMmaXRowChunks = kMmaSb * 2 + 2;       // 32 + 2 pad
constexpr uint32_t kMmaDTokChunks = kMmaSb * 4 / 16;      // 4: 16 fp32 scales per token

template <int RT, int TT, int KS>
struct MmaLayout {
    static constexpr int kNw = RT * TT * KS;
    static constexpr uint32_t kWChunks = RT * 16 * kMmaWRowChunks;
    static constexpr uint32_t kXChunks = TT * 16 * kMmaXRowChunks;
    static constexpr uint32_t kDChunks = TT * 16 * kMmaDTokChunks;
    static constexpr uint32_t kWInstr = (kWChunks + 63) / 64, kXInstr = (kXChunks + 63) / 64,
                              kDInstr = (kDChunks + 63) / 64;
    // copy slots per wave (instructions dealt round-robin)
    static constexpr uint32_t kWSlots = (kWInstr + kNw - 1) / kNw, kXSlots = (kXInstr + kNw - 1) / kNw,
                              kDSlots = (kDInstr + kNw - 1) / kNw;
    static constexpr uint32_t kSlots = kWSlots + kXSlots + kDSlots;  // copy instructions per wave per stage
    static constexpr uint32_t kXOff = kWChunks * 16, kDOff = kXOff + kXChunks * 16;
    static constexpr uint32_t kStageBytes = kDOff + kDChunks * 16;
};

template <int RT, int TT, int KS, int S>
__global__ void __launch_bounds__(RT * TT * KS * 64)
k_q8_0_mma(uint32_t N, uint32_t nb, uint32_t T, const uint8_t* __restrict__ W, const uint8_t* __restrict__ qws,
           uint32_t dx_off, uint32_t n_ttiles, float* __restrict__ y) {
    using L = MmaLayout<RT, TT, KS>;
    constexpr int NW = L::kNw;
    constexpr uint32_t kSbw = kMmaSb / KS;  // blocks of a stage per wave
    static_assert(kMmaSb % KS == 0, "KS divides the 16 residues");
    static_assert((S - 1) * L::kSlots < 64, "copies in flight exceed the vmcnt range");
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    int8_t* trash = smem + S * L::kStageBytes;  // 1 KB per wave for padding copies
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
    const uint32_t ks = wave % KS, tt = (wave / KS) % TT, rt = wave / (KS * TT);

    // workgroup tile: row tiles [rbase, rbase + RT), token tiles [tbase, tbase + TT)
    const uint32_t wg_t = blockIdx.x % ((n_ttiles + TT - 1) / TT), wg_r = blockIdx.x / ((n_ttiles + TT - 1) / TT);
    const uint32_t row_base = wg_r * RT * 16, tok_base = wg_t * TT * 16;
    const uint32_t rb = nb * 34;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(W, N * rb);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(qws, dx_off + T * nb * 4);
    const uint32_t nst = nb / kMmaSb;

    // per-slot source offsets at stage 0 (0x80000000: pad, dead row or token)
    uint32_t ow[L::kWSlots], ox[L::kXSlots], od[L::kDSlots];
#pragma unroll
    for (uint32_t q = 0; q < L::kWSlots; q++) {
        const uint32_t c = 64 * (q * NW + wave) + lane, r = c / kMmaWRowChunks, sub = c - r * kMmaWRowChunks;
        const uint32_t row = row_base + r;
        ow[q] = (c < L::kWChunks && sub < kMmaSb * 17 / 8 && row < N) ? row * rb + 16 * sub : 0x80000000u;
    }
#pragma unroll
    for (uint32_t q = 0; q < L::kXSlots; q++) {
        const uint32_t c = 64 * (q * NW + wave) + lane, t = c / kMmaXRowChunks, sub = c - t * kMmaXRowChunks;
        const uint32_t tok = tok_base + t;
        ox[q] = (c < L::kXChunks && sub < 2 * kMmaSb && tok < T) ? tok * nb * 32 + 16 * sub : 0x80000000u;
    }
#pragma unroll
    for (uint32_t q = 0; q < L::kDSlots; q++) {
        const uint32_t c = 64 * (q * NW + wave) + lane, t = c / kMmaDTokChunks, sub = c - t * kMmaDTokChunks;
        const uint32_t tok = tok_base + t;
        od[q] = (c < L::kDChunks && tok < T) ? dx_off + tok * nb * 4 + 16 * sub : 0x80000000u;
    }
    // one copy slot: instruction i of a region if it exists (lanes past the
    // region's last chunk masked; lane 0 is always live), else zeros into trash
    auto slot = [&](__amdgpu_buffer_rsrc_t r, int8_t* region, uint32_t ninstr, uint32_t nchunks, uint32_t q,
                    uint32_t src) {
        const uint32_t i = q * NW + wave;
        if (i < ninstr) {
            if (nchunks % 64 == 0 || i + 1 < ninstr || lane < nchunks % 64) copy16_to_lds(r, region + 1024 * i, src);
        } else if (S > 2) {  // padding that keeps vmcnt counts uniform
            copy16_to_lds(r, trash + 1024 * wave, 0x80000000u);
        }
    };
    auto issue = [&](uint32_t s) {
        int8_t* st = smem + (s % S) * L::kStageBytes;
        const bool on = s < nst;
#pragma unroll
        for (uint32_t q = 0; q < L::kWSlots; q++)
            slot(wr, st, L::kWInstr, L::kWChunks, q,
                 on && ow[q] != 0x80000000u ? ow[q] + s * (kMmaSb * 34) : 0x80000000u);
#pragma unroll
        for (uint32_t q = 0; q < L::kXSlots; q++)
            slot(xr, st + L::kXOff, L::kXInstr, L::kXChunks, q,
                 on && ox[q] != 0x80000000u ? ox[q] + s * (kMmaSb * 32) : 0x80000000u);
#pragma unroll
        for (uint32_t q = 0; q < L::kDSlots; q++)
            slot(xr, st + L::kDOff, L::kDInstr, L::kDChunks, q,
                 on && od[q] != 0x80000000u ? od[q] + s * (kMmaSb * 4) : 0x80000000u);
    };

    float p[kSbw][4];
#pragma unroll
    for (uint32_t b = 0; b < kSbw; b++)
#pragma unroll
        for (int i = 0; i < 4; i++) p[b][i] = 0.0f;
#pragma unroll
    for (int s = 0; s < S - 1; s++) issue(s);
    for (uint32_t s = 0; s < nst; s++) {
        wait_vmcnt<(S - 2) * L::kSlots>();  // this wave's copies of stage s have landed
        __builtin_amdgcn_s_barrier();       // everyone's have; everyone is done with stage s-1
        issue(s + S - 1);                    // refills the slot of stage s-1
        const int8_t* st = smem + (s % S) * L::kStageBytes;
        const int8_t* wa = st + (rt * 16 + c16) * (kMmaWRowChunks * 16);                  // A: weight row
        const int8_t* xb = st + L::kXOff + (tt * 16 + c16) * (kMmaXRowChunks * 16);      // B: token
        const float* dxs = reinterpret_cast<const float*>(st + L::kDOff) + (tt * 16 + c16) * kMmaSb;
        const int8_t* wrow = st + (rt * 16 + 4 * g) * (kMmaWRowChunks * 16);             // rows 4g.. for d_w
#pragma unroll
        for (uint32_t j = 0; j < kSbw; j++) {
            const uint32_t bb = ks * kSbw + j;  // block of the stage; b % 16 == bb
            const uint32_t o = 34 * bb + 2 + 8 * g;
            const uint32_t* a32 = reinterpret_cast<const uint32_t*>(wa + (o & ~3u));
            uint32_t a0, a1;
            static_assert(kSbw % 2 == 0, "bb and j share their parity");
            if (j & 1) {  // 34bb + 2 is 4-byte aligned for odd bb
                a0 = a32[0];
                a1 = a32[1];
                asm("" : "+v"(a0));  // two loads, not one fused load without alias information
            } else {
                const uint32_t d0 = a32[0], d1 = a32[1], d2 = a32[2];
                a0 = __builtin_amdgcn_alignbyte(d1, d0, 2);
                a1 = __builtin_amdgcn_alignbyte(d2, d1, 2);
            }
            const uint64_t av = (uint64_t)a0 | ((uint64_t)a1 << 32);
            const uint64_t bv = *reinterpret_cast<const uint64_t*>(xb + 32 * bb + 8 * g);
            const v4i acc = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)av, (long)bv, v4i{0, 0, 0, 0}, 0, 0, 0);
            const float dx = lds_load_settled_f32(dxs + bb);
#pragma unroll
            for (int i = 0; i < 4; i++) {  // output row 4g + i of the tile, token c16
                const uint16_t dwb = *reinterpret_cast<const uint16_t*>(wrow + i * (kMmaWRowChunks * 16) + 34 * bb);
                p[j][i] = __builtin_fmaf((float)acc[i], __fmul_rn(half_bits_to_float(dwb), dx), p[j][i]);
            }
        }
    }
    wait_vmcnt<0>();
    const uint32_t row0 = row_base + rt * 16, t0 = tok_base + tt * 16;
    if (KS > 1) {
        // partials [tile][residue][lane][4] over the ring; wave ks holds residues ks*kSbw ..
        __syncthreads();
        float4* ex = reinterpret_cast<float4*>(smem) + (uint64_t)(rt * TT + tt) * 16 * 64;
#pragma unroll
        for (uint32_t j = 0; j < kSbw; j++)
            ex[(ks * kSbw + j) * 64 + lane] = make_float4(p[j][0], p[j][1], p[j][2], p[j][3]);
        __syncthreads();
        if (ks == 0) {
            float q[16][4];
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float4 v = ex[r * 64 + lane];
                q[r][0] = v.x;
                q[r][1] = v.y;
                q[r][2] = v.z;
                q[r][3] = v.w;
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float t8[8], t4[4];
#pragma unroll
                for (int l = 0; l < 8; l++) t8[l] = q[2 * l][i] + q[2 * l + 1][i];
#pragma unroll
                for (int l = 0; l < 4; l++) t4[l] = t8[2 * l] + t8[2 * l + 1];
                const float v = (t4[0] + t4[1]) + (t4[2] + t4[3]);
                const uint32_t row = row0 + 4 * g + i, t = t0 + c16;
                if (row < N && t < T) y[(uint64_t)t * N + row] = v;
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float t8[8], t4[4];
#pragma unroll
            for (int l = 0; l < 8; l++) t8[l] = p[2 * l][i] + p[2 * l + 1][i];
#pragma unroll
            for (int l = 0; l < 4; l++) t4[l] = t8[2 * l] + t8[2 * l + 1];
            const float v = (t4[0] + t4[1]) + (t4[2] + t4[3]);
            const uint32_t row = row0 + 4 * g + i, t = t0 + c16;
            if (row < N && t < T) y[(uint64_t)t * N + row] = v;
        }
    }
}

template <int RT, int TT, int KS, int S>
int mma_launch(uint32_t N, uint32_t nb, uint32_t T, const void* W, const void* ws, uint32_t dx_off, float* y,
               hipStream_t s) {
    using L = MmaLayout<RT, TT, KS>;
    const uint64_t ring = (uint64_t)S * L::kStageBytes;
    const uint64_t exch = KS > 1 ? (uint64_t)RT * TT * 16 * 64 * 16 : 0;
    const uint32_t lds = (uint32_t)((ring > exch ? ring : exch) + 1024 * L::kNw);
    if (lds > kLdsLimit) return -1;
    auto fn = k_q8_0_mma<RT, TT, KS, S>;
    static StreamLaunchCache cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return ANE_ERR_HIP;
    const int occ = stream_occupancy(cache, reinterpret_cast<const void*>(fn), dev, L::kNw * 64, lds);
    if (occ < 0) return occ;
    const uint32_t rtiles = (N + 15) / 16, ttiles = (T + 15) / 16;
    const uint64_t grid = (uint64_t)((rtiles + RT - 1) / RT) * ((ttiles + TT - 1) / TT);
    hipLaunchKernelGGL(fn, dim3((uint32_t)grid), dim3(L::kNw * 64), lds, s, N, nb, T, (const uint8_t*)W,
                       (const uint8_t*)ws, dx_off, ttiles, y);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

// ====================================================== MFMA mul_mat, token-stationary
// G mode for 5+ tokens.  The same per-block arithmetic as k_q8_0_mma, with
// the MFMA operands swapped: A = 16 tokens' quantized activations, B = 16
// weight rows, so lane (g, c16) receives tokens 4g..4g+3 of a token tile for
// weight row c16.  A lane then converts its row's fp16 d_w once per block
// for all the token tiles it covers, and reads the four tokens' fp32 d_x
// with one 16-byte LDS read (the activation scales are block-major in the
// workspace: dx[b][t], t < ceil(T, 4)).
//
// A workgroup covers RT row tiles x TT token tiles with RT x KS waves; wave
// (rt, ks) computes row tile rt for every token tile of the workgroup, over
// the residues ks*16/KS .. (ks+1)*16/KS - 1 of each 16-block stage, so the
// weights of a stage are read from LDS once per wave and the activations
// once per row tile.  Each wave folds its residues with the lower levels of
// the FADDV tree (its residues are a contiguous, aligned quarter/half/...
// of the 16 leaves); the KS subtotals meet in LDS for the top levels.
constexpr uint32_t kMmtXRowChunks = kMmaSb * 2 + 1;  // 32 + 1 pad: token rows 4 banks apart

template <int RT, int TT, int KS>
struct MmtLayout {
    static constexpr int kNw = RT * KS;
    static constexpr uint32_t kTok = TT * 16;
    static constexpr uint32_t kWChunks = RT * 16 * kMmaWRowChunks;
    static constexpr uint32_t kXChunks = kTok * kMmtXRowChunks;
    static constexpr uint32_t kDChunks = kMmaSb * kTok / 4;
    static constexpr uint32_t kWInstr = (kWChunks + 63) / 64, kXInstr = (kXChunks + 63) / 64,
                              kDInstr = (kDChunks + 63) / 64;
    static constexpr uint32_t kWSlots = (kWInstr + kNw - 1) / kNw, kXSlots = (kXInstr + kNw - 1) / kNw,
                              kDSlots = (kDInstr + kNw - 1) / kNw;
    static constexpr uint32_t kSlots = kWSlots + kXSlots + kDSlots;
    static constexpr uint32_t kXOff = kWChunks * 16, kDOff = kXOff + kXChunks * 16;
    static constexpr uint32_t kStageBytes = kDOff + kDChunks * 16;
};

// Pairwise tree over n adjacent values, in place (a[0] is the result):
// ((a0+a1)+(a2+a3)) + ... exactly as the FADDV tree's levels.
template <int n>
__device__ __forceinline__ float tree_sum(float (&a)[n]) {
#pragma unroll
    for (int w = 1; w < n; w *= 2)
#pragma unroll
        for (int i = 0; i + w < n; i += 2 * w) a[i] = a[i] + a[i + w];
    return a[0];
}

template <int RT, int TT, int KS, int S>
__global__ void __launch_bounds__(RT * KS * 64)
k_q8_0_mmt(uint32_t N, uint32_t nb, uint32_t T, const uint8_t* __restrict__ W, const uint8_t* __restrict__ qws,
           uint32_t dx_off, uint32_t T4, uint32_t n_tgroups, float* __restrict__ y) {
    using L = MmtLayout<RT, TT, KS>;
    constexpr int NW = L::kNw;
    constexpr uint32_t kSbw = kMmaSb / KS;  // residues per wave
    static_assert(kMmaSb % KS == 0, "KS divides the 16 residues");
    static_assert((S - 1) * L::kSlots < 64, "copies in flight exceed the vmcnt range");
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    int8_t* trash = smem + S * L::kStageBytes;  // 1 KB, the target of padding copies
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
    const uint32_t ks = wave % KS, rt = wave / KS;

    const uint32_t wg_t = blockIdx.x % n_tgroups, wg_r = blockIdx.x / n_tgroups;
    const uint32_t row_base = wg_r * RT * 16, tok_base = wg_t * L::kTok;
    const uint32_t rb = nb * 34;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(W, N * rb);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(qws, dx_off + nb * T4 * 4);
    const uint32_t nst = nb / kMmaSb;

    uint32_t ow[L::kWSlots], ox[L::kXSlots], od[L::kDSlots];
#pragma unroll
    for (uint32_t q = 0; q < L::kWSlots; q++) {
        const uint32_t c = 64 * (q * NW + wave) + lane, r = c / kMmaWRowChunks, sub = c - r * kMmaWRowChunks;
        const uint32_t row = row_base + r;
        ow[q] = (c < L::kWChunks && sub < kMmaSb * 17 / 8 && row < N) ? row * rb + 16 * sub : 0x80000000u;
    }
#pragma unroll
    for (uint32_t q = 0; q < L::kXSlots; q++) {
        const uint32_t c = 64 * (q * NW + wave) + lane, t = c / kMmtXRowChunks, sub = c - t * kMmtXRowChunks;
        const uint32_t tok = tok_base + t;
        ox[q] = (c < L::kXChunks && sub < 2 * kMmaSb && tok < T) ? tok * nb * 32 + 16 * sub : 0x80000000u;
    }
#pragma unroll
    for (uint32_t q = 0; q < L::kDSlots; q++) {
        // chunk c: block c / (kTok/4) of the stage, tokens 4*(c % (kTok/4)) ..
        const uint32_t c = 64 * (q * NW + wave) + lane, b = c / (L::kTok / 4), t4 = c - b * (L::kTok / 4);
        const uint32_t tok = tok_base + 4 * t4;
        od[q] = (c < L::kDChunks && tok < T4) ? dx_off + (b * T4 + tok) * 4 : 0x80000000u;
    }
    auto slot = [&](__amdgpu_buffer_rsrc_t r, int8_t* region, uint32_t ninstr, uint32_t nchunks, uint32_t q,
                    uint32_t src) {
        const uint32_t i = q * NW + wave;
        if (i < ninstr) {
            if (nchunks % 64 == 0 || i + 1 < ninstr || lane < nchunks % 64) copy16_to_lds(r, region + 1024 * i, src);
        } else if (S > 2) {  // padding that keeps vmcnt counts uniform (none with two stages)
            copy16_to_lds(r, trash, 0x80000000u);
        }
    };
    auto issue = [&](uint32_t s) {
        int8_t* st = smem + (s % S) * L::kStageBytes;
        const bool on = s < nst;
#pragma unroll
        for (uint32_t q = 0; q < L::kWSlots; q++)
            slot(wr, st, L::kWInstr, L::kWChunks, q,
                 on && ow[q] != 0x80000000u ? ow[q] + s * (kMmaSb * 34) : 0x80000000u);
#pragma unroll
        for (uint32_t q = 0; q < L::kXSlots; q++)
            slot(xr, st + L::kXOff, L::kXInstr, L::kXChunks, q,
                 on && ox[q] != 0x80000000u ? ox[q] + s * (kMmaSb * 32) : 0x80000000u);
#pragma unroll
        for (uint32_t q = 0; q < L::kDSlots; q++)
            slot(xr, st + L::kDOff, L::kDInstr, L::kDChunks, q,
                 on && od[q] != 0x80000000u ? od[q] + s * (kMmaSb * T4 * 4) : 0x80000000u);
    };

    float p[kSbw][TT][4];
#pragma unroll
    for (uint32_t j = 0; j < kSbw; j++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++)
#pragma unroll
            for (int i = 0; i < 4; i++) p[j][tt][i] = 0.0f;
#pragma unroll
    for (int s = 0; s < S - 1; s++) issue(s);
    for (uint32_t s = 0; s < nst; s++) {
        wait_vmcnt<(S - 2) * L::kSlots>();  // this wave's copies of stage s have landed
        __builtin_amdgcn_s_barrier();       // everyone's have; everyone is done with stage s-1
        issue(s + S - 1);                    // refills the slot of stage s-1
        const int8_t* st = smem + (s % S) * L::kStageBytes;
        const int8_t* wrow = st + (rt * 16 + c16) * (kMmaWRowChunks * 16);      // B: weight row c16
        const int8_t* xt = st + L::kXOff + c16 * (kMmtXRowChunks * 16) + 8 * g;  // A: token c16 of a tile
        const float* dd = reinterpret_cast<const float*>(st + L::kDOff) + 4 * g;  // d_x of tokens 4g..4g+3
#pragma unroll
        for (uint32_t j = 0; j < kSbw; j++) {
            const uint32_t bb = ks * kSbw + j;  // block of the stage; b % 16 == bb
            const uint32_t o = 34 * bb + 2 + 8 * g;
            const uint32_t* a32 = reinterpret_cast<const uint32_t*>(wrow + (o & ~3u));
            uint32_t w0, w1;
            if (bb & 1) {  // 34bb + 2 is 4-byte aligned for odd bb
                w0 = a32[0];
                w1 = a32[1];
                // two loads, not one fused 64-bit load without alias information
                // (before which the compiler would wait for every copy to LDS)
                asm("" : "+v"(w0));
            } else {
                const uint32_t d0 = a32[0], d1 = a32[1], d2 = a32[2];
                w0 = __builtin_amdgcn_alignbyte(d1, d0, 2);
                w1 = __builtin_amdgcn_alignbyte(d2, d1, 2);
            }
            const uint64_t wv = (uint64_t)w0 | ((uint64_t)w1 << 32);
            const float dw = half_bits_to_float(*reinterpret_cast<const uint16_t*>(wrow + 34 * bb));
            float4 d4s[TT];  // d_x of every token tile: 64 bytes apart
            lds_load_settled_f4x<TT>(dd + bb * L::kTok, d4s);
#pragma unroll
            for (int tt = 0; tt < TT; tt++) {
                const uint64_t xv =
                    *reinterpret_cast<const uint64_t*>(xt + tt * 16 * (kMmtXRowChunks * 16) + 32 * bb);
                const v4i acc = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)xv, (long)wv, v4i{0, 0, 0, 0}, 0, 0, 0);
                const float4 d4 = d4s[tt];
                const float dx[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                for (int i = 0; i < 4; i++)  // token 4g + i of tile tt, weight row c16
                    p[j][tt][i] = __builtin_fmaf((float)acc[i], __fmul_rn(dw, dx[i]), p[j][tt][i]);
            }
        }
    }
    wait_vmcnt<0>();
    // this wave's subtree of the FADDV tree
    float v[TT][4];
#pragma unroll
    for (int tt = 0; tt < TT; tt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float a[kSbw];
#pragma unroll
            for (uint32_t j = 0; j < kSbw; j++) a[j] = p[j][tt][i];
            v[tt][i] = tree_sum(a);
        }
    const uint32_t row = row_base + rt * 16 + c16;
    if (KS == 1) {
#pragma unroll
        for (int tt = 0; tt < TT; tt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t t = tok_base + tt * 16 + 4 * g + i;
                if (row < N && t < T) y[(uint64_t)t * N + row] = v[tt][i];
            }
    } else {
        // subtotals [rt][tt][ks][lane] over the ring; the top levels of the
        // tree for token tile tt are taken by wave (rt, tt % KS)
        __syncthreads();
        float4* ex = reinterpret_cast<float4*>(smem);
#pragma unroll
        for (int tt = 0; tt < TT; tt++)
            ex[((rt * TT + tt) * KS + ks) * 64 + lane] = make_float4(v[tt][0], v[tt][1], v[tt][2], v[tt][3]);
        __syncthreads();
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            if ((uint32_t)(tt % KS) != ks) continue;
            float q[4][KS];
#pragma unroll
            for (int k = 0; k < KS; k++) {
                const float4 e = ex[((rt * TT + tt) * KS + k) * 64 + lane];
                q[0][k] = e.x;
                q[1][k] = e.y;
                q[2][k] = e.z;
                q[3][k] = e.w;
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float r = tree_sum(q[i]);
                const uint32_t t = tok_base + tt * 16 + 4 * g + i;
                if (row < N && t < T) y[(uint64_t)t * N + row] = r;
            }
        }
    }
}

// Activation quantizer for k_q8_0_mmt: qx [T][nb][32] at xq, the scales
// block-major dx[b * T4 + t] at xq + dx_off.  The same arithmetic as
// k_q8_act_quantize (8 lanes per block).
__global__ void __launch_bounds__(256)
k_q8_act_quantize_bm(uint32_t nblocks, uint32_t nb, uint32_t K, uint32_t T4, uint32_t dx_off,
                     const float* __restrict__ x, uint8_t* __restrict__ xq) {
    const uint32_t t = blockIdx.x * 256 + threadIdx.x, blk = t >> 3, part = t & 7;
    const uint32_t tok = blk / nb, b = blk - tok * nb;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(x, (nblocks / nb) * K * 4);
    const uint32_t o = blk < nblocks ? (tok * K + b * 32 + part * 4) * 4 : 0x80000000u;
    float f[4];
#pragma unroll
    for (int e = 0; e < 4; e++) f[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, o + 4 * e, 0, 0));
    const uint32_t m = max8_u32(max(max(abs_key(f[0]), abs_key(f[1])), max(abs_key(f[2]), abs_key(f[3]))));
    float scale, inv;
    quant_params(__uint_as_float(m), scale, inv);
    if (blk < nblocks) {
        reinterpret_cast<uint32_t*>(xq)[blk * 8 + part] = pack4(f[0], f[1], f[2], f[3], inv);
        if (part == 0) reinterpret_cast<float*>(xq + dx_off)[b * T4 + tok] = scale;
    }
}

template <int RT, int TT, int KS, int S>
int mmt_launch(uint32_t N, uint32_t nb, uint32_t T, const void* W, const void* ws, uint32_t dx_off, uint32_t T4,
               float* y, hipStream_t s) {
    using L = MmtLayout<RT, TT, KS>;
    const uint64_t ring = (uint64_t)S * L::kStageBytes;
    const uint64_t exch = KS > 1 ? (uint64_t)RT * TT * KS * 64 * 16 : 0;
    const uint32_t lds = (uint32_t)((ring > exch ? ring : exch) + 1024);
    if (lds > kLdsLimit) return -1;
    auto fn = k_q8_0_mmt<RT, TT, KS, S>;
    static StreamLaunchCache cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return ANE_ERR_HIP;
    const int occ = stream_occupancy(cache, reinterpret_cast<const void*>(fn), dev, L::kNw * 64, lds);
    if (occ < 0) return occ;
    const uint32_t rtiles = (N + 15) / 16, tgroups = (T + L::kTok - 1) / L::kTok;
    const uint64_t grid = (uint64_t)((rtiles + RT - 1) / RT) * tgroups;
    hipLaunchKernelGGL(fn, dim3((uint32_t)grid), dim3(L::kNw * 64), lds, s, N, nb, T, (const uint8_t*)W,
                       (const uint8_t*)ws, dx_off, T4, tgroups, y);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

// ====================================================== MFMA mul_mat, residue-split workgroups
// Token-stationary like k_q8_0_mmt (lane (g, c16) computes weight row c16
// for tokens 4g..4g+3 of a token tile), for matrices with few rows: the 16
// residues b % 16 of the blocks are split over KW = 16 / NR workgroups.
// Workgroup q of a row group takes residues NR*q .. NR*q + NR - 1, which are
// NR consecutive blocks of every 16-block group, so it copies only those
// bytes of its rows' weights and of the activations; it has one wave per
// (row tile, residue), and each wave's chain runs over its residue's blocks
// in order.  The NR leaves of a row tile meet in LDS for the lower levels
// of the FADDV tree (an aligned NR-leaf subtree); the KW subtotals meet in
// k_q8_0_mmr_reduce for the top levels.  A 4096-row matrix then keeps every
// CU busy with its weights read once and the activations copied once per
// 64 rows (k_q8_0_mma copies them once per 16 rows, k_q8_0_mmt has too few
// workgroups there).
//
// Stage s holds G 16-block groups.  Per group, a weight row contributes
// kWGroupChunks 16-byte chunks starting at chunk floor(34*NR*q / 16) of the
// group (the window's 34*NR bytes start o0 = 0 or 8 bytes in); a token
// contributes the 2*NR chunks of its qx blocks; the scales are block-major
// dx[b][t] (k_q8_act_quantize_bm), NR*G runs of the workgroup's tokens.
template <int RT, int TT, int NR, int G>
struct MmrLayout {
    static constexpr int kNw = RT * NR;
    static constexpr uint32_t kTok = TT * 16;
    static constexpr uint32_t kWGroupChunks = (8 + 34 * NR + 15) / 16;
    // row strides of 12 (weights) and 4 (tokens) dwords mod 64, as in k_q8_0_mmt
    static constexpr uint32_t kWRowChunks = G * kWGroupChunks + (3 + 16 - (G * kWGroupChunks) % 16) % 16;
    static constexpr uint32_t kXGroupChunks = 2 * NR;
    static constexpr uint32_t kXRowChunks = G * kXGroupChunks + (1 + 16 - (G * kXGroupChunks) % 16) % 16;
    static constexpr uint32_t kWChunks = RT * 16 * kWRowChunks;
    static constexpr uint32_t kXChunks = kTok * kXRowChunks;
    static constexpr uint32_t kDChunks = G * NR * kTok / 4;
    static constexpr uint32_t kWInstr = (kWChunks + 63) / 64, kXInstr = (kXChunks + 63) / 64,
                              kDInstr = (kDChunks + 63) / 64;
    static constexpr uint32_t kWSlots = (kWInstr + kNw - 1) / kNw, kXSlots = (kXInstr + kNw - 1) / kNw,
                              kDSlots = (kDInstr + kNw - 1) / kNw;
    static constexpr uint32_t kSlots = kWSlots + kXSlots + kDSlots;
    static constexpr uint32_t kXOff = kWChunks * 16, kDOff = kXOff + kXChunks * 16;
    static constexpr uint32_t kStageBytes = kDOff + kDChunks * 16;
    static_assert((kWRowChunks * 4) % 64 == 12 && (kXRowChunks * 4) % 64 == 4, "row strides");
};

template <int RT, int TT, int NR, int G, int S>
__global__ void __launch_bounds__(RT * NR * 64)
k_q8_0_mmr(uint32_t N, uint32_t nb, uint32_t T, const uint8_t* __restrict__ W, const uint8_t* __restrict__ qws,
           uint32_t dx_off, uint32_t T4, uint32_t n_tgroups, uint32_t n_units, float* __restrict__ out) {
    using L = MmrLayout<RT, TT, NR, G>;
    constexpr int NW = L::kNw;
    constexpr uint32_t KW = 16 / NR;
    static_assert(16 % NR == 0 && NR >= 2, "NR divides the 16 residues");
    static_assert((S - 1) * L::kSlots < 64, "copies in flight exceed the vmcnt range");
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    int8_t* trash = smem + S * L::kStageBytes;  // 1 KB, the target of padding copies
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
    const uint32_t r = wave % NR, rt = wave / NR;

    // Workgroups go to the 8 XCDs round-robin; the KW windows of one unit
    // (row group x token group) are consecutive slots of one XCD, so the
    // cache lines that two windows share are fetched into one L2.  The grid
    // is KW x the units rounded up to a multiple of 8; the surplus exits.
    const uint32_t xcd = blockIdx.x & 7, xslot = blockIdx.x >> 3;
    const uint32_t wq = xslot % KW, unit = xcd + 8 * (xslot / KW);
    if (unit >= n_units) return;
    const uint32_t wg_t = unit % n_tgroups, wg_r = unit / n_tgroups;
    const uint32_t row_base = wg_r * RT * 16, tok_base = wg_t * L::kTok;
    const uint32_t rb = nb * 34;
    const uint32_t c0 = (34 * NR * wq) / 16, o0 = 34 * NR * wq - 16 * c0;  // window start: chunk, byte
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(W, N * rb);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(qws, dx_off + nb * T4 * 4);
    const uint32_t nst = nb / (16 * G);

    uint32_t ow[L::kWSlots], ox[L::kXSlots], od[L::kDSlots];
#pragma unroll
    for (uint32_t q = 0; q < L::kWSlots; q++) {
        const uint32_t c = 64 * (q * NW + wave) + lane, rr = c / L::kWRowChunks, sub = c - rr * L::kWRowChunks;
        const uint32_t gi = sub / L::kWGroupChunks, cc = sub - gi * L::kWGroupChunks;
        const uint32_t row = row_base + rr;
        ow[q] = (c < L::kWChunks && gi < (uint32_t)G && row < N) ? row * rb + gi * 544 + 16 * (c0 + cc)
                                                                   : 0x80000000u;
    }
#pragma unroll
    for (uint32_t q = 0; q < L::kXSlots; q++) {
        const uint32_t c = 64 * (q * NW + wave) + lane, t = c / L::kXRowChunks, sub = c - t * L::kXRowChunks;
        const uint32_t gi = sub / L::kXGroupChunks, cc = sub - gi * L::kXGroupChunks;
        const uint32_t tok = tok_base + t;
        ox[q] = (c < L::kXChunks && gi < (uint32_t)G && tok < T)
                    ? tok * nb * 32 + gi * 512 + 32 * NR * wq + 16 * cc
                    : 0x80000000u;
    }
#pragma unroll
    for (uint32_t q = 0; q < L::kDSlots; q++) {
        // chunk c: group gi, residue rr of the window, tokens 4*t4 .. of the workgroup
        const uint32_t c = 64 * (q * NW + wave) + lane, gi = c / (NR * L::kTok / 4);
        const uint32_t rem = c - gi * (NR * L::kTok / 4), rr = rem / (L::kTok / 4), t4 = rem - rr * (L::kTok / 4);
        const uint32_t tok = tok_base + 4 * t4, b = 16 * gi + NR * wq + rr;
        od[q] = (c < L::kDChunks && tok < T4) ? dx_off + (b * T4 + tok) * 4 : 0x80000000u;
    }
    auto slot = [&](__amdgpu_buffer_rsrc_t rs, int8_t* region, uint32_t ninstr, uint32_t nchunks, uint32_t q,
                    uint32_t src) {
        const uint32_t i = q * NW + wave;
        if (i < ninstr) {
            if (nchunks % 64 == 0 || i + 1 < ninstr || lane < nchunks % 64) copy16_to_lds(rs, region + 1024 * i, src);
        } else if (S > 2) {  // padding that keeps vmcnt counts uniform (none with two stages)
            copy16_to_lds(rs, trash, 0x80000000u);
        }
    };
    auto issue = [&](uint32_t s) {
        int8_t* st = smem + (s % S) * L::kStageBytes;
        const bool on = s < nst;
#pragma unroll
        for (uint32_t q = 0; q < L::kWSlots; q++)
            slot(wr, st, L::kWInstr, L::kWChunks, q,
                 on && ow[q] != 0x80000000u ? ow[q] + s * (G * 544) : 0x80000000u);
#pragma unroll
        for (uint32_t q = 0; q < L::kXSlots; q++)
            slot(xr, st + L::kXOff, L::kXInstr, L::kXChunks, q,
                 on && ox[q] != 0x80000000u ? ox[q] + s * (G * 512) : 0x80000000u);
#pragma unroll
        for (uint32_t q = 0; q < L::kDSlots; q++)
            slot(xr, st + L::kDOff, L::kDInstr, L::kDChunks, q,
                 on && od[q] != 0x80000000u ? od[q] + s * (16 * G * T4 * 4) : 0x80000000u);
    };

    float p[TT][4];
#pragma unroll
    for (int tt = 0; tt < TT; tt++)
#pragma unroll
        for (int i = 0; i < 4; i++) p[tt][i] = 0.0f;
    // this wave's block inside a group's window, and whether its quants are 4-byte aligned
    const uint32_t bofs = o0 + 34 * r;
    const bool odd = ((bofs + 2) & 3) == 0;
#pragma unroll
    for (int s = 0; s < S - 1; s++) issue(s);
    for (uint32_t s = 0; s < nst; s++) {
        wait_vmcnt<(S - 2) * L::kSlots>();  // this wave's copies of stage s have landed
        __builtin_amdgcn_s_barrier();       // everyone's have; everyone is done with stage s-1
        issue(s + S - 1);                    // refills the slot of stage s-1
        const int8_t* st = smem + (s % S) * L::kStageBytes;
        const int8_t* wrow = st + (rt * 16 + c16) * (L::kWRowChunks * 16) + bofs;       // B: weight row c16
        const int8_t* xt = st + L::kXOff + c16 * (L::kXRowChunks * 16) + 32 * r + 8 * g;  // A: token c16
        const float* dd = reinterpret_cast<const float*>(st + L::kDOff) + r * L::kTok + 4 * g;
#pragma unroll
        for (int gi = 0; gi < G; gi++) {
            const int8_t* wb = wrow + gi * (L::kWGroupChunks * 16);
            const uint32_t o = 2 + 8 * g;
            uint32_t w0, w1;
            if (odd) {
                const uint32_t* a32 = reinterpret_cast<const uint32_t*>(wb + o);
                w0 = a32[0];
                w1 = a32[1];
            } else {
                const uint32_t* a32 = reinterpret_cast<const uint32_t*>(wb + o - 2);
                const uint32_t d0 = a32[0], d1 = a32[1], d2 = a32[2];
                w0 = __builtin_amdgcn_alignbyte(d1, d0, 2);
                w1 = __builtin_amdgcn_alignbyte(d2, d1, 2);
            }
            const uint64_t wv = (uint64_t)w0 | ((uint64_t)w1 << 32);
            const float dw = half_bits_to_float(*reinterpret_cast<const uint16_t*>(wb));
            float4 d4s[TT];  // d_x of every token tile: 64 bytes apart
            lds_load_settled_f4x<TT>(dd + gi * (NR * L::kTok), d4s);
#pragma unroll
            for (int tt = 0; tt < TT; tt++) {
                const uint64_t xv = *reinterpret_cast<const uint64_t*>(
                    xt + tt * 16 * (L::kXRowChunks * 16) + gi * (L::kXGroupChunks * 16));
                const v4i acc = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)xv, (long)wv, v4i{0, 0, 0, 0}, 0, 0, 0);
                const float4 d4 = d4s[tt];
                const float dx[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                for (int i = 0; i < 4; i++)  // token 4g + i of tile tt, weight row c16
                    p[tt][i] = __builtin_fmaf((float)acc[i], __fmul_rn(dw, dx[i]), p[tt][i]);
            }
        }
    }
    wait_vmcnt<0>();
    // leaves [rt][tt][r][lane] over the ring; wave (rt, tt % NR) takes the
    // subtree of token tile tt
    __syncthreads();
    float4* ex = reinterpret_cast<float4*>(smem);
#pragma unroll
    for (int tt = 0; tt < TT; tt++)
        ex[((rt * TT + tt) * NR + r) * 64 + lane] = make_float4(p[tt][0], p[tt][1], p[tt][2], p[tt][3]);
    __syncthreads();
    const uint32_t row = row_base + rt * 16 + c16;
#pragma unroll
    for (int tt = 0; tt < TT; tt++) {
        if ((uint32_t)(tt % NR) != r) continue;
        float q[4][NR];
#pragma unroll
        for (int k = 0; k < NR; k++) {
            const float4 e = ex[((rt * TT + tt) * NR + k) * 64 + lane];
            q[0][k] = e.x;
            q[1][k] = e.y;
            q[2][k] = e.z;
            q[3][k] = e.w;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float v = tree_sum(q[i]);
            const uint32_t t = tok_base + tt * 16 + 4 * g + i;
            // subtotal wq of y[t][row]: out[(wq * T + t) * N + row]
            if (row < N && t < T) out[((uint64_t)wq * T + t) * N + row] = v;
        }
    }
}

// y[t][row] = the top KW levels of the FADDV tree over the KW subtotals,
// four outputs per thread (16-byte loads and stores where n % 4 == 0 and y
// is 16-byte aligned; one output per lane step otherwise).
template <int KW>
__global__ void __launch_bounds__(256)
k_q8_0_mmr_reduce(uint64_t n, const float* __restrict__ part, float* __restrict__ y) {
    const uint64_t i4 = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i4 >= n) return;
    if ((n & 3) == 0 && (((uintptr_t)y) & 15) == 0) {
        float4 a[KW];
#pragma unroll
        for (int k = 0; k < KW; k++) a[k] = *reinterpret_cast<const float4*>(part + k * n + i4);
        float c[4][KW];
#pragma unroll
        for (int k = 0; k < KW; k++) {
            c[0][k] = a[k].x;
            c[1][k] = a[k].y;
            c[2][k] = a[k].z;
            c[3][k] = a[k].w;
        }
        const float4 v = make_float4(tree_sum(c[0]), tree_sum(c[1]), tree_sum(c[2]), tree_sum(c[3]));
        *reinterpret_cast<float4*>(y + i4) = v;
        return;
    }
    for (uint64_t i = i4; i < i4 + 4 && i < n; i++) {
        float a[KW];
#pragma unroll
        for (int k = 0; k < KW; k++) a[k] = part[k * n + i];
        y[i] = tree_sum(a);
    }
}

template <int RT, int TT, int NR, int G, int S>
int mmr_launch(uint32_t N, uint32_t nb, uint32_t T, const void* W, const void* ws, uint32_t dx_off, uint32_t T4,
               float* part, float* y, hipStream_t s) {
    using L = MmrLayout<RT, TT, NR, G>;
    constexpr uint32_t KW = 16 / NR;
    if (nb % (16 * G)) return -1;
    const uint64_t ring = (uint64_t)S * L::kStageBytes;
    const uint64_t exch = (uint64_t)RT * TT * NR * 64 * 16;
    const uint32_t lds = (uint32_t)((ring > exch ? ring : exch) + 1024);
    if (lds > kLdsLimit) return -1;
    auto fn = k_q8_0_mmr<RT, TT, NR, G, S>;
    static StreamLaunchCache cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return ANE_ERR_HIP;
    const int occ = stream_occupancy(cache, reinterpret_cast<const void*>(fn), dev, L::kNw * 64, lds);
    if (occ < 0) return occ;
    const uint32_t rgroups = (N + RT * 16 - 1) / (RT * 16), tgroups = (T + L::kTok - 1) / L::kTok;
    const uint64_t units = (uint64_t)rgroups * tgroups;
    const uint64_t grid = KW * ceil_to(units, 8);
    if (grid > 0x7fffffffull) return -1;
    hipLaunchKernelGGL(fn, dim3((uint32_t)grid), dim3(L::kNw * 64), lds, s, N, nb, T, (const uint8_t*)W,
                       (const uint8_t*)ws, dx_off, T4, tgroups, (uint32_t)units, part);
    ANE_HIP_CHECK_LAUNCH();
    const uint64_t n = (uint64_t)T * N;
    hipLaunchKernelGGL(k_q8_0_mmr_reduce<KW>, dim3((uint32_t)((n + 1023) / 1024)), dim3(256), 0, s, n, part, y);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

// The MFMA path: rows 16-byte aligned (as the streaming kernels need) and
// whole 16-block stages.  x is quantized into the workspace first.
//
// Kernel choice, measured on the config-4 projections (6144/4096/28672/4096
// rows, K 4096/14336) at T = 16, 32, 64:
//  * k_q8_0_mmt (d_w converted once per block for all of a wave's token
//    tiles) from four row tiles per CU up at any token count (gate_up
//    28672x4096: T = 64 104 -> 64 us on 4x4 tiles, T = 32 58 -> 48 us and
//    T = 16 35.9 -> 34.1 us on 2-row-tile workgroups), and from more than one
//    row tile per CU at 3+ token tiles (qkv T = 64: 30 -> 21.7 us, two token
//    groups of 2x2 tiles);
//  * k_q8_0_mma otherwise (at most one row tile per CU, where its split-K
//    over residues keeps 16+ waves per CU).
//  * k_q8_0_mmr (the residue windows of a 64-row group split over four
//    workgroups) for matrices with fewer rows, when the workspace holds its
//    subtotals (ane_hip_q8_0_mul_mat_workspace_size_n).
// Offset of k_q8_0_mmr's subtotals in the workspace: after the activation
// form with block-major scales.
uint64_t mmr_part_off(uint32_t nb, uint32_t T) {
    const uint64_t T4 = ((uint64_t)T + 3) & ~3ull;
    return ceil_to(ceil_to((uint64_t)T * nb * 32, 256) + (uint64_t)nb * T4 * 4, 256);
}
constexpr uint32_t kMmrWindows = 4;  // workgroups per row group on the residue-split route
// ... taken from this many blocks per row: measured on config 4 (XCD-grouped
// windows), down 4096 x 14336 (448 blocks) T = 16 / 32 / 64: 30.9 / 37.3 /
// 42.0 -> 26.9 / 29.6 / 36.9 us; at 128 blocks (o, qkv) the four 32-block
// stages do not repay the subtotal pass (o T = 64 17.2 -> 18.3 us).
constexpr uint32_t kMmrMinBlocks = 256;

int mma_mul_mat(uint32_t N, uint32_t nb, uint32_t K, uint32_t T, const float* x, const void* W, float* y,
                void* workspace, size_t workspace_bytes, hipStream_t s) {
    {
        // 16+ tokens at K = 4096 or 14336: activations held in VGPRs (q8_0_mmv.hip)
        const int r = mmv_mul_mat(N, nb, K, T, x, W, y, workspace, workspace_bytes, s);
        if (r != -1) return r;
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return ANE_ERR_HIP;
    const uint64_t cus = cu_count(dev);
    const uint64_t dx_off = ceil_to((uint64_t)T * nb * 32, 256);
    const uint32_t dxo = (uint32_t)dx_off;
    const uint32_t nblocks = T * nb;
    const uint64_t rtiles = (N + 15) / 16;
    const uint32_t ttiles = (T + 15) / 16;
    const uint32_t T4 = (T + 3) & ~3u;
    const bool many = rtiles >= 4 * cus;
    const bool bm_ok = dx_off + (uint64_t)nb * T4 * 4 < 0x80000000ull;
    const uint64_t part_off = mmr_part_off(nb, T);
    const bool mmr = !many && bm_ok && nb % 32 == 0 && nb >= kMmrMinBlocks &&
                     part_off + (uint64_t)kMmrWindows * T * N * 4 <= workspace_bytes;
    const bool mmt = !mmr && (many || (ttiles > 2 && rtiles > cus)) && bm_ok;
    if (mmr || mmt) {
        // activation scales block-major: dx[b][t] at dx_off
        hipLaunchKernelGGL(k_q8_act_quantize_bm, dim3((nblocks * 8 + 255) / 256), dim3(256), 0, s, nblocks, nb, K,
                           T4, dxo, x, static_cast<uint8_t*>(workspace));
        ANE_HIP_CHECK_LAUNCH();
        int r;
        if (mmr) {
            float* part = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + part_off);
            if (ttiles == 1)
                r = mmr_launch<4, 1, 4, 2, 2>(N, nb, T, W, workspace, dxo, T4, part, y, s);
            else if (ttiles == 2)
                r = mmr_launch<4, 2, 4, 2, 2>(N, nb, T, W, workspace, dxo, T4, part, y, s);
            else
                r = mmr_launch<4, 4, 4, 2, 2>(N, nb, T, W, workspace, dxo, T4, part, y, s);
        } else if (ttiles == 1) {
            r = mmt_launch<2, 1, 4, 2>(N, nb, T, W, workspace, dxo, T4, y, s);
        } else if (ttiles == 2 || !many) {
            r = mmt_launch<2, 2, 4, 2>(N, nb, T, W, workspace, dxo, T4, y, s);
        } else {
            r = mmt_launch<4, 4, 4, 2>(N, nb, T, W, workspace, dxo, T4, y, s);
        }
        if (r != -1) return r;
        // not launched: the token-major form below overwrites the workspace
    }
    if (dx_off + (uint64_t)T * nb * 4 >= 0x80000000ull) return -1;
    // nb % 16 == 0 here, so dx_off == T*nb*32: the Q8 activation form
    hipLaunchKernelGGL(k_q8_act_quantize, dim3((nblocks * 8 + 255) / 256), dim3(256), 0, s, nblocks, nb, K, x,
                       static_cast<uint8_t*>(workspace));
    ANE_HIP_CHECK_LAUNCH();
    const uint64_t tiles = rtiles * ttiles;
    const bool few = tiles < 4 * cus;  // fewer than 4 tiles per CU
    // split-K over residues pays wherever it keeps a workgroup's LDS small
    // enough for 16+ waves per CU
    if (ttiles == 1)
        return few ? mma_launch<1, 1, 8, 2>(N, nb, T, W, workspace, dxo, y, s)
                   : mma_launch<2, 1, 4, 2>(N, nb, T, W, workspace, dxo, y, s);
    return mma_launch<1, 2, 4, 2>(N, nb, T, W, workspace, dxo, y, s);
}

// A K-quant GEMV on the streaming kernel: NW waves per workgroup, SB
// super-blocks per item, SBF per item for matrices with few rows (4-wave
// workgroups).  -1 when the rows are not 16-byte aligned or a partial
// segment is not whole 16-byte chunks, so the caller takes k_qgemv.
template <int MODE, int NW, int SB, int SBF = SB>
int qk_stream(uint32_t M, uint32_t K, const float* x, const void* W, float* y, hipStream_t s) {
    constexpr uint64_t BB = kBlockBytes<MODE>;
    const uint32_t nsb = K >> 8;
    if (nsb == 0 || (((uintptr_t)W) & 15)) return -1;
    if ((nsb * BB) % 16) return -1;
    if ((uint64_t)M * nsb * BB >= 0x80000000ull || (uint64_t)K * 4 >= 0x80000000ull) return -1;
    const bool seg_ok = ((nsb % SB) * BB) % 16 == 0, segf_ok = ((nsb % SBF) * BB) % 16 == 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return ANE_ERR_HIP;
    const uint64_t units = ((uint64_t)M + kUnitRows - 1) / kUnitRows;
    int r = -1;
    if (units < (uint64_t)cu_count(dev) * ANE_Q8_SMALL_UNITS_PER_CU && segf_ok)
        r = try_stream<MODE, 4, SBF, 2, 1>(M, nsb, K, 1, x, W, y, s);
    if (r < 0 && seg_ok) r = try_stream<MODE, NW, SB, 2, 1>(M, nsb, K, 1, x, W, y, s);
    if (r < 0 && seg_ok) r = try_stream<MODE, 4, SB, 2, 1>(M, nsb, K, 1, x, W, y, s);
    return r;
}

}  // namespace

// The K-quant GEMVs on the streaming kernel: fmt 1..4 = Q4_K, Q2_K, Q3_K,
// Q5_K.  -1 when the shape does not fit it.  Shapes as measured at
// 14336x4096 and 4096x14336 (8 super-blocks per item for 4096 rows: Q4_K
// 41.2 -> 38.9 us, Q5_K 46.0 -> 41.7; and for Q2_K at any size: 18.2 ->
// 16.6, 27.7 -> 23.9); Q6_K (210-byte super-blocks, so 8 per item and
// 6.9 KB stages) measured slower here than on k_qgemv and stays there.
int qk_stream_gemv(int fmt, uint32_t M, uint32_t K, const float* x, const void* W, float* y, hipStream_t s) {
    switch (fmt) {
        case 1: return qk_stream<kModeQ4K, 4, 4, 8>(M, K, x, W, y, s);
        case 2: return qk_stream<kModeQ2K, 8, 8, 8>(M, K, x, W, y, s);
        case 3: return qk_stream<kModeQ3K, 8, 8>(M, K, x, W, y, s);
        case 4: return qk_stream<kModeQ5K, 4, 4, 8>(M, K, x, W, y, s);
    }
    return -1;
}

// q4_0_gemv on the streaming kernel (kModeR4) when the rows are 16-byte
// aligned (K/32 a multiple of 8, W 16-byte aligned); -1 when they are not
// or no configuration fits, so the caller takes the general kernel.
int q4_0_stream_gemv(uint32_t M, uint32_t K, const float* x, const void* W, float* y, hipStream_t s) {
    const uint32_t nb = K >> 5;
    if (!stream_eligible(M, nb, K, 1, W, 18)) return -1;
    return stream_auto<kModeR4, 1>(M, nb, K, 1, x, W, y, s);
}

}  // namespace ane

using namespace ane;

extern "C" int ane_hip_q8_0_gemv(uint32_t M, uint32_t K, const float* x, const void* W, float* y,
                                 void* stream) {
    if (M == 0) return ANE_OK;
    if (!y || ((K >> 5) && (!x || !W))) return ANE_ERR_BAD_POINTER;
    if ((((uintptr_t)W) & 1) != 0) return ANE_ERR_INVALID_ARG;
    const uint32_t nb = K >> 5;
    hipStream_t s = (hipStream_t)stream;
    if (stream_eligible(M, nb, K, 1, W)) {
        const int r = stream_auto<kModeR, 1>(M, nb, K, 1, x, W, y, s);
        if (r >= 0) return r;
    }
    const uint64_t grid = ((uint64_t)M + kRowsPerBlock - 1) / kRowsPerBlock;
    hipLaunchKernelGGL(k_q8_0_gemv_r, dim3((uint32_t)grid), dim3(256), 0, s, M, nb, x,
                       (const uint8_t*)W, y);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

extern "C" int ane_hip_q8_0_matvec_fused(uint32_t N, uint32_t K, const float* x, const float* norm_w,
                                         float eps, const void* W, const float* residual, float* y,
                                         void* stream) {
    if (N == 0) return ANE_OK;
    const uint32_t nb = K >> 5;
    if (!y || !x || !W || (K & 31)) return ANE_ERR_BAD_POINTER;
    if (!stream_eligible(N, nb, K, 1, W)) return ANE_ERR_INVALID_ARG;
    hipStream_t s = (hipStream_t)stream;
    const StreamFuse fz{norm_w, eps, residual};
    int r;
    if (norm_w && residual) r = stream_auto<kModeG, 1, kFuseNorm | kFuseResidual>(N, nb, K, 1, x, W, y, s, fz);
    else if (norm_w) r = stream_auto<kModeG, 1, kFuseNorm>(N, nb, K, 1, x, W, y, s, fz);
    else if (residual) r = stream_auto<kModeG, 1, kFuseResidual>(N, nb, K, 1, x, W, y, s, fz);
    else r = stream_auto<kModeG, 1>(N, nb, K, 1, x, W, y, s);
    return r < 0 ? ANE_ERR_INVALID_ARG : r;
}

extern "C" int ane_hip_q8_0_matvec_q8(uint32_t N, uint32_t K, const void* xq, const void* W,
                                      const float* residual, float* y, void* stream) {
    if (N == 0) return ANE_OK;
    const uint32_t nb = K >> 5;
    if (!y || !xq || !W || (K & 31)) return ANE_ERR_BAD_POINTER;
    if ((((uintptr_t)xq) & 15) || !stream_eligible(N, nb, K, 1, W)) return ANE_ERR_INVALID_ARG;
    hipStream_t s = (hipStream_t)stream;
    const float* xf = static_cast<const float*>(xq);
    const StreamFuse fz{nullptr, 0.0f, residual};
    const int r = residual ? stream_auto<kModeG, 1, kFusePreQuant | kFuseResidual>(N, nb, K, 1, xf, W, y, s, fz)
                           : stream_auto<kModeG, 1, kFusePreQuant>(N, nb, K, 1, xf, W, y, s, fz);
    return r < 0 ? ANE_ERR_INVALID_ARG : r;
}
extern "C" int ane_hip_q8_0_gate_up_silu_quant(uint32_t F, uint32_t K, const float* x, const float* norm_w,
                                               float eps, const void* W, void* xq, void* stream) {
    if (F == 0) return ANE_OK;
    const uint32_t nb = K >> 5, N = 2 * F;
    if (!x || !norm_w || !W || !xq || (K & 31)) return ANE_ERR_BAD_POINTER;
    if ((F & 31) || (((uintptr_t)xq) & 15) || !stream_eligible(N, nb, K, 1, W)) return ANE_ERR_INVALID_ARG;
    const int r = gate_up_silu_quant(N, nb, K, x, W, xq, (hipStream_t)stream, StreamFuse{norm_w, eps, nullptr});
    return r < 0 ? ANE_ERR_INVALID_ARG : r;
}
extern "C" int ane_hip_q8_0_matvec_silu(uint32_t N, uint32_t K, const float* gu, const void* W,
                                        const float* residual, float* y, void* stream) {
    if (N == 0) return ANE_OK;
    const uint32_t nb = K >> 5;
    if (!y || !gu || !W || (K & 31)) return ANE_ERR_BAD_POINTER;
    if (!stream_eligible(N, nb, K, 2, W)) return ANE_ERR_INVALID_ARG;
    hipStream_t s = (hipStream_t)stream;
    const StreamFuse fz{nullptr, 0.0f, residual};
    const int r = residual
        ? stream_auto<kModeG, 1, kFuseSiluMul | kFuseResidual>(N, nb, K, 1, gu, W, y, s, fz)
        : stream_auto<kModeG, 1, kFuseSiluMul>(N, nb, K, 1, gu, W, y, s, fz);
    return r < 0 ? ANE_ERR_INVALID_ARG : r;
}

// Single-token products quantize x inside the streaming kernel up to this
// many blocks (K = 8192); longer rows take the separate quantizer.
#ifndef ANE_Q8_INLINE_QUANT_BLOCKS
#define ANE_Q8_INLINE_QUANT_BLOCKS 256
#endif
constexpr uint32_t kQ8InlineQuantBlocks = ANE_Q8_INLINE_QUANT_BLOCKS;

extern "C" size_t ane_hip_q8_0_mul_mat_workspace_size(uint32_t K, uint32_t T) {
    const uint64_t nb = K >> 5;
    // qx, then the scales: token-major [T][nb] or block-major [nb][ceil(T, 4)];
    // for 2+ tokens, or the block-major form of ceil(T, 16) tokens (q8_0_mmv.hip)
    const uint64_t a = ceil_to((uint64_t)T * nb * 32, 256) + ceil_to(nb * (((uint64_t)T + 3) & ~3ull) * 4, 256) + 256;
    const uint64_t b = T >= 2 ? ceil_to(mmv_workspace_bound((uint32_t)nb, T), 256) : 0;
    return (size_t)(a > b ? a : b);
}

extern "C" size_t ane_hip_q8_0_mul_mat_workspace_size_n(uint32_t N, uint32_t K, uint32_t T) {
    const size_t base = ane_hip_q8_0_mul_mat_workspace_size(K, T);
    if (T <= kMaxStreamTokens) return base;
    const uint64_t with_part = mmr_part_off(K >> 5, T) + (uint64_t)kMmrWindows * T * N * 4;
    return with_part > base ? (size_t)with_part : base;
}

extern "C" int ane_hip_q8_0_mul_mat(uint32_t N, uint32_t K, uint32_t T, const float* x,
                                    const void* W, float* y, void* workspace,
                                    size_t workspace_bytes, void* stream) {
    if (N == 0 || T == 0) return ANE_OK;
    const uint32_t nb = K >> 5;
    if (!y || (nb && (!x || !W))) return ANE_ERR_BAD_POINTER;
    if ((((uintptr_t)W) & 1) != 0) return ANE_ERR_INVALID_ARG;
    if (!workspace || (((uintptr_t)workspace) & 255) ||
        workspace_bytes < ane_hip_q8_0_mul_mat_workspace_size(K, T))
        return ANE_ERR_WORKSPACE;
    hipStream_t s = (hipStream_t)stream;
    if (T >= 2 && T <= kMaxStreamTokens && nb % kMmaSb == 0 && stream_eligible(N, nb, K, T, W) &&
        mmv_fills_cus(N)) {
        // 2-4 tokens padded to one token tile of the activation-stationary kernel
        const int r = mmv_mul_mat(N, nb, K, T, x, W, y, workspace, workspace_bytes, s);
        if (r >= 0) return r;
    }
    if (T <= kMaxStreamTokens && stream_eligible(N, nb, K, T, W)) {
        int r;
        if (T == 1 && nb <= kQ8InlineQuantBlocks) {
            r = stream_auto<kModeG, 1>(N, nb, K, T, x, W, y, s);
        } else {
            // every workgroup would quantize all T*nb activation blocks: do it
            // once into the workspace (dx follows qx: nb % 8 == 0 here) and
            // copy the result into LDS
            const uint32_t nblocks = T * nb;
            hipLaunchKernelGGL(k_q8_act_quantize, dim3((nblocks * 8 + 255) / 256), dim3(256), 0, s, nblocks, nb,
                               K, x, static_cast<uint8_t*>(workspace));
            ANE_HIP_CHECK_LAUNCH();
            const float* xq = static_cast<const float*>(workspace);
            r = T == 1 ? stream_auto<kModeG, 1, kFusePreQuant>(N, nb, K, T, xq, W, y, s)
                       : stream_auto<kModeG, kMaxStreamTokens, kFusePreQuant>(N, nb, K, T, xq, W, y, s);
        }
        if (r >= 0) return r;
    }
    if (T > kMaxStreamTokens && nb % kMmaSb == 0 && stream_eligible(N, nb, K, T, W)) {
        const int r = mma_mul_mat(N, nb, K, T, x, W, y, workspace, workspace_bytes, s);
        if (r >= 0) return r;
    }
    int8_t* qx = (int8_t*)workspace;
    float* dx = (float*)((uint8_t*)workspace + ceil_to((uint64_t)T * nb * 32, 256));
    const uint64_t nblocks = (uint64_t)T * nb;
    if (nblocks) {
        hipLaunchKernelGGL(k_q8_0_quantize_x, dim3((uint32_t)((nblocks + 255) / 256)), dim3(256), 0,
                           s, nblocks, nb, K, x, qx, dx);
    }
    const uint64_t grid = ((uint64_t)N + kRowsPerBlock - 1) / kRowsPerBlock;
    hipLaunchKernelGGL(k_q8_0_mul_mat_g, dim3((uint32_t)grid), dim3(256), 0, s, N, nb, T, qx, dx,
                       (const uint8_t*)W, y);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

// ------------------------------------------- the no-allocation mul_mat
// ane_hip_q8_0_mul_mat_noalloc: the same product with its workspace (the
// quantized activations) in a file-scope device array instead of a caller
// buffer.  Each device holds its own copy of the array until the process
// ends; its address is looked up once per device (with that device
// current) and only that address is ever handed to kernels.  Every call on
// a device shares the array, so calls that overlap on one device race.  No
// byte of it needs to start at zero: every call writes the activations it
// reads (the padding entries past T feed only token columns that are never
// stored).
namespace {
constexpr size_t kNoAllocScratchBytes = (size_t)4 << 20;
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};

int scratch_ptr(void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return ANE_ERR_HIP;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
            (void)hipGetLastError();
            return ANE_ERR_HIP;
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return ANE_OK;
}
}  // namespace

extern "C" size_t ane_hip_q8_0_mul_mat_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int ane_hip_q8_0_mul_mat_noalloc(uint32_t N, uint32_t K, uint32_t T, const float* x, const void* W,
                                            float* y, void* stream) {
    if (N == 0 || T == 0) return ANE_OK;
    const size_t need = ane_hip_q8_0_mul_mat_workspace_size(K, T);
    if (need > kNoAllocScratchBytes) return ANE_ERR_WORKSPACE;
    void* ws = nullptr;
    const int st = scratch_ptr(&ws);
    if (st != ANE_OK) return st;
    return ane_hip_q8_0_mul_mat(N, K, T, x, W, y, ws, kNoAllocScratchBytes, stream);
}
