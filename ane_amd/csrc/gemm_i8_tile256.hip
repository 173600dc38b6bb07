// gemm_i8_tile256.hip -- the large-shape int8 contraction of dense_fused_i8
// (and gemm_s8_i32): C[M x N] = epilogue(A[M x K] . Bt[N x K]^T), both
// operands int8 row-major with K contiguous.
//
// Design (gfx950, one workgroup per CU):
//  * 256 x 256 output tile.  NW waves (4, 8 or 16) in a WM x WN grid; a
//    wave owns FM x FN blocks of v_mfma_i32_32x32x32_i8 accumulators.  With
//    8 or 16 waves, 2 or 4 share each SIMD, so one wave's barrier or LDS
//    wait is covered by the others' MFMAs.
//  * K advances in 128-byte slices through an LDS ring of STAGES stages
//    (2 x 64 KB for 256-tiles, 2 x 32 KB for 128-tiles, 3 x 32 KB for the
//    128-tiles of gemm_i8_tile128d.hip).  Each slice starts with a barrier
//    (every wave's copies of slice kt have landed, and every wave has
//    finished slice kt-1), after which the copies of slice kt+STAGES-1 go
//    into slice kt-1's stage.  Those copies are pinned one between MFMAs of the
//    slice's first two k-steps (sched_barrier): issuing a buffer_load ...
//    lds occupies the issuing wave for tens of cycles, and issued back to
//    back they drained the MFMA pipe after every barrier (4096^3: the K loop
//    about 2-3 us faster than a 4-stage ring of 64-byte slices whose copies
//    the compiler bunched; copies spread over all four k-steps land too
//    late).  The next k-step's fragment reads sit between the MFMAs the same
//    way.  When Kp is an odd multiple of 64, the last slice's upper half is
//    sent out of range per lane and lands as zeros.
//  * Slices are copied with buffer_load_dwordx4 ... lds (direct global ->
//    LDS, no VGPR staging; rows past the operand's end and the out-of-range
//    tail slices read as zeros through the buffer resource's range check, so
//    every slice issues the same number of copies).
//  * Synchronisation is s_waitcnt vmcnt + a bare s_barrier.  __syncthreads()
//    would add a release fence, i.e. vmcnt(0), draining the slices that are
//    meant to stay in flight.
//  * LDS layout per stage: [rows][128 bytes] for A then for Bt; the 16-byte
//    chunk c of row r sits in slot c ^ ((r >> 1) & 7).  A ds_read_b128 serves 16
//    lanes (16 consecutive rows, same chunk) per LDS cycle (64 banks x 4
//    bytes); g gives them 16 distinct bank groups.  Each copy
//    wave-instruction writes 1 KB of consecutive LDS, so the swizzle is
//    applied on the global side.
//  * Tiles are assigned XCD-major: dispatch round-robins workgroups over the
//    8 XCDs, so workgroup w is remapped to logical tile (w%8)*(T/8) + w/8 and
//    each XCD's L2 sees a compact 4 x 8 block of tiles.
//  * Epilogue: fmaxA(fadd(fmul((float)acc, s), bias), lo), one rounding per
//    operation, staged through LDS so each wave stores whole row segments
//    with 16-byte stores.
#include "gemm_i8.hpp"

namespace ane {
namespace {

// ANE_TILE selects the output tile: 256 (this file) or 128
// (gemm_i8_tile128.hip includes this file with ANE_TILE 128: the same loop
// at 128 x 128 with 4 waves, two workgroups per CU, for shapes with fewer
// 256-tiles than CUs).
#ifndef ANE_TILE
#define ANE_TILE 256
#endif
#if ANE_TILE == 256
#ifndef ANE_TILE_KERNEL
#define ANE_TILE_KERNEL k_gemm_i8_tile256
#define ANE_TILE_ELIGIBLE tile256_eligible
#define ANE_TILE_LAUNCH launch_gemm_tile256
#endif
#ifndef ANE_TILE_WAVES
#define ANE_TILE_WAVES 8
#endif
#elif ANE_TILE == 128
#ifndef ANE_TILE_KERNEL
#define ANE_TILE_KERNEL k_gemm_i8_tile128
#define ANE_TILE_ELIGIBLE tile128_eligible
#define ANE_TILE_LAUNCH launch_gemm_tile128
#endif
#ifndef ANE_TILE_WAVES
#define ANE_TILE_WAVES 4
#endif
#else
#error "ANE_TILE is 256 or 128"
#endif
// ANE_TILE_STAGES: LDS ring depth (2 by default).  Slice kt+STAGES-1 is
// copied while slice kt is multiplied, so STAGES-1 slices are in flight.
#ifndef ANE_TILE_STAGES
#define ANE_TILE_STAGES 2
#endif

constexpr int TM = ANE_TILE, TN = ANE_TILE;
constexpr int TK = 128;                       // bytes of K per slice
constexpr int STAGES = ANE_TILE_STAGES;       // LDS ring depth
constexpr int NW = ANE_TILE_WAVES;            // waves per workgroup
constexpr int kThreads = NW * 64;
constexpr int WN = NW == 16 ? 4 : 2;          // waves along N
constexpr int WM = NW / WN;                   // waves along M
constexpr int FM = TM / (WM * 32);            // 32x32 MFMA blocks per wave along M
constexpr int FN = TN / (WN * 32);            // ... along N
constexpr int kChunks = TK / 16;              // 16-byte chunks per row
constexpr int kStageA = TM * TK;
constexpr int kStageB = TN * TK;
constexpr int kStage = kStageA + kStageB;
constexpr int kLdsBytes = STAGES * kStage;
constexpr int kWgPerCu = 2 * kLdsBytes <= 160 * 1024 ? 2 : 1;  // 128-tiles on a 2-stage ring: two per CU
constexpr int kWavesPerEu = kWgPerCu * NW / 4;
constexpr int kRowsPerDma = 1024 / TK;        // rows covered by one copy wave-instruction
constexpr int kRowsPerWave = TM / NW;         // rows of A (and of Bt) each wave copies
constexpr int kDmaPerWave = kRowsPerWave / kRowsPerDma;
constexpr int kSteps = TK / 32;
static_assert(NW == 4 || NW == 8 || NW == 16, "4, 8 or 16 waves");
static_assert(STAGES >= 2 && (STAGES - 2) * 2 * kDmaPerWave < 64, "ring depth fits the vmcnt field");
static_assert(kLdsBytes <= 160 * 1024, "LDS ring exceeds 160 KB");
// Epilogue staging: per wave EPR rows x (FN*32) fp32 per pass, rows padded
// by 32 bytes (4 rows apart = 128 bytes mod 256: the two half-waves of a
// staging write land in different bank halves).
constexpr int kEpiCols = FN * 32;
constexpr int kEpiRowBytes = kEpiCols * 4 + 32;
constexpr int EPR = NW == 4 ? 32 : 16;
constexpr int kLanesPerRow = kEpiCols / 4;     // 16-byte stores per staged row
constexpr int kRowsPerStore = 64 / kLanesPerRow;
constexpr int kEpiWaveBytes = EPR * kEpiRowBytes;
static_assert(NW * kEpiWaveBytes <= kLdsBytes, "epilogue staging does not fit");

__device__ __forceinline__ uint32_t swz_g(uint32_t row) { return (row >> 1) & 7; }
__device__ __forceinline__ uint32_t swz(uint32_t row, uint32_t chunk) {
    return row * TK + ((chunk ^ swz_g(row)) << 4);
}

// One slice copy: wave w copies rows [w*kRowsPerWave, (w+1)*kRowsPerWave)
// of the tile's A rows and of its Bt rows; wave-instruction i covers
// kRowsPerDma rows (1 KB of consecutive LDS).  A lane whose 16 bytes lie at
// or past `kmax` bytes into the slice (kmax 0: the slice is past K) is sent
// out of range: its copy writes zeros without touching memory.
struct SliceCopy {
    __amdgpu_buffer_rsrc_t ra, rb;
    int8_t* stage;
    uint32_t wave, k0, kmax;
};

// Copy d of a slice (d < kDmaPerWave: A, else Bt); unrolled callers pass a
// constant d.  kofs[i]: this lane's byte offset inside the slice for copy i
// (its swizzled 16-byte chunk), the same for A and Bt.
__device__ __forceinline__ void issue_one(const SliceCopy& c, const uint32_t (&offA)[kDmaPerWave],
                                          const uint32_t (&offB)[kDmaPerWave],
                                          const uint32_t (&kofs)[kDmaPerWave], int d) {
    const int i = d % kDmaPerWave;
    const bool isB = d >= kDmaPerWave;
    int8_t* dst = c.stage + (c.wave * kRowsPerWave + i * kRowsPerDma) * TK + (isB ? kStageA : 0);
    const uint32_t o = kofs[i] < c.kmax ? (isB ? offB[i] : offA[i]) + c.k0 : 0x80000000u;
    copy16_to_lds(isB ? c.rb : c.ra, dst, o);
}

struct Frags {
    v4i a[FM], b[FN];
};

__device__ __forceinline__ void load_frags(const int8_t* stage, uint32_t rA, uint32_t rB,
                                           uint32_t chunk, Frags& f) {
#pragma unroll
    for (int mi = 0; mi < FM; mi++)
        f.a[mi] = *reinterpret_cast<const v4i*>(stage + swz(rA + mi * 32, chunk));
#pragma unroll
    for (int ni = 0; ni < FN; ni++)
        f.b[ni] = *reinterpret_cast<const v4i*>(stage + kStageA + swz(rB + ni * 32, chunk));
}

// One of the FM + FN fragment reads of a k-step, by index.
__device__ __forceinline__ void load_frag(const int8_t* stage, uint32_t rA, uint32_t rB, uint32_t chunk,
                                          Frags& f, int idx) {
    if (idx < FM)
        f.a[idx] = *reinterpret_cast<const v4i*>(stage + swz(rA + idx * 32, chunk));
    else
        f.b[idx - FM] = *reinterpret_cast<const v4i*>(stage + kStageA + swz(rB + (idx - FM) * 32, chunk));
}

// One slice: the copies of the next slice and the next k-step's fragment
// reads pinned between the MFMAs.  f0 holds the slice's first fragments on
// entry.
__device__ __forceinline__ void slice_pinned(v16i (&acc)[FM][FN], Frags& f0, Frags& f1, const int8_t* cur,
                                             uint32_t rA, uint32_t rB, uint32_t chalf, const SliceCopy& c,
                                             const uint32_t (&offA)[kDmaPerWave],
                                             const uint32_t (&offB)[kDmaPerWave],
                                             const uint32_t (&kofs)[kDmaPerWave]) {
    constexpr int nM = FM * FN, nD = FM + FN;
    constexpr int kCopySteps = 2;                       // k-steps that carry the copies
    constexpr int kPerStep = 2 * kDmaPerWave / kCopySteps;
    constexpr int kStride = nM / kPerStep;              // MFMAs per copy
    static_assert(kPerStep * kCopySteps == 2 * kDmaPerWave && kStride * kPerStep == nM && kCopySteps <= kSteps,
                  "copies must spread evenly over the MFMAs");
#pragma unroll
    for (int ks = 0; ks < kSteps; ks++) {
        Frags& fc = (ks & 1) ? f1 : f0;
        Frags& fn = (ks & 1) ? f0 : f1;
#pragma unroll
        for (int g = 0; g < nM; g++) {
            const int mi = g / FN, ni = g % FN;
            acc[mi][ni] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fc.a[mi], fc.b[ni], acc[mi][ni], 0, 0, 0);
            if (ks + 1 < kSteps && g < nD) load_frag(cur, rA, rB, 2 * (ks + 1) + chalf, fn, g);
            if (ks < kCopySteps && g % kStride == kStride - 1)
                issue_one(c, offA, offB, kofs, ks * kPerStep + g / kStride);
            __builtin_amdgcn_sched_barrier(0);
        }
        // fewer MFMAs than fragments per k-step (1 x 2 blocks per wave): the
        // rest of the next k-step's fragments after the last MFMA
#pragma unroll
        for (int g = nM; g < nD; g++)
            if (ks + 1 < kSteps) load_frag(cur, rA, rB, 2 * (ks + 1) + chalf, fn, g);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// A whole 16-byte store of C with the sc1 bit (agent scope): the line is
// written through the XCD's L2 instead of being left dirty there for the
// end-of-kernel write-back (4096^3: the op about 1.5 us faster than plain
// stores; a buffer_store with the same bit measured slower than this
// global_store).  Inline assembly, as no builtin sets the bit on a plain
// store.  The compiler does not count these stores in vmcnt; since vector
// memory operations complete in issue order, uncounted stores can only
// make its later vmcnt waits stricter, never release one early.  A VALU
// write to the data registers of a store wider than 8 bytes needs one wait
// state after the store; the compiler's hazard recognizer does not see
// inside the asm, so the s_nop provides it.
__device__ __forceinline__ void store16_sc1(uint32_t* dst, v4i v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 0" ::"v"(dst), "v"(v) : "memory");
}

__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kWavesPerEu, kWavesPerEu)))
ANE_TILE_KERNEL(GemmParams p, uint32_t tiles_m, uint32_t tiles_n) {
    __shared__ __attribute__((aligned(1024))) int8_t smem[kLdsBytes];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // XCD-major tile order, then groups of 4 tile-rows.
    const uint32_t total = tiles_m * tiles_n;
    const uint32_t wg = blockIdx.x;
    uint32_t logical = wg;
    if ((total & 7) == 0) logical = (wg & 7) * (total >> 3) + (wg >> 3);
    constexpr uint32_t GM = 4;
    const uint32_t per_group = GM * tiles_n;
    const uint32_t group = logical / per_group;
    const uint32_t first_m = group * GM;
    const uint32_t gm = (tiles_m - first_m) < GM ? (tiles_m - first_m) : GM;
    const uint32_t in = logical % per_group;
    const uint32_t row0 = (first_m + in % gm) * TM;
    const uint32_t col0 = (in / gm) * TN;

    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A, (uint32_t)(p.rowsA * p.lda));
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.B, (uint32_t)(p.colsB * p.ldb));
    uint32_t offA[kDmaPerWave], offB[kDmaPerWave], kofs[kDmaPerWave];
    {
        // lane l fills slot l % kChunks of row wave*kRowsPerWave + i*kRowsPerDma + l/kChunks
        const uint32_t r = wave * kRowsPerWave + lane / kChunks;
#pragma unroll
        for (int i = 0; i < kDmaPerWave; i++) {
            const uint32_t row = r + i * kRowsPerDma;
            const uint32_t chunk = (lane % kChunks) ^ swz_g(row);
            kofs[i] = chunk * 16;
            offA[i] = (row0 + row) * (uint32_t)p.lda + kofs[i];
            offB[i] = (col0 + row) * (uint32_t)p.ldb + kofs[i];
        }
    }

    // the epilogue multiplier, read before the K loop so its latency is hidden
    float s = p.s;
    if (p.sdev) s = __fmul_rn(__fmul_rn(p.sdev[0], p.sdev[1]), p.smul);

    const uint32_t wr0 = (wave / WN) * (FM * 32);
    const uint32_t wc0 = (wave % WN) * (FN * 32);
    const uint32_t rA = wr0 + (lane & 31);
    const uint32_t rB = wc0 + (lane & 31);
    const uint32_t chalf = lane >> 5;

    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

    // Split K (gridDim.y > 1, raw int32 output only): workgroup (x, y) takes
    // the slices [y * per, (y + 1) * per) and writes its int32 plane y of
    // Craw (Mout x ldc each); the planes are added afterwards (exact).
    const uint32_t nk = (p.Kp + TK - 1) / TK;
    const uint32_t per = (nk + gridDim.y - 1) / gridDim.y;
    const uint32_t kt0 = blockIdx.y * per < nk ? blockIdx.y * per : nk;
    const uint32_t kt1 = kt0 + per < nk ? kt0 + per : nk;
    int32_t* const craw = p.Craw ? p.Craw + (uint64_t)blockIdx.y * p.Mout * p.ldc : nullptr;
    auto kmax = [&](uint32_t k) -> uint32_t {  // bytes of slice k inside this range of Kp (0 past it)
        const uint32_t k0 = k * TK;
        return (k >= kt1 || k0 >= p.Kp) ? 0u : (p.Kp - k0 < (uint32_t)TK ? p.Kp - k0 : (uint32_t)TK);
    };
    Frags f0, f1;
#pragma unroll
    for (int j = 0; j < STAGES - 1; j++) {
        const SliceCopy c{ra, rb, smem + j * kStage, wave, (kt0 + j) * TK, kmax(kt0 + j)};
#pragma unroll
        for (int d = 0; d < 2 * kDmaPerWave; d++) issue_one(c, offA, offB, kofs, d);
    }
    uint32_t st = 0;  // stage of slice kt
    for (uint32_t kt = kt0; kt < kt1; kt++) {
        // this wave's copies of slice kt landed (those of the STAGES-2
        // slices after it may still be in flight; copies complete in order)
        wait_vmcnt<(STAGES - 2) * 2 * kDmaPerWave>();
        lds_barrier();    // everyone's did; everyone finished slice kt-1
        const int8_t* cur = smem + st * kStage;
        const uint32_t sn = st == 0 ? STAGES - 1 : st - 1;  // slice kt-1's stage takes slice kt+STAGES-1
        const SliceCopy c{ra, rb, smem + sn * kStage, wave, (kt + STAGES - 1) * TK, kmax(kt + STAGES - 1)};
        st = st + 1 == STAGES ? 0 : st + 1;
        load_frags(cur, rA, rB, chalf, f0);
        __builtin_amdgcn_sched_barrier(0);
        slice_pinned(acc, f0, f1, cur, rA, rB, chalf, c, offA, offB, kofs);
    }
    wait_vmcnt<0>();
    __syncthreads();  // all fragment reads done: the ring becomes epilogue staging

    float bj[FN];
#pragma unroll
    for (int ni = 0; ni < FN; ni++) {
        const uint32_t j = col0 + wc0 + ni * 32 + (lane & 31);
        bj[ni] = (p.bias && j < p.Nout) ? p.bias[j] : 0.0f;
    }
    int8_t* epi = smem + wave * kEpiWaveBytes;
    const bool vec_ok = (((uintptr_t)(craw ? (void*)craw : (void*)p.C)) & 15) == 0 && (p.ldc & 3) == 0;

#pragma unroll
    for (int mi = 0; mi < FM; mi++) {
#pragma unroll
        for (int h = 0; h < 32 / EPR; h++) {
            // rows [h*EPR, (h+1)*EPR) of the 32-row block mi -> LDS.  Lane l,
            // register r of a 32x32 MFMA block holds row 8(r/4) + 4(l/32) +
            // r%4, column l%32.
#pragma unroll
            for (int ni = 0; ni < FN; ni++) {
#pragma unroll
                for (int r = h * EPR / 2; r < (h + 1) * EPR / 2; r++) {
                    const uint32_t lr = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3) - h * EPR;
                    const uint32_t lc = ni * 32 + (lane & 31);
                    uint32_t bitsv;
                    if (craw) {
                        bitsv = (uint32_t)acc[mi][ni][r];
                    } else {
                        const float f = __fadd_rn(__fmul_rn((float)acc[mi][ni][r], s), bj[ni]);
                        bitsv = __float_as_uint(fmax_a(f, p.lo));
                    }
                    *reinterpret_cast<uint32_t*>(epi + lr * kEpiRowBytes + lc * 4) = bitsv;
                }
            }
            wait_lgkmcnt0();
            __builtin_amdgcn_wave_barrier();
            // 16 B per lane: kLanesPerRow lanes cover one staged row
#pragma unroll
            for (int q = 0; q < EPR / kRowsPerStore; q++) {
                const uint32_t lr = kRowsPerStore * q + lane / kLanesPerRow;
                const uint32_t lc = 4 * (lane % kLanesPerRow);
                const v4i v = *reinterpret_cast<const v4i*>(epi + lr * kEpiRowBytes + lc * 4);
                const uint32_t i = row0 + wr0 + mi * 32 + h * EPR + lr;
                const uint32_t j = col0 + wc0 + lc;
                if (i >= p.Mout) continue;
                uint32_t* dst = craw ? reinterpret_cast<uint32_t*>(craw) + (uint64_t)i * p.ldc + j
                                     : reinterpret_cast<uint32_t*>(p.C) + (uint64_t)i * p.ldc + j;
                if (vec_ok && j + 3 < p.Nout) {
                    store16_sc1(dst, v);
                } else {
                    if (j + 0 < p.Nout) dst[0] = (uint32_t)v.x;
                    if (j + 1 < p.Nout) dst[1] = (uint32_t)v.y;
                    if (j + 2 < p.Nout) dst[2] = (uint32_t)v.z;
                    if (j + 3 < p.Nout) dst[3] = (uint32_t)v.w;
                }
            }
            wait_lgkmcnt0();  // staging reads done before the next pass overwrites them;
            __builtin_amdgcn_wave_barrier();  // the global stores keep draining
        }
    }
}

}  // namespace

bool ANE_TILE_ELIGIBLE(const GemmParams& p, bool any_rows) {
    if ((!any_rows && p.Mout < TM) || p.Nout < TN) return false;
    if (p.Kp == 0 || (p.Kp % 64) != 0) return false;
    if ((p.lda & 15) || (p.ldb & 15)) return false;
    if ((((uintptr_t)p.A) & 15) || (((uintptr_t)p.B) & 15)) return false;
    if (p.rowsA < p.Mout || p.colsB < p.Nout) return false;
    // buffer offsets are 32-bit and 0x80000000 marks an empty copy: every
    // row of every tile, in range or not, stays below it (a lane's K offset
    // is sent only below Kp)
    const uint64_t rows_a = ceil_to(p.Mout, TM) + TM, rows_b = ceil_to(p.Nout, TN) + TN;
    if (rows_a * p.lda + p.Kp >= (1ull << 31) || rows_b * p.ldb + p.Kp >= (1ull << 31)) return false;
    return true;
}

int ANE_TILE_LAUNCH(const GemmParams& p, hipStream_t s, uint32_t ksplit) {
    const uint32_t tiles_m = (p.Mout + TM - 1) / TM;
    const uint32_t tiles_n = (p.Nout + TN - 1) / TN;
    const uint64_t total = (uint64_t)tiles_m * tiles_n;
    if (total > 0x7fffffffull || ksplit == 0 || ksplit > 65535) return ANE_ERR_INVALID_ARG;
    if (ksplit > 1 && !p.Craw) return ANE_ERR_INVALID_ARG;  // split K writes int32 planes
    hipLaunchKernelGGL(ANE_TILE_KERNEL, dim3((uint32_t)total, ksplit), dim3(kThreads), 0, s, p, tiles_m,
                       tiles_n);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

}  // namespace ane
