// q8_0_mmv.hip -- G-mode Q8_0 mul_mat for 16+ tokens with the activations
// held in VGPRs (ggml GGML_OP_MUL_MAT over ne11 tokens, ggml-ane.cpp:119-154,
// in this build's G arithmetic).
//
// Arithmetic (the same as every G-mode kernel): for output y[t][row], 16 fp32
// chains p[r], r = b mod 16, each over its blocks b = r, r+16, ... in
// increasing order, p[r] = fmaf((float)isum_b, fl(d_w * d_x), p[r]) with
// isum_b the exact int32 dot of the row's and the token's quantized block,
// then y = the FADDV pairwise tree over p[0..15].
//
// Layout of the work:
//  * A workgroup has NW waves (8 or 16); wave w owns the 16/NW consecutive
//    residues (16/NW)*w + q, an aligned subtree of the FADDV tree whose lower
//    levels it adds itself.  Lane (g, c16) of a
//    v_mfma_i32_16x16x32_i8 receives token c16 of a token tile as A and weight
//    row c16 of a row tile as B, so it holds the isums of weight row c16 for
//    tokens 4g..4g+3 (as in k_q8_0_mmt).
//  * The workgroup serves one token group (TT token tiles of 16 tokens) for
//    a run of row tiles.  Each wave loads, once, the activation bytes its
//    MFMAs use -- for every block b = r + 16j and token tile, lane (g, c16)'s
//    8 bytes 8g..8g+7 of token c16 -- into VGPRs (NBR = nb/16 blocks x TT
//    tiles x 2 VGPRs), from a block-major activation form (qxb[b][Tp][32],
//    so each load is 512 contiguous bytes).  The activations are read from
//    L2 once per workgroup instead of once per ring stage.
//  * Only the weights stream through LDS: a ring of 16 rows x 64 blocks in 2
//    stages, or x 32 blocks in 3 stages for one token tile (the row stride
//    padded to 12 dwords mod 64, as in k_q8_0_mmt), copied by
//    buffer_load_dwordx4 ... lds and read by all 16 waves, each taking its
//    residue's blocks of the stage.  The token scales d_x of the
//    group (block-major, nb x 16TT floats) are copied into LDS once.
//  * After a row tile's last stage the NW wave subtotals of every (row,
//    token) meet in LDS for the tree's upper levels.
//  * Stage 0's weights and the scales are copied before the activation loads
//    are issued, so the first stage waits only for them; each activation load
//    is waited for where its block is first multiplied.
// Workgroups go to the XCDs round-robin; the token groups of one run of row
// tiles are consecutive slots of one XCD, so its weights are fetched into one
// L2 for all of them.
#include "common.hpp"
#include "q8_0_mmv.hpp"

#include <atomic>

namespace ane {
namespace {

// The weight ring: kStages stages of 16 rows x kSbk blocks, the row stride
// padded to 12 dwords mod 64.  Measured: with one token tile (the least math
// per stage) 3 stages of 32 blocks, so that two stages' copies are in flight
// (gate_up T = 16 27.8 -> 26.5 us, down 19.7 -> 18.0); with more token tiles
// 2 stages of 64 (smaller stages measured 5-20 % slower there).
template <int TT>
struct MvRing {
    static constexpr uint32_t kSbk = TT == 1 ? 32 : 64;  // blocks per stage
    static constexpr uint32_t kStages = TT == 1 ? 3 : 2;
    static constexpr uint32_t kRowData = kSbk * 34 / 16;  // chunks of a row's stage
    static constexpr uint32_t kRowChunks = kRowData + (3 + 16 - kRowData % 16) % 16;
    static constexpr uint32_t kWChunks = 16 * kRowChunks;
    static constexpr uint32_t kWInstr = (kWChunks + 63) / 64;
    static constexpr uint32_t kStageBytes = kWChunks * 16;
    static_assert((kRowChunks * 4) % 64 == 12, "row stride");
};
constexpr uint32_t kMvMaxSbk = 64;  // every ring's stages divide rows of a multiple of 64 blocks
typedef unsigned int v2u __attribute__((ext_vector_type(2)));

// ((a0+a1)+(a2+a3)) + ... over n adjacent values: levels of the FADDV tree.
template <int n>
__device__ __forceinline__ float tree_sum(float (&a)[n]) {
#pragma unroll
    for (int w = 1; w < n; w *= 2)
#pragma unroll
        for (int i = 0; i + w < n; i += 2 * w) a[i] = a[i] + a[i + w];
    return a[0];
}

// Activation form for k_q8_0_mmv: qxb[b][Tp][32] int8 and dxb[b][Tp] fp32,
// tokens T..Tp-1 quantized from zeros (qx 0).  The arithmetic of
// k_q8_act_quantize (8 lanes per block, the 0x19 quantization), so the bits
// are the same.
__global__ void __launch_bounds__(256)
k_q8_act_quantize_bt(uint32_t T, uint32_t Tp, uint32_t nb, uint32_t K, const float* __restrict__ x,
                     uint8_t* __restrict__ qxb, float* __restrict__ dxb) {
    const uint32_t t = blockIdx.x * 256 + threadIdx.x, blk = t >> 3, part = t & 7;
    const uint32_t tok = blk / nb, b = blk - tok * nb;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(x, T * K * 4);
    const uint32_t o = tok < T ? (tok * K + b * 32 + part * 4) * 4 : 0x80000000u;
    float f[4];
#pragma unroll
    for (int e = 0; e < 4; e++) f[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, o + 4 * e, 0, 0));
    const uint32_t m = max8_u32(max(max(abs_key(f[0]), abs_key(f[1])), max(abs_key(f[2]), abs_key(f[3]))));
    float scale, inv;
    quant_params(__uint_as_float(m), scale, inv);
    if (tok < Tp) {
        reinterpret_cast<uint32_t*>(qxb)[(b * Tp + tok) * 8 + part] = pack4(f[0], f[1], f[2], f[3], inv);
        if (part == 0) dxb[b * Tp + tok] = scale;
    }
}

template <int NBR, int TT, int NW>
__global__ void __launch_bounds__(NW * 64)
k_q8_0_mmv(uint32_t N, uint32_t Tp, const uint8_t* __restrict__ W, const uint8_t* __restrict__ qxb,
           const float* __restrict__ dxb, uint32_t T, uint32_t n_tg, uint32_t rt_per_wg, uint32_t n_runs,
           float* __restrict__ y) {
    constexpr uint32_t nb = NBR * 16;
    constexpr uint32_t kTok = TT * 16;
    using R = MvRing<TT>;
    constexpr uint32_t kMvSbk = R::kSbk, kMvStages = R::kStages, kMvRowData = R::kRowData;
    constexpr uint32_t kMvRowChunks = R::kRowChunks, kMvWChunks = R::kWChunks, kMvWInstr = R::kWInstr;
    constexpr uint32_t kMvStageBytes = R::kStageBytes;
    constexpr uint32_t nsk = nb / kMvSbk;       // stages per row tile
    constexpr uint32_t kJps = kMvSbk / 16;      // a residue's blocks per stage
    constexpr int RPW = 16 / NW;                // residues per wave
    constexpr int kEx = TT < 32 / NW ? TT : 32 / NW;  // token tiles per subtotal exchange
    static_assert(TT % kEx == 0, "whole exchanges");
    static_assert(NW == 8 || NW == 16, "8 or 16 waves");
    static_assert(nb % kMvSbk == 0, "whole stages per row");
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    float* const dxs = reinterpret_cast<float*>(smem + kMvStages * kMvStageBytes);  // [nb][kTok]
    float4* const ex = reinterpret_cast<float4*>(smem + kMvStages * kMvStageBytes + nb * kTok * 4);  // [kEx][NW][64]

    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;

    // workgroup -> (run of row tiles, token group); a run's token groups on one XCD
    const uint32_t xcd = blockIdx.x & 7, xslot = blockIdx.x >> 3;
    const uint32_t tg = xslot % n_tg, run = xcd + 8 * (xslot / n_tg);
    if (run >= n_runs) return;
    const uint32_t rtiles = (N + 15) / 16;
    const uint32_t rt0 = run * rt_per_wg;
    const uint32_t rt1 = rt0 + rt_per_wg < rtiles ? rt0 + rt_per_wg : rtiles;
    if (rt0 >= rt1) return;
    const uint32_t tok0 = tg * kTok;
    const uint32_t rb = nb * 34;

    const __amdgpu_buffer_rsrc_t wr = make_rsrc(W, N * rb);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(qxb, nb * Tp * 32);
    const __amdgpu_buffer_rsrc_t dr = make_rsrc(dxb, nb * Tp * 4);

    // 1. stage 0's weight copies first, then the group's token scales, then
    // the activations in block order: the first stage waits only for the
    // weights and scales, and each activation load is waited for (by the
    // compiler's own vmcnt count) where its block's MFMA first needs it.
    constexpr uint32_t kSlots = (kMvWInstr + NW - 1) / NW;  // slot q of a wave: instruction q*NW + wave
    uint32_t ow[kSlots];
#pragma unroll
    for (uint32_t q = 0; q < kSlots; q++) {
        const uint32_t c = 64 * (q * NW + wave) + lane, row = c / kMvRowChunks, sub = c - row * kMvRowChunks;
        ow[q] = (c < kMvWChunks && sub < kMvRowData) ? row * rb + 16 * sub : 0x80000000u;
    }
    const uint32_t nst = (rt1 - rt0) * nsk;
    auto issue = [&](uint32_t s) {
        if (s >= nst) return;
        int8_t* st = smem + (s % kMvStages) * kMvStageBytes;
        const uint32_t rt = rt0 + s / nsk, ck = s % nsk;
        const uint32_t base = rt * 16 * rb + ck * (kMvSbk * 34);
#pragma unroll
        for (uint32_t q = 0; q < kSlots; q++) {
            const uint32_t i = q * NW + wave;
            if (i < kMvWInstr && (kMvWChunks % 64 == 0 || i + 1 < kMvWInstr || lane < kMvWChunks % 64)) {
                const uint32_t row = (64 * i + lane) / kMvRowChunks;
                const bool ok = ow[q] != 0x80000000u && rt * 16 + row < N;
                copy16_to_lds_nt(wr, st + 1024 * i, ok ? ow[q] + base : 0x80000000u);
            }
        }
    };
#pragma unroll
    for (uint32_t i = 0; i + 1 < kMvStages; i++) issue(i);
    {
        // chunk c of the scales: block c / (kTok/4), tokens 4 (c % (kTok/4)) ..
        constexpr uint32_t kDChunks = nb * kTok / 4, kDInstr = (kDChunks + 63) / 64;
#pragma unroll
        for (uint32_t q = 0; q < (kDInstr + NW - 1) / NW; q++) {
            const uint32_t i = q * NW + wave;
            if (i < kDInstr) {
                const uint32_t c = 64 * i + lane, b = c / (kTok / 4), t4 = c - b * (kTok / 4);
                if (kDChunks % 64 == 0 || c < kDChunks)
                    copy16_to_lds(dr, reinterpret_cast<int8_t*>(dxs) + 1024 * i, (b * Tp + tok0 + 4 * t4) * 4);
            }
        }
    }
    // the activation loads stay after those copies: the first stage's wait
    // counts on it
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    // this wave's residues RPW*wave + q (consecutive: an aligned subtree of the FADDV tree)
    uint64_t xv[RPW][NBR][TT];
#pragma unroll
    for (int j = 0; j < NBR; j++)
#pragma unroll
        for (int q = 0; q < RPW; q++)
#pragma unroll
            for (int tt = 0; tt < TT; tt++) {
                const uint32_t b = RPW * wave + q + 16 * j, tok = tok0 + tt * 16 + c16;
                const v2u v = __builtin_amdgcn_raw_buffer_load_b64(xr, ((b * Tp + tok) * 32 + 8 * g), 0, 0);
                xv[q][j][tt] = (uint64_t)v.x | ((uint64_t)v.y << 32);
            }
    constexpr int kActLoads = RPW * NBR * TT;
    constexpr int kFirstWait = kActLoads < 63 ? kActLoads : 63;
    // this wave's copies per stage: kSlots or kSlots - 1
    const bool full = (kSlots - 1) * NW + wave < kMvWInstr;

    uint32_t s = 0;
    for (uint32_t rt = rt0; rt < rt1; rt++) {
        float p[RPW][TT][4];
#pragma unroll
        for (int q = 0; q < RPW; q++)
#pragma unroll
            for (int tt = 0; tt < TT; tt++)
#pragma unroll
                for (int i = 0; i < 4; i++) p[q][tt][i] = 0.0f;
#pragma unroll
        for (uint32_t ck = 0; ck < nsk; ck++, s++) {
            // this wave's copies of stage s have landed: those of the stages
            // after it that are already issued may still be in flight (copies
            // complete in order); first, everything before the activation loads
            if (s == 0) {
                wait_vmcnt<kFirstWait>();
            } else {
                const uint32_t pending = nst - 1 - s < kMvStages - 2 ? nst - 1 - s : kMvStages - 2;
                static_assert(kMvStages <= 4, "the waits below count two pending stages at most");
                if (pending == 0)
                    wait_vmcnt<0>();
                else if (pending == 1)
                    full ? wait_vmcnt<kSlots>() : wait_vmcnt<kSlots - 1>();
                else
                    full ? wait_vmcnt<2 * kSlots>() : wait_vmcnt<2 * (kSlots - 1)>();
            }
            __builtin_amdgcn_s_barrier();  // everyone's; everyone is done with stage s-1
            issue(s + kMvStages - 1);      // into stage s-1's slot
            const int8_t* wrow = smem + (s % kMvStages) * kMvStageBytes + c16 * (kMvRowChunks * 16);
#pragma unroll
            for (uint32_t k = 0; k < kJps; k++)
#pragma unroll
            for (int q = 0; q < RPW; q++) {
                const uint32_t r = RPW * wave + q;
                const uint32_t j = ck * kJps + k;  // compile-time: the chain's next block, b = r + 16j
                const int8_t* wb = wrow + 34 * (r + 16 * k);
                // quants at 34*bl + 2 + 8g: 4-byte aligned for odd bl, 2 bytes past for even
                const bool odd = RPW >= 2 ? (q & 1) : (wave & 1);
                const uint32_t* a32 = reinterpret_cast<const uint32_t*>(wb + 8 * g + (odd ? 2 : 0));
                const uint32_t d0 = a32[0], d1 = a32[1], d2 = a32[2];
                const uint32_t w0 = __builtin_amdgcn_alignbyte(d1, d0, odd ? 0 : 2);
                const uint32_t w1 = __builtin_amdgcn_alignbyte(d2, d1, odd ? 0 : 2);
                const uint64_t wv = (uint64_t)w0 | ((uint64_t)w1 << 32);
                const float dw = half_bits_to_float(*reinterpret_cast<const uint16_t*>(wb));
                const float* dd = dxs + (r + 16 * j) * kTok + 4 * g;
                // d_x of the token tiles (64 bytes apart), two tiles per wait
                constexpr int kDB = TT < 2 ? TT : 2;
                float4 d4s[kDB];
#pragma unroll
                for (int tt = 0; tt < TT; tt++) {
                    const v4i acc = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)xv[q][j][tt], (long)wv,
                                                                          v4i{0, 0, 0, 0}, 0, 0, 0);
                    if (tt % kDB == 0) lds_load_settled_f4x<kDB>(dd + tt * 16, d4s);
                    const float4 d4 = d4s[tt % kDB];
                    const float dx[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                    for (int i = 0; i < 4; i++)  // token 4g + i of tile tt, weight row c16
                        p[q][tt][i] = __builtin_fmaf((float)acc[i], __fmul_rn(dw, dx[i]), p[q][tt][i]);
                }
                // the chain's step is taken here: pure arithmetic would otherwise
                // sink past the stage waits to the row tile's end, keeping every
                // MFMA result live until then
#pragma unroll
                for (int tt = 0; tt < TT; tt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) asm volatile("" : "+v"(p[q][tt][i]));
            }
        }
        // the FADDV tree: each wave's RPW leaves first (the lower levels), then
        // the NW wave subtotals of every (row, token) meet in LDS (the upper).
        // Token tiles [0, kEx) go to ex (32 KB); with TT = 2 kEx, tiles
        // [kEx, TT) go to the ring slot of the stage just finished, which no
        // wave reads once all are past the barrier after the first writes.
        // No barrier follows the reads: the next writes to either region come
        // after the next stage's barrier (the slot's refill is issued there).
        static_assert(TT == kEx || TT == 2 * kEx, "one or two exchange regions");
        static_assert(kEx * NW * 1024 <= kMvStageBytes, "a ring slot holds an exchange region");
        float4* const ex2 = reinterpret_cast<float4*>(smem + ((s - 1) % kMvStages) * kMvStageBytes);
        auto leaves = [&](int tt, float4* dst) {
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float a[RPW];
#pragma unroll
                for (int q = 0; q < RPW; q++) a[q] = p[q][tt][i];
                v[i] = tree_sum<RPW>(a);
            }
            lds_store_settled_f4(dst + wave * 64 + lane, make_float4(v[0], v[1], v[2], v[3]));
        };
#pragma unroll
        for (int te = 0; te < kEx; te++) leaves(te, ex + te * NW * 64);
        lds_barrier();  // the stores waited for themselves; y needs no fence here
        if constexpr (TT == 2 * kEx) {
#pragma unroll
            for (int te = 0; te < kEx; te++) leaves(kEx + te, ex2 + te * NW * 64);
            lds_barrier();
        }
#pragma unroll
        for (uint32_t o0 = 0; o0 < TT * 256; o0 += NW * 64) {
            const uint32_t o = o0 + threadIdx.x;
            if (TT * 256 % (NW * 64) == 0 || o < TT * 256) {
                const uint32_t tt = o >> 8, c = o & 15, u = (o >> 4) & 15;  // row c, token u of tile tt
                const uint32_t ln = 16 * (u >> 2) + c, e = u & 3;
                const float4* src = tt < (uint32_t)kEx ? ex + tt * NW * 64 : ex2 + (tt - kEx) * NW * 64;
                float a[NW];
#pragma unroll
                for (int k = 0; k < NW; k++) a[k] = reinterpret_cast<const float*>(src + k * 64 + ln)[e];
                const float v = tree_sum<NW>(a);
                const uint32_t row = rt * 16 + c, tok = tok0 + tt * 16 + u;
                if (row < N && tok < T) y[(uint64_t)tok * N + row] = v;
            }
        }
    }
}

template <int NBR, int TT, int NW>
int mmv_launch(uint32_t N, uint32_t T, uint32_t Tp, uint32_t n_tg, uint32_t rt_per_wg, const void* W,
               const uint8_t* qxb, const float* dxb, float* y, hipStream_t s) {
    constexpr uint32_t nb = NBR * 16;
    constexpr uint32_t kEx = TT < 32 / NW ? TT : 32 / NW;
    const uint32_t lds = MvRing<TT>::kStages * MvRing<TT>::kStageBytes + nb * TT * 16 * 4 + kEx * NW * 1024;
    if (lds > 160 * 1024) return -1;
    // the dynamic-LDS limit is a per-device attribute of the function
    static std::atomic<bool> attr_set[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return ANE_ERR_HIP;
    if (!attr_set[dev].load(std::memory_order_acquire)) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(k_q8_0_mmv<NBR, TT, NW>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
            return ANE_ERR_HIP;
        attr_set[dev].store(true, std::memory_order_release);
    }
    const uint32_t rtiles = (N + 15) / 16;
    const uint32_t n_runs = (rtiles + rt_per_wg - 1) / rt_per_wg;
    const uint32_t grid = (uint32_t)ceil_to((uint64_t)n_runs, 8) * n_tg;
    hipLaunchKernelGGL((k_q8_0_mmv<NBR, TT, NW>), dim3(grid), dim3(NW * 64), lds, s, N, Tp, (const uint8_t*)W, qxb, dxb,
                       T, n_tg, rt_per_wg, n_runs, y);
    ANE_HIP_CHECK_LAUNCH();
    return ANE_OK;
}

int cus_of_current_device() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (!n) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

}  // namespace

// Shape plan, from measurements on the config-4 projections (2-64 tokens;
// fewer than 16 tokens are padded to one token tile, the padding quantized
// from zeros and never stored): one token tile: TT = 1 on 16 waves (K = 14336 on 8 waves: 24.0
// against 21.7 us for down 4096 x 14336);
// at K = 4096 with two or four token tiles, TT = 2 on 16 waves, except for
// many row tiles (four per CU and more: gate_up 28672 x 4096 at 64 tokens,
// 52.9 us against 64.4 for TT = 2 and 59.8 for TT = 4 on 8 waves), where
// TT = 4 on 16 waves reads the activations once per workgroup.  Row tiles are dealt so that workgroups number at most one
// per CU.  Other shapes (K = 14336 with 17+ tokens, more than 64 tokens, other
// K) keep the older kernels, measured faster (down at 32 / 64 tokens: 29.7 /
// 37.0 us against 31.5 / 52.9 here with two / four token groups) or not
// measured here.
MmvPlan mmv_plan(uint32_t N, uint32_t nb, uint32_t T) {
    MmvPlan pl{};
    if (T < 2 || nb % kMvMaxSbk != 0) return pl;
    const uint32_t nbr = nb / 16;
    const uint32_t ttiles = (T + 15) / 16, rtiles = (N + 15) / 16, cus = (uint32_t)cus_of_current_device();
    uint32_t tt = 0, nw = 0;
    if (nbr == 28 && ttiles == 1) {
        tt = 1, nw = 16;
    } else if (nbr == 8 && ttiles <= 4) {
        if (ttiles == 1)
            tt = 1, nw = 16;
        else if (ttiles % 4 == 0 && rtiles >= 4 * cus)
            tt = 4, nw = 16;
        else if (ttiles % 2 == 0)
            tt = 2, nw = 16;
        else
            tt = 1, nw = 16;
    }
    if (!tt) return pl;
    pl.TT = tt;
    pl.NW = nw;
    pl.n_tg = ttiles / tt;
    const uint32_t per_tg = cus / pl.n_tg;
    pl.rt_per_wg = (rtiles + per_tg - 1) / per_tg;
    pl.Tp = ttiles * 16;
    return pl;
}

// Whether the row tiles of N rows deal evenly over the CUs (a whole number
// per CU, or four and more per CU).  For 2-4 tokens the padded token tile
// pays only then (measured: o, gate_up, down 8.6 / 31.7 / 18.5 -> 8.3 / 25.5
// / 17.9 us at 2 tokens; qkv's 384 row tiles on 256 CUs 10.3 -> 11.0 us).
bool mmv_fills_cus(uint32_t N) {
    const uint32_t rtiles = (N + 15) / 16, cus = (uint32_t)cus_of_current_device();
    return rtiles % cus == 0 || rtiles >= 4 * cus;
}

uint64_t mmv_workspace_bytes(uint32_t nb, const MmvPlan& pl) {
    return ceil_to((uint64_t)nb * pl.Tp * 32, 256) + (uint64_t)nb * pl.Tp * 4;
}

uint64_t mmv_workspace_bound(uint32_t nb, uint32_t T) {
    MmvPlan pl{};
    pl.Tp = (T + 15) / 16 * 16;
    return mmv_workspace_bytes(nb, pl);
}

int mmv_mul_mat(uint32_t N, uint32_t nb, uint32_t K, uint32_t T, const float* x, const void* W, float* y,
                void* workspace, size_t workspace_bytes, hipStream_t s) {
    const MmvPlan pl = mmv_plan(N, nb, T);
    if (!pl.TT) return -1;
    if (mmv_workspace_bytes(nb, pl) > workspace_bytes) return -1;
    if ((uint64_t)N * nb * 34 >= 0x80000000ull || (uint64_t)nb * pl.Tp * 32 >= 0x80000000ull ||
        (uint64_t)T * K * 4 >= 0x80000000ull)
        return -1;
    uint8_t* qxb = static_cast<uint8_t*>(workspace);
    float* dxb = reinterpret_cast<float*>(qxb + ceil_to((uint64_t)nb * pl.Tp * 32, 256));
    const uint32_t nthreads = nb * pl.Tp * 8;
    hipLaunchKernelGGL(k_q8_act_quantize_bt, dim3((nthreads + 255) / 256), dim3(256), 0, s, T, pl.Tp, nb, K, x, qxb,
                       dxb);
    ANE_HIP_CHECK_LAUNCH();
    if (nb / 16 == 28) return mmv_launch<28, 1, 16>(N, T, pl.Tp, pl.n_tg, pl.rt_per_wg, W, qxb, dxb, y, s);
    if (pl.TT == 4) return mmv_launch<8, 4, 16>(N, T, pl.Tp, pl.n_tg, pl.rt_per_wg, W, qxb, dxb, y, s);
    if (pl.TT == 2) return mmv_launch<8, 2, 16>(N, T, pl.Tp, pl.n_tg, pl.rt_per_wg, W, qxb, dxb, y, s);
    return mmv_launch<8, 1, 16>(N, T, pl.Tp, pl.n_tg, pl.rt_per_wg, W, qxb, dxb, y, s);
}

}  // namespace ane
