// gemm_i8.hpp -- parameters shared by the int8 contraction kernels.
#pragma once

#include "common.hpp"

namespace ane {

struct GemmParams {
    const int8_t* A;      // row-major, K contiguous
    uint64_t lda;         // bytes between rows of A
    const int8_t* B;      // Bt (N x K, K contiguous) or SMOPA panels
    uint64_t ldb;         // Bt: bytes between rows; panel: groups per panel (G)
    uint32_t rowsA;       // rows of A that may be read (others read as 0)
    uint32_t colsB;       // columns of B that may be read (others read as 0)
    uint32_t Kp;          // contraction length, multiple of 16
    uint32_t Mout, Nout;  // output rows / columns written
    float s;              // epilogue multiplier (when sdev == nullptr)
    const float* sdev;    // device {sa, sb}: s = (sa*sb)*smul
    float smul;
    const float* bias;    // fp32[Nout] or nullptr (adds +0.0f)
    float lo;             // ReLU floor: +0 or -FLT_MAX
    float* C;             // fp32 output, row stride ldc
    uint64_t ldc;
    int32_t* Craw;        // raw int32 output instead (debug entry)
};

// dense_fused_i8 operand preparation (quantize_fused.hip): absmax partials
// (kFusedPartials per tensor), qA (M x Kp), qBt (N x Kp), scales {sa, sb},
// and the launch's wait record wstatus: wstatus[0] = the number of
// workgroups that met at the grid-wide wait (0 on the two-pass route, which
// has none), wstatus[1 + w] = what workgroup w saw there (0, or timed-out /
// mixed-arrival bits).  Every launch writes it, so no clearing is needed.
constexpr uint32_t kFusedPartials = 1024;
int launch_fused_quantize(const float* A, const float* B, uint32_t M, uint32_t N, uint32_t K,
                          uint32_t Kp, uint32_t* partials, int8_t* qA, int8_t* qBt, float* scales,
                          uint32_t* wstatus, hipStream_t s);
// The whole of dense_fused_i8 for small operands (K <= 1024, at most 512
// tiles of 16 x 16): the absmax pass, then one launch that quantizes each tile's rows
// and columns into LDS and contracts them (quantize_fused.hip).  Writes C,
// the scales and the wait record, not qA / qBt.
bool small_fused_eligible(uint32_t M, uint32_t N, uint32_t K);
int launch_fused_small(const float* A, const float* B, uint32_t M, uint32_t N, uint32_t K, float smul, float lo,
                       float* C, uint32_t* partials, float* scales, uint32_t* wstatus, hipStream_t s);
// The whole of dense_fused_i8 for at most 16 rows of A in one launch with a
// grid-wide wait (quantize_fused.hip, k_fused_strip): M <= 16, K % 512 == 0,
// K <= 4096, N % 16 == 0, at most one 16-column strip of B per workgroup,
// 16-byte aligned operands and at least 12 MiB of B.  Writes C, the scales
// and the wait record, not qA / qBt.  Returns false when the route cannot
// run (nothing queued); true when it was queued (*status = ANE_ERR_HIP if the
// launch failed after that).
bool strip_fused_eligible(uint32_t M, uint32_t N, uint32_t K, const float* A, const float* B);
bool launch_fused_strip(const float* A, const float* B, uint32_t M, uint32_t N, uint32_t K, float smul, float lo,
                        float* C, uint32_t* partials, float* scales, uint32_t* wstatus, hipStream_t s,
                        int* status);
// The current device's record of failed grid-wide waits (sticky bits; 0 if
// the resident route never ran): read, and cleared together with the
// counters once the device is idle when nonzero.
int resident_slot_check(uint32_t* bits);
bool resident_mixed_bit(uint32_t bits);

// 256 x 256 tile kernel (gemm_i8_tile256.hip): Bt layout, signed A, K a
// multiple of 64 (run as 128-byte slices, an odd last half read as zeros),
// 16-byte aligned rows, and enough rows/columns to fill 256-wide tiles
// reasonably.
// any_rows: also fewer rows than one tile (rows past Mout read as zeros).
// ksplit > 1 splits K over gridDim.y workgroups per tile, each writing its
// int32 plane y of Craw (Mout x ldc): raw output only.
bool tile256_eligible(const GemmParams& p, bool any_rows = false);
int launch_gemm_tile256(const GemmParams& p, hipStream_t s, uint32_t ksplit = 1);

// The same loop at 128 x 128 tiles (gemm_i8_tile128.hip).
bool tile128_eligible(const GemmParams& p, bool any_rows = false);
int launch_gemm_tile128(const GemmParams& p, hipStream_t s, uint32_t ksplit = 1);
// The same at 128 x 128 tiles on a 3-stage ring with 8 waves, one workgroup
// per CU (gemm_i8_tile128d.hip): for launches of at most one workgroup per CU.
bool tile128d_eligible(const GemmParams& p, bool any_rows = false);
int launch_gemm_tile128d(const GemmParams& p, hipStream_t s, uint32_t ksplit = 1);

// Few-row kernel (gemm_i8_skinny.hip): Bt layout, signed A, M <= 128, one
// workgroup per 16 columns.
bool skinny_eligible(const GemmParams& p);
int launch_gemm_skinny(const GemmParams& p, hipStream_t s);

}  // namespace ane
