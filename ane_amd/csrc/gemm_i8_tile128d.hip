// gemm_i8_tile128d.hip -- the contraction loop of gemm_i8_tile256.hip at
// 128 x 128 output tiles for shapes with at most one such tile per CU
// (dense_fused_i8 at M = 129 .. 1024 with N = 4096, and the split-K route of
// 65 .. 128 rows): a 3-stage ring of 128-byte slices (96 KB), so two slices
// are in flight while one is multiplied, and 8 waves of 1 x 2
// v_mfma_i32_32x32x32_i8 blocks, two per SIMD.  With one workgroup per CU
// the 2-stage ring keeps only one 32 KB slice in flight: at M = 1024
// (256 tiles) 28.8 -> 24.8 us, M = 512 21.2 -> 19.1 us, bit-identical.
#define ANE_TILE 128
#define ANE_TILE_STAGES 3
#define ANE_TILE_WAVES 8
#define ANE_TILE_KERNEL k_gemm_i8_tile128d
#define ANE_TILE_ELIGIBLE tile128d_eligible
#define ANE_TILE_LAUNCH launch_gemm_tile128d
#include "gemm_i8_tile256.hip"
