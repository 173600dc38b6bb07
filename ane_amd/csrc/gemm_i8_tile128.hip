// gemm_i8_tile128.hip -- the contraction loop of gemm_i8_tile256.hip at
// 128 x 128 output tiles: 4 waves of 2 x 2 v_mfma_i32_32x32x32_i8 blocks, a
// 64 KB LDS ring, two workgroups per CU.  For shapes whose 256-tiles would
// leave CUs idle (dense_fused_i8 at M = 256 .. 2048 with N = 4096 has 16-128
// of them on 256 CUs).
#define ANE_TILE 128
#include "gemm_i8_tile256.hip"
