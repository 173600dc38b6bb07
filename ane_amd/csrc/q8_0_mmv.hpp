// q8_0_mmv.hpp -- the activation-stationary G-mode mul_mat (q8_0_mmv.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace ane {

// TT token tiles per workgroup of NW waves, n_tg token groups, rt_per_wg
// row tiles per workgroup, Tp tokens in the activation form; TT == 0: shape
// not served.
struct MmvPlan {
    uint32_t TT, NW, n_tg, rt_per_wg, Tp;
};
MmvPlan mmv_plan(uint32_t N, uint32_t nb, uint32_t T);
// Workspace bytes the plan's activation form takes.
bool mmv_fills_cus(uint32_t N);
uint64_t mmv_workspace_bytes(uint32_t nb, const MmvPlan& pl);
// The same for any plan of T tokens (the activation form of ceil16(T) tokens).
uint64_t mmv_workspace_bound(uint32_t nb, uint32_t T);
// y[T x N] = the G-mode product of x[T x K] with N Q8_0 rows of nb blocks;
// -1 when the shape or the workspace does not fit this kernel (nothing is
// launched), else an ane_status.
int mmv_mul_mat(uint32_t N, uint32_t nb, uint32_t K, uint32_t T, const float* x, const void* W, float* y,
                void* workspace, size_t workspace_bytes, hipStream_t s);

}  // namespace ane
