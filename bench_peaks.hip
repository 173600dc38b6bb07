// bench_peaks.hip -- measured ceilings that bench.py reports beside the
// datasheet peaks: an int8 MFMA loop with no memory traffic (and the shader
// clock it runs at), and plain HBM read and write streams.  Built into
// bench_peaks.so beside bench.py, which only the benchmark loads; it is not
// part of ane_amd or of ane's interface.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

namespace {

// Each wave chains `iters` rounds of 8 independent v_mfma_i32_32x32x32_i8
// (65,536 int8 ops each).  Eight accumulators keep the MFMA pipe issuing
// back to back.  The operands cycle through 8 A and 8 B fragments loaded
// from `data` (random bytes from the host), so the multipliers toggle like
// a real contraction's; the MFMA datapath's power, and with it the clock
// the chip holds, depends on that.  out[0..3] of workgroup 0, wave 0:
// shader-clock cycles (s_memtime) and 100 MHz real-time ticks
// (s_memrealtime) at start and end, from which the host derives the clock
// the loop ran at.  Every lane's checksum goes to sums[], so the loop cannot
// be removed.
__global__ void __launch_bounds__(512) k_mfma_i8_loop(uint32_t iters, const v4i* __restrict__ data,
                                                     int* sums, uint64_t* clocks) {
    const int lane = threadIdx.x & 63;
    v4i a[8], b[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        a[j] = data[j * 64 + lane];
        b[j] = data[(8 + j) * 64 + lane];
    }
    v16i acc[8];
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[j][r] = 0;
    const bool timer = blockIdx.x == 0 && threadIdx.x == 0;
    uint64_t c0 = 0, t0 = 0;
    if (timer) {
        c0 = __builtin_amdgcn_s_memtime();
        t0 = __builtin_amdgcn_s_memrealtime();
    }
    for (uint32_t i = 0; i < iters; i += 8) {
#pragma unroll
        for (int u = 0; u < 8; u++)
#pragma unroll
            for (int j = 0; j < 8; j++)
                acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[(u + j) & 7], b[(3 * u + j) & 7], acc[j],
                                                               0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) s += acc[j][r];
    sums[blockIdx.x * blockDim.x + threadIdx.x] = s;
    if (timer) {
        const uint64_t c1 = __builtin_amdgcn_s_memtime();
        const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
        clocks[0] = c0;
        clocks[1] = c1;
        clocks[2] = t0;
        clocks[3] = t1;
    }
}

// Read of n16 16-byte words: workgroup w streams its own contiguous
// 1/gridDim of the buffer, eight loads in flight per thread.  (Contiguous
// per-workgroup ranges measured faster on this HBM than a grid-stride
// interleave: 6.8 against 5.7 TB/s at 1 GiB.)  The XOR of everything read
// is compared with `magic` (chosen by the host), so the loads stay live
// without a store per thread.
__global__ void __launch_bounds__(256) k_read(const v4i* __restrict__ src, uint64_t n16, int magic, int* hit) {
    const uint64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const uint64_t b0 = (uint64_t)blockIdx.x * per;
    const uint64_t b1 = b0 + per < n16 ? b0 + per : n16;
    v4i acc = {0, 0, 0, 0};
    uint64_t i = b0 + threadIdx.x;
    for (; i + 7 * 256 < b1; i += 8 * 256) {
        v4i x[8];
#pragma unroll
        for (int u = 0; u < 8; u++) x[u] = __builtin_nontemporal_load(src + i + u * 256);
#pragma unroll
        for (int u = 0; u < 8; u++) acc ^= x[u];
    }
    for (; i < b1; i += 256) acc ^= src[i];
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == magic) hit[0] = 1;
}

// Write of n16 16-byte words, contiguous per workgroup like k_read.
__global__ void __launch_bounds__(256) k_write(v4i* __restrict__ dst, uint64_t n16, int v) {
    const uint64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const uint64_t b0 = (uint64_t)blockIdx.x * per;
    const uint64_t b1 = b0 + per < n16 ? b0 + per : n16;
    const v4i w = {v, v + 1, v + 2, v + 3};
    for (uint64_t i = b0 + threadIdx.x; i < b1; i += 256) __builtin_nontemporal_store(w, dst + i);
}

}  // namespace

extern "C" {

// wgs workgroups of `threads` (256 or 512) threads, `iters` (a multiple of
// 8) rounds; data holds 16 KB of operand bytes, sums wgs*threads ints,
// clocks 4 uint64.  Returns 0, or -1 for arguments the kernel does not take.
int ane_peak_mfma_i8(uint32_t wgs, uint32_t threads, uint32_t iters, const void* data, int* sums,
                     uint64_t* clocks, hipStream_t stream) {
    if (wgs == 0 || (threads != 256 && threads != 512) || (iters & 7) || !data || !sums || !clocks)
        return -1;
    hipLaunchKernelGGL(k_mfma_i8_loop, dim3(wgs), dim3(threads), 0, stream, iters,
                       static_cast<const v4i*>(data), sums, clocks);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Reads `bytes` (a multiple of 16, 16-byte aligned) with `wgs` workgroups.
int ane_peak_read(const void* src, uint64_t bytes, uint32_t wgs, int magic, int* hit,
                  hipStream_t stream) {
    if (!src || !hit || wgs == 0 || (bytes & 15) || ((uintptr_t)src & 15)) return -1;
    hipLaunchKernelGGL(k_read, dim3(wgs), dim3(256), 0, stream, static_cast<const v4i*>(src),
                       bytes / 16, magic, hit);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Writes `bytes` (a multiple of 16, 16-byte aligned) with `wgs` workgroups.
int ane_peak_write(void* dst, uint64_t bytes, uint32_t wgs, hipStream_t stream) {
    if (!dst || wgs == 0 || (bytes & 15) || ((uintptr_t)dst & 15)) return -1;
    hipLaunchKernelGGL(k_write, dim3(wgs), dim3(256), 0, stream, static_cast<v4i*>(dst), bytes / 16,
                       5);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // extern "C"
