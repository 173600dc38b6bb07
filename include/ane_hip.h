/*
 * ane_hip.h -- C ABI of the MI355X (gfx950) implementation of ane's
 * quantized compute path.
 *
 * Two layers, both exported by ane_amd/libane_amd.so:
 *
 *  1. The reference's own boundary: stream_exec(), the single entry point
 *     that ane::dispatch() serialises into (reference include/ane/ane.hpp:37-39,
 *     exported by src/bytecode_interpreter.s:11-12 as _stream_exec).  Same
 *     record layouts, same opcode numbers.  Operands are device pointers
 *     (hipMalloc / hipMallocManaged / hipHostMalloc); the call is synchronous
 *     like the reference's, and failures are reported through
 *     ane_last_error() because the reference signature returns void.
 *     Each operand's extent is checked against the HIP allocation that holds
 *     it.  That is per allocation, not per tensor: a caching allocator (such
 *     as torch's) carves many tensors out of one allocation, and a short
 *     tensor inside it passes the check (the Python records check tensor
 *     extents themselves before encoding).
 *
 *  2. The kernel-level ABI (ane_hip_*): device pointers, an explicit HIP
 *     stream (hipStream_t passed as void*, 0 = the null stream), an int
 *     status return (ANE_OK == 0), asynchronous with respect to the host.
 *     Entry points that need scratch memory take a caller-owned workspace
 *     (size from the matching *_workspace_size function) and never allocate.
 *
 * All functions are thread-safe.  Nothing here allocates device memory
 * except stream_exec (a grow-only per-device workspace for the opcodes that
 * need one, freed at process exit).
 */
#ifndef ANE_HIP_H
#define ANE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status */
enum ane_status {
    ANE_OK = 0,
    ANE_ERR_INVALID_ARG = 1,      /* shape/size outside the documented range  */
    ANE_ERR_BAD_POINTER = 2,      /* null or not device-accessible            */
    ANE_ERR_BUFFER_TOO_SMALL = 3, /* operand extent exceeds its allocation    */
    ANE_ERR_UNKNOWN_OPCODE = 4,   /* opcode this build does not implement     */
    ANE_ERR_TRUNCATED = 5,        /* record runs past the end of the stream   */
    ANE_ERR_HIP = 6,              /* a HIP runtime call failed                */
    ANE_ERR_NO_DEVICE = 7,        /* no gfx950 device                         */
    ANE_ERR_WORKSPACE = 8,        /* workspace pointer null or too small      */
    ANE_ERR_GRID_WAIT = 9         /* dense_fused_i8's grid-wide wait failed:  */
                                  /* its outputs are not valid                */
};

/* Opcodes served by this build (values identical to the reference's
 * enum class ane::Op, include/ane/ane.hpp:47-177, plus dense_fused_i8). */
#define ANE_OP_DENSE_I8 0x18
#define ANE_OP_QUANTIZE_FP32_I8 0x19
#define ANE_OP_DEQUANTIZE_I8_FP32 0x1A
#define ANE_OP_PACK_B_I8 0x1B
#define ANE_OP_QUANTIZE_FP32_I8_CHANNELWISE 0x1C
#define ANE_OP_DENSE_U8S8 0x1E
#define ANE_OP_RMS_NORM_FP32 0x51 /* declared in ane_decode.h with 0x54-0x56 */
#define ANE_OP_SILU_FP32 0x54
#define ANE_OP_ROPE_FP32 0x55
#define ANE_OP_SOFTMAX_FP32 0x56
#define ANE_OP_Q8_0_GEMV 0x57
#define ANE_OP_Q4_0_GEMV 0x58
#define ANE_OP_CBLAS_IGEMM 0x61
#define ANE_OP_CBLAS_UGEMM 0x62
#define ANE_OP_CBLAS_USGEMM 0x63
#define ANE_OP_Q4_K_GEMV 0x75
#define ANE_OP_Q2_K_GEMV 0x76
#define ANE_OP_Q3_K_GEMV 0x77
#define ANE_OP_Q5_K_GEMV 0x78
#define ANE_OP_Q6_K_GEMV 0x79
#define ANE_OP_GET_ROWS_Q8_0 0x7C
#define ANE_OP_GET_ROWS_Q4_0 0x7D
#define ANE_OP_DENSE_FUSED_I8 0x80 /* README.md:84-97; absent from the reference enum */

/* ------------------------------------------------- reference boundary */

/* Replaces extern "C" void stream_exec(const uint8_t*, size_t)
 * (reference include/ane/ane.hpp:37-39; bytecode_interpreter.s:11-36).
 * Decodes and runs every record of the stream on the calling thread's
 * stream (ane_set_stream), then synchronises it.  Stops at the first failing
 * record; ane_last_error() reports why (ANE_OK after a full run). */
void stream_exec(const uint8_t* data, size_t size);

/* Status of the last stream_exec on this thread, and a human-readable
 * message for it.  No reference counterpart (the reference validates
 * nothing: bytecode_interpreter.s:31-36). */
int ane_last_error(void);
const char* ane_last_error_message(void);

/* Stream used by stream_exec on this thread (void* = hipStream_t). */
void ane_set_stream(void* stream);

/* Host staging for stream_exec on this thread: 1 on, 0 off, -1 (the
 * default) follows the environment variable ANE_HOST_STAGING (on when set
 * to anything but "" or "0").  With staging on, an operand in plain host
 * memory (malloc, aligned_alloc, a stack array: the reference's callers,
 * tests/test_mnist_i8.cpp) is copied to a device staging buffer, the record
 * runs on the copy, and its outputs are copied back before the record
 * returns; records with staged operands are synchronous also under
 * ane_stream_exec_async.  With staging off, such an operand is refused
 * (ANE_ERR_BAD_POINTER).  Device memory is never staged.  No reference
 * counterpart: the reference reads and writes host memory directly. */
void ane_set_host_staging(int mode);

/* stream_exec without the final synchronisation and with an explicit
 * stream; returns the status instead of storing it.  Host-memory scalar
 * outputs (quantize scale_out, channelwise scales) still synchronise. */
int ane_stream_exec_async(const uint8_t* data, size_t size, void* stream);

/* ------------------------------------------------- kernel-level ABI */

/* 0x19 quantize_fp32_i8 (bytecode_interpreter.s:1876-1950).
 * Processes n = pad16 ? max(16, ceil16(count)) : count elements.
 * scale_out is a device pointer. */
size_t ane_hip_quantize_workspace_size(uint64_t n);
int ane_hip_quantize_fp32_i8(uint64_t count, int pad16, const float* src,
                             int8_t* dst, float* scale_out, void* workspace,
                             size_t workspace_bytes, void* stream);

/* 0x1A dequantize_i8_fp32 (bytecode_interpreter.s:1951-1977):
 * dst[i] = (float)src[i] * scale, i < ceil16(count). */
int ane_hip_dequantize_i8_fp32(uint64_t count, float scale, const int8_t* src,
                               float* dst, void* stream);

/* 0x1C quantize_fp32_i8_channelwise (bytecode_interpreter.s:2583-2662):
 * rows of width/stride cpad = max(16, ceil16(cols)). */
int ane_hip_quantize_channelwise(uint32_t rows, uint32_t cols, const float* src,
                                 int8_t* dst, float* scales, void* stream);

/* 0x1B pack_b_i8 (bytecode_interpreter.s:2447-2582): K x N row-major int8 ->
 * SMOPA panel format of ane_hip_packed_b_size(K, N) bytes. */
size_t ane_hip_packed_b_size(uint32_t K, uint32_t N);
int ane_hip_pack_b_i8(uint32_t K, uint32_t N, const int8_t* src, int8_t* dst,
                      void* stream);

/* 0x18 dense_i8 / 0x1E dense_u8s8 (bytecode_interpreter.s:1978-2446,
 * 2835-3300).  A: int8 (a_unsigned = 0) or uint8 (1), max(16,ceil16(M)) rows
 * of Kp = ceil64(K) bytes; Bp from pack_b_i8(Kp, N); bias fp32[N];
 * C fp32 rows 0 .. max(16, ceil16(M))-1, columns < N, row stride N. */
int ane_hip_dense_i8(uint32_t M, uint32_t N, uint32_t K, float sa, float sb,
                     uint8_t flags, const void* A, const int8_t* Bp,
                     const float* bias, float* C, int a_unsigned, void* stream);

/* Op::dense_fused_i8 (README.md:84-97; the reference defines no handler):
 * fp32 A (M x K, stride K) and B (K x N, stride N) each quantized per tensor
 * with the 0x19 arithmetic, int8 x int8 -> int32 on MFMA, then
 * C = fmaxA((float)acc * ((sa*sb)*scale) + 0.0f, relu ? +0 : -FLT_MAX).
 * Writes exactly M x N.  Optional outputs (may be null): the quantized
 * operands' scales (device float[2] = {sa, sb}).  The workspace is scratch:
 * small shapes (K <= 1024, at most 512 tiles of 16 x 16 in C) quantize
 * straight into each tile's LDS, and so do shapes with at most 16 rows of A
 * (K % 512 == 0, K <= 4096, N % 16 == 0, at most one 16-column strip of B
 * per CU, at least 12 MiB of B, 16-byte aligned A and B: one launch with
 * the grid-wide wait described below); both leave the workspace's
 * quantized-operand area unwritten; ane_hip_dense_fused_i8_quantize always
 * writes it. */
size_t ane_hip_dense_fused_i8_workspace_size(int32_t M, int32_t N, int32_t K);
int ane_hip_dense_fused_i8(int32_t M, int32_t N, int32_t K, float scale,
                           int relu, const float* A, const float* B, float* C,
                           float* scales_out, void* workspace,
                           size_t workspace_bytes, void* stream);

/* The operand quantizer of dense_fused_i8 runs, for large shapes (K % 128
 * == 0, N % 64 == 0, at least 12 MiB of operands), as one launch whose
 * workgroups (one per CU) exchange their maxima through a grid-wide wait;
 * so does the whole op at up to 16 rows (the strip route above), and what
 * follows applies to both.
 * Outside stream capture it is a cooperative launch: the runtime starts it
 * only with every workgroup resident, or refuses it and the two-pass route
 * (no wait) runs instead.  Under capture it is a plain launch.  Two such
 * launches must not run at once on one device (each needs every CU): calls
 * on different streams are ordered by the library (a call waits for the
 * previous call's launch), and under capture the route is taken only on the
 * stream of the previous call.  Replays of captured graphs are not ordered
 * by the library: a replay that overlaps another replay or an eager call on
 * another stream makes the waits of both either time out or count each
 * other's arrivals.  Neither is silent: the wait is bounded (2 s by
 * default), every launch is tagged, and a counter completed by arrivals of
 * two launches is detected; the outputs of such a call are not valid, and
 * the status calls below report it (ANE_ERR_GRID_WAIT).
 *
 * ane_hip_dense_fused_i8_status(workspace, stream) synchronizes the stream
 * and reports the last quantize call made with this workspace: every such
 * call writes a wait record into the workspace (one word per workgroup),
 * which this reads; it also reads, and clears, the device's record of
 * counters completed by mixed arrivals, which a call whose wait another
 * launch completed cannot see in its own record.  ANE_ERR_INVALID_ARG: no
 * quantize call has written this workspace.
 * ane_hip_grid_wait_status(stream) synchronizes the stream and returns
 * ANE_ERR_GRID_WAIT (and clears the device's record) if any such launch on
 * the current device gave up or saw mixed arrivals since the last call, else
 * ANE_OK; stream_exec checks it itself.  After a failure the device's
 * counters are returned to rest once the device is idle.
 * ane_hip_set_grid_wait_limit sets the bound, in ticks of the 100 MHz
 * realtime counter, for launches made after it (0: the default, 2 s). */
int ane_hip_dense_fused_i8_status(const void* workspace, void* stream);
int ane_hip_grid_wait_status(void* stream);
void ane_hip_set_grid_wait_limit(uint64_t ticks);

/* The two phases of ane_hip_dense_fused_i8, for callers that quantize an
 * operand pair once and run the contraction repeatedly (the reference's own
 * quantize-once / reuse pattern, tests/test_mnist_i8.cpp:198-207, 415):
 * _quantize writes both int8 operands and their scales into the workspace;
 * _gemm reads them from the same workspace and writes C. */
int ane_hip_dense_fused_i8_quantize(int32_t M, int32_t N, int32_t K,
                                    const float* A, const float* B,
                                    float* scales_out, void* workspace,
                                    size_t workspace_bytes, void* stream);
int ane_hip_dense_fused_i8_gemm(int32_t M, int32_t N, int32_t K, float scale,
                                int relu, float* C, const void* workspace,
                                size_t workspace_bytes, void* stream);

/* Raw int32 accumulators of the int8 MFMA contraction (test/debug entry):
 * acc[i*N+j] = sum_{k<K} A[i*lda+k] * Bt[j*ldb+k], wrapping int32.
 * A and Bt are int8 row-major with K contiguous. */
int ane_hip_gemm_s8_i32(uint32_t M, uint32_t N, uint32_t K, const int8_t* A,
                        uint32_t lda, const int8_t* Bt, uint32_t ldb,
                        int32_t* acc, void* stream);

/* 0x61 cblas_igemm / 0x62 cblas_ugemm / 0x63 cblas_usgemm
 * (bytecode_interpreter.s:8328-9139, the CBLAS_INTEGER_GEMM macro):
 * A and B int8 (variant SIGNED), uint8 (UNSIGNED) or uint8 A x int8 B
 * (MIXED); C fp32, rows < M and columns < N written with stride ldc >= N;
 * flags bit 0 transA, bit 1 transB; only K/64 whole blocks of K are used.
 * semantics ANE_IGEMM_REFERENCE reproduces the handler: C = fl(fl32(acc) *
 * alpha), where acc starts from the bit pattern of fl(beta * C) when beta's
 * bits are nonzero (:8402-8488), and with transA output row i reads
 * A[(i%16)*lda + (i - i%16) + k] (:8513-8514) -- this is what stream_exec
 * runs for the opcodes.  ANE_IGEMM_BLAS computes the documented form instead:
 * op(A) = A^T (A is K x M, stride lda) with transA, and
 * C = fl(fl(fl32(acc) * alpha) + fl(beta * C)), C not read when beta == 0.
 * Accumulation wraps modulo 2^32 in both. */
#define ANE_IGEMM_SIGNED 0
#define ANE_IGEMM_UNSIGNED 1
#define ANE_IGEMM_MIXED 2
#define ANE_IGEMM_REFERENCE 0
#define ANE_IGEMM_BLAS 1
size_t ane_hip_cblas_igemm_workspace_size(uint32_t M, uint32_t N, uint32_t K);
int ane_hip_cblas_igemm(int variant, int semantics, uint8_t flags, uint32_t M, uint32_t N,
                        uint32_t K, uint32_t lda, uint32_t ldb, uint32_t ldc, float alpha,
                        float beta, const void* A, const void* B, float* C, void* workspace,
                        size_t workspace_bytes, void* stream);

/* 0x57 q8_0_gemv "R mode" (bytecode_interpreter.s:7010-7063): fp32 x,
 * y[m] = FADDV16 of 16 fma lanes, bit-identical to the reference's
 * arithmetic.  W: M rows of (K/32) 34-byte blocks. */
int ane_hip_q8_0_gemv(uint32_t M, uint32_t K, const float* x, const void* W,
                      float* y, void* stream);

/* q8_0 "G mode" (x quantized to Q8_0 per 32-block on the fly, int8 dots):
 * y[t*N+m] for T tokens of x (T x K fp32).  Workspace holds the quantized
 * activations.  Serves the ggml GGML_OP_MUL_MAT hook
 * (reference src/ggml-backend/ggml-ane.cpp:119-154) for all ne11 tokens. */
size_t ane_hip_q8_0_mul_mat_workspace_size(uint32_t K, uint32_t T);
int ane_hip_q8_0_mul_mat(uint32_t N, uint32_t K, uint32_t T, const float* x,
                         const void* W, float* y, void* workspace,
                         size_t workspace_bytes, void* stream);
/* The workspace for every route of an N-row matrix: at 5+ tokens on
 * matrices with few rows (fewer than 4 x 16 rows per CU) and rows of 256+
 * blocks, where the activation-stationary kernel does not take the shape
 * (e.g. 17+ tokens at K = 14336), the fastest kernel splits each 64-row
 * group's block residues over four workgroups and keeps their subtotals
 * (4 x T x N fp32) in the workspace.  A workspace of
 * ane_hip_q8_0_mul_mat_workspace_size(K, T) bytes is still valid: that
 * route is then not taken.  The result is bit-identical either way. */
size_t ane_hip_q8_0_mul_mat_workspace_size_n(uint32_t N, uint32_t K, uint32_t T);

/* ane_hip_q8_0_mul_mat without a workspace argument and without allocating:
 * the quantized activations live in a static device array of
 * ane_hip_q8_0_mul_mat_noalloc_max_bytes() bytes (4 MiB; one per device,
 * held until the process ends).  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc).  Shapes whose
 * ane_hip_q8_0_mul_mat_workspace_size(K, T) exceeds that size return
 * ANE_ERR_WORKSPACE.  All calls on one device share the array: calls that
 * overlap on one device (two streams, two threads) race.  Results are
 * bit-identical to ane_hip_q8_0_mul_mat. */
size_t ane_hip_q8_0_mul_mat_noalloc_max_bytes(void);
int ane_hip_q8_0_mul_mat_noalloc(uint32_t N, uint32_t K, uint32_t T, const float* x,
                                 const void* W, float* y, void* stream);

/* The other weight formats, "R mode" like 0x57: fp32 x, y[m] = FADDV16 of
 * the handler's 16 fma lanes, bit-identical to the reference's arithmetic.
 * W: M rows of K/values blocks, any alignment; a remainder of K is ignored
 * as the handlers ignore it.
 *   0x58 q4_0_gemv  bytecode_interpreter.s:7071-7126  18-byte blocks of 32
 *   0x75 q4_k_gemv  :11024-11131  144-byte super-blocks of 256
 *   0x76 q2_k_gemv  :11146-11222  84
 *   0x77 q3_k_gemv  :11236-11358  110 (the second half of each sub-block
 *        decodes its 2-bit fields from the qs word shifted right by the bit
 *        pattern of the matching first-half input, as the handler does,
 *        :11323-11329: no shift for +0.0, zero fields for normal inputs)
 *   0x78 q5_k_gemv  :11372-11483  176
 *   0x79 q6_k_gemv  :11498-11626  210 */
int ane_hip_q4_0_gemv(uint32_t M, uint32_t K, const float* x, const void* W, float* y, void* stream);
int ane_hip_q4_k_gemv(uint32_t M, uint32_t K, const float* x, const void* W, float* y, void* stream);
int ane_hip_q2_k_gemv(uint32_t M, uint32_t K, const float* x, const void* W, float* y, void* stream);
int ane_hip_q3_k_gemv(uint32_t M, uint32_t K, const float* x, const void* W, float* y, void* stream);
int ane_hip_q5_k_gemv(uint32_t M, uint32_t K, const float* x, const void* W, float* y, void* stream);
int ane_hip_q6_k_gemv(uint32_t M, uint32_t K, const float* x, const void* W, float* y, void* stream);

/* 0x7C get_rows_q8_0 / 0x7D get_rows_q4_0 (bytecode_interpreter.s:12363-12408,
 * 12419-12469): out row r (dim fp32, rows contiguous) = table row indices[r]
 * dequantized.  dim % 32 == 0.  table_rows bounds the indices (the reference
 * reads past its table instead): a row whose index is >= table_rows is
 * written as zeros. */
int ane_hip_get_rows_q8_0(uint32_t n_rows, uint32_t dim, const void* table, uint64_t table_rows,
                          const uint32_t* indices, float* out, void* stream);
int ane_hip_get_rows_q4_0(uint32_t n_rows, uint32_t dim, const void* table, uint64_t table_rows,
                          const uint32_t* indices, float* out, void* stream);

/* Library/device information: returns ANE_OK if a gfx950 device is usable. */
int ane_hip_device_check(void);
const char* ane_hip_version(void);

#ifdef __cplusplus
}
#endif
#endif /* ANE_HIP_H */
