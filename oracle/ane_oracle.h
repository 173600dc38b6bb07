/*
 * ane_oracle.h -- CPU restatement of ane's quantized compute path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker the GPU path is compared
 * against (and the timed CPU baseline in bench.py).  The product library
 * (ane_amd/libane_amd.so) never links, loads or calls anything here; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may.
 *
 * Every function restates one opcode handler of the reference's
 * src/bytecode_interpreter.s (AArch64 SME2 assembly, which cannot be built
 * or run on this x86/amdgcn toolchain) in scalar C, with the same IEEE
 * binary32 operation sequence.  Citations are file:line in the reference.
 *
 * Pinning (what fixes each function independently of this restatement):
 *   quantize_fp32_i8 / channelwise / dequantize : tests/test_oracle.py
 *       numpy float32 restatement, the reference KAT
 *       tests/test_dsl_coverage.cpp:334-368 (x=(i-128)*0.1, err<1.5*scale),
 *       closed forms (sign symmetry, |q|<=127, amax element -> +-127).
 *   pack_b_i8      : brute-force index permutation on tiny shapes + the
 *       inverse map (unpack(pack(B)) == B, zero padding).
 *   dense_i8 / u8s8 / gemm_s8_i32 : exact int64 numpy matmul, the reference
 *       KATs test_remaining_ops.cpp:131-184 (A=(i%11)-5, B=(i%13)-6) and
 *       test_dsl_coverage.cpp:240-260 / test_program_demo.cpp:148-178
 *       (all-ones -> 4 and 16); epilogue = three float32 numpy ops.
 *   dense_fused_i8 : composition of the above; equals the reference's own
 *       composition quantize->pack_b_i8->dense_i8 (test_mnist_i8.cpp:198-207,
 *       303-314) at scale 1.0 (checked in tests).
 *   q8_0_gemv (R)  : block layout pinned by test_remaining_ops.cpp:230-325
 *       (get_rows_q8_0); FADDV tree and fma pinned by closed-form cases
 *       (one-hot x, power-of-two data that makes every sum exact, and a
 *       tree-order case whose sequential sum differs).
 *   cblas_igemm / ugemm / usgemm : the reference KAT
 *       test_remaining_ops.cpp:131-184 (16x32x64, alpha 1 and 0.5, beta 0),
 *       exact int64 numpy products of s8/u8 operands for every variant and
 *       transB (transB = 1 equals transB = 0 on the transposed matrix).
 *       The handler-only behaviours (transA's row addressing, the beta
 *       bit-pattern seed) have no reference test: they are restated from the
 *       cited lines and checked against their closed forms (K < 64 leaves
 *       only the seed; beta = -0.0 seeds; transA on a matrix whose row i
 *       equals the addressed bytes).
 *   q8_0 G mode    : the build's own definition (the reference has no
 *       quantized-activation matvec); isum_b pinned exactly by integer
 *       numpy, combination order pinned by an independent numpy loop with
 *       exact fma (float64 product/sum then a single rounding).
 */
#ifndef ANE_ORACLE_H
#define ANE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Threads used by the row-parallel loops (OpenMP).  Returns the count in use. */
int oracle_set_threads(int n);

/* 0x19  bytecode_interpreter.s:1885-1950.  Reads and writes
 * n = max(16, ceil16(count)) elements (the handler is a do-while over
 * 16-lane vectors).  Writes *scale_out. */
void oracle_quantize_fp32_i8(uint32_t count, const float* src, int8_t* dst,
                             float* scale_out);

/* Same arithmetic over exactly n elements (used by dense_fused_i8 and the
 * Q8_0 activation quantizer). */
void oracle_quantize_exact(size_t n, const float* src, int8_t* dst,
                           float* scale_out);

/* 0x1A  bytecode_interpreter.s:1951-1977.  dst[i] = (float)src[i] * scale for
 * ceil16(count) elements (count == 0 -> nothing). */
void oracle_dequantize_i8_fp32(uint32_t count, float scale, const int8_t* src,
                               float* dst);

/* 0x1C  bytecode_interpreter.s:2583-2662.  Per row absmax quantize; row
 * stride and processed width are cpad = max(16, ceil16(cols)). */
void oracle_quantize_fp32_i8_channelwise(uint32_t rows, uint32_t cols,
                                         const float* src, int8_t* dst,
                                         float* scales);

/* 0x1B  bytecode_interpreter.s:2447-2582.  SMOPA panel format. */
size_t oracle_packed_b_size(uint32_t K, uint32_t N);
void oracle_pack_b_i8(uint32_t K, uint32_t N, const int8_t* src, int8_t* dst);

/* 0x18 / 0x1E  bytecode_interpreter.s:1978-2446 / 2835-3300.
 * a_unsigned = 0 -> dense_i8 (smopa), 1 -> dense_u8s8 (usmopa).
 * Writes rows 0 .. max(16, ceil16(M))-1, columns 0..N-1 of C (stride N). */
void oracle_dense_i8(uint32_t M, uint32_t N, uint32_t K, float sa, float sb,
                     uint8_t flags, const void* A, const int8_t* Bp,
                     const float* bias, float* C, int a_unsigned);

/* Raw int32 accumulators of the dense_i8 contraction (no epilogue) over the
 * logical region: acc[i*N+j] = sum_{k<K} A[i*lda+k] * B[k*ldb+j]
 * (A int8 row-major, B int8 K x N row-major), wrapping int32. */
void oracle_gemm_s8_i32(uint32_t M, uint32_t N, uint32_t K, const int8_t* A,
                        uint32_t lda, const int8_t* B, uint32_t ldb,
                        int32_t* acc);

/* README.md:84-97 Op::dense_fused_i8 (not implemented by the reference; the
 * build's definition): per-tensor absmax quantize of A (M*K) and B (K*N),
 * int32 contraction, C = fmaxA((float)acc * ((sa*sb)*scale) + 0.0f, lo). */
void oracle_dense_fused_i8(int32_t M, int32_t N, int32_t K, float scale,
                           int relu, const float* A, const float* B, float* C);

/* Rows [row0, row1) of dense_fused_i8 given already-quantized operands
 * (used by the bounded CPU-baseline sample). */
void oracle_dense_fused_rows(int32_t row0, int32_t row1, int32_t N, int32_t K,
                             float s, int relu, const int8_t* qA,
                             const int8_t* qB, float* C);

/* 0x57  bytecode_interpreter.s:7010-7063, "R mode": fp32 x, 16 fma lanes per
 * row, FADDV pairwise tree.  W rows are concatenated 34-byte Q8_0 blocks. */
void oracle_q8_0_gemv(uint32_t M, uint32_t K, const float* x,
                      const uint8_t* W, float* y);

/* "G mode" activation quantizer: each 32-element block of x quantized with
 * the 0x19 arithmetic (absmax, zero guard), scale kept in fp32. */
void oracle_q8_0_quantize_x(uint32_t K, const float* x, int8_t* qx, float* dx);

/* "G mode" multi-token matvec: for t < T, m < N:
 *   isum_b = sum_i qw[m,b,i] * qx[t,b,i]           (exact int32)
 *   p[b % 16] = fmaf((float)isum_b, d_w[m,b] * dx[t,b], p[b % 16])  b ascending
 *   y[t*N + m] = FADDV tree of p[0..15] (the 0x57 horizontal sum order)
 * x is T x K fp32 (row stride K), y is T x N fp32 (row stride N). */
void oracle_q8_0_mul_mat_g(uint32_t N, uint32_t K, uint32_t T, const float* x,
                           const uint8_t* W, float* y);

/* The other weight formats of the reference, all "R mode" (fp32 x, 16 fma
 * lanes per row in the handler's element order, FADDV tree), y[0..M):
 *   0x58 q4_0_gemv  bytecode_interpreter.s:7071-7126   18 B / 32 values
 *   0x75 q4_k_gemv  :11024-11131                        144 B / 256
 *   0x76 q2_k_gemv  :11146-11222                        84 B / 256
 *   0x77 q3_k_gemv  :11236-11358 (with the handler's second-half shift by
 *                   the first half's input bits, :11323-11329)   110 B / 256
 *   0x78 q5_k_gemv  :11372-11483                        176 B / 256
 *   0x79 q6_k_gemv  :11498-11626                        210 B / 256 */
void oracle_q4_0_gemv(uint32_t M, uint32_t K, const float* x, const uint8_t* W, float* y);
void oracle_q4_k_gemv(uint32_t M, uint32_t K, const float* x, const uint8_t* W, float* y);
void oracle_q2_k_gemv(uint32_t M, uint32_t K, const float* x, const uint8_t* W, float* y);
void oracle_q3_k_gemv(uint32_t M, uint32_t K, const float* x, const uint8_t* W, float* y);
void oracle_q5_k_gemv(uint32_t M, uint32_t K, const float* x, const uint8_t* W, float* y);
void oracle_q6_k_gemv(uint32_t M, uint32_t K, const float* x, const uint8_t* W, float* y);

/* 0x7C / 0x7D  bytecode_interpreter.s:12363-12408, 12419-12469: gather
 * n_rows rows (u32 indices) of a Q8_0 / Q4_0 table of dim-wide rows and
 * dequantize them to fp32, out rows contiguous. */
void oracle_get_rows_q8_0(uint32_t n_rows, uint32_t dim, const uint8_t* table, const uint32_t* indices,
                          float* out);
void oracle_get_rows_q4_0(uint32_t n_rows, uint32_t dim, const uint8_t* table, const uint32_t* indices,
                          float* out);

/* 0x61 / 0x62 / 0x63 cblas_igemm / cblas_ugemm / cblas_usgemm
 * (bytecode_interpreter.s:8328-9139): variant 0 = s8 x s8, 1 = u8 x u8,
 * 2 = u8 x s8; flags bit 0 transA, bit 1 transB; C fp32 rows < M, columns
 * < N, stride ldc, updated in place.  semantics 0 = the handler's
 * arithmetic (K/64 blocks; transA reads A[(i%16)*lda + i - i%16 + k]; a
 * nonzero beta seeds the int32 accumulator with the bits of fl(beta*C);
 * C = fl(fl32(acc) * alpha)); semantics 1 = the BLAS form its header
 * describes (op(A) = A^T; C = fl(fl(fl32(acc)*alpha) + fl(beta*C)), C not
 * read when beta == 0). */
void oracle_cblas_igemm(int variant, int semantics, uint8_t flags, uint32_t M, uint32_t N, uint32_t K,
                        uint32_t lda, uint32_t ldb, uint32_t ldc, float alpha, float beta, const void* A,
                        const void* B, float* C);

/* The decode-step handlers in their exact fp32 sequence
 * (bytecode_interpreter.s:6508-7009), with FRSQRTE / FRECPE from the Arm
 * ARM pseudocode (FPRSqrtEstimate, FPRecipEstimate; FPCR.AH = 0):
 *   0x51 rms_norm_fp32  :6508-6565  dim % 16 == 0
 *   0x54 silu_fp32      :6617-6713
 *   0x55 rope_fp32      :6714-6912  adjacent pairs, ratio theta^(2/dim)
 *   0x56 softmax_fp32   :6913-7009  (dim % 16 != 0: absent lanes add nothing)
 * oracle_frsqrte / oracle_frecpe expose the two estimates. */
float oracle_frsqrte(float x);
float oracle_frecpe(float x);
void oracle_rms_norm_fp32(uint32_t dim, float eps, const float* in, const float* w, float* out);
void oracle_silu_fp32(uint32_t count, const float* in, float* out);
void oracle_rope_fp32(uint32_t dim, uint32_t pos, float theta, const float* in, float* out);
void oracle_softmax_fp32(uint32_t dim, const float* in, float* out);

/* The build's RMSNorm (fused decode kernels, ane_hip_rms_norm): fp64 sum of
 * squares in a fixed canonical order, inv = 1/sqrtf((float)(ss/K) + eps),
 * out = fl(fl(x*inv)*w). */
void oracle_rms_norm_build(uint32_t K, float eps, const float* x, const float* w, float* out);

/* Reference-arithmetic decode attention: scores fl(dot16(q, k_j) * fl(1/sqrt(128))),
 * softmax_fp32, then 16-lane fma chains over positions and FADDV. */
void oracle_attention_ref(uint32_t n_heads, uint32_t n_kv, uint32_t len, uint32_t ctx, const float* q,
                          const uint16_t* kc, const uint16_t* vc, float* out);

/* IEEE half -> float (exact), as fcvt s, h. */
float oracle_f16_to_f32(uint16_t h);

#ifdef __cplusplus
}
#endif
#endif /* ANE_ORACLE_H */
