/*
 * ane_decode.h -- single-token decode of a Llama-shaped model on MI355X with
 * every matrix product on the Q8_0 kernels of ane_hip.h (G mode).
 *
 * This is the driver around the GGML_OP_MUL_MAT hook: the steps on either
 * side of mul_mat in one decoder layer, as a ggml graph of a Llama model
 * runs them (the reference has SME kernels for these steps:
 * bytecode_interpreter.s:6508 rms_norm, 6617 silu, 6714 rope (adjacent
 * pairs, out[2i] = in[2i] cos - in[2i+1] sin), 11657 flash_attention; its
 * ggml backend routes MUL_MAT to the quantized path,
 * src/ggml-backend/ggml-ane.cpp:119-154):
 *
 *   qkv  = W_qkv . q8(rmsnorm(x) * attn_norm)       fused norm prologue
 *   attn = softmax(rope(q) rope(k)^T / sqrt(d)) v over positions 0..pos (GQA),
 *          k, v of pos appended to the fp16 cache      one fused kernel + combine,
 *                                                    which also emits q8(attn)
 *   x    = x + W_o . q8(attn)                        fused residual epilogue
 *   h    = q8(silu(gate) * up), gate|up = W_gate_up . q8(rmsnorm(x) * ffn_norm)
 *                                                    fused norm prologue and
 *                                                    SiLU/quantize epilogue
 *   x    = x + W_down . h                            fused residual epilogue
 *
 * q8(v) is the Q8 activation form of the G mode: per 32-block, amax/127 as
 * the fp32 scale and the values rounded to int8 (bytecode_interpreter.s
 * 0x19 arithmetic), stored as qx [K/32][32] int8 followed by dx [K/32] fp32.
 *
 * Layouts: weights are Q8_0 rows (ggml block layout) with the output
 * features as rows: W_qkv rows [q heads | k heads | v heads], W_gate_up rows
 * gate and up interleaved in groups of 32 (gate 0..31, up 0..31, gate
 * 32..63, up 32..63, ...), so that one workgroup owns both halves of every
 * 32-value block of SiLU(gate) * up.  KV cache: fp16 [n_kv_heads][ctx][head_dim].  RoPE table:
 * fp32 [ctx][head_dim/2][2] = (cos, sin) of pos * base^(-2i/head_dim),
 * applied to adjacent pairs (x[2i], x[2i+1]).  All pointers are device
 * memory; the layer array itself is host memory.
 */
#ifndef ANE_DECODE_H
#define ANE_DECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

struct ane_decode_config {
    uint32_t n_layers;
    uint32_t hidden;      /* model width (4096; a multiple of 256)         */
    uint32_t ffn;         /* feed-forward width (14336; a multiple of 256) */
    uint32_t n_heads;     /* query heads (32)                   */
    uint32_t n_kv_heads;  /* key/value heads (8)                */
    uint32_t head_dim;    /* 128 (the only supported value)     */
    uint32_t ctx;         /* KV cache capacity in positions (at most 2^20) */
    float eps;            /* RMSNorm epsilon                    */
};

struct ane_decode_layer {
    const void* w_qkv;      /* Q8_0 [(n_heads + 2 n_kv_heads) head_dim][hidden] */
    const void* w_o;        /* Q8_0 [hidden][n_heads head_dim]                  */
    const void* w_gate_up;  /* Q8_0 [2 ffn][hidden], gate/up in 32-row groups    */
    const void* w_down;     /* Q8_0 [hidden][ffn]                               */
    const float* attn_norm; /* [hidden]                                         */
    const float* ffn_norm;  /* [hidden]                                         */
    uint16_t* k_cache;      /* fp16 [n_kv_heads][ctx][head_dim]                 */
    uint16_t* v_cache;      /* fp16 [n_kv_heads][ctx][head_dim]                 */
};

/* Device workspace bytes for ane_decode_token (256-byte aligned sections). */
size_t ane_decode_workspace_size(const struct ane_decode_config* cfg);

/* One token at position pos (< ctx) through every layer: x (fp32 [hidden],
 * the residual stream) is updated in place, and k/v of pos are written into
 * each layer's cache; positions 0..pos of the caches are attended to.
 * Every step's preconditions are checked before the first launch (weights
 * 16-byte aligned, the products' LDS and rows-per-wave limits), so an error
 * return leaves x and the caches untouched.
 * Asynchronous on stream; returns an ane_status. */
int ane_decode_token(const struct ane_decode_config* cfg, const struct ane_decode_layer* layers,
                     const float* rope_table, uint32_t pos, float* x, void* workspace,
                     size_t workspace_bytes, void* stream);

/* The steps of ane_decode_token, for tests and for callers that schedule
 * them differently.  All asynchronous on stream. */

/* Q8_0 matvec (G mode, one token) with optional fusions: norm_w != NULL
 * applies x' = x * inv_rms(x) * norm_w before quantizing (inv_rms =
 * 1/sqrt(fl(fl(sum x^2 / K) + eps)), sum in fp64); residual != NULL adds
 * residual[n] to each output (residual may equal y). */
int ane_hip_q8_0_matvec_fused(uint32_t N, uint32_t K, const float* x, const float* norm_w, float eps,
                              const void* W, const float* residual, float* y, void* stream);

/* y = W . xq (+ residual) with xq already in the Q8 activation form (16-byte
 * aligned, K/32 * 36 bytes); bit-identical to ane_hip_q8_0_matvec_fused on
 * the fp32 vector xq was quantized from. */
int ane_hip_q8_0_matvec_q8(uint32_t N, uint32_t K, const void* xq, const void* W, const float* residual,
                           float* y, void* stream);

/* The gate|up product with SiLU*up fused into its epilogue: W has 2F rows,
 * gate and up interleaved in 32-row groups (rows 64k..64k+31 = gate rows
 * 32k.., rows 64k+32..64k+63 = up rows 32k..); with g|u = W . q8(rmsnorm(x)
 * * norm_w) (as ane_hip_q8_0_matvec_fused), xq = q8(silu(g) * u) in the Q8
 * activation form (F/32 * 36 bytes, 16-byte aligned, F % 32 == 0):
 * bit-identical to ane_hip_q8_0_matvec_fused + ane_hip_silu_mul_quant on
 * the de-interleaved output. */
int ane_hip_q8_0_gate_up_silu_quant(uint32_t F, uint32_t K, const float* x, const float* norm_w, float eps,
                                    const void* W, void* xq, void* stream);

/* y = W . q8(silu(gu[0..K)) * gu[K..2K)) (+ residual), silu(g) = g / (1 + e^-g):
 * the down projection with SiLU * up fused into its activation prologue;
 * bit-identical to ane_hip_silu_mul followed by ane_hip_q8_0_matvec_fused. */
int ane_hip_q8_0_matvec_silu(uint32_t N, uint32_t K, const float* gu, const void* W, const float* residual,
                             float* y, void* stream);

/* RoPE on the q and k heads of qkv (in place for q), then k and v of this
 * position converted to fp16 into the caches. */
int ane_hip_rope_kv_append(const struct ane_decode_config* cfg, float* qkv, const float* rope_table,
                           uint32_t pos, uint16_t* k_cache, uint16_t* v_cache, void* stream);

/* out[h] = softmax(q[h] . K[g]^T / sqrt(head_dim)) V[g] over positions
 * 0..len-1, g = h / (n_heads / n_kv_heads).  q: fp32 [n_heads][head_dim].
 * Two launches: per (kv head, chunk of the context) partial results, then a
 * merge per query head. */
size_t ane_hip_attention_workspace_size(const struct ane_decode_config* cfg);
int ane_hip_attention_decode(const struct ane_decode_config* cfg, const float* q, const uint16_t* k_cache,
                             const uint16_t* v_cache, uint32_t len, float* out, void* workspace,
                             size_t workspace_bytes, void* stream);

/* ane_hip_attention_decode at len = pos + 1 on unrotated q and k: RoPE of q
 * and k (as ane_hip_rope_kv_append) and the fp16 append of k and v at pos
 * happen inside the attention kernel; same results, one launch fewer.
 * out_q8 (optional, 16-byte aligned): out in the Q8 activation form too. */
int ane_hip_attention_decode_rope(const struct ane_decode_config* cfg, const float* qkv, const float* rope_table,
                                  uint32_t pos, uint16_t* k_cache, uint16_t* v_cache, float* out, void* out_q8,
                                  void* workspace, size_t workspace_bytes, void* stream);

/* h[i] = silu(gu[i]) * gu[n + i], i < n. */
int ane_hip_silu_mul(uint32_t n, const float* gu, float* h, void* stream);

/* xq = q8(h) for h as ane_hip_silu_mul computes it (n % 32 == 0, xq 16-byte
 * aligned, n/32 * 36 bytes). */
int ane_hip_silu_mul_quant(uint32_t n, const float* gu, void* xq, void* stream);

/* The build's RMSNorm on its own, one row: out = fl(fl(x * inv) * w),
 * inv = 1/sqrtf((float)(ss / K) + eps) with ss the fp64 sum of squares in
 * the fixed order the fused products use, so the output is bit-identical to
 * the normalised activation those kernels quantize.  K % 32 == 0,
 * K <= 2^19, x 16-byte aligned. */
int ane_hip_rms_norm(uint32_t K, const float* x, const float* w, float eps, float* out, void* stream);

/* out = fl(a + b), n elements (out may alias a or b). */
int ane_hip_add_fp32(uint32_t n, const float* a, const float* b, float* out, void* stream);

/* The reference's decode-step handlers in their exact fp32 operation
 * sequence (bytecode_interpreter.s; the estimates per the Arm ARM
 * pseudocode of FRSQRTE / FRECPE):
 *   0x51 rms_norm_fp32 (:6508-6565): rows x dim, out may alias in;
 *   0x54 silu_fp32     (:6617-6713): count elements;
 *   0x55 rope_fp32     (:6714-6912): rows x dim (each row rotated at pos,
 *        adjacent pairs, ratio theta^(2/dim));
 *   0x56 softmax_fp32  (:6913-7009): rows x dim, out may alias in.
 * The handlers loop in 16-lane vectors with no tail, so stream_exec refuses
 * dim % 16 != 0 for 0x51, 0x54 and 0x56; these kernel entries accept any
 * dim, a short last vector contributing nothing (identical for multiples
 * of 16). */
int ane_hip_rms_norm_fp32(uint32_t rows, uint32_t dim, float eps, const float* in, const float* w, float* out,
                          void* stream);
int ane_hip_silu_fp32(uint64_t count, const float* in, float* out, void* stream);
int ane_hip_rope_fp32(uint32_t rows, uint32_t dim, uint32_t pos, float theta, const float* in, float* out,
                      void* stream);
int ane_hip_softmax_fp32(uint32_t rows, uint32_t dim, const float* in, float* out, void* stream);

/* One token through the ggml backend (include/ggml-ane-hip.h): each layer's
 * four products are GGML_OP_MUL_MAT nodes computed by
 * ane_ggml_compute_forward on the backend's stream, with the steps around
 * them as separate kernels.
 *   ANE_DECODE_ARITH_BUILD: the products in G mode and the steps in the
 *     arithmetic of ane_decode_token (canonical fp64 RMSNorm, the RoPE table,
 *     the chunked attention, expf SiLU): x and the caches come out
 *     bit-identical to ane_decode_token's;
 *   ANE_DECODE_ARITH_REFERENCE: the products in R mode (opcode 0x57, what the
 *     reference hook runs) and the steps in the handlers' arithmetic:
 *     rms_norm_fp32, rope_fp32 at rope_theta on q and k (dim 128), an
 *     attention of 16-lane fma dot products scaled by fl(1/sqrt(128)),
 *     softmax_fp32 over positions 0..pos and 16-lane fma sums over the
 *     values, silu_fp32 times up, fp32 residual adds.
 * Sets the backend's Q8_0 mode accordingly.  x 16-byte aligned; workspace
 * from ane_decode_ggml_workspace_size (256-byte aligned).  Asynchronous. */
#define ANE_DECODE_ARITH_BUILD 0
#define ANE_DECODE_ARITH_REFERENCE 1
struct ane_ggml_backend;
size_t ane_decode_ggml_workspace_size(const struct ane_decode_config* cfg);
int ane_decode_token_ggml(const struct ane_decode_config* cfg, const struct ane_decode_layer* layers,
                          const float* rope_table, float rope_theta, uint32_t pos, float* x, void* workspace,
                          size_t workspace_bytes, struct ane_ggml_backend* backend, int arith);

#ifdef __cplusplus
}
#endif

#endif /* ANE_DECODE_H */
