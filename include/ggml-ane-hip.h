/*
 * ggml-ane-hip.h -- the ggml backend side of ane's quantized path on MI355X.
 *
 * The reference ships a ggml backend (src/ggml-backend/ggml-ane.h:20,
 * ggml-ane.cpp) whose GGML_OP_MUL_MAT hook sends Q8_0 and Q4_0 weights to
 * q8_0_gemv / q4_0_gemv (ggml-ane.cpp:119-154) and whose other hooks run
 * ADD, MUL, SCALE, RMS_NORM, SOFT_MAX, SILU, ROPE and CPY/CONT/DUP on fp32
 * tensors (ggml-ane.cpp:155-277).  ggml itself is not vendored there and no
 * version is pinned, so this header declares the minimal ggml subset the
 * hooks read.  Field names and meanings follow ggml's ggml_tensor: ne[]
 * element counts and nb[] byte strides, innermost first, op_params as ggml
 * packs them per op; type values follow ggml's on-disk enum ggml_type.  It
 * is an API-level shim: a maintainer plugging this backend into a real ggml
 * build copies ggml_tensor's ne/nb/type/op_params/data/src into these
 * fields per node and translates the op (ane_amd/ggml/ggml-ane.cpp does).
 *
 * Compared with the reference hooks, this backend:
 *   - computes every token (ne11) and every broadcast batch (ne12, ne13) of
 *     MUL_MAT, where the reference computes token 0 only;
 *   - honours nb[] strides and ggml's broadcasting in every op it claims,
 *     and claims an op only where it computes ggml's semantics (the
 *     reference's handlers ignore strides, broadcasting, the softmax mask
 *     and scale, and read RoPE's base and positions from other slots);
 *   - runs on device memory with an explicit HIP stream.
 */
#ifndef GGML_ANE_HIP_H
#define GGML_ANE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ANE_GGML_MAX_DIMS 4
#define ANE_GGML_MAX_SRC 10
#define ANE_GGML_MAX_OP_PARAMS 16 /* int32 words: ggml's GGML_MAX_OP_PARAMS bytes / 4 */

/* ggml_type values of the formats this hook distinguishes (ggml's enum). */
enum ane_ggml_type {
    ANE_GGML_TYPE_F32 = 0,
    ANE_GGML_TYPE_F16 = 1,
    ANE_GGML_TYPE_Q4_0 = 2,
    ANE_GGML_TYPE_Q8_0 = 8,
    ANE_GGML_TYPE_I32 = 26
};

/* Operations the hook distinguishes.  ggml's numeric op values depend on the
 * ggml version, so the caller translates its op into one of these. */
enum ane_ggml_op {
    ANE_GGML_OP_NONE = 0,
    ANE_GGML_OP_MUL_MAT = 1,
    ANE_GGML_OP_OTHER = 2, /* anything else: not supported by this backend */
    ANE_GGML_OP_ADD = 3,
    ANE_GGML_OP_MUL = 4,
    ANE_GGML_OP_SCALE = 5,
    ANE_GGML_OP_RMS_NORM = 6,
    ANE_GGML_OP_SOFT_MAX = 7,
    ANE_GGML_OP_SILU = 8, /* GGML_OP_UNARY with GGML_UNARY_OP_SILU */
    ANE_GGML_OP_ROPE = 9,
    ANE_GGML_OP_CPY = 10  /* GGML_OP_CPY, GGML_OP_CONT and GGML_OP_DUP */
};

/* Q8_0 arithmetic of MUL_MAT: G quantizes each activation row per 32-block
 * and dots int8 x int8 (the default); R is the reference opcode 0x57's fp32
 * arithmetic (bytecode_interpreter.s:7010-7063), one launch per token. */
enum ane_ggml_q8_mode { ANE_GGML_Q8_G = 0, ANE_GGML_Q8_R = 1 };

struct ane_ggml_tensor {
    int32_t type;                                /* enum ane_ggml_type        */
    int64_t ne[ANE_GGML_MAX_DIMS];               /* elements per dimension    */
    size_t nb[ANE_GGML_MAX_DIMS];                /* bytes between elements    */
    int32_t op;                                  /* enum ane_ggml_op          */
    struct ane_ggml_tensor* src[ANE_GGML_MAX_SRC];
    void* data;                                  /* device memory             */
    int32_t op_params[ANE_GGML_MAX_OP_PARAMS];   /* ggml's op_params, as is   */
};

typedef struct ane_ggml_backend* ane_ggml_backend_t;

/* Replaces ggml_backend_ane_reg() (ggml-ane.h:20): name of the backend and
 * of its single device ("ANE0" in the reference, ggml-ane.cpp:302-318). */
const char* ane_ggml_backend_name(void);
const char* ane_ggml_device_name(void);

/* Backend instance: owns a grow-only device workspace; compute runs on
 * `stream` (void* = hipStream_t, 0 = null stream).  Replaces
 * ane_dev_init_backend / ane_backend_free (ggml-ane.cpp:332-357, 102-104). */
ane_ggml_backend_t ane_ggml_backend_init(void* stream);
void ane_ggml_backend_free(ane_ggml_backend_t backend);
void ane_ggml_backend_set_q8_mode(ane_ggml_backend_t backend, int mode);

/* The HIP stream the backend computes on (set_stream: later nodes run on
 * `stream`; the workspace stays the backend's, so the caller orders the old
 * stream's work before the new one's). */
void* ane_ggml_backend_get_stream(ane_ggml_backend_t backend);
void ane_ggml_backend_set_stream(ane_ggml_backend_t backend, void* stream);

/* Replaces ane_dev_supports_op (ggml-ane.cpp:363-393): 1 if this backend
 * computes the node.  Every op but MUL_MAT wants F32 tensors whose
 * innermost stride is 4 bytes and whose other strides are multiples of 4.
 *   MUL_MAT  src0 Q8_0 or Q4_0 (the reference's routing, ggml-ane.cpp:135-146;
 *            Q4_0 in its q4_0_gemv arithmetic for every token), src1 and dst
 *            F32, ne00 == ne10, ne0 == ne01, ne1 == ne11, src1/dst batches
 *            broadcastable over src0's (ne12 % ne02 == 0, ne13 % ne03 == 0),
 *            weight rows contiguous.  F32 weights are not claimed.
 *   ADD, MUL dst = src0 (op) src1, src1 repeated over dst (ne0i % ne1i == 0).
 *   SCALE    dst = src0 * op_params[0] (float); a nonzero bias
 *            (op_params[1]) is not claimed.
 *   RMS_NORM eps = op_params[0] (float), rows of ne0 % 16 == 0 values, the
 *            rms_norm_fp32 arithmetic with unit weights.
 *   SOFT_MAX softmax(src0 * scale + mask) per row, scale = op_params[0],
 *            max_bias = op_params[1] must be 0, mask = src[1] (F32, rows of
 *            ne0 values, mask->ne[1] >= ne1, batches broadcast) or none, no
 *            sinks (src[2]), ne0 % 16 == 0; the softmax_fp32 arithmetic
 *            after the scale and mask, which are ggml's fl(fl(x*scale)+m).
 *   SILU     contiguous src0 and dst of the same shape, silu_fp32 arithmetic.
 *   ROPE     src1 I32 positions, one per ne2 index; ggml's op_params
 *            layout: [1] n_dims == ne0, [2] mode 0 (adjacent pairs),
 *            [5] freq_base, [6] freq_scale == 1, [7] ext_factor == 0,
 *            [8] attn_factor == 1, no freq factors (src[2]); the
 *            rope_fp32 arithmetic at theta = freq_base, pos = src1[i2].
 *   CPY      F32 to F32 of equal element counts, any strides (CPY into a
 *            view, CONT of a permuted tensor, DUP), element order row-major
 *            as ggml's dup. */
int ane_ggml_supports_op(const struct ane_ggml_tensor* node);

/* Replaces ane_compute_forward for one node (ggml-ane.cpp:109-154).
 * Asynchronous on the backend's stream; returns an ane_status. */
int ane_ggml_compute_forward(ane_ggml_backend_t backend, const struct ane_ggml_tensor* node);

/* Replaces ane_graph_compute (ggml-ane.cpp:287-299): computes the
 * nodes in order, then synchronises the stream once.  Returns the status of
 * the first failing node (ANE_ERR_INVALID_ARG for an unsupported one). */
int ane_ggml_graph_compute(ane_ggml_backend_t backend, struct ane_ggml_tensor* const* nodes,
                           int n_nodes);

#ifdef __cplusplus
}
#endif

#endif /* GGML_ANE_HIP_H */
