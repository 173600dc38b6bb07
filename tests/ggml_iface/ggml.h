/*
 * Test-only restatement of the part of ggml's ggml.h that
 * ane_amd/ggml/ggml-ane.cpp uses, so the adapter builds and runs in the
 * tests without a ggml tree.  It is not ggml: names and meanings follow
 * ggml's public header (the ggml_tensor members, the ggml_type values,
 * which are ggml's on-disk format; the graph accessors, ggml_get_unary_op),
 * the ggml_op and ggml_unary_op values here are this file's own, and the
 * adapter depends on none of them by value.  In a real build the adapter is
 * compiled against ggml's headers.
 */
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GGML_MAX_DIMS 4
#define GGML_MAX_SRC 10
#define GGML_MAX_OP_PARAMS 64
#define GGML_MAX_NAME 64
#define GGML_API

enum ggml_type {
    GGML_TYPE_F32 = 0,
    GGML_TYPE_F16 = 1,
    GGML_TYPE_Q4_0 = 2,
    GGML_TYPE_Q4_1 = 3,
    GGML_TYPE_Q5_0 = 6,
    GGML_TYPE_Q5_1 = 7,
    GGML_TYPE_Q8_0 = 8,
    GGML_TYPE_Q8_1 = 9,
    GGML_TYPE_Q2_K = 10,
    GGML_TYPE_Q3_K = 11,
    GGML_TYPE_Q4_K = 12,
    GGML_TYPE_Q5_K = 13,
    GGML_TYPE_Q6_K = 14,
    GGML_TYPE_I32 = 26,
};

enum ggml_op {
    GGML_OP_NONE = 0,
    GGML_OP_DUP,
    GGML_OP_ADD,
    GGML_OP_MUL,
    GGML_OP_SCALE,
    GGML_OP_RMS_NORM,
    GGML_OP_MUL_MAT,
    GGML_OP_CPY,
    GGML_OP_CONT,
    GGML_OP_RESHAPE,
    GGML_OP_VIEW,
    GGML_OP_PERMUTE,
    GGML_OP_TRANSPOSE,
    GGML_OP_SOFT_MAX,
    GGML_OP_ROPE,
    GGML_OP_UNARY,
    GGML_OP_COUNT,
};

enum ggml_unary_op {
    GGML_UNARY_OP_ABS,
    GGML_UNARY_OP_SGN,
    GGML_UNARY_OP_NEG,
    GGML_UNARY_OP_STEP,
    GGML_UNARY_OP_TANH,
    GGML_UNARY_OP_ELU,
    GGML_UNARY_OP_RELU,
    GGML_UNARY_OP_SIGMOID,
    GGML_UNARY_OP_GELU,
    GGML_UNARY_OP_GELU_QUICK,
    GGML_UNARY_OP_SILU,
    GGML_UNARY_OP_COUNT,
};

enum ggml_status {
    GGML_STATUS_ALLOC_FAILED = -2,
    GGML_STATUS_FAILED = -1,
    GGML_STATUS_SUCCESS = 0,
    GGML_STATUS_ABORTED = 1,
};

typedef uint8_t ggml_guid[16];
typedef ggml_guid* ggml_guid_t;

struct ggml_backend_buffer;

struct ggml_tensor {
    enum ggml_type type;
    struct ggml_backend_buffer* buffer;
    int64_t ne[GGML_MAX_DIMS];
    size_t nb[GGML_MAX_DIMS];
    enum ggml_op op;
    int32_t op_params[GGML_MAX_OP_PARAMS / sizeof(int32_t)];
    int32_t flags;
    struct ggml_tensor* src[GGML_MAX_SRC];
    struct ggml_tensor* view_src;
    size_t view_offs;
    void* data;
    char name[GGML_MAX_NAME];
    void* extra;
    char padding[8];
};

struct ggml_cgraph;

GGML_API int ggml_graph_n_nodes(struct ggml_cgraph* cgraph);
GGML_API struct ggml_tensor* ggml_graph_node(struct ggml_cgraph* cgraph, int i);
GGML_API bool ggml_is_empty(const struct ggml_tensor* tensor);
GGML_API size_t ggml_nbytes(const struct ggml_tensor* tensor);
GGML_API const char* ggml_op_name(enum ggml_op op);
GGML_API enum ggml_unary_op ggml_get_unary_op(const struct ggml_tensor* tensor);

#ifdef __cplusplus
}
#endif
