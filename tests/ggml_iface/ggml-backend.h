/*
 * Test-only restatement of the part of ggml's ggml-backend.h that
 * ane_amd/ggml/ggml-ane.cpp uses (see ggml.h in this folder).
 */
#pragma once

#include "ggml.h"

#ifdef __cplusplus
extern "C" {
#endif

#define GGML_BACKEND_API

typedef struct ggml_backend_buffer_type* ggml_backend_buffer_type_t;
typedef struct ggml_backend_buffer* ggml_backend_buffer_t;
typedef struct ggml_backend* ggml_backend_t;
typedef struct ggml_backend_reg* ggml_backend_reg_t;
typedef struct ggml_backend_device* ggml_backend_dev_t;
typedef struct ggml_backend_event* ggml_backend_event_t;
typedef void* ggml_backend_graph_plan_t;

enum ggml_backend_buffer_usage {
    GGML_BACKEND_BUFFER_USAGE_ANY = 0,
    GGML_BACKEND_BUFFER_USAGE_WEIGHTS = 1,
    GGML_BACKEND_BUFFER_USAGE_COMPUTE = 2,
};

enum ggml_backend_dev_type {
    GGML_BACKEND_DEVICE_TYPE_CPU,
    GGML_BACKEND_DEVICE_TYPE_GPU,
    GGML_BACKEND_DEVICE_TYPE_ACCEL,
};

struct ggml_backend_dev_caps {
    bool async;
    bool host_buffer;
    bool buffer_from_host_ptr;
    bool events;
};

struct ggml_backend_dev_props {
    const char* name;
    const char* description;
    size_t memory_free;
    size_t memory_total;
    enum ggml_backend_dev_type type;
    struct ggml_backend_dev_caps caps;
};

#ifdef __cplusplus
}
#endif
