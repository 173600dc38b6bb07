// ggml-ane.cpp -- the ggml backend registry of ane_amd: device "ANE0", a
// device-memory buffer type and a backend whose graph_compute runs
// GGML_OP_MUL_MAT with Q8_0 / Q4_0 weights and the fp32 ops ADD, MUL, SCALE,
// RMS_NORM, SOFT_MAX, SILU, ROPE and CPY/CONT/DUP on the MI355X kernels
// behind include/ggml-ane-hip.h (ane_ggml_supports_op /
// ane_ggml_compute_forward).
//
// Replaces src/ggml-backend/ggml-ane.cpp of the reference: registry
// (:412-436), device (:302-410), buffer type (:29-95), backend (:97-104,
// :287-299, :320-352).
//
// ggml interface targeted: ggml's backend interface as declared in ggml.h,
// ggml-backend.h and ggml-backend-impl.h at the revision the reference is
// written against, i.e. the one whose ggml_backend_i ends with
// graph_optimize (ggml-ane.cpp:347) and whose ggml_backend_dev_caps holds
// {async, host_buffer, buffer_from_host_ptr, events} (:325-330); ggml is not
// vendored by the reference and no commit is pinned.  The file depends on
// ggml only by name: every interface struct is zero-filled and its members
// assigned by name, the graph is walked with ggml_graph_n_nodes /
// ggml_graph_node, and ggml_backend_reg.api_version takes
// GGML_BACKEND_API_VERSION from the header it is compiled with, so
// declaration order and enum values are whatever that ggml says.
//
// Differences from the reference backend, on purpose:
//  - buffers are device memory (hipMalloc, zero-filled like the reference's),
//    is_host = false, and the device type is GPU; tensor uploads and
//    downloads are hipMemcpy;
//  - MUL_MAT computes every token (ne11) and broadcast batch with nb[]
//    strides (the reference computes token 0 only); F32 weights (the
//    reference's cblas_sgemm route) are not claimed, so ggml's scheduler
//    runs those products on its CPU backend;
//  - ADD, MUL, SCALE, RMS_NORM, SOFT_MAX, SILU, ROPE and CPY/CONT/DUP are
//    claimed only where the shim computes ggml's semantics (broadcasting,
//    strides, the softmax scale and mask, RoPE's freq_base and per-token
//    positions from ggml's op_params layout), which the reference's
//    handlers do not (:155-277); view ops are claimed and cost nothing;
//  - graph_compute launches every node on the backend's own HIP stream and
//    synchronises once at the end; a node it cannot run fails the graph with
//    GGML_STATUS_FAILED and one stderr line, like the reference (:291-295).
#include "ggml-ane.h"

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <mutex>

#include "ggml-backend-impl.h"
#include "ane_hip.h"
#include "ggml-ane-hip.h"
#include "ggml.h"

namespace {

constexpr size_t kAlign = 256;  // rows of the streaming kernels want 16-byte alignment

struct BufferCtx {
    void* data;
    size_t size;
};

struct BackendCtx {
    hipStream_t stream;
    ane_ggml_backend_t be;
};

ggml_backend_buffer_type g_buft;
ggml_backend_device g_dev;
ggml_backend_reg g_reg;
uint8_t g_guid[16] = {0x61, 0x6e, 0x65, 0x5f, 0x68, 0x69, 0x70, 0x5f,
                      0x67, 0x66, 0x78, 0x39, 0x35, 0x30, 0x00, 0x01};

bool is_view_op(enum ggml_op op) {
    return op == GGML_OP_NONE || op == GGML_OP_RESHAPE || op == GGML_OP_VIEW || op == GGML_OP_PERMUTE ||
           op == GGML_OP_TRANSPOSE;
}

// ggml_type -> the shim's type values (ggml's on-disk numbers for the
// formats it knows; -1 for any other type, which nothing claims).
int32_t ane_type(enum ggml_type t) {
    switch (t) {
        case GGML_TYPE_F32: return ANE_GGML_TYPE_F32;
        case GGML_TYPE_F16: return ANE_GGML_TYPE_F16;
        case GGML_TYPE_Q4_0: return ANE_GGML_TYPE_Q4_0;
        case GGML_TYPE_Q8_0: return ANE_GGML_TYPE_Q8_0;
        case GGML_TYPE_I32: return ANE_GGML_TYPE_I32;
        default: return -1;
    }
}

int32_t ane_op(const ggml_tensor* t) {
    switch (t->op) {
        case GGML_OP_MUL_MAT: return ANE_GGML_OP_MUL_MAT;
        case GGML_OP_ADD: return ANE_GGML_OP_ADD;
        case GGML_OP_MUL: return ANE_GGML_OP_MUL;
        case GGML_OP_SCALE: return ANE_GGML_OP_SCALE;
        case GGML_OP_RMS_NORM: return ANE_GGML_OP_RMS_NORM;
        case GGML_OP_SOFT_MAX: return ANE_GGML_OP_SOFT_MAX;
        case GGML_OP_ROPE: return ANE_GGML_OP_ROPE;
        case GGML_OP_UNARY:
            return ggml_get_unary_op(t) == GGML_UNARY_OP_SILU ? ANE_GGML_OP_SILU : ANE_GGML_OP_OTHER;
        case GGML_OP_CPY:
        case GGML_OP_CONT:
        case GGML_OP_DUP: return ANE_GGML_OP_CPY;
        default: return ANE_GGML_OP_OTHER;
    }
}

// The shim's tensor for one ggml tensor.
void to_ane(const ggml_tensor* t, ane_ggml_tensor* out) {
    std::memset(out, 0, sizeof(*out));
    out->type = ane_type(t->type);
    for (int d = 0; d < ANE_GGML_MAX_DIMS; d++) {
        out->ne[d] = t->ne[d];
        out->nb[d] = t->nb[d];
    }
    out->op = ane_op(t);
    static_assert(sizeof(out->op_params) <= sizeof(t->op_params), "ggml op_params smaller than the shim's");
    std::memcpy(out->op_params, t->op_params, sizeof(out->op_params));
    out->data = t->data;
}

// A node with its first three sources (MUL_MAT's weights and activations,
// a binary op's operands, SOFT_MAX's mask and sinks, ROPE's positions and
// frequency factors), in the shim's form.
struct Node {
    static constexpr int kSrc = 3;
    ane_ggml_tensor dst, src[kSrc];
    explicit Node(const ggml_tensor* node) {
        to_ane(node, &dst);
        for (int i = 0; i < kSrc; i++) {
            if (!node->src[i]) continue;
            to_ane(node->src[i], &src[i]);
            dst.src[i] = &src[i];
        }
    }
    // Sources past the third are not looked at by any op the shim claims;
    // a node that has one is not claimed.
    static bool fits(const ggml_tensor* node) {
        for (int i = kSrc; i < GGML_MAX_SRC; i++)
            if (node->src[i]) return false;
        return true;
    }
};

// ------------------------------------------------------------ buffers
void buf_free(ggml_backend_buffer_t buffer) {
    auto* c = static_cast<BufferCtx*>(buffer->context);
    (void)hipFree(c->data);
    delete c;
}
void* buf_base(ggml_backend_buffer_t buffer) { return static_cast<BufferCtx*>(buffer->context)->data; }
void buf_memset(ggml_backend_buffer_t, ggml_tensor* t, uint8_t value, size_t offset, size_t size) {
    (void)hipMemset(static_cast<char*>(t->data) + offset, value, size);
}
void buf_set(ggml_backend_buffer_t, ggml_tensor* t, const void* data, size_t offset, size_t size) {
    (void)hipMemcpy(static_cast<char*>(t->data) + offset, data, size, hipMemcpyHostToDevice);
}
void buf_get(ggml_backend_buffer_t, const ggml_tensor* t, void* data, size_t offset, size_t size) {
    (void)hipMemcpy(data, static_cast<const char*>(t->data) + offset, size, hipMemcpyDeviceToHost);
}
bool buf_cpy(ggml_backend_buffer_t, const ggml_tensor* src, ggml_tensor* dst) {
    if (!src->buffer || src->buffer->buft != &g_buft) return false;  // ggml copies through the host
    return hipMemcpy(dst->data, src->data, ggml_nbytes(src), hipMemcpyDeviceToDevice) == hipSuccess;
}
void buf_clear(ggml_backend_buffer_t buffer, uint8_t value) {
    auto* c = static_cast<BufferCtx*>(buffer->context);
    (void)hipMemset(c->data, value, c->size);
}

ggml_backend_buffer_i buffer_iface() {
    ggml_backend_buffer_i i;
    std::memset(&i, 0, sizeof(i));
    i.free_buffer = buf_free;
    i.get_base = buf_base;
    i.memset_tensor = buf_memset;
    i.set_tensor = buf_set;
    i.get_tensor = buf_get;
    i.cpy_tensor = buf_cpy;
    i.clear = buf_clear;
    return i;
}

const char* buft_name(ggml_backend_buffer_type_t) { return "ANE"; }
ggml_backend_buffer_t buft_alloc(ggml_backend_buffer_type_t buft, size_t size) {
    const size_t bytes = (size + kAlign - 1) / kAlign * kAlign;
    void* p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : kAlign) != hipSuccess) return nullptr;
    if (hipMemset(p, 0, bytes ? bytes : kAlign) != hipSuccess) {
        (void)hipFree(p);
        return nullptr;
    }
    auto* ctx = new BufferCtx{p, bytes};
    return ggml_backend_buffer_init(buft, buffer_iface(), ctx, size);
}
size_t buft_alignment(ggml_backend_buffer_type_t) { return kAlign; }
bool buft_is_host(ggml_backend_buffer_type_t) { return false; }

// ------------------------------------------------------------ backend
const char* be_name(ggml_backend_t) { return ane_ggml_backend_name(); }
void be_free(ggml_backend_t backend) {
    auto* c = static_cast<BackendCtx*>(backend->context);
    ane_ggml_backend_free(c->be);
    (void)hipStreamDestroy(c->stream);
    delete c;
    delete backend;
}
void be_sync(ggml_backend_t backend) {
    (void)hipStreamSynchronize(static_cast<BackendCtx*>(backend->context)->stream);
}
enum ggml_status be_graph_compute(ggml_backend_t backend, ggml_cgraph* cgraph) {
    auto* c = static_cast<BackendCtx*>(backend->context);
    const int n = ggml_graph_n_nodes(cgraph);
    for (int i = 0; i < n; i++) {
        ggml_tensor* node = ggml_graph_node(cgraph, i);
        if (ggml_is_empty(node) || is_view_op(node->op)) continue;
        const Node nd(node);
        const int st = Node::fits(node) ? ane_ggml_compute_forward(c->be, &nd.dst) : (int)ANE_ERR_INVALID_ARG;
        if (st != 0) {
            std::fprintf(stderr, "ANE backend: cannot compute node %d (%s, status %d)\n", i, ggml_op_name(node->op),
                         st);
            return GGML_STATUS_FAILED;
        }
    }
    return hipStreamSynchronize(c->stream) == hipSuccess ? GGML_STATUS_SUCCESS : GGML_STATUS_FAILED;
}

// ------------------------------------------------------------ device
const char* dev_name(ggml_backend_dev_t) { return ane_ggml_device_name(); }
const char* dev_description(ggml_backend_dev_t) { return "AMD Instinct MI355X (gfx950), ane_amd HIP kernels"; }
void dev_memory(ggml_backend_dev_t, size_t* free, size_t* total) {
    if (hipMemGetInfo(free, total) != hipSuccess) *free = *total = 0;
}
enum ggml_backend_dev_type dev_type(ggml_backend_dev_t) { return GGML_BACKEND_DEVICE_TYPE_GPU; }
void dev_props(ggml_backend_dev_t dev, ggml_backend_dev_props* props) {
    props->name = dev_name(dev);
    props->description = dev_description(dev);
    props->type = dev_type(dev);
    dev_memory(dev, &props->memory_free, &props->memory_total);
    props->caps.async = false;
    props->caps.host_buffer = false;
    props->caps.buffer_from_host_ptr = false;
    props->caps.events = false;
}
ggml_backend_t dev_init_backend(ggml_backend_dev_t dev, const char*) {
    hipStream_t s = nullptr;
    if (hipStreamCreate(&s) != hipSuccess) return nullptr;
    ane_ggml_backend_t be = ane_ggml_backend_init(s);
    if (!be) {
        (void)hipStreamDestroy(s);
        return nullptr;
    }
    ggml_backend_i i;
    std::memset(&i, 0, sizeof(i));
    i.get_name = be_name;
    i.free = be_free;
    i.synchronize = be_sync;
    i.graph_compute = be_graph_compute;
    auto* b = new ggml_backend;
    std::memset(static_cast<void*>(b), 0, sizeof(*b));
    b->guid = &g_guid;
    b->iface = i;
    b->device = dev;
    b->context = new BackendCtx{s, be};
    return b;
}
ggml_backend_buffer_type_t dev_buffer_type(ggml_backend_dev_t) { return &g_buft; }
bool dev_supports_op(ggml_backend_dev_t, const ggml_tensor* op) {
    if (is_view_op(op->op)) return true;
    if (!Node::fits(op)) return false;
    const Node nd(op);
    return ane_ggml_supports_op(&nd.dst) == 1;
}
bool dev_supports_buft(ggml_backend_dev_t, ggml_backend_buffer_type_t buft) { return buft == &g_buft; }

// ------------------------------------------------------------ registry
const char* reg_name(ggml_backend_reg_t) { return ane_ggml_backend_name(); }
size_t reg_device_count(ggml_backend_reg_t) { return 1; }
ggml_backend_dev_t reg_device(ggml_backend_reg_t, size_t index) { return index == 0 ? &g_dev : nullptr; }

void init_once() {
    ggml_backend_buffer_type_i bi;
    std::memset(&bi, 0, sizeof(bi));
    bi.get_name = buft_name;
    bi.alloc_buffer = buft_alloc;
    bi.get_alignment = buft_alignment;
    bi.is_host = buft_is_host;
    std::memset(static_cast<void*>(&g_buft), 0, sizeof(g_buft));
    g_buft.iface = bi;
    g_buft.device = &g_dev;

    ggml_backend_device_i di;
    std::memset(&di, 0, sizeof(di));
    di.get_name = dev_name;
    di.get_description = dev_description;
    di.get_memory = dev_memory;
    di.get_type = dev_type;
    di.get_props = dev_props;
    di.init_backend = dev_init_backend;
    di.get_buffer_type = dev_buffer_type;
    di.supports_op = dev_supports_op;
    di.supports_buft = dev_supports_buft;
    std::memset(static_cast<void*>(&g_dev), 0, sizeof(g_dev));
    g_dev.iface = di;
    g_dev.reg = &g_reg;

    ggml_backend_reg_i ri;
    std::memset(&ri, 0, sizeof(ri));
    ri.get_name = reg_name;
    ri.get_device_count = reg_device_count;
    ri.get_device = reg_device;
    std::memset(static_cast<void*>(&g_reg), 0, sizeof(g_reg));
    g_reg.api_version = GGML_BACKEND_API_VERSION;
    g_reg.iface = ri;
}

}  // namespace

ggml_backend_reg_t ggml_backend_ane_reg(void) {
    static std::once_flag once;
    std::call_once(once, init_once);
    return &g_reg;
}
