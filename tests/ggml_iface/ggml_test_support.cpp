// Test harness for ane_amd/ggml/ggml-ane.cpp: the few ggml functions the
// adapter calls (graph accessors, ggml_nbytes, ggml_backend_buffer_init ...),
// restated after ggml's definitions, and C entry points that drive the
// registry the way ggml's scheduler would (device -> buffer type -> buffer
// -> tensors -> graph_compute), for tests/test_ggml_registry.py and
// tests/test_ggml_ops.py.
#include <cstddef>
#include <cstdio>
#include <cstring>
#include <vector>

#include "ggml-ane.h"
#include "ggml-backend-impl.h"
#include "ggml.h"

struct ggml_cgraph {
    int n_nodes;
    ggml_tensor** nodes;
};

extern "C" {

int ggml_graph_n_nodes(ggml_cgraph* g) { return g->n_nodes; }
ggml_tensor* ggml_graph_node(ggml_cgraph* g, int i) { return g->nodes[i < 0 ? g->n_nodes + i : i]; }

bool ggml_is_empty(const ggml_tensor* t) {
    for (int d = 0; d < GGML_MAX_DIMS; d++)
        if (t->ne[d] == 0) return true;
    return false;
}

static size_t blck_size(ggml_type t) { return (t == GGML_TYPE_Q8_0 || t == GGML_TYPE_Q4_0) ? 32 : 1; }
static size_t type_size(ggml_type t) {
    switch (t) {
        case GGML_TYPE_F32: return 4;
        case GGML_TYPE_F16: return 2;
        case GGML_TYPE_Q4_0: return 18;
        case GGML_TYPE_Q8_0: return 34;
        default: return 0;
    }
}

size_t ggml_nbytes(const ggml_tensor* t) {
    const size_t bs = blck_size(t->type);
    size_t n = bs == 1 ? type_size(t->type) : (size_t)t->ne[0] * t->nb[0] / bs;
    for (int d = bs == 1 ? 0 : 1; d < GGML_MAX_DIMS; d++) n += (size_t)(t->ne[d] - 1) * t->nb[d];
    return n;
}

static const char* const kOpNames[GGML_OP_COUNT] = {
    "NONE", "DUP", "ADD", "MUL", "SCALE", "RMS_NORM", "MUL_MAT", "CPY", "CONT", "RESHAPE",
    "VIEW", "PERMUTE", "TRANSPOSE", "SOFT_MAX", "ROPE", "UNARY"};

const char* ggml_op_name(ggml_op op) { return op >= 0 && op < GGML_OP_COUNT ? kOpNames[op] : "?"; }

// ggml keeps a unary node's op in op_params[0].
ggml_unary_op ggml_get_unary_op(const ggml_tensor* t) { return (ggml_unary_op)t->op_params[0]; }

ggml_backend_buffer_t ggml_backend_buffer_init(ggml_backend_buffer_type_t buft, ggml_backend_buffer_i iface,
                                               void* context, size_t size) {
    auto* b = new ggml_backend_buffer;
    b->iface = iface;
    b->buft = buft;
    b->context = context;
    b->size = size;
    b->usage = GGML_BACKEND_BUFFER_USAGE_ANY;
    return b;
}

// ---------------------------------------------------------------- harness
// This header's ggml_op value for an op name (-1 if unknown), and the
// value of GGML_UNARY_OP_SILU, for tests that build ggml_tensor nodes.
int ggml_ane_test_op(const char* name) {
    for (int i = 0; i < GGML_OP_COUNT; i++)
        if (std::strcmp(kOpNames[i], name) == 0) return i;
    return -1;
}
int ggml_ane_test_unary_silu(void) { return GGML_UNARY_OP_SILU; }

// sizeof(ggml_tensor) and the offsets of its members, in declaration order.
int ggml_ane_test_layout(size_t* out, int n) {
    const size_t v[] = {sizeof(ggml_tensor), offsetof(ggml_tensor, type), offsetof(ggml_tensor, buffer),
                        offsetof(ggml_tensor, ne), offsetof(ggml_tensor, nb), offsetof(ggml_tensor, op),
                        offsetof(ggml_tensor, op_params), offsetof(ggml_tensor, flags), offsetof(ggml_tensor, src),
                        offsetof(ggml_tensor, view_src), offsetof(ggml_tensor, view_offs),
                        offsetof(ggml_tensor, data), offsetof(ggml_tensor, name), offsetof(ggml_tensor, extra),
                        offsetof(ggml_tensor, padding)};
    const int k = (int)(sizeof(v) / sizeof(v[0]));
    for (int i = 0; i < k && i < n; i++) out[i] = v[i];
    return k;
}

// The device's supports_op for a node built by the caller.
int ggml_ane_test_supports_node(const ggml_tensor* node) {
    ggml_backend_reg_t reg = ggml_backend_ane_reg();
    ggml_backend_dev_t dev = reg->iface.get_device(reg, 0);
    return dev->iface.supports_op(dev, node) ? 1 : 0;
}

// A backend of the device, and graph_compute over caller-built nodes whose
// data already point to device memory (as tensors in the backend's buffers
// do).
void* ggml_ane_test_backend_new(void) {
    ggml_backend_reg_t reg = ggml_backend_ane_reg();
    ggml_backend_dev_t dev = reg->iface.get_device(reg, 0);
    return dev->iface.init_backend(dev, nullptr);
}
void ggml_ane_test_backend_free(void* be) {
    auto* b = static_cast<ggml_backend_t>(be);
    if (b) b->iface.free(b);
}
int ggml_ane_test_graph(void* be, ggml_tensor** nodes, int n) {
    auto* b = static_cast<ggml_backend_t>(be);
    ggml_cgraph g{n, nodes};
    return (int)b->iface.graph_compute(b, &g);
}

static void contiguous(ggml_tensor* t, ggml_type type, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3) {
    std::memset(t, 0, sizeof(*t));
    t->type = type;
    t->ne[0] = ne0;
    t->ne[1] = ne1;
    t->ne[2] = ne2;
    t->ne[3] = ne3;
    t->nb[0] = type_size(type);
    t->nb[1] = t->nb[0] * (size_t)ne0 / blck_size(type);
    t->nb[2] = t->nb[1] * (size_t)ne1;
    t->nb[3] = t->nb[2] * (size_t)ne2;
}

// Registry facts as "key=value;" pairs (no device memory is touched).
int ggml_ane_test_registry(char* out, size_t n) {
    ggml_backend_reg_t reg = ggml_backend_ane_reg();
    ggml_backend_dev_t dev = reg->iface.get_device(reg, 0);
    ggml_backend_buffer_type_t buft = dev->iface.get_buffer_type(dev);
    ggml_backend_buffer_type other{};
    std::snprintf(out, n,
                  "reg=%s;api=%d;devices=%zu;dev1=%s;dev=%s;desc=%s;type=%d;dev_reg=%d;buft=%s;align=%zu;"
                  "is_host=%d;buft_dev=%d;own_buft=%d;other_buft=%d;same_reg=%d",
                  reg->iface.get_name(reg), reg->api_version, reg->iface.get_device_count(reg),
                  reg->iface.get_device(reg, 1) ? "yes" : "null", dev->iface.get_name(dev),
                  dev->iface.get_description(dev), (int)dev->iface.get_type(dev), dev->reg == reg ? 1 : 0,
                  buft->iface.get_name(buft), buft->iface.get_alignment(buft), buft->iface.is_host(buft) ? 1 : 0,
                  buft->device == dev ? 1 : 0, dev->iface.supports_buft(dev, buft) ? 1 : 0,
                  dev->iface.supports_buft(dev, &other) ? 1 : 0, ggml_backend_ane_reg() == reg ? 1 : 0);
    return 0;
}

// supports_op for a MUL_MAT of contiguous tensors (op 0), a VIEW (1) or an
// ADD (2); src1_row_pad widens src1's row stride by that many bytes.
int ggml_ane_test_supports(int op, int type0, int type1, int typed, long long ne00, long long ne01,
                           long long ne02, long long ne03, long long ne11, long long ne12, long long ne13,
                           long long src1_row_pad) {
    ggml_backend_reg_t reg = ggml_backend_ane_reg();
    ggml_backend_dev_t dev = reg->iface.get_device(reg, 0);
    ggml_tensor a, b, d;
    contiguous(&a, (ggml_type)type0, ne00, ne01, ne02, ne03);
    contiguous(&b, (ggml_type)type1, ne00, ne11, ne12, ne13);
    if (src1_row_pad) {
        b.nb[1] += (size_t)src1_row_pad;
        b.nb[2] = b.nb[1] * (size_t)ne11;
        b.nb[3] = b.nb[2] * (size_t)ne12;
    }
    contiguous(&d, (ggml_type)typed, ne01, ne11, ne12, ne13);
    d.op = op == 0 ? GGML_OP_MUL_MAT : op == 1 ? GGML_OP_VIEW : GGML_OP_ADD;
    d.src[0] = &a;
    d.src[1] = &b;
    return dev->iface.supports_op(dev, &d) ? 1 : 0;
}

// y[T][N] = MUL_MAT(W, x) through the registry: one buffer of the backend's
// type holds W, x and y; the graph is [VIEW of x, MUL_MAT].  Returns the
// graph status, or -100 .. -103 when a step before it fails.
int ggml_ane_test_mul_mat(int type0, int N, int K, int T, const void* W, const float* x, float* y) {
    ggml_backend_reg_t reg = ggml_backend_ane_reg();
    ggml_backend_dev_t dev = reg->iface.get_device(reg, 0);
    ggml_backend_buffer_type_t buft = dev->iface.get_buffer_type(dev);
    ggml_tensor w, xt, xv, yt;
    contiguous(&w, (ggml_type)type0, K, N, 1, 1);
    contiguous(&xt, GGML_TYPE_F32, K, T, 1, 1);
    contiguous(&yt, GGML_TYPE_F32, N, T, 1, 1);
    const size_t align = buft->iface.get_alignment(buft);
    auto up = [&](size_t v) { return (v + align - 1) / align * align; };
    const size_t ow = 0, ox = up(ggml_nbytes(&w)), oy = ox + up(ggml_nbytes(&xt));
    const size_t total = oy + up(ggml_nbytes(&yt));
    ggml_backend_buffer_t buf = buft->iface.alloc_buffer(buft, total);
    if (!buf) return -100;
    char* base = static_cast<char*>(buf->iface.get_base(buf));
    w.data = base + ow;
    xt.data = base + ox;
    yt.data = base + oy;
    w.buffer = xt.buffer = yt.buffer = buf;
    xv = xt;  // a view of x: no compute
    xv.op = GGML_OP_VIEW;
    xv.view_src = &xt;
    xv.src[0] = &xt;
    yt.op = GGML_OP_MUL_MAT;
    yt.src[0] = &w;
    yt.src[1] = &xv;
    buf->iface.set_tensor(buf, &w, W, 0, ggml_nbytes(&w));
    buf->iface.set_tensor(buf, &xt, x, 0, ggml_nbytes(&xt));
    buf->iface.memset_tensor(buf, &yt, 0xff, 0, ggml_nbytes(&yt));  // NaN until computed
    ggml_backend_t be = dev->iface.init_backend(dev, nullptr);
    if (!be) {
        buf->iface.free_buffer(buf);
        delete buf;
        return -101;
    }
    ggml_tensor* nodes[2] = {&xv, &yt};
    ggml_cgraph g{2, nodes};
    const int st = (int)be->iface.graph_compute(be, &g);
    buf->iface.get_tensor(buf, &yt, y, 0, ggml_nbytes(&yt));
    be->iface.free(be);
    buf->iface.free_buffer(buf);
    delete buf;
    return st;
}

// A graph holding a node the backend does not run (MUL_MAT with F32
// weights) fails with GGML_STATUS_FAILED before launching anything (the node
// is not touched: its data stay null).
int ggml_ane_test_unsupported_graph(void) {
    ggml_backend_reg_t reg = ggml_backend_ane_reg();
    ggml_backend_dev_t dev = reg->iface.get_device(reg, 0);
    ggml_backend_t be = dev->iface.init_backend(dev, nullptr);
    if (!be) return -101;
    ggml_tensor a, b, d;
    contiguous(&a, GGML_TYPE_F32, 64, 16, 1, 1);
    contiguous(&b, GGML_TYPE_F32, 64, 1, 1, 1);
    contiguous(&d, GGML_TYPE_F32, 16, 1, 1, 1);
    d.op = GGML_OP_MUL_MAT;
    d.src[0] = &a;
    d.src[1] = &b;
    ggml_tensor* nodes[1] = {&d};
    ggml_cgraph g{1, nodes};
    const int st = (int)be->iface.graph_compute(be, &g);
    be->iface.free(be);
    return st;
}

}  // extern "C"
