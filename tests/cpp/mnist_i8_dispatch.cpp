// The reference's int8 MNIST forward (tests/test_mnist_i8.cpp:198-207 pack,
// :303-314 forward) written against include/ane/ane.hpp exactly as the
// reference writes it: ane::dispatch with the same opcodes, argument types
// and order, linked against libane_amd.so.
//
//   mnist_i8_dispatch device|host <dir>
//
// Reads <dir>/{x_u8,W1,W2,logit_bias}.bin, runs
//   quantize_fp32_i8 W1 -> pack_b_i8, quantize_fp32_i8 W2 -> pack_b_i8,
//   dense_u8s8 (raw pixels x packed W1, ReLU), quantize_fp32_i8 hidden,
//   dense_i8 (hidden x packed W2 + logit mask),
// and writes <dir>/{hidden,logits,scales}.bin.
//  * device: every buffer is hipMalloc'ed (inputs copied in first);
//  * host: every buffer is plain aligned_alloc host memory, as in the
//    reference (its alloc64), and the program makes no call outside the
//    reference's API: the library stages the operands itself when run with
//    ANE_HOST_STAGING=1 in the environment.
// The scale outputs are host floats in both modes, as in the reference
// (&scale_W1, &ctx.scale_h).  Exit status 0 on success; on a failed
// dispatch it prints ane::last_error_message() and exits 1.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "ane/ane.hpp"

namespace {

constexpr int B = 50, INP_K = 832, HIDDEN_DIM = 128, HID_K = 128, OUT_PAD = 16, ROWS = 64;
constexpr float U8_SCALE = 1.0f / 255.0f;

int packed_b_size(int K, int N) {  // test_mnist_i8.cpp:165-169
    const int k_groups = ((K + 3) / 4 * 4) / 4;
    const int panels = ((N + 15) / 16 * 16) / 16;
    return panels * k_groups * 64;
}

bool g_device = true;

void* alloc_buf(size_t bytes) {
    const size_t n = (bytes + 63) / 64 * 64;
    void* p = nullptr;
    if (g_device) {
        if (hipMalloc(&p, n) != hipSuccess || hipMemset(p, 0, n) != hipSuccess) return nullptr;
    } else {
        p = std::aligned_alloc(64, n);
        if (p) std::memset(p, 0, n);
    }
    return p;
}

void free_buf(void* p) {
    if (g_device)
        (void)hipFree(p);
    else
        std::free(p);
}

bool read_file(const std::string& path, std::vector<char>& out) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return false;
    std::fseek(f, 0, SEEK_END);
    out.resize((size_t)std::ftell(f));
    std::fseek(f, 0, SEEK_SET);
    const bool ok = std::fread(out.data(), 1, out.size(), f) == out.size();
    std::fclose(f);
    return ok;
}

bool write_file(const std::string& path, const void* p, size_t n) {
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) return false;
    const bool ok = std::fwrite(p, 1, n, f) == n;
    std::fclose(f);
    return ok;
}

void* upload(const std::vector<char>& h) {
    void* p = alloc_buf(h.size());
    if (!p) return nullptr;
    if (g_device) {
        if (hipMemcpy(p, h.data(), h.size(), hipMemcpyHostToDevice) != hipSuccess) return nullptr;
    } else {
        std::memcpy(p, h.data(), h.size());
    }
    return p;
}

bool download(std::vector<char>& h, const void* p, size_t n) {
    h.resize(n);
    if (g_device) return hipMemcpy(h.data(), p, n, hipMemcpyDeviceToHost) == hipSuccess;
    std::memcpy(h.data(), p, n);
    return true;
}

#define DISPATCH_OR_FAIL(what, ...)                                                        \
    do {                                                                                   \
        ane::dispatch(__VA_ARGS__);                                                        \
        if (ane::last_error() != ANE_OK) {                                                 \
            std::fprintf(stderr, "%s failed: status %d: %s\n", what, ane::last_error(),    \
                         ane::last_error_message());                                       \
            return 1;                                                                      \
        }                                                                                  \
    } while (0)

}  // namespace

int main(int argc, char** argv) {
    if (argc != 3 || (std::strcmp(argv[1], "device") && std::strcmp(argv[1], "host"))) {
        std::fprintf(stderr, "usage: %s device|host <dir>\n", argv[0]);
        return 2;
    }
    g_device = std::strcmp(argv[1], "device") == 0;
    const std::string dir = argv[2];
    std::vector<char> hx, hw1, hw2, hbias;
    if (!read_file(dir + "/x_u8.bin", hx) || !read_file(dir + "/W1.bin", hw1) || !read_file(dir + "/W2.bin", hw2) ||
        !read_file(dir + "/logit_bias.bin", hbias) || hx.size() != (size_t)ROWS * INP_K ||
        hw1.size() != (size_t)INP_K * HIDDEN_DIM * 4 || hw2.size() != (size_t)HID_K * OUT_PAD * 4 ||
        hbias.size() != (size_t)OUT_PAD * 4) {
        std::fprintf(stderr, "missing or short input files in %s\n", dir.c_str());
        return 2;
    }
    const std::vector<char> hzero((size_t)INP_K * 4, 0);
    auto* xi_u8 = static_cast<const uint8_t*>(upload(hx));
    auto* W1 = static_cast<const float*>(upload(hw1));
    auto* W2 = static_cast<const float*>(upload(hw2));
    auto* logit_bias = static_cast<const float*>(upload(hbias));
    auto* zero_bias = static_cast<const float*>(upload(hzero));
    auto* W1_i8 = static_cast<int8_t*>(alloc_buf((size_t)INP_K * HIDDEN_DIM));
    auto* W1_packed = static_cast<int8_t*>(alloc_buf(packed_b_size(INP_K, HIDDEN_DIM)));
    auto* W2_i8 = static_cast<int8_t*>(alloc_buf((size_t)HID_K * OUT_PAD));
    auto* W2_packed = static_cast<int8_t*>(alloc_buf(packed_b_size(HID_K, OUT_PAD)));
    auto* hidden = static_cast<float*>(alloc_buf((size_t)ROWS * HIDDEN_DIM * 4));
    auto* hidden_i8 = static_cast<int8_t*>(alloc_buf((size_t)ROWS * HID_K));
    auto* logits = static_cast<float*>(alloc_buf((size_t)ROWS * OUT_PAD * 4));
    if (!xi_u8 || !W1 || !W2 || !logit_bias || !zero_bias || !W1_i8 || !W1_packed || !W2_i8 || !W2_packed ||
        !hidden || !hidden_i8 || !logits) {
        std::fprintf(stderr, "allocation failed\n");
        return 2;
    }
    float scale_W1 = 1.0f, scale_W2 = 1.0f, scale_h = 0.0f;
    const int batch_size = B;

    // SharedPackedParams::pack (test_mnist_i8.cpp:198-207)
    DISPATCH_OR_FAIL("quantize W1", ane::Op::quantize_fp32_i8, (uint32_t)(INP_K * HIDDEN_DIM), W1, W1_i8, &scale_W1);
    DISPATCH_OR_FAIL("pack W1", ane::Op::pack_b_i8, (uint32_t)INP_K, (uint32_t)HIDDEN_DIM, W1_i8, W1_packed);
    DISPATCH_OR_FAIL("quantize W2", ane::Op::quantize_fp32_i8, (uint32_t)(HID_K * OUT_PAD), W2, W2_i8, &scale_W2);
    DISPATCH_OR_FAIL("pack W2", ane::Op::pack_b_i8, (uint32_t)HID_K, (uint32_t)OUT_PAD, W2_i8, W2_packed);
    // the forward (test_mnist_i8.cpp:303-314)
    DISPATCH_OR_FAIL("dense_u8s8", ane::Op::dense_u8s8, batch_size, HIDDEN_DIM, INP_K, U8_SCALE, scale_W1, true,
                     xi_u8, W1_packed, zero_bias, hidden);
    DISPATCH_OR_FAIL("quantize hidden", ane::Op::quantize_fp32_i8, (uint32_t)(batch_size * HID_K), hidden, hidden_i8,
                     &scale_h);
    DISPATCH_OR_FAIL("dense_i8", ane::Op::dense_i8, batch_size, OUT_PAD, HID_K, scale_h, scale_W2, false, hidden_i8,
                     W2_packed, logit_bias, logits);

    std::vector<char> oh, ol;
    const float scales[3] = {scale_W1, scale_W2, scale_h};
    if (!download(oh, hidden, (size_t)ROWS * HIDDEN_DIM * 4) || !download(ol, logits, (size_t)ROWS * OUT_PAD * 4) ||
        !write_file(dir + "/hidden.bin", oh.data(), oh.size()) || !write_file(dir + "/logits.bin", ol.data(), ol.size()) ||
        !write_file(dir + "/scales.bin", scales, sizeof scales)) {
        std::fprintf(stderr, "writing outputs failed\n");
        return 2;
    }
    for (void* p : {(void*)xi_u8, (void*)W1, (void*)W2, (void*)logit_bias, (void*)zero_bias, (void*)W1_i8,
                    (void*)W1_packed, (void*)W2_i8, (void*)W2_packed, (void*)hidden, (void*)hidden_i8,
                    (void*)logits})
        free_buf(p);
    std::printf("mnist_i8_dispatch %s ok\n", argv[1]);
    return 0;
}
