// Serialises the hot-path records with include/ane/ane.hpp's ane::dispatch
// and prints them as hex, one line per record, so the Python mirror
// (ane_amd.encode) can be checked against the C++ header byte for byte.
// Links a stand-in stream_exec that only prints; no GPU or library needed.
#include <cstdio>

#include "ane/ane.hpp"

extern "C" void stream_exec(const uint8_t* data, size_t size) {
    for (size_t i = 0; i < size; i++) std::printf("%02x", data[i]);
    std::printf("\n");
}

int main() {
    auto* A = reinterpret_cast<const int8_t*>(0x1000);
    auto* B = reinterpret_cast<const int8_t*>(0x2000);
    auto* bias = reinterpret_cast<const float*>(0x3000);
    auto* C = reinterpret_cast<float*>(0x4000);
    auto* xf = reinterpret_cast<const float*>(0x5000);
    float* scale = reinterpret_cast<float*>(0x6000);
    // test_mnist_i8.cpp:310-313 argument types: int, int, int, float, float, bool, ptrs
    ane::dispatch(ane::Op::dense_i8, 50, 16, 128, 0.5f, 0.25f, false, A, B, bias, C);
    ane::dispatch(ane::Op::dense_u8s8, 50, 128, 832, 1.0f / 255.0f, 0.125f, true, A, B, bias, C);
    ane::dispatch(ane::Op::quantize_fp32_i8, (uint32_t)(832 * 128), xf, (int8_t*)A, scale);
    ane::dispatch(ane::Op::dequantize_i8_fp32, (uint32_t)256, 0.75f, A, C);
    ane::dispatch(ane::Op::pack_b_i8, (uint32_t)832, (uint32_t)128, A, (int8_t*)B);
    ane::dispatch(ane::Op::quantize_fp32_i8_channelwise, (uint32_t)7, (uint32_t)48, xf, (int8_t*)A,
                  scale);
    // ggml-ane.cpp:137-143: uint32_t N, K then uintptr_t x, W, y
    ane::dispatch(ane::Op::q8_0_gemv, uint32_t(4096), uint32_t(14336), reinterpret_cast<uintptr_t>(xf),
                  reinterpret_cast<uintptr_t>(B), reinterpret_cast<uintptr_t>(C));
    // README.md:87-97
    ane::dispatch(ane::Op::dense_fused_i8, 50, 128, 784, 1.0f, true, xf, xf, C);
    // test_remaining_ops.cpp:150-156: uint8_t flags, six uint32_t, two floats, uintptr_t A, B, C
    ane::dispatch(ane::Op::cblas_igemm, uint8_t(0), uint32_t(16), uint32_t(32), uint32_t(64), uint32_t(64),
                  uint32_t(32), uint32_t(32), 0.5f, 0.0f, reinterpret_cast<uintptr_t>(A),
                  reinterpret_cast<uintptr_t>(B), reinterpret_cast<uintptr_t>(C));
    ane::dispatch(ane::Op::cblas_usgemm, uint8_t(3), uint32_t(5), uint32_t(7), uint32_t(130), uint32_t(9),
                  uint32_t(140), uint32_t(11), -1.0f, 2.0f, reinterpret_cast<uintptr_t>(A),
                  reinterpret_cast<uintptr_t>(B), reinterpret_cast<uintptr_t>(C));
    // test_transformer.cpp:105-107, 184-185, 269-270; test_new_ops.cpp:589-590
    ane::dispatch(ane::Op::rms_norm_fp32, uint32_t(4096), 1e-5f, reinterpret_cast<uintptr_t>(xf),
                  reinterpret_cast<uintptr_t>(B), reinterpret_cast<uintptr_t>(C));
    ane::dispatch(ane::Op::softmax_fp32, uint32_t(4096), reinterpret_cast<uintptr_t>(xf),
                  reinterpret_cast<uintptr_t>(C));
    ane::dispatch(ane::Op::silu_fp32, uint32_t(14336), reinterpret_cast<uintptr_t>(xf),
                  reinterpret_cast<uintptr_t>(C));
    ane::dispatch(ane::Op::rope_fp32, uint32_t(128), uint32_t(7), 500000.0f, reinterpret_cast<uintptr_t>(xf),
                  reinterpret_cast<uintptr_t>(C));
    return 0;
}
