#pragma once
// ane/ane.hpp -- portable drop-in for the reference's public header
// (include/ane/ane.hpp of joshmorgan1000/ane) on MI355X.
//
// Keeps the reference's opcode numbering (enum class Op, ane.hpp:47-177), the
// variadic byte serialiser ane::dispatch (ane.hpp:206-220) and the single C
// entry point interpreter::stream_exec (ane.hpp:37-39), so caller code such as
// the reference's tests/test_mnist_i8.cpp:198-207 and :303-314 compiles
// unchanged against libane_amd.so.  Differences: no Apple <simd> types or
// SME tile helpers (the ZA register model has no GPU meaning), operands are
// device pointers, and Op gains dense_fused_i8 (README.md:84-97), which the
// reference documents but never defines.
//
// Only the quantized path's opcodes are executed by this build; any other
// opcode stops the stream with ANE_ERR_UNKNOWN_OPCODE (ane::last_error()).
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <type_traits>

#include "../ane_hip.h"

namespace ane {
namespace interpreter {
using ::stream_exec;  // extern "C" void stream_exec(const uint8_t*, size_t)
}  // namespace interpreter

/// Opcode numbering of the reference interpreter's jump table
/// (src/bytecode_interpreter.s:42-170).  Values are wire format: never renumber.
enum class Op : uint8_t {
    reserved_0x00 = 0x00,
    zero_za = 0x01,
    acc_smopa = 0x02,
    acc_umopa = 0x03,
    acc_usmopa = 0x04,
    acc_sumopa = 0x05,
    store_tiles = 0x06,
    smopa_2x2 = 0x07,
    umopa_2x2 = 0x08,
    usmopa_2x2 = 0x09,
    load_bias = 0x0A,
    scale_store = 0x0B,
    elementwise_add_fp32 = 0x0C,
    elementwise_scaled_add_fp32 = 0x0D,
    elementwise_mul_fp32 = 0x0E,
    relu_backward_fp32 = 0x0F,
    scatter_tile_fp32 = 0x10,
    transpose_fp32 = 0x11,
    softmax_argmax_fp32 = 0x12,
    luti4_op = 0x13,
    luti2_op = 0x14,
    dense_fp32 = 0x15,
    count_matches = 0x16,
    reduce_sum_fp32 = 0x17,
    dense_i8 = 0x18,                      ///< served: int8 GEMM, packed B, fused epilogue
    quantize_fp32_i8 = 0x19,              ///< served: per-tensor absmax quantize
    dequantize_i8_fp32 = 0x1A,            ///< served
    pack_b_i8 = 0x1B,                     ///< served: SMOPA panel packing
    quantize_fp32_i8_channelwise = 0x1C,  ///< served
    transpose_i8 = 0x1D,
    dense_u8s8 = 0x1E,                    ///< served: uint8 A variant of dense_i8
    load = 0x1F,
    store = 0x20,
    l2_squared_fp32 = 0x21,
    l2_squared_bf16 = 0x22,
    l2_squared_f64 = 0x23,
    cosine_dist_fp32 = 0x24,
    cosine_dist_bf16 = 0x25,
    cosine_dist_f64 = 0x26,
    normalize_fp32 = 0x27,
    dct2_forward_fp32 = 0x28,
    dct2_inverse_fp32 = 0x29,
    threshold_bitmap_fp32 = 0x2A,
    welford_stats_fp32 = 0x2B,
    quantize_pack_4bit_fp32 = 0x2C,
    threshold_8bit = 0x2D,
    quantize_accum_2bit = 0x2E,
    accum_8bit = 0x2F,
    soa_sub_scale_bf16 = 0x30,
    soa_luti2_accum = 0x31,
    soa_luti4_accum = 0x32,
    bitmap_score_pipeline = 0x33,
    mov_zreg = 0x34,
    loop_begin = 0x35,
    loop_end = 0x36,
    set_param = 0x37,
    load_param = 0x38,
    store_param = 0x39,
    advance_param = 0x3A,
    fadd_zreg = 0x3B,
    fsub_zreg = 0x3C,
    fmul_zreg = 0x3D,
    fmla_zreg = 0x3E,
    and_zreg = 0x3F,
    orr_zreg = 0x40,
    eor_zreg = 0x41,
    not_zreg = 0x42,
    lsl_zreg = 0x43,
    lsr_zreg = 0x44,
    asr_zreg = 0x45,
    load_zt0 = 0x46,
    luti2_zreg = 0x47,
    luti4_zreg = 0x48,
    smopa_zreg = 0x49,
    umopa_zreg = 0x4A,
    usmopa_zreg = 0x4B,
    fmopa_zreg = 0x4C,
    cblas_sgemm = 0x4D,
    fclamp_zreg = 0x4E,
    faddv_zreg = 0x4F,
    frsqrt_zreg = 0x50,
    rms_norm_fp32 = 0x51,
    broadcast_scalar_zreg = 0x52,
    fscale_zreg = 0x53,
    silu_fp32 = 0x54,
    rope_fp32 = 0x55,
    softmax_fp32 = 0x56,
    q8_0_gemv = 0x57,                     ///< served: Q8_0 GEMV, reference arithmetic
    q4_0_gemv = 0x58,
    fdot_zreg = 0x59,
    fmla_wide_zreg = 0x5A,
    fadd_wide_zreg = 0x5B,
    fsub_wide_zreg = 0x5C,
    fmul_wide_zreg = 0x5D,
    load_wide_param = 0x5E,
    store_wide_param = 0x5F,
    cblas_bfgemm = 0x60,
    cblas_igemm = 0x61,
    cblas_ugemm = 0x62,
    cblas_usgemm = 0x63,
    gemm_tile_fp32 = 0x64,
    softmax_partial_fp32 = 0x65,
    softmax_correct_fp32 = 0x66,
    reduce_sum_sq_fp32 = 0x67,
    reduce_col_sum_fp32 = 0x68,
    silu_backward_fp32 = 0x69,
    softmax_backward_fp32 = 0x6A,
    gelu_fp32 = 0x6B,
    layer_norm_fp32 = 0x6C,
    causal_mask_fp32 = 0x6D,
    adam_step_fp32 = 0x6E,
    gelu_backward_fp32 = 0x6F,
    rms_norm_backward_fp32 = 0x70,
    layer_norm_backward_fp32 = 0x71,
    rope_backward_fp32 = 0x72,
    cross_entropy_fp32 = 0x73,
    elementwise_sub_fp32 = 0x74,
    q4_k_gemv = 0x75,
    q2_k_gemv = 0x76,
    q3_k_gemv = 0x77,
    q5_k_gemv = 0x78,
    q6_k_gemv = 0x79,
    flash_attention_fp32 = 0x7A,
    get_rows_fp32 = 0x7B,
    get_rows_q8_0 = 0x7C,
    get_rows_q4_0 = 0x7D,
    dense_strided_fp32 = 0x7E,
    advance_param_stride = 0x7F,
    dense_fused_i8 = 0x80,  ///< served: README.md:84-97 (M,N,K:int, scale:f32, relu:bool, A,B,C)
    NUM_OPCODES = 0x81,
};

/// Argument types dispatch() serialises (reference AllowedParameterTypes,
/// ane.hpp:193-199, minus the Apple z_vector/z_stream handle types).
template <typename T>
concept AllowedParameterTypes = std::is_arithmetic_v<T> || std::is_pointer_v<T>;

/// Serialise (op, args...) as [op:u8][each arg's object bytes, in order] and
/// run it (ane.hpp:206-220).  int/uint32_t/float -> 4 bytes, bool/uint8_t ->
/// 1 byte, any pointer -> 8 bytes.  Synchronous; check ane::last_error().
template <typename... Args>
    requires(AllowedParameterTypes<Args> && ...)
inline void dispatch(Op op, Args... args) {
    constexpr size_t size_needed = 1 + (sizeof(Args) + ... + 0);
    alignas(8) uint8_t bytecodes[size_needed] = {};
    bytecodes[0] = static_cast<uint8_t>(op);
    size_t offset = 1;
    auto emit = [&](auto arg) {
        std::memcpy(&bytecodes[offset], &arg, sizeof(arg));
        offset += sizeof(arg);
    };
    (emit(args), ...);
    interpreter::stream_exec(bytecodes, size_needed);
}

/// Status of the calling thread's last dispatch (ANE_OK == 0).
inline int last_error() { return ::ane_last_error(); }
inline const char* last_error_message() { return ::ane_last_error_message(); }

/// dispatch() that throws std::runtime_error on failure.
template <typename... Args>
inline void dispatch_checked(Op op, Args... args) {
    dispatch(op, args...);
    if (last_error() != ANE_OK) throw std::runtime_error(std::string("ane: ") + last_error_message());
}

}  // namespace ane
