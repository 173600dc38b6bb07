"""ane_amd -- MI355X (gfx950) implementation of ane's quantized compute path.

Python mirror of the reference's C++ entry points for this path:

* ``Op`` -- the opcode numbering of the reference's ``enum class ane::Op``
  (include/ane/ane.hpp:47-177) plus ``dense_fused_i8`` (README.md:84-97).
* ``encode`` / ``dispatch`` -- ``ane::dispatch`` (include/ane/ane.hpp:206-220):
  ``[op:u8]`` followed by each argument's little-endian bytes, handed to the
  C entry point ``stream_exec`` of ``libane_amd.so``.
* thin wrappers over the kernel-level C ABI (``include/ane_hip.h``) that take
  torch tensors for device memory and the current torch stream.

The native library is required: importing works without it (so the CPU test
suite can inspect the package), but every call raises if it is missing.
"""
from __future__ import annotations

import ctypes
import enum
import os
import struct
from pathlib import Path
from typing import Any, Iterable

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libane_amd.so"


class Op(enum.IntEnum):
    """Opcode numbers served by this build (reference include/ane/ane.hpp:47-177)."""

    dense_i8 = 0x18
    quantize_fp32_i8 = 0x19
    dequantize_i8_fp32 = 0x1A
    pack_b_i8 = 0x1B
    quantize_fp32_i8_channelwise = 0x1C
    dense_u8s8 = 0x1E
    rms_norm_fp32 = 0x51
    silu_fp32 = 0x54
    rope_fp32 = 0x55
    softmax_fp32 = 0x56
    q8_0_gemv = 0x57
    q4_0_gemv = 0x58
    cblas_igemm = 0x61
    cblas_ugemm = 0x62
    cblas_usgemm = 0x63
    q4_k_gemv = 0x75
    q2_k_gemv = 0x76
    q3_k_gemv = 0x77
    q5_k_gemv = 0x78
    q6_k_gemv = 0x79
    get_rows_q8_0 = 0x7C
    get_rows_q4_0 = 0x7D
    dense_fused_i8 = 0x80


# R-mode GEMV formats besides Q8_0: name -> (bytes, values) per (super-)block
QFORMATS = {"q4_0": (18, 32), "q4_k": (144, 256), "q2_k": (84, 256), "q3_k": (110, 256),
            "q5_k": (176, 256), "q6_k": (210, 256)}


class AneError(RuntimeError):
    """A call into libane_amd.so returned a non-zero ane_status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"ane status {status}: {message}")
        self.status = status


STATUS = {
    0: "ANE_OK",
    1: "ANE_ERR_INVALID_ARG",
    2: "ANE_ERR_BAD_POINTER",
    3: "ANE_ERR_BUFFER_TOO_SMALL",
    4: "ANE_ERR_UNKNOWN_OPCODE",
    5: "ANE_ERR_TRUNCATED",
    6: "ANE_ERR_HIP",
    7: "ANE_ERR_NO_DEVICE",
    8: "ANE_ERR_WORKSPACE",
    9: "ANE_ERR_GRID_WAIT",
}

# Symbols include/ane_hip.h, include/ggml-ane-hip.h and include/ane_decode.h
# declare; the library must export every one.
EXPORTS = (
    "stream_exec",
    "ane_last_error",
    "ane_last_error_message",
    "ane_set_stream",
    "ane_set_host_staging",
    "ane_stream_exec_async",
    "ane_hip_quantize_workspace_size",
    "ane_hip_quantize_fp32_i8",
    "ane_hip_dequantize_i8_fp32",
    "ane_hip_quantize_channelwise",
    "ane_hip_packed_b_size",
    "ane_hip_pack_b_i8",
    "ane_hip_dense_i8",
    "ane_hip_dense_fused_i8_workspace_size",
    "ane_hip_dense_fused_i8",
    "ane_hip_dense_fused_i8_quantize",
    "ane_hip_dense_fused_i8_gemm",
    "ane_hip_dense_fused_i8_status",
    "ane_hip_grid_wait_status",
    "ane_hip_set_grid_wait_limit",
    "ane_hip_gemm_s8_i32",
    "ane_hip_q8_0_gemv",
    "ane_hip_cblas_igemm_workspace_size",
    "ane_hip_cblas_igemm",
    "ane_hip_q4_0_gemv",
    "ane_hip_q4_k_gemv",
    "ane_hip_q2_k_gemv",
    "ane_hip_q3_k_gemv",
    "ane_hip_q5_k_gemv",
    "ane_hip_q6_k_gemv",
    "ane_hip_get_rows_q8_0",
    "ane_hip_get_rows_q4_0",
    "ane_hip_q8_0_mul_mat_workspace_size",
    "ane_hip_q8_0_mul_mat_workspace_size_n",
    "ane_hip_q8_0_mul_mat",
    "ane_hip_q8_0_mul_mat_noalloc_max_bytes",
    "ane_hip_q8_0_mul_mat_noalloc",
    "ane_hip_device_check",
    "ane_hip_version",
    # include/ggml-ane-hip.h
    "ane_ggml_backend_name",
    "ane_ggml_device_name",
    "ane_ggml_backend_init",
    "ane_ggml_backend_free",
    "ane_ggml_backend_set_q8_mode",
    "ane_ggml_supports_op",
    "ane_ggml_compute_forward",
    "ane_ggml_graph_compute",
    # include/ane_decode.h
    "ane_decode_workspace_size",
    "ane_decode_token",
    "ane_hip_q8_0_matvec_fused",
    "ane_hip_rope_kv_append",
    "ane_hip_attention_workspace_size",
    "ane_hip_attention_decode",
    "ane_hip_silu_mul",
    "ane_hip_q8_0_matvec_silu",
    "ane_hip_attention_decode_rope",
    "ane_hip_q8_0_matvec_q8",
    "ane_hip_q8_0_gate_up_silu_quant",
    "ane_hip_silu_mul_quant",
    "ane_hip_rms_norm",
    "ane_hip_add_fp32",
    "ane_hip_rms_norm_fp32",
    "ane_hip_silu_fp32",
    "ane_hip_rope_fp32",
    "ane_hip_softmax_fp32",
    "ane_decode_ggml_workspace_size",
    "ane_decode_token_ggml",
    "ane_ggml_backend_get_stream",
    "ane_ggml_backend_set_stream",
)

_lib: ctypes.CDLL | None = None

_c = ctypes
_P = _c.c_void_p
_SIGS: dict[str, tuple[Any, list[Any]]] = {
    "stream_exec": (None, [_P, _c.c_size_t]),
    "ane_last_error": (_c.c_int, []),
    "ane_last_error_message": (_c.c_char_p, []),
    "ane_set_stream": (None, [_P]),
    "ane_set_host_staging": (None, [_c.c_int]),
    "ane_stream_exec_async": (_c.c_int, [_P, _c.c_size_t, _P]),
    "ane_hip_quantize_workspace_size": (_c.c_size_t, [_c.c_uint64]),
    "ane_hip_quantize_fp32_i8": (_c.c_int, [_c.c_uint64, _c.c_int, _P, _P, _P, _P, _c.c_size_t, _P]),
    "ane_hip_dequantize_i8_fp32": (_c.c_int, [_c.c_uint64, _c.c_float, _P, _P, _P]),
    "ane_hip_quantize_channelwise": (_c.c_int, [_c.c_uint32, _c.c_uint32, _P, _P, _P, _P]),
    "ane_hip_packed_b_size": (_c.c_size_t, [_c.c_uint32, _c.c_uint32]),
    "ane_hip_pack_b_i8": (_c.c_int, [_c.c_uint32, _c.c_uint32, _P, _P, _P]),
    "ane_hip_dense_i8": (
        _c.c_int,
        [_c.c_uint32, _c.c_uint32, _c.c_uint32, _c.c_float, _c.c_float, _c.c_uint8, _P, _P, _P, _P,
         _c.c_int, _P],
    ),
    "ane_hip_dense_fused_i8_workspace_size": (_c.c_size_t, [_c.c_int32, _c.c_int32, _c.c_int32]),
    "ane_hip_dense_fused_i8": (
        _c.c_int,
        [_c.c_int32, _c.c_int32, _c.c_int32, _c.c_float, _c.c_int, _P, _P, _P, _P, _P, _c.c_size_t, _P],
    ),
    "ane_hip_dense_fused_i8_quantize": (
        _c.c_int, [_c.c_int32, _c.c_int32, _c.c_int32, _P, _P, _P, _P, _c.c_size_t, _P]),
    "ane_hip_dense_fused_i8_gemm": (
        _c.c_int, [_c.c_int32, _c.c_int32, _c.c_int32, _c.c_float, _c.c_int, _P, _P, _c.c_size_t, _P]),
    "ane_hip_dense_fused_i8_status": (_c.c_int, [_P, _P]),
    "ane_hip_grid_wait_status": (_c.c_int, [_P]),
    "ane_hip_set_grid_wait_limit": (None, [_c.c_uint64]),
    "ane_hip_gemm_s8_i32": (
        _c.c_int,
        [_c.c_uint32, _c.c_uint32, _c.c_uint32, _P, _c.c_uint32, _P, _c.c_uint32, _P, _P],
    ),
    "ane_hip_q8_0_gemv": (_c.c_int, [_c.c_uint32, _c.c_uint32, _P, _P, _P, _P]),
    "ane_hip_cblas_igemm_workspace_size": (_c.c_size_t, [_c.c_uint32, _c.c_uint32, _c.c_uint32]),
    "ane_hip_cblas_igemm": (
        _c.c_int,
        [_c.c_int, _c.c_int, _c.c_uint8, _c.c_uint32, _c.c_uint32, _c.c_uint32, _c.c_uint32, _c.c_uint32,
         _c.c_uint32, _c.c_float, _c.c_float, _P, _P, _P, _P, _c.c_size_t, _P],
    ),
    **{f"ane_hip_{f}_gemv": (_c.c_int, [_c.c_uint32, _c.c_uint32, _P, _P, _P, _P]) for f in QFORMATS},
    "ane_hip_get_rows_q8_0": (_c.c_int, [_c.c_uint32, _c.c_uint32, _P, _c.c_uint64, _P, _P, _P]),
    "ane_hip_get_rows_q4_0": (_c.c_int, [_c.c_uint32, _c.c_uint32, _P, _c.c_uint64, _P, _P, _P]),
    "ane_hip_q8_0_mul_mat_workspace_size": (_c.c_size_t, [_c.c_uint32, _c.c_uint32]),
    "ane_hip_q8_0_mul_mat_workspace_size_n": (_c.c_size_t, [_c.c_uint32, _c.c_uint32, _c.c_uint32]),
    "ane_hip_q8_0_mul_mat": (
        _c.c_int,
        [_c.c_uint32, _c.c_uint32, _c.c_uint32, _P, _P, _P, _P, _c.c_size_t, _P],
    ),
    "ane_hip_q8_0_mul_mat_noalloc_max_bytes": (_c.c_size_t, []),
    "ane_hip_q8_0_mul_mat_noalloc": (_c.c_int, [_c.c_uint32, _c.c_uint32, _c.c_uint32, _P, _P, _P, _P]),
    "ane_hip_device_check": (_c.c_int, []),
    "ane_hip_version": (_c.c_char_p, []),
    "ane_ggml_backend_name": (_c.c_char_p, []),
    "ane_ggml_device_name": (_c.c_char_p, []),
    "ane_ggml_backend_init": (_P, [_P]),
    "ane_ggml_backend_free": (None, [_P]),
    "ane_ggml_backend_set_q8_mode": (None, [_P, _c.c_int]),
    "ane_ggml_supports_op": (_c.c_int, [_P]),
    "ane_ggml_compute_forward": (_c.c_int, [_P, _P]),
    "ane_ggml_graph_compute": (_c.c_int, [_P, _P, _c.c_int]),
    "ane_decode_workspace_size": (_c.c_size_t, [_P]),
    "ane_decode_token": (_c.c_int, [_P, _P, _P, _c.c_uint32, _P, _P, _c.c_size_t, _P]),
    "ane_hip_q8_0_matvec_fused": (_c.c_int, [_c.c_uint32, _c.c_uint32, _P, _P, _c.c_float, _P, _P, _P, _P]),
    "ane_hip_rope_kv_append": (_c.c_int, [_P, _P, _P, _c.c_uint32, _P, _P, _P]),
    "ane_hip_attention_workspace_size": (_c.c_size_t, [_P]),
    "ane_hip_attention_decode": (_c.c_int, [_P, _P, _P, _P, _c.c_uint32, _P, _P, _c.c_size_t, _P]),
    "ane_hip_silu_mul": (_c.c_int, [_c.c_uint32, _P, _P, _P]),
    "ane_hip_q8_0_matvec_silu": (_c.c_int, [_c.c_uint32, _c.c_uint32, _P, _P, _P, _P, _P]),
    "ane_hip_attention_decode_rope": (_c.c_int, [_P, _P, _P, _c.c_uint32, _P, _P, _P, _P, _P, _c.c_size_t, _P]),
    "ane_hip_q8_0_matvec_q8": (_c.c_int, [_c.c_uint32, _c.c_uint32, _P, _P, _P, _P, _P]),
    "ane_hip_q8_0_gate_up_silu_quant": (_c.c_int, [_c.c_uint32, _c.c_uint32, _P, _P, _c.c_float, _P, _P, _P]),
    "ane_hip_silu_mul_quant": (_c.c_int, [_c.c_uint32, _P, _P, _P]),
    "ane_hip_rms_norm": (_c.c_int, [_c.c_uint32, _P, _P, _c.c_float, _P, _P]),
    "ane_hip_add_fp32": (_c.c_int, [_c.c_uint32, _P, _P, _P, _P]),
    "ane_hip_rms_norm_fp32": (_c.c_int, [_c.c_uint32, _c.c_uint32, _c.c_float, _P, _P, _P, _P]),
    "ane_hip_silu_fp32": (_c.c_int, [_c.c_uint64, _P, _P, _P]),
    "ane_hip_rope_fp32": (_c.c_int, [_c.c_uint32, _c.c_uint32, _c.c_uint32, _c.c_float, _P, _P, _P]),
    "ane_hip_softmax_fp32": (_c.c_int, [_c.c_uint32, _c.c_uint32, _P, _P, _P]),
    "ane_decode_ggml_workspace_size": (_c.c_size_t, [_P]),
    "ane_decode_token_ggml": (_c.c_int, [_P, _P, _P, _c.c_float, _c.c_uint32, _P, _P, _c.c_size_t, _P, _c.c_int]),
    "ane_ggml_backend_get_stream": (_P, [_P]),
    "ane_ggml_backend_set_stream": (None, [_P, _P]),
}


def lib() -> ctypes.CDLL:
    """Load libane_amd.so (built by ``python -m ane_amd.build``); raise if absent."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m ane_amd.build` "
                "(there is no CPU fallback for this library)"
            )
        handle = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | ctypes.RTLD_GLOBAL)
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


# ---------------------------------------------------------------- encoding
class _Arg:
    __slots__ = ("fmt", "value", "keep")

    def __init__(self, fmt: str, value: Any, keep: Any = None):
        self.fmt = fmt
        self.value = value
        self.keep = keep


class Record(bytes):
    """An encoded record that also holds the tensors its pointers refer to,
    so a temporary operand cannot be freed (and its memory reused) between
    encoding and execution."""

    keep: tuple = ()


def u8(v: int) -> _Arg:
    return _Arg("<B", int(v))


def boolean(v: bool) -> _Arg:
    return _Arg("<B", 1 if v else 0)


def u32(v: int) -> _Arg:
    return _Arg("<I", int(v))


def i32(v: int) -> _Arg:
    return _Arg("<i", int(v))


def f32(v: float) -> _Arg:
    return _Arg("<f", float(v))


def ptr(v: Any) -> _Arg:
    """Any pointer operand: a torch tensor (its data_ptr) or an integer address."""
    if hasattr(v, "data_ptr"):
        return _Arg("<Q", int(v.data_ptr()), keep=v)
    return _Arg("<Q", int(v or 0))


def encode(op: int, *args: _Arg) -> Record:
    """Byte record of ane::dispatch(op, args...) (include/ane/ane.hpp:206-220)."""
    out = bytearray([int(op) & 0xFF])
    keep = []
    for a in args:
        if not isinstance(a, _Arg):
            raise TypeError("dispatch arguments must be typed: u32/i32/f32/u8/boolean/ptr")
        out += struct.pack(a.fmt, a.value)
        if a.keep is not None:
            keep.append(a.keep)
    rec = Record(bytes(out))
    rec.keep = tuple(keep)
    return rec


def _ceil(x: int, m: int) -> int:
    return (x + m - 1) // m * m


def _need(t: Any, nbytes: int, what: str) -> None:
    """Raise AneError(ANE_ERR_BUFFER_TOO_SMALL) if tensor ``t`` holds fewer
    than ``nbytes`` bytes from its first element to the end of its storage.

    stream_exec checks every operand against its HIP allocation, but torch's
    caching allocator carves tensors out of larger allocations, so a short
    tensor would pass that check and the kernel would touch its neighbours.
    Raw integer addresses are left to stream_exec's check."""
    if nbytes <= 0 or not hasattr(t, "untyped_storage"):
        return
    have = t.untyped_storage().nbytes() - t.storage_offset() * t.element_size()
    if have < nbytes:
        raise AneError(3, f"{what} needs {nbytes} bytes, the tensor holds {have}")


# Typed records with the reference's argument order (Appendix of the opcode
# table: bytecode_interpreter.s parse sites cited in ane_amd/csrc/stream_exec.cpp).
# Tensor operands are checked against the extents the opcode reads and writes.
def rec_dense_i8(M, N, K, sa, sb, relu, A, Bp, bias, C, unsigned_a=False) -> bytes:
    op = Op.dense_u8s8 if unsigned_a else Op.dense_i8
    if N:
        Mp, Kp = max(16, _ceil(M, 16)), _ceil(K, 64)
        _need(A, Mp * Kp, "dense A")
        _need(Bp, _ceil(N, 16) // 16 * (Kp // 4) * 64, "dense B_packed")
        _need(bias, 4 * N, "dense bias")
        _need(C, 4 * Mp * N, "dense C")
    return encode(op, u32(M), u32(N), u32(K), f32(sa), f32(sb), boolean(relu), ptr(A), ptr(Bp),
                  ptr(bias), ptr(C))


def rec_quantize(count, src, dst, scale_out) -> bytes:
    n = max(16, _ceil(count, 16))
    _need(src, 4 * n, "quantize_fp32_i8 src")
    _need(dst, n, "quantize_fp32_i8 dst")
    _need(scale_out, 4, "quantize_fp32_i8 scale_out")
    return encode(Op.quantize_fp32_i8, u32(count), ptr(src), ptr(dst), ptr(scale_out))


def rec_dequantize(count, scale, src, dst) -> bytes:
    n = _ceil(count, 16)
    _need(src, n, "dequantize_i8_fp32 src")
    _need(dst, 4 * n, "dequantize_i8_fp32 dst")
    return encode(Op.dequantize_i8_fp32, u32(count), f32(scale), ptr(src), ptr(dst))


def rec_pack_b(K, N, src, dst) -> bytes:
    _need(src, K * N, "pack_b_i8 src")
    _need(dst, _ceil(N, 16) // 16 * (_ceil(K, 4) // 4) * 64, "pack_b_i8 dst")
    return encode(Op.pack_b_i8, u32(K), u32(N), ptr(src), ptr(dst))


def rec_channelwise(rows, cols, src, dst, scales) -> bytes:
    if rows:
        cpad = max(16, _ceil(cols, 16))
        _need(src, 4 * rows * cpad, "channelwise src")
        _need(dst, rows * cpad, "channelwise dst")
        _need(scales, 4 * rows, "channelwise scales")
    return encode(Op.quantize_fp32_i8_channelwise, u32(rows), u32(cols), ptr(src), ptr(dst), ptr(scales))


def rec_q8_0_gemv(M, K, x, W, y) -> bytes:
    if M:
        nb = K >> 5
        _need(x, 4 * 32 * nb, "q8_0_gemv x")
        _need(W, M * nb * 34, "q8_0_gemv W")
        _need(y, 4 * M, "q8_0_gemv y")
    return encode(Op.q8_0_gemv, u32(M), u32(K), ptr(x), ptr(W), ptr(y))


def rec_q_gemv(fmt, M, K, x, W, y) -> bytes:
    """Record of one of the QFORMATS GEMVs (same layout as q8_0_gemv)."""
    if M:
        bb, vals = QFORMATS[fmt]
        nsb = K // vals
        _need(x, 4 * vals * nsb, f"{fmt}_gemv x")
        _need(W, M * nsb * bb, f"{fmt}_gemv W")
        _need(y, 4 * M, f"{fmt}_gemv y")
    return encode(Op[f"{fmt}_gemv"], u32(M), u32(K), ptr(x), ptr(W), ptr(y))


def rec_get_rows(fmt, n_rows, dim, table, indices, out) -> bytes:
    """get_rows_q8_0 / get_rows_q4_0 record: [n_rows:u32][dim:u32][table][indices][out]."""
    if n_rows and dim >= 32:
        _need(indices, 4 * n_rows, f"get_rows_{fmt} indices")
        _need(out, 4 * n_rows * (dim >> 5) * 32, f"get_rows_{fmt} out")
    return encode(Op[f"get_rows_{fmt}"], u32(n_rows), u32(dim), ptr(table), ptr(indices), ptr(out))


IGEMM_VARIANTS = {"igemm": 0, "ugemm": 1, "usgemm": 2}


def _igemm_extents(flags, M, N, K, lda, ldb, ldc):
    """Bytes of A, B and C the integer GEMM handler's arithmetic touches."""
    Ke = K // 64 * 64
    a = b = 0
    if Ke and M and N:
        if flags & 1:
            g = (M - 1) - (M - 1) % 16
            mx = ((M - 1) % 16) * lda + g
            if M > 16:
                mx = max(mx, 15 * lda + g - 16)
            a = mx + Ke
        else:
            a = (M - 1) * lda + Ke
        b = (N - 1) * ldb + Ke if flags & 2 else (Ke - 1) * ldb + N
    c = 4 * ((M - 1) * ldc + N) if M and N else 0
    return a, b, c


def rec_cblas_igemm(kind, flags, M, N, K, lda, ldb, ldc, alpha, beta, A, B, C) -> bytes:
    """cblas_igemm / cblas_ugemm / cblas_usgemm (kind "igemm", "ugemm",
    "usgemm"): [op][flags:u8][M N K lda ldb ldc:u32][alpha beta:f32][A][B][C]
    (bytecode_interpreter.s:8355-8369)."""
    a, b, c = _igemm_extents(flags, M, N, K, lda, ldb, ldc)
    _need(A, a, f"cblas_{kind} A")
    _need(B, b, f"cblas_{kind} B")
    _need(C, c, f"cblas_{kind} C")
    return encode(Op.cblas_igemm + IGEMM_VARIANTS[kind], u8(flags), u32(M), u32(N), u32(K), u32(lda), u32(ldb),
                  u32(ldc), f32(alpha), f32(beta), ptr(A), ptr(B), ptr(C))


def rec_rms_norm(dim, eps, x, w, out) -> bytes:
    """rms_norm_fp32 (0x51): [dim:u32][eps:f32][in][weight][out] (bytecode_interpreter.s:6509-6514)."""
    for t, nm in ((x, "in"), (w, "weight"), (out, "out")):
        _need(t, 4 * dim, f"rms_norm_fp32 {nm}")
    return encode(Op.rms_norm_fp32, u32(dim), f32(eps), ptr(x), ptr(w), ptr(out))


def rec_silu(count, x, out) -> bytes:
    """silu_fp32 (0x54): [count:u32][in][out] (:6618-6621)."""
    _need(x, 4 * count, "silu_fp32 in")
    _need(out, 4 * count, "silu_fp32 out")
    return encode(Op.silu_fp32, u32(count), ptr(x), ptr(out))


def rec_rope(dim, pos, theta, x, out) -> bytes:
    """rope_fp32 (0x55): [dim:u32][pos:u32][theta:f32][in][out] (:6715-6720)."""
    _need(x, 4 * (dim // 2 * 2), "rope_fp32 in")
    _need(out, 4 * (dim // 2 * 2), "rope_fp32 out")
    return encode(Op.rope_fp32, u32(dim), u32(pos), f32(theta), ptr(x), ptr(out))


def rec_softmax(dim, x, out) -> bytes:
    """softmax_fp32 (0x56): [dim:u32][in][out] (:6914-6917)."""
    _need(x, 4 * dim, "softmax_fp32 in")
    _need(out, 4 * dim, "softmax_fp32 out")
    return encode(Op.softmax_fp32, u32(dim), ptr(x), ptr(out))


def rec_dense_fused_i8(M, N, K, scale, relu, A, B, C) -> bytes:
    if M > 0 and N > 0:
        _need(A, 4 * M * K, "dense_fused_i8 A")
        _need(B, 4 * K * N, "dense_fused_i8 B")
        _need(C, 4 * M * N, "dense_fused_i8 C")
    return encode(Op.dense_fused_i8, i32(M), i32(N), i32(K), f32(scale), boolean(relu), ptr(A), ptr(B),
                  ptr(C))


# ---------------------------------------------------------------- execution
def _stream_handle(stream: Any = None) -> int:
    if stream is None:
        import torch

        stream = torch.cuda.current_stream()
    if hasattr(stream, "cuda_stream"):
        return int(stream.cuda_stream)
    return int(stream or 0)


def stream_exec(data: bytes | Iterable[bytes], stream: Any = None) -> None:
    """Run encoded records through the C entry point ``stream_exec`` on
    ``stream`` (default: torch's current stream) and raise AneError on failure."""
    records = [data] if isinstance(data, (bytes, bytearray)) else list(data)
    data = b"".join(records)  # `records` keeps every operand alive until the call returns
    L = lib()
    L.ane_set_stream(_stream_handle(stream))
    buf = ctypes.create_string_buffer(bytes(data), len(data))
    L.stream_exec(buf, len(data))
    st = L.ane_last_error()
    del records
    if st != 0:
        raise AneError(st, L.ane_last_error_message().decode(errors="replace"))


def dispatch(op: int, *args: _Arg, stream: Any = None) -> None:
    """``ane::dispatch(op, args...)`` with explicitly typed arguments."""
    stream_exec(encode(op, *args), stream=stream)


def check(status: int, what: str = "") -> None:
    if status != 0:
        raise AneError(status, f"{what}: {STATUS.get(status, '?')}")


def _p(t: Any) -> int:
    if t is None:
        return 0
    return int(t.data_ptr()) if hasattr(t, "data_ptr") else int(t)


def _scratch(nbytes: int, device, stream: Any = None, zero: bool = False):
    """A temporary device workspace for a call launched on ``stream``.

    It is allocated on that stream (torch's caching allocator keys blocks by
    the stream they were allocated on), so when the tensor is dropped right
    after the asynchronous call the block is only reused by work ordered
    after the kernels on that same stream."""
    import torch

    if stream is None:
        s = torch.cuda.current_stream(device)
    elif isinstance(stream, torch.cuda.Stream):
        s = stream
    else:
        s = torch.cuda.ExternalStream(_stream_handle(stream), device=device)
    with torch.cuda.stream(s):
        return (torch.zeros if zero else torch.empty)(max(int(nbytes), 1), dtype=torch.uint8, device=device)


# Kernel-level wrappers (device tensors, current torch stream unless given).
def quantize_fp32_i8(src, dst, scale_out, count=None, pad16=True, workspace=None, stream=None):
    n = src.numel() if count is None else count
    L = lib()
    wsb = L.ane_hip_quantize_workspace_size(n)
    ws = workspace if workspace is not None else _scratch(wsb, src.device, stream)
    check(L.ane_hip_quantize_fp32_i8(n, 1 if pad16 else 0, _p(src), _p(dst), _p(scale_out), _p(ws), wsb,
                                     _stream_handle(stream)), "quantize_fp32_i8")


def _capturing(stream: Any = None) -> bool:
    """True when ``stream`` (default: torch's current stream) is capturing a graph."""
    import torch

    if stream is None:
        return torch.cuda.is_current_stream_capturing()
    if not isinstance(stream, torch.cuda.Stream):
        h = _stream_handle(stream)
        if h == 0:
            return False  # the null stream never captures
        stream = torch.cuda.ExternalStream(h)
    s = stream
    with torch.cuda.stream(s):
        return torch.cuda.is_current_stream_capturing()


def dense_fused_i8_status(workspace, stream=None) -> None:
    """Raise AneError(ANE_ERR_GRID_WAIT) if the last quantize call made with
    ``workspace`` ran a grid-wide wait that gave up or was completed by
    another launch's arrivals (its outputs are then not valid).
    Synchronizes the stream; not allowed while it is capturing."""
    check(lib().ane_hip_dense_fused_i8_status(_p(workspace), _stream_handle(stream)), "dense_fused_i8")


def _want_check(check_arg, stream) -> bool:
    return (not _capturing(stream)) if check_arg is None else bool(check_arg)


def dense_fused_i8(M, N, K, scale, relu, A, B, C, scales_out=None, workspace=None, stream=None, check_wait=None):
    """Op::dense_fused_i8 on the kernel ABI.  check_wait: None (default)
    checks the quantizer's wait record after the call (dense_fused_i8_status,
    which synchronizes the stream) unless the stream is capturing; False
    leaves that to the caller; True always checks."""
    L = lib()
    wsb = L.ane_hip_dense_fused_i8_workspace_size(M, N, K)
    ws = workspace if workspace is not None else _scratch(wsb, A.device, stream)
    check(L.ane_hip_dense_fused_i8(M, N, K, scale, 1 if relu else 0, _p(A), _p(B), _p(C), _p(scales_out),
                                   _p(ws), wsb, _stream_handle(stream)), "dense_fused_i8")
    if M > 0 and N > 0 and _want_check(check_wait, stream):
        dense_fused_i8_status(ws, stream)


def dense_fused_i8_quantize(M, N, K, A, B, workspace, scales_out=None, stream=None, check_wait=None):
    """The quantize phase of dense_fused_i8; check_wait as for dense_fused_i8."""
    check(lib().ane_hip_dense_fused_i8_quantize(M, N, K, _p(A), _p(B), _p(scales_out), _p(workspace),
                                                workspace.numel(), _stream_handle(stream)),
          "dense_fused_i8_quantize")
    if M > 0 and N > 0 and _want_check(check_wait, stream):
        dense_fused_i8_status(workspace, stream)


def dense_fused_i8_gemm(M, N, K, scale, relu, C, workspace, stream=None):
    check(lib().ane_hip_dense_fused_i8_gemm(M, N, K, scale, 1 if relu else 0, _p(C), _p(workspace),
                                            workspace.numel(), _stream_handle(stream)),
          "dense_fused_i8_gemm")


def dense_fused_i8_workspace_size(M, N, K) -> int:
    return int(lib().ane_hip_dense_fused_i8_workspace_size(M, N, K))


def gemm_s8_i32(A, Bt, acc, M, N, K, lda=None, ldb=None, stream=None):
    check(lib().ane_hip_gemm_s8_i32(M, N, K, _p(A), lda or K, _p(Bt), ldb or K, _p(acc),
                                    _stream_handle(stream)), "gemm_s8_i32")


def cblas_igemm(kind, flags, M, N, K, lda, ldb, ldc, alpha, beta, A, B, C, blas=False, workspace=None,
                stream=None):
    """The integer GEMMs on the kernel-level ABI; blas=False reproduces the
    handler (what stream_exec runs), blas=True the BLAS form."""
    L = lib()
    wsb = L.ane_hip_cblas_igemm_workspace_size(M, N, K)
    ws = workspace if workspace is not None else _scratch(wsb, C.device, stream)
    check(L.ane_hip_cblas_igemm(IGEMM_VARIANTS[kind], 1 if blas else 0, flags, M, N, K, lda, ldb, ldc, alpha, beta,
                                _p(A), _p(B), _p(C), _p(ws), wsb, _stream_handle(stream)), f"cblas_{kind}")


def q8_0_gemv(M, K, x, W, y, stream=None):
    check(lib().ane_hip_q8_0_gemv(M, K, _p(x), _p(W), _p(y), _stream_handle(stream)), "q8_0_gemv")


def q_gemv(fmt, M, K, x, W, y, stream=None):
    """y = W x for W in one of QFORMATS (the reference's R-mode arithmetic)."""
    if fmt not in QFORMATS:
        raise ValueError(f"unknown format {fmt!r}")
    check(getattr(lib(), f"ane_hip_{fmt}_gemv")(M, K, _p(x), _p(W), _p(y), _stream_handle(stream)),
          f"{fmt}_gemv")


def get_rows(fmt, n_rows, dim, table, table_rows, indices, out, stream=None):
    """out[r] = dequantized table row indices[r] (fmt "q8_0" or "q4_0")."""
    if fmt not in ("q8_0", "q4_0"):
        raise ValueError(f"unknown format {fmt!r}")
    check(getattr(lib(), f"ane_hip_get_rows_{fmt}")(n_rows, dim, _p(table), table_rows, _p(indices), _p(out),
                                                     _stream_handle(stream)), f"get_rows_{fmt}")


def q8_0_mul_mat_workspace_size(K, T, N=None) -> int:
    """Workspace bytes for q8_0_mul_mat: with N, enough for every route of
    an N-row matrix (ane_hip_q8_0_mul_mat_workspace_size_n); without, the
    minimum (some routes are then not taken; results are the same)."""
    if N is None:
        return int(lib().ane_hip_q8_0_mul_mat_workspace_size(K, T))
    return int(lib().ane_hip_q8_0_mul_mat_workspace_size_n(N, K, T))


def q8_0_mul_mat(N, K, T, x, W, y, workspace=None, stream=None):
    L = lib()
    if workspace is None:
        wsb = L.ane_hip_q8_0_mul_mat_workspace_size_n(N, K, T)
        ws = _scratch(wsb, W.device, stream)
    else:
        ws = workspace
        wsb = (workspace.numel() * workspace.element_size() if hasattr(workspace, "numel")
               else L.ane_hip_q8_0_mul_mat_workspace_size(K, T))
    check(L.ane_hip_q8_0_mul_mat(N, K, T, _p(x), _p(W), _p(y), _p(ws), wsb, _stream_handle(stream)),
          "q8_0_mul_mat")


def q8_0_mul_mat_noalloc(N, K, T, x, W, y, stream=None):
    """q8_0_mul_mat with its workspace in the library's static device array
    (no allocation; calls overlapping on one device race)."""
    check(lib().ane_hip_q8_0_mul_mat_noalloc(N, K, T, _p(x), _p(W), _p(y), _stream_handle(stream)),
          "q8_0_mul_mat_noalloc")


def pack_b_i8(K, N, src, dst, stream=None):
    check(lib().ane_hip_pack_b_i8(K, N, _p(src), _p(dst), _stream_handle(stream)), "pack_b_i8")


def packed_b_size(K, N) -> int:
    return int(lib().ane_hip_packed_b_size(K, N))


def dense_i8(M, N, K, sa, sb, relu, A, Bp, bias, C, unsigned_a=False, stream=None):
    check(lib().ane_hip_dense_i8(M, N, K, sa, sb, 1 if relu else 0, _p(A), _p(Bp), _p(bias), _p(C),
                                 1 if unsigned_a else 0, _stream_handle(stream)), "dense_i8")


def require_gpu() -> None:
    """Raise unless libane_amd.so is loadable and a gfx950 device is present."""
    st = lib().ane_hip_device_check()
    if st != 0:
        raise AneError(st, "no usable gfx950 device")


# ---------------------------------------------------------------- ggml hook
class GgmlType:
    """ggml_type values the hook distinguishes (include/ggml-ane-hip.h)."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q8_0 = 8
    I32 = 26


class GgmlOp:
    """enum ane_ggml_op (include/ggml-ane-hip.h)."""
    NONE = 0
    MUL_MAT = 1
    OTHER = 2
    ADD = 3
    MUL = 4
    SCALE = 5
    RMS_NORM = 6
    SOFT_MAX = 7
    SILU = 8
    ROPE = 9
    CPY = 10


class GgmlTensor(ctypes.Structure):
    """Mirror of struct ane_ggml_tensor (ggml's ne/nb/type/op/src/data)."""


GgmlTensor._fields_ = [
    ("type", ctypes.c_int32),
    ("ne", ctypes.c_int64 * 4),
    ("nb", ctypes.c_size_t * 4),
    ("op", ctypes.c_int32),
    ("src", ctypes.POINTER(GgmlTensor) * 10),
    ("data", ctypes.c_void_p),
    ("op_params", ctypes.c_int32 * 16),
]

_TYPE_SIZE = {GgmlType.F32: (1, 4), GgmlType.F16: (1, 2), GgmlType.Q4_0: (32, 18), GgmlType.Q8_0: (32, 34),
              GgmlType.I32: (1, 4)}


def ggml_op_params(*values) -> list:
    """op_params words from ints and floats (floats stored as their fp32
    bits, as ggml's memcpy into op_params does)."""
    import struct

    out = []
    for v in values:
        out.append(struct.unpack("<i", struct.pack("<f", v))[0] if isinstance(v, float) else int(v))
    return out


def ggml_tensor(type_, ne, data=None, nb=None, op=GgmlOp.NONE, src=(), op_params=()) -> GgmlTensor:
    """A node with ggml's default (contiguous) strides unless nb is given;
    op_params: int32 words (ggml_op_params packs floats)."""
    ne = list(ne) + [1] * (4 - len(ne))
    t = GgmlTensor()
    t.type = type_
    t.op = op
    for i in range(4):
        t.ne[i] = ne[i]
    if nb is None:
        blk, size = _TYPE_SIZE[type_]
        nb = [size, size * (ne[0] // blk)]
        nb.append(nb[1] * ne[1])
        nb.append(nb[2] * ne[2])
    for i in range(4):
        t.nb[i] = nb[i]
    for i, s_ in enumerate(src):
        if s_ is not None:
            t.src[i] = ctypes.pointer(s_)
    for i, w in enumerate(op_params):
        t.op_params[i] = w
    t.data = _p(data) or None
    return t


class GgmlBackend:
    """The backend instance of include/ggml-ane-hip.h (device workspace, stream)."""

    def __init__(self, stream=None, q8_mode: int = 0):
        self.L = lib()
        self.h = self.L.ane_ggml_backend_init(_stream_handle(stream))
        if not self.h:
            raise AneError(6, "ane_ggml_backend_init failed")
        self.L.ane_ggml_backend_set_q8_mode(self.h, q8_mode)

    @property
    def stream(self) -> int:
        return int(self.L.ane_ggml_backend_get_stream(self.h) or 0)

    def set_stream(self, stream) -> None:
        self.L.ane_ggml_backend_set_stream(self.h, _stream_handle(stream))

    def supports(self, node: GgmlTensor) -> bool:
        return bool(self.L.ane_ggml_supports_op(ctypes.byref(node)))

    def compute(self, node: GgmlTensor) -> None:
        check(self.L.ane_ggml_compute_forward(self.h, ctypes.byref(node)), "ane_ggml_compute_forward")

    def graph_compute(self, nodes) -> None:
        arr = (ctypes.POINTER(GgmlTensor) * len(nodes))(*[ctypes.pointer(n) for n in nodes])
        check(self.L.ane_ggml_graph_compute(self.h, arr, len(nodes)), "ane_ggml_graph_compute")

    def close(self) -> None:
        if self.h:
            self.L.ane_ggml_backend_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------- decode step
class DecodeConfig(ctypes.Structure):
    """Mirror of struct ane_decode_config (include/ane_decode.h)."""

    _fields_ = [(n, ctypes.c_uint32) for n in ("n_layers", "hidden", "ffn", "n_heads", "n_kv_heads",
                                                "head_dim", "ctx")] + [("eps", ctypes.c_float)]


class DecodeLayer(ctypes.Structure):
    """Mirror of struct ane_decode_layer (device pointers)."""

    _fields_ = [(n, ctypes.c_void_p) for n in ("w_qkv", "w_o", "w_gate_up", "w_down", "attn_norm",
                                                "ffn_norm", "k_cache", "v_cache")]


def rope_table(ctx: int, head_dim: int = 128, base: float = 500000.0):
    """(cos, sin) of pos * base^(-2i/head_dim), fp32 [ctx][head_dim/2][2],
    computed in float64 and rounded once."""
    import numpy as np

    i = np.arange(head_dim // 2, dtype=np.float64)
    theta = np.power(base, -2.0 * i / head_dim)
    ang = np.arange(ctx, dtype=np.float64)[:, None] * theta[None, :]
    return np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)


def q8_0_matvec_fused(N, K, x, W, y, norm_w=None, eps=0.0, residual=None, stream=None):
    check(lib().ane_hip_q8_0_matvec_fused(N, K, _p(x), _p(norm_w), eps, _p(W), _p(residual), _p(y),
                                          _stream_handle(stream)), "q8_0_matvec_fused")


def rope_kv_append(cfg, qkv, table, pos, k_cache, v_cache, stream=None):
    check(lib().ane_hip_rope_kv_append(ctypes.byref(cfg), _p(qkv), _p(table), pos, _p(k_cache), _p(v_cache),
                                       _stream_handle(stream)), "rope_kv_append")


def attention_decode(cfg, q, k_cache, v_cache, length, out, workspace=None, stream=None):
    L = lib()
    wsb = L.ane_hip_attention_workspace_size(ctypes.byref(cfg))
    ws = workspace if workspace is not None else _scratch(wsb, q.device, stream, zero=True)
    check(L.ane_hip_attention_decode(ctypes.byref(cfg), _p(q), _p(k_cache), _p(v_cache), length, _p(out), _p(ws),
                                     wsb, _stream_handle(stream)), "attention_decode")


def q8_0_matvec_silu(N, K, gu, W, y, residual=None, stream=None):
    check(lib().ane_hip_q8_0_matvec_silu(N, K, _p(gu), _p(W), _p(residual), _p(y), _stream_handle(stream)),
          "q8_0_matvec_silu")


def attention_decode_rope(cfg, qkv, table, pos, k_cache, v_cache, out, workspace=None, stream=None, out_q8=None):
    L = lib()
    wsb = L.ane_hip_attention_workspace_size(ctypes.byref(cfg))
    ws = workspace if workspace is not None else _scratch(wsb, qkv.device, stream, zero=True)
    check(L.ane_hip_attention_decode_rope(ctypes.byref(cfg), _p(qkv), _p(table), pos, _p(k_cache), _p(v_cache),
                                          _p(out), _p(out_q8), _p(ws), wsb, _stream_handle(stream)),
          "attention_decode_rope")


def silu_mul(n, gu, h, stream=None):
    check(lib().ane_hip_silu_mul(n, _p(gu), _p(h), _stream_handle(stream)), "silu_mul")


def q8_act_bytes(n):
    """Bytes of the Q8 activation form of n values: qx [n/32][32] int8, then dx [n/32] fp32."""
    return n // 32 * 36


def silu_mul_quant(n, gu, xq, stream=None):
    check(lib().ane_hip_silu_mul_quant(n, _p(gu), _p(xq), _stream_handle(stream)), "silu_mul_quant")


def q8_0_gate_up_silu_quant(F, K, x, norm_w, W, xq, eps=1e-5, stream=None):
    """xq = q8(silu(gate) * up) of the gate|up product (rows interleaved in 32-row groups)."""
    check(lib().ane_hip_q8_0_gate_up_silu_quant(F, K, _p(x), _p(norm_w), float(eps), _p(W), _p(xq),
                                                 _stream_handle(stream)), "q8_0_gate_up_silu_quant")


def interleave_gate_up(W_gate, W_up):
    """Rows of the decode step's w_gate_up: gate and up in alternating 32-row groups."""
    import numpy as np

    F = W_gate.shape[0]
    assert W_up.shape == W_gate.shape and F % 32 == 0
    return np.stack([W_gate.reshape(F // 32, 32, -1), W_up.reshape(F // 32, 32, -1)], axis=1).reshape(2 * F, -1)


def q8_0_matvec_q8(N, K, xq, W, y, residual=None, stream=None):
    check(lib().ane_hip_q8_0_matvec_q8(N, K, _p(xq), _p(W), _p(residual), _p(y), _stream_handle(stream)),
          "q8_0_matvec_q8")


def decode_workspace(cfg, device="cuda"):
    """A device workspace for decode_token."""
    import torch

    return torch.zeros(lib().ane_decode_workspace_size(ctypes.byref(cfg)), dtype=torch.uint8, device=device)


ARITH_BUILD = 0
ARITH_REFERENCE = 1


def rms_norm(K, x, w, eps, out, stream=None):
    """The build's RMSNorm (the fused products' arithmetic), one row."""
    check(lib().ane_hip_rms_norm(K, _p(x), _p(w), float(eps), _p(out), _stream_handle(stream)), "rms_norm")


def rms_norm_fp32(rows, dim, eps, x, w, out, stream=None):
    check(lib().ane_hip_rms_norm_fp32(rows, dim, float(eps), _p(x), _p(w), _p(out), _stream_handle(stream)),
          "rms_norm_fp32")


def silu_fp32(count, x, out, stream=None):
    check(lib().ane_hip_silu_fp32(count, _p(x), _p(out), _stream_handle(stream)), "silu_fp32")


def rope_fp32(rows, dim, pos, theta, x, out, stream=None):
    check(lib().ane_hip_rope_fp32(rows, dim, pos, float(theta), _p(x), _p(out), _stream_handle(stream)),
          "rope_fp32")


def softmax_fp32(rows, dim, x, out, stream=None):
    check(lib().ane_hip_softmax_fp32(rows, dim, _p(x), _p(out), _stream_handle(stream)), "softmax_fp32")


def decode_ggml_workspace(cfg, device="cuda"):
    import torch

    return torch.zeros(lib().ane_decode_ggml_workspace_size(ctypes.byref(cfg)), dtype=torch.uint8, device=device)


def decode_token_ggml(cfg, layers, table, pos, x, workspace, backend, arith=ARITH_BUILD, theta=500000.0):
    """One token through the ggml backend (GgmlBackend): MUL_MAT nodes for the
    products, the steps around them in the build's or the reference's arithmetic."""
    check(lib().ane_decode_token_ggml(ctypes.byref(cfg), layers, _p(table), float(theta), pos, _p(x),
                                      _p(workspace), workspace.numel(), backend.h, arith), "decode_token_ggml")


def decode_token(cfg, layers, table, pos, x, workspace, stream=None):
    """layers: a ctypes array of DecodeLayer (host memory)."""
    L = lib()
    check(L.ane_decode_token(ctypes.byref(cfg), layers, _p(table), pos, _p(x), _p(workspace),
                             workspace.numel(), _stream_handle(stream)), "decode_token")
