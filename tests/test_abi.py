"""The C-ABI boundary without a GPU: exports, byte encoding, decoder errors.

Covers include/ane_hip.h, ggml-ane-hip.h and ane_decode.h (every declared function is exported by
libane_amd.so), the Python mirror of ane::dispatch against the C++ header
(include/ane/ane.hpp compiled with g++), and the decoder's error paths that
return before any HIP call.
"""
import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

import ane_amd
from ane_amd import Op, boolean, encode, f32, i32, ptr, u32

ROOT = Path(__file__).resolve().parents[1]
HEADERS = [ROOT / "include" / "ane_hip.h", ROOT / "include" / "ggml-ane-hip.h", ROOT / "include" / "ane_decode.h"]


def declared_functions() -> list[str]:
    names = set()
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        text = re.sub(r"^\s*(?:struct|enum|typedef)\b.*?;", "", text, flags=re.S | re.M)
        names |= set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(\w+)\s*\(", text, flags=re.M))
    return sorted(n for n in names if n not in ("if", "defined"))


def test_header_matches_python_export_list():
    assert declared_functions() == sorted(ane_amd.EXPORTS)


def test_library_exports_every_declared_symbol():
    assert ane_amd.LIB_PATH.exists(), "build libane_amd.so first (python -m ane_amd.build)"
    L = ane_amd.lib()
    for name in declared_functions():
        assert hasattr(L, name), name
    nm = shutil.which("nm")
    if nm:
        out = subprocess.run([nm, "-D", "--defined-only", str(ane_amd.LIB_PATH)],
                             capture_output=True, text=True, check=True).stdout
        exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
        assert set(declared_functions()) <= exported


def test_pure_host_queries():
    L = ane_amd.lib()
    assert L.ane_hip_version().startswith(b"ane_amd")
    assert L.ane_hip_packed_b_size(832, 128) == 8 * 208 * 64
    assert L.ane_hip_packed_b_size(128, 10) == 1 * 32 * 64
    assert L.ane_hip_dense_fused_i8_workspace_size(4096, 4096, 4096) >= 2 * 4096 * 4096
    assert L.ane_hip_q8_0_mul_mat_workspace_size(4096, 1) >= 4096 + 128 * 4


def test_mul_mat_workspace_covers_both_activation_forms():
    """ane_hip_q8_0_mul_mat_workspace_size(K, T) must hold the token-major
    Q8 form (T x nb x 32 bytes, then scales over ceil4(T) tokens) and, from
    2 tokens, the block-major form of ceil16(T) tokens that the
    activation-stationary kernel writes (nb x Tp x 32 bytes at a 256-byte
    boundary, then nb x Tp scales), ragged T included."""
    L = ane_amd.lib()
    L.ane_hip_q8_0_mul_mat_workspace_size.restype = ctypes.c_size_t

    def ceil(x, m):
        return (x + m - 1) // m * m

    for K in (4096, 14336, 8192, 512):
        nb = K // 32
        for T in (1, 4, 5, 15, 16, 17, 20, 33, 48, 60, 64, 100):
            got = L.ane_hip_q8_0_mul_mat_workspace_size(K, T)
            assert got >= ceil(T * nb * 32, 256) + ceil(nb * ceil(T, 4) * 4, 256), (K, T)
            if T >= 2:
                tp = ceil(T, 16)
                assert got >= ceil(nb * tp * 32, 256) + nb * tp * 4, (K, T)


def test_record_sizes():
    """Appendix of the opcode table: dense 54 B, quantize 29, dequantize 25,
    pack 25, channelwise 33, q8_0_gemv 33, dense_fused_i8 42."""
    assert len(ane_amd.rec_dense_i8(1, 2, 3, 1.0, 1.0, True, 0, 0, 0, 0)) == 54
    assert len(ane_amd.rec_quantize(16, 0, 0, 0)) == 29
    assert len(ane_amd.rec_dequantize(16, 1.0, 0, 0)) == 25
    assert len(ane_amd.rec_pack_b(4, 16, 0, 0)) == 25
    assert len(ane_amd.rec_channelwise(1, 16, 0, 0, 0)) == 33
    assert len(ane_amd.rec_q8_0_gemv(1, 32, 0, 0, 0)) == 33
    assert len(ane_amd.rec_dense_fused_i8(1, 1, 1, 1.0, True, 0, 0, 0)) == 42
    assert len(ane_amd.rec_cblas_igemm("ugemm", 0, 1, 1, 64, 64, 1, 1, 1.0, 0.0, 0, 0, 0)) == 58  # :8355-8369
    assert len(ane_amd.rec_rms_norm(16, 1e-5, 0, 0, 0)) == 33  # :6506, 6509-6514
    assert len(ane_amd.rec_silu(16, 0, 0)) == 21
    assert len(ane_amd.rec_rope(16, 0, 10000.0, 0, 0)) == 29
    assert len(ane_amd.rec_softmax(16, 0, 0)) == 21


def test_python_encoding_matches_cpp_header(tmp_path):
    gxx = shutil.which("g++")
    if not gxx:
        pytest.skip("g++ not available")
    exe = tmp_path / "encode_dump"
    subprocess.run([gxx, "-std=c++20", f"-I{ROOT / 'include'}", str(ROOT / "tests/cpp/encode_dump.cpp"),
                    "-o", str(exe)], check=True)
    lines = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    A, B, bias, C, xf, scale = 0x1000, 0x2000, 0x3000, 0x4000, 0x5000, 0x6000
    expect = [
        ane_amd.rec_dense_i8(50, 16, 128, 0.5, 0.25, False, A, B, bias, C),
        ane_amd.rec_dense_i8(50, 128, 832, ctypes.c_float(1.0 / 255.0).value, 0.125, True, A, B, bias, C,
                             unsigned_a=True),
        ane_amd.rec_quantize(832 * 128, xf, A, scale),
        ane_amd.rec_dequantize(256, 0.75, A, C),
        ane_amd.rec_pack_b(832, 128, A, B),
        ane_amd.rec_channelwise(7, 48, xf, A, scale),
        ane_amd.rec_q8_0_gemv(4096, 14336, xf, B, C),
        ane_amd.rec_dense_fused_i8(50, 128, 784, 1.0, True, xf, xf, C),
        ane_amd.rec_cblas_igemm("igemm", 0, 16, 32, 64, 64, 32, 32, 0.5, 0.0, A, B, C),
        ane_amd.rec_cblas_igemm("usgemm", 3, 5, 7, 130, 9, 140, 11, -1.0, 2.0, A, B, C),
        ane_amd.rec_rms_norm(4096, ctypes.c_float(1e-5).value, xf, B, C),
        ane_amd.rec_softmax(4096, xf, C),
        ane_amd.rec_silu(14336, xf, C),
        ane_amd.rec_rope(128, 7, 500000.0, xf, C),
    ]
    assert lines == [e.hex() for e in expect]


def test_encode_requires_typed_args():
    with pytest.raises(TypeError):
        encode(Op.dense_i8, 1, 2)
    assert encode(Op.dense_fused_i8, i32(-1))[1:] == b"\xff\xff\xff\xff"
    assert encode(Op.q8_0_gemv, u32(1), f32(1.0), boolean(True), ptr(7)) == (
        bytes([0x57]) + b"\x01\0\0\0" + b"\0\0\x80\x3f" + b"\x01" + b"\x07" + b"\0" * 7)


def _run_async(data: bytes):
    L = ane_amd.lib()
    buf = ctypes.create_string_buffer(data, len(data))
    st = L.ane_stream_exec_async(buf, len(data), None)
    return st, L.ane_last_error_message().decode()


def test_decoder_unknown_opcode():
    st, msg = _run_async(bytes([0x15]) + b"\0" * 40)  # dense_fp32: not on this path
    assert st == 4 and "0x15" in msg


def test_decoder_truncated_record():
    rec = ane_amd.rec_dense_i8(16, 16, 64, 1.0, 1.0, False, 0, 0, 0, 0)
    st, msg = _run_async(rec[:-3])
    assert st == 5 and "truncated" in msg


def test_decoder_stops_at_exit_opcode():
    """Slot 0x00 of the jump table is .L_exit: bytes after it are not run."""
    st, _ = _run_async(bytes([0x00, 0x15, 0x15]))
    assert st == 0


def test_decoder_null_operand():
    st, msg = _run_async(ane_amd.rec_quantize(64, 0, 0, 0))
    assert st == 2 and "null" in msg


def test_empty_stream_is_ok():
    st, _ = _run_async(b"")
    assert st == 0


def test_records_refuse_short_tensors():
    """A tensor shorter than the extent its opcode touches is refused while
    encoding (the caching allocator's segments would hide it from the
    per-allocation check inside stream_exec)."""
    import torch

    src = torch.zeros(100, dtype=torch.float32)
    with pytest.raises(ane_amd.AneError) as e:
        ane_amd.rec_quantize(100, src, torch.zeros(112, dtype=torch.int8), torch.zeros(1))  # pads to 112
    assert e.value.status == 3
    big = torch.zeros(4096, dtype=torch.float32)
    view = big[4000:]  # 96 floats from its first element to the storage end
    with pytest.raises(ane_amd.AneError):
        ane_amd.rec_dense_fused_i8(4, 4, 32, 1.0, True, view, big, big[:16])  # A needs 128 floats
    rec = ane_amd.rec_dense_fused_i8(4, 4, 8, 1.0, True, big[:32], big, big[:16])
    assert len(rec) == 42
    with pytest.raises(ane_amd.AneError):
        ane_amd.rec_q8_0_gemv(3, 64, big, torch.zeros(3 * 2 * 34 - 1, dtype=torch.uint8), big)
