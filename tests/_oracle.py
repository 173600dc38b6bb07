"""ctypes binding of the CPU oracle (oracle/libane_oracle.so).

Test infrastructure only: the checker the GPU results are compared with.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_SO = ROOT / "oracle" / "libane_oracle.so"

_lib = None

# weight formats with an R-mode GEMV besides Q8_0: name -> (bytes, values) per block
QFORMATS = {"q4_0": (18, 32), "q4_k": (144, 256), "q2_k": (84, 256), "q3_k": (110, 256),
            "q5_k": (176, 256), "q6_k": (210, 256)}


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


class Oracle:
    def __init__(self, lib):
        self.lib = lib
        c = ctypes
        P = c.c_void_p
        sig = {
            "oracle_set_threads": (c.c_int, [c.c_int]),
            "oracle_quantize_fp32_i8": (None, [c.c_uint32, P, P, P]),
            "oracle_quantize_exact": (None, [c.c_size_t, P, P, P]),
            "oracle_dequantize_i8_fp32": (None, [c.c_uint32, c.c_float, P, P]),
            "oracle_quantize_fp32_i8_channelwise": (None, [c.c_uint32, c.c_uint32, P, P, P]),
            "oracle_packed_b_size": (c.c_size_t, [c.c_uint32, c.c_uint32]),
            "oracle_pack_b_i8": (None, [c.c_uint32, c.c_uint32, P, P]),
            "oracle_dense_i8": (None, [c.c_uint32, c.c_uint32, c.c_uint32, c.c_float, c.c_float,
                                       c.c_uint8, P, P, P, P, c.c_int]),
            "oracle_gemm_s8_i32": (None, [c.c_uint32, c.c_uint32, c.c_uint32, P, c.c_uint32, P,
                                          c.c_uint32, P]),
            "oracle_dense_fused_i8": (None, [c.c_int32, c.c_int32, c.c_int32, c.c_float, c.c_int,
                                             P, P, P]),
            "oracle_dense_fused_rows": (None, [c.c_int32, c.c_int32, c.c_int32, c.c_int32,
                                               c.c_float, c.c_int, P, P, P]),
            "oracle_q8_0_gemv": (None, [c.c_uint32, c.c_uint32, P, P, P]),
            "oracle_q8_0_quantize_x": (None, [c.c_uint32, P, P, P]),
            "oracle_q8_0_mul_mat_g": (None, [c.c_uint32, c.c_uint32, c.c_uint32, P, P, P]),
            "oracle_f16_to_f32": (c.c_float, [c.c_uint16]),
            "oracle_get_rows_q8_0": (None, [c.c_uint32, c.c_uint32, P, P, P]),
            "oracle_get_rows_q4_0": (None, [c.c_uint32, c.c_uint32, P, P, P]),
            "oracle_frsqrte": (c.c_float, [c.c_float]),
            "oracle_frecpe": (c.c_float, [c.c_float]),
            "oracle_rms_norm_fp32": (None, [c.c_uint32, c.c_float, P, P, P]),
            "oracle_silu_fp32": (None, [c.c_uint32, P, P]),
            "oracle_rope_fp32": (None, [c.c_uint32, c.c_uint32, c.c_float, P, P]),
            "oracle_softmax_fp32": (None, [c.c_uint32, P, P]),
            "oracle_rms_norm_build": (None, [c.c_uint32, c.c_float, P, P, P]),
            "oracle_attention_ref": (None, [c.c_uint32, c.c_uint32, c.c_uint32, c.c_uint32, P, P, P, P]),
            "oracle_cblas_igemm": (None, [c.c_int, c.c_int, c.c_uint8, c.c_uint32, c.c_uint32, c.c_uint32,
                                          c.c_uint32, c.c_uint32, c.c_uint32, c.c_float, c.c_float, P, P, P]),
        }
        for fmt in QFORMATS:
            sig[f"oracle_{fmt}_gemv"] = (None, [c.c_uint32, c.c_uint32, P, P, P])
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args

    def set_threads(self, n: int) -> int:
        return self.lib.oracle_set_threads(n)

    # 0x19 with the reference's padding: returns (q over n padded elems, scale)
    def quantize(self, x: np.ndarray, count: int | None = None):
        x = np.ascontiguousarray(x, dtype=np.float32)
        count = x.size if count is None else count
        n = max(16, -(-count // 16) * 16)
        assert x.size >= n
        q = np.zeros(n, np.int8)
        s = np.zeros(1, np.float32)
        self.lib.oracle_quantize_fp32_i8(count, _p(x), _p(q), _p(s))
        return q, s[0]

    def quantize_exact(self, x: np.ndarray):
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        q = np.zeros(max(x.size, 1), np.int8)
        s = np.zeros(1, np.float32)
        self.lib.oracle_quantize_exact(x.size, _p(x), _p(q), _p(s))
        return q[: x.size], s[0]

    def dequantize(self, q: np.ndarray, scale: float, count: int | None = None):
        q = np.ascontiguousarray(q, dtype=np.int8)
        count = q.size if count is None else count
        n = -(-count // 16) * 16
        out = np.zeros(max(n, 1), np.float32)
        self.lib.oracle_dequantize_i8_fp32(count, scale, _p(q), _p(out))
        return out[:n]

    def channelwise(self, x: np.ndarray, rows: int, cols: int):
        cpad = max(16, -(-cols // 16) * 16)
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        assert x.size >= rows * cpad
        q = np.zeros(rows * cpad, np.int8)
        s = np.zeros(max(rows, 1), np.float32)
        self.lib.oracle_quantize_fp32_i8_channelwise(rows, cols, _p(x), _p(q), _p(s))
        return q, s[:rows]

    def packed_b_size(self, K: int, N: int) -> int:
        return int(self.lib.oracle_packed_b_size(K, N))

    def pack_b(self, B: np.ndarray, K: int, N: int):
        B = np.ascontiguousarray(B, dtype=np.int8).ravel()
        out = np.zeros(max(self.packed_b_size(K, N), 1), np.int8)
        self.lib.oracle_pack_b_i8(K, N, _p(B), _p(out))
        return out[: self.packed_b_size(K, N)]

    def dense_i8(self, M, N, K, sa, sb, flags, A, Bp, bias, unsigned_a=False):
        Mp = max(16, -(-M // 16) * 16)
        A = np.ascontiguousarray(A)
        Bp = np.ascontiguousarray(Bp, dtype=np.int8)
        bias = np.ascontiguousarray(bias, dtype=np.float32)
        C = np.zeros((Mp, max(N, 1)), np.float32)
        self.lib.oracle_dense_i8(M, N, K, sa, sb, flags, _p(A), _p(Bp), _p(bias), _p(C),
                                 1 if unsigned_a else 0)
        return C[:, :N]

    def gemm_s8_i32(self, A, B, M, N, K):
        A = np.ascontiguousarray(A, dtype=np.int8)
        B = np.ascontiguousarray(B, dtype=np.int8)
        acc = np.zeros((M, N), np.int32)
        self.lib.oracle_gemm_s8_i32(M, N, K, _p(A), K, _p(B), N, _p(acc))
        return acc

    def dense_fused_i8(self, M, N, K, scale, relu, A, B):
        A = np.ascontiguousarray(A, dtype=np.float32)
        B = np.ascontiguousarray(B, dtype=np.float32)
        C = np.zeros((M, N), np.float32)
        self.lib.oracle_dense_fused_i8(M, N, K, scale, 1 if relu else 0, _p(A), _p(B), _p(C))
        return C

    def dense_fused_rows(self, row0, row1, N, K, s, relu, qA, qB):
        qA = np.ascontiguousarray(qA, dtype=np.int8)
        qB = np.ascontiguousarray(qB, dtype=np.int8)
        C = np.zeros((row1, N), np.float32)  # rows below row0 untouched
        self.lib.oracle_dense_fused_rows(row0, row1, N, K, s, 1 if relu else 0, _p(qA), _p(qB),
                                         _p(C))
        return C[row0:row1]

    def q8_0_gemv(self, M, K, x, W):
        x = np.ascontiguousarray(x, dtype=np.float32)
        W = np.ascontiguousarray(W, dtype=np.uint8)
        y = np.zeros(max(M, 1), np.float32)
        self.lib.oracle_q8_0_gemv(M, K, _p(x), _p(W), _p(y))
        return y[:M]

    def q8_0_quantize_x(self, K, x):
        nb = K >> 5
        x = np.ascontiguousarray(x, dtype=np.float32)
        qx = np.zeros(max(nb * 32, 1), np.int8)
        dx = np.zeros(max(nb, 1), np.float32)
        self.lib.oracle_q8_0_quantize_x(K, _p(x), _p(qx), _p(dx))
        return qx[: nb * 32], dx[:nb]

    def q8_0_mul_mat_g(self, N, K, T, x, W):
        x = np.ascontiguousarray(x, dtype=np.float32)
        W = np.ascontiguousarray(W, dtype=np.uint8)
        y = np.zeros((max(T, 1), max(N, 1)), np.float32)
        self.lib.oracle_q8_0_mul_mat_g(N, K, T, _p(x), _p(W), _p(y))
        return y[:T, :N]

    def q_gemv(self, fmt, M, K, x, W):
        """R-mode GEMV of one of QFORMATS (q4_0, q4_k, q2_k, q3_k, q5_k, q6_k)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        W = np.ascontiguousarray(W, dtype=np.uint8)
        y = np.zeros(max(M, 1), np.float32)
        getattr(self.lib, f"oracle_{fmt}_gemv")(M, K, _p(x), _p(W), _p(y))
        return y[:M]

    def get_rows(self, fmt, n_rows, dim, table, indices):
        table = np.ascontiguousarray(table, dtype=np.uint8)
        idx = np.ascontiguousarray(indices, dtype=np.uint32)
        out = np.zeros((max(n_rows, 1), max(dim // 32 * 32, 1)), np.float32)
        getattr(self.lib, f"oracle_get_rows_{fmt}")(n_rows, dim, _p(table), _p(idx), _p(out))
        return out[:n_rows, : dim // 32 * 32]

    def cblas_igemm(self, variant, flags, M, N, K, lda, ldb, ldc, alpha, beta, A, B, C, semantics=0):
        """0x61-0x63 on host buffers: returns a copy of C updated in place
        (variant 0 igemm, 1 ugemm, 2 usgemm; semantics 0 handler, 1 BLAS)."""
        A = np.ascontiguousarray(A).view(np.uint8)
        B = np.ascontiguousarray(B).view(np.uint8)
        C = np.array(C, dtype=np.float32, copy=True)
        self.lib.oracle_cblas_igemm(variant, semantics, flags, M, N, K, lda, ldb, ldc, np.float32(alpha),
                                    np.float32(beta), _p(A), _p(B), _p(C))
        return C

    # the decode-step handlers 0x51 / 0x54 / 0x55 / 0x56 and the build's RMSNorm
    def frsqrte(self, x) -> np.float32:
        return np.float32(self.lib.oracle_frsqrte(np.float32(x)))

    def frecpe(self, x) -> np.float32:
        return np.float32(self.lib.oracle_frecpe(np.float32(x)))

    def rms_norm_fp32(self, x, w, eps):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        out = np.zeros(max(x.size, 1), np.float32)
        self.lib.oracle_rms_norm_fp32(x.size, np.float32(eps), _p(x), _p(w), _p(out))
        return out[: x.size]

    def silu_fp32(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(max(x.size, 1), np.float32)
        self.lib.oracle_silu_fp32(x.size, _p(x), _p(out))
        return out[: x.size]

    def rope_fp32(self, x, pos, theta):
        x = np.ascontiguousarray(x, np.float32)
        out = x.copy()
        self.lib.oracle_rope_fp32(x.size, pos, np.float32(theta), _p(x), _p(out))
        return out

    def softmax_fp32(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(max(x.size, 1), np.float32)
        self.lib.oracle_softmax_fp32(x.size, _p(x), _p(out))
        return out[: x.size]

    def rms_norm_build(self, x, w, eps):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        out = np.zeros(max(x.size, 1), np.float32)
        self.lib.oracle_rms_norm_build(x.size, np.float32(eps), _p(x), _p(w), _p(out))
        return out[: x.size]

    def attention_ref(self, q, kc, vc, length):
        """q [n_heads][128] fp32, kc/vc fp16 [n_kv][ctx][128] -> [n_heads][128]."""
        q = np.ascontiguousarray(q, np.float32)
        kc = np.ascontiguousarray(kc, np.float16)
        vc = np.ascontiguousarray(vc, np.float16)
        nh, nkv, ctx = q.shape[0], kc.shape[0], kc.shape[1]
        out = np.zeros((nh, 128), np.float32)
        self.lib.oracle_attention_ref(nh, nkv, length, ctx, _p(q), _p(kc.view(np.uint16)),
                                      _p(vc.view(np.uint16)), _p(out))
        return out

    def f16_to_f32(self, h: int) -> float:
        return self.lib.oracle_f16_to_f32(h)


def load() -> Oracle:
    global _lib
    if _lib is None:
        if not ORACLE_SO.exists():
            subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
        _lib = Oracle(ctypes.CDLL(str(ORACLE_SO)))
    return _lib
