"""Independent numpy / exact-rational restatement of the path, used to pin
the C oracle (test infrastructure only).

Written from the reference's instruction semantics, not from the oracle's C:
numpy float32 ufuncs round once per operation (IEEE binary32, RNE),
``np.rint`` is round-half-even, integer matmuls are exact in int64, and
``fma_f32`` rounds an exact rational a*b+c once to binary32.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np

F32 = np.float32
FLT_MAX = F32(3.4028234663852886e38)


def fmax_a(a: np.ndarray, lo) -> np.ndarray:
    """AArch64 FMAX with a non-NaN second operand: NaN stays NaN, max(-0,+0)=+0."""
    a = np.asarray(a, F32)
    lo = F32(lo)
    out = np.where(a > lo, a, lo).astype(F32)
    return np.where(np.isnan(a), a, out).astype(F32)


def quant_params(amax: np.float32):
    amax = F32(amax)
    if amax == 0:
        return F32(1.0), F32(127.0)
    return F32(amax / F32(127.0)), F32(F32(127.0) / amax)


def quantize_exact(x: np.ndarray):
    """bytecode_interpreter.s:1885-1950 over exactly x.size elements."""
    x = np.asarray(x, F32).ravel()
    with np.errstate(invalid="ignore", over="ignore"):
        ab = np.abs(x)
        amax = F32(0.0) if x.size == 0 else (F32(np.nan) if np.isnan(ab).any() else F32(ab.max()))
        scale, inv = quant_params(amax)
        t = (x * inv).astype(F32)
        nan = np.isnan(t)
        t = np.clip(np.where(nan, F32(0), t), F32(-127), F32(127))
        q = np.rint(t).astype(np.int32)
        q[nan] = 0
    return q.astype(np.int8), scale


def quantize_ref(x: np.ndarray, count: int):
    """0x19 with its do-while padding: n = max(16, ceil16(count))."""
    n = max(16, -(-count // 16) * 16)
    return quantize_exact(np.asarray(x, F32).ravel()[:n])


def pack_b(B: np.ndarray, K: int, N: int) -> np.ndarray:
    """bytecode_interpreter.s:2459-2582 by brute-force index enumeration."""
    B = np.asarray(B, np.int8).reshape(K, N) if K * N else np.zeros((K, N), np.int8)
    G = -(-K // 4)
    P = -(-N // 16)
    out = np.zeros(P * G * 64, np.int8)
    for p in range(P):
        for g in range(G):
            for c in range(16):
                for d in range(4):
                    k, col = 4 * g + d, 16 * p + c
                    if k < K and col < N:
                        out[(p * G + g) * 64 + 4 * c + d] = B[k, col]
    return out


def unpack_b(Bp: np.ndarray, Kp: int, N: int) -> np.ndarray:
    """Inverse view used by dense_i8: B[k][j] = Bp[((j//16)*G + k//4)*64 + (j%16)*4 + k%4]."""
    G = Kp // 4
    k = np.arange(Kp)[:, None]
    j = np.arange(N)[None, :]
    idx = ((j // 16) * G + k // 4) * 64 + (j % 16) * 4 + (k % 4)
    return np.asarray(Bp, np.int8)[idx]


def dense_i8(M, N, K, sa, sb, flags, A, Bp, bias, unsigned_a=False):
    """bytecode_interpreter.s:1995-2446 with an int64 numpy matmul."""
    Kp = -(-K // 64) * 64
    Mp = max(16, -(-M // 16) * 16)
    Aint = np.asarray(A, np.uint8 if unsigned_a else np.int8).reshape(-1)[: Mp * Kp]
    Aint = Aint.reshape(Mp, Kp).astype(np.int64)
    B = unpack_b(Bp, Kp, N).astype(np.int64)
    acc = (Aint @ B).astype(np.int64)
    acc32 = ((acc + 2**31) % 2**32 - 2**31).astype(np.int32)
    s = F32(F32(sa) * F32(sb))
    lo = F32(0.0) if (flags & 1) else -FLT_MAX
    v = (acc32.astype(F32) * s).astype(F32)
    v = (v + np.asarray(bias, F32)[:N][None, :]).astype(F32)
    return fmax_a(v, lo)


def dense_fused_i8(M, N, K, scale, relu, A, B):
    """The build's definition of README.md:84-97's dense_fused_i8."""
    qA, sa = quantize_exact(np.asarray(A, F32).ravel()[: M * K])
    qB, sb = quantize_exact(np.asarray(B, F32).ravel()[: K * N])
    acc = qA.reshape(M, K).astype(np.int64) @ qB.reshape(K, N).astype(np.int64)
    s = F32(F32(sa * sb) * F32(scale))
    v = (acc.astype(np.int32).astype(F32) * s).astype(F32)
    v = (v + F32(0.0)).astype(F32)
    return fmax_a(v, F32(0.0) if relu else -FLT_MAX), qA, qB, sa, sb


# ----------------------------------------------------------- exact rounding
def round_f32(x: Fraction) -> np.float32:
    """Round an exact rational to the nearest binary32 (ties to even)."""
    if x == 0:
        return F32(0.0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)  # subnormal range shares the 2^-149 quantum
    q = Fraction(2) ** (e - 23)
    m = a / q
    n = m.numerator // m.denominator
    r = m - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    val = n * q
    if val >= Fraction(2) ** 128:
        return F32(sign * np.inf)
    return F32(sign * float(val))


def fma_f32(a, b, c) -> np.float32:
    return round_f32(Fraction(float(F32(a))) * Fraction(float(F32(b))) + Fraction(float(F32(c))))


def faddv16(v) -> np.float32:
    """FADDV: recursive halving with lo + hi at each level (float32 adds)."""
    v = [F32(x) for x in v]
    while len(v) > 1:
        v = [F32(v[2 * i] + v[2 * i + 1]) for i in range(len(v) // 2)]
    return v[0]


def q8_0_blocks(W: np.ndarray, M: int, K: int):
    """(d fp32 [M, nb], qs int8 [M, nb, 32]) decoded with numpy's float16."""
    nb = K // 32
    Wb = np.asarray(W, np.uint8).reshape(M, nb, 34)
    d = Wb[:, :, :2].copy().view(np.float16).reshape(M, nb).astype(F32)
    qs = Wb[:, :, 2:].view(np.int8)
    return d, qs


def q8_0_gemv_r(M, K, x, W):
    """bytecode_interpreter.s:7016-7063, exact per-lane fma chains (slow: tiny shapes)."""
    nb = K // 32
    d, qs = q8_0_blocks(W, M, K)
    x = np.asarray(x, F32)
    y = np.zeros(M, F32)
    for m in range(M):
        acc = [F32(0.0)] * 16
        for b in range(nb):
            for h in range(2):
                for l in range(16):
                    w = F32(F32(qs[m, b, 16 * h + l]) * d[m, b])
                    acc[l] = fma_f32(w, x[32 * b + 16 * h + l], acc[l])
        y[m] = faddv16(acc)
    return y


def q8_0_quantize_x(K, x):
    nb = K // 32
    qx = np.zeros(nb * 32, np.int8)
    dx = np.zeros(nb, F32)
    for b in range(nb):
        q, s = quantize_exact(np.asarray(x, F32)[32 * b: 32 * b + 32])
        qx[32 * b: 32 * b + 32] = q
        dx[b] = s
    return qx, dx


def q8_0_mul_mat_g(N, K, T, x, W):
    """G mode: 16 strided fma partials per (row, token), FADDV tree (tiny shapes)."""
    nb = K // 32
    d, qs = q8_0_blocks(W, N, K)
    x = np.asarray(x, F32).reshape(T, K)
    y = np.zeros((T, N), F32)
    for t in range(T):
        qx, dx = q8_0_quantize_x(K, x[t])
        isum = (qs.astype(np.int64) * qx.reshape(nb, 32)[None].astype(np.int64)).sum(-1)
        for m in range(N):
            p = [F32(0.0)] * 16
            for b in range(nb):
                dd = F32(d[m, b] * dx[b])
                p[b % 16] = fma_f32(F32(isum[m, b]), dd, p[b % 16])
            y[t, m] = faddv16(p)
    return y
