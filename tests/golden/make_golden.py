#!/usr/bin/env python3
"""Writes the committed golden fixtures of tests/golden/ (*.npz, no pickles).

Each fixture holds inputs and expected outputs for one opcode of the path.
Expected outputs come from the C oracle (oracle/libane_oracle.so).  Every
one is also recomputed here by an independent route, and a fixture is
written only if the two agree bit for bit:
  * the reference tests' own closed-form expectations, where a reference
    KAT exists;
  * the numpy / exact-rational restatement in tests/npref.py otherwise.

Run from the repository root after building the oracle:
    python -m ane_amd.build && python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from tests import _oracle, data, npref  # noqa: E402

OUT = Path(__file__).resolve().parent
F32 = np.float32


def save(name: str, source: str, **arrays) -> None:
    np.savez_compressed(OUT / f"{name}.npz", source=np.array(source), **arrays)
    print(f"wrote {name}.npz: " + ", ".join(f"{k}{tuple(v.shape)}" for k, v in arrays.items()))


def same_bits(a, b) -> bool:
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and a.dtype == b.dtype and a.tobytes() == b.tobytes()


def main() -> None:
    o = _oracle.load()

    # -- quantize_fp32_i8: reference KAT test_dsl_coverage.cpp:334-368
    x = ((np.arange(256) - 128) * F32(0.1)).astype(F32)
    q, s = o.quantize(x)
    qn, sn = npref.quantize_ref(x, 256)
    assert same_bits(q, qn) and same_bits(np.float32(s), np.float32(sn))
    err = np.abs(q.astype(F32) * s - x).max()
    assert err < 1.5 * s  # the reference test's own bound
    save("quantize_kat", "reference tests/test_dsl_coverage.cpp:334-368 (x=(i-128)*0.1, N=256)",
         x=x, q=q, scale=np.array([s], F32))

    # -- int8 contraction: reference KAT test_remaining_ops.cpp:131-184 (cblas_igemm)
    M, N, K = 16, 32, 64
    A = ((np.arange(M * K) % 11) - 5).astype(np.int8).reshape(M, K)
    B = ((np.arange(K * N) % 13) - 6).astype(np.int8).reshape(K, N)
    acc = o.gemm_s8_i32(A, B, M, N, K)
    ref = A.astype(np.int64) @ B.astype(np.int64)  # the test's triple loop
    assert same_bits(acc, ref.astype(np.int32))
    Bp = o.pack_b(B, K, N)
    assert same_bits(Bp, npref.pack_b(B, K, N))
    C = o.dense_i8(M, N, K, F32(1.0), F32(1.0), 0, A, Bp, np.zeros(32, F32))
    assert same_bits(C[:M], ref.astype(F32))  # |acc| < 2^24: exact in fp32
    save("igemm_kat", "reference tests/test_remaining_ops.cpp:131-184 (M=16 N=32 K=64, A=(i%11)-5, "
         "B=(i%13)-6); dense_i8 with sa=sb=1 over the pack_b_i8 panels", A=A, B=B, acc=acc, Bp=Bp, C=C[:M])

    # -- Q8_0 block layout: reference KAT test_remaining_ops.cpp:230-325 (get_rows_q8_0),
    #    read through q8_0_gemv with one-hot x: y[v] = fl(q[v][i] * d_v)
    for dim, scale_of, val_of in (
        (32, lambda v, b: 0.1 * (v + 1), lambda q, v, b: (q + v * 7) % 21 - 10),
        (64, lambda v, b: 0.05 * (v + b + 1), lambda q, v, b: (q + v * 3 + b * 5) % 19 - 9),
    ):
        vocab, nb = 4, dim // 32
        W = np.zeros((vocab, nb, 34), np.uint8)
        deq = np.zeros((vocab, dim), F32)
        for v in range(vocab):
            for b in range(nb):
                d16 = np.array([scale_of(v, b)], np.float32).astype(np.float16)
                W[v, b, :2] = d16.view(np.uint8)
                qs = np.array([val_of(q, v, b) for q in range(32)], np.int8)
                W[v, b, 2:] = qs.view(np.uint8)
                deq[v, 32 * b: 32 * b + 32] = qs.astype(F32) * d16.astype(F32)[0]
        W = W.reshape(vocab, nb * 34)
        Y = np.zeros((dim, vocab), F32)
        for i in range(dim):
            xi = np.zeros(dim, F32)
            xi[i] = 1.0
            Y[i] = o.q8_0_gemv(vocab, dim, xi, W)
        assert same_bits(Y.T, deq)  # the KAT's (float)qval * scale, every element
        save(f"q8_0_get_rows_kat_{dim}", "reference tests/test_remaining_ops.cpp:230-325 "
             "(get_rows_q8_0 tables); column i of y is q8_0_gemv with x = e_i", W=W, Y=Y)

    # -- dense_fused_i8, config-1 shapes (MNIST MLP), first 16 rows; inputs fp16-representable
    x, w1, w2 = data.mnist_inputs(seed=1, batch=16)
    x = x.astype(np.float16).astype(F32)
    w1 = w1.astype(np.float16).astype(F32)
    w2 = w2.astype(np.float16).astype(F32)
    C1 = o.dense_fused_i8(16, 128, 784, F32(1.0), True, x, w1)
    C2 = o.dense_fused_i8(16, 10, 128, F32(1.0), False, C1, w2)
    assert same_bits(C1, npref.dense_fused_i8(16, 128, 784, 1.0, True, x, w1)[0])
    assert same_bits(C2, npref.dense_fused_i8(16, 10, 128, 1.0, False, C1, w2)[0])
    save("dense_fused_mnist", "config 1 shapes (layer 1 M=16 K=784 N=128 relu, layer 2 K=128 N=10), "
         "seed 1, inputs rounded to fp16 values and stored as fp16",
         x=x.astype(np.float16), w1=w1.astype(np.float16), w2=w2.astype(np.float16), C1=C1, C2=C2)

    # -- dense_u8s8 with the reference's MNIST-i8 scales (test_mnist_i8.cpp:304-307)
    g = data.rng(7)
    M, N, K = 20, 40, 96
    Au = g.integers(0, 256, size=(32, 128), dtype=np.uint8)  # Mp x Kp (Kp = ceil64(K))
    Bs = g.integers(-127, 128, size=(K, N), dtype=np.int8)
    bias = g.standard_normal(64).astype(F32)
    Bpad = np.zeros((128, N), np.int8)  # callers pack B at the padded K (test_mnist_i8.cpp:165-169)
    Bpad[:K] = Bs
    Bp = o.pack_b(Bpad, 128, N)
    sa, sb = F32(1.0 / 255.0), F32(0.01)
    Cu = o.dense_i8(M, N, K, sa, sb, 1, Au, Bp, bias, unsigned_a=True)
    Cn = npref.dense_i8(M, N, K, sa, sb, 1, Au, Bp, bias, unsigned_a=True)
    assert same_bits(Cu, Cn)
    save("dense_u8s8_small", "dense_u8s8 (0x1E), M=20 N=40 K=96, relu, sa=1/255, bias; rows up to ceil16(M)",
         A=Au, B=Bs, Bp=Bp, bias=bias, sa=np.array([sa]), sb=np.array([sb]), C=Cu)

    # -- channelwise quantize (0x1C), ragged columns
    rows, cols = 5, 37
    cpad = 48
    xc = np.zeros((rows, cpad), F32)
    xc[:, :cols] = g.standard_normal((rows, cols)).astype(F32)
    qc, sc = o.channelwise(xc, rows, cols)
    for r in range(rows):
        qr, sr = npref.quantize_exact(xc[r])
        assert same_bits(qc[r * cpad:(r + 1) * cpad], qr) and same_bits(sc[r], np.float32(sr))
    save("channelwise_small", "quantize_fp32_i8_channelwise (0x1C), rows=5 cols=37 (row stride 48)",
         x=xc, q=qc.reshape(rows, cpad), scales=sc)

    # -- Q8_0 R and G modes, small seeded case
    N, K, T = 24, 256, 3
    W = data.q8_0_weights(N, K, seed=11)
    xs = data.activations(T, K, seed=12)
    yr = o.q8_0_gemv(N, K, xs[0], W)
    assert same_bits(yr, npref.q8_0_gemv_r(N, K, xs[0], W))
    yg = o.q8_0_mul_mat_g(N, K, T, xs, W)
    assert same_bits(yg, npref.q8_0_mul_mat_g(N, K, T, xs, W))
    save("q8_0_small", "q8_0_gemv R mode (token 0) and G mode (3 tokens), N=24 K=256, seeds 11/12",
         W=W, x=xs, y_r=yr, y_g=yg)


def cblas_fixtures() -> None:
    """The integer GEMM opcodes (0x61-0x63) through the oracle's restatement
    of their handler, each checked against an exact int64 product."""
    o = _oracle.load()
    # reference KAT tests/test_remaining_ops.cpp:131-184: flags 0, lda=K,
    # ldb=ldc=N, beta 0, alpha 1 then 0.5; expected = (float)sum * alpha
    M, N, K = 16, 32, 64
    A = ((np.arange(M * K) % 11) - 5).astype(np.int8)
    B = ((np.arange(K * N) % 13) - 6).astype(np.int8)
    ref = A.reshape(M, K).astype(np.int64) @ B.reshape(K, N).astype(np.int64)  # the test's triple loop
    C0 = np.zeros((M, N), F32)
    c1 = o.cblas_igemm(0, 0, M, N, K, K, N, N, 1.0, 0.0, A, B, C0)
    c05 = o.cblas_igemm(0, 0, M, N, K, K, N, N, 0.5, 0.0, A, B, C0)
    assert same_bits(c1, (ref.astype(F32) * F32(1.0)).astype(F32))
    assert same_bits(c05, (ref.astype(F32) * F32(0.5)).astype(F32))
    assert same_bits(c05, (c1 * F32(0.5)).astype(F32))  # the test's own alpha-scaling check, exactly
    # u8 x u8 and u8 x s8 with transB, strides and a K remainder
    g = np.random.default_rng(21)
    M2, N2, K2, lda, ldb, ldc = 21, 37, 200, 203, 205, 40
    Au = g.integers(0, 256, size=M2 * lda).astype(np.uint8)
    Bu = g.integers(0, 256, size=N2 * ldb).astype(np.uint8)
    Bs = g.integers(-128, 128, size=N2 * ldb).astype(np.int8)
    C2 = g.standard_normal((M2, ldc)).astype(F32)
    am = Au.reshape(M2, lda)[:, :192].astype(np.int64)
    outs = {}
    for name, variant, Bx in (("ugemm", 1, Bu), ("usgemm", 2, Bs)):
        acc = am @ Bx.reshape(N2, ldb)[:, :192].T.astype(np.int64)
        c = o.cblas_igemm(variant, 2, M2, N2, K2, lda, ldb, ldc, -1.25, 0.0, Au, Bx, C2)
        assert same_bits(c[:, :N2], (acc.astype(F32) * F32(-1.25)).astype(F32))
        assert same_bits(c[:, N2:], C2[:, N2:])
        outs[f"C_{name}"] = c
    save("cblas_igemm_kat", "reference tests/test_remaining_ops.cpp:131-184 (cblas_igemm 16x32x64, A=(i%11)-5, "
         "B=(i%13)-6, alpha 1 and 0.5, beta 0), plus ugemm / usgemm 21x37, K=200 (192 used), transB, "
         "lda 203, ldb 205, ldc 40, alpha -1.25 over C2",
         A=A, B=B, C_alpha1=c1, C_alpha05=c05, Au=Au, Bu=Bu, Bs=Bs, C2=C2, **outs)


if __name__ == "__main__":
    if sys.argv[1:] == ["cblas"]:
        cblas_fixtures()
    else:
        main()
        cblas_fixtures()
