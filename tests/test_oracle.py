"""Pins the CPU oracle (oracle/ane_oracle.c) before it is trusted as the
checker: reference test expectations, closed forms and an independent numpy /
exact-rational restatement (tests/npref.py).  CPU only."""
import numpy as np
import pytest

from tests import data, npref

F32 = np.float32


def special_values(n: int, seed: int) -> np.ndarray:
    g = np.random.default_rng(seed)
    x = g.standard_normal(n).astype(F32)
    specials = np.array([0.0, -0.0, 1e-40, -1e-40, 1e-45, 3.4e38, -3.4e38, 0.5, -0.5, 1.5, 2.5],
                        F32)
    x[: specials.size] = specials
    return x


# ------------------------------------------------------------ quantize (0x19)
def test_quantize_reference_kat(oracle):
    """tests/test_dsl_coverage.cpp:334-368: x_i = (i-128)*0.1f, N=256;
    quantize -> dequantize round trip within 1.5*scale."""
    x = (np.arange(256, dtype=F32) - F32(128)) * F32(0.1)
    q, s = oracle.quantize(x)
    back = oracle.dequantize(q, s)
    assert np.max(np.abs(back - x)) < 1.5 * s
    # closed form: amax = |-128 * 0.1f|, scale = amax/127, the amax element -> -127
    amax = np.abs(F32(-128) * F32(0.1))
    assert s == F32(amax / F32(127))
    assert q[0] == -127
    assert q[128] == 0
    assert np.all(np.abs(q.astype(int)) <= 127)


@pytest.mark.parametrize("count", [0, 1, 15, 16, 17, 100, 1000, 4096 + 3])
def test_quantize_matches_numpy(oracle, count):
    n = max(16, -(-count // 16) * 16)
    x = special_values(n, count)
    q, s = oracle.quantize(x, count)
    q2, s2 = npref.quantize_ref(x, count)
    assert q.size == n
    assert s.tobytes() == F32(s2).tobytes()
    np.testing.assert_array_equal(q, q2)


def test_quantize_zero_and_sign_symmetry(oracle):
    z = np.zeros(32, F32)
    q, s = oracle.quantize(z)
    assert s == 1.0 and not q.any()
    x = np.random.default_rng(5).standard_normal(64).astype(F32)
    q1, s1 = oracle.quantize(x)
    q2, s2 = oracle.quantize(-x)
    assert s1 == s2
    np.testing.assert_array_equal(q1, -q2)


def test_quantize_nan_gives_zeros(oracle):
    x = np.ones(32, F32)
    x[7] = np.nan
    q, s = oracle.quantize(x)
    assert np.isnan(s)
    assert not q.any()


def test_quantize_padding_is_read(oracle):
    """count=17 processes 32 elements: the padding element can set amax."""
    x = np.zeros(32, F32)
    x[0] = 1.0
    x[31] = 4.0
    q, s = oracle.quantize(x, 17)
    assert s == F32(F32(4.0) / F32(127))
    assert q[31] == 127


def test_dequantize_matches_numpy(oracle):
    q = np.arange(-128, 128, dtype=np.int8)
    out = oracle.dequantize(q, F32(0.0371))
    np.testing.assert_array_equal(out, (q.astype(F32) * F32(0.0371)).astype(F32))


def test_channelwise_matches_numpy(oracle):
    rows, cols = 7, 40
    cpad = 48
    x = special_values(rows * cpad, 11).reshape(rows, cpad)
    x[3] = 0.0
    q, s = oracle.channelwise(x, rows, cols)
    for r in range(rows):
        q2, s2 = npref.quantize_exact(x[r])
        assert s[r].tobytes() == F32(s2).tobytes()
        np.testing.assert_array_equal(q.reshape(rows, cpad)[r], q2)


# ------------------------------------------------------------ pack_b (0x1B)
@pytest.mark.parametrize("K,N", [(1, 1), (4, 16), (5, 17), (64, 10), (13, 40), (128, 32)])
def test_pack_b_matches_bruteforce(oracle, K, N):
    B = np.random.default_rng(K * 100 + N).integers(-128, 128, size=(K, N), dtype=np.int8)
    p = oracle.pack_b(B, K, N)
    assert p.size == oracle.packed_b_size(K, N) == (-(-N // 16)) * (-(-K // 4)) * 64
    np.testing.assert_array_equal(p, npref.pack_b(B, K, N))
    # inverse: the dense_i8 view recovers B and zero padding
    Kp = -(-K // 4) * 4
    back = npref.unpack_b(p, Kp, N)
    np.testing.assert_array_equal(back[:K], B)
    assert not back[K:].any()


# ------------------------------------------------------------ dense_i8 (0x18/0x1E)
def _dense_case(M, N, K, seed, unsigned_a=False):
    g = np.random.default_rng(seed)
    Kp = -(-K // 64) * 64
    Mp = max(16, -(-M // 16) * 16)
    if unsigned_a:
        A = g.integers(0, 256, size=(Mp, Kp), dtype=np.uint8)
    else:
        A = g.integers(-127, 128, size=(Mp, Kp), dtype=np.int8)
    B = np.zeros((Kp, N), np.int8)
    B[:K] = g.integers(-127, 128, size=(K, N), dtype=np.int8)
    bias = g.standard_normal(-(-N // 32) * 32 or 32).astype(F32)
    return A, B, bias


@pytest.mark.parametrize("M,N,K,unsigned_a", [
    (50, 128, 832, True), (50, 16, 128, False), (1, 10, 64, False), (17, 33, 100, False),
    (16, 32, 64, True), (0, 5, 64, False),
])
def test_dense_i8_matches_numpy(oracle, M, N, K, unsigned_a):
    A, B, bias = _dense_case(M, N, K, M * 7 + N + K, unsigned_a)
    Kp = -(-K // 64) * 64
    Bp = oracle.pack_b(B, Kp, N)
    for flags in (0, 1):
        C = oracle.dense_i8(M, N, K, F32(0.013), F32(0.021), flags, A, Bp, bias, unsigned_a)
        C2 = npref.dense_i8(M, N, K, F32(0.013), F32(0.021), flags, A, Bp, bias, unsigned_a)
        assert C.shape == C2.shape == (max(16, -(-M // 16) * 16), N)
        np.testing.assert_array_equal(C.view(np.uint32), C2.view(np.uint32))


def test_dense_i8_igemm_kat(oracle):
    """tests/test_remaining_ops.cpp:131-184 pattern (A=(i%11)-5, B=(i%13)-6,
    16x32x64) through dense_i8 with unit scales: exact integer results."""
    M, N, K = 16, 32, 64
    A = ((np.arange(M * K) % 11) - 5).astype(np.int8).reshape(M, K)
    B = ((np.arange(K * N) % 13) - 6).astype(np.int8).reshape(K, N)
    ref = A.astype(np.int64) @ B.astype(np.int64)
    Bp = oracle.pack_b(B, K, N)
    C = oracle.dense_i8(M, N, K, 1.0, 1.0, 0, A, Bp, np.zeros(N, F32))
    np.testing.assert_array_equal(C, ref.astype(F32))
    C2 = oracle.dense_i8(M, N, K, 0.5, 1.0, 0, A, Bp, np.zeros(N, F32))
    np.testing.assert_array_equal(C2, (ref * 0.5).astype(F32))


@pytest.mark.parametrize("ksteps,expect", [(1, 4), (4, 16)])
def test_dense_i8_all_ones_kat(oracle, ksteps, expect):
    """tests/test_dsl_coverage.cpp:240-260 (smopa all-ones -> 4) and
    tests/test_program_demo.cpp:148-178 (4 accumulation steps -> 16)."""
    M, N, K = 16, 16, 64
    A = np.zeros((M, K), np.int8)
    A[:, : 4 * ksteps] = 1
    B = np.zeros((K, N), np.int8)
    B[: 4 * ksteps] = 1
    C = oracle.dense_i8(M, N, K, 1.0, 1.0, 0, A, oracle.pack_b(B, K, N), np.zeros(N, F32))
    assert np.all(C == expect)


def test_dense_i8_relu_and_epilogue_order(oracle):
    """fmax(-0, +0) = +0 with ReLU; -inf becomes -FLT_MAX without ReLU."""
    M, N, K = 16, 16, 64
    A = np.zeros((M, K), np.int8)
    Bp = oracle.pack_b(np.zeros((K, N), np.int8), K, N)
    bias = np.full(N, -0.0, F32)
    bias[1] = -np.inf
    # acc = 0 and s = -1: 0 * -1 = -0, -0 + -0 = -0; ReLU floors it to +0.
    C = oracle.dense_i8(M, N, K, -1.0, 1.0, 1, A, Bp, bias)
    assert np.all(C == 0) and not np.signbit(C[:, 0]).any()
    C = oracle.dense_i8(M, N, K, -1.0, 1.0, 0, A, Bp, bias)
    assert np.signbit(C[0, 0]) and C[0, 0] == 0
    C = oracle.dense_i8(M, N, K, 1.0, 1.0, 0, A, Bp, bias)
    assert not np.signbit(C[0, 0])  # +0 + -0 = +0
    assert C[0, 1] == -np.finfo(F32).max


def test_gemm_s8_i32_exact(oracle):
    g = np.random.default_rng(9)
    A = g.integers(-128, 128, size=(9, 70), dtype=np.int8)
    B = g.integers(-128, 128, size=(70, 13), dtype=np.int8)
    acc = oracle.gemm_s8_i32(A, B, 9, 13, 70)
    np.testing.assert_array_equal(acc, A.astype(np.int64) @ B.astype(np.int64))


# ------------------------------------------------------------ dense_fused_i8
@pytest.mark.parametrize("M,N,K,relu", [(50, 128, 784, True), (50, 10, 128, False),
                                        (3, 5, 7, True), (64, 64, 1, False)])
def test_dense_fused_matches_numpy(oracle, M, N, K, relu):
    A, B = data.gemm_inputs(M, N, K, seed=M + N + K)
    C = oracle.dense_fused_i8(M, N, K, F32(1.0), relu, A, B)
    C2, *_ = npref.dense_fused_i8(M, N, K, F32(1.0), relu, A, B)
    np.testing.assert_array_equal(C.view(np.uint32), C2.view(np.uint32))


def test_dense_fused_equals_reference_composition(oracle):
    """At scale 1.0 dense_fused_i8 equals the reference's own composition
    quantize -> pack_b_i8(Kp) -> dense_i8(zero bias) of
    tests/test_mnist_i8.cpp:198-207 and :303-314, on config 1 (MNIST MLP)."""
    x, w1, w2 = data.mnist_inputs(seed=1)
    M, K1, N1 = 50, 784, 128
    Kp = 832
    for (A, B, M_, K_, N_, relu) in [(x, w1, M, K1, N1, True)]:
        fused = oracle.dense_fused_i8(M_, N_, K_, F32(1.0), relu, A, B)
        qa, sa = oracle.quantize(A.ravel())
        qb, sb = oracle.quantize(B.ravel())
        Apad = np.zeros((64, Kp), np.int8)
        Apad[:M_, :K_] = qa.reshape(M_, K_)
        Bpad = np.zeros((Kp, N_), np.int8)
        Bpad[:K_] = qb.reshape(K_, N_)
        comp = oracle.dense_i8(M_, N_, Kp, sa, sb, 1 if relu else 0, Apad,
                               oracle.pack_b(Bpad, Kp, N_), np.zeros(N_ + 32, F32))
        np.testing.assert_array_equal(fused.view(np.uint32), comp[:M_].view(np.uint32))
    # layer 2 of the MLP: A = layer-1 output, no ReLU
    h = oracle.dense_fused_i8(M, N1, K1, F32(1.0), True, x, w1)
    out = oracle.dense_fused_i8(M, 10, N1, F32(1.0), False, h, w2)
    out2, *_ = npref.dense_fused_i8(M, 10, N1, F32(1.0), False, h, w2)
    np.testing.assert_array_equal(out, out2)


# ------------------------------------------------------------ Q8_0
def _q8_table(vocab, dim, scale_fn, val_fn):
    """The get_rows_q8_0 fixture of tests/test_remaining_ops.cpp:230-325."""
    nb = dim // 32
    W = np.zeros((vocab, nb * 34), np.uint8)
    for v in range(vocab):
        for b in range(nb):
            blk = W[v, b * 34:(b + 1) * 34]
            blk[:2] = np.array([scale_fn(v, b)], np.float16).view(np.uint8)
            blk[2:] = np.array([val_fn(q, v, b) for q in range(32)], np.int8).view(np.uint8)
    return W


def test_f16_decode_all_values(oracle):
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(F32)
    got = np.array([oracle.f16_to_f32(int(v)) for v in h], F32)
    finite = ~np.isnan(ref)
    np.testing.assert_array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.isnan(got[~finite]).all()


@pytest.mark.parametrize("dim", [32, 64])
def test_q8_0_layout_get_rows_kat(oracle, dim):
    """A one-hot x turns q8_0_gemv into the get_rows_q8_0 dequant of the
    reference test: y[v] = (float)qs * f16(d) exactly."""
    if dim == 32:
        W = _q8_table(4, 32, lambda v, b: 0.1 * (v + 1), lambda q, v, b: (q + v * 7) % 21 - 10)
    else:
        W = _q8_table(4, 64, lambda v, b: 0.05 * (v + b + 1),
                      lambda q, v, b: (q + v * 3 + b * 5) % 19 - 9)
    d, qs = npref.q8_0_blocks(W, 4, dim)
    for k in range(dim):
        x = np.zeros(dim, F32)
        x[k] = 1.0
        y = oracle.q8_0_gemv(4, dim, x, W)
        ref = (qs[:, k // 32, k % 32].astype(F32) * d[:, k // 32]).astype(F32)
        np.testing.assert_array_equal(y, ref)


def test_q8_0_r_exact_when_sums_exact(oracle):
    """Power-of-two scales and small integers: every fma and add is exact, so
    y equals the exact integer dot product."""
    M, K = 8, 256
    g = np.random.default_rng(3)
    W = np.zeros((M, K // 32 * 34), np.uint8)
    qs = g.integers(-20, 21, size=(M, K // 32, 32)).astype(np.int8)
    Wb = W.reshape(M, K // 32, 34)
    Wb[:, :, :2] = np.array([0.25], np.float16).view(np.uint8)
    Wb[:, :, 2:] = qs.view(np.uint8)
    x = g.integers(-8, 9, size=K).astype(F32)
    y = oracle.q8_0_gemv(M, K, x, W)
    exact = (qs.reshape(M, K).astype(np.int64) @ x.astype(np.int64)) * 0.25
    np.testing.assert_array_equal(y, exact.astype(F32))


def test_q8_0_r_tree_order(oracle):
    """Lane sums (1e8, 1, -1e8, 1, 0...): the FADDV tree gives
    (1e8+1)+(-1e8+1) = 0 in fp32, a left-to-right sum gives 1."""
    K = 32
    W = np.zeros((1, 34), np.uint8)
    W[0, :2] = np.array([1.0], np.float16).view(np.uint8)
    q = np.zeros(32, np.int8)
    q[[0, 1, 2, 3]] = [1, 1, -1, 1]
    W[0, 2:] = q.view(np.uint8)
    x = np.zeros(K, F32)
    x[[0, 1, 2, 3]] = [1e8, 1.0, 1e8, 1.0]
    y = oracle.q8_0_gemv(1, K, x, W)
    lanes = [F32(1e8), F32(1), F32(-1e8), F32(1)] + [F32(0)] * 12
    assert y[0] == npref.faddv16(lanes) == F32(0.0)
    s = F32(0)
    for v in lanes:
        s = F32(s + v)
    assert s == F32(1.0)


@pytest.mark.parametrize("M,K", [(3, 64), (2, 96), (1, 32)])
def test_q8_0_r_matches_exact_fma(oracle, M, K):
    W = data.q8_0_weights(M, K, seed=M * K)
    x = data.activations(1, K, seed=K)[0]
    y = oracle.q8_0_gemv(M, K, x, W)
    np.testing.assert_array_equal(y, npref.q8_0_gemv_r(M, K, x, W))


def test_q8_0_quantize_x_matches_numpy(oracle):
    K = 128
    x = data.activations(1, K, seed=8)[0]
    x[32:64] = 0.0
    qx, dx = oracle.q8_0_quantize_x(K, x)
    qx2, dx2 = npref.q8_0_quantize_x(K, x)
    np.testing.assert_array_equal(qx, qx2)
    np.testing.assert_array_equal(dx, dx2)
    assert dx[1] == 1.0


@pytest.mark.parametrize("N,K,T", [(3, 64, 1), (2, 1024, 2), (4, 96, 3)])
def test_q8_0_g_matches_exact_fma(oracle, N, K, T):
    W = data.q8_0_weights(N, K, seed=N + K)
    x = data.activations(T, K, seed=T)
    y = oracle.q8_0_mul_mat_g(N, K, T, x, W)
    np.testing.assert_array_equal(y, npref.q8_0_mul_mat_g(N, K, T, x, W))


def test_q8_0_g_close_to_r(oracle):
    """G mode differs from R only by activation quantization: within the
    bound sum_b d_w * sum|qw| * d_x/2 (plus fp32 slack)."""
    N, K = 16, 512
    W = data.q8_0_weights(N, K, seed=21)
    x = data.activations(1, K, seed=22)[0]
    yr = oracle.q8_0_gemv(N, K, x, W)
    yg = oracle.q8_0_mul_mat_g(N, K, 1, x, W)[0]
    d, qs = npref.q8_0_blocks(W, N, K)
    _, dx = oracle.q8_0_quantize_x(K, x)
    bound = (d * np.abs(qs.astype(F32)).sum(-1) * (dx[None, :] / 2)).sum(-1)
    assert np.all(np.abs(yg - yr) <= bound * 1.001 + 1e-5)


# ---------------------------------------------------------------- cblas integer GEMMs (0x61-0x63)
def _igemm_operands(variant, M, N, K, lda, ldb, tb, seed):
    g = np.random.default_rng(seed)
    au, bu = variant in (1, 2), variant == 1
    A = g.integers(0 if au else -128, 256 if au else 128, size=M * lda).astype(np.uint8 if au else np.int8)
    nb = (N * ldb) if tb else (K * ldb)
    B = g.integers(0 if bu else -128, 256 if bu else 128, size=nb).astype(np.uint8 if bu else np.int8)
    return A, B


@pytest.mark.parametrize("variant", [0, 1, 2])
@pytest.mark.parametrize("tb", [0, 1])
@pytest.mark.parametrize("M,N,K", [(16, 32, 64), (5, 7, 130), (33, 40, 256)])
def test_cblas_igemm_matches_int64_numpy(oracle, variant, tb, M, N, K):
    """Every variant and transB against an exact int64 numpy product over the
    K/64 whole blocks, then the two float32 roundings (scvtf, fmul alpha)."""
    lda, ldb, ldc = K + 3, (K + 5) if tb else (N + 2), N + 1
    A, B = _igemm_operands(variant, M, N, K, lda, ldb, tb, seed=M + N + K + variant)
    Ke = K // 64 * 64
    Am = A.reshape(M, lda)[:, :Ke].astype(np.int64)
    Bm = (B.reshape(N, ldb)[:, :Ke].T if tb else B.reshape(K, ldb)[:Ke, :N]).astype(np.int64)
    acc = (Am @ Bm).astype(np.int64)
    assert np.abs(acc).max() < 2 ** 31
    want = (acc.astype(np.float32) * F32(-0.75)).astype(F32)
    C0 = np.full((M, ldc), 3.0, F32)
    got = oracle.cblas_igemm(variant, tb << 1, M, N, K, lda, ldb, ldc, -0.75, 0.0, A, B, C0)
    np.testing.assert_array_equal(got[:, :N].view(np.uint32), want.view(np.uint32))
    assert (got[:, N:] == 3.0).all()  # columns past N are never written


def test_cblas_igemm_transb_equals_transposed_copy(oracle):
    M, N, K = 9, 20, 192
    A, B = _igemm_operands(0, M, N, K, K, N, 0, seed=1)
    Bt = np.ascontiguousarray(B.reshape(K, N).T)
    C0 = np.zeros((M, N), F32)
    c0 = oracle.cblas_igemm(0, 0, M, N, K, K, N, N, 1.0, 0.0, A, B, C0)
    c1 = oracle.cblas_igemm(0, 2, M, N, K, K, K, N, 1.0, 0.0, A, Bt, C0)
    assert np.array_equal(c0, c1)


def test_cblas_igemm_beta_seeds_accumulator_bits(oracle):
    """K < 64 leaves no products: the handler stores fl(fl32(seed) * alpha),
    seed = the bits of fl(beta * C) whenever beta's bits are nonzero
    (bytecode_interpreter.s:8402-8488), so beta = -0.0 seeds too."""
    A = np.zeros(64, np.int8)
    C0 = np.array([[1.0, 2.0, -1.5]], F32)
    out = oracle.cblas_igemm(0, 0, 1, 3, 32, 32, 3, 3, 1.0, 1.0, A, A, C0)
    assert out[0, 0] == F32(0x3F800000)           # bits of 1.0 as an integer
    assert out[0, 1] == F32(0x40000000)
    assert out[0, 2] == F32(np.int32(np.uint32(0xBFC00000)))  # negative as int32
    out = oracle.cblas_igemm(0, 0, 1, 3, 32, 32, 3, 3, 1.0, -0.0, A, A, C0)
    assert out[0, 0] == F32(-2.0 ** 31) and out[0, 2] == 0.0  # -0.0 -> INT32_MIN, +0.0 -> 0
    out = oracle.cblas_igemm(0, 0, 1, 3, 32, 32, 3, 3, 2.0, 0.0, A, A, C0)
    assert (out == 0.0).all()
    # the BLAS form on the same inputs: alpha*0 + beta*C
    out = oracle.cblas_igemm(0, 0, 1, 3, 32, 32, 3, 3, 1.0, 1.0, A, A, C0, semantics=1)
    assert np.array_equal(out, C0)


def test_cblas_igemm_beta_seed_adds_to_products(oracle):
    """With products the seed and the sum wrap together: seed + acc as int32."""
    M, N, K = 4, 8, 64
    A, B = _igemm_operands(0, M, N, K, K, N, 0, seed=5)
    C0 = np.random.default_rng(6).standard_normal((M, N)).astype(F32)
    acc = A.reshape(M, K).astype(np.int64) @ B.reshape(K, N).astype(np.int64)
    seed = (C0 * F32(0.5)).astype(F32).view(np.int32).astype(np.int64)
    tot = ((acc + seed + 2 ** 31) % 2 ** 32 - 2 ** 31).astype(np.int64)
    want = (tot.astype(np.float32) * F32(1.0)).astype(F32)
    got = oracle.cblas_igemm(0, 0, M, N, K, K, N, N, 1.0, 0.5, A, B, C0)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    blas = oracle.cblas_igemm(0, 0, M, N, K, K, N, N, 1.0, 0.5, A, B, C0, semantics=1)
    np.testing.assert_array_equal(blas, (acc.astype(F32) + (C0 * F32(0.5)).astype(F32)).astype(F32))


def test_cblas_igemm_transa_handler_addressing(oracle):
    """transA: the handler adds the k offset to A + ti and steps rows by lda,
    so the first 16 rows read exactly what transA = 0 reads, and row 16 + r
    starts at byte 16 + r * lda (not A^T)."""
    M, N, K, lda = 20, 8, 64, 80
    size = 15 * lda + 16 + K
    g = np.random.default_rng(9)
    A = g.integers(-128, 128, size=size).astype(np.int8)
    B = g.integers(-128, 128, size=K * N).astype(np.int8)
    C0 = np.zeros((M, N), F32)
    t1 = oracle.cblas_igemm(0, 1, M, N, K, lda, N, N, 1.0, 0.0, A, B, C0)
    rows = np.stack([A[(i % 16) * lda + (i - i % 16):][:K] for i in range(M)]).astype(np.int64)
    want = (rows @ B.reshape(K, N).astype(np.int64)).astype(F32)
    assert np.array_equal(t1, want)
    t0 = oracle.cblas_igemm(0, 0, 16, N, K, lda, N, N, 1.0, 0.0, A, B, C0[:16])
    assert np.array_equal(t1[:16], t0)
    # the BLAS form: A is K x M with stride lda
    At = g.integers(-128, 128, size=K * lda).astype(np.int8)
    tb = oracle.cblas_igemm(0, 1, M, N, K, lda, N, N, 1.0, 0.0, At, B, C0, semantics=1)
    want = (At.reshape(K, lda)[:, :M].T.astype(np.int64) @ B.reshape(K, N).astype(np.int64)).astype(F32)
    assert np.array_equal(tb, want)
