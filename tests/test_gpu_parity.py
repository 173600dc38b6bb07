"""GPU parity: libane_amd.so (through the C ABI) against the CPU oracle on the
same seeded inputs.  Integer/byte results and the fp32 outputs of the
reference opcodes are compared bit for bit (the epilogues are single-rounding
fp32 sequences, so bit equality is the bar; NaNs compare as NaN)."""
import ctypes

import numpy as np
import pytest

from tests import data

pytestmark = pytest.mark.gpu
F32 = np.float32


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def zeros(n, dtype):
    import torch

    return torch.zeros(n, dtype=dtype, device="cuda")


def bits(a):
    a = np.ascontiguousarray(a, F32)
    return a.view(np.uint32)


def assert_f32_identical(got, want):
    got = np.asarray(got, F32)
    want = np.asarray(want, F32)
    assert got.shape == want.shape
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(bits(got)[~nan], bits(want)[~nan])


def mul_mat_both_routes(ane, N, K, T, x, W):
    """y of ane.q8_0_mul_mat twice: with the full workspace of an N-row
    matrix (ane_hip_q8_0_mul_mat_workspace_size_n, every route allowed) and
    with the minimum one (the residue-split route then not taken)."""
    import torch

    xd, Wd = dev(x), dev(W)
    outs = []
    for n_aware in (True, False):
        wsb = ane.q8_0_mul_mat_workspace_size(K, T, N=N if n_aware else None)
        ws = torch.empty(max(wsb, 256), dtype=torch.uint8, device="cuda")
        y = zeros(T * N, torch.float32)
        ane.q8_0_mul_mat(N, K, T, xd, Wd, y, workspace=ws)
        outs.append(host(y).reshape(T, N))
    return outs


# ---------------------------------------------------------------- MFMA core
@pytest.mark.parametrize("M,N,K", [(1, 1, 16), (32, 32, 32), (50, 130, 784), (128, 128, 128),
                                   (300, 200, 1008), (257, 129, 4096), (64, 512, 48),
                                   # 256 x 256 tile kernel: full, partial and odd tile grids
                                   (256, 256, 128), (1000, 600, 896), (513, 257, 4096),
                                   (2048, 1536, 256), (768, 2304, 1152),
                                   # few-row kernel: partial 64-byte steps, ragged columns, 1..8 row blocks
                                   (5, 17, 80), (100, 1000, 2064), (128, 1024, 4096), (17, 33, 16),
                                   (48, 300, 592),
                                   # 256-tiles again once they fill every CU: full and ragged grids
                                   (4096, 4096, 128), (4352, 4096, 64),
                                   # K an odd multiple of 64: the last 128-byte slice half zeros
                                   # (256-tiles, 128-tiles, both with a ragged grid)
                                   (4096, 4096, 192), (4100, 4096, 4160), (1000, 600, 960),
                                   (513, 257, 4160),
                                   # more 128-tiles than CUs (the 2-stage ring, two per CU;
                                   # the shapes above with fewer take the 3-stage ring)
                                   (2048, 2304, 192), (1100, 4000, 320)])
def test_gemm_s8_i32_exact(ane, M, N, K):
    import torch

    g = np.random.default_rng(M + N + K)
    A = g.integers(-128, 128, size=(M, K), dtype=np.int8)
    Bt = g.integers(-128, 128, size=(N, K), dtype=np.int8)
    acc = torch.zeros((M, N), dtype=torch.int32, device="cuda")
    ane.gemm_s8_i32(dev(A), dev(Bt), acc, M, N, K)
    want = A.astype(np.int64) @ Bt.astype(np.int64).T
    np.testing.assert_array_equal(host(acc), want.astype(np.int32))


@pytest.mark.parametrize("M,N,K,pad", [(4096, 4096, 192, 64), (1000, 600, 960, 48), (4100, 4096, 4160, 16)])
def test_gemm_s8_i32_padded_rows(ane, M, N, K, pad):
    """Rows wider than K (lda = ldb = K + pad) filled with nonzero bytes past
    K, K an odd multiple of 64: the contraction kernels run 128-byte K slices
    and must send the last slice's upper half out of range rather than read
    the padding (256-tiles, then 128-tiles)."""
    import torch

    g = np.random.default_rng(M + 7 * K)
    ld = K + pad
    A = g.integers(-128, 128, size=(M, ld), dtype=np.int8)
    Bt = g.integers(-128, 128, size=(N, ld), dtype=np.int8)
    A[:, K:] = 77
    Bt[:, K:] = -91
    acc = torch.zeros((M, N), dtype=torch.int32, device="cuda")
    ane.gemm_s8_i32(dev(A), dev(Bt), acc, M, N, K, lda=ld, ldb=ld)
    want = A[:, :K].astype(np.int64) @ Bt[:, :K].astype(np.int64).T
    np.testing.assert_array_equal(host(acc), want.astype(np.int32))


# ---------------------------------------------------------------- quantize
@pytest.mark.parametrize("count", [1, 16, 17, 1000, 4096 + 5, 1 << 20])
def test_quantize_opcode_parity(ane, oracle, count):
    n = max(16, -(-count // 16) * 16)
    x = np.random.default_rng(count).standard_normal(n).astype(F32) * F32(3)
    x[:4] = [0.0, -0.0, 1e-41, -7.5]
    q_ref, s_ref = oracle.quantize(x, count)
    src, dst, sc = dev(x), zeros(n, ane_torch_int8()), zeros(1, ane_torch_f32())
    ane.stream_exec(ane.rec_quantize(count, src, dst, sc))
    np.testing.assert_array_equal(host(dst), q_ref)
    assert host(sc)[0].tobytes() == F32(s_ref).tobytes()


def ane_torch_int8():
    import torch

    return torch.int8


def ane_torch_f32():
    import torch

    return torch.float32


def test_quantize_host_scale_pointer(ane, oracle):
    """The reference writes the scale through a host pointer
    (tests/test_mnist_i8.cpp:307-308); a host scale_out is staged back."""
    x = np.random.default_rng(1).standard_normal(4096).astype(F32)
    q_ref, s_ref = oracle.quantize(x)
    scale = np.zeros(1, F32)
    dst = zeros(4096, ane_torch_int8())
    ane.stream_exec(ane.rec_quantize(4096, dev(x), dst, scale.ctypes.data))
    assert scale[0] == s_ref
    np.testing.assert_array_equal(host(dst), q_ref)


def test_quantize_nan_and_zero(ane):
    x = np.ones(64, F32)
    x[9] = np.nan
    dst, sc = zeros(64, ane_torch_int8()), zeros(1, ane_torch_f32())
    ane.stream_exec(ane.rec_quantize(64, dev(x), dst, sc))
    assert np.isnan(host(sc)[0]) and not host(dst).any()
    ane.stream_exec(ane.rec_quantize(64, dev(np.zeros(64, F32)), dst, sc))
    assert host(sc)[0] == 1.0 and not host(dst).any()


def test_quantize_exact_count_kernel_abi(ane, oracle):
    x = np.random.default_rng(3).standard_normal(1003).astype(F32)
    q_ref, s_ref = oracle.quantize_exact(x)
    dst, sc = zeros(1003, ane_torch_int8()), zeros(1, ane_torch_f32())
    ane.quantize_fp32_i8(dev(x), dst, sc, count=1003, pad16=False)
    np.testing.assert_array_equal(host(dst), q_ref)
    assert host(sc)[0] == s_ref


def test_dequantize_parity(ane, oracle):
    q = np.random.default_rng(2).integers(-128, 128, size=4096 + 16, dtype=np.int8)
    out = zeros(q.size, ane_torch_f32())
    ane.stream_exec(ane.rec_dequantize(q.size - 3, 0.0173, dev(q), out))
    ref = oracle.dequantize(q, F32(0.0173), q.size - 3)
    assert_f32_identical(host(out)[: ref.size], ref)


def test_channelwise_parity(ane, oracle):
    rows, cols = 33, 100
    cpad = 112
    x = np.random.default_rng(4).standard_normal(rows * cpad).astype(F32)
    x[cpad * 5: cpad * 6] = 0.0
    q_ref, s_ref = oracle.channelwise(x, rows, cols)
    dst, sc = zeros(rows * cpad, ane_torch_int8()), zeros(rows, ane_torch_f32())
    ane.stream_exec(ane.rec_channelwise(rows, cols, dev(x), dst, sc))
    np.testing.assert_array_equal(host(dst), q_ref)
    np.testing.assert_array_equal(host(sc), s_ref)


@pytest.mark.parametrize("K,N", [(832, 128), (128, 16), (5, 17), (4096, 4096), (100, 10)])
def test_pack_b_parity(ane, oracle, K, N):
    B = np.random.default_rng(K + N).integers(-128, 128, size=(K, N), dtype=np.int8)
    ref = oracle.pack_b(B, K, N)
    dst = zeros(ref.size, ane_torch_int8())
    ane.stream_exec(ane.rec_pack_b(K, N, dev(B), dst))
    np.testing.assert_array_equal(host(dst), ref)


# ---------------------------------------------------------------- dense_i8 / u8s8
def _dense_inputs(M, N, K, seed, unsigned_a):
    g = np.random.default_rng(seed)
    Kp = -(-K // 64) * 64
    Mp = max(16, -(-M // 16) * 16)
    if unsigned_a:
        A = g.integers(0, 256, size=(Mp, Kp), dtype=np.uint8)
    else:
        A = g.integers(-127, 128, size=(Mp, Kp), dtype=np.int8)
    B = np.zeros((Kp, N), np.int8)
    B[:K] = g.integers(-127, 128, size=(K, N), dtype=np.int8)
    bias = g.standard_normal(max(N, 1)).astype(F32)
    return A, B, bias, Mp, Kp


@pytest.mark.parametrize("M,N,K,unsigned_a", [
    (50, 128, 832, True), (50, 16, 128, False), (1, 10, 64, False), (17, 33, 100, False),
    (16, 32, 64, True), (0, 5, 64, False), (200, 300, 1000, False), (129, 257, 4096, True),
])
def test_dense_i8_parity(ane, oracle, M, N, K, unsigned_a):
    A, B, bias, Mp, Kp = _dense_inputs(M, N, K, M * 3 + N + K, unsigned_a)
    Bp = oracle.pack_b(B, Kp, N)
    dA, dBp, dbias = dev(A), dev(Bp), dev(bias)
    for flags in (0, 1):
        ref = oracle.dense_i8(M, N, K, F32(0.013), F32(0.021), flags, A, Bp, bias, unsigned_a)
        C = zeros(Mp * N, ane_torch_f32())
        ane.stream_exec(ane.rec_dense_i8(M, N, K, 0.013, 0.021, bool(flags), dA, dBp, dbias, C,
                                         unsigned_a=unsigned_a))
        assert_f32_identical(host(C).reshape(Mp, N), ref)


def test_dense_i8_igemm_kat_on_gpu(ane):
    """tests/test_remaining_ops.cpp:131-184 pattern, exact integers."""
    M, N, K = 16, 32, 64
    A = ((np.arange(M * K) % 11) - 5).astype(np.int8).reshape(M, K)
    B = ((np.arange(K * N) % 13) - 6).astype(np.int8).reshape(K, N)
    ref = (A.astype(np.int64) @ B.astype(np.int64)).astype(F32)
    Bp = zeros(K * N * 2, ane_torch_int8())
    ane.stream_exec(ane.rec_pack_b(K, N, dev(B), Bp))
    C = zeros(M * N, ane_torch_f32())
    ane.stream_exec(ane.rec_dense_i8(M, N, K, 1.0, 1.0, False, dev(A), Bp, dev(np.zeros(N, F32)), C))
    np.testing.assert_array_equal(host(C).reshape(M, N), ref)


def test_mnist_i8_composition(ane, oracle):
    """The reference's int8 forward (tests/test_mnist_i8.cpp:198-207, 303-314):
    quantize+pack W, dense_u8s8 on raw pixels, quantize hidden, dense_i8 with
    the -1000 logit mask, as one multi-record stream."""
    g = np.random.default_rng(12)
    B, INP_K, HID, HID_K, OUT_PAD = 50, 832, 128, 128, 16
    x_u8 = np.zeros((64, INP_K), np.uint8)
    x_u8[:B, :784] = g.integers(0, 256, size=(B, 784))
    W1 = np.zeros((INP_K, HID), F32)
    W1[:784] = g.standard_normal((784, HID)) * 0.05
    W2 = (g.standard_normal((HID_K, OUT_PAD)) * 0.05).astype(F32)
    logit_bias = np.array([0] * 10 + [-1000.0] * 6, F32)
    zero_bias = np.zeros(INP_K, F32)
    # oracle
    w1q, s1 = oracle.quantize(W1.ravel())
    w1p = oracle.pack_b(w1q, INP_K, HID)
    w2q, s2 = oracle.quantize(W2.ravel())
    w2p = oracle.pack_b(w2q, HID_K, OUT_PAD)
    h = oracle.dense_i8(B, HID, INP_K, F32(1 / 255), s1, 1, x_u8, w1p, zero_bias, unsigned_a=True)
    hq, sh = oracle.quantize(h[:B].ravel(), B * HID_K)
    hq_pad = np.zeros((64, HID_K), np.int8)
    hq_pad[:B] = hq.reshape(B, HID_K)
    logits = oracle.dense_i8(B, OUT_PAD, HID_K, sh, s2, 0, hq_pad, w2p, logit_bias)
    # device, same call sequence
    import torch

    dW1, dW2 = dev(W1), dev(W2)
    dw1q = zeros(INP_K * HID, torch.int8)
    dw1p = zeros(oracle.packed_b_size(INP_K, HID), torch.int8)
    dw2q = zeros(HID_K * OUT_PAD, torch.int8)
    dw2p = zeros(oracle.packed_b_size(HID_K, OUT_PAD), torch.int8)
    scales = zeros(3, torch.float32)
    ane.stream_exec([
        ane.rec_quantize(INP_K * HID, dW1, dw1q, scales.data_ptr()),
        ane.rec_pack_b(INP_K, HID, dw1q, dw1p),
        ane.rec_quantize(HID_K * OUT_PAD, dW2, dw2q, scales.data_ptr() + 4),
        ane.rec_pack_b(HID_K, OUT_PAD, dw2q, dw2p),
    ])
    sc = host(scales)
    assert sc[0] == s1 and sc[1] == s2
    dh = zeros(64 * HID, torch.float32)
    ane.stream_exec(ane.rec_dense_i8(B, HID, INP_K, 1 / 255, float(sc[0]), True, dev(x_u8), dw1p,
                                     dev(zero_bias), dh, unsigned_a=True))
    assert_f32_identical(host(dh).reshape(64, HID), h)
    dhq = zeros(64 * HID_K, torch.int8)
    sh_host = np.zeros(1, F32)
    ane.stream_exec(ane.rec_quantize(B * HID_K, dh, dhq, sh_host.ctypes.data))
    assert sh_host[0] == sh
    dlog = zeros(64 * OUT_PAD, torch.float32)
    ane.stream_exec(ane.rec_dense_i8(B, OUT_PAD, HID_K, float(sh_host[0]), float(sc[1]), False, dhq, dw2p,
                                     dev(logit_bias), dlog))
    assert_f32_identical(host(dlog).reshape(64, OUT_PAD), logits)


# ---------------------------------------------------------------- dense_fused_i8
def test_dense_fused_mnist_mlp(ane, oracle):
    """Config 1: 50x784 -> 128 (ReLU) -> 10, through stream_exec."""
    x, w1, w2 = data.mnist_inputs(seed=1)
    h_ref = oracle.dense_fused_i8(50, 128, 784, F32(1.0), True, x, w1)
    o_ref = oracle.dense_fused_i8(50, 10, 128, F32(1.0), False, h_ref, w2)
    import torch

    h = zeros(50 * 128, torch.float32)
    o = zeros(50 * 10, torch.float32)
    ane.stream_exec([ane.rec_dense_fused_i8(50, 128, 784, 1.0, True, dev(x), dev(w1), h),
                     ane.rec_dense_fused_i8(50, 10, 128, 1.0, False, h, dev(w2), o)])
    assert_f32_identical(host(h).reshape(50, 128), h_ref)
    assert_f32_identical(host(o).reshape(50, 10), o_ref)


@pytest.mark.parametrize("M,N,K,relu,scale", [(3, 5, 7, True, 1.0), (64, 64, 1, False, 2.5),
                                              (1, 4096, 4096, True, 1.0), (16, 4096, 4096, False, 1.0),
                                              (129, 257, 1000, False, 0.75), (7, 9, 0, True, 1.0),
                                              (300, 700, 333, True, 1.0), (1024, 512, 4096, False, 1.0),
                                              (128, 4096, 4096, True, 1.0), (33, 1000, 4000, True, 1.0),
                                              # few rows on split K (65..128 rows): ragged columns and K,
                                              # two to four splits, a range shorter than its share, and
                                              # one 128-byte slice (no split)
                                              (100, 1000, 4000, False, 1.0), (65, 130, 640, True, 0.5),
                                              (127, 4100, 2048, True, 1.0), (96, 256, 128, False, 1.0),
                                              (120, 640, 1200, True, 1.0), (70, 512, 1152, False, 1.0)])
def test_dense_fused_parity(ane, oracle, M, N, K, relu, scale):
    """dense_fused_i8 through stream_exec against the oracle, bit for bit."""
    A, B = data.gemm_inputs(M, N, K, seed=M + N + K)
    ref = oracle.dense_fused_i8(M, N, K, F32(scale), relu, A, B)
    import torch

    C = zeros(M * N, torch.float32)
    ane.stream_exec(ane.rec_dense_fused_i8(M, N, K, scale, relu, dev(A), dev(B), C))
    assert_f32_identical(host(C).reshape(M, N), ref)


_SPECIAL = [(c, *shape) for c in ("a_nan", "b_inf", "a_neg_inf", "a_zero", "b_tiny")
            for shape in ((129, 257, 1000), (256, 512, 2048), (256, 2048, 2048))]
_SPECIAL += [("a_nan", 5000, 64, 4096), ("b_inf", 5000, 64, 4096), ("a_neg_inf", 5000, 64, 4096)]


@pytest.mark.parametrize("case,M,N,K", _SPECIAL)
def test_dense_fused_special_operands(ane, oracle, case, M, N, K):
    """The fused max|x| and quantize passes on operands the quantizer
    special-cases: a NaN or an infinity (NaN or infinite per-tensor scale),
    an all-zero tensor (the zero guard) and a tensor of denormals and signed
    zeros only (127 / amax overflows to +inf, so 0 * inf reaches the
    quantizer).  256 x 2048 x 2048 (18 MiB of operands) takes the one-launch
    resident quantizer, the others the two-pass one.  5000 x 64 x 4096 takes
    the resident quantizer with A's share larger than LDS and registers hold
    (its rest re-read after the B tiles on the exact pack4 route that a
    non-finite scale selects); the NaN sits in that re-read rest."""
    import torch

    A, B = data.gemm_inputs(M, N, K, seed=M + K)
    if case == "a_nan":
        A[M // 2, K // 3] = np.nan
        if M == 5000:  # in workgroup 0's re-read rest: float4 15232 + 3 * 512 onward of its share
            A.ravel()[4 * (15232 + 3 * 512) + 7] = np.nan
    elif case == "b_inf":
        B[K - 1, N // 2] = np.inf
    elif case == "a_neg_inf":
        A[0, 0] = -np.inf
    elif case == "a_zero":
        A[:] = 0.0
    else:
        B[:] = np.where(np.arange(K * N).reshape(K, N) % 3 == 0, -0.0, F32(1e-40))
        B[1, 2] = F32(-3e-39)
    oracle.set_threads(0)
    try:
        ref = oracle.dense_fused_i8(M, N, K, F32(1.0), True, A, B)
    finally:
        oracle.set_threads(1)
    C = zeros(M * N, torch.float32)
    ane.stream_exec(ane.rec_dense_fused_i8(M, N, K, 1.0, True, dev(A), dev(B), C))
    assert_f32_identical(host(C).reshape(M, N), ref)


_FEW_TILE = [(50, 128, 784, True, 1.0, True), (50, 10, 128, False, 1.0, True), (1, 1, 1, True, 1.0, True),
             (3, 5, 7, False, 2.5, True), (17, 33, 1023, True, 0.75, True), (16, 16, 1024, False, 1.0, True),
             (64, 100, 64, True, 1.0, True), (31, 47, 65, False, 1.0, True), (128, 128, 1000, True, 1.0, True),
             (100, 1, 513, False, 1.0, True), (256, 512, 1024, True, 1.0, True),
             # past the route's bounds: K > 1024, more than 512 tiles
             (17, 33, 1025, True, 0.75, False), (512, 512, 256, False, 1.0, False)]


@pytest.mark.parametrize("M,N,K,relu,scale,few", _FEW_TILE)
def test_dense_fused_few_tile_route(ane, oracle, M, N, K, relu, scale, few):
    """dense_fused_i8 on small operands (K <= 1024, at most 512 tiles of
    16 x 16 in C: the MNIST layers among them) runs as the absmax pass plus
    one launch that quantizes each tile's rows and columns into LDS and
    contracts them.  Bit for bit against the oracle (C and the two scales),
    with ragged M, N and K (K % 4 != 0 reads A element by element), the
    largest K, one column.  That launch leaves the workspace's qA bytes as
    they were (filled with 0x5A here), which shows the route was taken; the
    shapes past its bounds take the two-launch quantizer, which writes them."""
    import torch

    A, B = data.gemm_inputs(M, N, K, seed=M * 7 + N + K)
    ref = oracle.dense_fused_i8(M, N, K, F32(scale), relu, A, B)
    _, sa = oracle.quantize_exact(A.ravel())
    _, sb = oracle.quantize_exact(B.ravel())
    wsb = ane.dense_fused_i8_workspace_size(M, N, K)
    ws = torch.full((wsb,), 0x5A, dtype=torch.uint8, device="cuda")
    C = zeros(M * N, torch.float32)
    sc = zeros(2, torch.float32)
    ane.dense_fused_i8(M, N, K, scale, relu, dev(A), dev(B), C, scales_out=sc, workspace=ws)
    assert_f32_identical(host(C).reshape(M, N), ref)
    assert host(sc).tobytes() == np.array([sa, sb], F32).tobytes()
    qa = host(ws)[12800: 12800 + M * K]  # qA of the workspace layout (gemm_i8.hip, fused_layout)
    assert (qa == 0x5A).all() == few


@pytest.mark.parametrize("case", ["a_nan", "b_inf", "a_neg_inf", "a_zero", "b_tiny", "b_nan_tail"])
def test_dense_fused_few_tile_special_operands(ane, oracle, case):
    """The few-tile route on the operands the quantizer special-cases (as
    test_dense_fused_special_operands): a NaN or an infinity (the exact
    pack4 route), an all-zero tensor, a tensor of denormals and signed zeros
    (127 / amax = +inf), and a NaN in B's last row and column (the ragged
    edge of the last tile), through stream_exec at 50 x 130 x 783."""
    import torch

    M, N, K = 50, 130, 783
    A, B = data.gemm_inputs(M, N, K, seed=11)
    if case == "a_nan":
        A[M // 2, K // 3] = np.nan
    elif case == "b_inf":
        B[K - 1, N // 2] = np.inf
    elif case == "a_neg_inf":
        A[0, 0] = -np.inf
    elif case == "a_zero":
        A[:] = 0.0
    elif case == "b_tiny":
        B[:] = np.where(np.arange(K * N).reshape(K, N) % 3 == 0, -0.0, F32(1e-40))
        B[1, 2] = F32(-3e-39)
    else:
        B[K - 1, N - 1] = np.nan
    ref = oracle.dense_fused_i8(M, N, K, F32(1.0), True, A, B)
    C = zeros(M * N, torch.float32)
    ane.stream_exec(ane.rec_dense_fused_i8(M, N, K, 1.0, True, dev(A), dev(B), C))
    assert_f32_identical(host(C).reshape(M, N), ref)


@pytest.mark.parametrize("M,N,K", [(256, 2048, 2048), (5000, 64, 4096), (777, 2048, 4096), (64, 2048, 2048)])
def test_dense_fused_resident_quantizer_shapes(ane, oracle, M, N, K):
    """Shapes on the one-launch resident quantizer (K % 128 == 0, N % 64 == 0,
    at least 12 MiB of operands): a workgroup's share of A all in LDS
    (256, 777 and 64 rows; 777 rows give every workgroup a ragged share), and
    past LDS into registers and the batched re-read (5000 x 4096: 20,000
    float4 per workgroup, the last batch ragged)."""
    import torch

    A, B = data.gemm_inputs(M, N, K, seed=M + 3 * N + K)
    oracle.set_threads(0)
    try:
        ref = oracle.dense_fused_i8(M, N, K, F32(1.0), False, A, B)
    finally:
        oracle.set_threads(1)
    C = zeros(M * N, torch.float32)
    ane.stream_exec(ane.rec_dense_fused_i8(M, N, K, 1.0, False, dev(A), dev(B), C))
    assert_f32_identical(host(C).reshape(M, N), ref)


@pytest.mark.parametrize("M,N,K", [(256, 2048, 2048), (1, 4096, 4096), (5000, 64, 4096), (300, 700, 333)])
def test_dense_fused_quantize_phase_bytes(ane, oracle, M, N, K):
    """The quantize phase alone (ane_hip_dense_fused_i8_quantize), byte for
    byte: the workspace's qA (M x Kp) and qBt (N x Kp, B transposed), zeros
    for k >= K, and the two scales, against the oracle's per-tensor
    quantization of A and of B.  The first three shapes take the one-launch
    resident quantizer (1 row; 5000 rows, whose workgroup shares run past
    LDS and registers), the last the two-pass one (K % 128 != 0).
    Workspace layout (gemm_i8.hip, fused_layout): scales at 0, the partial
    maxima at 256 (2 x 1024 uint32) and the wait record after them
    (1 + 1024 uint32), qA at 12800, qBt after qA rounded up to 256 bytes;
    Kp = ceil(K / 128) * 128.  The wait record holds 0 entries on the
    two-pass route and one zero per workgroup on the resident one."""
    import torch

    A, B = data.gemm_inputs(M, N, K, seed=M + N + 5)
    qa_ref, sa = oracle.quantize_exact(A.ravel())
    qb_ref, sb = oracle.quantize_exact(B.ravel())
    Kp = -(-K // 128) * 128
    want_a = np.zeros((M, Kp), np.int8)
    want_a[:, :K] = qa_ref[: M * K].reshape(M, K)
    want_b = np.zeros((N, Kp), np.int8)
    want_b[:, :K] = qb_ref[: K * N].reshape(K, N).T
    ws = torch.full((ane.dense_fused_i8_workspace_size(M, N, K),), 0x5A, dtype=torch.uint8, device="cuda")
    sc = zeros(2, torch.float32)
    ane.dense_fused_i8_quantize(M, N, K, dev(A), dev(B), ws, scales_out=sc)
    w = host(ws)
    rec = w[256 + 8192: 256 + 8192 + 4 * 1025].view(np.uint32)
    resident = K % 128 == 0 and N % 64 == 0 and 4 * (M * K + K * N) >= 12 << 20
    assert (rec[0] > 0) == resident and rec[0] <= 1024
    assert not rec[1: 1 + rec[0]].any()
    off_a = 12800
    off_b = off_a + -(-(M * Kp) // 256) * 256
    got_a = w[off_a: off_a + M * Kp].view(np.int8).reshape(M, Kp)
    got_b = w[off_b: off_b + N * Kp].view(np.int8).reshape(N, Kp)
    np.testing.assert_array_equal(got_a, want_a)
    np.testing.assert_array_equal(got_b, want_b)
    assert host(sc).tobytes() == np.array([sa, sb], F32).tobytes()


_STRIP = [(1, 4096, 4096, True, 1.0), (16, 4096, 4096, False, 1.0), (5, 4096, 3072, False, 2.5),
          (9, 3072, 4096, True, 0.75), (4, 4096, 1536, True, 1.0), (3, 2048, 4096, False, 1.0),
          (8, 4096, 4096, True, 1.0), (12, 2048, 2048 * 3, False, 1.0), (2, 8192, 2048, True, 1.0)]


@pytest.mark.parametrize("M,N,K,relu,scale", _STRIP)
def test_dense_fused_strip_route(ane, oracle, M, N, K, relu, scale):
    """dense_fused_i8 with at most 16 rows, K % 512 == 0 and at least 12 MiB
    of B runs in one launch, each CU holding a 16-column strip of B (qBt
    never written).  Bit for bit against the oracle (C and both scales):
    rows loaded before the wait only (M <= 4), with the second batch (5-8)
    and the third (9-16), K of 1536 (rows of 384 float4, half a thread's
    second load), fewer strips than workgroups (N = 2048: half the
    workgroups hold A's share and wait only), K past 4096 (12 x 2048 x
    6144) and more strips than a 256-CU device has workgroups (2 x 8192 x
    2048), which the route does not take.  The workspace's qA bytes stay as
    they were (0x5A) exactly when the strip route ran."""
    import torch

    A, B = data.gemm_inputs(M, N, K, seed=M * 5 + N + K)
    oracle.set_threads(0)
    try:
        ref = oracle.dense_fused_i8(M, N, K, F32(scale), relu, A, B)
    finally:
        oracle.set_threads(1)
    _, sa = oracle.quantize_exact(A.ravel())
    _, sb = oracle.quantize_exact(B.ravel())
    wsb = ane.dense_fused_i8_workspace_size(M, N, K)
    ws = torch.full((wsb,), 0x5A, dtype=torch.uint8, device="cuda")
    C = zeros(M * N, torch.float32)
    sc = zeros(2, torch.float32)
    ane.dense_fused_i8(M, N, K, scale, relu, dev(A), dev(B), C, scales_out=sc, workspace=ws)
    assert_f32_identical(host(C).reshape(M, N), ref)
    assert host(sc).tobytes() == np.array([sa, sb], F32).tobytes()
    qa = host(ws)[12800: 12800 + M * K]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert (qa == 0x5A).all() == (K <= 4096 and N // 16 <= cus)


@pytest.mark.parametrize("case", ["a_nan", "b_inf", "a_neg_inf", "a_zero", "b_tiny", "b_nan_last",
                                  "a_nan_row12", "a_inf_row15"])
def test_dense_fused_strip_special_operands(ane, oracle, case):
    """The strip route (7 x 4096 x 4096; 16 rows for the last two cases) on
    the operands the quantizer special-cases: a NaN or an infinity (the exact
    pack4 for that tensor), an all-zero A, a B of denormals and signed zeros
    (127 / amax = +inf), a NaN in B's last row and column (the last strip's
    last thread), and a NaN or an infinity in A's rows 8-15, which are
    loaded after the grid-wide wait."""
    import torch

    M, N, K = (16 if case in ("a_nan_row12", "a_inf_row15") else 7), 4096, 4096
    A, B = data.gemm_inputs(M, N, K, seed=13)
    if case == "a_nan_row12":
        A[12, K - 5] = np.nan
    elif case == "a_inf_row15":
        A[15, 600] = -np.inf
    elif case == "a_nan":
        A[M - 1, K // 3] = np.nan
    elif case == "b_inf":
        B[K // 2, N // 3] = np.inf
    elif case == "a_neg_inf":
        A[0, 0] = -np.inf
    elif case == "a_zero":
        A[:] = 0.0
    elif case == "b_tiny":
        B[:] = np.where(np.arange(K * N).reshape(K, N) % 3 == 0, -0.0, F32(1e-40))
        B[1, 2] = F32(-3e-39)
    else:
        B[K - 1, N - 1] = np.nan
    oracle.set_threads(0)
    try:
        ref = oracle.dense_fused_i8(M, N, K, F32(1.0), True, A, B)
    finally:
        oracle.set_threads(1)
    C = zeros(M * N, torch.float32)
    ane.stream_exec(ane.rec_dense_fused_i8(M, N, K, 1.0, True, dev(A), dev(B), C))
    assert_f32_identical(host(C).reshape(M, N), ref)


@pytest.mark.parametrize("M,N,K", [(256, 2048, 2048), (8, 4096, 4096)])
def test_dense_fused_grid_wait_limit(ane, oracle, M, N, K):
    """The bounded grid-wide wait of the resident quantizer (256 x 2048 x
    2048) and of the strip route (8 x 4096 x 4096), forced from the host
    to a one-tick limit: every workgroup still finishes, and a launch whose
    workgroups gave up is reported (C is then not valid) by stream_exec, by
    the kernel ABI's wait record (ane_hip_dense_fused_i8_status) and by the
    Python wrapper, each with ANE_ERR_GRID_WAIT; one that did not is exact.
    Restored to the default, the same calls are exact and report nothing."""
    import torch

    A, B = data.gemm_inputs(M, N, K, seed=11)
    oracle.set_threads(0)
    try:
        ref = oracle.dense_fused_i8(M, N, K, F32(1.0), True, A, B)
    finally:
        oracle.set_threads(1)
    dA, dB = dev(A), dev(B)
    lib = ane.lib()
    C = zeros(M * N, torch.float32)
    wsb = ane.dense_fused_i8_workspace_size(M, N, K)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    stream = ane._stream_handle(None)
    grid_wait = 9  # ANE_ERR_GRID_WAIT
    try:
        lib.ane_hip_set_grid_wait_limit(1)
        # opcode boundary
        try:
            ane.stream_exec(ane.rec_dense_fused_i8(M, N, K, 1.0, True, dA, dB, C))
        except ane.AneError as e:
            assert e.status == grid_wait and "grid-wide wait" in str(e)
        else:
            assert_f32_identical(host(C).reshape(M, N), ref)
        # kernel ABI: the wait record in the caller's workspace
        C.zero_()
        assert lib.ane_hip_dense_fused_i8(M, N, K, 1.0, 1, ane._p(dA), ane._p(dB), ane._p(C), 0, ane._p(ws),
                                          wsb, stream) == 0
        st = lib.ane_hip_dense_fused_i8_status(ane._p(ws), stream)
        assert st in (0, grid_wait)
        if st == 0:
            assert_f32_identical(host(C).reshape(M, N), ref)
        assert lib.ane_hip_grid_wait_status(stream) == 0  # the status call cleared the device record
        # Python wrapper: checks after the call by default
        C.zero_()
        try:
            ane.dense_fused_i8(M, N, K, 1.0, True, dA, dB, C, workspace=ws)
        except ane.AneError as e:
            assert e.status == grid_wait
        else:
            assert_f32_identical(host(C).reshape(M, N), ref)
        assert lib.ane_hip_grid_wait_status(stream) == 0
    finally:
        lib.ane_hip_set_grid_wait_limit(0)
    for how in ("stream_exec", "abi", "python"):
        C.zero_()
        if how == "stream_exec":
            ane.stream_exec(ane.rec_dense_fused_i8(M, N, K, 1.0, True, dA, dB, C))
        elif how == "abi":
            assert lib.ane_hip_dense_fused_i8(M, N, K, 1.0, 1, ane._p(dA), ane._p(dB), ane._p(C), 0, ane._p(ws),
                                              wsb, stream) == 0
            assert lib.ane_hip_dense_fused_i8_status(ane._p(ws), stream) == 0
        else:
            ane.dense_fused_i8(M, N, K, 1.0, True, dA, dB, C, workspace=ws)
        assert lib.ane_hip_grid_wait_status(stream) == 0
        assert_f32_identical(host(C).reshape(M, N), ref)


def test_dense_fused_status_unwritten_workspace(ane):
    """ane_hip_dense_fused_i8_status on a workspace no quantize call wrote
    (its record count word past the largest grid) is ANE_ERR_INVALID_ARG;
    a misaligned or null workspace is ANE_ERR_WORKSPACE."""
    import torch

    ws = torch.full((16384,), 0xFF, dtype=torch.uint8, device="cuda")
    lib = ane.lib()
    stream = ane._stream_handle(None)
    assert lib.ane_hip_dense_fused_i8_status(ane._p(ws), stream) == 1
    assert lib.ane_hip_dense_fused_i8_status(ane._p(ws) + 4, stream) == 8
    assert lib.ane_hip_dense_fused_i8_status(0, stream) == 8


@pytest.mark.parametrize("M,N,K", [(256, 2048, 2048), (16, 4096, 4096)])
def test_dense_fused_resident_two_streams(ane, oracle, M, N, K):
    """Two dense_fused_i8 calls with a grid-wide wait (the resident
    quantizer, 256 x 2048 x 2048; the strip route, 16 x 4096 x 4096) issued
    back to back on two streams with nothing between them: each grid needs
    every CU, so the library orders the second launch after the first (a
    stream-event wait); both results are exact and no wait gives up."""
    import torch

    ins = [data.gemm_inputs(M, N, K, seed=s) for s in (21, 22)]
    oracle.set_threads(0)
    try:
        refs = [oracle.dense_fused_i8(M, N, K, F32(1.0), True, A, B) for A, B in ins]
    finally:
        oracle.set_threads(1)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    wsb = ane.dense_fused_i8_workspace_size(M, N, K)
    bufs = [(dev(A), dev(B), zeros(M * N, torch.float32), torch.empty(wsb, dtype=torch.uint8, device="cuda"))
            for A, B in ins]
    torch.cuda.synchronize()
    for rep in range(3):
        for (dA, dB, C, ws), st in zip(bufs, streams):
            ane.dense_fused_i8(M, N, K, 1.0, True, dA, dB, C, workspace=ws, stream=st, check_wait=False)
        for (dA, dB, C, ws), st in zip(bufs, streams):
            ane.dense_fused_i8_status(ws, stream=st)
            assert ane.lib().ane_hip_grid_wait_status(ane._stream_handle(st)) == 0
        for (dA, dB, C, ws), ref in zip(bufs, refs):
            assert_f32_identical(host(C).reshape(M, N), ref)
            C.zero_()


@pytest.mark.parametrize("M,N,K,route", [(8, 4096, 4096, "strip"), (256, 2048, 2048, "resident"),
                                         (50, 128, 784, "few-tile"), (300, 700, 333, "two-pass")])
def test_dense_fused_graph_replays(ane, oracle, M, N, K, route):
    """dense_fused_i8 captured in a HIP graph, as bench.py times it, on each
    route: the strip route and the resident quantizer (grid-wide waits: a
    plain launch under capture, its tag fixed at capture time), the
    few-tile route and the two-pass quantizer.  The call is made once
    eagerly on the capture stream (so the grid-wide-wait routes may be
    captured there), then the graph is replayed three times with eager work
    (a fill of C) and synchronizations between the replays; every replay's
    C is bit-identical to the oracle and no wait gave up.  The one-launch
    routes leave the workspace's qA bytes as they were (0x5A), which shows
    the route the graph holds."""
    import torch

    A, B = data.gemm_inputs(M, N, K, seed=M + 2 * N + K)
    oracle.set_threads(0)
    try:
        ref = oracle.dense_fused_i8(M, N, K, F32(1.0), True, A, B)
    finally:
        oracle.set_threads(1)
    dA, dB = dev(A), dev(B)
    C = zeros(M * N, torch.float32)
    wsb = ane.dense_fused_i8_workspace_size(M, N, K)
    ws = torch.full((wsb,), 0x5A, dtype=torch.uint8, device="cuda")
    lib = ane.lib()
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        ane.dense_fused_i8(M, N, K, 1.0, True, dA, dB, C, workspace=ws, stream=s)
        s.synchronize()
        assert_f32_identical(host(C).reshape(M, N), ref)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            ane.dense_fused_i8(M, N, K, 1.0, True, dA, dB, C, workspace=ws, stream=s, check_wait=False)
    torch.cuda.synchronize()
    for _ in range(3):
        C.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert lib.ane_hip_grid_wait_status(ane._stream_handle(s)) == 0
        ane.dense_fused_i8_status(ws, stream=s)
        assert_f32_identical(host(C).reshape(M, N), ref)
    qa = host(ws)[12800: 12800 + M * K]
    assert (qa == 0x5A).all() == (route in ("strip", "few-tile"))
    del g


def test_dense_fused_4096_cubed_sampled(ane, oracle):
    """Config 2 at full size: both per-tensor scales exact, and a sample of
    rows of C identical to the oracle's contraction of the oracle-quantized
    operands (the full 4096^3 scalar product is too slow for a test)."""
    import torch

    M = N = K = 4096
    A, B = data.gemm_inputs(M, N, K, seed=2)
    qA, sa = oracle.quantize_exact(A.ravel())
    qB, sb = oracle.quantize_exact(B.ravel())
    C = zeros(M * N, torch.float32)
    scales = zeros(2, torch.float32)
    ane.dense_fused_i8(M, N, K, 1.0, True, dev(A), dev(B), C, scales_out=scales)
    s = host(scales)
    assert s[0] == sa and s[1] == sb
    Ch = host(C).reshape(M, N)
    oracle.set_threads(0)
    try:
        st = F32(F32(sa * sb) * F32(1.0))
        for r0 in (0, 1337, 4088):
            rows = oracle.dense_fused_rows(r0, r0 + 8, N, K, st, True, qA, qB)
            assert_f32_identical(Ch[r0: r0 + 8], rows)
    finally:
        oracle.set_threads(1)
    assert (Ch >= 0).all()


def test_dense_fused_4096_cubed_all_rows(ane, oracle):
    """Config 2's headline shape, every row of C: the GPU's 4096 x 4096
    output is bit-identical to the oracle's quantize + contraction +
    epilogue (the oracle runs multi-threaded over rows)."""
    import torch

    M = N = K = 4096
    A, B = data.gemm_inputs(M, N, K, seed=2)
    C = zeros(M * N, torch.float32)
    ane.stream_exec(ane.rec_dense_fused_i8(M, N, K, 1.0, True, dev(A), dev(B), C))
    Ch = host(C).reshape(M, N)
    oracle.set_threads(0)
    try:
        qA, sa = oracle.quantize_exact(A.ravel())
        qB, sb = oracle.quantize_exact(B.ravel())
        st = F32(F32(sa * sb) * F32(1.0))
        for r0 in range(0, M, 512):
            rows = oracle.dense_fused_rows(r0, r0 + 512, N, K, st, True, qA, qB)
            assert_f32_identical(Ch[r0: r0 + 512], rows)
    finally:
        oracle.set_threads(1)


@pytest.mark.parametrize("M", [1, 16, 128, 1024])
def test_dense_fused_config2_m_sweep_shapes(ane, oracle, M):
    """Config 2's M sweep at its exact shapes (N = K = 4096), every output."""
    import torch

    N = K = 4096
    A, B = data.gemm_inputs(M, N, K, seed=2 + M)
    oracle.set_threads(0)
    try:
        ref = oracle.dense_fused_i8(M, N, K, F32(1.0), True, A, B)
    finally:
        oracle.set_threads(1)
    C = zeros(M * N, torch.float32)
    ane.stream_exec(ane.rec_dense_fused_i8(M, N, K, 1.0, True, dev(A), dev(B), C))
    assert_f32_identical(host(C).reshape(M, N), ref)


def test_stream_exec_workspace_two_threads_one_stream(ane, oracle):
    """Two host threads share the null stream (and so stream_exec's workspace
    for it) and alternate small and large dense_fused_i8 records, so the
    workspace grows while the other thread's records use it."""
    import threading

    import torch

    shapes = [(64, 64, 256), (384, 512, 1024), (32, 100, 64), (512, 256, 2048)]
    cases = []
    for i, (M, N, K) in enumerate(shapes):
        A, B = data.gemm_inputs(M, N, K, seed=70 + i)
        cases.append((M, N, K, dev(A), dev(B), oracle.dense_fused_i8(M, N, K, F32(1.0), i % 2 == 0, A, B)))
    torch.cuda.synchronize()
    errors = []

    def worker(order):
        try:
            for it in range(6):
                for i in order:
                    M, N, K, A, B, ref = cases[i]
                    C = torch.full((M * N,), 9.0, dtype=torch.float32, device="cuda")
                    ane.stream_exec(ane.rec_dense_fused_i8(M, N, K, 1.0, i % 2 == 0, A, B, C), stream=0)
                    got = C.cpu().numpy().reshape(M, N)
                    if not np.array_equal(got.view(np.uint32), ref.view(np.uint32)):
                        errors.append(f"case {i} iteration {it}")
        except Exception as e:  # reported below, on the test's thread
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(o,)) for o in ([0, 1, 2, 3], [3, 2, 1, 0])]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors


# ---------------------------------------------------------------- cblas integer GEMMs
def _igemm_case(kind, flags, M, N, K, lda, ldb, ldc, seed):
    a_ext, b_ext, _ = ane_amd_extents(flags, M, N, K, lda, ldb, ldc)
    g = np.random.default_rng(seed)
    au, bu = kind in ("ugemm", "usgemm"), kind == "ugemm"
    A = g.integers(0 if au else -128, 256 if au else 128, size=max(a_ext, 1)).astype(np.uint8 if au else np.int8)
    B = g.integers(0 if bu else -128, 256 if bu else 128, size=max(b_ext, 1)).astype(np.uint8 if bu else np.int8)
    C = g.standard_normal((M, ldc)).astype(F32)
    return A, B, C


def ane_amd_extents(*args):
    import ane_amd

    return ane_amd._igemm_extents(*args)


IGEMM_VARIANT = {"igemm": 0, "ugemm": 1, "usgemm": 2}


@pytest.mark.parametrize("kind", ["igemm", "ugemm", "usgemm"])
@pytest.mark.parametrize("flags", [0, 1, 2, 3])
@pytest.mark.parametrize("M,N,K,beta", [(16, 32, 64, 0.0), (5, 7, 130, 0.5), (37, 300, 256, -0.0),
                                        (300, 200, 512, 0.0), (20, 70, 40, 1.0), (1, 4096, 4096, 0.0)])
def test_cblas_igemm_opcodes_parity(ane, oracle, kind, flags, M, N, K, beta):
    """0x61-0x63 through stream_exec: every variant, transA/transB, strides
    past the logical sizes, K remainders and K < 64, and beta seeding the
    accumulator bits, bit-identical to the handler's arithmetic."""
    lda = (K + 3) if not flags & 1 else (M + 5)
    ldb = (N + 2) if not flags & 2 else (K + 7)
    ldc = N + 3
    A, B, C = _igemm_case(kind, flags, M, N, K, lda, ldb, ldc, seed=M + N + K + flags)
    oracle.set_threads(0)
    try:
        ref = oracle.cblas_igemm(IGEMM_VARIANT[kind], flags, M, N, K, lda, ldb, ldc, -0.75, beta, A, B, C)
    finally:
        oracle.set_threads(1)
    Cd = dev(C)
    ane.stream_exec(ane.rec_cblas_igemm(kind, flags, M, N, K, lda, ldb, ldc, -0.75, beta, dev(A), dev(B), Cd))
    assert_f32_identical(host(Cd), ref)


@pytest.mark.parametrize("flags", [0, 1, 2, 3])
@pytest.mark.parametrize("M,N,K,lda,ldb,beta", [(64, 96, 320, 352, 336, 0.0), (1024, 1024, 1024, 1024, 1024, 0.5),
                                                (100, 130, 200, 208, 224, 0.0), (7, 48, 64, 64, 80, -1.0)])
def test_cblas_igemm_in_place_operands(ane, oracle, flags, M, N, K, lda, ldb, beta):
    """cblas_igemm (0x61, signed) with 16-byte multiples for lda and ldb: the
    contraction reads A's rows (no transA) and B's rows (transB) in place
    instead of gathering them, and only the first 64 * floor(K / 64) bytes of
    each row (K = 200: the last 8 bytes of each row and the padding past K
    are nonzero and ignored).  With transA or without transB the operand is
    gathered as before.  Bit for bit against the handler's arithmetic."""
    kind = "igemm"
    lda_ = lda if not flags & 1 else M + 16
    ldb_ = ldb if flags & 2 else N + 16
    ldc = N + 1
    A, B, C = _igemm_case(kind, flags, M, N, K, lda_, ldb_, ldc, seed=M + N + K + 7 * flags)
    oracle.set_threads(0)
    try:
        ref = oracle.cblas_igemm(IGEMM_VARIANT[kind], flags, M, N, K, lda_, ldb_, ldc, 1.25, beta, A, B, C)
    finally:
        oracle.set_threads(1)
    Cd = dev(C)
    ane.stream_exec(ane.rec_cblas_igemm(kind, flags, M, N, K, lda_, ldb_, ldc, 1.25, beta, dev(A), dev(B), Cd))
    assert_f32_identical(host(Cd), ref)


@pytest.mark.parametrize("kind", ["igemm", "ugemm", "usgemm"])
@pytest.mark.parametrize("flags", [0, 1, 2, 3])
@pytest.mark.parametrize("M,N,K,beta", [(33, 40, 256, 0.5), (1024, 1024, 1024, 0.0), (260, 520, 192, -2.0)])
def test_cblas_igemm_blas_semantics(ane, oracle, kind, flags, M, N, K, beta):
    """The kernel-level BLAS form: op(A) = A^T with transA (A is K x M), and
    C = alpha*acc + beta*C with two roundings; for igemm, lda and ldb are
    16-byte multiples here, so A (without transA) and B (with transB) are
    read in place."""
    lda = (K + 16) if not flags & 1 else (M + 16)
    ldb = (N + 16) if not flags & 2 else (K + 16)
    ldc = N
    g = np.random.default_rng(M + N + flags)
    au, bu = kind in ("ugemm", "usgemm"), kind == "ugemm"
    na = (K * lda) if flags & 1 else (M * lda)
    nb = (N * ldb) if flags & 2 else (K * ldb)
    A = g.integers(0 if au else -128, 256 if au else 128, size=na).astype(np.uint8 if au else np.int8)
    B = g.integers(0 if bu else -128, 256 if bu else 128, size=nb).astype(np.uint8 if bu else np.int8)
    C = g.standard_normal((M, ldc)).astype(F32)
    oracle.set_threads(0)
    try:
        ref = oracle.cblas_igemm(IGEMM_VARIANT[kind], flags, M, N, K, lda, ldb, ldc, 0.5, beta, A, B, C, semantics=1)
    finally:
        oracle.set_threads(1)
    Cd = dev(C)
    ane.cblas_igemm(kind, flags, M, N, K, lda, ldb, ldc, 0.5, beta, dev(A), dev(B), Cd, blas=True)
    assert_f32_identical(host(Cd), ref)


def test_cblas_igemm_short_a_rejected(ane):
    """transA's handler addressing reaches 15*lda + 16*floor((M-1)/16) - 16
    + Ke bytes: one byte less in A's allocation is refused before anything
    runs."""
    import torch

    M, N, K, lda = 40, 8, 64, 100
    a_ext, b_ext, _ = ane_amd_extents(1, M, N, K, lda, N, N)
    assert a_ext == 15 * lda + 32 - 16 + 64
    hip = _hip()
    p = ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(p), ctypes.c_size_t(a_ext - 1)) == 0
    try:
        C = torch.full((M * N,), 2.0, dtype=torch.float32, device="cuda")
        B = zeros(b_ext, torch.int8)
        with pytest.raises(ane.AneError) as e:
            ane.stream_exec(ane.rec_cblas_igemm("igemm", 1, M, N, K, lda, N, N, 1.0, 0.0, p.value, B, C))
        assert e.value.status == 3
        assert (host(C) == 2.0).all()
    finally:
        hip.hipFree(p)


# ---------------------------------------------------------------- Q8_0
@pytest.mark.parametrize("M,K", [(1, 32), (3, 40), (4096, 4096), (14336, 4096), (4096, 14336), (77, 96),
                                 # streaming kernel: partial last segment, ragged row split, K % 32 != 0
                                 (1001, 2304), (5, 261), (4097, 512)])
def test_q8_0_gemv_r_parity(ane, oracle, M, K):
    """Opcode 0x57 through stream_exec, bit-identical to the reference arithmetic."""
    import torch

    K32 = K - K % 32
    W = data.q8_0_weights(M, K32, seed=M + K)
    x = data.activations(1, K, seed=K)[0]
    oracle.set_threads(0)
    try:
        ref = oracle.q8_0_gemv(M, K, x, W)
    finally:
        oracle.set_threads(1)
    y = zeros(M, torch.float32)
    ane.stream_exec(ane.rec_q8_0_gemv(M, K, dev(x), dev(W), y))
    assert_f32_identical(host(y), ref)


@pytest.mark.parametrize("N,K,T", [(4096, 4096, 1), (14336, 4096, 1), (4096, 14336, 1), (6144, 4096, 4),
                                   (4096, 4096, 16), (1024, 4096, 64), (100, 96, 3), (5, 50, 2),
                                   # streaming kernel: partial segment, ragged rows, unaligned x rows, T 2..4
                                   (1001, 2304, 1), (37, 261, 3), (4097, 512, 2), (28672, 4096, 4),
                                   (3, 256, 1),
                                   # activations quantized once into the workspace: one token
                                   # past 256 blocks, 2..4 tokens at any K
                                   (333, 8448, 1), (1001, 8192, 1), (4096, 14336, 3), (50, 8192, 2),
                                   # MFMA kernel (T > 4, K % 512 == 0): ragged row and token tiles,
                                   # several stages, T past 64
                                   (300, 512, 5), (17, 4096, 17), (4096, 14336, 16), (2000, 8192, 33),
                                   (64, 1024, 100), (6144, 4096, 64),
                                   # the workgroup shapes for many tiles: 2 row tiles of one token
                                   # tile on the token-stationary kernel, 1x2 + split 4, 1x2
                                   (28672, 512, 16), (8192, 1024, 32), (6000, 512, 40),
                                   # token-stationary MFMA kernel: 4 row x 4 token tiles (ragged
                                   # rows and tokens, two token groups); 2 x 2 tiles at two token
                                   # tiles, and at three or four just past one row tile per CU
                                   (28672, 512, 64), (16392, 1024, 40), (16384, 512, 100),
                                   (19990, 512, 20), (4100, 1024, 50),
                                   # residue-split kernel (256+ blocks per row, fewer than 64 row
                                   # tiles per CU): ragged 64-row groups and token tiles, rows
                                   # fewer than one group, the unit count not a multiple of 8,
                                   # token groups past 64, one and two token tiles
                                   (4100, 8192, 40), (300, 9216, 20), (37, 8192, 5), (1000, 16384, 64),
                                   (200, 8192, 100), (4096, 14336, 32), (130, 8192, 16),
                                   # activation-stationary kernel (K 4096 with 16-64 tokens, K 14336
                                   # with 16): three token groups of one tile, two groups of two
                                   # tiles with ragged rows, several row tiles per workgroup, four
                                   # tiles on 8 waves with ragged rows and tokens, K 14336 with
                                   # ragged rows
                                   (4100, 4096, 48), (6000, 4096, 64), (20000, 4096, 32),
                                   (28677, 4096, 60), (5000, 14336, 16),
                                   # ... with a remainder of K past the last whole block (ignored)
                                   (300, 4100, 16), (33, 14350, 16),
                                   # ... for 2-15 tokens padded to one token tile (2-4 tokens where
                                   # the row tiles fill the CUs): ragged rows, K 14336, and rows
                                   # that keep 2-4 tokens on the streaming kernel
                                   (4096, 4096, 2), (28672, 4096, 3), (4096, 14336, 4), (6144, 4096, 5),
                                   (4100, 4096, 8), (300, 4096, 12), (5000, 14336, 7), (4100, 4096, 4)])
def test_q8_0_mul_mat_g_parity(ane, oracle, N, K, T):
    import torch

    W = data.q8_0_weights(N, K - K % 32, seed=N + K)
    x = data.activations(T, K, seed=T + 100)
    oracle.set_threads(0)
    try:
        ref = oracle.q8_0_mul_mat_g(N, K, T, x, W)
    finally:
        oracle.set_threads(1)
    for got in mul_mat_both_routes(ane, N, K, T, x, W):
        assert_f32_identical(got, ref)


# config 4: the four Llama-3-8B projections (rows x K) at every token count
CONFIG4 = {"qkv": (6144, 4096), "o": (4096, 4096), "gate_up": (28672, 4096), "down": (4096, 14336)}


@pytest.mark.parametrize("T", [1, 2, 4, 8, 16, 64])
@pytest.mark.parametrize("proj", list(CONFIG4))
def test_q8_0_mul_mat_config4_shapes(ane, oracle, proj, T):
    """Config 4 at its exact shapes: every (projection, tokens) pair, every
    output bit-identical to the oracle's G-mode definition, on the routes
    of both workspace sizes (the residue-split kernel at 16 and 64 tokens
    on the 4096- and 6144-row projections, the older kernels otherwise)."""
    N, K = CONFIG4[proj]
    W = data.q8_0_weights(N, K, seed=N + K + 1)
    x = data.activations(T, K, seed=T + 200)
    oracle.set_threads(0)
    try:
        ref = oracle.q8_0_mul_mat_g(N, K, T, x, W)
    finally:
        oracle.set_threads(1)
    for got in mul_mat_both_routes(ane, N, K, T, x, W):
        assert_f32_identical(got, ref)


@pytest.mark.parametrize("T,K,N", [(2, 1024, 300), (20, 1024, 300), (1, 9216, 300), (3, 9216, 300),
                                   (40, 512, 4100), (20, 9216, 300), (64, 8192, 130)])
def test_q8_0_mul_mat_g_special_values(ane, oracle, T, K, N):
    """Zero, NaN and infinite activation blocks (0x19 zero guard and NaN rules
    per block), on the streaming (T = 2, and the separately quantized T = 1
    and 3 at K = 9216), MFMA (T = 20), token-stationary MFMA (T = 40 over
    4100 rows) and residue-split (T = 20 and 64 at K = 9216 / 8192)
    kernels."""
    import torch

    W = data.q8_0_weights(N, K, seed=11)
    x = data.activations(T, K, seed=12)
    x[0, 0:32] = 0.0
    x[0, 64] = np.nan
    x[T - 1, 100] = np.inf
    x[T - 1, 200] = -1e-40  # denormal
    ref = oracle.q8_0_mul_mat_g(N, K, T, x, W)
    for got in mul_mat_both_routes(ane, N, K, T, x, W):
        assert_f32_identical(got, ref)


@pytest.mark.parametrize("mode,N,K,T", [("R", 300, 1024, 1), ("G", 300, 1024, 1), ("G", 300, 1024, 2),
                                        ("G", 300, 9216, 3), ("G", 300, 1024, 20), ("G", 4100, 1024, 40),
                                        ("G", 16384, 512, 16), ("G", 300, 9216, 20), ("G", 200, 8192, 64)])
def test_q8_0_special_weight_scales(ane, oracle, mode, N, K, T):
    """Weight block scales of every fp16 class (infinities, NaN, subnormals,
    signed zeros, the largest finite), with all-zero blocks among them so
    0 * inf reaches the fma, on the R matvec, the G streaming kernel (T = 1,
    2, and 3 on separately quantized activations), the MFMA kernel (T = 20),
    the token-stationary MFMA kernel (2 x 2 and 2 x 1 tile shapes) and the
    residue-split kernel (T = 20 and 40 with the full workspace)."""
    import torch

    nb = K // 32
    W = data.q8_0_weights(N, K, seed=31).reshape(N, nb, 34).copy()
    specials = np.array([0x7C00, 0xFC00, 0x7E00, 0x0001, 0x83FF, 0x8000, 0x0000, 0x7BFF, 0xBC00],
                        dtype=np.uint16)
    rng = np.random.default_rng(32)
    d = rng.choice(specials, size=(N, nb))
    d[rng.random((N, nb)) < 0.97] = 0x2E66  # leave most blocks ordinary
    W[:, :, 0:2] = d.view(np.uint8).reshape(N, nb, 2)
    W[rng.random((N, nb)) < 0.05, 2:] = 0  # isum 0 against an infinite scale gives NaN
    W = W.reshape(N, -1)
    x = data.activations(T, K, seed=33)
    if mode == "R":
        ref = oracle.q8_0_gemv(N, K, x[0], W)
        y = zeros(N, torch.float32)
        ane.q8_0_gemv(N, K, dev(x[0]), dev(W), y)
        assert_f32_identical(host(y), ref)
    else:
        ref = oracle.q8_0_mul_mat_g(N, K, T, x, W)
        for got in mul_mat_both_routes(ane, N, K, T, x, W):
            assert_f32_identical(got, ref)
    # the cases reach NaN, finite and (G: one isum per block) infinite outputs;
    # an R-mode infinite block mixes both signs across its lanes, giving NaN
    assert np.isnan(ref).any() and np.isfinite(ref).any() and (mode == "R" or np.isinf(ref).any())


def test_q8_0_degenerate_shapes(ane, oracle):
    """No rows or no tokens leave y untouched; K < 32 (nb = K >> 5 = 0 blocks)
    writes the empty sum, as the oracle does."""
    import torch

    x = data.activations(3, 64, seed=51)
    W = data.q8_0_weights(7, 64, seed=52)
    y = torch.full((21,), 7.0, dtype=torch.float32, device="cuda")
    ane.q8_0_gemv(0, 64, dev(x[0]), dev(W), y)
    ane.q8_0_mul_mat(0, 64, 3, dev(x), dev(W), y)
    ane.q8_0_mul_mat(7, 64, 0, dev(x), dev(W), y)
    assert (host(y) == 7.0).all()
    for K in (0, 20):
        xs = data.activations(3, K, seed=53)
        Wk = np.zeros((7, 0), np.uint8)
        ane.q8_0_gemv(7, K, dev(xs[0]), dev(Wk), y)
        assert_f32_identical(host(y)[:7], oracle.q8_0_gemv(7, K, xs[0], Wk))
        y.fill_(7.0)
        ane.q8_0_mul_mat(7, K, 3, dev(xs), dev(Wk), y)
        assert_f32_identical(host(y).reshape(3, 7), oracle.q8_0_mul_mat_g(7, K, 3, xs, Wk))
        y.fill_(7.0)


def test_q8_0_mul_mat_concurrent_host_threads(ane, oracle):
    """Host threads on their own streams call the same kernel instantiations
    with different LDS sizes at once (the launch caches are shared): every
    result stays bit-identical to the oracle."""
    import threading

    import torch

    N = 520
    cases = []
    for i, K in enumerate((1024, 2048, 4096, 8192)):
        W = data.q8_0_weights(N, K, seed=40 + i)
        x = data.activations(1, K, seed=50 + i)
        cases.append((K, W, x, oracle.q8_0_mul_mat_g(N, K, 1, x, W)[0], oracle.q8_0_gemv(N, K, x[0], W)))
    errors = []

    def worker(K, W, x, ref_g, ref_r):
        try:
            st = torch.cuda.Stream()
            Wd, xd = dev(W), dev(x)
            yg = torch.zeros(N, dtype=torch.float32, device="cuda")
            yr = torch.zeros(N, dtype=torch.float32, device="cuda")
            ws = torch.empty(ane.q8_0_mul_mat_workspace_size(K, 1), dtype=torch.uint8, device="cuda")
            torch.cuda.synchronize()
            for _ in range(25):
                ane.q8_0_mul_mat(N, K, 1, xd, Wd, yg, workspace=ws, stream=st)
                ane.q8_0_gemv(N, K, xd[0], Wd, yr, stream=st)
            st.synchronize()
            if not np.array_equal(yg.cpu().numpy().view(np.uint32), ref_g.view(np.uint32)):
                errors.append(f"G K={K}")
            if not np.array_equal(yr.cpu().numpy().view(np.uint32), ref_r.view(np.uint32)):
                errors.append(f"R K={K}")
        except Exception as e:  # reported below, on the test's thread
            errors.append(f"K={K}: {e!r}")

    threads = [threading.Thread(target=worker, args=c) for c in cases]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors


@pytest.mark.parametrize("mode", ["R", "G"])
def test_q8_0_misaligned_weights(ane, oracle, mode):
    """W starting 2 bytes into an allocation (rows not 16-byte aligned): general kernels."""
    import torch

    N, K = 513, 1024
    W = data.q8_0_weights(N, K, seed=5)
    x = data.activations(1, K, seed=6)[0]
    buf = torch.zeros(W.size + 16, dtype=torch.uint8, device="cuda")
    buf[2: 2 + W.size] = dev(W.reshape(-1))
    Wv = buf[2: 2 + W.size]
    y = zeros(N, torch.float32)
    if mode == "R":
        ref = oracle.q8_0_gemv(N, K, x, W)
        ane.q8_0_gemv(N, K, dev(x), Wv, y)
    else:
        ref = oracle.q8_0_mul_mat_g(N, K, 1, x[None, :], W)[0]
        ane.q8_0_mul_mat(N, K, 1, dev(x), Wv, y)
    assert_f32_identical(host(y), ref)


# ---------------------------------------------------------------- error paths
def _hip():
    return ctypes.CDLL("libamdhip64.so")


def test_host_pointer_rejected(ane):
    x = np.ones(64, F32)
    q = np.zeros(64, np.int8)
    with pytest.raises(ane.AneError) as e:
        ane.stream_exec(ane.rec_quantize(64, x.ctypes.data, q.ctypes.data, 0))
    assert e.value.status == 2


def test_short_buffer_rejected(ane):
    hip = _hip()
    p = ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(p), ctypes.c_size_t(1024)) == 0
    try:
        import torch

        dst = zeros(8192, torch.int8)
        sc = zeros(1, torch.float32)
        with pytest.raises(ane.AneError) as e:
            ane.stream_exec(ane.rec_quantize(4096, p.value, dst, sc))
        assert e.value.status == 3
    finally:
        hip.hipFree(p)


def test_unknown_opcode_stops_stream(ane):
    import torch

    x = dev(np.ones(64, F32))
    dst, sc = zeros(64, torch.int8), zeros(1, torch.float32)
    with pytest.raises(ane.AneError) as e:
        ane.stream_exec([bytes([0x15]), ane.rec_quantize(64, x, dst, sc)])
    assert e.value.status == 4
    assert not host(dst).any()
