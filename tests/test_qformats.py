"""GPU parity of the other weight formats (Q4_0 and K-quant GEMVs, Q8_0/Q4_0
row gathers) against the CPU oracle, bit for bit, through the C ABI and
through stream_exec records."""
import ctypes

import numpy as np
import pytest

from tests import data
from tests.test_gpu_parity import _hip
from tests.test_oracle_q import kat_expected, kat_q4_0_table, kat_q8_0_table

pytestmark = pytest.mark.gpu
F32 = np.float32
FMTS = ["q4_0", "q4_k", "q2_k", "q3_k", "q5_k", "q6_k"]


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def assert_same(got, want):
    np.testing.assert_array_equal(np.asarray(got, F32).view(np.uint32)[~np.isnan(want)],
                                  np.asarray(want, F32).view(np.uint32)[~np.isnan(want)])
    assert np.array_equal(np.isnan(got), np.isnan(want))


def weights_at(W, offset):
    """W on the device starting `offset` bytes past a 256-byte boundary."""
    import torch

    flat = np.ascontiguousarray(W).reshape(-1)
    buf = torch.zeros(flat.size + 256, dtype=torch.uint8, device="cuda")
    buf[offset:offset + flat.size] = torch.from_numpy(flat).cuda()
    return buf, buf[offset:]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,K", [(300, 4096), (17, 256), (33, 512), (4096, 4096), (5, 16640), (3, 8448),
                                 (2100, 768)])
def test_q_gemv_exact(ane, oracle, fmt, M, K):
    """K = 16640 / 8448: inputs in several 4096-value chunks and a partial last
    stage.  The general kernel takes 4, 8 or 16 rows per workgroup by the row
    count (on 256 CUs: 300, 2100 and 4096 rows)."""
    import torch

    W = data.q_weights(fmt, M, K, seed=M + K)
    x = data.activations(1, K, seed=K)[0]
    y = torch.full((M,), 7.0, dtype=torch.float32, device="cuda")
    oracle.set_threads(0)
    try:
        ref = oracle.q_gemv(fmt, M, K, x, W)
    finally:
        oracle.set_threads(1)
    ane.q_gemv(fmt, M, K, dev(x), dev(W), y)
    assert_same(host(y), ref)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("offset", [1, 2, 3, 14])
def test_q_gemv_unaligned_weights(ane, oracle, fmt, offset):
    import torch

    M, K = 37, 1024
    W = data.q_weights(fmt, M, K, seed=offset)
    x = data.activations(1, K, seed=3)[0]
    buf, Wd = weights_at(W, offset)
    y = torch.zeros(M, dtype=torch.float32, device="cuda")
    ane.q_gemv(fmt, M, K, dev(x), Wd, y)
    assert_same(host(y), oracle.q_gemv(fmt, M, K, x, W))


def test_q4_0_special_scales(ane, oracle):
    """Block scales of every fp16 class (infinities, NaN, subnormals, signed
    zeros, the largest finite) against every nibble value."""
    import torch

    M, K = 40, 1024
    W = data.q_weights("q4_0", M, K, seed=21).reshape(M, K // 32, 18).copy()
    specials = np.array([0x7C00, 0xFC00, 0x7E00, 0x0001, 0x83FF, 0x8000, 0x0000, 0x7BFF, 0xBC00, 0x3C00],
                        dtype=np.uint16)
    rng = np.random.default_rng(22)
    d = rng.choice(specials, size=(M, K // 32))
    d[rng.random((M, K // 32)) < 0.5] = 0x2E66  # leave about half of the blocks ordinary
    W[:, :, 0:2] = d.view(np.uint8).reshape(M, K // 32, 2)
    W[:, :, 2:] = rng.integers(0, 256, size=(M, K // 32, 16), dtype=np.uint8)
    W = W.reshape(M, -1)
    x = data.activations(1, K, seed=23)[0]
    y = torch.zeros(M, dtype=torch.float32, device="cuda")
    ane.q_gemv("q4_0", M, K, dev(x), dev(W), y)
    assert_same(host(y), oracle.q_gemv("q4_0", M, K, x, W))


@pytest.mark.parametrize("fmt", ["q4_k", "q2_k", "q3_k", "q5_k", "q6_k"])
@pytest.mark.parametrize("offset", [0, 2])
def test_k_quant_special_scales(ane, oracle, fmt, offset):
    """Super-block d and dmin of every fp16 class (infinities, NaN,
    subnormals, signed zeros, the largest finite), on the streaming kernel
    (aligned rows) and on k_qgemv (rows 2 bytes off)."""
    import torch

    M, K = 64, 4096
    sbb, _, fp16_at = data.Q_BLOCK[fmt]
    W = data.q_weights(fmt, M, K, seed=41).reshape(M, K // 256, sbb).copy()
    specials = np.array([0x7C00, 0xFC00, 0x7E00, 0x0001, 0x83FF, 0x8000, 0x0000, 0x7BFF, 0xBC00],
                        dtype=np.uint16)
    rng = np.random.default_rng(42)
    for pos in fp16_at:
        d = W[:, :, pos:pos + 2].copy().view(np.uint16)[..., 0]
        pick = rng.random(d.shape) < 0.1
        d[pick] = rng.choice(specials, size=int(pick.sum()))
        W[:, :, pos:pos + 2] = d.view(np.uint8).reshape(M, K // 256, 2)
    W = W.reshape(M, -1)
    x = data.activations(1, K, seed=43)[0]
    buf, Wd = weights_at(W, offset)
    y = torch.zeros(M, dtype=torch.float32, device="cuda")
    ane.q_gemv(fmt, M, K, dev(x), Wd, y)
    ref = oracle.q_gemv(fmt, M, K, x, W)
    assert_same(host(y), ref)
    assert np.isnan(ref).any() and np.isfinite(ref).any()


@pytest.mark.parametrize("fmt", FMTS)
def test_q_gemv_degenerate_shapes(ane, oracle, fmt):
    """No rows leave y untouched; K below one block (the handlers' K >> 5 or
    K >> 8 is 0) writes the empty sum, as the oracle does."""
    import torch

    y = torch.full((9,), 7.0, dtype=torch.float32, device="cuda")
    x = data.activations(1, 512, seed=61)[0]
    ane.q_gemv(fmt, 0, 512, dev(x), dev(data.q_weights(fmt, 2, 512, seed=62)), y)
    assert (host(y) == 7.0).all()
    for K in (0, 20):
        xk = data.activations(1, K, seed=63)[0]
        Wk = np.zeros((9, 0), np.uint8)
        ane.q_gemv(fmt, 9, K, dev(xk), dev(Wk), y)
        assert_same(host(y), oracle.q_gemv(fmt, 9, K, xk, Wk))
        y.fill_(7.0)


@pytest.mark.parametrize("first", ["zero", "denormal", "special"])
def test_q3_k_first_half_inputs(ane, oracle, first):
    """The second halves' decode depends on the first halves' input bits."""
    import torch

    M, K = 64, 2048
    W = data.q_weights("q3_k", M, K, seed=9)
    x = data.activations(1, K, seed=10)[0]
    for j in range(K // 32):
        if first == "zero":
            x[32 * j:32 * j + 16] = 0.0
        elif first == "denormal":
            x[32 * j:32 * j + 16] = (np.arange(16, dtype=np.uint32) * 2 + j % 3).view(F32)
        else:
            x[32 * j:32 * j + 16] = np.array([0.0, -0.0, 1e-45, 3e-45, -1e-45, 1.0, 2.5e-44, 5.0] * 2, F32)
    y = torch.zeros(M, dtype=torch.float32, device="cuda")
    ane.q_gemv("q3_k", M, K, dev(x), dev(W), y)
    assert_same(host(y), oracle.q_gemv("q3_k", M, K, x, W))


@pytest.mark.parametrize("fmt", FMTS)
def test_q_gemv_record(ane, oracle, fmt):
    """The reference's byte records of 0x58 / 0x75-0x79 through stream_exec."""
    import torch

    M, K = 70, 1280
    W = data.q_weights(fmt, M, K, seed=77)
    x = data.activations(1, K, seed=78)[0]
    y = torch.zeros(M, dtype=torch.float32, device="cuda")
    xd, Wd = dev(x), dev(W)
    ane.stream_exec(ane.rec_q_gemv(fmt, M, K, xd, Wd, y))
    assert_same(host(y), oracle.q_gemv(fmt, M, K, x, W))
    # W in an allocation of exactly its size; a record that claims 200 more
    # rows (past any allocation rounding) is refused before anything runs
    hip = _hip()
    p = ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(p), ctypes.c_size_t(W.nbytes)) == 0
    try:
        assert hip.hipMemcpy(p, W.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(W.nbytes), 1) == 0
        y2 = torch.zeros(M + 200, dtype=torch.float32, device="cuda")
        with pytest.raises(ane.AneError) as e:
            ane.stream_exec(ane.rec_q_gemv(fmt, M + 200, K, xd, p.value, y2))
        assert e.value.status == 3
        assert not host(y2).any()
    finally:
        hip.hipFree(p)


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0"])
@pytest.mark.parametrize("dim", [32, 64])
def test_get_rows_reference_kat(ane, fmt, dim):
    """test_remaining_ops.cpp:230-430 on the GPU."""
    import torch

    T = kat_q8_0_table(dim) if fmt == "q8_0" else kat_q4_0_table(dim)
    idx = [1, 3] if fmt == "q8_0" else [0, 2]
    out = torch.zeros((2, dim), dtype=torch.float32, device="cuda")
    ane.get_rows(fmt, 2, dim, dev(T), 4, dev(np.array(idx, np.uint32)), out)
    assert host(out).tobytes() == kat_expected(T, fmt, dim, idx).tobytes()
    out.zero_()
    ane.stream_exec(ane.rec_get_rows(fmt, 2, dim, dev(T), dev(np.array(idx, np.uint32)), out))
    assert host(out).tobytes() == kat_expected(T, fmt, dim, idx).tobytes()


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0"])
def test_get_rows_exact(ane, oracle, fmt):
    import torch

    vocab, dim, n = 1000, 4096, 37
    W = data.q8_0_weights(vocab, dim, seed=5) if fmt == "q8_0" else data.q_weights("q4_0", vocab, dim, seed=5)
    idx = data.rng(6).integers(0, vocab, n).astype(np.uint32)
    idx[3] = idx[7]  # repeated rows
    out = torch.zeros((n, dim), dtype=torch.float32, device="cuda")
    ane.get_rows(fmt, n, dim, dev(W), vocab, dev(idx), out)
    assert host(out).tobytes() == oracle.get_rows(fmt, n, dim, W, idx).tobytes()


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0"])
def test_get_rows_out_of_table(ane, oracle, fmt):
    """An index past the table: zeros from the kernel-level entry, an error
    (and nothing launched) from the byte stream."""
    import torch

    vocab, dim = 8, 96
    W = data.q8_0_weights(vocab, dim, seed=1) if fmt == "q8_0" else data.q_weights("q4_0", vocab, dim, seed=1)
    idx = np.array([2, 1000, 5], np.uint32)
    out = torch.full((3, dim), 5.0, dtype=torch.float32, device="cuda")
    idd = dev(idx)
    hip = _hip()
    p = ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(p), ctypes.c_size_t(W.nbytes)) == 0
    try:
        assert hip.hipMemcpy(p, W.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(W.nbytes), 1) == 0
        ane.get_rows(fmt, 3, dim, p.value, vocab, idd, out)
        got = host(out)
        ref = oracle.get_rows(fmt, 2, dim, W, idx[[0, 2]])
        assert got[0].tobytes() == ref[0].tobytes() and got[2].tobytes() == ref[1].tobytes()
        assert not got[1].any()
        out.fill_(5.0)
        with pytest.raises(ane.AneError) as e:
            ane.stream_exec(ane.rec_get_rows(fmt, 3, dim, p.value, idd, out))
        assert e.value.status == 3
        assert (host(out) == 5.0).all()
        with pytest.raises(ane.AneError) as e:
            ane.get_rows(fmt, 3, 100, p.value, vocab, idd, out)
        assert e.value.status == 1
    finally:
        hip.hipFree(p)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,K", [(37, 300), (300, 33), (4096, 520), (5, 4200)])
def test_q_gemv_k_remainder_exact_x(ane, oracle, fmt, M, K):
    """K with a remainder the handlers ignore (K >> 5, K >> 8): x lives in an
    allocation of exactly the values the blocks consume, and the record
    passes stream_exec's extent check, so no kernel may stage x past it."""
    import torch

    vals = ane.QFORMATS[fmt][1]
    nsb = K // vals
    if nsb == 0:
        pytest.skip("no whole block")
    W = data.q_weights(fmt, M, K, seed=M + 7 * K)
    x = data.activations(1, K, seed=K + 1)[0]
    hip = _hip()
    p = ctypes.c_void_p()
    nbytes = nsb * vals * 4
    assert hip.hipMalloc(ctypes.byref(p), ctypes.c_size_t(nbytes)) == 0
    try:
        assert hip.hipMemcpy(p, x.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(nbytes), 1) == 0
        y = torch.full((M,), 3.0, dtype=torch.float32, device="cuda")
        ane.stream_exec(ane.rec_q_gemv(fmt, M, K, p.value, dev(W), y))
        assert_same(host(y), oracle.q_gemv(fmt, M, K, x, W))
    finally:
        hip.hipFree(p)
