"""GPU parity of the decode-step handlers rms_norm_fp32 (0x51), silu_fp32
(0x54), rope_fp32 (0x55) and softmax_fp32 (0x56) against the oracle's
restatement, bit for bit, through stream_exec records and the kernel-level
entries; and of the build's standalone RMSNorm against the oracle."""
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


def same(got, want):
    got, want = np.asarray(got, F32), np.asarray(want, F32)
    assert got.shape == want.shape
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got.view(np.uint32)[~nan], want.view(np.uint32)[~nan])


SPECIAL = np.array([0.0, -0.0, 1e-40, -1e-40, 1e-30, np.inf, -np.inf, np.nan, 88.0, -88.0, 89.0, -89.0,
                    127.5, -128.5, 1e10, -1e10, 3.4e38, -3.4e38, 0.5, -0.5], F32)


@pytest.mark.parametrize("dim", [16, 256, 4096, 14336])
def test_rms_norm_fp32_opcode(ane, oracle, dim):
    import torch

    g = np.random.default_rng(dim)
    for scale in (1.0, 1e-8, 1e4):
        x = (g.standard_normal(dim) * scale).astype(F32)
        w = (1 + 0.1 * g.standard_normal(dim)).astype(F32)
        out = torch.full((dim,), 7.0, dtype=torch.float32, device="cuda")
        ane.stream_exec(ane.rec_rms_norm(dim, 1e-5, dev(x), dev(w), out))
        same(host(out), oracle.rms_norm_fp32(x, w, 1e-5))


def test_rms_norm_fp32_many_rows(ane, oracle):
    """1000 rows whose mean squares sweep the frsqrte table (both exponent
    parities, every top fraction byte) and the two Newton steps."""
    import torch

    rows, dim = 1000, 64
    g = np.random.default_rng(1)
    x = (g.standard_normal((rows, dim)) * np.exp(g.uniform(-20, 20, (rows, 1)))).astype(F32)
    w = (1 + 0.1 * g.standard_normal(dim)).astype(F32)
    out = torch.zeros((rows, dim), dtype=torch.float32, device="cuda")
    ane.rms_norm_fp32(rows, dim, 1e-6, dev(x), dev(w), out)
    got = host(out)
    for r in range(rows):
        same(got[r], oracle.rms_norm_fp32(x[r], w, 1e-6))


def rsqrte_bucket(t):
    """FRSQRTE's table input for a positive normal float32 t: 256 + the top
    8 fraction bits for an even biased exponent, 128 + the top 7 for odd."""
    u = np.asarray(t, F32).view(np.uint32)
    e, fr = (u >> 23) & 0xFF, u & 0x7FFFFF
    return np.where(e % 2 == 0, 256 + (fr >> 15), 128 + (fr >> 16)) + 1000 * (e % 2)


def test_rms_norm_fp32_frsqrte_table_and_denormals(ane, oracle):
    """Every one of the 384 FRSQRTE table inputs (both exponent parities),
    checked by the rows' mean squares, plus rows whose mean square is a
    denormal (eps = 0), which FRSQRTE normalises first."""
    import torch

    g = np.random.default_rng(5)
    rows, dim = 6000, 16
    x = (g.standard_normal((rows, dim)) * np.exp(g.uniform(-30, 30, (rows, 1)))).astype(F32)
    w = (1 + 0.1 * g.standard_normal(dim)).astype(F32)
    t = (np.mean(x.astype(np.float64) ** 2, axis=1) + 1e-6).astype(F32)
    assert len(np.unique(rsqrte_bucket(t))) >= 380  # (float64 means: edge rows may shift a bucket)
    out = torch.zeros((rows, dim), dtype=torch.float32, device="cuda")
    ane.rms_norm_fp32(rows, dim, 1e-6, dev(x), dev(w), out)
    got = host(out)
    for r in range(rows):
        same(got[r], oracle.rms_norm_fp32(x[r], w, 1e-6))
    tiny = (g.standard_normal((64, dim)) * np.exp(g.uniform(-52, -44, (64, 1)))).astype(F32)
    assert (np.mean(tiny.astype(np.float64) ** 2, axis=1) < 1.2e-38).all()  # denormal mean squares
    out = torch.zeros((64, dim), dtype=torch.float32, device="cuda")
    ane.rms_norm_fp32(64, dim, 0.0, dev(tiny), dev(w), out)
    got = host(out)
    for r in range(64):
        same(got[r], oracle.rms_norm_fp32(tiny[r], w, 0.0))


@pytest.mark.parametrize("n", [32, 4096, 1 << 20])
def test_silu_fp32_opcode(ane, oracle, n):
    import torch

    g = np.random.default_rng(n)
    x = (g.standard_normal(n) * 8).astype(F32)
    x[: SPECIAL.size] = SPECIAL
    out = torch.zeros(n, dtype=torch.float32, device="cuda")
    ane.stream_exec(ane.rec_silu(n, dev(x), out))
    same(host(out), oracle.silu_fp32(x))


def test_silu_fp32_every_exponent(ane, oracle):
    """Inputs at every binade from 2^-149 to 2^127 of both signs: the
    clamped exponent injection, its wrap for large negative inputs, and frecpe
    over its whole range."""
    import torch

    e = np.arange(-149, 128, dtype=np.float64)
    x = np.concatenate([np.ldexp(1.3, e.astype(int)), -np.ldexp(1.7, e.astype(int))]).astype(F32)
    x = x[np.isfinite(x)]
    x = np.concatenate([x, np.zeros((-x.size) % 16, F32)])
    out = torch.zeros(x.size, dtype=torch.float32, device="cuda")
    ane.silu_fp32(x.size, dev(x), out)
    same(host(out), oracle.silu_fp32(x))


@pytest.mark.parametrize("dim,theta", [(16, 10000.0), (128, 10000.0), (128, 500000.0), (64, 1e6), (6, 2.0),
                                       (7, 10000.0), (4096, 10000.0)])
@pytest.mark.parametrize("pos", [0, 1, 42, 4095, 100000])
def test_rope_fp32_opcode(ane, oracle, dim, theta, pos):
    """Any dim (pairs dim/2; an odd last element is left as it was), chunks
    past 16 pairs, positions up to 1e5."""
    import torch

    x = data.activations(1, dim, seed=dim + pos)[0]
    out = dev(np.full(dim, 3.0, F32))
    ane.stream_exec(ane.rec_rope(dim, pos, theta, dev(x), out))
    want = oracle.rope_fp32(x, pos, theta)
    if dim % 2:
        want[-1] = 3.0
    same(host(out), want)


def test_rope_fp32_rows(ane, oracle):
    import torch

    rows, dim = 40, 128
    x = data.activations(rows, dim, seed=5)
    out = torch.zeros((rows, dim), dtype=torch.float32, device="cuda")
    ane.rope_fp32(rows, dim, 777, 500000.0, dev(x), out)
    got = host(out)
    for r in range(rows):
        same(got[r], oracle.rope_fp32(x[r], 777, 500000.0))


@pytest.mark.parametrize("dim", [16, 4096, 16384])
def test_softmax_fp32_opcode(ane, oracle, dim):
    import torch

    g = np.random.default_rng(dim)
    x = (g.standard_normal(dim) * 6).astype(F32)
    out = torch.zeros(dim, dtype=torch.float32, device="cuda")
    ane.stream_exec(ane.rec_softmax(dim, dev(x), out))
    same(host(out), oracle.softmax_fp32(x))
    xd = dev(x)  # in place, as the handler allows
    ane.stream_exec(ane.rec_softmax(dim, xd, xd))
    same(host(xd), oracle.softmax_fp32(x))


def test_softmax_fp32_special_and_ragged(ane, oracle):
    import torch

    for x in (np.array([0.0] * 15 + [np.inf], F32), np.array([1.0] * 15 + [np.nan], F32),
              np.array([-np.inf] * 8 + [0.0] * 8, F32), np.full(32, -1e30, F32)):
        out = torch.zeros(x.size, dtype=torch.float32, device="cuda")
        ane.softmax_fp32(1, x.size, dev(x), out)
        same(host(out), oracle.softmax_fp32(x))
    for dim in (1, 5, 17, 1001):  # kernel entry: a short last vector adds nothing
        x = data.activations(1, dim, seed=dim)[0]
        out = torch.zeros(dim, dtype=torch.float32, device="cuda")
        ane.softmax_fp32(1, dim, dev(x), out)
        same(host(out), oracle.softmax_fp32(x))


def test_opcodes_refuse_partial_vectors(ane):
    """The handlers step 16 lanes with no tail: a length that is not a
    multiple of 16 never ends there, and stream_exec refuses it."""
    import torch

    x = torch.zeros(40, dtype=torch.float32, device="cuda")
    for rec in (ane.rec_rms_norm(20, 1e-5, x, x, x), ane.rec_silu(20, x, x), ane.rec_softmax(20, x, x)):
        with pytest.raises(ane.AneError) as e:
            ane.stream_exec(rec)
        assert e.value.status == 1


@pytest.mark.parametrize("K", [32, 512, 4096, 4128, 14336, 16384, 40960])
def test_rms_norm_build_matches_oracle(ane, oracle, K):
    """K = 4128: a last pass with one block; above 16384 the kernel holds
    x in batches and reloads it for the output."""
    import torch

    x = (data.activations(1, K, seed=K)[0] * 3).astype(F32)
    w = (1 + 0.1 * data.activations(1, K, seed=K + 1)[0]).astype(F32)
    out = torch.zeros(K, dtype=torch.float32, device="cuda")
    ane.rms_norm(K, dev(x), dev(w), 1e-5, out)
    same(host(out), oracle.rms_norm_build(x, w, 1e-5))


@pytest.mark.parametrize("N,K", [(6144, 4096), (300, 4096), (64, 8192), (28672, 4096)])
def test_fused_norm_equals_standalone_norm(ane, oracle, N, K):
    """The fused products' norm prologue and the standalone norm give the same
    activation bits: the product of the standalone output equals the fused
    product, whatever workgroup shape the product takes."""
    import torch

    W = data.q8_0_weights(N, K, seed=N + K)
    x = (data.activations(1, K, seed=11)[0] * 2).astype(F32)
    w = (1 + 0.1 * data.activations(1, K, seed=12)[0]).astype(F32)
    xn = torch.zeros(K, dtype=torch.float32, device="cuda")
    ane.rms_norm(K, dev(x), dev(w), 1e-5, xn)
    y1 = torch.zeros(N, dtype=torch.float32, device="cuda")
    y2 = torch.zeros(N, dtype=torch.float32, device="cuda")
    ane.q8_0_mul_mat(N, K, 1, xn, dev(W), y1)
    ane.q8_0_matvec_fused(N, K, dev(x), dev(W), y2, norm_w=dev(w), eps=1e-5)
    assert host(y1).tobytes() == host(y2).tobytes()
    ref = oracle.q8_0_mul_mat_g(N, K, 1, oracle.rms_norm_build(x, w, 1e-5)[None, :], W)[0]
    same(host(y2), ref)
