"""The identity behind the resident quantizer's fast path (pack4_fast in
ane_amd/csrc/common.hpp), checked on the CPU against the oracle's
quantize_fp32_i8 (oracle/ane_oracle.c, bytecode_interpreter.s:1885-1950).

When a tensor's max |x| and inv = 127 / max are both finite, t = fl(x * inv)
is finite with |t| <= 127 (1 + 2^-24)^2 < 127.5 for every element x, so the
handler's clamp to [-127, 127] cannot bind after rounding, and its
q = fcvtzs(frintn(clamp(t, -127, 127))) equals the low byte of the bits of
fl(t + 1.5 * 2^23): that sum lies in [2^23, 2^24), where the fp32 ulp is 1,
so the one rounding of the addition is round-half-to-even to an integer
(frintn), and the integer's two's-complement byte is the low byte of the
float's bits (which the kernel's SDWA add writes straight into its byte of
the packed result).  numpy float32 arithmetic rounds each operation to
nearest-even, as the GPU's fmul and fadd do, so the restatement below is the
kernel's arithmetic, and the oracle is the reference's.  CPU only."""
import numpy as np
import pytest

F32 = np.float32
MAGIC = F32(12582912.0)  # 1.5 * 2^23


def fast_q(x: np.ndarray, amax: np.float32) -> np.ndarray:
    inv = F32(127.0) / amax if amax != 0 else F32(127.0)
    assert np.isfinite(amax) and np.isfinite(inv)
    t = (x.astype(F32) * inv).astype(F32)
    s = (t + MAGIC).astype(F32)  # no clamp: |t| < 127.5
    return (s.view(np.uint32) & 0xFF).astype(np.uint8).view(np.int8)


def oracle_q(oracle, x: np.ndarray):
    # the handler processes ceil16(count) elements: pad with zeros, which
    # change neither the maximum nor the other outputs
    n = max(16, -(-x.size // 16) * 16)
    xp = np.zeros(n, F32)
    xp[: x.size] = x
    q, s = oracle.quantize(xp, x.size)
    return q[: x.size], s


def amax_of(x: np.ndarray) -> np.float32:
    return F32(np.max(np.abs(x))) if x.size else F32(0)


@pytest.mark.parametrize("seed,n", [(1, 4096), (2, 65536), (3, 1000)])
def test_fast_identity_random(oracle, seed, n):
    x = np.random.default_rng(seed).standard_normal(n).astype(F32)
    q, _ = oracle_q(oracle, x)
    np.testing.assert_array_equal(fast_q(x, amax_of(x)), q)


def test_fast_identity_every_tie_and_the_clamp(oracle):
    """amax = 127 gives inv = 1, so t = x: every half-integer tie in
    [-127, 127] (half-to-even, including +-0.5 -> 0), values just inside
    and at the clamp, and signed zeros."""
    ties = np.arange(-127, 127, dtype=F32) + F32(0.5)
    near = np.array([126.49999, 126.5, 126.50001, 126.99999, -126.5, -126.99999, 0.49999997, -0.49999997,
                     0.0, -0.0, 1e-30, -1e-30, 1e-40, -1e-40], F32)
    x = np.concatenate([ties, near, np.array([127.0, -127.0], F32)])
    assert amax_of(x) == F32(127.0)
    q, _ = oracle_q(oracle, x)
    got = fast_q(x, amax_of(x))
    np.testing.assert_array_equal(got, q)
    assert got[list(ties).index(F32(0.5))] == 0 and got[list(ties).index(F32(-0.5))] == 0
    assert got[list(ties).index(F32(1.5))] == 2 and got[list(ties).index(F32(2.5))] == 2


@pytest.mark.parametrize("amax", [3.0, 4.5, 1e-30, 1e-36, 1e30, 3.0e38])
def test_fast_identity_scales(oracle, amax):
    """Tensors whose max sets inv to ordinary, very large (amax 1e-36: inv
    ~1.27e38, still finite) and very small values; the element at +-amax may
    round just past 127 in t, and still rounds to +-127."""
    g = np.random.default_rng(int(np.log10(amax) + 50))
    x = (g.uniform(-1, 1, 8192) * amax).astype(F32)
    x[0], x[1] = F32(amax), F32(-amax)
    a = amax_of(x)
    inv = F32(127.0) / a
    assert np.isfinite(inv)
    q, _ = oracle_q(oracle, x)
    np.testing.assert_array_equal(fast_q(x, a), q)


def test_fast_path_condition_excludes_overflowing_inv():
    """A max below 127 / FLT_MAX makes inv infinite: the kernel's condition
    (fast_quant_ok) then sends the tensor to the exact quantizer, where
    0 * inf gives NaN and NaN gives 0."""
    for amax in (F32(1e-40), F32(3e-39)):
        with np.errstate(over="ignore", divide="ignore"):
            assert not np.isfinite(F32(127.0) / amax)


def test_fast_path_bound_at_the_max():
    """The bound the missing clamp rests on: t = fl(amax * fl(127 / amax))
    stays below 127.5 (it is 127 up to a few ulps) for maxima over the whole
    fp32 range where inv is finite (amax >= 127 / FLT_MAX; random bit
    patterns, whose subnormals and tiny normals drop out with an infinite
    inv), including every power of two and its neighbours."""
    g = np.random.default_rng(7)
    bits = g.integers(1, 0x7F7FFFFF, 400_000, dtype=np.uint32)  # positive finite floats
    pow2 = (np.arange(1, 255, dtype=np.uint32) << 23)
    edges = np.concatenate([pow2 - 1, pow2, pow2 + 1]).astype(np.uint32)
    amax = np.concatenate([bits, edges]).view(F32)
    with np.errstate(over="ignore", divide="ignore"):
        inv = (F32(127.0) / amax).astype(F32)
    ok = np.isfinite(inv)
    t = (amax[ok] * inv[ok]).astype(F32)
    assert ok.sum() > 390_000
    assert np.all(np.abs(t) < F32(127.5)), np.abs(t).max()
    assert np.abs(t - F32(127.0)).max() <= F32(127.0) * F32(2.0 ** -22)
    # and the fast form at x = +-amax is +-127 exactly
    q = (((t + MAGIC).astype(F32)).view(np.uint32) & 0xFF).astype(np.uint8).view(np.int8)
    assert np.all(q == 127)

