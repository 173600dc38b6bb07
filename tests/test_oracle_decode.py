"""The oracle's restatement of the decode-step handlers (rms_norm_fp32 0x51,
silu_fp32 0x54, rope_fp32 0x55, softmax_fp32 0x56, bytecode_interpreter.s
:6508-7009) and of the build's canonical RMSNorm, pinned without the GPU:

* the reference's own tests of these opcodes (tests/test_transformer.cpp
  :100-390 and test_new_ops.cpp:575-600): the same inputs, the same double
  precision references and the same tolerances;
* the Arm ARM's FRSQRTE / FRECPE: 8-bit estimates (relative error below
  2^-8 over every table entry of both exponent parities), exact scaling by
  powers of four / two, the special values, monotonicity;
* closed forms: silu(0) = 0, softmax sums to one and is invariant to a
  shift, rope at pos 0 is the identity and preserves each pair's norm, the
  two Newton steps of the norm leave it within a few ulps of 1/sqrt;
* the canonical norm against an exact rational sum of squares.
"""
from fractions import Fraction

import numpy as np
import pytest

F32 = np.float32


def close(got, want, tol):
    return np.max(np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))) <= tol


# ------------------------------------------------- the reference tests' references (double precision)
def ref_rms_norm(x, w, eps):
    x = np.asarray(x, np.float64)
    rms = np.sqrt(np.sum(x * x) / x.size + eps)
    return (x / rms * np.asarray(w, np.float64)).astype(F32)


def ref_softmax(x):
    x = np.asarray(x, np.float64)
    e = np.exp(x - x.max()).astype(F32).astype(np.float64)
    return (e / e.sum()).astype(F32)


def ref_silu(x):
    x = np.asarray(x, np.float64)
    return (x / (1.0 + np.exp(-x))).astype(F32)


def ref_rope(x, pos, theta):
    dim = x.size
    out = np.empty(dim, F32)
    for i in range(0, dim, 2):
        f = pos / np.power(float(theta), (2.0 * (i // 2)) / dim)
        c, s = np.cos(f), np.sin(f)
        out[i] = x[i] * c - x[i + 1] * s
        out[i + 1] = x[i] * s + x[i + 1] * c
    return out


def test_reference_rms_norm_tests(oracle):
    """test_transformer.cpp:100-170: five cases and their tolerances."""
    eps = F32(1e-5)
    i16 = np.arange(16, dtype=F32)
    cases = [(i16 + 1, np.ones(16, F32), 1e-4), (i16 + 1, (0.5 + 0.1 * i16).astype(F32), 1e-4),
             (np.full(16, 5.0, F32), np.ones(16, F32), 1e-4), (np.full(16, 1e-8, F32), np.ones(16, F32), 1e-2),
             (np.sin(np.arange(256, dtype=F32) * F32(0.1)).astype(F32), np.ones(256, F32), 1e-3)]
    for x, w, tol in cases:
        assert close(oracle.rms_norm_fp32(x, w, eps), ref_rms_norm(x, w, eps), tol)


def test_reference_softmax_tests(oracle):
    """test_transformer.cpp:175-258."""
    i16 = np.arange(16, dtype=F32)
    one_hot = np.zeros(16, F32)
    one_hot[7] = 100.0
    cases = [(np.ones(16, F32), 1e-5), (one_hot, 1e-5), (i16 - 8, 1e-4),
             (1000.0 + i16, 1e-4), (np.sin(np.arange(256, dtype=F32) * F32(0.05)).astype(F32) * F32(3), 1e-3)]
    for x, tol in cases:
        got = oracle.softmax_fp32(x)
        assert close(got, ref_softmax(x), tol)
    assert abs(float(np.sum(oracle.softmax_fp32(i16 * F32(0.5)), dtype=np.float32)) - 1.0) <= 1e-5
    assert abs(float(np.sum(oracle.softmax_fp32(1000.0 + i16), dtype=np.float32)) - 1.0) <= 1e-4


def test_reference_silu_tests(oracle):
    """test_transformer.cpp:262-330."""
    i16 = np.arange(16, dtype=F32)
    for x, tol in ((i16 - 8, 5e-3), ((-5.0 + 10.0 * i16 / 15).astype(F32), 5e-3),
                   ((-10.0 + 20.0 * np.arange(256, dtype=F32) / 255).astype(F32), 5e-3)):
        assert close(oracle.silu_fp32(x), ref_silu(x), tol)
    assert oracle.silu_fp32(np.zeros(16, F32))[0] == 0.0
    assert abs(oracle.silu_fp32(np.full(16, 10.0, F32))[0] - 10.0) <= 5e-2
    assert abs(oracle.silu_fp32(np.full(16, -10.0, F32))[0]) <= 5e-3


def test_reference_rope_tests(oracle):
    """test_transformer.cpp:336-390 (theta 10000) and the forward half of
    test_new_ops.cpp:584-593."""
    theta = F32(10000.0)
    x = np.arange(1, 17, dtype=F32)
    assert close(oracle.rope_fp32(x, 0, theta), x, 1e-4)
    e = np.zeros(16, F32)
    e[0], e[3] = 1.0, 1.0
    assert close(oracle.rope_fp32(e, 1, theta), ref_rope(e, 1, theta), 1e-3)
    assert close(oracle.rope_fp32(x, 42, theta), ref_rope(x, 42, theta), 1e-2)
    x128 = np.sin(np.arange(128, dtype=F32) * F32(0.1)).astype(F32)
    assert close(oracle.rope_fp32(x128, 100, theta), ref_rope(x128, 100, theta), 5e-2)
    x64 = (0.1 * np.arange(1, 65)).astype(F32)
    assert close(oracle.rope_fp32(x64, 7, theta), ref_rope(x64, 7, theta), 5e-3)


# ------------------------------------------------- estimates (Arm ARM FRSQRTE / FRECPE)
def _table_inputs():
    """Every (exponent parity, top fraction byte) of a normal float, mid-bucket."""
    out = []
    for e in (126, 127):
        for top in range(256):
            out.append(np.uint32((e << 23) | (top << 15) | (1 << 14)).view(F32))
    return np.array(out, F32)


def test_frsqrte_is_an_8_bit_estimate(oracle):
    xs = _table_inputs()
    est = np.array([oracle.frsqrte(x) for x in xs], np.float64)
    rel = np.abs(est * np.sqrt(xs.astype(np.float64)) - 1.0)
    assert rel.max() < 2.0 ** -8
    # an exponent step of two scales the estimate by exactly one half
    for x in xs[::17]:
        assert oracle.frsqrte(x * F32(4.0)) == oracle.frsqrte(x) * F32(0.5)
    srt = np.sort(xs)
    e2 = np.array([oracle.frsqrte(x) for x in srt])
    assert np.all(np.diff(e2) <= 0)  # non-increasing
    assert oracle.frsqrte(1.0) == F32(0.998046875)  # FRSQRTE(1.0) = 511/512
    assert np.isinf(oracle.frsqrte(0.0)) and oracle.frsqrte(np.inf) == 0.0
    assert np.isnan(oracle.frsqrte(-1.0)) and np.isnan(oracle.frsqrte(np.nan))
    d = np.uint32(3 << 20).view(F32)  # a denormal: normalised before the table
    assert abs(float(oracle.frsqrte(d)) * np.sqrt(float(d)) - 1.0) < 2.0 ** -8


def test_frecpe_is_an_8_bit_estimate(oracle):
    xs = _table_inputs()
    est = np.array([oracle.frecpe(x) for x in xs], np.float64)
    assert np.abs(est * xs.astype(np.float64) - 1.0).max() < 2.0 ** -8
    for x in xs[::13]:
        assert oracle.frecpe(x * F32(2.0)) == oracle.frecpe(x) * F32(0.5)
        assert oracle.frecpe(-x) == -oracle.frecpe(x)
    assert oracle.frecpe(1.0) == F32(0.998046875)
    assert np.isinf(oracle.frecpe(0.0)) and oracle.frecpe(np.inf) == 0.0
    assert np.isinf(oracle.frecpe(np.uint32(1 << 20).view(F32)))  # below 2^-128: overflows to inf
    big = F32(2.0 ** 126)  # result in the denormal range, still an 8-bit estimate
    assert abs(float(oracle.frecpe(big)) * 2.0 ** 126 - 1.0) < 2.0 ** -8


# ------------------------------------------------- closed forms
def test_rms_norm_newton_steps_reach_rsqrt(oracle):
    """After frsqrte and two frsqrts steps the scale is within 4 ulps of
    1/sqrt(mean + eps): x = c * ones gives out = fl(c * r), r ~ 1/|c|."""
    for c in (0.37, 1.0, 3.5, 123.25, 1e-3):
        x = np.full(32, c, F32)
        out = oracle.rms_norm_fp32(x, np.ones(32, F32), 0.0)
        r = float(out[0]) / c
        assert abs(r * c - 1.0) < 4 * 2.0 ** -23


def test_softmax_shift_invariance_and_sum(oracle):
    g = np.random.default_rng(3)
    x = g.standard_normal(4096).astype(F32) * F32(4)
    p = oracle.softmax_fp32(x)
    assert abs(float(np.sum(p, dtype=np.float64)) - 1.0) < 1e-5
    assert np.array_equal(p, oracle.softmax_fp32(x + F32(64.0))) or close(p, oracle.softmax_fp32(x + F32(64)), 1e-6)
    # the degree-4 exp polynomial: about 7e-4 relative at worst (measured)
    r = ref_softmax(x)
    assert np.all(np.abs(p.astype(np.float64) - r) <= 1e-3 * r + 1e-30)
    q = oracle.softmax_fp32(x[:1001])  # not a multiple of 16: absent lanes add nothing
    r = ref_softmax(x[:1001])
    assert np.all(np.abs(q.astype(np.float64) - r) <= 1e-3 * r + 1e-30)


def test_rope_preserves_pair_norms(oracle):
    g = np.random.default_rng(4)
    x = g.standard_normal(128).astype(F32)
    for pos in (0, 1, 17, 300, 4095):
        y = oracle.rope_fp32(x, pos, 500000.0)
        n0 = x[0::2].astype(np.float64) ** 2 + x[1::2].astype(np.float64) ** 2
        n1 = y[0::2].astype(np.float64) ** 2 + y[1::2].astype(np.float64) ** 2
        # sin to r^7 and cos to r^6 on [-pi/2, pi/2] (Taylor) keep sin^2 + cos^2
        # within about 2e-3 of one
        assert np.allclose(n1, n0, rtol=3e-3)
    # theta^(2/dim) comes from low-order ln / exp polynomials, so the phases
    # drift from the exact rotation as pos grows (at theta 500000, pos 4095 the
    # handler's output is off by up to ~4): only small positions are close
    assert close(oracle.rope_fp32(x, 0, 500000.0), x, 0.0)
    assert close(oracle.rope_fp32(x, 1, 500000.0), ref_rope(x, 1, F32(500000.0)), 5e-3)


def test_silu_large_inputs_follow_the_handler(oracle):
    """exp(-x) underflows to +0 through the clamped exponent for large x, so
    silu(x) = fl(x * fl(frecpe-refined 1)): within an ulp of x; for large
    negative x the injected exponent wraps, and the result is what the
    integer steps give (finite or zero, never a NaN from a finite input)."""
    x = np.array([20.0, 88.0, 100.0, 1e10], F32)
    y = oracle.silu_fp32(np.tile(x, 4))[:4]
    assert np.all(np.abs(y / x - 1.0) <= 2.0 ** -22)
    z = oracle.silu_fp32(np.tile(np.array([-20.0, -88.0, -89.0, -1e10], F32), 4))
    assert not np.isnan(z).any()


# ------------------------------------------------- the build's canonical RMSNorm
@pytest.mark.parametrize("K", [32, 512, 4096, 14336])
def test_rms_norm_build_against_exact_sum(oracle, K):
    g = np.random.default_rng(K)
    x = (g.standard_normal(K) * 3).astype(F32)
    w = (1 + 0.1 * g.standard_normal(K)).astype(F32)
    eps = F32(1e-5)
    out = oracle.rms_norm_build(x, w, eps)
    exact = sum(Fraction(float(v)) ** 2 for v in x)
    ms = np.float32(float(exact / K))  # the exact sum rounded once (fp64 errors are far below fp32's)
    inv = F32(1.0) / np.sqrt(np.float32(ms + eps))
    want = ((x * inv).astype(F32) * w).astype(F32)
    assert np.array_equal(out, want)
