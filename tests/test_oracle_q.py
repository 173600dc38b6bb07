"""Pins of the oracle's other weight formats (CPU only).

get_rows_q8_0 / get_rows_q4_0: the reference's own known-answer tables
(test_remaining_ops.cpp:230-325, 328-430), rebuilt here byte for byte.

q4_0_gemv: a one-hot x turns the GEMV into element n of each dequantized row
(one nonzero lane, an exact fma and an exact FADDV), so every element of
gemv(e_n) must equal get_rows_q4_0's, which the reference's table pins.

Q*_K GEMVs (no reference test exists): the element layout of each handler
(bytecode_interpreter.s:11024-11626) restated a second way, as vectorized
numpy dequantizers, and checked through one-hot probes (bit-exact) and
through integer-valued cases where every product and sum is exact, so the
result is the exact dot product whatever the summation order.  Q3_K's
second-half shift by the first half's input bits is checked in its closed
forms: +0.0 inputs (no shift), normal inputs (field 0) and tiny denormals
(shift by the denormal's bit pattern).
"""
import numpy as np
import pytest

from tests import _oracle, data

F32 = np.float32


@pytest.fixture(scope="module")
def oracle():
    return _oracle.load()


def f16(v) -> np.ndarray:
    """float_to_fp16 of the reference tests: a float32 value cast to __fp16 (RNE)."""
    return np.array(v, dtype=F32).astype(np.float16)


# ------------------------------------------------------------ get_rows KATs
def kat_q8_0_table(dim):
    vocab, bpr = 4, dim // 32
    T = np.zeros((vocab, bpr, 34), np.uint8)
    for v in range(vocab):
        for b in range(bpr):
            if dim == 32:
                scale = F32(0.1) * F32(v + 1)
                vals = [(q + v * 7) % 21 - 10 for q in range(32)]
            else:
                scale = F32(0.05) * F32(v + b + 1)
                vals = [(q + v * 3 + b * 5) % 19 - 9 for q in range(32)]
            T[v, b, :2] = f16(scale).reshape(1).view(np.uint8)
            T[v, b, 2:] = np.array(vals, np.int8).view(np.uint8)
    return T.reshape(vocab, bpr * 34)


def kat_q4_0_table(dim):
    vocab, bpr = 4, dim // 32
    T = np.zeros((vocab, bpr, 18), np.uint8)
    for v in range(vocab):
        for b in range(bpr):
            if dim == 32:
                scale = F32(0.2) * F32(v + 1)
                lo = [(i + v) % 16 for i in range(16)]
                hi = [(i + v + 3) % 16 for i in range(16)]
            else:
                scale = F32(0.15) * F32(v + b + 1)
                lo = [(i + v + b * 2) % 16 for i in range(16)]
                hi = [(i + v + b * 2 + 5) % 16 for i in range(16)]
            T[v, b, :2] = f16(scale).reshape(1).view(np.uint8)
            T[v, b, 2:] = (np.array(hi, np.uint8) << 4) | np.array(lo, np.uint8)
    return T.reshape(vocab, bpr * 18)


def kat_expected(table, fmt, dim, indices):
    """The tests' CPU reference loops: (float)qval * (float)fp16 scale."""
    bpr = dim // 32
    bb = 34 if fmt == "q8_0" else 18
    out = np.zeros((len(indices), dim), F32)
    for r, idx in enumerate(indices):
        for b in range(bpr):
            blk = table[idx, b * bb:(b + 1) * bb]
            scale = F32(blk[:2].view(np.float16)[0])
            if fmt == "q8_0":
                q = blk[2:].view(np.int8).astype(F32)
                out[r, b * 32:(b + 1) * 32] = q * scale
            else:
                out[r, b * 32:b * 32 + 16] = ((blk[2:] & 15).astype(np.int32) - 8).astype(F32) * scale
                out[r, b * 32 + 16:b * 32 + 32] = ((blk[2:] >> 4).astype(np.int32) - 8).astype(F32) * scale
    return out


@pytest.mark.parametrize("dim", [32, 64])
def test_get_rows_q8_0_reference_kat(oracle, dim):
    T = kat_q8_0_table(dim)
    idx = [1, 3]
    got = oracle.get_rows("q8_0", 2, dim, T, idx)
    assert got.tobytes() == kat_expected(T, "q8_0", dim, idx).tobytes()


@pytest.mark.parametrize("dim", [32, 64])
def test_get_rows_q4_0_reference_kat(oracle, dim):
    T = kat_q4_0_table(dim)
    idx = [0, 2]
    got = oracle.get_rows("q4_0", 2, dim, T, idx)
    assert got.tobytes() == kat_expected(T, "q4_0", dim, idx).tobytes()


# ------------------------------------------------------------ Q4_0 GEMV
def test_q4_0_gemv_one_hot_equals_get_rows(oracle):
    M, K = 5, 96
    W = data.q_weights("q4_0", M, K, seed=21)
    rows = oracle.get_rows("q4_0", M, K, W, np.arange(M))
    for n in range(K):
        x = np.zeros(K, F32)
        x[n] = 1.0
        assert np.array_equal(oracle.q_gemv("q4_0", M, K, x, W), rows[:, n]), n


def test_q4_0_gemv_integer_exact(oracle):
    """d = 1 and small integer x: every fma and add is exact."""
    M, K = 7, 256
    W = data.q_weights("q4_0", M, K, seed=22).reshape(M, K // 32, 18)
    W[:, :, :2] = np.array([1.0], np.float16).view(np.uint8)
    W = W.reshape(M, -1)
    x = data.rng(23).integers(-9, 10, K).astype(F32)
    q = np.zeros((M, K), np.int64)
    Wb = W.reshape(M, K // 32, 18)
    for b in range(K // 32):
        q[:, 32 * b:32 * b + 16] = (Wb[:, b, 2:] & 15).astype(np.int64) - 8
        q[:, 32 * b + 16:32 * b + 32] = (Wb[:, b, 2:] >> 4).astype(np.int64) - 8
    ref = (q @ x.astype(np.int64)).astype(F32)
    assert oracle.q_gemv("q4_0", M, K, x, W).tobytes() == ref.tobytes()


# ------------------------------------------------------------ K-quants
def _h(b, off):
    return b[..., off:off + 2].copy().view(np.float16)[..., 0].astype(F32)


def _u32(b, off):
    v = b[..., off:off + 4].astype(np.uint32)
    return v[..., 0] | (v[..., 1] << 8) | (v[..., 2] << 16) | (v[..., 3] << 24)


def _u16(b, off):
    v = b[..., off:off + 2].astype(np.uint32)
    return v[..., 0] | (v[..., 1] << 8)


def _scale_min_6bit(s, j):
    s = s.astype(np.uint32)
    if j < 4:
        return s[..., j] & 63, s[..., j + 4] & 63
    return (s[..., j + 4] & 15) | ((s[..., j - 4] >> 6) << 4), (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4)


def deq(fmt, W, K, xfirst_bits=None):
    """Dequantized rows [M][K] (float32), one super-block at a time.
    xfirst_bits [K] (uint32): the input bit patterns Q3_K's second halves
    are shifted by (None: +0.0 everywhere)."""
    M = W.shape[0]
    nsb = K // 256
    out = np.zeros((M, K), F32)
    for sb in range(nsb):
        if fmt == "q4_k" or fmt == "q5_k":
            B = W[:, sb * (144 if fmt == "q4_k" else 176):][:, :176]
            d, nmin = _h(B, 0), -_h(B, 2)
            for j in range(8):
                sc, m = _scale_min_6bit(B[:, 4:16], j)
                ds, dm = d * sc.astype(F32), nmin * m.astype(F32)
                qoff = 16 if fmt == "q4_k" else 48
                q = B[:, qoff + 16 * j: qoff + 16 * j + 16].astype(np.uint32)
                lo, hi = q & 15, q >> 4
                if fmt == "q5_k":
                    h = _u32(B, 16 + 4 * j)[:, None]
                    ll = np.arange(16, dtype=np.uint32)
                    lo = lo | (((h & 0xFFFF) >> ll) & 1) << 4
                    hi = hi | (((h >> 16) >> ll) & 1) << 4
                base = 256 * sb + 32 * j
                out[:, base:base + 16] = lo.astype(F32) * ds[:, None] + dm[:, None]
                out[:, base + 16:base + 32] = hi.astype(F32) * ds[:, None] + dm[:, None]
        elif fmt == "q2_k":
            B = W[:, sb * 84:(sb + 1) * 84]
            d, nmin = _h(B, 80), -_h(B, 82)
            for j in range(16):
                sc, m = (B[:, j] & 15).astype(F32), (B[:, j] >> 4).astype(F32)
                w = _u32(B, 16 + 4 * j)[:, None] >> (2 * np.arange(16, dtype=np.uint32)) & 3
                out[:, 256 * sb + 16 * j:256 * sb + 16 * j + 16] = (
                    w.astype(F32) * (d * sc)[:, None] + (nmin * m)[:, None])
        elif fmt == "q3_k":
            B = W[:, sb * 110:(sb + 1) * 110]
            d = _h(B, 108)
            ll = np.arange(16, dtype=np.uint32)
            for j in range(8):
                sc, _ = _scale_min_6bit(B[:, 96:108], j)
                ds = d * (sc.astype(np.int32) - 32).astype(F32)
                qa, qb = _u32(B, 32 + 8 * j)[:, None], _u32(B, 32 + 8 * j + 4)[:, None]
                ha, hb = _u16(B, 4 * j)[:, None], _u16(B, 4 * j + 2)[:, None]
                base = 256 * sb + 32 * j
                sh = np.zeros(16, np.uint64) if xfirst_bits is None else xfirst_bits[base:base + 16].astype(np.uint64)
                qb_sh = np.where(sh >= 32, 0, qb.astype(np.uint64) >> np.minimum(sh, 31)).astype(np.uint32)
                a = ((qa >> (2 * ll)) & 3) | (((ha >> ll) & 1) << 2)
                b = ((qb_sh >> (2 * ll)) & 3) | (((hb >> ll) & 1) << 2)
                out[:, base:base + 16] = (a.astype(np.int32) - 4).astype(F32) * ds[:, None]
                out[:, base + 16:base + 32] = (b.astype(np.int32) - 4).astype(F32) * ds[:, None]
        elif fmt == "q6_k":
            B = W[:, sb * 210:(sb + 1) * 210]
            d = _h(B, 208)
            n = np.arange(16)
            for j in range(16):
                ds = d * B[:, 192 + j].view(np.int8).astype(F32)
                byte = B[:, 8 * j + n // 2].astype(np.uint32)
                nib = np.where(n % 2 == 1, byte >> 4, byte & 15)
                h = _u32(B, 128 + 4 * j)[:, None]
                q = nib | (((h >> (2 * n.astype(np.uint32))) & 3) << 4)
                out[:, 256 * sb + 16 * j:256 * sb + 16 * j + 16] = (q.astype(np.int32) - 32).astype(F32) * ds[:, None]
    return out


KQ = ["q4_k", "q2_k", "q3_k", "q5_k", "q6_k"]


@pytest.mark.parametrize("fmt", KQ)
def test_kquant_one_hot_equals_dequant(oracle, fmt):
    M, K = 3, 512
    W = data.q_weights(fmt, M, K, seed=30 + KQ.index(fmt))
    D = deq(fmt, W, K)
    for n in range(K):
        x = np.zeros(K, F32)
        x[n] = 1.0
        # (value equality: a zero weight of negative scale dequantizes to -0.0,
        # the probe's fma chain to +0.0).  Q3_K: a 1.0 in a first half zeroes
        # that lane's second-half field, whose input is 0 here.
        assert np.array_equal(oracle.q_gemv(fmt, M, K, x, W), D[:, n]), (fmt, n)


@pytest.mark.parametrize("fmt", KQ)
def test_kquant_integer_exact(oracle, fmt):
    """fp16 scales 1 (and dmin 1): every dequantized value is a small
    integer, x holds small integers, so the GEMV is the exact dot product."""
    M, K = 4, 768
    nbytes, _, fp16_at = data.Q_BLOCK[fmt]
    W = data.q_weights(fmt, M, K, seed=40 + KQ.index(fmt)).reshape(M, K // 256, nbytes)
    for off in fp16_at:
        W[:, :, off:off + 2] = np.array([1.0], np.float16).view(np.uint8)
    W = W.reshape(M, -1)
    x = data.rng(41).integers(-3, 4, K).astype(F32)
    if fmt == "q3_k":  # first halves +0.0 keep the plain second-half decode
        for j in range(K // 32):
            x[32 * j:32 * j + 16] = 0.0
    D = deq(fmt, W, K)
    assert np.all(D == np.round(D)) and np.abs(D).max() < 2 ** 12
    ref = (D.astype(np.float64) @ x.astype(np.float64)).astype(F32)
    assert oracle.q_gemv(fmt, M, K, x, W).tobytes() == ref.tobytes()


@pytest.mark.parametrize("first", ["zero", "normal", "denormal"])
def test_q3_k_second_half_shift(oracle, first):
    """x holds v at element 32j+l (first half) and 1 at 32j+16+l, zeros
    elsewhere, and d = 1 makes every weight an integer; lane l then ends at
    fl(wa * v + wb) exactly, where wb decodes its 2-bit field from the qs word
    shifted right by the bit pattern of v: no shift for +0.0, a zero field
    for a normal v, a shift by k for the denormal k * 2^-149."""
    M, K = 3, 256
    W = data.q_weights("q3_k", M, K, seed=50).reshape(M, 1, 110)
    W[:, :, 108:110] = np.array([1.0], np.float16).view(np.uint8)
    W = W.reshape(M, -1)
    for j in (0, 3, 7):
        for l in (0, 5, 15):
            bits = {"zero": 0, "normal": 0x3F800000, "denormal": 2 * l + 1}[first]
            v = np.array(bits, np.uint32).view(F32)
            x = np.zeros(K, F32)
            x[32 * j + l] = v
            x[32 * j + 16 + l] = 1.0
            xb = np.zeros(K, np.uint32)
            xb[32 * j + l] = bits
            D = deq("q3_k", W, K, xfirst_bits=xb)
            wa, wb = D[:, 32 * j + l], D[:, 32 * j + 16 + l]
            if first == "normal":  # field 0: (hbit << 2) - 4 in {-4, 0}, times the scale
                ds = data_q3_ds(W, j)
                assert np.all((wb == F32(-4) * ds) | (wb == F32(0) * ds))
            expect = (wa.astype(np.float64) * np.float64(v) + wb.astype(np.float64)).astype(F32)
            got = oracle.q_gemv("q3_k", M, K, x, W)
            assert np.array_equal(got, expect), (first, j, l)
        if first != "zero":  # the quirk changes the decode somewhere in this matrix
            assert not np.array_equal(deq("q3_k", W, K, xfirst_bits=xb), deq("q3_k", W, K))


def data_q3_ds(W, j):
    B = W[:, :110]
    d = _h(B, 108)
    sc, _ = _scale_min_6bit(B[:, 96:108], j)
    return d * (sc.astype(np.int32) - 32).astype(F32)
