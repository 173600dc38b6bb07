"""The fp32 ops of the ggml backend -- ADD, MUL, SCALE, RMS_NORM, SOFT_MAX,
SILU (GGML_OP_UNARY), ROPE and CPY/CONT/DUP, the ops the reference backend
maps besides MUL_MAT (ref src/ggml-backend/ggml-ane.cpp:155-277, :369-383)
-- driven through ggml_backend_ane_reg() (ane_amd/ggml/ggml-ane.cpp) with
ggml_tensor nodes built here after the restated tests/ggml_iface/ggml.h,
as ggml's scheduler hands them over.

Oracle:
* ADD, MUL, SCALE and the copies are single IEEE fp32 operations (or
  moves): numpy float32 computes the same bits;
* RMS_NORM, SOFT_MAX, SILU and ROPE run the reference handlers' arithmetic
  (0x51, 0x56, 0x54, 0x55), so each row is compared bit for bit with the
  oracle's restatement of that handler (oracle/ane_oracle.c), composed with
  ggml's semantics around it: unit weights; the softmax pre-pass
  fl(fl(x * scale) + mask) in numpy float32; a -inf after the pre-pass
  gives 0, which the handler arithmetic gives for -1e30 (exp_poly's
  exponent saturates), so the oracle row has -1e30 there; RoPE's position
  per token (src1[i2]) and base from op_params[5];
* each of those is also checked against float64 closed forms (RMS norm,
  softmax with the mask, the rotation by pos * base^(-2i/n)) to the
  handlers' accuracy (the exp polynomial's ~7e-4, RoPE's base-dependent
  ratio error at small positions), so that a wrong row, mask row,
  position or pairing fails even where the oracle composition above would
  share the mistake.

CPU: the ctypes mirror of the restated ggml_tensor against the C layout, and
supports_op decisions (claimed and refused cases) through the registry.
GPU: each op, its broadcast / strided / in-place forms, and one graph of a
transformer block's nodes (norm, weight multiply, Q8_0 products, SiLU gate,
residual add, scale, reshape, RoPE, copy into a cache view) computed in one
graph_compute, bit-identical to the oracle's composition.
"""
import ctypes
import shutil
import struct
import subprocess

import numpy as np
import pytest

import ane_amd
from ane_amd import build as ane_build
from tests import data

F32 = np.float32
T_F32, T_F16, T_Q8, T_I32 = 0, 1, 8, 26


class GTensor(ctypes.Structure):
    """ctypes mirror of the restated ggml_tensor (tests/ggml_iface/ggml.h)."""


GTensor._fields_ = [
    ("type", ctypes.c_int),
    ("buffer", ctypes.c_void_p),
    ("ne", ctypes.c_int64 * 4),
    ("nb", ctypes.c_size_t * 4),
    ("op", ctypes.c_int),
    ("op_params", ctypes.c_int32 * 16),
    ("flags", ctypes.c_int32),
    ("src", ctypes.POINTER(GTensor) * 10),
    ("view_src", ctypes.POINTER(GTensor)),
    ("view_offs", ctypes.c_size_t),
    ("data", ctypes.c_void_p),
    ("name", ctypes.c_char * 64),
    ("extra", ctypes.c_void_p),
    ("padding", ctypes.c_char * 8),
]
_FIELDS = ("type", "buffer", "ne", "nb", "op", "op_params", "flags", "src", "view_src", "view_offs", "data", "name",
           "extra", "padding")


def _f(v: float) -> int:
    return struct.unpack("<i", struct.pack("<f", v))[0]


def _load(path):
    ane_amd.lib()  # libane_amd.so first (RTLD_GLOBAL)
    t = ctypes.CDLL(str(path))
    t.ggml_ane_test_op.argtypes = [ctypes.c_char_p]
    t.ggml_ane_test_layout.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.c_int]
    t.ggml_ane_test_supports_node.argtypes = [ctypes.POINTER(GTensor)]
    t.ggml_ane_test_backend_new.restype = ctypes.c_void_p
    t.ggml_ane_test_backend_free.argtypes = [ctypes.c_void_p]
    t.ggml_ane_test_graph.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.POINTER(GTensor)), ctypes.c_int]
    return t


class Graph:
    """Builds restated ggml_tensor nodes (keeping their data alive) and runs
    them through the registry's backend."""

    def __init__(self, lib):
        self.L = lib
        self.keep = []
        self.silu = lib.ggml_ane_test_unary_silu()

    def op(self, name: str) -> int:
        v = self.L.ggml_ane_test_op(name.encode())
        assert v >= 0, name
        return v

    def tensor(self, ne, data=None, nb=None, type_=T_F32, op="NONE", src=(), params=()):
        ne = list(ne) + [1] * (4 - len(ne))
        t = GTensor()
        t.type = type_
        for i in range(4):
            t.ne[i] = ne[i]
        if nb is None:
            es = 4 if type_ in (T_F32, T_I32) else 2
            nb = [es, es * ne[0], es * ne[0] * ne[1], es * ne[0] * ne[1] * ne[2]]
        for i in range(4):
            t.nb[i] = nb[i]
        t.op = self.op(op)
        for i, w in enumerate(params):
            t.op_params[i] = _f(w) if isinstance(w, float) else int(w)
        for i, s in enumerate(src):
            if s is not None:
                t.src[i] = ctypes.pointer(s)
        if data is not None:
            t.data = data.data_ptr() if hasattr(data, "data_ptr") else int(data)
            self.keep.append(data)
        self.keep.append(t)
        return t

    def supports(self, node) -> bool:
        return self.L.ggml_ane_test_supports_node(ctypes.byref(node)) == 1

    def run(self, nodes) -> int:
        be = self.L.ggml_ane_test_backend_new()
        assert be
        try:
            arr = (ctypes.POINTER(GTensor) * len(nodes))(*[ctypes.pointer(n) for n in nodes])
            return self.L.ggml_ane_test_graph(be, arr, len(nodes))
        finally:
            self.L.ggml_ane_test_backend_free(be)


@pytest.fixture(scope="module")
def fresh(tmp_path_factory):
    """The adapter and harness compiled now, into a temporary library."""
    if not shutil.which("g++"):
        pytest.skip("g++ not available")
    out = tmp_path_factory.mktemp("ggml_ops") / "libggml_ane_test.so"
    res = subprocess.run(ane_build.ggml_adapter_cmd(out), capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    return _load(out)


# ------------------------------------------------------------------ CPU
def test_ggml_tensor_mirror_layout(fresh):
    buf = (ctypes.c_size_t * 32)()
    n = fresh.ggml_ane_test_layout(buf, 32)
    assert n == 1 + len(_FIELDS)
    assert list(buf[:n]) == [ctypes.sizeof(GTensor)] + [getattr(GTensor, f).offset for f in _FIELDS]


def _rope(g, x, pos, n_dims=None, mode=0, base=10000.0, fscale=1.0, ext=0.0, attn=1.0, ff=None):
    n_dims = x.ne[0] if n_dims is None else n_dims
    params = [0, n_dims, mode, 0, 4096, base, fscale, ext, attn, 32.0, 1.0]
    return g.tensor(list(x.ne), op="ROPE", src=(x, pos, ff), params=params)


def test_supports_fp32_ops(fresh):
    g = Graph(fresh)
    a = g.tensor([64, 7, 3])
    b = g.tensor([64, 7, 3])
    row = g.tensor([64])
    for op in ("ADD", "MUL"):
        assert g.supports(g.tensor([64, 7, 3], op=op, src=(a, b)))
        assert g.supports(g.tensor([64, 7, 3], op=op, src=(a, row)))  # src1 repeated over rows
        assert g.supports(g.tensor([64, 7, 3], op=op, src=(a, g.tensor([16, 7]))))  # 16 | 64, 1 | 3
        assert not g.supports(g.tensor([64, 7, 3], op=op, src=(a, g.tensor([48]))))  # 48 does not divide 64
        assert not g.supports(g.tensor([64, 7, 3], op=op, src=(g.tensor([64, 7]), b)))  # src0 is not dst's shape
        assert not g.supports(g.tensor([64, 7, 3], op=op, src=(a, g.tensor([64, 7, 3], type_=T_F16))))
    assert g.supports(g.tensor([64, 7, 3], op="SCALE", src=(a,), params=[0.5]))
    assert not g.supports(g.tensor([64, 7, 3], op="SCALE", src=(a,), params=[0.5, 1.0]))  # scale with bias
    assert g.supports(g.tensor([64, 7, 3], op="RMS_NORM", src=(a,), params=[1e-5]))
    assert not g.supports(g.tensor([60, 7], op="RMS_NORM", src=(g.tensor([60, 7]),), params=[1e-5]))  # 60 % 16
    sm = g.tensor([37, 5, 4])
    assert g.supports(g.tensor([37, 5, 4], op="SOFT_MAX", src=(sm,), params=[1.0, 0.0]))
    assert g.supports(g.tensor([37, 5, 4], op="SOFT_MAX", src=(sm, g.tensor([37, 8])), params=[0.125, 0.0]))
    assert g.supports(g.tensor([37, 5, 4], op="SOFT_MAX", src=(sm, g.tensor([37, 5, 2])), params=[0.125, 0.0]))
    assert not g.supports(g.tensor([37, 5, 4], op="SOFT_MAX", src=(sm, g.tensor([37, 4])), params=[1.0, 0.0]))
    assert not g.supports(g.tensor([37, 5, 4], op="SOFT_MAX", src=(sm, g.tensor([37, 5, 3])), params=[1.0, 0.0]))
    assert not g.supports(g.tensor([37, 5, 4], op="SOFT_MAX", src=(sm,), params=[1.0, 8.0]))  # ALiBi
    assert not g.supports(g.tensor([37, 5, 4], op="SOFT_MAX", src=(sm, None, g.tensor([4])), params=[1.0, 0.0]))
    assert not g.supports(g.tensor([37, 5, 4], op="SOFT_MAX", src=(sm, g.tensor([37, 8], type_=T_F16)),
                                   params=[1.0, 0.0]))
    assert g.supports(g.tensor([64, 7, 3], op="UNARY", src=(a,), params=[g.silu]))
    assert not g.supports(g.tensor([64, 7, 3], op="UNARY", src=(a,), params=[g.silu - 1]))  # another unary op
    strided = g.tensor([64, 7, 3], nb=[4, 4 * 72, 4 * 72 * 7, 4 * 72 * 21])
    assert not g.supports(g.tensor([64, 7, 3], op="UNARY", src=(strided,), params=[g.silu]))
    x = g.tensor([128, 8, 5])
    pos = g.tensor([5], type_=T_I32)
    assert g.supports(_rope(g, x, pos))
    assert g.supports(_rope(g, g.tensor([128, 8, 5], nb=[4, 512, 512 * 12, 512 * 60]), pos))  # a view of qkv
    assert not g.supports(_rope(g, x, pos, mode=2))          # NEOX pairs
    assert not g.supports(_rope(g, x, pos, n_dims=64))       # partial rotation
    assert not g.supports(_rope(g, x, pos, fscale=0.25))     # linear scaling
    assert not g.supports(_rope(g, x, pos, ext=1.0))         # YaRN
    assert not g.supports(_rope(g, x, pos, attn=2.0))
    assert not g.supports(_rope(g, x, pos, ff=g.tensor([64])))  # frequency factors
    assert not g.supports(_rope(g, x, g.tensor([4], type_=T_I32)))  # one position per token
    assert not g.supports(_rope(g, x, g.tensor([5])))           # F32 positions
    t = g.tensor([7, 64], nb=[4 * 64, 4, 4 * 64 * 7, 4 * 64 * 7])  # a transposed view
    for op in ("CPY", "CONT", "DUP"):
        assert g.supports(g.tensor([7, 64], op=op, src=(t,)))
    assert g.supports(g.tensor([448], op="CPY", src=(t,)))       # equal element counts
    assert not g.supports(g.tensor([440], op="CPY", src=(t,)))
    assert not g.supports(g.tensor([448], type_=T_F16, op="CPY", src=(t,)))  # F32 -> F16 stays on the CPU
    for op in ("RESHAPE", "VIEW", "PERMUTE", "TRANSPOSE"):
        assert g.supports(g.tensor([64, 7, 3], op=op, src=(a,)))


# ------------------------------------------------------------------ GPU
@pytest.fixture(scope="module")
def built():
    if not ane_build.GGML_TEST_LIB.exists():
        pytest.fail(f"{ane_build.GGML_TEST_LIB} is missing: run python -m ane_amd.build")
    return _load(ane_build.GGML_TEST_LIB)


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def same(got, want):
    got = np.ascontiguousarray(got, F32)
    want = np.ascontiguousarray(want, F32)
    assert got.shape == want.shape
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{bad.size} differ, first at {bad[0]}: {got.ravel()[bad[0]]} vs {want.ravel()[bad[0]]}"


def _ok(g, nodes):
    assert g.run(nodes) == 0  # GGML_STATUS_SUCCESS


def rnd(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(F32)


def nb_of(a: np.ndarray):
    """ggml nb[] (innermost first) of a C-ordered numpy array of ndim <= 4."""
    return list(reversed(a.strides)) + [a.nbytes] * (4 - a.ndim)


@pytest.mark.gpu
@pytest.mark.parametrize("op", ["ADD", "MUL"])
@pytest.mark.parametrize("bshape", [(3, 7, 64), (1, 1, 64), (1, 7, 64), (3, 1, 16), (1, 7, 1)])
def test_binary_broadcast(ane, built, op, bshape):
    g = Graph(built)
    A = rnd((3, 7, 64), 1)
    B = rnd(bshape, 2)
    Ad, Bd = dev(A), dev(B)
    Od = dev(np.full((3, 7, 64), np.nan, F32))
    a = g.tensor([64, 7, 3], Ad)
    b = g.tensor(list(reversed(bshape)), Bd)
    _ok(g, [g.tensor([64, 7, 3], Od, op=op, src=(a, b))])
    Bt = np.tile(B, (3 // bshape[0], 7 // bshape[1], 64 // bshape[2]))
    same(host(Od), A + Bt if op == "ADD" else A * Bt)


@pytest.mark.gpu
def test_binary_strided_and_inplace(ane, built):
    """src0 a view with padded rows, dst another padded view, then ADD in
    place into src0's own buffer (ggml_add_inplace)."""
    g = Graph(built)
    A = rnd((5, 72), 3)  # 5 rows of 64 used + 8 padding
    B = rnd((5, 64), 4)
    Ad, Bd = dev(A), dev(B)
    Od = dev(np.zeros((5, 80), F32))
    a = g.tensor([64, 5], Ad, nb=[4, 72 * 4, 72 * 4 * 5, 72 * 4 * 5])
    b = g.tensor([64, 5], Bd)
    _ok(g, [g.tensor([64, 5], Od, nb=[4, 80 * 4, 80 * 4 * 5, 80 * 4 * 5], op="MUL", src=(a, b))])
    got = host(Od)
    same(got[:, :64], A[:, :64] * B)
    assert not got[:, 64:].any()  # the gaps between dst rows are not written
    _ok(g, [g.tensor([64, 5], Ad, nb=[4, 72 * 4, 72 * 4 * 5, 72 * 4 * 5], op="ADD", src=(a, b))])
    got = host(Ad)
    same(got[:, :64], A[:, :64] + B)
    same(got[:, 64:], A[:, 64:])


@pytest.mark.gpu
@pytest.mark.parametrize("s", [0.125, 1.0 / 3.0, -7.5])
def test_scale(ane, built, s):
    g = Graph(built)
    A = rnd((5, 100), 5)
    Ad, Od = dev(A), dev(np.zeros((5, 100), F32))
    a = g.tensor([100, 5], Ad)
    _ok(g, [g.tensor([100, 5], Od, op="SCALE", src=(a,), params=[s])])
    same(host(Od), A * F32(s))
    _ok(g, [g.tensor([100, 5], Ad, op="SCALE", src=(a,), params=[s, 0.0])])  # in place, zero bias
    same(host(Ad), A * F32(s))


def rms_ref64(x, eps):
    x64 = x.astype(np.float64)
    return x64 / np.sqrt((x64 * x64).mean(axis=-1, keepdims=True) + eps)


@pytest.mark.gpu
@pytest.mark.parametrize("shape,eps", [((3, 4096), 1e-5), ((2, 5, 64), 1e-6), ((1, 1, 16), 0.0)])
def test_rms_norm(ane, oracle, built, shape, eps):
    g = Graph(built)
    X = rnd(shape, 6, 2.0)
    Xd, Od = dev(X), dev(np.zeros(shape, F32))
    ne = list(reversed(shape))
    _ok(g, [g.tensor(ne, Od, op="RMS_NORM", src=(g.tensor(ne, Xd),), params=[eps])])
    got = host(Od).reshape(-1, shape[-1])
    ones = np.ones(shape[-1], F32)
    for r, row in enumerate(X.reshape(-1, shape[-1])):
        same(got[r], oracle.rms_norm_fp32(row, ones, eps))
    np.testing.assert_allclose(got, rms_ref64(X.reshape(-1, shape[-1]), eps), rtol=2e-6, atol=1e-6)


@pytest.mark.gpu
def test_rms_norm_strided_rows_inplace(ane, oracle, built):
    """Rows of a wider buffer (a view), normalised in place."""
    g = Graph(built)
    X = rnd((6, 300), 7)  # rows of 256 used
    Xd = dev(X)
    nb = [4, 300 * 4, 300 * 4 * 3, 300 * 4 * 6]
    x = g.tensor([256, 3, 2], Xd, nb=nb)
    _ok(g, [g.tensor([256, 3, 2], Xd, nb=nb, op="RMS_NORM", src=(x,), params=[1e-5])])
    got = host(Xd)
    ones = np.ones(256, F32)
    for r in range(6):
        same(got[r, :256], oracle.rms_norm_fp32(X[r, :256], ones, 1e-5))
    same(got[:, 256:], X[:, 256:])


def softmax_oracle(oracle, pre):
    """Rows of the pre-pass values through the handler arithmetic; -inf
    entries become -1e30 (both give e = 0 there)."""
    pre = np.where(np.isneginf(pre), F32(-1e30), pre).astype(F32)
    return np.stack([oracle.softmax_fp32(r) for r in pre.reshape(-1, pre.shape[-1])]).reshape(pre.shape)


def softmax64(pre):
    p = pre.astype(np.float64)
    e = np.exp(p - p.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


@pytest.mark.gpu
@pytest.mark.parametrize("n", [256, 100, 37, 9000])
def test_soft_max_plain(ane, oracle, built, n):
    g = Graph(built)
    X = rnd((2, 3, n), 8, 3.0)
    Xd, Od = dev(X), dev(np.zeros(X.shape, F32))
    _ok(g, [g.tensor([n, 3, 2], Od, op="SOFT_MAX", src=(g.tensor([n, 3, 2], Xd),), params=[1.0, 0.0])])
    got = host(Od)
    same(got, softmax_oracle(oracle, X))
    np.testing.assert_allclose(got, softmax64(X), rtol=1.5e-3, atol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("mask_ne2", [1, 2])
def test_soft_max_scale_and_mask(ane, oracle, built, mask_ne2):
    """Attention scores [n_kv, T, heads] with ggml's causal-style mask:
    rows of the mask hold -inf past each token's position, the mask has
    more rows than tokens (padding) and is repeated over the heads."""
    g = Graph(built)
    n_kv, T, H = 80, 3, 4
    scale = 1.0 / np.sqrt(128.0)
    X = rnd((H, T, n_kv), 9, 8.0)
    M = np.zeros((mask_ne2, 8, n_kv), F32)
    for h in range(mask_ne2):
        for t in range(8):
            M[h, t, 70 + t + h:] = -np.inf
            M[h, t, :5] = -0.5 * (h + 1)
    Xd, Md, Od = dev(X), dev(M), dev(np.zeros(X.shape, F32))
    x = g.tensor([n_kv, T, H], Xd)
    m = g.tensor([n_kv, 8, mask_ne2], Md)
    _ok(g, [g.tensor([n_kv, T, H], Od, op="SOFT_MAX", src=(x, m), params=[float(scale), 0.0])])
    got = host(Od)
    Mb = np.stack([M[h % mask_ne2, :T] for h in range(H)])
    pre = (X * F32(scale)).astype(F32) + Mb
    same(got, softmax_oracle(oracle, pre))
    np.testing.assert_allclose(got, softmax64(pre), rtol=1.5e-3, atol=0)
    assert (got[np.isneginf(pre)] == 0).all()


@pytest.mark.gpu
def test_silu(ane, oracle, built):
    g = Graph(built)
    X = rnd((3, 1000), 10, 4.0)
    Xd, Od = dev(X), dev(np.zeros(X.shape, F32))
    _ok(g, [g.tensor([1000, 3], Od, op="UNARY", src=(g.tensor([1000, 3], Xd),), params=[g.silu])])
    same(host(Od).ravel(), oracle.silu_fp32(X.ravel()))


def rope64(x, pos, base):
    """ggml's normal-mode rotation in float64: pair (2i, 2i+1) of a row at
    position p turns by p * base^(-2i/n)."""
    n = x.shape[-1]
    th = pos[:, None, None] * np.power(float(base), -2.0 * np.arange(n // 2) / n)[None, None, :]
    a, b = x[..., 0::2].astype(np.float64), x[..., 1::2].astype(np.float64)
    out = np.empty(x.shape, np.float64)
    out[..., 0::2] = a * np.cos(th) - b * np.sin(th)
    out[..., 1::2] = a * np.sin(th) + b * np.cos(th)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("base", [10000.0, 500000.0])
def test_rope(ane, oracle, built, base):
    g = Graph(built)
    T, H, D = 5, 8, 128
    X = rnd((T, H, D), 11)
    P = np.array([3, 17, 4095, 0, 100], np.int32)
    Xd, Pd, Od = dev(X), dev(P), dev(np.zeros(X.shape, F32))
    x = g.tensor([D, H, T], Xd)
    pos = g.tensor([T], Pd, type_=T_I32)
    params = [0, D, 0, 0, 4096, base, 1.0, 0.0, 1.0, 32.0, 1.0]
    _ok(g, [g.tensor([D, H, T], Od, op="ROPE", src=(x, pos), params=params)])
    got = host(Od)
    for t in range(T):
        for h in range(H):
            same(got[t, h], oracle.rope_fp32(X[t, h], int(P[t]), F32(base)))
    if base == 10000.0:
        # The handler's theta^(2/dim) comes from a cubic log polynomial (off
        # by ~4e-4 at base 1e4, ~7e-2 at 5e5), so only small positions at
        # base 1e4 stay near the exact rotation; a wrong pairing, position
        # or base is off by O(|x|).
        near = P <= 100
        want = rope64(X[near], P[near].astype(np.float64), base)
        np.testing.assert_allclose(got[near], want, rtol=0, atol=0.02)


@pytest.mark.gpu
def test_rope_view_of_qkv_inplace(ane, oracle, built):
    """The k heads of a fused qkv activation ([D, 2 heads, T] at an offset,
    token rows 12 heads apart), rotated in place."""
    g = Graph(built)
    T, D = 3, 64
    QKV = rnd((T, 12, D), 12)
    P = np.array([7, 8, 9], np.int32)
    Qd, Pd = dev(QKV), dev(P)
    nb = [4, D * 4, 12 * D * 4, 12 * D * 4 * T]
    base_ptr = Qd.data_ptr() + 8 * D * 4  # heads 8 and 9
    k = g.tensor([D, 2, T], base_ptr, nb=nb)
    g.keep.append(Qd)
    pos = g.tensor([T], Pd, type_=T_I32)
    _ok(g, [g.tensor([D, 2, T], base_ptr, nb=nb, op="ROPE", src=(k, pos),
                     params=[0, D, 0, 0, 4096, 10000.0, 1.0, 0.0, 1.0])])
    got = host(Qd)
    for t in range(T):
        for h in (8, 9):
            same(got[t, h], oracle.rope_fp32(QKV[t, h], int(P[t]), F32(10000.0)))
    same(np.delete(got, [8, 9], axis=1), np.delete(QKV, [8, 9], axis=1))


@pytest.mark.gpu
@pytest.mark.parametrize("op", ["CPY", "CONT", "DUP"])
def test_copies(ane, built, op):
    g = Graph(built)
    A = rnd((7, 64), 13)
    Ad = dev(A)
    # contiguous to contiguous (a plain device copy)
    Od = dev(np.zeros(448, F32))
    _ok(g, [g.tensor([448], Od, op=op, src=(g.tensor([64, 7], Ad),))])
    same(host(Od), A.ravel())
    # a transposed view made contiguous (element order of the view)
    Td = dev(np.zeros((64, 7), F32))
    t = g.tensor([7, 64], Ad, nb=[64 * 4, 4, 64 * 7 * 4, 64 * 7 * 4])
    _ok(g, [g.tensor([7, 64], Td, op=op, src=(t,))])
    same(host(Td), A.T)
    # same shape into a strided view (a cache slot per row)
    C = np.full((7, 100), -1.0, F32)
    Cd = dev(C)
    _ok(g, [g.tensor([64, 7], Cd, nb=[4, 400, 2800, 2800], op=op, src=(g.tensor([64, 7], Ad),))])
    got = host(Cd)
    same(got[:, :64], A)
    same(got[:, 64:], C[:, 64:])
    # a transposed view into a 1-D destination (row-major order of the source)
    Fd = dev(np.zeros(448, F32))
    _ok(g, [g.tensor([448], Fd, op=op, src=(t,))])
    same(host(Fd), A.T.ravel())


@pytest.mark.gpu
def test_unsupported_nodes_fail_the_graph(ane, built):
    g = Graph(built)
    A = dev(rnd((4, 64), 14))
    a = g.tensor([64, 4], A)
    Od = dev(np.zeros((4, 64), F32))
    assert g.run([g.tensor([64, 4], Od, op="UNARY", src=(a,), params=[g.silu - 1])]) == -1
    assert g.run([g.tensor([64, 4], Od, op="RMS_NORM", src=(a,), params=[1e-5]),
                  g.tensor([64, 4], Od, op="SCALE", src=(a,), params=[2.0, 1.0])]) == -1


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 3])
def test_block_graph(ane, oracle, built, T):
    """One graph_compute over a transformer block's nodes:
        xn = RMS_NORM(x); xw = MUL(xn, norm_w)
        g = MUL_MAT(W_gate, xw); u = MUL_MAT(W_up, xw)
        h = MUL(UNARY_SILU(g), u); y = MUL_MAT(W_down, h); o = ADD(y, x)
        s = SCALE(o, 0.5); q = RESHAPE(s) [64, H/64, T]; r = ROPE(q, pos)
        CPY(r, cache view at the tokens' slots)
    against the oracle's composition (G-mode Q8_0 products, the handler
    arithmetic for norm, SiLU and RoPE, numpy fp32 for the rest)."""
    H, F, D, CTX = 256, 512, 64, 16
    g = Graph(built)
    X = rnd((T, H), 20)
    NW = rnd((H,), 21, 0.5) + F32(1.0)
    Wg = data.q8_0_weights(F, H, seed=22)
    Wu = data.q8_0_weights(F, H, seed=23)
    Wdn = data.q8_0_weights(H, F, seed=24)
    P = np.arange(5, 5 + T, dtype=np.int32)
    cache = np.full((CTX, H // D, D), -2.0, F32)
    bufs = {k: dev(v) for k, v in dict(X=X, NW=NW, Wg=Wg, Wu=Wu, Wd=Wdn, P=P, cache=cache).items()}
    scratch = {k: dev(np.full(shape, np.nan, F32)) for k, shape in
               dict(xn=(T, H), xw=(T, H), g=(T, F), u=(T, F), sg=(T, F), h=(T, F), y=(T, H), o=(T, H),
                    s=(T, H), r=(T, H)).items()}
    x = g.tensor([H, T], bufs["X"])
    nw = g.tensor([H], bufs["NW"])
    rb = lambda K: (K // 32) * 34  # noqa: E731
    wg = g.tensor([H, F], bufs["Wg"], type_=T_Q8, nb=[34, rb(H), rb(H) * F, rb(H) * F])
    wu = g.tensor([H, F], bufs["Wu"], type_=T_Q8, nb=[34, rb(H), rb(H) * F, rb(H) * F])
    wd = g.tensor([F, H], bufs["Wd"], type_=T_Q8, nb=[34, rb(F), rb(F) * H, rb(F) * H])
    xn = g.tensor([H, T], scratch["xn"], op="RMS_NORM", src=(x,), params=[1e-5])
    xw = g.tensor([H, T], scratch["xw"], op="MUL", src=(xn, nw))
    gt = g.tensor([F, T], scratch["g"], op="MUL_MAT", src=(wg, xw))
    ut = g.tensor([F, T], scratch["u"], op="MUL_MAT", src=(wu, xw))
    sg = g.tensor([F, T], scratch["sg"], op="UNARY", src=(gt,), params=[g.silu])
    ht = g.tensor([F, T], scratch["h"], op="MUL", src=(sg, ut))
    yt = g.tensor([H, T], scratch["y"], op="MUL_MAT", src=(wd, ht))
    ot = g.tensor([H, T], scratch["o"], op="ADD", src=(yt, x))
    st = g.tensor([H, T], scratch["s"], op="SCALE", src=(ot,), params=[0.5])
    q = g.tensor([D, H // D, T], scratch["s"], op="RESHAPE", src=(st,))
    pos = g.tensor([T], bufs["P"], type_=T_I32)
    rt = g.tensor([D, H // D, T], scratch["r"], op="ROPE", src=(q, pos),
                  params=[0, D, 0, 0, 4096, 500000.0, 1.0, 0.0, 1.0])
    slot = bufs["cache"].data_ptr() + int(P[0]) * H * 4
    view = g.tensor([D, H // D, T], slot, op="VIEW")
    cp = g.tensor([D, H // D, T], slot, op="CPY", src=(rt, view))
    nodes = [xn, xw, gt, ut, sg, ht, yt, ot, st, q, rt, view, cp]
    _ok(g, nodes)

    ones = np.ones(H, F32)
    xn_w = np.stack([oracle.rms_norm_fp32(X[t], ones, 1e-5) for t in range(T)])
    xw_w = xn_w * NW
    g_w = oracle.q8_0_mul_mat_g(F, H, T, xw_w, Wg)
    u_w = oracle.q8_0_mul_mat_g(F, H, T, xw_w, Wu)
    h_w = oracle.silu_fp32(g_w.ravel()).reshape(T, F) * u_w
    o_w = oracle.q8_0_mul_mat_g(H, F, T, h_w, Wdn) + X
    s_w = o_w * F32(0.5)
    r_w = np.stack([[oracle.rope_fp32(s_w[t].reshape(H // D, D)[h], int(P[t]), F32(500000.0))
                     for h in range(H // D)] for t in range(T)])
    for name, want in (("xn", xn_w), ("xw", xw_w), ("g", g_w), ("u", u_w), ("h", h_w), ("o", o_w), ("s", s_w),
                       ("r", r_w.reshape(T, H))):
        same(host(scratch[name]), want)
    want_cache = cache.copy()
    want_cache[P[0]:P[0] + T] = r_w
    same(host(bufs["cache"]), want_cache)
