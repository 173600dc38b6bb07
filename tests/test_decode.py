"""The decode step (include/ane_decode.h, ane_amd/csrc/decode.hip and the
fused variants of the streaming Q8_0 kernel).

Bit-exact against numpy + the oracle: the fused RMSNorm / residual matvec
(fp32 ops and the G-mode definition), RoPE and the fp16 KV append.
Tolerance against float64 references (the GPU uses expf): attention
(rtol 2e-5, atol 1e-6), SiLU * up (rtol 1e-6), and a 2-layer model over
several tokens (relative L2 error of the residual stream < 1e-3: a
last-ulp difference after expf can move one activation across an int8
rounding boundary of the next layer's quantizer).
"""
import ctypes
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

import ane_amd
from tests import data

ROOT = Path(__file__).resolve().parents[1]
F32 = np.float32


# ------------------------------------------------------------------ references
def np_rmsnorm(x, w, eps):
    ss = np.sum(np.asarray(x, np.float64) ** 2)
    ms = np.float32(ss / x.size)
    inv = np.float32(1.0) / np.sqrt(np.float32(ms + np.float32(eps)))
    return ((np.asarray(x, F32) * inv).astype(F32) * np.asarray(w, F32)).astype(F32)


def np_rope(v, cs):
    """v: [heads][128] fp32; cs: [64][2] fp32; adjacent pairs, fp32 ops."""
    a, b = v[:, 0::2], v[:, 1::2]
    c, s = cs[:, 0], cs[:, 1]
    out = np.empty_like(v)
    out[:, 0::2] = ((a * c).astype(F32) - (b * s).astype(F32)).astype(F32)
    out[:, 1::2] = ((a * s).astype(F32) + (b * c).astype(F32)).astype(F32)
    return out


def np_attention(q, kc, vc, length, n_heads, n_kv):
    """q [n_heads][128] fp32, caches fp16 [n_kv][ctx][128] -> fp64 softmax attention."""
    G = n_heads // n_kv
    out = np.zeros((n_heads, 128))
    for h in range(n_heads):
        g = h // G
        k = kc[g, :length].astype(np.float64)
        v = vc[g, :length].astype(np.float64)
        s = k @ q[h].astype(np.float64) / np.sqrt(128.0)
        p = np.exp(s - s.max())
        out[h] = (p @ v) / p.sum()
    return out


def np_silu_mul(gu, n):
    g = gu[:n].astype(np.float64)
    return g / (1.0 + np.exp(-g)) * gu[n:2 * n].astype(np.float64)


# ------------------------------------------------------------------ CPU
def test_struct_layouts_match_c(tmp_path):
    gcc = shutil.which("gcc")
    if not gcc:
        pytest.skip("gcc not available")
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "ane_decode.h"\n'
        "int main(void) { printf(\"%zu %zu %zu %zu\\n\", sizeof(struct ane_decode_config),"
        " offsetof(struct ane_decode_config, eps), sizeof(struct ane_decode_layer),"
        " offsetof(struct ane_decode_layer, v_cache)); return 0; }\n")
    exe = tmp_path / "layout"
    subprocess.run([gcc, "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    C, L = ane_amd.DecodeConfig, ane_amd.DecodeLayer
    assert got == [ctypes.sizeof(C), C.eps.offset, ctypes.sizeof(L), L.v_cache.offset]


def test_workspace_sizes():
    L = ane_amd.lib()
    cfg = ane_amd.DecodeConfig(32, 4096, 14336, 32, 8, 128, 4096, 1e-5)
    assert L.ane_decode_workspace_size(ctypes.byref(cfg)) >= 4 * (6144 + 4096 + 2 * 14336 + 14336)
    assert L.ane_hip_attention_workspace_size(ctypes.byref(cfg)) >= 32 * 32 * 128 * 4
    bad = ane_amd.DecodeConfig(32, 4096, 14336, 32, 8, 64, 4096, 1e-5)  # head_dim 64 unsupported
    assert L.ane_decode_workspace_size(ctypes.byref(bad)) == 0


def test_decode_refuses_unsupported_configs_before_launching():
    """Shapes the products cannot take (ffn not a multiple of 256) and
    misaligned weights are refused up front: nothing is launched, so x and
    the caches (here fake addresses that are never touched) stay as they
    were.  No GPU is needed to reach these checks."""
    L = ane_amd.lib()
    x = (ctypes.c_float * 4096)(*([1.5] * 4096))
    ws = ctypes.create_string_buffer(1 << 16)
    table = ctypes.c_void_p(0x1000)
    for cfg in (ane_amd.DecodeConfig(2, 4096, 14336 + 32, 32, 8, 128, 4096, 1e-5),
                ane_amd.DecodeConfig(2, 4096 + 32, 14336, 32, 8, 128, 4096, 1e-5)):
        layers = (ane_amd.DecodeLayer * 2)(*[ane_amd.DecodeLayer(*([0x10000] * 8)) for _ in range(2)])
        assert L.ane_decode_token(ctypes.byref(cfg), layers, table, 0, x, ws, len(ws), None) == 1
        assert L.ane_decode_workspace_size(ctypes.byref(cfg)) == 0
    cfg = ane_amd.DecodeConfig(2, 4096, 14336, 32, 8, 128, 4096, 1e-5)
    need = L.ane_decode_workspace_size(ctypes.byref(cfg))
    big = ctypes.create_string_buffer(need + 256)
    base = (ctypes.addressof(big) + 255) & ~255
    layers = (ane_amd.DecodeLayer * 2)(ane_amd.DecodeLayer(*([0x10000] * 8)),
                                       ane_amd.DecodeLayer(0x10008, *([0x10000] * 7)))  # layer 1's w_qkv misaligned
    assert L.ane_decode_token(ctypes.byref(cfg), layers, table, 0, x, base, need, None) == 1
    assert list(x)[:4] == [1.5] * 4


def test_rms_norm_refuses_sizes_before_launching():
    """The standalone norm keeps K/32 fp64 block sums in LDS: K past 2^19,
    or not a multiple of 32, is refused before any launch (the fake
    addresses are never touched, so no GPU is needed)."""
    L = ane_amd.lib()
    p = ctypes.c_void_p(0x10000)
    for K in ((1 << 19) + 32, 1 << 20, 100):
        assert L.ane_hip_rms_norm(K, p, p, ctypes.c_float(1e-5), p, None) == 1


# ------------------------------------------------------------------ GPU
def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("N,K,norm,resid", [(6144, 4096, True, False), (4096, 4096, False, True),
                                            (4096, 14336, False, True), (28672, 4096, True, False),
                                            (512, 1024, True, True), (300, 256, False, False),
                                            # split-K: a last workgroup with a 2-row unit and an empty
                                            # slot; 8 items per wave; 4 items per wave
                                            (4098, 2048, True, True), (4100, 16384, False, True),
                                            (1030, 8192, True, False)])
def test_matvec_fused_exact(ane, oracle, N, K, norm, resid):
    import torch

    W = data.q8_0_weights(N, K, seed=N + K)
    x = data.activations(1, K, seed=7)[0] * F32(3.0)
    w = (1.0 + 0.1 * data.activations(1, K, seed=8)[0]).astype(F32)
    r = data.activations(1, N, seed=9)[0]
    eps = F32(1e-5)
    xin = np_rmsnorm(x, w, eps) if norm else x
    oracle.set_threads(0)
    try:
        ref = oracle.q8_0_mul_mat_g(N, K, 1, xin, W)[0]
    finally:
        oracle.set_threads(1)
    if resid:
        ref = (ref + r).astype(F32)
    y = dev(r) if resid else torch.zeros(N, dtype=torch.float32, device="cuda")
    ane.q8_0_matvec_fused(N, K, dev(x), dev(W), y, norm_w=dev(w) if norm else None, eps=float(eps),
                          residual=y if resid else None)
    assert host(y).tobytes() == ref.tobytes()


@pytest.mark.gpu
def test_rope_kv_append_exact(ane):
    import torch

    cfg = ane.DecodeConfig(1, 1024, 2048, 8, 2, 128, 16, 1e-5)
    table = ane.rope_table(16)
    qkv = data.activations(1, (8 + 4) * 128, seed=3)[0]
    kc = torch.zeros((2, 16, 128), dtype=torch.float16, device="cuda")
    vc = torch.zeros((2, 16, 128), dtype=torch.float16, device="cuda")
    qd = dev(qkv)
    ane.rope_kv_append(cfg, qd, dev(table), 5, kc, vc)
    q_ref = np_rope(qkv[:1024].reshape(8, 128), table[5])
    k_ref = np_rope(qkv[1024:1280].reshape(2, 128), table[5]).astype(np.float16)
    v_ref = qkv[1280:].reshape(2, 128).astype(np.float16)
    got = host(qd)
    assert got[:1024].tobytes() == q_ref.reshape(-1).tobytes()
    assert got[1024:].tobytes() == qkv[1024:].tobytes()  # k and v stay unrotated in qkv
    kh, vh = host(kc), host(vc)
    assert kh[:, 5].tobytes() == k_ref.tobytes() and vh[:, 5].tobytes() == v_ref.tobytes()
    assert not kh[:, :5].any() and not kh[:, 6:].any()


@pytest.mark.gpu
@pytest.mark.parametrize("length,ctx", [(1, 4096), (100, 4096), (128, 4096), (129, 4096), (1000, 4096),
                                        (4096, 4096), (5000, 8192), (8192, 8192)])
def test_attention_decode(ane, length, ctx):
    """Against a float64 softmax; contexts past 64 chunks take the merge's second batch."""
    import torch

    cfg = ane.DecodeConfig(1, 4096, 14336, 32, 8, 128, ctx, 1e-5)
    g = np.random.default_rng(length)
    kc = g.standard_normal((8, ctx, 128)).astype(np.float16)
    vc = g.standard_normal((8, ctx, 128)).astype(np.float16)
    q = (g.standard_normal((32, 128)) * 2.0).astype(F32)
    out = torch.zeros(32 * 128, dtype=torch.float32, device="cuda")
    ws = torch.zeros(ane.lib().ane_hip_attention_workspace_size(ctypes.byref(cfg)), dtype=torch.uint8, device="cuda")
    qd, kd, vd = dev(q), dev(kc), dev(vc)
    ane.attention_decode(cfg, qd, kd, vd, length, out, workspace=ws)
    ref = np_attention(q, kc, vc, length, 32, 8)
    first = host(out).reshape(32, 128)
    np.testing.assert_allclose(first, ref, rtol=2e-5, atol=1e-6)
    out.zero_()
    ane.attention_decode(cfg, qd, kd, vd, length, out, workspace=ws)  # the same workspace again
    assert host(out).reshape(32, 128).tobytes() == first.tobytes()


@pytest.mark.gpu
def test_silu_mul(ane):
    import torch

    n = 14336
    gu = (data.activations(1, 2 * n, seed=4)[0] * 4.0).astype(F32)
    h = torch.zeros(n, dtype=torch.float32, device="cuda")
    ane.silu_mul(n, dev(gu), h)
    np.testing.assert_allclose(host(h), np_silu_mul(gu, n), rtol=1e-6, atol=1e-30)


def small_model(seed=0, layers=2, hidden=512, ffn=1024, n_heads=8, n_kv=2, ctx=64):
    g = np.random.default_rng(seed)
    nqkv = (n_heads + 2 * n_kv) * 128
    m = []
    for l in range(layers):
        m.append({
            "w_qkv": data.q8_0_weights(nqkv, hidden, seed=100 * l + 1),
            "w_o": data.q8_0_weights(hidden, n_heads * 128, seed=100 * l + 2),
            "w_gate_up": data.q8_0_weights(2 * ffn, hidden, seed=100 * l + 3),
            "w_down": data.q8_0_weights(hidden, ffn, seed=100 * l + 4),
            "attn_norm": (1.0 + 0.1 * g.standard_normal(hidden)).astype(F32),
            "ffn_norm": (1.0 + 0.1 * g.standard_normal(hidden)).astype(F32),
        })
    return m


def np_decode_token(oracle, cfg, m, caches, table, pos, x):
    H, F, nh, nkv = cfg.hidden, cfg.ffn, cfg.n_heads, cfg.n_kv_heads
    nq = nh * 128
    for l, L in enumerate(m):
        kc, vc = caches[l]
        xn = np_rmsnorm(x, L["attn_norm"], cfg.eps)
        qkv = oracle.q8_0_mul_mat_g((nh + 2 * nkv) * 128, H, 1, xn, L["w_qkv"])[0]
        q = np_rope(qkv[:nq].reshape(nh, 128), table[pos])
        kc[:, pos] = np_rope(qkv[nq:nq + nkv * 128].reshape(nkv, 128), table[pos]).astype(np.float16)
        vc[:, pos] = qkv[nq + nkv * 128:].reshape(nkv, 128).astype(np.float16)
        attn = np_attention(q, kc, vc, pos + 1, nh, nkv).astype(F32).reshape(-1)
        x = (x + oracle.q8_0_mul_mat_g(H, nq, 1, attn, L["w_o"])[0]).astype(F32)
        xn = np_rmsnorm(x, L["ffn_norm"], cfg.eps)
        gu = oracle.q8_0_mul_mat_g(2 * F, H, 1, xn, L["w_gate_up"])[0]  # gate/up in 32-row groups
        gu = gu.reshape(F // 32, 2, 32).transpose(1, 0, 2).reshape(-1)
        h = np_silu_mul(gu, F).astype(F32)
        x = (x + oracle.q8_0_mul_mat_g(H, F, 1, h, L["w_down"])[0]).astype(F32)
    return x


@pytest.mark.gpu
def test_decode_tokens_small_model(ane, oracle):
    import torch

    cfg = ane.DecodeConfig(2, 512, 1024, 8, 2, 128, 64, 1e-5)
    m = small_model()
    table = ane.rope_table(64)
    keep = []
    layers = (ane.DecodeLayer * cfg.n_layers)()
    dev_caches = []
    for l, L in enumerate(m):
        t = {k: dev(v) for k, v in L.items()}
        kc = torch.zeros((2, 64, 128), dtype=torch.float16, device="cuda")
        vc = torch.zeros((2, 64, 128), dtype=torch.float16, device="cuda")
        keep += [t, kc, vc]
        dev_caches.append((kc, vc))
        layers[l] = ane.DecodeLayer(*[t[k].data_ptr() for k in ("w_qkv", "w_o", "w_gate_up", "w_down",
                                                                  "attn_norm", "ffn_norm")],
                                    kc.data_ptr(), vc.data_ptr())
    ws = torch.empty(ane.lib().ane_decode_workspace_size(ctypes.byref(cfg)), dtype=torch.uint8, device="cuda")
    ws.fill_(0xAB)  # no initialisation is needed
    x0 = data.activations(5, 512, seed=21).astype(F32)
    xd = torch.zeros(512, dtype=torch.float32, device="cuda")
    tab = dev(table)
    np_caches = [(np.zeros((2, 64, 128), np.float16), np.zeros((2, 64, 128), np.float16)) for _ in m]
    for pos in range(5):
        xd.copy_(dev(x0[pos]))
        ane.decode_token(cfg, layers, tab, pos, xd, ws)
        ref = np_decode_token(oracle, cfg, m, np_caches, table, pos, x0[pos])
        got = host(xd)
        err = np.linalg.norm(got.astype(np.float64) - ref) / np.linalg.norm(ref)
        assert err < 1e-3, (pos, err)
        if pos == 0:  # first layer, first token: every step before attention is exact
            assert host(dev_caches[0][0])[:, 0].tobytes() == np_caches[0][0][:, 0].tobytes()


@pytest.mark.gpu
@pytest.mark.parametrize("pos", [0, 5, 127, 128, 300])
def test_attention_rope_fused_matches_separate(ane, oracle, pos):
    """RoPE + append inside the attention kernel == rope_kv_append then attention,
    bit for bit; non-finite garbage at and past pos in the cache is never used;
    the Q8 form of the output is the oracle's quantization of it."""
    import torch

    cfg = ane.DecodeConfig(1, 4096, 14336, 32, 8, 128, 512, 1e-5)
    table = dev(ane.rope_table(512))
    g = np.random.default_rng(pos)
    qkv = (g.standard_normal(48 * 128) * 2).astype(F32)
    kc = g.standard_normal((8, 512, 128)).astype(np.float16)
    vc = g.standard_normal((8, 512, 128)).astype(np.float16)
    kc[:, pos:] = np.inf
    vc[:, pos:] = np.nan
    k1, v1, k2, v2 = dev(kc), dev(vc), dev(kc), dev(vc)
    q1 = dev(qkv)
    out1 = torch.zeros(4096, dtype=torch.float32, device="cuda")
    out2 = torch.zeros(4096, dtype=torch.float32, device="cuda")
    ane.rope_kv_append(cfg, q1, table, pos, k1, v1)
    ane.attention_decode(cfg, q1, k1, v1, pos + 1, out1)
    q8 = torch.full((ane.q8_act_bytes(4096),), 0x55, dtype=torch.uint8, device="cuda")
    ane.attention_decode_rope(cfg, dev(qkv), table, pos, k2, v2, out2, out_q8=q8)
    o1, o2 = host(out1), host(out2)
    assert np.isfinite(o2).all()
    assert o1.tobytes() == o2.tobytes()
    qx, dx = oracle.q8_0_quantize_x(4096, o2)
    assert host(q8).tobytes() == qx.tobytes() + dx.tobytes()
    assert host(k1)[:, :pos + 1].tobytes() == host(k2)[:, :pos + 1].tobytes()
    assert host(v1)[:, :pos + 1].tobytes() == host(v2)[:, :pos + 1].tobytes()


@pytest.mark.gpu
@pytest.mark.parametrize("resid", [False, True])
def test_matvec_silu_matches_separate(ane, resid):
    import torch

    N, F = 4096, 14336
    W = dev(data.q8_0_weights(N, F, seed=41))
    gu = dev((data.activations(1, 2 * F, seed=42)[0] * 3).astype(F32))
    r = data.activations(1, N, seed=43)[0]
    h = torch.zeros(F, dtype=torch.float32, device="cuda")
    y1 = dev(r) if resid else torch.zeros(N, dtype=torch.float32, device="cuda")
    y2 = dev(r) if resid else torch.zeros(N, dtype=torch.float32, device="cuda")
    ane.silu_mul(F, gu, h)
    ane.q8_0_matvec_fused(N, F, h, W, y1, residual=y1 if resid else None)
    ane.q8_0_matvec_silu(N, F, gu, W, y2, residual=y2 if resid else None)
    assert host(y1).tobytes() == host(y2).tobytes()


@pytest.mark.gpu
@pytest.mark.parametrize("n", [14336, 96, 8224])
def test_silu_mul_quant_exact(ane, oracle, n):
    """silu_mul_quant == the oracle's Q8 activation quantization of silu_mul's output."""
    import torch

    gu = dev((data.activations(1, 2 * n, seed=n)[0] * 3).astype(F32))
    gu_h = host(gu)
    gu_h[5] = 0.0
    gu_h[n + 37: n + 69] = 0.0  # an all-zero block (scale 1)
    gu = dev(gu_h)
    h = torch.zeros(n, dtype=torch.float32, device="cuda")
    xq = torch.full((ane.q8_act_bytes(n),), 0x55, dtype=torch.uint8, device="cuda")
    ane.silu_mul(n, gu, h)
    ane.silu_mul_quant(n, gu, xq)
    qx, dx = oracle.q8_0_quantize_x(n, host(h))
    assert host(xq).tobytes() == qx.tobytes() + dx.tobytes()


@pytest.mark.gpu
@pytest.mark.parametrize("N,K,resid", [(4096, 14336, True), (4096, 4096, True), (28672, 4096, False),
                                       (301, 256, True), (6, 1024, False)])
def test_matvec_q8_exact(ane, oracle, N, K, resid):
    """A pre-quantized activation gives the oracle's G-mode result bit for bit."""
    import torch

    W = data.q8_0_weights(N, K, seed=N + 3 * K)
    x = data.activations(1, K, seed=11)[0] * F32(2.5)
    qx, dx = oracle.q8_0_quantize_x(K, x)
    xq = dev(np.frombuffer(qx.tobytes() + dx.tobytes(), np.uint8).copy())
    r = data.activations(1, N, seed=12)[0]
    oracle.set_threads(0)
    try:
        ref = oracle.q8_0_mul_mat_g(N, K, 1, x, W)[0]
    finally:
        oracle.set_threads(1)
    if resid:
        ref = (ref + r).astype(F32)
    y = dev(r) if resid else torch.zeros(N, dtype=torch.float32, device="cuda")
    ane.q8_0_matvec_q8(N, K, xq, dev(W), y, residual=y if resid else None)
    assert host(y).tobytes() == ref.tobytes()


@pytest.mark.gpu
@pytest.mark.parametrize("F,K", [(14336, 4096), (1024, 512), (96, 256)])
def test_gate_up_silu_quant_matches_separate(ane, F, K):
    """The fused gate|up product == the norm-fused product, de-interleaved, then
    silu_mul_quant, bit for bit (and the interleaving helper round-trips)."""
    import torch

    Wg, Wu = data.q8_0_weights(F, K, seed=F + 1), data.q8_0_weights(F, K, seed=F + 2)
    W = ane.interleave_gate_up(Wg, Wu)
    assert (W[32:64] == Wu[:32]).all() and (W[64:96] == Wg[32:64]).all()
    x = data.activations(1, K, seed=5)[0] * F32(2.0)
    w = (1.0 + 0.1 * data.activations(1, K, seed=6)[0]).astype(F32)
    xd, wd, Wd = dev(x), dev(w), dev(W)
    gu = torch.zeros(2 * F, dtype=torch.float32, device="cuda")
    ane.q8_0_matvec_fused(2 * F, K, xd, Wd, gu, norm_w=wd, eps=1e-5)
    gu2 = gu.view(F // 32, 2, 32).transpose(0, 1).reshape(-1).contiguous()
    ref = torch.full((ane.q8_act_bytes(F),), 0x55, dtype=torch.uint8, device="cuda")
    ane.silu_mul_quant(F, gu2, ref)
    got = torch.full((ane.q8_act_bytes(F),), 0x33, dtype=torch.uint8, device="cuda")
    ane.q8_0_gate_up_silu_quant(F, K, xd, wd, Wd, got, eps=1e-5)
    assert host(got).tobytes() == host(ref).tobytes()
