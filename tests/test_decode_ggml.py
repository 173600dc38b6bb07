"""The config-5 decode through the ggml hook (ane_decode_token_ggml), on the GPU.

* Build arithmetic: the four products are GGML_OP_MUL_MAT nodes and the
  steps around them separate kernels, yet x and the KV caches come out
  bit-identical to the fused ane_decode_token, token after token -- at a
  small width, at the config-5 width, and over all 32 layers of config 5.
* Reference arithmetic: the products in R mode (opcode 0x57, what the
  reference's hook runs) and every step in the handlers' arithmetic
  (rms_norm_fp32, rope_fp32, softmax_fp32, silu_fp32): bit-identical to the
  oracle's composition of the same restated handlers, at the config-5 width
  with 2 layers, at the first positions and at the end of a 4096-position
  context.
* The fused route at the config-5 width against a float64 model on the
  oracle's products: every step but the expf-based ones is exact.
"""
import functools

import numpy as np
import pytest

from tests import data
from tests.test_decode import np_attention, np_rope

pytestmark = pytest.mark.gpu
F32 = np.float32
THETA = 500000.0


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


@functools.lru_cache(maxsize=2)
def _host_model(seed, layers, hidden, ffn, n_heads, n_kv):
    g = np.random.default_rng(seed)
    nqkv = (n_heads + 2 * n_kv) * 128
    m = []
    for l in range(layers):
        m.append({
            "w_qkv": data.q8_0_weights(nqkv, hidden, seed=seed + 100 * l + 1),
            "w_o": data.q8_0_weights(hidden, n_heads * 128, seed=seed + 100 * l + 2),
            "w_gate_up": data.q8_0_weights(2 * ffn, hidden, seed=seed + 100 * l + 3),
            "w_down": data.q8_0_weights(hidden, ffn, seed=seed + 100 * l + 4),
            "attn_norm": (1.0 + 0.1 * g.standard_normal(hidden)).astype(F32),
            "ffn_norm": (1.0 + 0.1 * g.standard_normal(hidden)).astype(F32),
        })
    return m


def host_model(seed, layers, hidden, ffn, n_heads, n_kv):
    """Seeded host weights (cached: the config-5-width models are large)."""
    return [dict(L) for L in _host_model(seed, layers, hidden, ffn, n_heads, n_kv)]


class Model:
    """Device weights, two sets of KV caches (one per route) and the layer
    arrays pointing at them."""

    def __init__(self, ane, cfg, weights, cache_init=None):
        import torch

        self.cfg = cfg
        self.keep = []
        self.layers = {}
        self.caches = {}
        for route in ("a", "b"):
            arr = (ane.DecodeLayer * cfg.n_layers)()
            cs = []
            for l in range(cfg.n_layers):
                t = weights[l] if isinstance(weights[l]["w_qkv"], torch.Tensor) else \
                    {k: dev(v) for k, v in weights[l].items()}
                if route == "a":
                    weights[l] = t
                shape = (cfg.n_kv_heads, cfg.ctx, 128)
                if cache_init is None:
                    kc = torch.zeros(shape, dtype=torch.float16, device="cuda")
                    vc = torch.zeros(shape, dtype=torch.float16, device="cuda")
                else:
                    kc, vc = (dev(c) for c in cache_init[l])
                self.keep += [t, kc, vc]
                cs.append((kc, vc))
                arr[l] = ane.DecodeLayer(*[t[k].data_ptr() for k in ("w_qkv", "w_o", "w_gate_up", "w_down",
                                                                      "attn_norm", "ffn_norm")],
                                         kc.data_ptr(), vc.data_ptr())
            self.layers[route] = arr
            self.caches[route] = cs


def oracle_ref_token(oracle, cfg, m, caches, pos, x):
    """The reference-arithmetic composition on the oracle: R-mode products,
    rms_norm_fp32, rope_fp32 on q and k, fp16 append, the reference-mode
    attention, silu_fp32(gate) * up, fp32 residual adds."""
    H, F, nh, nkv = cfg.hidden, cfg.ffn, cfg.n_heads, cfg.n_kv_heads
    nq = nh * 128
    x = np.asarray(x, F32)
    for l, L in enumerate(m):
        kc, vc = caches[l]
        xn = oracle.rms_norm_fp32(x, L["attn_norm"], cfg.eps)
        qkv = oracle.q8_0_gemv((nh + 2 * nkv) * 128, H, xn, L["w_qkv"])
        q = np.stack([oracle.rope_fp32(qkv[h * 128:(h + 1) * 128], pos, THETA) for h in range(nh)])
        for g in range(nkv):
            kc[g, pos] = oracle.rope_fp32(qkv[nq + g * 128: nq + (g + 1) * 128], pos, THETA).astype(np.float16)
            vc[g, pos] = qkv[nq + nkv * 128 + g * 128: nq + nkv * 128 + (g + 1) * 128].astype(np.float16)
        attn = oracle.attention_ref(q, kc, vc, pos + 1).reshape(-1)
        x = (x + oracle.q8_0_gemv(H, nq, attn, L["w_o"])).astype(F32)
        xn = oracle.rms_norm_fp32(x, L["ffn_norm"], cfg.eps)
        gu = oracle.q8_0_gemv(2 * F, H, xn, L["w_gate_up"]).reshape(F // 32, 2, 32)
        h = (oracle.silu_fp32(gu[:, 0].reshape(-1)) * gu[:, 1].reshape(-1)).astype(F32)
        x = (x + oracle.q8_0_gemv(H, F, h, L["w_down"])).astype(F32)
    return x


def np_build_token(oracle, cfg, m, caches, table, pos, x):
    """The fused route's arithmetic on the host: the oracle's canonical norm
    and G-mode products are exact, the attention and SiLU in float64."""
    H, F, nh, nkv = cfg.hidden, cfg.ffn, cfg.n_heads, cfg.n_kv_heads
    nq = nh * 128
    for l, L in enumerate(m):
        kc, vc = caches[l]
        xn = oracle.rms_norm_build(x, L["attn_norm"], cfg.eps)
        qkv = oracle.q8_0_mul_mat_g((nh + 2 * nkv) * 128, H, 1, xn[None, :], L["w_qkv"])[0]
        q = np_rope(qkv[:nq].reshape(nh, 128), table[pos])
        kc[:, pos] = np_rope(qkv[nq:nq + nkv * 128].reshape(nkv, 128), table[pos]).astype(np.float16)
        vc[:, pos] = qkv[nq + nkv * 128:].reshape(nkv, 128).astype(np.float16)
        attn = np_attention(q, kc, vc, pos + 1, nh, nkv).astype(F32).reshape(-1)
        x = (x + oracle.q8_0_mul_mat_g(H, nq, 1, attn[None, :], L["w_o"])[0]).astype(F32)
        xn = oracle.rms_norm_build(x, L["ffn_norm"], cfg.eps)
        gu = oracle.q8_0_mul_mat_g(2 * F, H, 1, xn[None, :], L["w_gate_up"])[0].reshape(F // 32, 2, 32)
        g, u = gu[:, 0].reshape(-1).astype(np.float64), gu[:, 1].reshape(-1).astype(np.float64)
        h = (g / (1.0 + np.exp(-g)) * u).astype(F32)
        x = (x + oracle.q8_0_mul_mat_g(H, F, 1, h[None, :], L["w_down"])[0]).astype(F32)
    return x


def run_routes(ane, model, table, xs, positions, ws_a, ws_b, backend):
    """Token by token: the fused route on caches 'a', the ggml route (build)
    on caches 'b'; returns the two x sequences."""
    import torch

    cfg = model.cfg
    xa = torch.zeros(cfg.hidden, dtype=torch.float32, device="cuda")
    xb = torch.zeros(cfg.hidden, dtype=torch.float32, device="cuda")
    outs = []
    for x0, pos in zip(xs, positions):
        xa.copy_(dev(x0))
        xb.copy_(dev(x0))
        ane.decode_token(model.cfg, model.layers["a"], table, pos, xa, ws_a)
        ane.decode_token_ggml(model.cfg, model.layers["b"], table, pos, xb, ws_b, backend, ane.ARITH_BUILD)
        outs.append((host(xa), host(xb)))
    return outs


@pytest.mark.parametrize("hidden,ffn,nh,nkv,ctx", [(512, 1024, 8, 2, 64), (4096, 14336, 32, 8, 4096)])
def test_ggml_route_build_bit_identical_to_fused(ane, hidden, ffn, nh, nkv, ctx):
    import torch

    cfg = ane.DecodeConfig(2, hidden, ffn, nh, nkv, 128, ctx, 1e-5)
    model = Model(ane, cfg, host_model(3, 2, hidden, ffn, nh, nkv))
    table = dev(ane.rope_table(ctx))
    be = ane.GgmlBackend()
    ws_a, ws_b = ane.decode_workspace(cfg), ane.decode_ggml_workspace(cfg)
    xs = data.activations(4, hidden, seed=31)
    for xa, xb in run_routes(ane, model, table, xs, [0, 1, 2, 3], ws_a, ws_b, be):
        assert np.isfinite(xa).all()
        assert xa.tobytes() == xb.tobytes()
    for l in range(2):
        for c in range(2):
            assert host(model.caches["a"][l][c]).tobytes() == host(model.caches["b"][l][c]).tobytes()
    be.close()


@pytest.mark.parametrize("positions,prefill", [([0, 1, 2], False), ([4093, 4094, 4095], True)])
def test_ggml_route_reference_arithmetic_config5_width(ane, oracle, positions, prefill):
    """hidden 4096, FFN 14336, 32/8 heads, ctx 4096, 2 layers: every bit of x
    and of the appended k and v equals the oracle's composition of the
    restated handlers, at the first positions and at the end of a context
    prefilled with random fp16 keys and values."""
    import torch

    H, F, NH, NKV, CTX = 4096, 14336, 32, 8, 4096
    cfg = ane.DecodeConfig(2, H, F, NH, NKV, 128, CTX, 1e-5)
    m = host_model(7, 2, H, F, NH, NKV)
    g = np.random.default_rng(8)
    caches = [tuple(g.standard_normal((NKV, CTX, 128)).astype(np.float16) if prefill else
                    np.zeros((NKV, CTX, 128), np.float16) for _ in range(2)) for _ in range(2)]
    model = Model(ane, cfg, host_model(7, 2, H, F, NH, NKV), cache_init=caches)
    be = ane.GgmlBackend()
    ws = ane.decode_ggml_workspace(cfg)
    xs = data.activations(len(positions), H, seed=41)
    x = torch.zeros(H, dtype=torch.float32, device="cuda")
    oracle.set_threads(0)
    try:
        for x0, pos in zip(xs, positions):
            x.copy_(dev(x0))
            ane.decode_token_ggml(cfg, model.layers["b"], None, pos, x, ws, be, ane.ARITH_REFERENCE, theta=THETA)
            want = oracle_ref_token(oracle, cfg, m, caches, pos, x0)
            got = host(x)
            assert np.isfinite(want).all()
            assert got.tobytes() == want.tobytes(), (pos, np.max(np.abs(got - want)))
            for l in range(2):
                assert host(model.caches["b"][l][0])[:, pos].tobytes() == caches[l][0][:, pos].tobytes()
                assert host(model.caches["b"][l][1])[:, pos].tobytes() == caches[l][1][:, pos].tobytes()
    finally:
        oracle.set_threads(1)
    be.close()


def test_fused_route_config5_width(ane, oracle):
    """ane_decode_token at the config-5 width (2 layers, ctx 4096) against the
    host model: the norm, the products, RoPE and the fp16 appends are exact
    (so layer 0's k and v of every token match bit for bit); only softmax
    and SiLU use expf, whose last-bit differences can move a quantized
    activation across a rounding boundary: the whole token stays within
    1e-3 relative (it measures about 1e-6 when nothing flips)."""
    import torch

    H, F, NH, NKV, CTX = 4096, 14336, 32, 8, 4096
    cfg = ane.DecodeConfig(2, H, F, NH, NKV, 128, CTX, 1e-5)
    m = host_model(9, 2, H, F, NH, NKV)
    model = Model(ane, cfg, host_model(9, 2, H, F, NH, NKV))
    table_h = ane.rope_table(CTX)
    table = dev(table_h)
    ws = ane.decode_workspace(cfg)
    caches = [(np.zeros((NKV, CTX, 128), np.float16), np.zeros((NKV, CTX, 128), np.float16)) for _ in range(2)]
    xs = data.activations(3, H, seed=51)
    x = torch.zeros(H, dtype=torch.float32, device="cuda")
    oracle.set_threads(0)
    try:
        for pos in range(3):
            x.copy_(dev(xs[pos]))
            ane.decode_token(cfg, model.layers["a"], table, pos, x, ws)
            ref = np_build_token(oracle, cfg, m, caches, table_h, pos, xs[pos])
            got = host(x).astype(np.float64)
            err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
            print(f"pos {pos}: relative L2 error {err:.3g}")
            assert err < 1e-3, (pos, err)
            assert host(model.caches["a"][0][0])[:, pos].tobytes() == caches[0][0][:, pos].tobytes()
            assert host(model.caches["a"][0][1])[:, pos].tobytes() == caches[0][1][:, pos].tobytes()
    finally:
        oracle.set_threads(1)


def test_ggml_route_32_layers_matches_fused(ane):
    """Config 5 in full (32 layers, hidden 4096, FFN 14336, ctx 4096, weights
    generated on the GPU): the ggml route's x equals the fused route's bit
    for bit at the end of a prefilled context, every value finite, and a
    second run from the same state repeats every bit."""
    import torch

    H, F, NH, NKV, CTX, NL = 4096, 14336, 32, 8, 4096, 32
    cfg = ane.DecodeConfig(NL, H, F, NH, NKV, 128, CTX, 1e-5)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(12)

    def q8(N, K):
        nb = K // 32
        W = torch.empty((N, nb, 34), dtype=torch.uint8, device="cuda")
        W[:, :, :2] = (torch.randn((N, nb), generator=gen, device="cuda") * 0.01).abs().half() \
            .view(torch.uint8).view(N, nb, 2)
        W[:, :, 2:] = torch.randint(-127, 128, (N, nb, 32), generator=gen, device="cuda",
                                    dtype=torch.int8).view(torch.uint8)
        return W.view(N, nb * 34)

    weights = [{"w_qkv": q8((NH + 2 * NKV) * 128, H), "w_o": q8(H, NH * 128), "w_gate_up": q8(2 * F, H),
                "w_down": q8(H, F), "attn_norm": 1.0 + 0.1 * torch.randn(H, generator=gen, device="cuda"),
                "ffn_norm": 1.0 + 0.1 * torch.randn(H, generator=gen, device="cuda")} for _ in range(NL)]
    kv0 = [(torch.randn((NKV, CTX, 128), generator=gen, device="cuda").half(),
            torch.randn((NKV, CTX, 128), generator=gen, device="cuda").half()) for _ in range(NL)]
    model = Model(ane, cfg, weights)
    table = dev(ane.rope_table(CTX))
    be = ane.GgmlBackend()
    ws_a, ws_b = ane.decode_workspace(cfg), ane.decode_ggml_workspace(cfg)
    x0 = torch.randn(H, generator=gen, device="cuda").cpu().numpy()
    results = []
    for rep in range(2):
        for route in ("a", "b"):
            for l in range(NL):
                model.caches[route][l][0].copy_(kv0[l][0])
                model.caches[route][l][1].copy_(kv0[l][1])
        (xa, xb), = run_routes(ane, model, table, [x0], [CTX - 1], ws_a, ws_b, be)
        assert np.isfinite(xa).all()
        assert xa.tobytes() == xb.tobytes()
        results.append(xa)
    assert results[0].tobytes() == results[1].tobytes()
    be.close()
