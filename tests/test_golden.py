"""Committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py).

CPU tests pin the oracle to the vectors and to the reference KATs' closed
forms.  GPU tests run the HIP path through the C ABI on the same inputs and
must reproduce every stored output bit for bit.
"""
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
F32 = np.float32


def fx(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def same_bits(a, b):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype
    assert a.tobytes() == b.tobytes()


def test_fixture_set_complete():
    names = sorted(p.stem for p in GOLDEN.glob("*.npz"))
    assert names == sorted(["quantize_kat", "igemm_kat", "q8_0_get_rows_kat_32", "q8_0_get_rows_kat_64",
                            "dense_fused_mnist", "dense_u8s8_small", "channelwise_small", "q8_0_small",
                            "cblas_igemm_kat"])
    for n in names:
        assert str(fx(n)["source"])  # every fixture names its origin


# ------------------------------------------------------------------ CPU: oracle
def test_oracle_quantize_kat(oracle):
    f = fx("quantize_kat")
    q, s = oracle.quantize(f["x"])
    same_bits(q, f["q"])
    same_bits(np.array([s], F32), f["scale"])
    # the reference test's bound and closed forms: amax = 12.8 -> +-127, sign symmetry
    assert np.abs(f["q"].astype(F32) * f["scale"][0] - f["x"]).max() < 1.5 * f["scale"][0]
    assert f["q"][0] == -127 and f["q"][128] == 0


def test_oracle_igemm_kat(oracle):
    f = fx("igemm_kat")
    same_bits(oracle.gemm_s8_i32(f["A"], f["B"], 16, 32, 64), f["acc"])
    same_bits(f["acc"], (f["A"].astype(np.int64) @ f["B"].astype(np.int64)).astype(np.int32))
    same_bits(oracle.pack_b(f["B"], 64, 32), f["Bp"])
    C = oracle.dense_i8(16, 32, 64, F32(1), F32(1), 0, f["A"], f["Bp"], np.zeros(32, F32))
    same_bits(C, f["C"])


def test_oracle_cblas_igemm_kat(oracle):
    """Opcode 0x61 on the reference KAT: the stored C equals the test's own
    expectation (float)sum * alpha, and alpha 0.5 halves alpha 1 exactly."""
    f = fx("cblas_igemm_kat")
    A, B = f["A"], f["B"]
    ref = (A.reshape(16, 64).astype(np.int64) @ B.reshape(64, 32).astype(np.int64)).astype(F32)
    same_bits(f["C_alpha1"], ref)
    same_bits(f["C_alpha05"], (ref * F32(0.5)).astype(F32))
    z = np.zeros((16, 32), F32)
    same_bits(oracle.cblas_igemm(0, 0, 16, 32, 64, 64, 32, 32, 1.0, 0.0, A, B, z), f["C_alpha1"])
    same_bits(oracle.cblas_igemm(0, 0, 16, 32, 64, 64, 32, 32, 0.5, 0.0, A, B, z), f["C_alpha05"])
    for name, variant, Bx in (("ugemm", 1, f["Bu"]), ("usgemm", 2, f["Bs"])):
        same_bits(oracle.cblas_igemm(variant, 2, 21, 37, 200, 203, 205, 40, -1.25, 0.0, f["Au"], Bx, f["C2"]),
                  f[f"C_{name}"])


@pytest.mark.parametrize("dim", [32, 64])
def test_oracle_q8_0_get_rows_kat(oracle, dim):
    f = fx(f"q8_0_get_rows_kat_{dim}")
    W, Y = f["W"], f["Y"]
    d = W.reshape(4, dim // 32, 34)[:, :, :2].copy().view(np.float16).reshape(4, dim // 32).astype(F32)
    qs = W.reshape(4, dim // 32, 34)[:, :, 2:].view(np.int8).astype(F32)
    same_bits(Y.T, (qs * d[:, :, None]).reshape(4, dim).astype(F32))
    for i in (0, dim // 2 + 3, dim - 1):
        x = np.zeros(dim, F32)
        x[i] = 1
        same_bits(oracle.q8_0_gemv(4, dim, x, W), Y[i])


def test_oracle_dense_fused_mnist(oracle):
    f = fx("dense_fused_mnist")
    x, w1, w2 = (f[k].astype(F32) for k in ("x", "w1", "w2"))
    C1 = oracle.dense_fused_i8(16, 128, 784, F32(1), True, x, w1)
    same_bits(C1, f["C1"])
    same_bits(oracle.dense_fused_i8(16, 10, 128, F32(1), False, C1, w2), f["C2"])


def test_oracle_dense_u8s8(oracle):
    f = fx("dense_u8s8_small")
    C = oracle.dense_i8(20, 40, 96, f["sa"][0], f["sb"][0], 1, f["A"], f["Bp"], f["bias"], unsigned_a=True)
    same_bits(C, f["C"])


def test_oracle_channelwise(oracle):
    f = fx("channelwise_small")
    q, s = oracle.channelwise(f["x"], 5, 37)
    same_bits(q.reshape(5, 48), f["q"])
    same_bits(s, f["scales"])


def test_oracle_q8_0_small(oracle):
    f = fx("q8_0_small")
    same_bits(oracle.q8_0_gemv(24, 256, f["x"][0], f["W"]), f["y_r"])
    same_bits(oracle.q8_0_mul_mat_g(24, 256, 3, f["x"], f["W"]), f["y_g"])


# ------------------------------------------------------------------ GPU: HIP path
def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.gpu
def test_gpu_quantize_kat(ane):
    import torch

    f = fx("quantize_kat")
    q = torch.zeros(256, dtype=torch.int8, device="cuda")
    s = torch.zeros(1, dtype=torch.float32, device="cuda")
    ane.stream_exec(ane.rec_quantize(256, dev(f["x"]), q, s))
    same_bits(host(q), f["q"])
    same_bits(host(s), f["scale"])


@pytest.mark.gpu
def test_gpu_cblas_igemm_kat(ane):
    """The reference KAT through stream_exec records 0x61 (alpha 1 and 0.5),
    and the ugemm / usgemm fixture through 0x62 / 0x63."""
    import torch

    f = fx("cblas_igemm_kat")
    A, B = dev(f["A"]), dev(f["B"])
    C1 = torch.full((16, 32), 7.0, dtype=torch.float32, device="cuda")
    C05 = torch.full((16, 32), 7.0, dtype=torch.float32, device="cuda")
    ane.stream_exec([ane.rec_cblas_igemm("igemm", 0, 16, 32, 64, 64, 32, 32, 1.0, 0.0, A, B, C1),
                     ane.rec_cblas_igemm("igemm", 0, 16, 32, 64, 64, 32, 32, 0.5, 0.0, A, B, C05)])
    same_bits(host(C1), f["C_alpha1"])
    same_bits(host(C05), f["C_alpha05"])
    for kind, Bx in (("ugemm", f["Bu"]), ("usgemm", f["Bs"])):
        C = dev(f["C2"])
        ane.stream_exec(ane.rec_cblas_igemm(kind, 2, 21, 37, 200, 203, 205, 40, -1.25, 0.0, dev(f["Au"]), dev(Bx), C))
        same_bits(host(C), f[f"C_{kind}"])


@pytest.mark.gpu
def test_gpu_igemm_kat(ane):
    import torch

    f = fx("igemm_kat")
    acc = torch.zeros((16, 32), dtype=torch.int32, device="cuda")
    ane.gemm_s8_i32(dev(f["A"]), dev(np.ascontiguousarray(f["B"].T)), acc, 16, 32, 64)
    same_bits(host(acc), f["acc"])
    Bp = torch.zeros(f["Bp"].size, dtype=torch.int8, device="cuda")
    ane.stream_exec(ane.rec_pack_b(64, 32, dev(f["B"]), Bp))
    same_bits(host(Bp), f["Bp"])
    C = torch.zeros((16, 32), dtype=torch.float32, device="cuda")
    bias = torch.zeros(32, dtype=torch.float32, device="cuda")
    ane.stream_exec(ane.rec_dense_i8(16, 32, 64, 1.0, 1.0, False, dev(f["A"]), Bp, bias, C))
    same_bits(host(C), f["C"])


@pytest.mark.gpu
@pytest.mark.parametrize("dim", [32, 64])
def test_gpu_q8_0_get_rows_kat(ane, dim):
    import torch

    f = fx(f"q8_0_get_rows_kat_{dim}")
    W = dev(f["W"])
    eye = dev(np.eye(dim, dtype=F32))
    Y = torch.zeros((dim, 4), dtype=torch.float32, device="cuda")
    ane.stream_exec([ane.rec_q8_0_gemv(4, dim, eye[i], W, Y[i]) for i in range(dim)])
    same_bits(host(Y), f["Y"])


@pytest.mark.gpu
def test_gpu_dense_fused_mnist(ane):
    import torch

    f = fx("dense_fused_mnist")
    x, w1, w2 = (dev(f[k].astype(F32)) for k in ("x", "w1", "w2"))
    C1 = torch.zeros((16, 128), dtype=torch.float32, device="cuda")
    C2 = torch.zeros((16, 10), dtype=torch.float32, device="cuda")
    ane.stream_exec([ane.rec_dense_fused_i8(16, 128, 784, 1.0, True, x, w1, C1),
                     ane.rec_dense_fused_i8(16, 10, 128, 1.0, False, C1, w2, C2)])
    same_bits(host(C1), f["C1"])
    same_bits(host(C2), f["C2"])


@pytest.mark.gpu
def test_gpu_dense_u8s8(ane):
    import torch

    f = fx("dense_u8s8_small")
    C = torch.zeros((32, 40), dtype=torch.float32, device="cuda")
    ane.stream_exec(ane.rec_dense_i8(20, 40, 96, float(f["sa"][0]), float(f["sb"][0]), True, dev(f["A"]),
                                     dev(f["Bp"]), dev(f["bias"]), C, unsigned_a=True))
    same_bits(host(C), f["C"])


@pytest.mark.gpu
def test_gpu_channelwise(ane):
    import torch

    f = fx("channelwise_small")
    q = torch.zeros((5, 48), dtype=torch.int8, device="cuda")
    s = torch.zeros(5, dtype=torch.float32, device="cuda")
    ane.stream_exec(ane.rec_channelwise(5, 37, dev(f["x"]), q, s))
    same_bits(host(q), f["q"])
    same_bits(host(s), f["scales"])


@pytest.mark.gpu
def test_gpu_q8_0_small(ane):
    import torch

    f = fx("q8_0_small")
    W, x = dev(f["W"]), dev(f["x"])
    yr = torch.zeros(24, dtype=torch.float32, device="cuda")
    ane.stream_exec(ane.rec_q8_0_gemv(24, 256, x[0], W, yr))
    same_bits(host(yr), f["y_r"])
    yg = torch.zeros((3, 24), dtype=torch.float32, device="cuda")
    ane.q8_0_mul_mat(24, 256, 3, x, W, yg)
    same_bits(host(yg), f["y_g"])
