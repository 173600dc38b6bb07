"""The ggml MUL_MAT hook (include/ggml-ane-hip.h, ane_amd/csrc/ggml_backend.hip).

CPU: the ctypes mirror of struct ane_ggml_tensor against the C layout
(gcc), and supports_op decisions (pure host logic, no HIP call).
GPU: every token (ne11), broadcast batches (ne12/ne13 over ne02/ne03),
strided activation and output rows, R and G arithmetic, and a two-node
graph, all bit-identical to the oracle applied per batch.
"""
import ctypes
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

import ane_amd
from ane_amd import GgmlOp, GgmlTensor, GgmlType, ggml_tensor
from tests import data

ROOT = Path(__file__).resolve().parents[1]
F32 = np.float32


def mul_mat_node(N, K, T, B2=1, B3=1, A2=1, A3=1, nb1=None, nb_dst1=None, q4=False):
    """A MUL_MAT node with null data pointers (layout only)."""
    a = ggml_tensor(GgmlType.Q4_0 if q4 else GgmlType.Q8_0, [K, N, A2, A3])
    xs = nb1 or 4 * K
    b = ggml_tensor(GgmlType.F32, [K, T, B2, B3], nb=[4, xs, xs * T, xs * T * B2])
    ys = nb_dst1 or 4 * N
    d = ggml_tensor(GgmlType.F32, [N, T, B2, B3], nb=[4, ys, ys * T, ys * T * B2], op=GgmlOp.MUL_MAT,
                    src=(a, b))
    return a, b, d


def test_struct_layout_matches_c(tmp_path):
    gcc = shutil.which("gcc")
    if not gcc:
        pytest.skip("gcc not available")
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "ggml-ane-hip.h"\n'
        "int main(void) { printf(\"%zu %zu %zu %zu %zu %zu %zu\\n\", sizeof(struct ane_ggml_tensor),"
        " offsetof(struct ane_ggml_tensor, ne), offsetof(struct ane_ggml_tensor, nb),"
        " offsetof(struct ane_ggml_tensor, op), offsetof(struct ane_ggml_tensor, src),"
        " offsetof(struct ane_ggml_tensor, data), offsetof(struct ane_ggml_tensor, op_params)); return 0; }\n")
    exe = tmp_path / "layout"
    subprocess.run([gcc, "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    fields = ("ne", "nb", "op", "src", "data", "op_params")
    want = [ctypes.sizeof(GgmlTensor)] + [getattr(GgmlTensor, f).offset for f in fields]
    assert got == want


def test_backend_names():
    L = ane_amd.lib()
    assert L.ane_ggml_backend_name() == b"ANE"
    assert L.ane_ggml_device_name() == b"ANE0"


def test_supports_op_decisions():
    L = ane_amd.lib()

    def sup(node):
        return L.ane_ggml_supports_op(ctypes.byref(node))

    _, _, d = mul_mat_node(300, 512, 7)
    assert sup(d) == 1
    _, _, d = mul_mat_node(300, 512, 3, B2=4, B3=2, A2=2, A3=1, nb1=4 * 512 + 64, nb_dst1=4 * 300 + 16)
    assert sup(d) == 1                       # broadcast + strided rows
    _, _, d = mul_mat_node(300, 512, 3, B2=3, A2=2)
    assert sup(d) == 0                       # 3 % 2 != 0: not broadcastable
    _, _, d = mul_mat_node(300, 500, 1)
    assert sup(d) == 0                       # K % 32 != 0
    a, b, d = mul_mat_node(300, 512, 1)
    a.type = GgmlType.F16
    d.src[0] = ctypes.pointer(a)
    assert sup(d) == 0                       # weights not Q8_0
    a, b, d = mul_mat_node(300, 512, 1)
    a.nb[1] = 16 * 34 + 34                   # padded weight rows
    d.src[0] = ctypes.pointer(a)
    assert sup(d) == 0
    _, _, d = mul_mat_node(300, 512, 1)
    d.op = GgmlOp.OTHER
    assert sup(d) == 0
    a, b, d = mul_mat_node(300, 512, 3, q4=True)
    assert sup(d) == 1                       # Q4_0 weights (18-byte blocks)
    a.nb[0] = 34
    d.src[0] = ctypes.pointer(a)
    assert sup(d) == 0                       # Q4_0 with Q8_0 strides


def test_unsupported_node_is_rejected_without_gpu():
    be = ane_amd.GgmlBackend(stream=0)
    try:
        _, _, d = mul_mat_node(300, 512, 1)
        d.op = GgmlOp.OTHER
        with pytest.raises(ane_amd.AneError) as e:
            be.compute(d)
        assert e.value.status == 1
    finally:
        be.close()


# ------------------------------------------------------------------ GPU
def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def run_mul_mat(oracle, N, K, T, B2=1, B3=1, A2=1, A3=1, x_pad=0, y_pad=0, mode=0, seed=0):
    """Computes one MUL_MAT node on the GPU and checks it against the
    oracle per (i2, i3) batch.  x_pad / y_pad: extra floats per row."""
    import torch

    W = np.stack([data.q8_0_weights(N, K, seed=seed + 10 * i) for i in range(A2 * A3)])  # [A3*A2, N, rb]
    X = data.activations(B3 * B2 * T, K + x_pad, seed=seed + 1).reshape(B3, B2, T, K + x_pad)
    Wd, Xd = dev(W), dev(X)
    Yd = torch.full((B3, B2, T, N + y_pad), 7.0, dtype=torch.float32, device="cuda")
    rb = K // 32 * 34
    a = ggml_tensor(GgmlType.Q8_0, [K, N, A2, A3], data=Wd)
    xs, ys = 4 * (K + x_pad), 4 * (N + y_pad)
    b = ggml_tensor(GgmlType.F32, [K, T, B2, B3], data=Xd, nb=[4, xs, xs * T, xs * T * B2])
    d = ggml_tensor(GgmlType.F32, [N, T, B2, B3], data=Yd, nb=[4, ys, ys * T, ys * T * B2],
                    op=GgmlOp.MUL_MAT, src=(a, b))
    assert a.nb[1] == rb
    be = ane_amd.GgmlBackend(q8_mode=mode)
    try:
        assert be.supports(d)
        be.graph_compute([d])
    finally:
        be.close()
    Y = host(Yd)
    r2, r3 = B2 // A2, B3 // A3
    for i3 in range(B3):
        for i2 in range(B2):
            Wb = W[(i3 // r3) * A2 + i2 // r2]
            xb = np.ascontiguousarray(X[i3, i2, :, :K])
            if mode == 0:
                ref = oracle.q8_0_mul_mat_g(N, K, T, xb, Wb)
            else:
                ref = np.stack([oracle.q8_0_gemv(N, K, xb[t], Wb) for t in range(T)])
            got = Y[i3, i2, :, :N]
            assert got.tobytes() == np.ascontiguousarray(ref, F32).tobytes(), (i3, i2)
            if y_pad:
                assert (Y[i3, i2, :, N:] == 7.0).all()  # padding of strided output rows untouched


@pytest.mark.gpu
@pytest.mark.parametrize("N,K,T", [(4096, 4096, 1), (300, 512, 4), (300, 512, 7), (1000, 2304, 16)])
def test_ggml_mul_mat_all_tokens(ane, oracle, N, K, T):
    oracle.set_threads(0)
    try:
        run_mul_mat(oracle, N, K, T)
    finally:
        oracle.set_threads(1)


@pytest.mark.gpu
def test_ggml_mul_mat_strided_rows(ane, oracle):
    run_mul_mat(oracle, 257, 512, 3, x_pad=16, y_pad=5)


@pytest.mark.gpu
@pytest.mark.parametrize("B2,B3,A2,A3", [(2, 3, 1, 1), (4, 1, 2, 1), (2, 2, 2, 2), (3, 2, 1, 2)])
def test_ggml_mul_mat_broadcast_batches(ane, oracle, B2, B3, A2, A3):
    run_mul_mat(oracle, 130, 256, 3, B2=B2, B3=B3, A2=A2, A3=A3)


@pytest.mark.gpu
def test_ggml_mul_mat_r_mode(ane, oracle):
    run_mul_mat(oracle, 200, 512, 3, B2=2, mode=1)


@pytest.mark.gpu
def test_ggml_graph_two_nodes(ane, oracle):
    """x -> W1 (Q8_0) -> h -> W2 (Q8_0) -> y in one graph_compute."""
    import torch

    K, H, N, T = 512, 256, 96, 5
    W1, W2 = data.q8_0_weights(H, K, seed=31), data.q8_0_weights(N, H, seed=32)
    x = data.activations(T, K, seed=33)
    h = torch.zeros((T, H), dtype=torch.float32, device="cuda")
    y = torch.zeros((T, N), dtype=torch.float32, device="cuda")
    W1d, W2d, xd = dev(W1), dev(W2), dev(x)
    a1 = ggml_tensor(GgmlType.Q8_0, [K, H], data=W1d)
    b1 = ggml_tensor(GgmlType.F32, [K, T], data=xd)
    n1 = ggml_tensor(GgmlType.F32, [H, T], data=h, op=GgmlOp.MUL_MAT, src=(a1, b1))
    a2 = ggml_tensor(GgmlType.Q8_0, [H, N], data=W2d)
    n2 = ggml_tensor(GgmlType.F32, [N, T], data=y, op=GgmlOp.MUL_MAT, src=(a2, n1))
    be = ane_amd.GgmlBackend()
    try:
        be.graph_compute([n1, n2])
    finally:
        be.close()
    h_ref = oracle.q8_0_mul_mat_g(H, K, T, x, W1)
    y_ref = oracle.q8_0_mul_mat_g(N, H, T, h_ref, W2)
    assert host(h).tobytes() == h_ref.tobytes()
    assert host(y).tobytes() == y_ref.tobytes()


@pytest.mark.gpu
@pytest.mark.parametrize("B2,A2", [(1, 1), (4, 2)])
def test_ggml_mul_mat_q4_0_all_tokens(ane, oracle, B2, A2):
    """Q4_0 weights: every token, in the reference's q4_0_gemv arithmetic."""
    import torch

    N, K, T = 260, 1024, 5
    W = np.stack([data.q_weights("q4_0", N, K, seed=60 + i) for i in range(A2)])
    X = data.activations(B2 * T, K, seed=61).reshape(B2, T, K)
    Y = torch.zeros((B2, T, N), dtype=torch.float32, device="cuda")
    Wd, Xd = dev(W), dev(X)  # the nodes hold raw pointers: keep the tensors alive
    a = ggml_tensor(GgmlType.Q4_0, [K, N, A2], data=Wd)
    b = ggml_tensor(GgmlType.F32, [K, T, B2], data=Xd)
    d = ggml_tensor(GgmlType.F32, [N, T, B2], data=Y, op=GgmlOp.MUL_MAT, src=(a, b))
    assert a.nb[0] == 18 and a.nb[1] == K // 32 * 18
    be = ane_amd.GgmlBackend()
    try:
        assert be.supports(d)
        be.graph_compute([d])
    finally:
        be.close()
    got = host(Y)
    for i2 in range(B2):
        for t in range(T):
            ref = oracle.q_gemv("q4_0", N, K, X[i2, t], W[i2 // (B2 // A2)])
            assert got[i2, t].tobytes() == ref.tobytes(), (i2, t)
