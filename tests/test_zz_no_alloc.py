"""The no-allocation entry point ane_hip_q8_0_mul_mat_noalloc, through the C
ABI: bit-identical to ane_hip_q8_0_mul_mat (which takes a caller workspace)
on two calls in a row, the second with a smaller input, and a clear error
for shapes past its static scratch array."""
import ctypes

import numpy as np
import pytest

from tests import data

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _run(ane, fn_name, N, K, T, x, W):
    import torch

    L = ane.lib()
    y = torch.full((T * N,), 5.0, dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    if fn_name == "noalloc":
        st = L.ane_hip_q8_0_mul_mat_noalloc(N, K, T, x.data_ptr(), W.data_ptr(), y.data_ptr(), s)
    else:
        wsb = L.ane_hip_q8_0_mul_mat_workspace_size(K, T)
        ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
        st = L.ane_hip_q8_0_mul_mat(N, K, T, x.data_ptr(), W.data_ptr(), y.data_ptr(), ws.data_ptr(), wsb, s)
    assert st == 0, (fn_name, st)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("big,small", [((4096, 4096, 64), (300, 512, 5)),      # MFMA kernels
                                       ((6144, 4096, 4), (4096, 14336, 1)),    # streaming, pre-quantized
                                       ((28672, 4096, 16), (100, 96, 3))])     # MFMA, then general kernel
def test_noalloc_matches_workspace_entry(ane, big, small):
    for i, (N, K, T) in enumerate((big, small)):
        W = _dev(data.q8_0_weights(N, K - K % 32, seed=N + K + i))
        x = _dev(data.activations(T, K, seed=T + 11 * i))
        want = _run(ane, "workspace", N, K, T, x, W)
        got = _run(ane, "noalloc", N, K, T, x, W)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (N, K, T)


def test_noalloc_rejects_shapes_past_scratch(ane):
    import torch

    L = ane.lib()
    cap = L.ane_hip_q8_0_mul_mat_noalloc_max_bytes()
    assert cap == 4 << 20
    N, K, T = 64, 14336, 300  # 300 tokens of 14336 values need more than 4 MiB
    assert L.ane_hip_q8_0_mul_mat_workspace_size(K, T) > cap
    y = torch.full((T * N,), 5.0, dtype=torch.float32, device="cuda")
    W = torch.zeros(N * (K // 32) * 34, dtype=torch.uint8, device="cuda")
    x = torch.zeros(T * K, dtype=torch.float32, device="cuda")
    st = L.ane_hip_q8_0_mul_mat_noalloc(N, K, T, x.data_ptr(), W.data_ptr(), y.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream)
    assert st == 8  # ANE_ERR_WORKSPACE, before anything runs
    torch.cuda.synchronize()
    assert (y.cpu().numpy() == 5.0).all()
