"""The C++ boundary end to end on the GPU: tests/cpp/mnist_i8_dispatch.cpp,
the reference's int8 MNIST call sequence (tests/test_mnist_i8.cpp:198-207
and :303-314) written with ane::dispatch from include/ane/ane.hpp and
linked against libane_amd.so, runs as a child process and its outputs are
compared bit for bit with the CPU oracle's composition of the same opcodes.

* device buffers (hipMalloc);
* plain host buffers (aligned_alloc, as the reference allocates them) with
  ANE_HOST_STAGING=1, so the program makes no call outside the reference's
  API;
* plain host buffers without staging: the first dispatch is refused
  (ANE_ERR_BAD_POINTER) instead of faulting.
"""
import os
import subprocess
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parents[1]
EXE = ROOT / "tests" / "cpp" / "mnist_i8_dispatch"
F32 = np.float32
B, INP_K, HID, HID_K, OUT_PAD, ROWS = 50, 832, 128, 128, 16, 64


def _inputs(seed=12):
    g = np.random.default_rng(seed)
    x_u8 = np.zeros((ROWS, INP_K), np.uint8)
    x_u8[:B, :784] = g.integers(0, 256, size=(B, 784))
    W1 = np.zeros((INP_K, HID), F32)
    W1[:784] = g.standard_normal((784, HID)) * 0.05
    W2 = (g.standard_normal((HID_K, OUT_PAD)) * 0.05).astype(F32)
    logit_bias = np.array([0] * 10 + [-1000.0] * 6, F32)
    return x_u8, W1, W2, logit_bias


def _oracle_forward(oracle, x_u8, W1, W2, logit_bias):
    w1q, s1 = oracle.quantize(W1.ravel())
    w1p = oracle.pack_b(w1q, INP_K, HID)
    w2q, s2 = oracle.quantize(W2.ravel())
    w2p = oracle.pack_b(w2q, HID_K, OUT_PAD)
    h = oracle.dense_i8(B, HID, INP_K, F32(1 / 255), s1, 1, x_u8, w1p, np.zeros(INP_K, F32), unsigned_a=True)
    hq, sh = oracle.quantize(h[:B].ravel(), B * HID_K)
    hq_pad = np.zeros((ROWS, HID_K), np.int8)
    hq_pad[:B] = hq.reshape(B, HID_K)
    logits = oracle.dense_i8(B, OUT_PAD, HID_K, sh, s2, 0, hq_pad, w2p, logit_bias)
    return h, logits, np.array([s1, s2, sh], F32)


def _run(mode, tmp, staging):
    assert EXE.exists(), "build tests/cpp/mnist_i8_dispatch first (python -m ane_amd.build)"
    env = dict(os.environ)
    env.pop("ANE_HOST_STAGING", None)
    if staging:
        env["ANE_HOST_STAGING"] = "1"
    print(f"mnist_i8_dispatch {mode} staging={staging}", flush=True)
    return subprocess.run([str(EXE), mode, str(tmp)], env=env, capture_output=True, text=True, timeout=120)


def _bits(a):
    return np.ascontiguousarray(a, F32).view(np.uint32)


@pytest.fixture(scope="module")
def case(oracle, tmp_path_factory):
    tmp = tmp_path_factory.mktemp("mnist_i8")
    x_u8, W1, W2, logit_bias = _inputs()
    for name, a in (("x_u8", x_u8), ("W1", W1), ("W2", W2), ("logit_bias", logit_bias)):
        (tmp / f"{name}.bin").write_bytes(np.ascontiguousarray(a).tobytes())
    return tmp, _oracle_forward(oracle, x_u8, W1, W2, logit_bias)


@pytest.mark.parametrize("mode,staging", [("device", False), ("host", True)])
def test_mnist_i8_through_cpp_dispatch(case, mode, staging):
    tmp, (h, logits, scales) = case
    for f in ("hidden.bin", "logits.bin", "scales.bin"):
        (tmp / f).unlink(missing_ok=True)
    r = _run(mode, tmp, staging)
    assert r.returncode == 0, r.stdout + r.stderr
    got_s = np.fromfile(tmp / "scales.bin", F32)
    np.testing.assert_array_equal(_bits(got_s), _bits(scales))
    got_h = np.fromfile(tmp / "hidden.bin", F32).reshape(ROWS, HID)
    np.testing.assert_array_equal(_bits(got_h), _bits(h))
    got_l = np.fromfile(tmp / "logits.bin", F32).reshape(ROWS, OUT_PAD)
    np.testing.assert_array_equal(_bits(got_l), _bits(logits))


def test_host_buffers_refused_without_staging(case):
    tmp, _ = case
    r = _run("host", tmp, staging=False)
    assert r.returncode == 1, r.stdout + r.stderr
    assert "quantize W1 failed: status 2" in r.stderr and "not device-accessible" in r.stderr


def test_host_staging_inout_operand(ane):
    """cblas_igemm with beta != 0 and ldc > N reads C as well as writing it
    (and leaves the gaps between rows alone): with host staging, numpy host
    buffers give the same bytes as device tensors, including the untouched
    gap columns."""
    import torch

    M, N, K, lda, ldb, ldc = 37, 29, 192, 200, 192, 33
    g = np.random.default_rng(5)
    A = g.integers(-127, 128, size=(M, lda), dtype=np.int8)
    Bt = g.integers(-127, 128, size=(N, ldb), dtype=np.int8)
    C0 = g.standard_normal((M, ldc)).astype(F32)
    Cd = torch.from_numpy(C0.copy()).cuda()
    ane.stream_exec(ane.rec_cblas_igemm("igemm", 2, M, N, K, lda, ldb, ldc, 0.5, 0.25,
                                        torch.from_numpy(A).cuda(), torch.from_numpy(Bt).cuda(), Cd))
    want = Cd.cpu().numpy()
    Ch = C0.copy()
    lib = ane.lib()
    lib.ane_set_host_staging(1)
    try:
        ane.stream_exec(ane.rec_cblas_igemm("igemm", 2, M, N, K, lda, ldb, ldc, 0.5, 0.25,
                                            A.ctypes.data, Bt.ctypes.data, Ch.ctypes.data))
    finally:
        lib.ane_set_host_staging(-1)
    np.testing.assert_array_equal(_bits(Ch), _bits(want))
    np.testing.assert_array_equal(_bits(Ch[:, N:]), _bits(C0[:, N:]))
    with pytest.raises(ane.AneError) as e:
        lib.ane_set_host_staging(0)
        try:
            ane.stream_exec(ane.rec_cblas_igemm("igemm", 2, M, N, K, lda, ldb, ldc, 0.5, 0.25,
                                                A.ctypes.data, Bt.ctypes.data, Ch.ctypes.data))
        finally:
            lib.ane_set_host_staging(-1)
    assert e.value.status == 2
