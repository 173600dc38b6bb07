"""The ggml registry adapter (ane_amd/ggml/ggml-ane.cpp): ggml_backend_ane_reg()
with its device, buffer type and backend, driven as ggml's scheduler would
through tests/ggml_iface (a restatement of the ggml declarations it uses and
a small C harness).

CPU: the adapter compiles with g++ against that interface; the registry's
names, counts, device type, buffer-type facts and supports_op decisions
(host logic only).
GPU: MUL_MAT through the registry (device buffer, set_tensor, a graph with
a view node, graph_compute, get_tensor) bit-identical to the oracle, for
Q8_0 (every token) and Q4_0 weights; a graph holding an op the backend does
not run (MUL_MAT with F32 weights) fails with GGML_STATUS_FAILED.  The fp32
ops are covered in tests/test_ggml_ops.py.

ggml's own behaviour around the backend (its scheduler, its op numbering)
is not available here and stays unpinned.
"""
import ctypes
import shutil
import subprocess

import numpy as np
import pytest

import ane_amd
from ane_amd import build as ane_build
from tests import data

F32 = np.float32
T_Q8, T_Q4, T_F32, T_F16 = 8, 2, 0, 1


def _load(path):
    ane_amd.lib()  # libane_amd.so first (RTLD_GLOBAL)
    t = ctypes.CDLL(str(path))
    t.ggml_ane_test_registry.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
    t.ggml_ane_test_supports.argtypes = [ctypes.c_int] * 4 + [ctypes.c_longlong] * 8
    t.ggml_ane_test_mul_mat.argtypes = [ctypes.c_int] * 4 + [ctypes.c_void_p] * 3
    t.ggml_ane_test_unsupported_graph.argtypes = []
    return t


@pytest.fixture(scope="module")
def fresh(tmp_path_factory):
    """The adapter and harness compiled now, into a temporary library."""
    if not shutil.which("g++"):
        pytest.skip("g++ not available")
    out = tmp_path_factory.mktemp("ggml") / "libggml_ane_test.so"
    res = subprocess.run(ane_build.ggml_adapter_cmd(out), capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    return _load(out)


def registry(t) -> dict:
    buf = ctypes.create_string_buffer(1024)
    assert t.ggml_ane_test_registry(buf, len(buf)) == 0
    return dict(kv.split("=", 1) for kv in buf.value.decode().split(";"))


def test_registry_facts(fresh):
    r = registry(fresh)
    assert r["reg"] == "ANE" and r["dev"] == "ANE0"  # the reference's names (ggml-ane.cpp:302-304, 412-414)
    assert r["devices"] == "1" and r["dev1"] == "null"
    assert r["api"] == "1"  # GGML_BACKEND_API_VERSION of the header it was compiled with
    assert r["type"] == "1"  # GGML_BACKEND_DEVICE_TYPE_GPU: buffers are device memory
    assert r["dev_reg"] == "1" and r["same_reg"] == "1"
    assert r["buft"] == "ANE" and r["align"] == "256" and r["is_host"] == "0" and r["buft_dev"] == "1"
    assert r["own_buft"] == "1" and r["other_buft"] == "0"


def supports(t, op=0, type0=T_Q8, type1=T_F32, typed=T_F32, K=4096, N=64, A2=1, A3=1, T=3, B2=1, B3=1, pad=0):
    return t.ggml_ane_test_supports(op, type0, type1, typed, K, N, A2, A3, T, B2, B3, pad) == 1


def test_supports_op_decisions(fresh):
    t = fresh
    assert supports(t)                       # Q8_0 weights, every token
    assert supports(t, type0=T_Q4)           # Q4_0 weights (q4_0_gemv arithmetic)
    assert supports(t, T=1) and supports(t, T=64)
    assert supports(t, A2=2, B2=4)           # broadcast batches
    assert supports(t, pad=64)               # strided activation rows
    assert not supports(t, type0=T_F32)      # F32 weights stay on ggml's CPU backend
    assert not supports(t, type1=T_F16)      # activations must be F32
    assert not supports(t, typed=T_F16)
    assert not supports(t, A2=3, B2=4)       # not broadcastable
    assert supports(t, op=1, type0=T_F32, K=16, N=1, T=1)    # a view: no compute
    assert supports(t, op=2, type0=T_F32, K=16, N=16, T=16)  # ADD of equal shapes
    assert not supports(t, op=2, type0=T_F32, K=16, N=1, T=1)  # ADD of src0 [16,1] into dst [1,1]


# ------------------------------------------------------------------ GPU
@pytest.fixture(scope="module")
def built():
    if not ane_build.GGML_TEST_LIB.exists():
        pytest.fail(f"{ane_build.GGML_TEST_LIB} is missing: run python -m ane_amd.build")
    return _load(ane_build.GGML_TEST_LIB)


@pytest.mark.gpu
@pytest.mark.parametrize("N,K,T", [(4096, 4096, 1), (300, 512, 3), (1000, 2304, 16)])
def test_registry_mul_mat_q8_0(ane, oracle, built, N, K, T):
    W = data.q8_0_weights(N, K, seed=71)
    X = data.activations(T, K, seed=72)
    Y = np.zeros((T, N), F32)
    st = built.ggml_ane_test_mul_mat(T_Q8, N, K, T, W.ctypes.data, X.ctypes.data, Y.ctypes.data)
    assert st == 0  # GGML_STATUS_SUCCESS
    ref = oracle.q8_0_mul_mat_g(N, K, T, X, W)
    assert Y.tobytes() == np.ascontiguousarray(ref, F32).tobytes()


@pytest.mark.gpu
def test_registry_mul_mat_q4_0(ane, oracle, built):
    N, K, T = 260, 1024, 5
    W = data.q_weights("q4_0", N, K, seed=73)
    X = data.activations(T, K, seed=74)
    Y = np.zeros((T, N), F32)
    assert built.ggml_ane_test_mul_mat(T_Q4, N, K, T, W.ctypes.data, X.ctypes.data, Y.ctypes.data) == 0
    for t in range(T):
        assert Y[t].tobytes() == oracle.q_gemv("q4_0", N, K, X[t], W).tobytes(), t


@pytest.mark.gpu
def test_registry_graph_with_unsupported_node_fails(ane, built):
    assert built.ggml_ane_test_unsupported_graph() == -1  # GGML_STATUS_FAILED
