"""Seeded synthetic inputs shaped like the benchmark configurations.

Shared by the tests, bench.py and __graft_entry__.smoke() so every consumer
sees the same bytes for a given (config, seed).
"""
from __future__ import annotations

import numpy as np


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def mnist_inputs(seed: int = 1, batch: int = 50):
    """Config 1: x 50x784 in [0,1] with ~80% exact zeros, W1 784x128 and
    W2 128x10 ~ N(0, 0.05), all fp32."""
    g = rng(seed)
    x = g.uniform(0.0, 1.0, size=(batch, 784)).astype(np.float32)
    x[g.uniform(size=x.shape) < 0.8] = 0.0
    w1 = (g.standard_normal((784, 128)) * 0.05).astype(np.float32)
    w2 = (g.standard_normal((128, 10)) * 0.05).astype(np.float32)
    return x, w1, w2


def gemm_inputs(M: int, N: int, K: int, seed: int = 2):
    """Config 2: A (M x K) and B (K x N) ~ N(0, 1) fp32."""
    g = rng(seed)
    A = g.standard_normal((M, K), dtype=np.float32)
    B = g.standard_normal((K, N), dtype=np.float32)
    return A, B


def q8_0_weights(N: int, K: int, seed: int = 3) -> np.ndarray:
    """Config 3/4 weights: N rows of K/32 Q8_0 blocks; qs ~ U{-127..127},
    d = fp16(|N(0, 0.01)|).  Returns the raw bytes, shape (N, K/32*34)."""
    g = rng(seed)
    nb = K // 32
    qs = g.integers(-127, 128, size=(N, nb, 32), dtype=np.int8)
    d = np.abs(g.standard_normal((N, nb)) * 0.01).astype(np.float16)
    W = np.empty((N, nb, 34), np.uint8)
    W[:, :, :2] = d.view(np.uint8).reshape(N, nb, 2)
    W[:, :, 2:] = qs.view(np.uint8)
    return W.reshape(N, nb * 34)


# byte offsets of the fp16 fields of one block of each R-mode format (the
# layouts of bytecode_interpreter.s:7071-7126 and 11024-11626)
Q_BLOCK = {"q4_0": (18, 32, (0,)), "q4_k": (144, 256, (0, 2)), "q2_k": (84, 256, (80, 82)),
           "q3_k": (110, 256, (108,)), "q5_k": (176, 256, (0, 2)), "q6_k": (210, 256, (208,))}


def q_weights(fmt: str, N: int, K: int, seed: int = 5) -> np.ndarray:
    """N rows of K/values blocks of format fmt: random quant and scale bytes,
    the fp16 super-scales (d, dmin) = fp16(|N(0, 0.01)|).  Shape (N, row bytes)."""
    g = rng(seed)
    nbytes, nvals, fp16_at = Q_BLOCK[fmt]
    nb = K // nvals
    W = g.integers(0, 256, size=(N, nb, nbytes), dtype=np.uint8)
    for off in fp16_at:
        d = np.abs(g.standard_normal((N, nb)) * 0.01).astype(np.float16)
        W[:, :, off:off + 2] = d.view(np.uint8).reshape(N, nb, 2)
    return W.reshape(N, nb * nbytes)


def activations(T: int, K: int, seed: int = 4) -> np.ndarray:
    return rng(seed).standard_normal((T, K), dtype=np.float32)
