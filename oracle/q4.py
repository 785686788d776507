"""Oracle: 4-bit affine group-64 quantised linear layer (MLX quantized format).

Test infrastructure only (see ``oracle/__init__.py``).

Format (adapters.py:63-71 calls ``mx.quantized_matmul(x, w, scales, biases,
transpose=True, group_size=64, bits=4)`` on ``nn.QuantizedLinear`` weights made
by ``quantize_model``, api.py:46-54):

* ``wq``     uint32 [N, K/8]: element k of row n is nibble k % 8 of word k // 8,
  i.e. bits [4 (k % 8), 4 (k % 8) + 4).
* ``scales`` bf16 [N, K/64], ``biases`` bf16 [N, K/64].
* ``W[n, k] = scales[n, k // 64] * q[n, k] + biases[n, k // 64]``, q in [0, 15].

y = x W^T is evaluated here in float64 on the dequantised matrix. What pins
it: exact integer packing round trips, the closed-form dequantisation, and the
affine-group identity ``x . (s q + b) = s (x . q) + b (sum x)`` per group that
the HIP kernel evaluates (tests/test_oracle_q4.py). The nibble order inside
MLX's words and the rounding of ``mx.quantized_matmul`` itself are MLX
internals: parity unpinned beyond the logit tolerance.
"""
from __future__ import annotations

import numpy as np

GROUP = 64


def pack_nibbles(q: np.ndarray) -> np.ndarray:
    """q uint8 [N, K] in [0, 15] -> uint32 [N, K/8] (element k at bits 4 (k % 8))."""
    q = np.asarray(q, np.uint32)
    n, k = q.shape
    assert k % 8 == 0 and q.max(initial=0) < 16
    q = q.reshape(n, k // 8, 8)
    return np.bitwise_or.reduce(q << (4 * np.arange(8, dtype=np.uint32)), axis=-1).astype(np.uint32)


def unpack_nibbles(wq: np.ndarray) -> np.ndarray:
    """uint32 [N, K/8] -> uint8 [N, K]."""
    wq = np.asarray(wq, np.uint32)
    n, kw = wq.shape
    return ((wq[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).astype(np.uint8).reshape(n, kw * 8)


def dequantize(wq: np.ndarray, scales: np.ndarray, biases: np.ndarray) -> np.ndarray:
    """float64 [N, K] = scales * q + biases per group of 64 (scales/biases as float arrays)."""
    q = unpack_nibbles(wq).astype(np.float64)
    n, k = q.shape
    s = np.repeat(np.asarray(scales, np.float64), GROUP, axis=1)[:, :k]
    b = np.repeat(np.asarray(biases, np.float64), GROUP, axis=1)[:, :k]
    return s * q + b


def q4_matmul(x: np.ndarray, wq: np.ndarray, scales: np.ndarray, biases: np.ndarray) -> np.ndarray:
    """y = x W^T in float64."""
    return np.asarray(x, np.float64) @ dequantize(wq, scales, biases).T


def q4_matmul_grouped(x: np.ndarray, wq: np.ndarray, scales: np.ndarray, biases: np.ndarray) -> np.ndarray:
    """The same product through the per-group affine identity
    y = sum_g s_g (x_g . q_g) + b_g (sum x_g), in float64."""
    x = np.asarray(x, np.float64)
    q = unpack_nibbles(wq).astype(np.float64)
    n, k = q.shape
    y = np.zeros((x.shape[0], n))
    s = np.asarray(scales, np.float64)
    b = np.asarray(biases, np.float64)
    for g in range(k // GROUP):
        sl = slice(g * GROUP, (g + 1) * GROUP)
        y += (x[:, sl] @ q[:, sl].T) * s[:, g] + np.outer(x[:, sl].sum(1), b[:, g])
    return y


def random_q4(n: int, k: int, rng: np.random.Generator):
    """Synthetic q4 layer: nibbles uniform in [0, 15], scales |N(0, 0.02)| * 8,
    biases N(0, 0.01), scales/biases rounded to bf16 (returned as bf16 bit
    patterns, uint16)."""
    from .qwen3 import f32_to_bf16_bits

    q = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
    scales = f32_to_bf16_bits((np.abs(rng.standard_normal((n, k // GROUP))) * 0.02 * 8).astype(np.float32))
    biases = f32_to_bf16_bits((rng.standard_normal((n, k // GROUP)) * 0.01).astype(np.float32))
    return pack_nibbles(q), scales, biases
