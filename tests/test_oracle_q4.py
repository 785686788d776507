"""Pins of the q4 group-64 oracle (oracle/q4.py) without MLX.

MLX's quantized layout (adapters.py:63-71, api.py:46-54) stores element k of a
row as nibble k % 8 of uint32 word k // 8 and dequantises W = s q + b per
group of 64. The packing is pinned by exact known-answer words and round
trips; the product by the closed-form dequantisation and by the grouped affine
identity the HIP kernel evaluates (s (x.q) + b (sum x) per group)."""
import numpy as np
import pytest

from oracle import q4 as o4
from oracle.qwen3 import bf16_to_f32


def test_nibble_order_known_words():
    q = np.array([[0, 1, 2, 3, 4, 5, 6, 7, 15, 14, 13, 12, 11, 10, 9, 8]], np.uint8)
    w = o4.pack_nibbles(q)
    assert w.tolist() == [[0x76543210, 0x89ABCDEF]]
    assert o4.unpack_nibbles(w).tolist() == q.tolist()


@pytest.mark.parametrize("seed", range(3))
def test_pack_unpack_round_trip(seed):
    g = np.random.default_rng(seed)
    q = g.integers(0, 16, size=(5, 128), dtype=np.uint8)
    assert np.array_equal(o4.unpack_nibbles(o4.pack_nibbles(q)), q)
    w = g.integers(0, 2 ** 32, size=(3, 24), dtype=np.uint64).astype(np.uint32)
    assert np.array_equal(o4.pack_nibbles(o4.unpack_nibbles(w)), w)


def test_dequantize_closed_form():
    # one row, two groups: q = k % 16, s = (0.5, 2), b = (-1, 3)
    q = (np.arange(128) % 16).astype(np.uint8)[None]
    W = o4.dequantize(o4.pack_nibbles(q), np.array([[0.5, 2.0]]), np.array([[-1.0, 3.0]]))
    expect = np.concatenate([0.5 * (np.arange(64) % 16) - 1.0, 2.0 * (np.arange(64) % 16) + 3.0])
    assert np.array_equal(W[0], expect)


@pytest.mark.parametrize("seed", range(3))
def test_grouped_affine_identity(seed):
    g = np.random.default_rng(seed)
    wq, s, b = o4.random_q4(96, 256, g)
    x = g.standard_normal((7, 256))
    dense = o4.q4_matmul(x, wq, bf16_to_f32(s), bf16_to_f32(b))
    grouped = o4.q4_matmul_grouped(x, wq, bf16_to_f32(s), bf16_to_f32(b))
    assert np.abs(dense - grouped).max() <= 1e-12 * np.abs(dense).max()
    # a planted mistake in the oracle (scale and bias swapped) breaks it
    wrong = o4.q4_matmul(x, wq, bf16_to_f32(b), bf16_to_f32(s))
    assert np.abs(wrong - dense).max() > 1e-3 * np.abs(dense).max()


def test_random_q4_statistics():
    g = np.random.default_rng(0)
    wq, s, b = o4.random_q4(256, 1024, g)
    q = o4.unpack_nibbles(wq)
    assert q.min() == 0 and q.max() == 15
    sf, bf = bf16_to_f32(s), bf16_to_f32(b)
    assert (sf >= 0).all() and abs(sf.mean() - 0.02 * 8 * np.sqrt(2 / np.pi)) < 0.01
    assert abs(bf.std() - 0.01) < 0.002
