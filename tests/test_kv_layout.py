"""The KV cache's page block layout (host side; no GPU).

The attention kernels load K and V operand fragments of v_mfma_f32_32x32x16
straight from the cache pages, one contiguous kilobyte per wavefront load.
These tests pin the block layout (dtree_hip.cache.k_block_index /
v_block_index, the same formulas as kv_k_off / kv_v_off in csrc/common.h)
against the MFMA operand layouts of CDNA3/CDNA4 stated independently here:

* A operand (32 x 16): lane l holds row l % 32, k elements 8 (l // 32) .. +7.
* C / D (32 x 32): lane l, register i holds row 8 (i // 4) + 4 (l // 32) + i % 4,
  column l % 32.

and check the host's logical views and writes round-trip.
"""
import numpy as np
import pytest
import torch

from dtree_hip.cache import PAGE, PagedKVCache, k_block_index, v_block_index


def _inverse(idx: torch.Tensor) -> np.ndarray:
    """offset -> (slot, dim)"""
    S, D = idx.shape
    inv = np.full((S * D, 2), -1, np.int64)
    flat = idx.reshape(-1).numpy()
    inv[flat, 0] = np.repeat(np.arange(S), D)
    inv[flat, 1] = np.tile(np.arange(D), S)
    return inv


@pytest.mark.parametrize("D", [128, 256])
def test_blocks_are_permutations(D):
    for idx in (k_block_index(D), v_block_index(D)):
        assert idx.shape == (PAGE, D)
        assert torch.equal(torch.sort(idx.reshape(-1)).values, torch.arange(PAGE * D))


def _c_row(lane: int, reg: int) -> int:
    return 8 * (reg // 4) + 4 * (lane // 32) + reg % 4


@pytest.mark.parametrize("D", [128, 256])
def test_fragments_are_contiguous_kilobytes(D):
    """Every K fragment (key half b, dim step j) and V fragment (key step st,
    dim block db) is one kilobyte, the fragments of a key half (K) and of a
    key step (V) are consecutive kilobytes: lane l's 16 bytes at 16 l of it hold the
    A-operand elements that lane needs, and the keys of the K rows make the
    S^T accumulator of a lane half hold runs of 8 consecutive keys, which
    are the keys the same lane's V fragment holds (so P^T comes straight from
    the S^T registers)."""
    ki, vi = _inverse(k_block_index(D)), _inverse(v_block_index(D))
    for b in range(2):
        row_key = {}
        for j in range(D // 16):
            base = (b * (D // 16) + j) * 512
            for lane in range(64):
                els = ki[base + 8 * lane: base + 8 * lane + 8]
                keys, dims = set(els[:, 0]), els[:, 1]
                assert len(keys) == 1  # one A row per lane
                assert list(dims) == [16 * j + 8 * (lane // 32) + e for e in range(8)]
                key = keys.pop()
                assert key // 32 == b
                assert row_key.setdefault(lane % 32, key) == key  # same key for every dim step
        # S^T = K Q^T: C row rho of a lane holds the key loaded as A row rho
        for lane in range(64):
            for half in range(2):
                keys = [row_key[_c_row(lane, 8 * half + e)] for e in range(8)]
                first = 32 * b + 16 * half + 8 * (lane // 32)
                assert keys == list(range(first, first + 8))
    for st in range(PAGE // 16):
        for db in range(D // 32):
            base = (st * (D // 32) + db) * 512
            for lane in range(64):
                els = vi[base + 8 * lane: base + 8 * lane + 8]
                assert list(els[:, 1]) == [32 * db + lane % 32] * 8
                assert list(els[:, 0]) == [16 * st + 8 * (lane // 32) + e for e in range(8)]


def test_logical_views_round_trip():
    torch.manual_seed(0)
    order = torch.tensor([3, 0, 2, 1], dtype=torch.int32)
    c = PagedKVCache(layers=2, kv_heads=3, head_dim=128, capacity=4 * PAGE, device="cpu", page_order=order)
    T = 150
    k = torch.randn(T, 3, 128).to(torch.bfloat16)
    v = torch.randn(T, 3, 128).to(torch.bfloat16)
    c.write_logical(1, k[:100], v[:100])
    c.write_logical(1, k[100:], v[100:], start=100)
    assert torch.equal(c.logical_keys(1, T), k)
    assert torch.equal(c.logical_values(1, T), v)
    assert not c.k_pages[0].any() and not c.v_pages[0].any()
    # position t, dim d of layer 1 sits where the block formulas put it
    t, h, d = 77, 2, 45
    page = int(order[t // PAGE])
    assert c.k_pages[1, page, h, int(k_block_index(128)[t % PAGE, d])] == k[t, h, d]
    assert c.v_pages[1, page, h, int(v_block_index(128)[t % PAGE, d])] == v[t, h, d]
