"""Paged bf16 KV cache for the tree-verify kernels.

Layout (all layers in one allocation each, so compaction is one launch):
  k_pages, v_pages [layers, n_pages, kv_heads, PAGE * head_dim]: one block of
          PAGE positions x head_dim dims per (page, kv head), each in the
          order the attention MFMAs read their operands, so a wavefront's
          16-byte-per-lane load of one operand fragment is one contiguous
          kilobyte (``k_block_index`` / ``v_block_index``; the kernels use the
          same formulas, kv_k_off / kv_v_off in csrc/common.h).
  page_table [n_pages] int32: logical page -> physical page.

Logical position t of a layer lives in physical page page_table[t // PAGE] at
slot t % PAGE. ``offset`` is the number of committed positions (the KVCache
offset of mlx-lm that dtree_runtime / the adapters read).
"""
from __future__ import annotations

import functools

import torch

from ._native import PAGE


def _pi(r: torch.Tensor) -> torch.Tensor:
    """Swap bits 2 and 3 (an involution on 0..31)."""
    return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1)


@functools.lru_cache(maxsize=None)
def _block_index(head_dim: int, which: str) -> torch.Tensor:
    slot = torch.arange(PAGE).view(PAGE, 1)
    d = torch.arange(head_dim).view(1, head_dim)
    if which == "k":
        # S^T = K Q^T fragment (key half b = slot // 32, dim step j = d // 16):
        # kilobyte b * (head_dim // 16) + j, lane 32 * ((d // 8) % 2) + pi(slot % 32), element d % 8
        off = ((((slot >> 5) * (head_dim >> 4) + (d >> 4)) * 64 + ((d >> 3) & 1) * 32 + _pi(slot & 31)) << 3) + (d & 7)
    else:
        # O^T = V^T P^T fragment (key step st = slot // 16, dim block db = d // 32):
        # kilobyte st * (head_dim // 32) + db, lane 32 * ((slot // 8) % 2) + d % 32, element slot % 8
        off = ((((slot >> 4) * (head_dim >> 5) + (d >> 5)) * 64 + ((slot >> 3) & 1) * 32 + (d & 31)) << 3) + (slot & 7)
    return off


def k_block_index(head_dim: int) -> torch.Tensor:
    """[PAGE, head_dim] int64: element offset of K (slot, dim) inside a (page, kv head) block."""
    return _block_index(head_dim, "k")


def v_block_index(head_dim: int) -> torch.Tensor:
    """[PAGE, head_dim] int64: element offset of V (slot, dim) inside a (page, kv head) block."""
    return _block_index(head_dim, "v")


class LayerCacheView:
    """Per-layer handle with the fields the reference runtime reads (offset)."""

    def __init__(self, cache: "PagedKVCache", layer: int):
        self._c = cache
        self.layer = layer

    @property
    def offset(self) -> int:
        return self._c.offset

    @property
    def keys(self) -> torch.Tensor:
        return self._c.logical_keys(self.layer)

    @property
    def values(self) -> torch.Tensor:
        return self._c.logical_values(self.layer)


class PagedKVCache:
    def __init__(self, layers: int, kv_heads: int, head_dim: int, capacity: int, device="cuda",
                 page_order: torch.Tensor | None = None):
        self.layers = layers
        self.kv_heads = kv_heads
        self.head_dim = head_dim
        self.n_pages = (capacity + PAGE - 1) // PAGE
        self.capacity = self.n_pages * PAGE
        dev = torch.device(device)
        if head_dim % 32:
            raise ValueError("head_dim must be a multiple of 32 (the cache's 32-dim fragment blocks)")
        self.k_pages = torch.zeros(layers, self.n_pages, kv_heads, PAGE * head_dim, dtype=torch.bfloat16, device=dev)
        self.v_pages = torch.zeros(layers, self.n_pages, kv_heads, PAGE * head_dim, dtype=torch.bfloat16, device=dev)
        if page_order is None:
            page_order = torch.arange(self.n_pages, dtype=torch.int32)
        if sorted(page_order.tolist()) != list(range(self.n_pages)):
            raise ValueError("page_order must be a permutation of the pages")
        self.page_table = page_order.to(device=dev, dtype=torch.int32).contiguous()
        self.offset = 0

    @property
    def layer_stride(self) -> int:
        return self.n_pages * self.kv_heads * PAGE * self.head_dim

    def k_ptr(self, layer: int) -> int:
        return self.k_pages.data_ptr() + 2 * layer * self.layer_stride

    def v_ptr(self, layer: int) -> int:
        return self.v_pages.data_ptr() + 2 * layer * self.layer_stride

    def __len__(self) -> int:
        return self.layers

    def __getitem__(self, i: int) -> LayerCacheView:
        if not 0 <= i < self.layers:
            raise IndexError(i)
        return LayerCacheView(self, i)

    def __iter__(self):
        return (LayerCacheView(self, i) for i in range(self.layers))

    # ---- logical views (tests, checkers, cache import) -------------------
    def _pages_for(self, length: int) -> torch.Tensor:
        n = (length + PAGE - 1) // PAGE
        return self.page_table[:n].long()

    def _logical(self, pages: torch.Tensor, T: int, which: str) -> torch.Tensor:
        pg = pages[self._pages_for(T)]  # [np, Hkv, PAGE * D]
        idx = _block_index(self.head_dim, which).to(pg.device).reshape(-1)
        rows = pg[:, :, idx].view(-1, self.kv_heads, PAGE, self.head_dim)
        return rows.permute(0, 2, 1, 3).reshape(-1, self.kv_heads, self.head_dim)[:T]

    def logical_keys(self, layer: int, length: int | None = None) -> torch.Tensor:
        """[T, kv_heads, head_dim] bf16, logical order."""
        return self._logical(self.k_pages[layer], self.offset if length is None else length, "k")

    def logical_values(self, layer: int, length: int | None = None) -> torch.Tensor:
        return self._logical(self.v_pages[layer], self.offset if length is None else length, "v")

    def write_logical(self, layer: int, keys: torch.Tensor, values: torch.Tensor, start: int = 0) -> None:
        """Store [T, kv_heads, head_dim] rows at logical positions start..start+T-1."""
        T = keys.shape[0]
        if start + T > self.capacity:
            raise ValueError("cache capacity exceeded")
        dev = self.k_pages.device
        keys = keys.to(dev, torch.bfloat16)
        values = values.to(dev, torch.bfloat16)
        pos = torch.arange(start, start + T, device=dev)
        page = self.page_table.long()[pos // PAGE].view(T, 1, 1)
        slot = pos % PAGE
        head = torch.arange(self.kv_heads, device=dev).view(1, -1, 1)
        for pages, rows, which in ((self.k_pages[layer], keys, "k"), (self.v_pages[layer], values, "v")):
            off = _block_index(self.head_dim, which).to(dev)[slot].view(T, 1, self.head_dim)
            pages[page, head, off] = rows

    def reset(self, offset: int = 0) -> None:
        self.offset = offset


class Qwen35Cache:
    """Committed state of a Qwen3.5 hybrid: a paged KV cache for the gated
    attention layers and, per GatedDeltaNet layer, the conv window
    [K - 1, conv_dim] and the recurrent state [Hv, Dv, Dk], both fp32 (the
    ArraysCache entries [conv_state, state] of mlx-lm, qwen35_tree.py:85-101).
    ``offset`` counts committed positions, as the KVCache offset does.

    The windows and states are held twice: ``windows`` / ``states`` are the
    committed ones, ``windows_next`` / ``states_next`` the spare that a tree
    commit writes (it reads the committed state and the accepted path).
    ``flip()`` makes the spare the committed state. A verify step that is not
    kept (``commit=False``) therefore leaves the state it started from
    untouched and can be replayed as it is."""

    def __init__(self, cfg, capacity: int, device="cuda", page_order: torch.Tensor | None = None):
        self.cfg = cfg
        self.attn_layers = cfg.attention_layers
        self.gdn_layers = cfg.linear_layers
        self.kv = PagedKVCache(len(self.attn_layers), cfg.num_key_value_heads, cfg.head_dim, capacity,
                               device=device, page_order=page_order)
        dev = torch.device(device)
        nG = len(self.gdn_layers)
        self._windows = torch.zeros(2, nG, cfg.linear_conv_kernel_dim - 1, cfg.conv_dim, dtype=torch.float32,
                                    device=dev)
        self._states = torch.zeros(2, nG, cfg.linear_num_value_heads, cfg.linear_value_head_dim,
                                   cfg.linear_key_head_dim, dtype=torch.float32, device=dev)
        self.parity = 0
        self.slot = {li: i for i, li in enumerate(self.attn_layers)}
        self.slot.update({li: i for i, li in enumerate(self.gdn_layers)})

    @property
    def windows(self) -> torch.Tensor:
        """Committed conv windows [nG, K - 1, conv_dim]."""
        return self._windows[self.parity]

    @property
    def states(self) -> torch.Tensor:
        """Committed recurrent states [nG, Hv, Dv, Dk]."""
        return self._states[self.parity]

    @property
    def windows_next(self) -> torch.Tensor:
        return self._windows[1 - self.parity]

    @property
    def states_next(self) -> torch.Tensor:
        return self._states[1 - self.parity]

    def flip(self) -> None:
        """Keep the last commit: its output becomes the committed state."""
        self.parity = 1 - self.parity

    @property
    def offset(self) -> int:
        return self.kv.offset

    @offset.setter
    def offset(self, v: int) -> None:
        self.kv.offset = v

    @property
    def capacity(self) -> int:
        return self.kv.capacity

    def reset(self, offset: int = 0) -> None:
        self.kv.offset = offset
        if offset == 0:
            self._windows.zero_()
            self._states.zero_()
