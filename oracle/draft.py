"""Oracle: DFlash drafter forward in fp32 numpy.

Test infrastructure only (see ``oracle/__init__.py``).

Restates (reference paths relative to the DrHB/dtree-mlx checkout):
- ``KVCacheO``          <- mlx-lm ``KVCache`` as the drafter drives it:
  ``update_and_fetch`` writes at ``offset`` and returns every row up to the new
  offset (draft.py:206, 257), ``trim(n)`` drops the last ``min(n, offset)``
  rows (runtime.py:22-26 calls it after each draft block).
- ``ContextOnlyO``      <- ``ContextOnlyDraftKVCache`` (draft.py:67-110): the
  context rows only, trimmed to the first ``sink`` and the last ``window``
  rows after every append; ``trim`` is a no-op.
- ``OracleDraft.prepare_target_hidden`` <- draft.py:331-332
  (``hidden_norm(fc(target_hidden))``).
- ``OracleDraft.precompute_context_kv`` <- draft.py:186-206 and :334-346
  (k = RoPE(k_norm(k_proj(h))) at the cache offset, v = v_proj(h); no input
  norm on the context rows).
- ``OracleDraft.attention`` <- ``DFlashAttention.__call__`` (draft.py:208-272):
  queries and noise keys RoPE'd at the cache offset (or at the context length
  without a cache, context keys then at 0); keys = [context ; noise]; mask
  "causal" only for a KV cache / no cache with mask mode "causal" and more
  than one query, else none.
- ``OracleDraft.layer``   <- ``DFlashDecoderLayer.__call__`` (draft.py:285-305).
- ``OracleDraft.forward`` <- ``DFlashDraftModel.__call__`` (draft.py:349-364).

Pinned by: the reference test's cached-versus-uncached equality for both cache
modes and its trim/offset check (tests/test_draft.py:35-70), restated at
several context lengths and over consecutive blocks; the sink/window
invariants of the context-only cache (first ``sink`` rows kept, last
``window`` rows are the newest, against a position-tagged brute force); and
reductions to the already pinned Qwen3 oracle: a one-layer drafter whose fc
is the identity and whose hidden_norm weight is its input_layernorm weight
is, in mask mode "causal", a causal Qwen3 decoder layer over [context ;
block] (its block rows equal ``oracle.qwen3`` on that chain), and with an
empty context in mask mode "none" the stack is Qwen3 layers under an all-ones
mask. A planted mistake (no hidden_norm, context chunks roped from 0) fails.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .qwen3 import bf16_to_f32, rms_norm, rope, sdpa, silu


@dataclass
class DraftConfig:
    hidden: int
    layers: int
    ffn: int
    heads: int
    kv_heads: int
    head_dim: int
    eps: float
    rope_base: float
    n_target_layers: int
    block_size: int = 16


class KVCacheO:
    """mlx KVCache semantics for one layer (rows [T, Hkv, D])."""

    def __init__(self):
        self.keys = None
        self.values = None
        self.offset = 0

    def update_and_fetch(self, k: np.ndarray, v: np.ndarray):
        if self.keys is None:
            self.keys, self.values = k, v
        else:
            self.keys = np.concatenate([self.keys[: self.offset], k], axis=0)
            self.values = np.concatenate([self.values[: self.offset], v], axis=0)
        self.offset += k.shape[0]
        return self.keys[: self.offset], self.values[: self.offset]

    def trim(self, n: int) -> int:
        n = min(self.offset, int(n))
        self.offset -= n
        return n


class ContextOnlyO:
    """ContextOnlyDraftKVCache (draft.py:67-110) for one layer."""

    def __init__(self, sink_size: int = 64, window_size: int = 1024):
        self.sink_size = int(sink_size)
        self.window_size = int(window_size)
        self.keys = None
        self.values = None
        self.offset = 0

    def append_context(self, k: np.ndarray, v: np.ndarray, num_positions: int) -> None:
        if k is None or v is None or int(num_positions) <= 0:
            return
        if self.keys is None:
            self.keys, self.values = k, v
        else:
            self.keys = np.concatenate([self.keys, k], axis=0)
            self.values = np.concatenate([self.values, v], axis=0)
        self.offset += int(num_positions)
        n = self.keys.shape[0]
        if n > self.sink_size + self.window_size:
            keep = np.r_[0:self.sink_size, n - self.window_size:n]
            self.keys, self.values = self.keys[keep], self.values[keep]

    def fetch(self):
        return self.keys, self.values

    def trim(self, num_tokens: int) -> None:
        del num_tokens


class OracleDraft:
    """fp32 drafter forward over a weight accessor ``weight(layer, name)``:
    per-layer names as ``oracle.qwen3`` (input_norm, q, k, v, q_norm, k_norm,
    o, post_norm, gate, up, down) and ``weight(None, name)`` for fc,
    hidden_norm and norm."""

    def __init__(self, cfg: DraftConfig, weight):
        self.cfg = cfg
        self._w = weight
        self._memo: dict = {}
        self.mask_mode = "none"
        self.cache_mode = "kv"

    def w(self, layer, name):
        key = (layer, name)
        if key not in self._memo:
            self._memo[key] = bf16_to_f32(np.asarray(self._w(layer, name)))
        return self._memo[key]

    def make_cache(self):
        if self.cache_mode == "context-only":
            return [ContextOnlyO() for _ in range(self.cfg.layers)]
        return [KVCacheO() for _ in range(self.cfg.layers)]

    def prepare_target_hidden(self, th: np.ndarray) -> np.ndarray:
        return rms_norm(th.astype(np.float32) @ self.w(None, "fc").T, self.w(None, "hidden_norm"), self.cfg.eps)

    def _project_kv(self, li, h):
        c = self.cfg
        T = h.shape[0]
        k = rms_norm((h @ self.w(li, "k").T).reshape(T, c.kv_heads, c.head_dim), self.w(li, "k_norm"), c.eps)
        v = (h @ self.w(li, "v").T).reshape(T, c.kv_heads, c.head_dim).astype(np.float32)
        return k, v

    def precompute_context_kv(self, li, th, cache) -> None:
        T = th.shape[0]
        if cache is None or T <= 0:
            return
        k, v = self._project_kv(li, th)
        k = rope(k, cache.offset + np.arange(T), self.cfg.rope_base)
        if isinstance(cache, ContextOnlyO):
            cache.append_context(k, v, T)
        else:
            cache.update_and_fetch(k, v)

    def attention(self, li, h, th, cache):
        c = self.cfg
        Lq = h.shape[0]
        if cache is not None and th is not None:
            self.precompute_context_kv(li, th, cache)
            th = None
        q = rms_norm((h @ self.w(li, "q").T).reshape(Lq, c.heads, c.head_dim), self.w(li, "q_norm"), c.eps)
        nk, nv = self._project_kv(li, h)
        if cache is not None:
            off = cache.offset
            q = rope(q, off + np.arange(Lq), c.rope_base)
            nk = rope(nk, off + np.arange(Lq), c.rope_base)
            if isinstance(cache, ContextOnlyO):
                ck, cv = cache.fetch()
                if ck is None:
                    raise ValueError("Context-only draft cache is missing precomputed context.")
                K, V = np.concatenate([ck, nk], axis=0), np.concatenate([cv, nv], axis=0)
            else:
                K, V = cache.update_and_fetch(nk, nv)
        else:
            if th is None:
                raise ValueError("Draft attention requires target_hidden when cache is disabled.")
            T = th.shape[0]
            ck, cv = self._project_kv(li, th)
            q = rope(q, T + np.arange(Lq), c.rope_base)
            ck = rope(ck, np.arange(T), c.rope_base)
            nk = rope(nk, T + np.arange(Lq), c.rope_base)
            K, V = np.concatenate([ck, nk], axis=0), np.concatenate([cv, nv], axis=0)
        S = K.shape[0]
        mask = np.ones((Lq, S), bool)
        if not isinstance(cache, ContextOnlyO) and self.mask_mode == "causal" and Lq > 1:
            # mlx "causal" with more keys than queries: query i sees keys <= S - Lq + i
            mask = np.arange(S)[None, :] <= (S - Lq + np.arange(Lq))[:, None]
        a = sdpa(q, K, V, mask, c.head_dim ** -0.5).reshape(Lq, -1)
        return a @ self.w(li, "o").T

    def layer(self, li, x, th, cache):
        c = self.cfg
        h = rms_norm(x, self.w(li, "input_norm"), c.eps)
        x = x + self.attention(li, h, th, cache)
        h = rms_norm(x, self.w(li, "post_norm"), c.eps)
        x = x + (silu(h @ self.w(li, "gate").T) * (h @ self.w(li, "up").T)) @ self.w(li, "down").T
        return x.astype(np.float32)

    def forward(self, noise_embedding: np.ndarray, target_hidden: np.ndarray, cache=None,
                return_prenorm: bool = False):
        """noise_embedding [L, H], target_hidden [T, n_target_layers * H] -> [L, H]."""
        x = noise_embedding.astype(np.float32)
        th = self.prepare_target_hidden(target_hidden)
        if cache is None:
            caches = [None] * self.cfg.layers
        else:
            caches = cache
            for li, lc in enumerate(caches):
                if lc is not None:
                    self.precompute_context_kv(li, th, lc)
        for li, lc in enumerate(caches):
            x = self.layer(li, x, None if lc is not None else th, lc)
        out = rms_norm(x, self.w(None, "norm"), self.cfg.eps)
        return (out, x) if return_prenorm else out
