"""Oracle: Qwen3 tree-verify forward in fp32 numpy.

Test infrastructure only (see ``oracle/__init__.py``).

Restates (reference paths relative to the DrHB/dtree-mlx checkout):
- ``rms_norm``      <- mlx ``nn.RMSNorm`` / ``mx.fast.rms_norm`` as used by
  ``qwen3_tree.py:47, 54-59, 81``: ``x * rsqrt(mean(x^2) + eps) * w``.
- ``rope``          <- ``qwen3_tree.py:22-27`` (per-token offsets) with mlx
  ``nn.RoPE(traditional=False)``: half-split rotation, angle = pos * base^(-2i/D).
- ``sdpa``          <- ``qwen3_tree.py:69-76`` (mask True = attend, GQA head
  h reads KV head h // (Hq/Hkv), scale D^-0.5, softmax in fp32).
- ``layer_forward`` <- ``qwen3_tree.py:38-83`` (compiled tree block).
- ``forward_tree``  <- ``adapters.py:568-597``.
- ``lm_head_logits`` / ``argmax_first`` <- ``adapters.py:489-492, 114-118``
  (tied embedding, first index on ties).
- ``compact``       <- ``adapters.py:635-668``.

Weights are supplied as bf16 bit patterns (uint16) or fp32 arrays; bf16 is
widened exactly to fp32 before use, so the oracle computes "the reference MLX
path run in fp32" on the same weights as the device path.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    """Exact widening of bf16 bit patterns (uint16 / int16) to fp32."""
    if a.dtype == np.float32:
        return a
    u = a.view(np.uint16).astype(np.uint32) << 16
    return u.view(np.float32)


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u >> 16) & 1) + 0x7FFF
    return ((u + r) >> 16).astype(np.uint16)


def rms_norm(x: np.ndarray, w: np.ndarray | None, eps: float) -> np.ndarray:
    x = x.astype(np.float32)
    ms = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
    y = x * (1.0 / np.sqrt(ms + np.float32(eps))).astype(np.float32)
    return y if w is None else y * w.astype(np.float32)


def rope_cos_sin(pos: np.ndarray, dim: int, base: float) -> tuple[np.ndarray, np.ndarray]:
    half = dim // 2
    inv = base ** (-np.arange(0, half, dtype=np.float64) * 2.0 / dim)
    ang = pos.astype(np.float64)[:, None] * inv[None, :]
    return np.cos(ang), np.sin(ang)


def rope(x: np.ndarray, pos: np.ndarray, base: float) -> np.ndarray:
    """x: [L, H, D]; pos: [L]. Non-traditional (half-split) rotation."""
    D = x.shape[-1]
    half = D // 2
    c, s = rope_cos_sin(pos, D, base)
    c = c[:, None, :]
    s = s[:, None, :]
    x1 = x[..., :half].astype(np.float64)
    x2 = x[..., half:].astype(np.float64)
    out = np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=-1)
    return out.astype(np.float32)


def sdpa(q: np.ndarray, k: np.ndarray, v: np.ndarray, mask: np.ndarray, scale: float,
         dtype=np.float32) -> np.ndarray:
    """q [L, Hq, D], k/v [T, Hkv, D], mask [L, T] bool -> out [L, Hq, D]."""
    L, Hq, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    out = np.empty((L, Hq, v.shape[-1]), dtype=dtype)
    for h in range(Hq):
        kh = k[:, h // G, :].astype(dtype)
        vh = v[:, h // G, :].astype(dtype)
        s = (q[:, h, :].astype(dtype) @ kh.T) * dtype(scale)
        s = np.where(mask, s, -np.inf)
        m = s.max(axis=-1, keepdims=True)
        p = np.exp(s - m)
        p = p / p.sum(axis=-1, keepdims=True)
        out[:, h, :] = p @ vh
    return out


def silu(x: np.ndarray) -> np.ndarray:
    return x / (1.0 + np.exp(-x))


@dataclass
class Qwen3Config:
    hidden: int = 2560
    layers: int = 36
    ffn: int = 9728
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    vocab: int = 151936
    eps: float = 1e-6
    rope_base: float = 1_000_000.0


@dataclass
class OracleCache:
    """Per-layer fp32 K/V, [T, Hkv, D] in logical position order."""
    keys: list = field(default_factory=list)
    values: list = field(default_factory=list)

    @property
    def offset(self) -> int:
        return 0 if not self.keys else self.keys[0].shape[0]


class OracleQwen3:
    """fp32 forward over a weight accessor.

    ``weight(layer, name)`` returns an fp32 or bf16-bits array; names:
    input_norm, q, k, v, q_norm, k_norm, o, post_norm, gate, up, down
    (nn.Linear layout [out, in]); ``weight(None, name)`` for embed / final_norm.
    """

    def __init__(self, cfg: Qwen3Config, weight):
        self.cfg = cfg
        self._w = weight

    def w(self, layer, name):
        return bf16_to_f32(np.asarray(self._w(layer, name)))

    def embed(self, ids: np.ndarray) -> np.ndarray:
        E = self._w(None, "embed")
        return bf16_to_f32(np.asarray(E)[ids])

    def layer_forward(self, li: int, x: np.ndarray, k_prefix: np.ndarray, v_prefix: np.ndarray,
                      pos: np.ndarray, mask: np.ndarray):
        c = self.cfg
        L = x.shape[0]
        h = rms_norm(x, self.w(li, "input_norm"), c.eps)
        q = (h @ self.w(li, "q").T).reshape(L, c.heads, c.head_dim)
        k = (h @ self.w(li, "k").T).reshape(L, c.kv_heads, c.head_dim)
        v = (h @ self.w(li, "v").T).reshape(L, c.kv_heads, c.head_dim)
        q = rms_norm(q, self.w(li, "q_norm"), c.eps)
        k = rms_norm(k, self.w(li, "k_norm"), c.eps)
        q = rope(q, pos, c.rope_base)
        k = rope(k, pos, c.rope_base)
        K = np.concatenate([k_prefix, k], axis=0)
        V = np.concatenate([v_prefix, v], axis=0)
        a = sdpa(q, K, V, mask, c.head_dim ** -0.5).reshape(L, -1)
        x = x + a @ self.w(li, "o").T
        h = rms_norm(x, self.w(li, "post_norm"), c.eps)
        act = silu(h @ self.w(li, "gate").T) * (h @ self.w(li, "up").T)
        x = x + act @ self.w(li, "down").T
        return x.astype(np.float32), k, v

    def forward_tree(self, ids: np.ndarray, pos: np.ndarray, mask: np.ndarray,
                     cache: OracleCache, layer_ids=(), layers: int | None = None):
        """Returns (norm_hidden [L,H], verifier_hidden [L, n*H], new K list, new V list).
        Cache is not modified; the caller appends / compacts."""
        c = self.cfg
        nl = c.layers if layers is None else layers
        x = self.embed(ids)
        sel = []
        new_k, new_v = [], []
        want = set(layer_ids)
        for li in range(nl):
            x, k, v = self.layer_forward(li, x, cache.keys[li], cache.values[li], pos, mask)
            new_k.append(k)
            new_v.append(v)
            if li in want:
                sel.append(x)
        norm = rms_norm(x, self.w(None, "final_norm"), c.eps)
        vh = np.concatenate(sel, axis=-1) if sel else np.zeros((x.shape[0], 0), np.float32)
        return norm, vh, new_k, new_v

    def lm_head_logits(self, h: np.ndarray, rows: slice | None = None) -> np.ndarray:
        E = np.asarray(self._w(None, "embed"))
        if rows is not None:
            E = E[rows]
        return h.astype(np.float32) @ bf16_to_f32(E).T


def argmax_first(logits: np.ndarray) -> np.ndarray:
    """First index on ties (numpy argmax semantics; adapters.py:78-81)."""
    return np.argmax(logits, axis=-1)


def chunked_argmax(h: np.ndarray, E_bf16: np.ndarray, chunk: int = 16384):
    """Argmax of h @ E^T over the vocab in chunks; returns (idx, top1, top2)."""
    L = h.shape[0]
    best = np.full(L, -np.inf, np.float32)
    second = np.full(L, -np.inf, np.float32)
    idx = np.zeros(L, np.int64)
    for s in range(0, E_bf16.shape[0], chunk):
        lg = h.astype(np.float32) @ bf16_to_f32(E_bf16[s:s + chunk]).T
        i = np.argmax(lg, axis=-1)
        v = lg[np.arange(L), i]
        lg2 = lg.copy()
        lg2[np.arange(L), i] = -np.inf
        v2 = lg2.max(axis=-1)
        take = v > best
        second = np.where(take, np.maximum(best, v2), np.maximum(second, v))
        idx = np.where(take, i + s, idx)
        best = np.where(take, v, best)
    return idx, best, second


def compact(keys: np.ndarray, past_length: int, keep: list[int]) -> np.ndarray:
    """keys [T, ...] in logical order; rows [P, P+len(keep)) <- rows P+keep."""
    out = keys.copy()
    if not keep:
        return out[:past_length]
    rows = keys[[past_length + i for i in keep]]
    out[past_length:past_length + len(keep)] = rows
    return out[:past_length + len(keep)]
