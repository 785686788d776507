"""Oracle: Qwen3.5 hybrid (GatedDeltaNet + gated full attention) tree-verify
forward and path commit, in fp32 numpy (GDN recurrence in float64).

Test infrastructure only (see ``oracle/__init__.py``).

Restates (reference paths relative to the DrHB/dtree-mlx checkout):
- ``gdn_layer``   <- ``_forward_linear_tree_batched{,_kernel}``
  (qwen35_tree.py:180-327, 329-480): in_proj_qkv / z / b / a, tree conv1d +
  SiLU (conv weight [K, C] = conv1d.weight[:, :, 0].T, qwen35_tree.py:358),
  split q | k | v (key_dim, key_dim, value_dim), q = Dk^-1 rms_norm(q),
  k = Dk^-1/2 rms_norm(k) (eps 1e-6, qwen35_tree.py:304-306),
  g = exp(-exp(A_log) softplus(a + dt_bias)) (mlx-lm 0.31.2
  gated_delta.compute_g, called at qwen35_tree.py:307), beta = sigmoid(b),
  tree recurrence (oracle/gdn.py), RMSNormGated(y, z) = rms_norm(y) * w *
  silu(z) per value head (mlx-lm Qwen3NextRMSNormGated, used at
  qwen35_tree.py:322), out_proj, residual, post-norm MLP.
- ``attn_layer``  <- ``forward_full_attention_tree_block``
  (qwen35_tree.py:552-626): q_proj output per head = [q (D) | gate (D)]
  (:578-584), q_norm / k_norm (RMSNorm over D), partial RoPE on the first
  ``rope_dims`` dims (mlx-lm Qwen3NextAttention: nn.RoPE(D * partial_rotary_factor,
  traditional=False)), masked SDPA with scale D^-0.5
  (qwen35_target.py:428-493: every branch is exact SDPA), o_proj(out *
  sigmoid(gate)) (:613), residual, post-norm MLP.
- ``forward_tree`` <- ``forward_qwen35_tree_with_hidden_states``
  (qwen35_tree.py:629-705): layer i is full attention when
  (i + 1) % full_attention_interval == 0 (custom_qwen35_model.py:896); the
  cache is left untouched and the per-node results are returned as pending.
- ``commit``      <- ``commit_qwen35_tree_path`` (qwen35_tree.py:708-732):
  attention layers append K/V of the accepted nodes; GDN layers take the conv
  window and state of the last accepted node (replayed along the path here,
  which equals the tree's node state by the path decomposition of the tree).

Pinned (tests/test_oracle_qwen35.py) against transformers' Qwen3.5 text
model (an independent implementation of the same architecture): chain trees
equal its causal forward, every tree node equals its forward over the prefix
plus that node's root path, and commit followed by a second step equals one
forward over the concatenated tokens.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import gdn
from .qwen3 import bf16_to_f32, rms_norm, sdpa, silu


@dataclass
class Qwen35Config:
    hidden: int = 2560
    layers: int = 32
    ffn: int = 9216
    heads: int = 16
    kv_heads: int = 4
    head_dim: int = 256
    rope_dims: int = 64
    lin_k_heads: int = 16
    lin_v_heads: int = 32
    lin_k_dim: int = 128
    lin_v_dim: int = 128
    conv_kernel: int = 4
    full_attention_interval: int = 4
    vocab: int = 151936
    eps: float = 1e-6
    rope_base: float = 100_000.0

    @property
    def key_dim(self) -> int:
        return self.lin_k_heads * self.lin_k_dim

    @property
    def value_dim(self) -> int:
        return self.lin_v_heads * self.lin_v_dim

    @property
    def conv_dim(self) -> int:
        return 2 * self.key_dim + self.value_dim

    def is_linear(self, li: int) -> bool:
        return (li + 1) % self.full_attention_interval != 0


def softplus(x):
    return np.logaddexp(0.0, x)


def partial_rope(x: np.ndarray, pos: np.ndarray, dims: int, base: float) -> np.ndarray:
    """Non-traditional RoPE on the first `dims` dims of x [L, H, D] (pairs
    (j, j + dims/2)); the remaining dims pass through."""
    half = dims // 2
    inv = base ** (-np.arange(0, half, dtype=np.float64) * 2.0 / dims)
    ang = pos.astype(np.float64)[:, None] * inv[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    x1 = x[..., :half].astype(np.float64)
    x2 = x[..., half:dims].astype(np.float64)
    rot = np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=-1)
    return np.concatenate([rot, x[..., dims:].astype(np.float64)], axis=-1).astype(np.float32)


def tree_mask(parents, past: int) -> np.ndarray:
    """[L, past + L] bool: every prefix column, then ancestor-or-self columns."""
    L = len(parents)
    anc = np.zeros((L, L), bool)
    for t in range(L):
        p = int(parents[t])
        if p >= 0:
            anc[t] = anc[p]
        anc[t, t] = True
    return np.concatenate([np.ones((L, past), bool), anc], axis=1)


@dataclass
class Qwen35Cache:
    """Committed state: per layer either (keys, values) [T, Hkv, D] fp32 for
    attention layers or (window [keep, C], state [Hv, Dv, Dk]) for GDN layers."""
    layers: list = field(default_factory=list)
    offset: int = 0


class OracleQwen35:
    """fp32 forward over a weight accessor ``weight(layer, name)`` returning
    bf16 bit patterns or fp32 arrays (nn.Linear [out, in] layout).

    Global names: embed, final_norm. GDN layers: input_norm, in_qkv, in_z,
    in_b, in_a, conv ([K, C]), A_log, dt_bias, gnorm ([Dv]), out, post_norm,
    gate, up, down. Attention layers: input_norm, q ([Hq * 2D, H], per head
    q | gate), k, v, q_norm, k_norm, o, post_norm, gate, up, down.
    """

    def __init__(self, cfg: Qwen35Config, weight):
        self.cfg = cfg
        self._w = weight

    def w(self, layer, name):
        return bf16_to_f32(np.asarray(self._w(layer, name)))

    def new_cache(self) -> Qwen35Cache:
        c = self.cfg
        layers = []
        for li in range(c.layers):
            if c.is_linear(li):
                layers.append((np.zeros((c.conv_kernel - 1, c.conv_dim), np.float32),
                               np.zeros((c.lin_v_heads, c.lin_v_dim, c.lin_k_dim), np.float64)))
            else:
                layers.append((np.zeros((0, c.kv_heads, c.head_dim), np.float32),
                               np.zeros((0, c.kv_heads, c.head_dim), np.float32)))
        return Qwen35Cache(layers=layers, offset=0)

    def mlp(self, li, x):
        c = self.cfg
        h = rms_norm(x, self.w(li, "post_norm"), c.eps)
        act = silu(h @ self.w(li, "gate").T) * (h @ self.w(li, "up").T)
        return (x + act @ self.w(li, "down").T).astype(np.float32)

    def gdn_prep(self, li, x):
        """Input norm + projections + the q/k/v/g/beta of qwen35_tree.py:304-308
        before the conv (returns the conv input, z, a, b)."""
        c = self.cfg
        h = rms_norm(x, self.w(li, "input_norm"), c.eps)
        return h @ self.w(li, "in_qkv").T, h @ self.w(li, "in_z").T, h @ self.w(li, "in_a").T, h @ self.w(li, "in_b").T

    def gdn_inputs(self, li, conv_out, a, b):
        """conv output [T, C], a/b [T, Hv] -> q, k [T, Hk, Dk], v [T, Hv, Dv], g, beta [T, Hv]."""
        c = self.cfg
        T = conv_out.shape[0]
        kd = c.key_dim
        q = conv_out[:, :kd].reshape(T, c.lin_k_heads, c.lin_k_dim)
        k = conv_out[:, kd:2 * kd].reshape(T, c.lin_k_heads, c.lin_k_dim)
        v = conv_out[:, 2 * kd:].reshape(T, c.lin_v_heads, c.lin_v_dim)
        inv = c.lin_k_dim ** -0.5

        def rms(t):
            t = np.asarray(t, np.float64)
            return t / np.sqrt((t * t).mean(-1, keepdims=True) + 1e-6)

        q = inv * inv * rms(q)
        k = inv * rms(k)
        A_log = np.asarray(self._w(li, "A_log"), np.float64)
        dt_bias = np.asarray(self._w(li, "dt_bias"), np.float64)
        g = np.exp(-np.exp(A_log)[None, :] * softplus(np.asarray(a, np.float64) + dt_bias[None, :]))
        beta = 1.0 / (1.0 + np.exp(-np.asarray(b, np.float64)))
        return q, k, np.asarray(v, np.float64), g, beta

    def gated_norm(self, li, y, z):
        """RMSNormGated per value head: rms_norm(y) * w * silu(z); y, z [T, Hv, Dv]."""
        c = self.cfg
        w = self.w(li, "gnorm").astype(np.float64)
        y = np.asarray(y, np.float64)
        yn = y / np.sqrt((y * y).mean(-1, keepdims=True) + c.eps) * w
        z = np.asarray(z, np.float64)
        return (yn * (z / (1.0 + np.exp(-z)))).astype(np.float32)

    def gdn_layer(self, li, x, window, state, parents):
        c = self.cfg
        T = x.shape[0]
        xin, z, a, b = self.gdn_prep(li, x)
        conv_w = np.asarray(self.w(li, "conv"), np.float64)
        conv_out, _ = gdn.tree_conv1d(xin, window, conv_w, parents)
        q, k, v, g, beta = self.gdn_inputs(li, conv_out, a, b)
        y, _ = gdn.tree_gated_delta(q, k, v, g, beta, state, parents)
        o = self.gated_norm(li, y, z.reshape(T, c.lin_v_heads, c.lin_v_dim)).reshape(T, -1)
        x = x + o @ self.w(li, "out").T
        pending = dict(kind="gdn", x=xin.astype(np.float32), q=q, k=k, v=v, g=g, beta=beta)
        return self.mlp(li, x), pending

    def attn_layer(self, li, x, keys, values, pos, mask):
        c = self.cfg
        L = x.shape[0]
        D = c.head_dim
        h = rms_norm(x, self.w(li, "input_norm"), c.eps)
        qg = (h @ self.w(li, "q").T).reshape(L, c.heads, 2 * D)
        q, gate = qg[..., :D], qg[..., D:].reshape(L, c.heads * D)
        k = (h @ self.w(li, "k").T).reshape(L, c.kv_heads, D)
        v = (h @ self.w(li, "v").T).reshape(L, c.kv_heads, D)
        q = partial_rope(rms_norm(q, self.w(li, "q_norm"), c.eps), pos, c.rope_dims, c.rope_base)
        k = partial_rope(rms_norm(k, self.w(li, "k_norm"), c.eps), pos, c.rope_dims, c.rope_base)
        K = np.concatenate([keys, k], axis=0)
        V = np.concatenate([values, v.astype(np.float32)], axis=0)
        a = sdpa(q, K, V, mask, D ** -0.5).reshape(L, -1)
        a = a * (1.0 / (1.0 + np.exp(-gate)))
        x = x + a @ self.w(li, "o").T
        pending = dict(kind="attn", k=k, v=v.astype(np.float32))
        return self.mlp(li, x), pending

    def embed(self, ids):
        return bf16_to_f32(np.asarray(self._w(None, "embed"))[np.asarray(ids)])

    def forward_tree(self, ids, pos, parents, cache: Qwen35Cache, layer_ids=(), layers: int | None = None):
        """Returns (norm_hidden [L, H], verifier_hidden [L, n * H], pending list).
        The cache is not modified (qwen35_tree.py:629-705)."""
        c = self.cfg
        nl = c.layers if layers is None else layers
        pos = np.asarray(pos)
        mask = tree_mask(parents, cache.offset)
        x = self.embed(ids)
        sel, pending = [], []
        want = set(layer_ids)
        for li in range(nl):
            a, b = cache.layers[li]
            if c.is_linear(li):
                x, pend = self.gdn_layer(li, x, a, b, parents)
            else:
                x, pend = self.attn_layer(li, x, a, b, pos, mask)
            pending.append(pend)
            if li in want:
                sel.append(x)
        norm = rms_norm(x, self.w(None, "final_norm"), c.eps)
        vh = np.concatenate(sel, axis=-1) if sel else np.zeros((x.shape[0], 0), np.float32)
        return norm, vh, pending

    def chain_prefill(self, ids, layers: int):
        """The first `layers` layers over a causal chain of prompt tokens from
        an empty cache, committing all of it: forward_tree + commit of the whole
        chain, with the chain forms of the conv and the recurrence (no per-node
        states kept, so long prompts fit). Returns (x after those layers, the
        committed cache of those layers: (window, state) or (keys, values))."""
        c = self.cfg
        ids = np.asarray(ids)
        T = len(ids)
        pos = np.arange(T)
        x = self.embed(ids)
        out = []
        for li in range(layers):
            if c.is_linear(li):
                xin, z, a, b = self.gdn_prep(li, x)
                conv_out, win = gdn.chain_conv1d(xin, np.zeros((c.conv_kernel - 1, c.conv_dim)),
                                                 np.asarray(self.w(li, "conv"), np.float64))
                q, k, v, g, beta = self.gdn_inputs(li, conv_out, a, b)
                y, state = gdn.chain_gated_delta(q, k, v, g, beta,
                                                 np.zeros((c.lin_v_heads, c.lin_v_dim, c.lin_k_dim)))
                o = self.gated_norm(li, y, z.reshape(T, c.lin_v_heads, c.lin_v_dim)).reshape(T, -1)
                x = self.mlp(li, x + o @ self.w(li, "out").T)
                out.append((win.astype(np.float32), state))
            else:
                empty = np.zeros((0, c.kv_heads, c.head_dim), np.float32)
                x, pend = self.attn_layer(li, x, empty, empty, pos, np.tril(np.ones((T, T), bool)))
                out.append((pend["k"], pend["v"]))
        return x, out

    def commit(self, cache: Qwen35Cache, pending: list, parents, accepted) -> None:
        """commit_qwen35_tree_path: accepted = root path (accepted[0] = 0)."""
        if not accepted:
            return
        acc = list(accepted)
        for li, pend in enumerate(pending):
            a, b = cache.layers[li]
            if pend["kind"] == "attn":
                cache.layers[li] = (np.concatenate([a, pend["k"][acc]], axis=0),
                                    np.concatenate([b, pend["v"][acc]], axis=0))
            else:
                win, st = gdn.commit(pend["x"], a, pend["q"], pend["k"], pend["v"], pend["g"], pend["beta"], b,
                                     parents, acc)
                cache.layers[li] = (win.astype(np.float32), st)
        cache.offset += len(acc)

    def lm_head_logits(self, h):
        return h.astype(np.float32) @ self.w(None, "embed").T
