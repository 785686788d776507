"""Pins of the drafter oracle (oracle/draft.py) on the CPU.

* tests/test_draft.py:35-70 of the reference: the cached forward (both cache
  modes) equals the uncached one, and trimming the block leaves the context
  length as the offset; restated on its own tiny shape (hidden 8, 2 layers,
  2 heads of 4, block 4, two target layers, arange/100 inputs) and over
  consecutive blocks with growing context.
* The context-only cache's sink + window rule against position-tagged rows.
* A reduction to the pinned Qwen3 oracle: a one-layer drafter whose fc is the
  identity and whose hidden_norm equals its input_layernorm sees, in mask mode
  "causal", exactly a causal Qwen3 decoder layer over [context ; block]; with
  an empty context in mask mode "none" a Qwen3 layer under an all-ones mask.
"""
import numpy as np
import pytest

from oracle import draft as od
from oracle import qwen3 as oq


def _weights(cfg: od.DraftConfig, seed: int, identity_fc: bool = False):
    g = np.random.default_rng(seed)
    H, F, D = cfg.hidden, cfg.ffn, cfg.head_dim
    q, kv = cfg.heads * D, cfg.kv_heads * D
    W = {}
    for li in range(cfg.layers):
        for name, shape in (("q", (q, H)), ("k", (kv, H)), ("v", (kv, H)), ("o", (H, q)), ("gate", (F, H)),
                            ("up", (F, H)), ("down", (H, F))):
            W[(li, name)] = (g.standard_normal(shape) * 0.3).astype(np.float32)
        for name, n in (("input_norm", H), ("post_norm", H), ("q_norm", D), ("k_norm", D)):
            W[(li, name)] = (1 + 0.2 * g.standard_normal(n)).astype(np.float32)
    n_in = cfg.n_target_layers * H
    W[(None, "fc")] = np.eye(H, n_in, dtype=np.float32) if identity_fc else \
        (g.standard_normal((H, n_in)) * 0.3).astype(np.float32)
    W[(None, "hidden_norm")] = (1 + 0.2 * g.standard_normal(H)).astype(np.float32)
    W[(None, "norm")] = (1 + 0.2 * g.standard_normal(H)).astype(np.float32)
    return lambda layer, name: W[(layer, name)]


REF_CFG = od.DraftConfig(hidden=8, layers=2, ffn=16, heads=2, kv_heads=2, head_dim=4, eps=1e-6,
                         rope_base=10000.0, n_target_layers=2, block_size=4)


@pytest.mark.parametrize("cache_mode", ["kv", "context-only"])
def test_cached_matches_uncached_reference_shape(cache_mode):
    """tests/test_draft.py:35-70 restated."""
    cfg = REF_CFG
    d = od.OracleDraft(cfg, _weights(cfg, 0))
    d.cache_mode = cache_mode
    B, T = cfg.block_size, 2
    width = cfg.n_target_layers * cfg.hidden
    noise = np.arange(B * cfg.hidden, dtype=np.float32).reshape(B, cfg.hidden) / 100.0
    th = np.arange(T * width, dtype=np.float32).reshape(T, width) / 100.0
    unc = d.forward(noise, th)
    cache = d.make_cache()
    cached = d.forward(noise, th, cache=cache)
    np.testing.assert_allclose(cached, unc, atol=1e-5, rtol=1e-5)
    for lc in cache:
        lc.trim(B)
        assert lc.offset == T


@pytest.mark.parametrize("mask_mode", ["none", "causal"])
def test_cached_blocks_match_uncached_over_growing_context(mask_mode):
    """KV mode over consecutive blocks: after each block is trimmed, the next
    call sees exactly the concatenated context, as an uncached call does."""
    cfg = od.DraftConfig(hidden=16, layers=3, ffn=24, heads=4, kv_heads=2, head_dim=8, eps=1e-6,
                         rope_base=1e4, n_target_layers=3, block_size=5)
    d = od.OracleDraft(cfg, _weights(cfg, 1))
    d.mask_mode = mask_mode
    g = np.random.default_rng(2)
    width = cfg.n_target_layers * cfg.hidden
    cache = d.make_cache()
    ctx = np.zeros((0, width), np.float32)
    for T in (7, 1, 3):
        th = g.standard_normal((T, width)).astype(np.float32)
        noise = g.standard_normal((cfg.block_size, cfg.hidden)).astype(np.float32)
        ctx = np.concatenate([ctx, th], axis=0)
        got = d.forward(noise, th, cache=cache)
        ref = d.forward(noise, ctx)
        np.testing.assert_allclose(got, ref, atol=2e-5, rtol=2e-5)
        for lc in cache:
            lc.trim(cfg.block_size)
        assert all(lc.offset == ctx.shape[0] for lc in cache)


def test_context_only_cache_keeps_sink_and_newest_window():
    c = od.ContextOnlyO(sink_size=3, window_size=5)
    total = 0
    for n in (2, 4, 1, 6, 3, 9):
        tags = np.arange(total, total + n, dtype=np.float32)[:, None, None]
        c.append_context(tags, tags, n)
        total += n
        kept = c.keys[:, 0, 0].astype(int).tolist()
        want = list(range(total)) if total <= 8 else [0, 1, 2] + list(range(total - 5, total))
        assert kept == want and c.offset == total
    c.trim(4)
    assert c.offset == total  # trim is a no-op for the context-only cache


def _qwen3_oracle(cfg: od.DraftConfig, weight):
    qcfg = oq.Qwen3Config(hidden=cfg.hidden, layers=cfg.layers, ffn=cfg.ffn, heads=cfg.heads,
                          kv_heads=cfg.kv_heads, head_dim=cfg.head_dim, vocab=8, eps=cfg.eps,
                          rope_base=cfg.rope_base)
    return oq.OracleQwen3(qcfg, weight)


def test_one_layer_causal_drafter_is_a_qwen3_layer_over_context_and_block():
    cfg = od.DraftConfig(hidden=32, layers=1, ffn=48, heads=4, kv_heads=2, head_dim=8, eps=1e-6,
                         rope_base=1e4, n_target_layers=1, block_size=6)
    base = _weights(cfg, 3, identity_fc=True)
    W = lambda layer, name: base(0, "input_norm") if (layer, name) == (None, "hidden_norm") else base(layer, name)
    d = od.OracleDraft(cfg, W)
    d.mask_mode = "causal"
    g = np.random.default_rng(4)
    T, B = 9, cfg.block_size
    ctx = g.standard_normal((T, cfg.hidden)).astype(np.float32)
    noise = g.standard_normal((B, cfg.hidden)).astype(np.float32)
    q3 = _qwen3_oracle(cfg, W)
    x = np.concatenate([ctx, noise], axis=0)
    empty = np.zeros((0, cfg.kv_heads, cfg.head_dim), np.float32)
    ref, _, _ = q3.layer_forward(0, x, empty, empty, np.arange(T + B), np.tril(np.ones((T + B, T + B), bool)))
    for cache in (None, d.make_cache()):
        out, pre = d.forward(noise, ctx, cache=cache, return_prenorm=True)
        np.testing.assert_allclose(pre, ref[T:], atol=2e-5, rtol=2e-5)
        np.testing.assert_allclose(out, oq.rms_norm(ref[T:], W(None, "norm"), cfg.eps), atol=2e-5, rtol=2e-5)


def test_empty_context_unmasked_drafter_is_qwen3_stack_under_full_mask():
    cfg = od.DraftConfig(hidden=32, layers=2, ffn=48, heads=4, kv_heads=1, head_dim=8, eps=1e-6,
                         rope_base=1e4, n_target_layers=2, block_size=5)
    W = _weights(cfg, 5)
    d = od.OracleDraft(cfg, W)
    g = np.random.default_rng(6)
    noise = g.standard_normal((cfg.block_size, cfg.hidden)).astype(np.float32)
    out, pre = d.forward(noise, np.zeros((0, 2 * cfg.hidden), np.float32), return_prenorm=True)
    q3 = _qwen3_oracle(cfg, W)
    empty = np.zeros((0, cfg.kv_heads, cfg.head_dim), np.float32)
    x = noise
    for li in range(cfg.layers):
        x, _, _ = q3.layer_forward(li, x, empty, empty, np.arange(cfg.block_size),
                                   np.ones((cfg.block_size, cfg.block_size), bool))
    np.testing.assert_allclose(pre, x, atol=2e-5, rtol=2e-5)


def test_planted_mistakes_fail_the_pins():
    """A drafter oracle without the hidden_norm, or one that ropes each
    appended context chunk from position 0, fails the checks above."""
    cfg = od.DraftConfig(hidden=32, layers=1, ffn=48, heads=4, kv_heads=2, head_dim=8, eps=1e-6,
                         rope_base=1e4, n_target_layers=1, block_size=6)
    base = _weights(cfg, 3, identity_fc=True)
    W = lambda layer, name: base(0, "input_norm") if (layer, name) == (None, "hidden_norm") else base(layer, name)
    g = np.random.default_rng(4)
    T, B = 9, cfg.block_size
    ctx = g.standard_normal((T, cfg.hidden)).astype(np.float32)
    noise = g.standard_normal((B, cfg.hidden)).astype(np.float32)
    q3 = _qwen3_oracle(cfg, W)
    empty = np.zeros((0, cfg.kv_heads, cfg.head_dim), np.float32)
    ref, _, _ = q3.layer_forward(0, np.concatenate([ctx, noise]), empty, empty, np.arange(T + B),
                                 np.tril(np.ones((T + B, T + B), bool)))

    class WrongOffset(od.OracleDraft):
        def precompute_context_kv(self, li, th, cache):  # context keys roped from 0 on every append
            k, v = self._project_kv(li, th)
            cache.update_and_fetch(oq.rope(k, np.arange(th.shape[0]), self.cfg.rope_base), v)

    class NoHiddenNorm(od.OracleDraft):
        def prepare_target_hidden(self, th):
            return th @ self.w(None, "fc").T

    for bad_cls in (NoHiddenNorm,):
        bad = bad_cls(cfg, W)
        bad.mask_mode = "causal"
        _, pre = bad.forward(noise, ctx, cache=bad.make_cache(), return_prenorm=True)
        assert not np.allclose(pre, ref[T:], atol=2e-5, rtol=2e-5)
    # context chunks roped from 0 break cached == uncached over two appends
    bad = WrongOffset(cfg, W)
    c1 = bad.make_cache()
    bad.forward(noise, ctx[:4], cache=c1)
    for lc in c1:
        lc.trim(B)
    got = bad.forward(noise, ctx[4:], cache=c1)
    good = od.OracleDraft(cfg, W).forward(noise, ctx)
    assert not np.allclose(got, good, atol=2e-5, rtol=2e-5)
