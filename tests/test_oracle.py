"""Pins for the CPU oracle (oracle/qwen3.py): closed forms, special cases and
an independent library implementation (transformers' Qwen3), so that a dropped
term, wrong sign / index or transposed operand in the oracle fails here. CPU only."""
import numpy as np
import pytest
import torch

from oracle import qwen3 as oq
from oracle import tree as otree


def test_bf16_roundtrip_and_rounding():
    x = np.array([1.0, -2.5, 3.140625, 1e-3, 65504.0, 1.00390625, 1.01171875], dtype=np.float32)
    bits = oq.f32_to_bf16_bits(x)
    back = oq.bf16_to_f32(bits)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(back, ref)  # round-to-nearest-even as torch


def test_rms_norm_closed_form():
    g = np.random.default_rng(0)
    x = g.standard_normal((3, 64)).astype(np.float32)
    w = g.standard_normal(64).astype(np.float32)
    y = oq.rms_norm(x, w, 1e-6)
    ref = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-6)
    # scale invariance (up to eps)
    np.testing.assert_allclose(oq.rms_norm(7.0 * x, w, 0.0), oq.rms_norm(x, w, 0.0), rtol=1e-5, atol=1e-6)


def test_rope_is_complex_rotation():
    g = np.random.default_rng(1)
    L, H, D = 5, 3, 16
    x = g.standard_normal((L, H, D)).astype(np.float32)
    pos = np.array([0, 1, 7, 1000, 123456])
    y = oq.rope(x, pos, 1e6)
    z = x[..., : D // 2].astype(np.float64) + 1j * x[..., D // 2:].astype(np.float64)
    ang = pos[:, None, None] * (1e6 ** (-np.arange(D // 2) / (D // 2)))[None, None, :]
    zr = z * np.exp(1j * ang)
    np.testing.assert_allclose(y[..., : D // 2], zr.real, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(y[..., D // 2:], zr.imag, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(y[0], x[0])  # position 0 is the identity
    # relative-position property: <rope(q,m), rope(k,n)> depends on m - n only
    q, k = x[0:1, 0:1], x[1:2, 0:1]
    a = (oq.rope(q, np.array([10]), 1e4) * oq.rope(k, np.array([3]), 1e4)).sum()
    b = (oq.rope(q, np.array([107]), 1e4) * oq.rope(k, np.array([100]), 1e4)).sum()
    np.testing.assert_allclose(a, b, rtol=1e-4)


def _naive_attention(q, k, v, visible):
    """Per-(head, query) loops in fp64 with explicit KV-head repetition."""
    L, Hq, D = q.shape
    Hkv = k.shape[1]
    krep = np.repeat(k, Hq // Hkv, axis=1).astype(np.float64)
    vrep = np.repeat(v, Hq // Hkv, axis=1).astype(np.float64)
    out = np.zeros((L, Hq, v.shape[-1]))
    for h in range(Hq):
        for i in range(L):
            idx = [j for j in range(k.shape[0]) if visible(i, j)]
            s = np.array([q[i, h] @ krep[j, h] for j in idx]) / np.sqrt(D)
            p = np.exp(s - s.max())
            p /= p.sum()
            out[i, h] = (p[:, None] * vrep[idx, h]).sum(0)
    return out


@pytest.mark.parametrize("shape", ["chain", "star", "decode", "random"])
def test_sdpa_tree_special_cases(shape):
    g = np.random.default_rng(2)
    P, Hq, Hkv, D = 9, 4, 2, 8
    L = 1 if shape == "decode" else 6
    if shape == "chain":
        parents = [-1] + list(range(L - 1))
    elif shape == "star":
        parents = [-1] + [0] * (L - 1)
    elif shape == "decode":
        parents = [-1]
    else:
        parents = [-1, 0, 0, 1, 3, 2]
    anc = [set() for _ in range(L)]
    for i in range(L):
        anc[i] = ({i} | anc[parents[i]]) if i else {0}
    q = g.standard_normal((L, Hq, D)).astype(np.float32)
    k = g.standard_normal((P + L, Hkv, D)).astype(np.float32)
    v = g.standard_normal((P + L, Hkv, D)).astype(np.float32)
    mask = np.zeros((L, P + L), bool)
    mask[:, :P] = True
    for i in range(L):
        for j in anc[i]:
            mask[i, P + j] = True
    got = oq.sdpa(q, k, v, mask, D ** -0.5)
    if shape == "chain":
        ref = _naive_attention(q, k, v, lambda i, j: j < P + i + 1)  # causal
    elif shape == "star":
        ref = _naive_attention(q, k, v, lambda i, j: j < P or j == P or j == P + i)
    else:
        ref = _naive_attention(q, k, v, lambda i, j: j < P or (j - P) in anc[i])
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


def _tiny_cfg():
    return oq.Qwen3Config(hidden=64, layers=2, ffn=96, heads=4, kv_heads=2, head_dim=16, vocab=50,
                          eps=1e-6, rope_base=1e6)


def _tiny_weights(cfg, seed=0):
    g = np.random.default_rng(seed)
    W = {}
    H, F, D = cfg.hidden, cfg.ffn, cfg.head_dim
    for li in range(cfg.layers):
        W[(li, "input_norm")] = (1 + 0.1 * g.standard_normal(H)).astype(np.float32)
        W[(li, "post_norm")] = (1 + 0.1 * g.standard_normal(H)).astype(np.float32)
        W[(li, "q_norm")] = (1 + 0.1 * g.standard_normal(D)).astype(np.float32)
        W[(li, "k_norm")] = (1 + 0.1 * g.standard_normal(D)).astype(np.float32)
        W[(li, "q")] = (0.1 * g.standard_normal((cfg.heads * D, H))).astype(np.float32)
        W[(li, "k")] = (0.1 * g.standard_normal((cfg.kv_heads * D, H))).astype(np.float32)
        W[(li, "v")] = (0.1 * g.standard_normal((cfg.kv_heads * D, H))).astype(np.float32)
        W[(li, "o")] = (0.1 * g.standard_normal((H, cfg.heads * D))).astype(np.float32)
        W[(li, "gate")] = (0.1 * g.standard_normal((F, H))).astype(np.float32)
        W[(li, "up")] = (0.1 * g.standard_normal((F, H))).astype(np.float32)
        W[(li, "down")] = (0.1 * g.standard_normal((H, F))).astype(np.float32)
    W[(None, "embed")] = g.standard_normal((cfg.vocab, H)).astype(np.float32)
    W[(None, "final_norm")] = (1 + 0.1 * g.standard_normal(H)).astype(np.float32)
    return W


def _empty_cache(cfg):
    c = oq.OracleCache()
    for _ in range(cfg.layers):
        c.keys.append(np.zeros((0, cfg.kv_heads, cfg.head_dim), np.float32))
        c.values.append(np.zeros((0, cfg.kv_heads, cfg.head_dim), np.float32))
    return c


def test_oracle_forward_matches_transformers_qwen3():
    """Chain tree over an empty cache == causal forward of transformers' Qwen3."""
    from transformers import Qwen3Config as HFConfig
    from transformers import Qwen3ForCausalLM

    cfg = _tiny_cfg()
    W = _tiny_weights(cfg)
    hf = HFConfig(vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.ffn,
                  num_hidden_layers=cfg.layers, num_attention_heads=cfg.heads, num_key_value_heads=cfg.kv_heads,
                  head_dim=cfg.head_dim, rms_norm_eps=cfg.eps, rope_theta=cfg.rope_base, tie_word_embeddings=True,
                  attention_bias=False, max_position_embeddings=4096)
    hf.rope_parameters = {"rope_type": "default", "rope_theta": cfg.rope_base}
    model = Qwen3ForCausalLM(hf).float().eval()
    sd = {}
    for li in range(cfg.layers):
        p = f"model.layers.{li}."
        sd[p + "input_layernorm.weight"] = W[(li, "input_norm")]
        sd[p + "post_attention_layernorm.weight"] = W[(li, "post_norm")]
        sd[p + "self_attn.q_norm.weight"] = W[(li, "q_norm")]
        sd[p + "self_attn.k_norm.weight"] = W[(li, "k_norm")]
        for n, m in (("q", "q_proj"), ("k", "k_proj"), ("v", "v_proj"), ("o", "o_proj")):
            sd[p + f"self_attn.{m}.weight"] = W[(li, n)]
        for n, m in (("gate", "gate_proj"), ("up", "up_proj"), ("down", "down_proj")):
            sd[p + f"mlp.{m}.weight"] = W[(li, n)]
    sd["model.embed_tokens.weight"] = W[(None, "embed")]
    sd["model.norm.weight"] = W[(None, "final_norm")]
    sd["lm_head.weight"] = W[(None, "embed")]
    model.load_state_dict({k: torch.from_numpy(v) for k, v in sd.items()}, strict=True)

    ids = np.array([3, 17, 5, 42, 8, 8, 1])
    with torch.no_grad():
        ref = model(torch.from_numpy(ids)[None]).logits[0].numpy()
    orc = oq.OracleQwen3(cfg, lambda li, n: W[(li, n)])
    L = len(ids)
    vis = np.tril(np.ones((L, L), bool))
    _, _, mask = otree.compile_tree(int(ids[0]), 0, ids[1:].tolist(), list(range(1, L)), vis, 0)
    norm, _, _, _ = orc.forward_tree(ids, np.arange(L), mask, _empty_cache(cfg))
    got = orc.lm_head_logits(norm)
    np.testing.assert_allclose(got, ref, rtol=2e-4, atol=2e-4)


def test_oracle_tree_equals_sequential_decode():
    """Verifying a chain tree on top of a prefix == decoding its tokens one by one."""
    cfg = _tiny_cfg()
    W = _tiny_weights(cfg, seed=3)
    orc = oq.OracleQwen3(cfg, lambda li, n: W[(li, n)])
    prefix = np.array([4, 9, 2])
    chain = np.array([7, 11, 13, 6])
    cache = _empty_cache(cfg)
    P = len(prefix)
    _, _, k, v = orc.forward_tree(prefix, np.arange(P), np.tril(np.ones((P, P), bool)), cache)
    cache.keys, cache.values = k, v
    L = len(chain)
    mask = np.ones((L, P + L), bool)
    mask[:, P:] = np.tril(np.ones((L, L), bool))
    tree_norm, _, _, _ = orc.forward_tree(chain, P + np.arange(L), mask, cache)
    seq = oq.OracleCache(keys=list(cache.keys), values=list(cache.values))
    for i, t in enumerate(chain):
        n1, _, k1, v1 = orc.forward_tree(np.array([t]), np.array([P + i]), np.ones((1, P + i + 1), bool), seq)
        np.testing.assert_allclose(n1[0], tree_norm[i], rtol=1e-4, atol=1e-4)
        seq.keys = [np.concatenate([a, b]) for a, b in zip(seq.keys, k1)]
        seq.values = [np.concatenate([a, b]) for a, b in zip(seq.values, v1)]


def test_argmax_first_index_on_ties():
    # tests/test_adapters.py:51-81: equal maxima at 0 and 70 -> 0
    lg = np.zeros((1, 128), np.float32)
    lg[0, 0] = lg[0, 70] = 1.0
    assert oq.argmax_first(lg)[0] == 0
    E = np.zeros((128, 64), np.float32)
    E[0] = E[70] = 1.0
    idx, top1, top2 = oq.chunked_argmax(np.ones((1, 64), np.float32), oq.f32_to_bf16_bits(E), chunk=64)
    assert idx[0] == 0 and top1[0] == top2[0] == 64.0


def test_compact_invariants():
    g = np.random.default_rng(5)
    P, L = 6, 7
    k = g.standard_normal((P + L, 2, 4)).astype(np.float32)
    keep = [0, 2, 3, 6]
    out = oq.compact(k, P, keep)
    assert out.shape[0] == P + len(keep)
    np.testing.assert_array_equal(out[:P], k[:P])
    for j, i in enumerate(keep):
        np.testing.assert_array_equal(out[P + j], k[P + i])
    assert oq.compact(k, P, []).shape[0] == P
