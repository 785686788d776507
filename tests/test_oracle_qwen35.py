"""Pins of the Qwen3.5 hybrid oracle (oracle/qwen35.py) against transformers'
Qwen3.5 text model, an independent implementation of the same architecture
(GatedDeltaNet with l2-normalised q/k and a chunked delta rule, gated
attention with partial RoPE, (1 + w) RMSNorm weights).

Weight mapping: transformers' RMSNorm weights are the oracle's minus 1; its
conv1d weight [C, 1, K] is the oracle's [K, C] transposed. Its l2norm puts
eps inside the sum, the reference's rms_norm * d^-1/2 puts d * eps there: a
relative difference below 1e-6 at these magnitudes.

Checks:
* a chain tree with an empty cache equals the causal forward;
* after a committed prefix, every node of a branching tree equals the causal
  forward over prefix + the node's root path (the path decomposition of the
  tree, checked against an implementation that knows nothing of trees);
* commit of an accepted path followed by a second step equals one causal
  forward over prefix + accepted tokens + the new tokens (conv window, delta
  state and KV append of the commit).
"""
import numpy as np
import pytest
import torch

from oracle import gdn
from oracle.qwen3 import f32_to_bf16_bits, bf16_to_f32
from oracle.qwen35 import OracleQwen35, Qwen35Config

transformers = pytest.importorskip("transformers")
from transformers.models.qwen3_5 import modeling_qwen3_5 as M  # noqa: E402
from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig  # noqa: E402

CFG = Qwen35Config(hidden=256, layers=4, ffn=512, heads=4, kv_heads=2, head_dim=64, rope_dims=16,
                   lin_k_heads=2, lin_v_heads=4, lin_k_dim=32, lin_v_dim=32, conv_kernel=4, vocab=512,
                   rope_base=100_000.0)


def _bf(a):
    return bf16_to_f32(f32_to_bf16_bits(np.asarray(a, np.float32)))


def _weights(cfg: Qwen35Config, seed=0):
    g = np.random.default_rng(seed)
    H, F = cfg.hidden, cfg.ffn
    W = {(None, "embed"): _bf(g.normal(0, 0.5, (cfg.vocab, H))),
         (None, "final_norm"): _bf(1 + g.normal(0, 0.1, H))}

    def lin(n, k, s=0.06):
        return _bf(g.normal(0, s, (n, k)))

    for li in range(cfg.layers):
        W[li, "input_norm"] = _bf(1 + g.normal(0, 0.1, H))
        W[li, "post_norm"] = _bf(1 + g.normal(0, 0.1, H))
        W[li, "gate"], W[li, "up"], W[li, "down"] = lin(F, H), lin(F, H), lin(H, F, 0.04)
        if cfg.is_linear(li):
            W[li, "in_qkv"] = lin(cfg.conv_dim, H)
            W[li, "in_z"] = lin(cfg.value_dim, H)
            W[li, "in_b"] = lin(cfg.lin_v_heads, H, 0.2)
            W[li, "in_a"] = lin(cfg.lin_v_heads, H, 0.2)
            W[li, "conv"] = _bf(g.uniform(-0.5, 0.5, (cfg.conv_kernel, cfg.conv_dim)))
            W[li, "A_log"] = np.log(g.uniform(0.5, 16, cfg.lin_v_heads)).astype(np.float32)
            W[li, "dt_bias"] = (1 + g.normal(0, 0.2, cfg.lin_v_heads)).astype(np.float32)
            W[li, "gnorm"] = _bf(1 + g.normal(0, 0.1, cfg.lin_v_dim))
            W[li, "out"] = lin(H, cfg.value_dim)
        else:
            D = cfg.head_dim
            W[li, "q"] = lin(cfg.heads * 2 * D, H)
            W[li, "k"] = lin(cfg.kv_heads * D, H)
            W[li, "v"] = lin(cfg.kv_heads * D, H)
            W[li, "q_norm"] = _bf(1 + g.normal(0, 0.1, D))
            W[li, "k_norm"] = _bf(1 + g.normal(0, 0.1, D))
            W[li, "o"] = lin(H, cfg.heads * D)
    return W


def _hf_model(cfg: Qwen35Config, W):
    hc = Qwen3_5TextConfig(
        vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.ffn, num_hidden_layers=cfg.layers,
        num_attention_heads=cfg.heads, num_key_value_heads=cfg.kv_heads, head_dim=cfg.head_dim,
        linear_key_head_dim=cfg.lin_k_dim, linear_value_head_dim=cfg.lin_v_dim,
        linear_num_key_heads=cfg.lin_k_heads, linear_num_value_heads=cfg.lin_v_heads,
        linear_conv_kernel_dim=cfg.conv_kernel, tie_word_embeddings=True, rms_norm_eps=cfg.eps,
        rope_parameters={"rope_type": "default", "rope_theta": cfg.rope_base,
                         "partial_rotary_factor": cfg.rope_dims / cfg.head_dim,
                         "mrope_section": [cfg.rope_dims // 4, cfg.rope_dims // 8, cfg.rope_dims // 8]})
    hc._attn_implementation = "eager"
    m = M.Qwen3_5ForCausalLM(hc).eval()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32))  # noqa: E731
    sd = {"model.embed_tokens.weight": t(W[None, "embed"]), "model.norm.weight": t(W[None, "final_norm"] - 1),
          "lm_head.weight": t(W[None, "embed"])}
    for li in range(cfg.layers):
        p = f"model.layers.{li}."
        sd[p + "input_layernorm.weight"] = t(W[li, "input_norm"] - 1)
        sd[p + "post_attention_layernorm.weight"] = t(W[li, "post_norm"] - 1)
        sd[p + "mlp.gate_proj.weight"] = t(W[li, "gate"])
        sd[p + "mlp.up_proj.weight"] = t(W[li, "up"])
        sd[p + "mlp.down_proj.weight"] = t(W[li, "down"])
        if cfg.is_linear(li):
            q = p + "linear_attn."
            sd[q + "in_proj_qkv.weight"] = t(W[li, "in_qkv"])
            sd[q + "in_proj_z.weight"] = t(W[li, "in_z"])
            sd[q + "in_proj_b.weight"] = t(W[li, "in_b"])
            sd[q + "in_proj_a.weight"] = t(W[li, "in_a"])
            sd[q + "conv1d.weight"] = t(W[li, "conv"].T[:, None, :])
            sd[q + "A_log"] = t(W[li, "A_log"])
            sd[q + "dt_bias"] = t(W[li, "dt_bias"])
            sd[q + "norm.weight"] = t(W[li, "gnorm"])
            sd[q + "out_proj.weight"] = t(W[li, "out"])
        else:
            q = p + "self_attn."
            for n, key in (("q", "q_proj"), ("k", "k_proj"), ("v", "v_proj"), ("o", "o_proj")):
                sd[q + key + ".weight"] = t(W[li, n])
            sd[q + "q_norm.weight"] = t(W[li, "q_norm"] - 1)
            sd[q + "k_norm.weight"] = t(W[li, "k_norm"] - 1)
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in k for k in missing), (missing, unexpected)
    return m


@pytest.fixture(scope="module")
def models():
    W = _weights(CFG)
    return OracleQwen35(CFG, lambda li, n: W[li, n]), _hf_model(CFG, W)


def _hf_hidden(m, tokens):
    with torch.no_grad():
        out = m.model(input_ids=torch.tensor([list(tokens)]), use_cache=False)
    return out.last_hidden_state[0].numpy()


def _close(a, b, tol=2e-4):
    err = np.abs(np.asarray(a, np.float64) - b).max()
    assert err <= tol * max(1.0, np.abs(b).max()), err


def test_chain_tree_equals_causal_forward(models):
    orc, hf = models
    toks = np.random.default_rng(1).integers(0, CFG.vocab, 12)
    cache = orc.new_cache()
    norm, _, _ = orc.forward_tree(toks, np.arange(12), [-1] + list(range(11)), cache)
    _close(norm, _hf_hidden(hf, toks))


PARENTS = [-1, 0, 0, 1, 1, 2, 4, 3]


def _prefixed(orc, n_prefix, seed):
    g = np.random.default_rng(seed)
    prefix = g.integers(0, CFG.vocab, n_prefix)
    cache = orc.new_cache()
    _, _, pend = orc.forward_tree(prefix, np.arange(n_prefix), [-1] + list(range(n_prefix - 1)), cache)
    orc.commit(cache, pend, [-1] + list(range(n_prefix - 1)), list(range(n_prefix)))
    return prefix, cache


def test_tree_nodes_equal_root_path_forwards(models):
    orc, hf = models
    prefix, cache = _prefixed(orc, 9, 2)
    toks = np.random.default_rng(3).integers(0, CFG.vocab, len(PARENTS))
    depth = [0] * len(PARENTS)
    for t in range(1, len(PARENTS)):
        depth[t] = depth[PARENTS[t]] + 1
    norm, _, _ = orc.forward_tree(toks, 9 + np.array(depth), PARENTS, cache)
    for t in range(len(PARENTS)):
        path = gdn.root_path(PARENTS, t)
        ref = _hf_hidden(hf, np.concatenate([prefix, toks[path]]))[-1]
        _close(norm[t], ref)


def test_commit_then_next_step_equals_one_forward(models):
    orc, hf = models
    prefix, cache = _prefixed(orc, 7, 4)
    toks = np.random.default_rng(5).integers(0, CFG.vocab, len(PARENTS))
    depth = [0] * len(PARENTS)
    for t in range(1, len(PARENTS)):
        depth[t] = depth[PARENTS[t]] + 1
    _, _, pend = orc.forward_tree(toks, 7 + np.array(depth), PARENTS, cache)
    accepted = [0, 1, 4, 6]
    orc.commit(cache, pend, PARENTS, accepted)
    assert cache.offset == 7 + len(accepted)
    nxt = np.random.default_rng(6).integers(0, CFG.vocab, 3)
    norm, _, _ = orc.forward_tree(nxt, cache.offset + np.arange(3), [-1, 0, 1], cache)
    ref = _hf_hidden(hf, np.concatenate([prefix, toks[accepted], nxt]))[-3:]
    _close(norm, ref)


def test_chain_prefill_equals_forward_and_commit(models):
    """chain_prefill (chain conv / recurrence, the form used for long prompts)
    == forward_tree over the chain + commit of every token: the hidden rows
    after the layers and every committed window, state, key and value."""
    orc, _ = models
    toks = np.random.default_rng(8).integers(0, CFG.vocab, 14)
    chain = [-1] + list(range(13))
    cache = orc.new_cache()
    _, _, pend = orc.forward_tree(toks, np.arange(14), chain, cache)
    orc.commit(cache, pend, chain, list(range(14)))
    x, layers = orc.chain_prefill(toks, CFG.layers)
    for li, (a, b) in enumerate(layers):
        _close(a, cache.layers[li][0], 1e-5)
        _close(b, cache.layers[li][1], 1e-5)
    # hidden rows: forward_tree's normalised output equals the final norm of x
    from oracle.qwen3 import rms_norm
    norm, _, _ = orc.forward_tree(toks, np.arange(14), chain, orc.new_cache())
    _close(rms_norm(x, orc.w(None, "final_norm"), CFG.eps), norm, 1e-5)

