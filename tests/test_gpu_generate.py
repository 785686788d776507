"""End-to-end DTree decoding on the GPU through the reference-shaped surface,
for the Qwen3 target and the Qwen3.5 hybrid (lazy exact walk and full-tree
verify).

``dtree_generate`` (dtree_runtime.py:293-586) drives the HIP target through the
adapter methods of adapters.py (forward_with_hidden_states, embed_tokens,
lm_head_logits / lm_head_argmax, forward_tree_with_hidden_states,
compact_kv_caches) or the fused verify graph. At temperature 0, speculative
decoding must emit the target's greedy continuation whatever the drafter
proposes: every emitted token is checked against the fp32 oracle run over the
emitted sequence itself (teacher forcing), to be its argmax within the 2e-2
relative logit tolerance (and exactly its argmax on nearly every position).

The drafter is scripted: it proposes the target's own sequential greedy decode
(computed on the GPU beforehand) through the tied LM head (hidden row =
24 * (1024 / hidden) * E[token], so the draft logits peak at that token), and plants one wrong
token at a depth that cycles over the steps, so the accepted lengths cover
1 .. the full chain."""
import numpy as np
import pytest
import torch

from oracle import qwen3 as oq
from oracle import qwen35 as o35

from dtree_hip.adapters import load_target_model
from dtree_hip.config import Qwen35Config, tiny_qwen3, tiny_qwen35
from dtree_hip.dtree_runtime import dtree_generate

pytestmark = pytest.mark.gpu

TOL = 2e-2
BLOCK = 8


def _oracle_teacher_forced(target, seq):
    """fp32 oracle logits of every position of `seq` under a causal mask
    (row i predicts seq[i + 1])."""
    cfg = target.model.args
    if isinstance(cfg, Qwen35Config):
        ocfg = o35.Qwen35Config(
            hidden=cfg.hidden_size, layers=cfg.num_hidden_layers, ffn=cfg.intermediate_size,
            heads=cfg.num_attention_heads, kv_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
            rope_dims=cfg.rope_dims, lin_k_heads=cfg.linear_num_key_heads, lin_v_heads=cfg.linear_num_value_heads,
            lin_k_dim=cfg.linear_key_head_dim, lin_v_dim=cfg.linear_value_head_dim,
            conv_kernel=cfg.linear_conv_kernel_dim, full_attention_interval=cfg.full_attention_interval,
            vocab=cfg.vocab_size, eps=cfg.rms_norm_eps, rope_base=cfg.rope_theta)
        orc35 = o35.OracleQwen35(ocfg, target.model.weights.host_accessor())
        T = len(seq)
        norm, _, _ = orc35.forward_tree(np.asarray(seq, np.int64), np.arange(T), [-1] + list(range(T - 1)),
                                        orc35.new_cache())
        return orc35.lm_head_logits(norm)
    ocfg = oq.Qwen3Config(hidden=cfg.hidden_size, layers=cfg.num_hidden_layers, ffn=cfg.intermediate_size,
                          heads=cfg.num_attention_heads, kv_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                          vocab=cfg.vocab_size, eps=cfg.rms_norm_eps, rope_base=cfg.rope_theta)
    orc = oq.OracleQwen3(ocfg, target.model.weights.host_accessor())
    nl, Hkv, D = cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim
    empty = oq.OracleCache(keys=[np.zeros((0, Hkv, D), np.float32)] * nl,
                           values=[np.zeros((0, Hkv, D), np.float32)] * nl)
    T = len(seq)
    norm, _, _, _ = orc.forward_tree(np.asarray(seq, np.int64), np.arange(T), np.tril(np.ones((T, T), bool)), empty)
    return orc.lm_head_logits(norm)


def _gpu_sequential_greedy(target, prompt, n_new):
    """The target's greedy continuation one token per forward (chain of 1)."""
    cache = target.make_cache()
    logits, _ = target.forward_with_hidden_states(torch.tensor(prompt)[None], cache, [0, 1])
    out = [int(torch.argmax(logits[0, -1]).item())]
    while len(out) < n_new:
        logits, _ = target.forward_with_hidden_states(torch.tensor([out[-1]])[None], cache, [0, 1])
        out.append(int(torch.argmax(logits[0, -1]).item()))
    return out


class ScriptedDrafter:
    """Drafter with the interface dtree_generate uses (draft.py:312-367 shape):
    mask_token_id, block_size, make_cache(), __call__(noise_embedding,
    target_hidden, cache) -> hidden [1, block, H].

    It proposes the target's own greedy continuation of the sequence actually
    committed so far, with one planted wrong token per step. It rebuilds that
    sequence from what it is handed (the count of committed rows since its
    last call, which are the root and accepted tokens of its previous block,
    and the new root token, read from the noise embedding's first row), so a
    step whose verify resolves a near-tie of the tiny random model the other
    way than the precomputed sequential decode (both within the logit
    tolerance) costs that step's acceptance only; the proposals then follow
    the new prefix (a fresh sequential greedy decode from it)."""

    mask_token_id = 0
    block_size = BLOCK

    def __init__(self, target, seq):
        self.target = target
        self.seq = seq  # prompt + the target's sequential greedy continuation
        V = target.model.args.vocab_size
        self._emb = target.model.weights.embed_rows(torch.arange(V, device="cuda"))

    def make_cache(self):
        return {"actual": None, "block": None, "calls": 0, "plan": list(self.seq)}

    def _root_token(self, noise_embedding) -> int:
        hit = (self._emb == noise_embedding[0, 0].to(self._emb.dtype)).all(-1).nonzero()
        return int(hit[0, 0]) if hit.numel() else -1

    def __call__(self, noise_embedding, target_hidden, cache):
        # Committed rows since the last call: the prompt first, then the root
        # and the accepted draft tokens of the previous block.
        n = int(target_hidden.shape[1])
        if cache["actual"] is None:
            cache["actual"] = list(self.seq[:n])
        else:
            cache["actual"] += cache["block"][:n]
        root = self._root_token(noise_embedding)
        prefix = cache["actual"] + [root]
        start = len(prefix) - 1
        plan = cache["plan"]
        if plan[:len(prefix)] != prefix:  # a near-tie went the other way: follow the actual prefix
            plan = prefix + _gpu_sequential_greedy(self.target, prefix, BLOCK)
            cache["plan"] = plan
        wrong = cache["calls"] % BLOCK  # 0: whole chain right, else the depth that is wrong
        cache["calls"] += 1
        V = self.target.model.args.vocab_size
        toks = []
        for d in range(BLOCK):
            p = start + d
            t = plan[p] if p < len(plan) else (7 * p) % V
            if d == wrong and d > 0:
                t = (t + 1) % V
            toks.append(t)
        cache["block"] = toks
        E = self.target.model.weights.embed_rows(torch.tensor(toks, device="cuda")).float()
        # peak logit 24 * 1024 * 0.02^2 ~ 9.8 whatever the hidden size, so the
        # best-first tree follows the scripted chain
        H = self.target.model.args.hidden_size
        return (24.0 * 1024 / H * E)[None]


CASES = [("qwen3", "parallel-greedy-argmax", None), ("qwen3", "parallel-replay", None),
         # Qwen3.5: the reference's default lazy exact walk, and the full-tree
         # verify (DTREE_QWEN35_TREE_MODE=full_tree) fused and per method.
         ("qwen3_5", "parallel-greedy-argmax", None), ("qwen3_5", "parallel-greedy-argmax", "full_tree"),
         ("qwen3_5", "parallel-replay", "full_tree")]


@pytest.mark.parametrize("family,verify_mode,tree_mode", CASES)
def test_dtree_generate_emits_greedy_tokens(gpu_device, monkeypatch, family, verify_mode, tree_mode):
    if tree_mode:
        monkeypatch.setenv("DTREE_QWEN35_TREE_MODE", tree_mode)
    else:
        monkeypatch.delenv("DTREE_QWEN35_TREE_MODE", raising=False)
    cfg = tiny_qwen3() if family == "qwen3" else tiny_qwen35()
    target = load_target_model(cfg, seed=0, max_past=256, device="cuda", layer_ids=[0, 1],
                               norm_jitter=0.0 if family == "qwen3" else 0.1)
    rng = np.random.default_rng(5)
    prompt = rng.integers(1, cfg.vocab_size, 40).tolist()
    n_new = 40
    plan = _gpu_sequential_greedy(target, prompt, n_new)
    drafter = ScriptedDrafter(target, prompt + plan)
    out, metrics = dtree_generate(target, drafter, prompt, max_new_tokens=n_new, temperature=0.0,
                                  stop_token_ids=set(), layer_ids=[0, 1], speculative_tokens=BLOCK,
                                  tree_budget=12, verify_mode=verify_mode, tree_topk=4)
    gen = out[len(prompt):]
    assert len(gen) == n_new
    # Every emitted token is the oracle's argmax within the logit tolerance,
    # given the tokens before it, and nearly all are its exact argmax.
    logits = _oracle_teacher_forced(target, out[:-1])[len(prompt) - 1:]
    scale = np.abs(logits).max(axis=-1)
    chosen = logits[np.arange(n_new), gen]
    assert np.all(chosen >= logits.max(axis=-1) - TOL * scale)
    assert np.mean(np.argmax(logits, axis=-1) == np.asarray(gen)) >= 0.9
    # The drafter proposed the target's own greedy path with one planted error
    # per step, so acceptance lengths span single tokens to long chains.
    acc = metrics["acceptance_lengths"]
    assert max(acc) >= 5 and min(acc) == 1, acc
    assert target.model.args.model_type == target.adapter.family


def test_dtree_generate_twice_on_one_model(gpu_device, monkeypatch):
    """Two decode calls on one resident model: each builds its own cache, and
    the captured verify graph (which holds one cache's page pointers) must be
    replayed only for the cache it was captured for, even when the second
    cache reuses the first one's id after it is freed. Both runs must emit the
    oracle's greedy continuation."""
    import gc

    monkeypatch.delenv("DTREE_QWEN35_TREE_MODE", raising=False)
    cfg = tiny_qwen3()
    target = load_target_model(cfg, seed=0, max_past=256, device="cuda", layer_ids=[0, 1])
    rng = np.random.default_rng(11)
    for run in range(2):
        prompt = rng.integers(1, cfg.vocab_size, 30 + 7 * run).tolist()
        n_new = 24
        plan = _gpu_sequential_greedy(target, prompt, n_new)
        drafter = ScriptedDrafter(target, prompt + plan)
        out, metrics = dtree_generate(target, drafter, prompt, max_new_tokens=n_new, temperature=0.0,
                                      stop_token_ids=set(), layer_ids=[0, 1], speculative_tokens=BLOCK,
                                      tree_budget=12, verify_mode="parallel-greedy-argmax", tree_topk=4)
        gc.collect()  # the first run's cache dies here; its graph is queued for destruction
        gen = out[len(prompt):]
        assert len(gen) == n_new
        logits = _oracle_teacher_forced(target, out[:-1])[len(prompt) - 1:]
        scale = np.abs(logits).max(axis=-1)
        chosen = logits[np.arange(n_new), gen]
        assert np.all(chosen >= logits.max(axis=-1) - TOL * scale), f"run {run}"
        assert np.mean(np.argmax(logits, axis=-1) == np.asarray(gen)) >= 0.9, f"run {run}"
    eng = target.model.engine
    assert len(eng._graphs) <= 1
