"""Tree build / compile / walk: reference known-answer tests (ported from
tests/test_dtree_runtime.py of DrHB/dtree-mlx) plus brute-force pinning of the
best-first tree on tiny inputs. CPU only."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from dtree_hip.dtree_runtime import (build_dtree_tree, compile_dtree_tree, follow_verified_tree,
                                     lazy_follow_tree_exact)
from oracle import tree as otree

KAT_LOGITS = np.array([[5.0, 4.0, 1.0], [6.0, 2.0, 1.0], [7.0, 3.0, 1.0]], dtype=np.float32)


@pytest.mark.parametrize("impl", ["product", "oracle"])
def test_build_tree_returns_prefix_closed_visibility(impl):
    # tests/test_dtree_runtime.py:15-40
    if impl == "product":
        ids, depths, parents, child_maps, vis, _ = build_dtree_tree(torch.from_numpy(KAT_LOGITS), budget=4)
        vis = vis.numpy()
    else:
        ids, depths, parents, child_maps, vis = otree.build_tree(KAT_LOGITS, budget=4)
    assert ids and len(ids) == len(depths)
    assert parents[0] == -1
    assert vis.shape[0] == 1 + len(ids)
    assert bool(vis[0, 0])
    for i in range(1, len(parents)):
        p = parents[i]
        assert p < i
        assert child_maps[p][ids[i - 1]] == i
        assert bool(vis[i, p]) and bool(vis[i, i])


def test_build_tree_kat_exact_nodes():
    # Hand-derived for the KAT logits, budget 4 (topk = min(budget, V) = 3):
    # log-probs per row are sorted by token id here, row-0 best is token 0.
    ids, depths, parents, _, _, _ = build_dtree_tree(torch.from_numpy(KAT_LOGITS), budget=4)
    chosen, toks = otree.brute_force_tree(KAT_LOGITS, budget=4, topk=3)
    assert ids == toks
    assert depths == [len(r) for r in chosen]
    # chain 0 -> 0 -> 0 has log-prob sum ~ -0.38 - 0.02 - 0.02; sibling token 1 at depth 1 ~ -1.38
    assert ids[:3] == [0, 0, 0] and parents[:4] == [-1, 0, 1, 2]


@pytest.mark.parametrize("seed", range(8))
def test_build_tree_matches_brute_force(seed):
    g = np.random.default_rng(seed)
    D, V, k = int(g.integers(2, 5)), int(g.integers(4, 9)), int(g.integers(2, 4))
    budget = int(g.integers(1, min(30, sum(k ** d for d in range(1, D + 1))) + 1))
    logits = (g.standard_normal((D, V)) * 3).astype(np.float32)
    chosen, toks = otree.brute_force_tree(logits, budget, k)
    ids, depths, parents, child_maps, vis, _ = build_dtree_tree(torch.from_numpy(logits), budget, topk=k)
    o_ids, o_depths, o_parents, _, o_vis = otree.build_tree(logits, budget, topk=k)
    assert ids == toks == o_ids
    assert depths == [len(r) for r in chosen] == o_depths
    assert parents == o_parents
    # parent of each node is the node whose rank tuple is its prefix
    index = {r: i + 1 for i, r in enumerate(chosen)}
    for i, r in enumerate(chosen):
        assert parents[i + 1] == (0 if len(r) == 1 else index[r[:-1]])
    assert np.array_equal(vis.numpy(), o_vis)
    for i in range(len(parents)):
        anc = set()
        j = i
        while j >= 0:
            anc.add(j)
            j = parents[j]
        assert set(np.nonzero(o_vis[i])[0].tolist()) == anc


def test_build_tree_empty_budget():
    ids, depths, parents, child_maps, vis, _ = build_dtree_tree(torch.zeros(3, 5), budget=0)
    assert ids == [] and parents == [-1] and vis.shape == (1, 1)


@pytest.mark.parametrize("impl", ["product", "oracle"])
def test_follow_verified_tree_walks_matching_children(impl):
    # tests/test_dtree_runtime.py:43-52
    child_maps = [{11: 1, 12: 2}, {21: 3}, {}, {}]
    fn = follow_verified_tree if impl == "product" else otree.follow_verified_tree
    accepted, nxt = fn(child_maps, [11, 21, 99, 0])
    assert accepted == [0, 1, 3]
    assert nxt == 0


def test_build_node_lineages_returns_root_to_parent_paths():
    # tests/test_dtree_runtime.py:55-64
    assert otree.build_node_lineages([-1, 0, 0, 1, 3, 2]) == [[], [0], [0], [0, 1], [0, 1, 3], [0, 2]]
    with pytest.raises(ValueError):
        otree.build_node_lineages([-1, 1])
    assert otree.tree_depth_groups([-1, 0, 0, 1, 3, 2]) == [[0], [1, 2], [3, 5], [4]]


def test_lazy_follow_tree_exact_walks_only_the_taken_branch():
    # tests/test_dtree_runtime.py:67-106, with torch tensors
    class FakeTextModel:
        def forward_dflash(self, inputs, cache, layer_ids):
            token = int(inputs[0, 0].item())
            return (torch.tensor([[[float(token)]]]), torch.tensor([[[float(token + 1000)]]]))

    class FakeTarget:
        def __init__(self):
            self.adapter = SimpleNamespace(family="qwen3_5")
            self.model = SimpleNamespace(language_model=SimpleNamespace(model=FakeTextModel()))

        def lm_head_argmax(self, hidden_states):
            token = int(hidden_states[0, 0, 0].item())
            return torch.tensor([[{10: 100, 11: 300, 21: 999}[token]]])

    accepted, nxt, vh = lazy_follow_tree_exact(
        target=FakeTarget(), target_cache=[], layer_ids=[], tree_tokens=[10, 11, 12, 21],
        child_maps=[{100: 1, 200: 2}, {300: 3}, {}, {}], temperature=0.0,
        verify_mode="parallel-greedy-argmax", profile_times=None)
    assert accepted == [0, 1, 3]
    assert nxt == 999
    assert vh.tolist() == [[[1010.0], [1011.0], [1021.0]]]


def test_lazy_follow_rejects_other_families():
    with pytest.raises(NotImplementedError):
        lazy_follow_tree_exact(SimpleNamespace(adapter=SimpleNamespace(family="qwen3")), [], [], [1], [{}], 0.0,
                               "parallel-greedy-argmax", None)


def test_compile_tree_mask_semantics():
    ids, depths, parents, child_maps, vis, _ = build_dtree_tree(torch.from_numpy(KAT_LOGITS), budget=4)
    P = 5
    ids_buf = torch.zeros(1, 5, dtype=torch.int64)
    pos_buf = torch.zeros(1, 5, dtype=torch.int64)
    mask_buf = torch.zeros(5, 20, dtype=torch.bool)  # deliberately not all-ones
    vids, tokens, vpos, mask = compile_dtree_tree(42, P, ids, depths, vis, P, ids_buf, pos_buf, mask_buf)
    o_ids, o_pos, o_mask = otree.compile_tree(42, P, ids, depths, vis.numpy(), P)
    assert tokens == [42, *ids]
    assert vids[0].tolist() == o_ids.tolist()
    assert vpos[0].tolist() == o_pos.tolist() == [P, *[P + d for d in depths]]
    assert np.array_equal(mask.numpy(), o_mask)
    assert mask[:, :P].all()


def test_qwen35_compaction_requires_pending_tree_state():
    """adapters.py:441-442: compact_kv_caches without a pending tree raises
    (checked before any device work)."""
    from dtree_hip.adapters import ADAPTERS, Qwen35TargetAdapter

    ad = ADAPTERS["qwen3_5"]()
    assert isinstance(ad, Qwen35TargetAdapter) and ad.family == "qwen3_5"
    assert ad.supports_tree_verification()
    with pytest.raises(RuntimeError, match="pending tree state"):
        ad.compact_kv_caches(None, None, past_length=0, keep_current_indices=[0])
    # an empty accepted list commits nothing but consumes the pending state
    ad._pending_tree_state = (5, 3, [-1, 0, 1])
    ad.compact_kv_caches(None, None, past_length=5, keep_current_indices=[])
    assert ad._pending_tree_state is None
    # accepted indices must be a root path of the pending tree
    ad._pending_tree_state = (5, 3, [-1, 0, 0])
    with pytest.raises(ValueError, match="root path"):
        ad.compact_kv_caches(None, None, past_length=5, keep_current_indices=[0, 1, 2])


def test_dflash_prefix_match_and_chain_inputs():
    """runtime.py:32-38 longest_prefix_match and the chain-shaped verify
    inputs of the linear decode: parents -1, 0, 1, ..; positions start + i;
    every prefix column visible, causal over the block."""
    from dtree_hip.runtime import _chain_inputs, longest_prefix_match

    assert longest_prefix_match([1, 2, 3], [1, 2, 4]) == 2
    assert longest_prefix_match([1, 2], [1, 2, 3]) == 2
    assert longest_prefix_match([5], [4]) == 0
    assert longest_prefix_match([], [1]) == 0
    ids, pos, parents, mask = _chain_inputs([9, 8, 7, 6], start=5)
    assert ids.tolist() == [[9, 8, 7, 6]] and pos.tolist() == [[5, 6, 7, 8]]
    assert parents == [-1, 0, 1, 2]
    assert mask.shape == (4, 9) and bool(mask[:, :5].all())
    for i in range(4):
        for j in range(4):
            assert bool(mask[i, 5 + j]) == (j <= i)


def test_generator_rejects_unsupported_quantisation():
    from dtree_hip.api import DFlashGenerator

    with pytest.raises(NotImplementedError):
        DFlashGenerator(target_model="random:qwen3-4b", target_quant_bits=8)
    with pytest.raises(NotImplementedError):
        DFlashGenerator(target_model="random:qwen3-4b", target_quant_bits=4, target_quant_group_size=32)


def test_draft_config_and_cache_bookkeeping():
    """Drafter host logic (draft.py:25-110, runtime.py:22-26): config fields,
    target layer spread, cache offsets under trim in both modes."""
    from dtree_hip.config import QWEN3_4B, QWEN35_4B
    from dtree_hip.draft import DFlashDraftCache, DraftArgs, build_target_layer_ids, random_draft_config
    from dtree_hip.runtime import trim_draft_cache

    a = random_draft_config(QWEN3_4B, "dflash-b16")
    assert (a.block_size, a.num_hidden_layers, a.num_attention_heads, a.num_key_value_heads) == (16, 5, 32, 8)
    assert a.dflash_config["target_layer_ids"] == [1, 9, 17, 25, 33]
    assert a.dflash_config["mask_token_id"] == QWEN3_4B.vocab_size - 1
    assert random_draft_config(QWEN35_4B, "dflash-b16-l3").dflash_config["target_layer_ids"] == [1, 15, 29]
    assert build_target_layer_ids(2, 5) == [1]
    assert DraftArgs.from_dict({**a.__dict__, "unknown": 1}) == a
    with pytest.raises(NotImplementedError):
        random_draft_config(QWEN3_4B, "eagle")
    with pytest.raises(NotImplementedError):
        DraftArgs.from_dict({**a.__dict__, "attention_bias": True}).stack_config()

    kv = DFlashDraftCache(3, 2, 128, "kv", max_past=256, block=32, device="cpu")
    for lc in kv:
        lc.offset = 40
    trim_draft_cache(kv, 16)
    assert kv.offset == 24 and kv.stored_length() == 24
    trim_draft_cache(kv, 100)
    assert kv.offset == 0
    co = DFlashDraftCache(3, 2, 128, "context-only", max_past=256, block=32, device="cpu")
    assert co.capacity == 64 + 1024
    for lc in co:
        lc.offset = 5000
    trim_draft_cache(co, 16)
    assert co.offset == 5000 and co.stored_length() == 1088
    co.layers[1].offset = 4999
    with pytest.raises(ValueError):
        co.offset
