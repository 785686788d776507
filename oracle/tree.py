"""Oracle: DTree tree construction, verify-input compile and accept walk.

Test infrastructure only (see ``oracle/__init__.py``).

Restates, in numpy / pure Python:
- ``build_tree``          <- ``dtree_runtime.py:82-163`` (best-first heap over
  per-depth top-k ranks, cumulative log-prob scores); ``heap_tree`` is its
  heap half over given top-k lists.
- ``brute_force_tree``    -- independent check of ``build_tree``: every rank
  tuple (r_1..r_d), r_i < k, d <= D, scored by sum_i lp[i-1, r_i] in fp64,
  sorted by (-score, ranks); the first ``budget`` tuples are the tree. This
  holds because each tuple is pushed only after its predecessor (left sibling
  or parent) was popped and scores never increase along those edges.
- ``compile_tree``        <- ``dtree_runtime.py:166-192`` (ids, positions
  start+depth, mask [L, P+L] with every prefix column visible and tree columns
  = ancestor-or-self visibility).
- ``follow_verified_tree`` <- ``dtree_runtime.py:195-208``.
- ``build_node_lineages`` <- ``qwen35_tree.py:41-55``.
- ``tree_depth_groups``   <- ``qwen35_tree.py:104-123``.
"""
from __future__ import annotations

import heapq
import itertools

import numpy as np


def _topk_sorted(logits: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """Per-row top-k token ids sorted by logit descending (ties: lower id first)
    and their log-probs (logit - logsumexp, fp32), dtree_runtime.py:96-104."""
    x = logits.astype(np.float32)
    order = np.argsort(-x, axis=-1, kind="stable")[:, :k]
    top = np.take_along_axis(x, order, axis=-1)
    mx = x.max(axis=-1, keepdims=True)
    lse = (mx + np.log(np.exp(x - mx).sum(axis=-1, keepdims=True))).astype(np.float32)
    return order.astype(np.int64), (top - lse).astype(np.float32)


def build_tree(draft_logits: np.ndarray, budget: int, topk: int | None = None):
    """Returns (node_token_ids, node_depths, parents, child_maps, visibility)."""
    if budget <= 0 or draft_logits.shape[0] == 0:
        return [], [], [-1], [dict()], np.ones((1, 1), dtype=bool)
    k = min(budget, draft_logits.shape[-1]) if topk is None else min(topk, draft_logits.shape[-1])
    tok, lp = _topk_sorted(draft_logits, k)
    return heap_tree(tok, lp, budget)


def heap_tree(tok: np.ndarray, lp: np.ndarray, budget: int):
    """The heap half of build_tree (dtree_runtime.py:112-160) over given per-depth
    top-k token ids [D, k] and fp32 log-probs [D, k]."""
    if budget <= 0 or tok.shape[0] == 0:
        return [], [], [-1], [dict()], np.ones((1, 1), dtype=bool)
    k = tok.shape[1]
    depth_limit = tok.shape[0]
    lp = np.asarray(lp, dtype=np.float32)
    first = float(lp[0, 0])
    heap = [(-first, (0,), 0, 1, 0, first)]
    node_ids: list[int] = []
    depths: list[int] = []
    parents = [-1]
    child_maps: list[dict[int, int]] = [dict()]
    while heap and len(node_ids) < budget:
        _, ranks, parent, depth, rank, logw = heapq.heappop(heap)
        t = int(tok[depth - 1, rank])
        idx = len(node_ids) + 1
        node_ids.append(t)
        depths.append(depth)
        parents.append(parent)
        child_maps.append(dict())
        child_maps[parent][t] = idx
        if rank + 1 < k:
            sib = logw - float(lp[depth - 1, rank]) + float(lp[depth - 1, rank + 1])
            heapq.heappush(heap, (-sib, ranks[:-1] + (rank + 1,), parent, depth, rank + 1, sib))
        if depth < depth_limit:
            ch = logw + float(lp[depth, 0])
            heapq.heappush(heap, (-ch, ranks + (0,), idx, depth + 1, 0, ch))

    n = 1 + len(node_ids)
    vis = np.zeros((n, n), dtype=bool)
    vis[0, 0] = True
    for i in range(1, n):
        vis[i, :i] = vis[parents[i], :i]
        vis[i, i] = True
    return node_ids, depths, parents, child_maps, vis


def brute_force_tree(draft_logits: np.ndarray, budget: int, topk: int):
    """Rank tuples of the best ``budget`` nodes, in pop order (tiny inputs only)."""
    tok, lp = _topk_sorted(draft_logits, topk)
    D = draft_logits.shape[0]
    cands = []
    for d in range(1, D + 1):
        for ranks in itertools.product(range(topk), repeat=d):
            score = sum(float(lp[i, r]) for i, r in enumerate(ranks))
            cands.append((-score, ranks))
    cands.sort()
    chosen = [r for _, r in cands[:budget]]
    token_ids = [int(tok[len(r) - 1, r[-1]]) for r in chosen]
    return chosen, token_ids


def compile_tree(root_token: int, start: int, node_ids, node_depths, visibility: np.ndarray,
                 past_length: int):
    """ids [L], positions [L], mask [L, past_length + L] (True = attend)."""
    ids = np.array([root_token, *node_ids], dtype=np.int64)
    pos = np.array([start, *[start + d for d in node_depths]], dtype=np.int64)
    L = len(ids)
    mask = np.ones((L, past_length + L), dtype=bool)
    mask[:, past_length:] = visibility
    return ids, pos, mask


def follow_verified_tree(child_maps, posterior_tokens):
    acc = [0]
    cur = 0
    nxt = int(posterior_tokens[0])
    while nxt in child_maps[cur]:
        cur = child_maps[cur][nxt]
        acc.append(cur)
        nxt = int(posterior_tokens[cur])
    return acc, nxt


def build_node_lineages(parents):
    if not parents:
        return []
    if parents[0] != -1:
        raise ValueError(f"tree root parent must be -1, got {parents[0]}")
    out = [[]]
    for i in range(1, len(parents)):
        p = int(parents[i])
        if p < 0 or p >= i:
            raise ValueError(f"tree parent index must precede child, got parents[{i}]={p}")
        out.append([*out[p], p])
    return out


def tree_depth_groups(parents):
    if not parents:
        return []
    if parents[0] != -1:
        raise ValueError(f"tree root parent must be -1, got {parents[0]}")
    depth = [0] * len(parents)
    groups = [[0]]
    for i in range(1, len(parents)):
        p = int(parents[i])
        if p < 0 or p >= i:
            raise ValueError(f"tree parent index must precede child, got parents[{i}]={p}")
        depth[i] = depth[p] + 1
        while len(groups) <= depth[i]:
            groups.append([])
        groups[depth[i]].append(i)
    return groups
