"""Seeded synthetic verify-step workloads (random-init weights, no datasets).

Seeds: weights 0, prefix tokens 1, draft tree 2, acceptance path 3.

Draft tree: per draft depth, logits = N(0,1) + Gumbel noise, with four
random tokens boosted so the best token is confident (top-1 probability
varies per depth); build_dtree_tree with top-4 branching and the given budget
(depth <= number of draft rows) then picks nodes best-first by cumulative
log-prob, as the reference does with real drafter logits.

Acceptance pass: a seeded root-to-leaf path of the tree is walked from the
top; at each depth, with probability p, the node's token is replaced by the
target's own argmax at its parent (computed on the device path), swapping
with a sibling that already holds that token so child tokens stay unique.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from .dtree_runtime import build_dtree_tree


@dataclass
class Tree:
    tokens: list[int]        # root first
    depths: list[int]        # root 0
    parents: list[int]       # root -1
    child_maps: list[dict[int, int]]
    visibility: np.ndarray   # [L, L] bool

    @property
    def size(self) -> int:
        return len(self.tokens)

    def positions(self, start: int) -> list[int]:
        return [start + d for d in self.depths]

    def children(self, i: int) -> list[int]:
        return [j for j in range(i + 1, self.size) if self.parents[j] == i]

    def rebuild_child_maps(self) -> None:
        self.child_maps = [dict() for _ in range(self.size)]
        for j in range(1, self.size):
            self.child_maps[self.parents[j]][self.tokens[j]] = j


def draft_logits(depth: int, vocab: int, seed: int = 2) -> torch.Tensor:
    g = np.random.default_rng(seed)
    x = g.standard_normal((depth, vocab), dtype=np.float32)
    x += g.gumbel(size=(depth, vocab)).astype(np.float32)
    for d in range(depth):
        toks = g.choice(vocab, size=4, replace=False)
        top = 10.0 + 8.0 * g.random()
        x[d, toks] += np.array([top, top - 2.0 - 2.0 * g.random(), top - 4.0, top - 5.0], dtype=np.float32)
    return torch.from_numpy(x)


def make_tree(root_token: int, vocab: int, budget: int = 24, depth: int = 15, topk: int = 4, seed: int = 2) -> Tree:
    ids, depths, parents, child_maps, vis, _ = build_dtree_tree(draft_logits(depth, vocab, seed), budget, topk=topk)
    return Tree(tokens=[int(root_token), *ids], depths=[0, *depths], parents=list(parents),
                child_maps=child_maps, visibility=vis.numpy())


def random_prefix(n: int, vocab: int, seed: int = 1) -> list[int]:
    return [int(t) for t in np.random.default_rng(seed).integers(0, vocab, size=n)]


def root_to_leaf_path(tree: Tree, seed: int = 3) -> list[int]:
    g = np.random.default_rng(seed)
    path = [0]
    while True:
        ch = tree.children(path[-1])
        if not ch:
            return path
        path.append(int(ch[int(g.integers(0, len(ch)))]))


def acceptance_rewrite(tree: Tree, argmax_at, p: float = 0.85, seed: int = 3) -> list[int]:
    """Rewrite tokens along a seeded path; ``argmax_at(tree) -> posterior list``
    evaluates the target on the current tree. Returns the path."""
    g = np.random.default_rng(seed)
    path = root_to_leaf_path(tree, seed)
    for d in range(1, len(path)):
        if g.random() >= p:
            continue
        node, parent = path[d], path[d - 1]
        want = int(argmax_at(tree)[parent])
        if tree.tokens[node] == want:
            continue
        for sib in tree.children(parent):
            if sib != node and tree.tokens[sib] == want:
                tree.tokens[sib] = tree.tokens[node]
                break
        tree.tokens[node] = want
        tree.rebuild_child_maps()
    return path
