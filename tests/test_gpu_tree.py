"""The draft tree built on the GPU (dtree_tree_build, dtree_runtime.py:82-192)
against the oracle (oracle/tree.py).

* Per-row top-k token ids equal the oracle's (logit desc, token id asc) bit
  for bit, including exact ties inside and across the 8192-logit chunks and
  -inf logits; log-probs agree within fp32 rounding of the logsumexp.
* The heap is bit-exact: the device tree equals the oracle's heap run on the
  device's own top-k lists and log-probs (same fp32 inputs, so the fp64 score
  sums and the tuple tie-break must match exactly).
* The step descriptor holds compile_dtree_tree's verify inputs for that tree
  (tokens, positions = P + depth, parents, ancestor-or-self bitsets).
* End to end, dtree_generate's fused greedy verify builds its trees on the
  device and still emits the target's greedy continuation.
"""
import numpy as np
import pytest
import torch

from oracle import tree as otree

from dtree_hip import _native as N
from dtree_hip.engine import ancestor_bitsets
from dtree_hip.synthetic import draft_logits as peaked_logits

pytestmark = pytest.mark.gpu


def _run(logits: torch.Tensor, k: int, budget: int, root: int, past: int):
    lib = N.lib()
    D, V = logits.shape
    dev = logits.device
    ws = torch.zeros(max(lib.dtree_tree_build_workspace_bytes(D, V, k), 256), dtype=torch.uint8, device=dev)
    desc = torch.zeros(lib.dtree_step_desc_bytes(), dtype=torch.uint8, device=dev)
    tree_out = torch.zeros(1 + 3 * N.MAX_NODES, dtype=torch.int32, device=dev)
    ids = torch.zeros(max(D * k, 1), dtype=torch.int32, device=dev)
    lps = torch.zeros(max(D * k, 1), dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    N.check(lib.dtree_tree_build(logits.data_ptr(), V, D, V, k, budget, root, past, ws.data_ptr(), ws.numel(),
                                 desc.data_ptr(), tree_out.data_ptr(), ids.data_ptr(), lps.data_ptr(), st),
            "tree build")
    torch.cuda.synchronize()
    rec = desc.cpu().numpy().view(N.STEP_DESC_DTYPE)[0]
    return (ids.cpu().numpy()[:D * k].reshape(D, k), lps.cpu().numpy()[:D * k].reshape(D, k),
            tree_out.cpu().numpy(), rec)


def _logits(kind: str, D: int, V: int, seed: int) -> np.ndarray:
    g = np.random.default_rng(seed)
    if kind == "peaked":
        return peaked_logits(D, V, seed=seed).float().numpy()
    if kind == "flat":
        return g.standard_normal((D, V)).astype(np.float32)
    if kind == "ties":  # few distinct values: long runs of exact ties, also across chunk edges
        x = np.round(g.standard_normal((D, V)) * 1.5).astype(np.float32)
        x[:, 8190:8194] = 9.0  # equal maxima straddling the first chunk boundary
        return x
    if kind == "neginf":
        x = g.standard_normal((D, V)).astype(np.float32)
        x[:, ::3] = -np.inf
        return x
    raise ValueError(kind)


CASES = [  # kind, D, V, k, budget
    ("peaked", 15, 151936, 24, 24),   # the reference default k = min(budget, V)
    ("peaked", 15, 151936, 4, 24),    # top-4 branching of the synthetic workloads
    ("flat", 15, 151936, 64, 64),     # 65-node trees
    ("ties", 15, 151936, 24, 24),
    ("neginf", 6, 20000, 10, 30),
    ("flat", 18, 4096, 127, 127),     # the limits
    ("ties", 3, 100, 8, 20),
    ("flat", 1, 8, 5, 5),             # k clamped to the vocabulary by the caller
    ("flat", 5, 20000, 16, 0),        # budget 0: the root alone
]


@pytest.mark.parametrize("kind,D,V,k,budget", CASES)
def test_tree_build_matches_oracle(gpu_device, kind, D, V, k, budget):
    print(f"tree build kind={kind} D={D} V={V} k={k} budget={budget}", flush=True)
    x = _logits(kind, D, V, seed=D * 7 + k)
    root, past = 11, 1000
    ids, lps, out, rec = _run(torch.from_numpy(x).to(gpu_device), k, budget, root, past)
    if budget > 0:
        o_ids, o_lp = otree._topk_sorted(x, k)
        assert np.array_equal(ids, o_ids), "top-k ids"
        # the oracle's fp32 logsumexp as the fp64 reference of both
        m = x.max(axis=-1, keepdims=True).astype(np.float64)
        lse = m + np.log(np.exp(x.astype(np.float64) - m).sum(axis=-1, keepdims=True))
        ref_lp = np.take_along_axis(x, o_ids, axis=-1).astype(np.float64) - lse
        assert np.abs(lps - ref_lp).max() <= 1e-5 * max(1.0, float(np.abs(ref_lp[np.isfinite(ref_lp)]).max()))
        node_ids, depths, parents, child_maps, vis = otree.heap_tree(ids.astype(np.int64), lps, budget)
    else:
        node_ids, depths, parents, child_maps, vis = [], [], [-1], [dict()], np.ones((1, 1), bool)
    n = int(out[0])
    M = N.MAX_NODES
    assert n == len(node_ids)
    assert out[1:1 + n].tolist() == node_ids
    assert out[1 + M:1 + M + n].tolist() == depths
    assert [-1] + out[1 + 2 * M:1 + 2 * M + n].tolist() == parents
    L = n + 1
    assert rec["num_nodes"] == L and rec["past_length"] == past and rec["n_accepted"] == 0
    assert rec["tokens"][:L].tolist() == [root, *node_ids]
    assert rec["positions"][:L].tolist() == [past] + [past + d for d in depths]
    assert rec["parents"][:L].tolist() == parents
    assert np.array_equal(rec["ancestors"][:L], ancestor_bitsets(parents))
    assert not rec["tokens"][L:].any() and (rec["parents"][L:] == -1).all() and not rec["ancestors"][L:].any()
    # the visibility the reference returns is the ancestor-or-self relation of these parents
    anc = ancestor_bitsets(parents)
    bits = np.array([[(int(anc[i][j // 32]) >> (j % 32)) & 1 for j in range(L)] for i in range(L)], bool)
    assert np.array_equal(bits, vis)


def test_tree_build_equals_host_path_on_peaked_logits(gpu_device):
    """The product's host build_dtree_tree and the device build agree on the
    synthetic peaked draft logits (no near-ties for fp32 rounding to flip)."""
    from dtree_hip.dtree_runtime import build_dtree_tree

    for seed in range(4):
        x = peaked_logits(15, 151936, seed=seed).to(gpu_device)
        for k, budget in ((None, 24), (4, 24), (None, 15)):
            host = build_dtree_tree(x, budget, topk=k)
            kk = min(budget if k is None else k, x.shape[1])
            _, _, out, _ = _run(x.float().contiguous(), kk, budget, 0, 0)
            n = int(out[0])
            assert out[1:1 + n].tolist() == host[0] and [-1] + out[1 + 2 * N.MAX_NODES:1 + 2 * N.MAX_NODES + n].tolist() == host[2]


def test_dtree_generate_builds_trees_on_device(gpu_device, monkeypatch):
    from test_gpu_api import _check_greedy, _setup
    from test_gpu_generate import BLOCK

    from dtree_hip.api import Generator

    monkeypatch.delenv("DTREE_TREE_BUILD", raising=False)
    target, prompt, n_new, drafter = _setup("qwen3", seed=9)
    gen = Generator(target_model=target, draft_model=drafter)
    res = gen.generate_from_tokens(prompt, max_new_tokens=n_new, speculative_tokens=BLOCK, decode_mode="dtree",
                                   tree_budget=12, verify_mode="parallel-greedy-argmax")
    assert res.metrics["tree_build"] == "device"
    _check_greedy(target, prompt, res.output_tokens, n_new)
    acc = res.metrics["acceptance_lengths"]
    assert max(acc) >= 5, acc
