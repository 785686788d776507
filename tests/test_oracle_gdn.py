"""Pins of the GatedDeltaNet tree oracle (oracle/gdn.py).

Inputs follow the reference's kernel tests (tests/test_qwen35_tree_kernels.py:
seeded default_rng(0..3) draws, parents [-1, 0, 0, 1, 2]). Each check compares
the oracle with an independent formulation, so a dropped term, a wrong parent
index or a transposed state fails:

* tree conv: the closed form "conv input of node t = last K rows of (base
  window ++ inputs along t's root path)";
* tree recurrence: path decomposition (each node's output and state equal the
  plain sequential recurrence run along its root path) and, for chains,
  transformers' torch_recurrent_gated_delta_rule (library implementation; its
  state is [Dk, Dv], its q is scaled by Dk^-0.5 inside and its g is a
  log-decay);
* commit: window and state of the last accepted node."""
import numpy as np
import pytest
import torch

from oracle import gdn

PARENTS = [-1, 0, 0, 1, 2]


def _ref_conv_inputs():
    x = np.random.default_rng(0).normal(size=(1, 5, 8)).astype(np.float32)[0]
    base = np.random.default_rng(1).normal(size=(1, 3, 8)).astype(np.float32)[0]
    w = np.random.default_rng(2).normal(size=(4, 8)).astype(np.float32)
    return x, base, w


def _ref_delta_inputs():
    rng = np.random.default_rng(3)
    q = rng.normal(size=(1, 5, 1, 32)).astype(np.float32)[0]
    k = rng.normal(size=(1, 5, 1, 32)).astype(np.float32)[0]
    v = rng.normal(size=(1, 5, 1, 8)).astype(np.float32)[0]
    g = rng.normal(size=(1, 5, 1)).astype(np.float32)[0]
    beta = rng.normal(size=(1, 5, 1)).astype(np.float32)[0]
    state = rng.normal(size=(1, 1, 8, 32)).astype(np.float32)[0]
    return q, k, v, g, beta, state


def test_tree_conv_matches_path_window_closed_form():
    x, base, w = _ref_conv_inputs()
    out, win = gdn.tree_conv1d(x, base, w, PARENTS)
    for t in range(5):
        seq = np.concatenate([base, x[gdn.root_path(PARENTS, t)]], axis=0)
        inp = seq[-4:]
        acc = (inp.astype(np.float64) * w).sum(0)
        np.testing.assert_allclose(out[t], acc / (1 + np.exp(-acc)), rtol=1e-12, atol=1e-12)
        np.testing.assert_array_equal(win[t], seq[-3:])
    # siblings 1 and 2 share the root's window; node 3 sees (b2, x0, x1)
    np.testing.assert_array_equal(win[3][:2], np.stack([x[0], x[1]]))


def _chain(q, k, v, g, beta, state, order):
    """Plain sequential recurrence over the nodes `order` (GQA by h // group)."""
    S = state.astype(np.float64).copy()
    Hv, Hk = v.shape[1], k.shape[1]
    ys = []
    for t in order:
        for h in range(Hv):
            kk, qq = k[t, h // (Hv // Hk)], q[t, h // (Hv // Hk)]
            S[h] *= g[t, h]
            kv = S[h] @ kk
            S[h] += np.outer((v[t, h] - kv) * beta[t, h], kk)
        ys.append(np.stack([S[h] @ q[t, h // (Hv // Hk)] for h in range(Hv)]))
    return np.stack(ys), S


def test_tree_recurrence_equals_chains_along_root_paths():
    q, k, v, g, beta, state = _ref_delta_inputs()
    y, states = gdn.tree_gated_delta(q, k, v, g, beta, state, PARENTS)
    for t in range(5):
        ys, S = _chain(q, k, v, g, beta, state, gdn.root_path(PARENTS, t))
        np.testing.assert_allclose(y[t], ys[-1], rtol=1e-10, atol=1e-10)
        np.testing.assert_allclose(states[t], S, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("Hk,Hv", [(2, 2), (2, 4)])
def test_chain_recurrence_matches_transformers(Hk, Hv):
    from transformers.models.qwen3_5.modeling_qwen3_5 import torch_recurrent_gated_delta_rule

    g_ = np.random.default_rng(11)
    T, Dk, Dv = 6, 16, 8
    q = g_.normal(size=(T, Hk, Dk))
    k = g_.normal(size=(T, Hk, Dk)) / np.sqrt(Dk)
    v = g_.normal(size=(T, Hv, Dv))
    decay = np.exp(-np.abs(g_.normal(size=(T, Hv))))
    beta = 1 / (1 + np.exp(-g_.normal(size=(T, Hv))))
    state = g_.normal(size=(Hv, Dv, Dk))
    y, states = gdn.tree_gated_delta(q, k, v, decay, beta, state, [-1] + list(range(T - 1)))
    rep = Hv // Hk  # interleaved GQA: v-head h reads k-head h // rep
    tq = torch.from_numpy(np.repeat(q, rep, axis=1) * np.sqrt(Dk))[None]
    tk = torch.from_numpy(np.repeat(k, rep, axis=1))[None]
    out, last = torch_recurrent_gated_delta_rule(
        tq, tk, torch.from_numpy(v)[None], torch.from_numpy(np.log(decay))[None], torch.from_numpy(beta)[None],
        torch.from_numpy(state.transpose(0, 2, 1).copy())[None], output_final_state=True)
    np.testing.assert_allclose(y, out[0].double().numpy(), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(states[-1], last[0].double().numpy().transpose(0, 2, 1), rtol=1e-5, atol=1e-5)


def test_commit_takes_last_accepted_node():
    x, base, w = _ref_conv_inputs()
    q, k, v, g, beta, state = _ref_delta_inputs()
    win, S = gdn.commit(x, base, q, k, v, g, beta, state, PARENTS, [0, 1, 3])
    _, wins = gdn.tree_conv1d(x, base, w, PARENTS)
    _, states = gdn.tree_gated_delta(q, k, v, g, beta, state, PARENTS)
    np.testing.assert_array_equal(win, wins[3])
    np.testing.assert_array_equal(S, states[3])
    np.testing.assert_array_equal(win, np.stack([x[0], x[1], x[3]]))


def test_chain_forms_equal_the_tree_forms_on_a_chain():
    """chain_conv1d / chain_gated_delta (the memory-light forms used for long
    prompts) against tree_conv1d / tree_gated_delta with chain parents, on
    grouped heads and a nonzero base window and state; a planted off-by-one in
    the conv rows (the window shifted by one) must fail."""
    rng = np.random.default_rng(7)
    T, Hk, Hv, Dk, Dv, C, keep = 23, 2, 4, 16, 8, 12, 3
    x = rng.normal(size=(T, C))
    base = rng.normal(size=(keep, C))
    w = rng.normal(size=(keep + 1, C))
    chain = [-1] + list(range(T - 1))
    out, win = gdn.tree_conv1d(x, base, w, chain)
    cout, cwin = gdn.chain_conv1d(x, base, w)
    np.testing.assert_allclose(cout, out, rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(cwin, win[-1])
    bad, _ = gdn.chain_conv1d(np.concatenate([x[1:], x[:1]]), base, w)
    assert np.abs(bad - out).max() > 1e-3
    q = rng.normal(size=(T, Hk, Dk))
    k = rng.normal(size=(T, Hk, Dk)) / 4
    v = rng.normal(size=(T, Hv, Dv))
    g = rng.uniform(0.5, 1.0, size=(T, Hv))
    beta = rng.uniform(0.0, 1.0, size=(T, Hv))
    state = rng.normal(size=(Hv, Dv, Dk))
    y, states = gdn.tree_gated_delta(q, k, v, g, beta, state, chain)
    cy, cs = gdn.chain_gated_delta(q, k, v, g, beta, state)
    np.testing.assert_allclose(cy, y, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(cs, states[-1], rtol=1e-12, atol=1e-12)

