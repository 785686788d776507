"""Oracle: Qwen3.5 GatedDeltaNet tree primitives (tree conv1d + SiLU, tree
gated-delta recurrence) and the commit of an accepted path, in float64 numpy.

Test infrastructure only (see ``oracle/__init__.py``).

Follows qwen35_tree_kernels.py:8-152 (the Metal kernels) and the numpy loops
of the reference's tests (tests/test_qwen35_tree_kernels.py:35-52, 74-95):

* tree conv (K taps, Keep = K - 1): node t's conv input is its parent's window
  (the base window for the root) followed by x[t]; out[t] = silu(sum_k
  input[k] * w[k]); window[t] = input[1:].
* tree gated delta, state [Hv, Dv, Dk] per node: S = parent_state * g[t, h];
  kv[dv] = S[dv] . k[t, h // (Hv / Hk)]; delta = (v[t, h] - kv) * beta[t, h];
  S += delta (outer) k; y[t, h, dv] = S[dv] . q[t, hk]; states[t] = S.
  ``g`` is the multiplicative decay (compute_g already exponentiated).
* commit (qwen35_tree.py:708-732): the base window / state become those of the
  last accepted node.

Pinned (tests/test_oracle_gdn.py) by: the closed form of the conv window (last
K rows of base + inputs along the root path), the chain-tree case against
transformers' torch_recurrent_gated_delta_rule (an independent library
implementation, after transposing its [Dk, Dv] state, scaling its q by
sqrt(Dk) and passing log-decays), and the path decomposition of the tree
(every node equals the chain along its root path).
"""
from __future__ import annotations

import numpy as np


def silu(x):
    with np.errstate(over="ignore"):  # exp(-x) -> inf gives the limit -0 for x -> -inf
        return x / (1.0 + np.exp(-x))


def tree_conv1d(x: np.ndarray, base: np.ndarray, w: np.ndarray, parents) -> tuple[np.ndarray, np.ndarray]:
    """x [T, C], base [Keep, C], w [Keep + 1, C] -> (out [T, C], windows [T, Keep, C])."""
    x = np.asarray(x, np.float64)
    base = np.asarray(base, np.float64)
    w = np.asarray(w, np.float64)
    T, C = x.shape
    keep = base.shape[0]
    out = np.zeros((T, C))
    win = np.zeros((T, keep, C))
    for t in range(T):
        p = int(parents[t])
        prev = base if p < 0 else win[p]
        inp = np.concatenate([prev, x[t:t + 1]], axis=0)
        out[t] = silu((inp * w).sum(0))
        win[t] = inp[1:]
    return out, win


def tree_gated_delta(q, k, v, g, beta, state, parents) -> tuple[np.ndarray, np.ndarray]:
    """q, k [T, Hk, Dk]; v [T, Hv, Dv]; g, beta [T, Hv]; state [Hv, Dv, Dk]
    -> (y [T, Hv, Dv], states [T, Hv, Dv, Dk])."""
    q, k, v, g, beta, state = (np.asarray(a, np.float64) for a in (q, k, v, g, beta, state))
    T, Hk, Dk = k.shape
    Hv, Dv = v.shape[1], v.shape[2]
    grp = Hv // Hk
    y = np.zeros((T, Hv, Dv))
    states = np.zeros((T, Hv, Dv, Dk))
    for t in range(T):
        p = int(parents[t])
        S = (state if p < 0 else states[p]) * g[t][:, None, None]
        kk = k[t][np.arange(Hv) // grp]            # [Hv, Dk]
        qq = q[t][np.arange(Hv) // grp]
        kv = np.einsum("hvd,hd->hv", S, kk)
        delta = (v[t] - kv) * beta[t][:, None]
        S = S + delta[:, :, None] * kk[:, None, :]
        y[t] = np.einsum("hvd,hd->hv", S, qq)
        states[t] = S
    return y, states


def chain_conv1d(x: np.ndarray, base: np.ndarray, w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """tree_conv1d for a chain (parents t - 1) without the per-node windows:
    input row j of node t is row t + j of (base ++ x). -> (out [T, C], the
    last node's window [Keep, C])."""
    x = np.asarray(x, np.float64)
    base = np.asarray(base, np.float64)
    w = np.asarray(w, np.float64)
    keep = base.shape[0]
    rows = np.concatenate([base, x], axis=0)
    T = x.shape[0]
    acc = np.zeros_like(x)
    for j in range(keep + 1):
        acc += rows[j:j + T] * w[j]
    return silu(acc), rows[T:T + keep]


def chain_gated_delta(q, k, v, g, beta, state) -> tuple[np.ndarray, np.ndarray]:
    """tree_gated_delta for a chain, keeping only the running state:
    -> (y [T, Hv, Dv], the last node's state [Hv, Dv, Dk])."""
    q, k, v, g, beta = (np.asarray(a, np.float64) for a in (q, k, v, g, beta))
    S = np.array(state, np.float64)
    T, Hk, _ = k.shape
    Hv, Dv = v.shape[1], v.shape[2]
    grp = Hv // Hk
    y = np.zeros((T, Hv, Dv))
    for t in range(T):
        S *= g[t][:, None, None]
        kk = k[t][np.arange(Hv) // grp]
        qq = q[t][np.arange(Hv) // grp]
        delta = (v[t] - np.einsum("hvd,hd->hv", S, kk)) * beta[t][:, None]
        S += delta[:, :, None] * kk[:, None, :]
        y[t] = np.einsum("hvd,hd->hv", S, qq)
    return y, S


def root_path(parents, t: int) -> list[int]:
    path = []
    while t >= 0:
        path.append(t)
        t = int(parents[t])
    return path[::-1]


def commit(x, base_window, q, k, v, g, beta, state, parents, accepted):
    """New (window, state) after accepting nodes `accepted` (a root path,
    accepted[0] = 0): the window and state of accepted[-1]."""
    _, win = tree_conv1d(x, base_window, np.zeros((base_window.shape[0] + 1, x.shape[1])), parents)
    _, states = tree_gated_delta(q, k, v, g, beta, state, parents)
    last = accepted[-1]
    return win[last], states[last]
