"""Helpers shared by the GPU parity tests (no kernels launched at import)."""
from __future__ import annotations

import ctypes as C
import warnings

import numpy as np
import pytest
import torch

from dtree_hip import _native as N
from dtree_hip.engine import ancestor_bitsets


def to_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def bf16_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def device_desc(tokens, positions, parents, past_length, device, accepted=None, ancestors=None) -> torch.Tensor:
    d = N.StepDesc()
    L = len(tokens)
    anc = ancestor_bitsets(parents) if ancestors is None else ancestors
    d.past_length = past_length
    d.num_nodes = L
    for i in range(L):
        d.tokens[i] = int(tokens[i])
        d.positions[i] = int(positions[i])
        d.parents[i] = int(parents[i])
        for w in range(N.MASK_WORDS):
            d.ancestors[i][w] = int(anc[i, w])
    if accepted is not None:
        d.n_accepted = len(accepted)
        for i, a in enumerate(accepted):
            d.accepted[i] = int(a)
    buf = (C.c_uint8 * C.sizeof(d)).from_buffer_copy(bytes(d))
    host = torch.frombuffer(bytearray(bytes(buf)), dtype=torch.uint8)
    return host.to(device)


def read_desc(t: torch.Tensor) -> N.StepDesc:
    raw = bytes(t.cpu().numpy().tobytes())
    return N.StepDesc.from_buffer_copy(raw)


def tree_mask(parents, P: int) -> np.ndarray:
    """[L, P + L] visibility: every prefix key, and each node's ancestors and
    itself (walked from the parent list, independent of the bitset packing)."""
    L = len(parents)
    m = np.zeros((L, P + L), bool)
    m[:, :P] = True
    for i in range(L):
        j = i
        while j >= 0:
            m[i, P + j] = True
            j = parents[j]
    return m


def random_tree(L: int, seed: int) -> list[int]:
    g = np.random.default_rng(seed)
    return [-1] + [int(g.integers(0, i)) for i in range(1, L)]


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def compare_accepted_path(res, child_maps, oracle_post, decided, log=print, note: str = "") -> int:
    """Accepted path of the device walk against the oracle's walk over the
    oracle's own argmax (follow_verified_tree, dtree_runtime.py:195-208).

    ``decided[i]`` says row i's argmax is pinned (its oracle top-2 margin
    clears the logit tolerance). Both walks visit the same nodes up to and
    including the first walked node whose row is not decided; past it the
    device may legitimately take another branch. Asserts equality on that
    prefix (and of the bonus token when the whole oracle path is decided) and
    returns how many path nodes were compared. ``note`` (e.g. the logit
    error) is appended to the record."""
    from oracle import tree as otree

    o_acc, o_bonus = otree.follow_verified_tree(child_maps, [int(t) for t in oracle_post])
    k = next((j for j, i in enumerate(o_acc) if not decided[i]), None)
    if k is None:
        assert res.accepted == o_acc and res.bonus_token == o_bonus, (res.accepted, o_acc)
        compared = len(o_acc)
    else:
        assert res.accepted[:k + 1] == o_acc[:k + 1], (res.accepted, o_acc, k)
        compared = k + 1
    msg = (f"accepted path: device {res.accepted} bonus {res.bonus_token}; oracle {o_acc} bonus {o_bonus}; "
           f"compared {compared} of {len(o_acc)} nodes" + ("" if k is None else f" (node {o_acc[k]} undecided)")
           + (f"; {note}" if note else ""))
    log(msg)
    # a record pytest -q shows in its warnings summary
    warnings.warn(PathParityRecord(msg), stacklevel=2)
    assert compared >= 1, msg
    return compared


class PathParityRecord(UserWarning):
    """How many accepted-path nodes a parity test compared bit for bit."""


def require_path_compared(compared: int, what: str) -> None:
    """Full-size steps: a path comparison that covered the root alone (its row
    undecided, or the oracle walk stopping there) proves nothing; mark the
    test xfail with the reason instead of passing it."""
    if compared < 2:
        pytest.xfail(f"{what}: the accepted-path comparison covered only {compared} node(s) (the root)")
