"""GatedDeltaNet tree primitives on the GPU against the float64 oracle
(oracle/gdn.py), through the C-ABI: the reference kernel tests' own seeded
inputs (tests/test_qwen35_tree_kernels.py, tolerance 1e-5 as there), the
Qwen3.5 layer shapes (conv_dim 8192; 16 key / 32 value heads of 128) on 25- and
65-node trees, and the lazy commit of an accepted path."""
import ctypes as C

import numpy as np
import pytest
import torch

from gpu_util import random_tree, stream
from oracle import gdn

from dtree_hip import _native as N
from dtree_hip._native import DtreeError

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def _conv(x, base, w, parents, dev, want_windows=True):
    T, Cc = x.shape
    keep = base.shape[0]
    out = torch.zeros(T, Cc, device=dev)
    win = torch.zeros(T, keep, Cc, device=dev) if want_windows else None
    par = torch.tensor(parents, dtype=torch.int32, device=dev)
    xs, bs, ws = _t(x, dev), _t(base, dev), _t(w, dev)  # held until the kernel has run
    N.check(N.lib().dtree_gdn_tree_conv(xs.data_ptr(), bs.data_ptr(), ws.data_ptr(),
                                        par.data_ptr(), T, Cc, keep, out.data_ptr(),
                                        win.data_ptr() if win is not None else None, stream()), "gdn conv")
    torch.cuda.synchronize()
    return out.cpu().numpy(), (win.cpu().numpy() if win is not None else None)


def _delta(q, k, v, g, beta, state, parents, dev, want_states=True):
    T, Hk, Dk = k.shape
    Hv, Dv = v.shape[1], v.shape[2]
    y = torch.zeros(T, Hv, Dv, device=dev)
    st = torch.zeros(T, Hv, Dv, Dk, device=dev) if want_states else None
    par = torch.tensor(parents, dtype=torch.int32, device=dev)
    keep = [_t(a, dev) for a in (q, k, v, g, beta, state)]
    N.check(N.lib().dtree_gdn_tree_recurrence(*[a.data_ptr() for a in keep], par.data_ptr(), T, Hk, Hv, Dk, Dv,
                                              y.data_ptr(), st.data_ptr() if st is not None else None, stream()),
            "gdn recurrence")
    torch.cuda.synchronize()
    return y.cpu().numpy(), (st.cpu().numpy() if st is not None else None)


def test_reference_seeded_conv():
    x = np.random.default_rng(0).normal(size=(1, 5, 8)).astype(np.float32)[0]
    base = np.random.default_rng(1).normal(size=(1, 3, 8)).astype(np.float32)[0]
    w = np.random.default_rng(2).normal(size=(4, 8)).astype(np.float32)
    out, win = _conv(x, base, w, [-1, 0, 0, 1, 2], "cuda")
    ro, rw = gdn.tree_conv1d(x, base, w, [-1, 0, 0, 1, 2])
    np.testing.assert_allclose(out, ro, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(win, rw, atol=1e-5, rtol=1e-5)


def test_reference_seeded_recurrence():
    rng = np.random.default_rng(3)
    q = rng.normal(size=(1, 5, 1, 32)).astype(np.float32)[0]
    k = rng.normal(size=(1, 5, 1, 32)).astype(np.float32)[0]
    v = rng.normal(size=(1, 5, 1, 8)).astype(np.float32)[0]
    g = rng.normal(size=(1, 5, 1)).astype(np.float32)[0]
    beta = rng.normal(size=(1, 5, 1)).astype(np.float32)[0]
    state = rng.normal(size=(1, 1, 8, 32)).astype(np.float32)[0]
    y, st = _delta(q, k, v, g, beta, state, [-1, 0, 0, 1, 2], "cuda")
    ry, rs = gdn.tree_gated_delta(q, k, v, g, beta, state, [-1, 0, 0, 1, 2])
    np.testing.assert_allclose(y, ry, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(st, rs, atol=1e-5, rtol=1e-5)


def _layer_inputs(T, seed, Hk=16, Hv=32, D=128):
    """Recurrence inputs at the Qwen3.5 GDN scales: q = rms(q) / D, k = rms(k) /
    sqrt(D) (qwen35_tree.py:304-306), decay in (0, 1), beta = sigmoid."""
    g_ = np.random.default_rng(seed)

    def rms(a):
        return a / np.sqrt((a * a).mean(-1, keepdims=True) + 1e-6)

    q = rms(g_.normal(size=(T, Hk, D))) / D
    k = rms(g_.normal(size=(T, Hk, D))) / np.sqrt(D)
    v = g_.normal(size=(T, Hv, D))
    g = np.exp(-np.exp(g_.normal(size=(T, Hv)) * 0.5) * 0.3)
    beta = 1 / (1 + np.exp(-g_.normal(size=(T, Hv))))
    state = g_.normal(size=(Hv, D, D)) * 0.1
    return q, k, v, g, beta, state


@pytest.mark.parametrize("T,seed", [(25, 0), (65, 1), (96, 2)])
def test_layer_shapes_conv_and_recurrence(T, seed):
    parents = random_tree(T, seed)
    g_ = np.random.default_rng(100 + seed)
    x = g_.normal(size=(T, 8192))
    base = g_.normal(size=(3, 8192))
    w = g_.normal(size=(4, 8192)) * 0.5
    out, win = _conv(x, base, w, parents, "cuda")
    ro, rw = gdn.tree_conv1d(x, base, w, parents)
    np.testing.assert_allclose(out, ro, atol=2e-5, rtol=2e-5)
    np.testing.assert_array_equal(win, rw.astype(np.float32))
    q, k, v, g, beta, state = _layer_inputs(T, seed)
    y, st = _delta(q, k, v, g, beta, state, parents, "cuda")
    ry, rs = gdn.tree_gated_delta(q, k, v, g, beta, state, parents)
    assert np.abs(y - ry).max() <= 1e-5 * max(1.0, np.abs(ry).max())
    assert np.abs(st - rs).max() <= 1e-5 * max(1.0, np.abs(rs).max())
    # lazy mode (no node states / windows written) gives the same outputs; it
    # runs the matrix form (gdn_tree_chunk_kernel up to 32 nodes,
    # gdn_tree_blocks_kernel up to 96), which sums in another order
    y2, _ = _delta(q, k, v, g, beta, state, parents, "cuda", want_states=False)
    out2, _ = _conv(x, base, w, parents, "cuda", want_windows=False)
    assert np.array_equal(out, out2)
    assert np.abs(y2 - ry).max() <= 1e-5 * max(1.0, np.abs(ry).max())


def _star(T):
    return [-1] + [0] * (T - 1)


@pytest.mark.parametrize("parents,scale", [
    (random_tree(25, 11), "model"), (random_tree(32, 12), "model"), (list(range(-1, 31)), "model"),
    (_star(32), "model"), ([-1], "model"), (random_tree(17, 13), "strong_decay"),
    (random_tree(25, 14), "no_decay"), (random_tree(25, 15), "signed"),
], ids=["rand25", "rand32", "chain32", "star32", "root_only", "strong_decay", "no_decay", "signed_g_beta"])
def test_matrix_form_recurrence(parents, scale):
    """Trees of up to 32 nodes without node states run the matrix form
    (gdn_tree_chunk_kernel: Gram matrices and S_0 products on MFMA, a forward
    substitution per value row). Against the node-by-node float64 oracle on
    model-scale inputs, a 32-deep chain and a 31-leaf star, decays that
    vanish (g ~ 1e-30) or are exactly 1, and the reference kernel test's
    signed g / beta (no positivity assumed)."""
    T = len(parents)
    q, k, v, g, beta, state = _layer_inputs(T, 500 + T)
    if scale == "strong_decay":
        g = np.where(np.arange(T)[:, None] % 3 == 1, 1e-30, g)
    elif scale == "no_decay":
        g = np.ones_like(g)
    elif scale == "signed":
        r = np.random.default_rng(7)
        g, beta = r.normal(size=g.shape) * 0.9, r.normal(size=beta.shape)
    y, _ = _delta(q, k, v, g, beta, state, parents, "cuda", want_states=False)
    ry, _ = gdn.tree_gated_delta(q, k, v, g, beta, state, parents)
    assert np.abs(y - ry).max() <= 1e-5 * max(1.0, np.abs(ry).max())


def _chain_tree(T, depth, seed):
    """Nodes 0 .. depth form a chain (the deepest node at depth `depth`); the
    rest hang off random earlier nodes."""
    g_ = np.random.default_rng(seed)
    return [-1] + list(range(depth)) + [int(g_.integers(0, i)) for i in range(depth + 1, T)]


def _caterpillar(n_branching):
    """A path whose first n_branching nodes each also carry a leaf: node 2j is
    path node j (children: leaf 2j + 1 and path node 2j + 2), so path node j
    has j branching ancestors."""
    par = [-1]
    for j in range(n_branching):
        par += [2 * j, 2 * j]
    return par


@pytest.mark.parametrize("parents", [
    _chain_tree(40, 30, 70), _chain_tree(96, 21, 117), _chain_tree(65, 15, 80), _chain_tree(33, 1, 34),
    list(range(-1, 95)),   # a 96-node chain (prompt prefill runs such chains): no stack slot
    _caterpillar(31),      # 63 nodes, 31 nested branching nodes: the stack's last slot
], ids=["chain30+9", "chain21+74", "chain15+49", "bushy33", "chain96", "caterpillar31"])
def test_recurrence_depth_first_trees(parents):
    """33-96 nodes run depth first, keeping the states of branching nodes on a
    stack (gdn_tree_dfs_kernel): deep chains with side branches, a plain
    96-node chain, a bushy tree and a caterpillar that fills the stack, against
    the float64 oracle."""
    T = len(parents)
    q, k, v, g, beta, state = _layer_inputs(T, T)
    y, st = _delta(q, k, v, g, beta, state, parents, "cuda")
    ry, rs = gdn.tree_gated_delta(q, k, v, g, beta, state, parents)
    assert np.abs(y - ry).max() <= 1e-5 * max(1.0, np.abs(ry).max())
    assert np.abs(st - rs).max() <= 1e-5 * max(1.0, np.abs(rs).max())
    # without node states the same trees run the blocked matrix form
    y2, _ = _delta(q, k, v, g, beta, state, parents, "cuda", want_states=False)
    assert np.abs(y2 - ry).max() <= 1e-5 * max(1.0, np.abs(ry).max())


@pytest.mark.parametrize("parents,scale", [
    (random_tree(65, 21), "model"), (random_tree(96, 22), "model"), (list(range(-1, 95)), "model"),
    (_star(96), "model"), (_caterpillar(32), "model"), (_caterpillar(47), "model"),
    (_chain_tree(64, 40, 23), "model"), (random_tree(33, 24), "model"), (random_tree(80, 25), "strong_decay"),
    (random_tree(70, 26), "no_decay"), (random_tree(65, 27), "signed"),
], ids=["rand65", "rand96", "chain96", "star96", "caterpillar32", "caterpillar47", "chain40+23", "rand33",
        "strong_decay", "no_decay", "signed_g_beta"])
def test_blocked_matrix_form_recurrence(parents, scale):
    """Trees of 33-96 nodes without node states run the matrix form in
    32-node blocks (gdn_tree_blocks_kernel: each block's diagonal inverted by
    squaring, earlier blocks entering through their finished Delta rows).
    Against the node-by-node float64 oracle: random trees, a 96-deep chain
    (31 in-block ancestors in every block), a 95-leaf star, caterpillars
    past the depth-first walk's 31 nested branch points (no limit here),
    vanishing, unit and signed decays."""
    T = len(parents)
    q, k, v, g, beta, state = _layer_inputs(T, 700 + T)
    if scale == "strong_decay":
        g = np.where(np.arange(T)[:, None] % 3 == 1, 1e-30, g)
    elif scale == "no_decay":
        g = np.ones_like(g)
    elif scale == "signed":
        r = np.random.default_rng(9)
        g, beta = r.normal(size=g.shape) * 0.9, r.normal(size=beta.shape)
    y, _ = _delta(q, k, v, g, beta, state, parents, "cuda", want_states=False)
    ry, _ = gdn.tree_gated_delta(q, k, v, g, beta, state, parents)
    assert np.abs(y - ry).max() <= 1e-5 * max(1.0, np.abs(ry).max())


def test_recurrence_forest_of_roots():
    """Nodes without a valid parent (-1, or an index not below the node) start
    from the committed state; the depth-first order visits each root's subtree
    in turn."""
    T = 48
    parents = random_tree(T, 11)
    for t in (5, 17, 30):
        parents[t] = -1
    parents[40] = 45  # not below the node: treated as a root
    q, k, v, g, beta, state = _layer_inputs(T, 12)
    y, _ = _delta(q, k, v, g, beta, state, parents, "cuda", want_states=False)
    ref_par = [p if 0 <= p < t else -1 for t, p in enumerate(parents)]
    ry, _ = gdn.tree_gated_delta(q, k, v, g, beta, state, ref_par)
    assert np.abs(y - ry).max() <= 1e-5 * max(1.0, np.abs(ry).max())


def test_recurrence_past_the_stack_writes_nan():
    """32 nested branching nodes (a 65-node caterpillar) do not fit the
    depth-first walk's 32-slot stack (the walk runs when node states are
    asked for): the kernel, called on such a tree anyway, writes NaN, never a
    silently wrong value (the host check dtree_gdn_tree_check rejects the
    tree before launch: tests/test_native_abi.py, and the hybrid engine
    below)."""
    parents = _caterpillar(32)
    T = len(parents)
    q, k, v, g, beta, state = _layer_inputs(T, 13)
    y, _ = _delta(q, k, v, g, beta, state, parents, "cuda", want_states=True)
    assert np.isnan(y).all()


def test_hybrid_engine_rejects_trees_past_the_stack(gpu_device):
    """The hybrid engine checks caller trees of more than 32 nodes on the host
    (dtree_gdn_tree_check) and raises before any launch."""
    from dtree_hip import Qwen35TreeEngine, Qwen35Weights, tiny_qwen35
    cfg = tiny_qwen35()
    w = Qwen35Weights.random(cfg, seed=5, device=gpu_device)
    eng = Qwen35TreeEngine(cfg, w, max_past=64, max_nodes=96)
    par = _caterpillar(32)
    with pytest.raises(DtreeError, match="nested branching"):
        eng.set_step([3] * len(par), [10] * len(par), par, 10)
    ok = _caterpillar(31)
    eng.set_step([3] * len(ok), [10] * len(ok), ok, 10)


def test_recurrence_rejects_trees_past_96_nodes():
    """Head dim 128: trees of up to 96 nodes run register-resident (up to 32
    nodes) or depth first; larger ones do not fit the LDS-resident fallback
    either and are rejected."""
    q, k, v, g, beta, state = _layer_inputs(128, 3)
    with pytest.raises(DtreeError, match="too large"):
        _delta(q, k, v, g, beta, state, random_tree(128, 3), "cuda")


def test_commit_replays_accepted_path():
    T = 25
    parents = random_tree(T, 7)
    # accepted = root path of the deepest node
    depth = [0] * T
    for t in range(1, T):
        depth[t] = depth[parents[t]] + 1
    path = gdn.root_path(parents, int(np.argmax(depth)))
    g_ = np.random.default_rng(8)
    x = g_.normal(size=(T, 8192))
    base = g_.normal(size=(3, 8192))
    q, k, v, g, beta, state = _layer_inputs(T, 9)
    dev = "cuda"
    win_d, st_d = _t(base, dev), _t(state, dev)
    pbuf = torch.zeros(129, dtype=torch.int32, device=dev)
    pbuf[: len(path)] = torch.tensor(path, dtype=torch.int32)
    plen = torch.tensor([len(path)], dtype=torch.int32, device=dev)
    keep = [_t(a, dev) for a in (x, q, k, v, g, beta)]
    N.check(N.lib().dtree_gdn_commit(keep[0].data_ptr(), win_d.data_ptr(), 8192, 3, *[a.data_ptr() for a in keep[1:]],
                                     st_d.data_ptr(), pbuf.data_ptr(), plen.data_ptr(), 16, 32, 128, 128, stream()),
            "gdn commit")
    torch.cuda.synchronize()
    rw, rs = gdn.commit(x, base, q, k, v, g, beta, state, parents, path)
    np.testing.assert_array_equal(win_d.cpu().numpy(), rw.astype(np.float32))
    assert np.abs(st_d.cpu().numpy() - rs).max() <= 1e-5 * max(1.0, np.abs(rs).max())
    # a one-node path (only the root accepted) shifts the window by one row
    win1 = _t(base, dev)
    plen.fill_(1)
    N.check(N.lib().dtree_gdn_commit(keep[0].data_ptr(), win1.data_ptr(), 8192, 3, None, None, None, None, None, None,
                                     pbuf.data_ptr(), plen.data_ptr(), 16, 32, 128, 128, stream()), "gdn commit")
    torch.cuda.synchronize()
    np.testing.assert_array_equal(win1.cpu().numpy(), np.concatenate([base[1:], x[path[:1]]]).astype(np.float32))


@pytest.mark.parametrize("T,seed", [(25, 3), (32, 4), (1, 5), (17, 6)])
def test_layer_prep_and_recurrence_in_one_launch(gpu_device, T, seed):
    """dtree_gdn_layer_prep_recurrence (one launch for trees of up to 32 nodes)
    against dtree_gdn_layer_prep + dtree_gdn_layer_recurrence on the same
    inputs: v, g and beta bit for bit (same conv window, tap order and
    formulas), q and k to the rounding of the RMS sum's order, y to 1e-5 of its
    scale. Both read the node count and parents from the step descriptor."""
    from gpu_util import device_desc

    dev = gpu_device
    g_ = np.random.default_rng(seed)
    Hk, Hv, D, keep, MP = 16, 32, 128, 3, 32
    key_dim, value_dim = Hk * D, Hv * D
    conv_c = 2 * key_dim + value_dim
    ld = conv_c + value_dim + 2 * Hv
    parents = random_tree(T, seed)
    desc = device_desc([0] * T, [5] * T, parents, 100, dev)
    proj = torch.zeros(MP, ld, device=dev)
    proj[:T] = torch.from_numpy(g_.normal(size=(T, ld)).astype(np.float32)).to(dev)
    window = torch.from_numpy(g_.normal(size=(keep, conv_c)).astype(np.float32)).to(dev)
    conv_w = torch.from_numpy((g_.normal(size=(keep + 1, conv_c)) * 0.5).astype(np.float32)).to(dev)
    A_log = torch.from_numpy(g_.uniform(0, 2.7, size=Hv).astype(np.float32)).to(dev)
    dt_bias = torch.ones(Hv, device=dev)
    state = torch.from_numpy((g_.normal(size=(Hv, D, D)) * 0.1).astype(np.float32)).to(dev)

    def run(fused):
        out = {n: torch.full((MP, w), 7.0, device=dev) for n, w in
               (("q", key_dim), ("k", key_dim), ("v", value_dim), ("g", Hv), ("beta", Hv), ("y", value_dim))}
        a = N.GdnArgs()
        a.desc = desc.data_ptr(); a.rows_padded = MP
        a.num_k_heads = Hk; a.num_v_heads = Hv; a.head_k_dim = D; a.head_v_dim = D; a.conv_keep = keep
        a.proj = proj.data_ptr(); a.ld_proj = ld
        a.window = window.data_ptr(); a.conv_w = conv_w.data_ptr()
        a.A_log = A_log.data_ptr(); a.dt_bias = dt_bias.data_ptr(); a.state = state.data_ptr()
        a.q = out["q"].data_ptr(); a.k = out["k"].data_ptr(); a.v = out["v"].data_ptr()
        a.g = out["g"].data_ptr(); a.beta = out["beta"].data_ptr(); a.y = out["y"].data_ptr()
        lib = N.lib()
        if fused:
            N.check(lib.dtree_gdn_layer_prep_recurrence(C.byref(a), stream()), "prep + recurrence")
        else:
            N.check(lib.dtree_gdn_layer_prep(C.byref(a), stream()), "prep")
            N.check(lib.dtree_gdn_layer_recurrence(C.byref(a), stream()), "recurrence")
        torch.cuda.synchronize()
        return {n: t[:T].cpu().numpy() for n, t in out.items()}

    window0, state0 = window.clone(), state.clone()
    sep, fus, fus2 = run(False), run(True), run(True)
    for n in ("v", "g", "beta"):
        assert np.array_equal(sep[n], fus[n]), n
    for n in ("q", "k"):
        np.testing.assert_allclose(fus[n], sep[n], rtol=1e-5, atol=1e-7, err_msg=n)
    assert np.abs(fus["y"] - sep["y"]).max() <= 1e-5 * max(1.0, np.abs(sep["y"]).max())
    for n in fus:
        assert np.array_equal(fus[n], fus2[n]), n  # repeatable
    # the committed window and state are read, not written
    assert torch.equal(window, window0) and torch.equal(state, state0) and np.isfinite(fus["y"]).all()


@pytest.mark.parametrize("nl", [3, 34])
def test_layers_commit_in_one_launch(gpu_device, nl):
    """dtree_gdn_layers_commit against dtree_gdn_layer_commit per layer (the
    same body on each layer's window and state): bit for bit. 34 layers take
    two launches (32 layers per launch)."""
    from gpu_util import device_desc

    dev = gpu_device
    g_ = np.random.default_rng(11 + nl)
    Hk, Hv, D, keep, MP = 16, 32, 128, 3, 32
    key_dim, value_dim = Hk * D, Hv * D
    conv_c = 2 * key_dim + value_dim
    ld = conv_c + value_dim + 2 * Hv
    parents = random_tree(25, 7)
    desc = device_desc([0] * 25, [5] * 25, parents, 100, dev, accepted=[0, 3, 9, 14])

    def t(*shape, scale=1.0):
        return torch.from_numpy((g_.normal(size=shape) * scale).astype(np.float32)).to(dev)

    layers = [dict(proj=t(MP, ld), window=t(keep, conv_c), state=t(Hv, D, D, scale=0.1), q=t(MP, key_dim),
                   k=t(MP, key_dim, scale=0.1), v=t(MP, value_dim), g=torch.rand(MP, Hv, device=dev),
                   beta=torch.rand(MP, Hv, device=dev)) for _ in range(nl)]

    def args(ly):
        a = N.GdnArgs()
        a.desc = desc.data_ptr(); a.rows_padded = MP
        a.num_k_heads = Hk; a.num_v_heads = Hv; a.head_k_dim = D; a.head_v_dim = D; a.conv_keep = keep
        a.proj = ly["proj"].data_ptr(); a.ld_proj = ld
        a.window = ly["window"].data_ptr(); a.state = ly["state"].data_ptr()
        for n in ("q", "k", "v", "g", "beta"):
            setattr(a, n, ly[n].data_ptr())
        return a

    before = [{n: ly[n].clone() for n in ("window", "state")} for ly in layers]
    for ly in layers:
        N.check(N.lib().dtree_gdn_layer_commit(C.byref(args(ly)), stream()), "commit")
    torch.cuda.synchronize()
    one = [{n: ly[n].clone() for n in ("window", "state")} for ly in layers]
    for ly, b in zip(layers, before):
        for n in ("window", "state"):
            ly[n].copy_(b[n])
    arr = (N.GdnArgs * nl)(*[args(ly) for ly in layers])
    N.check(N.lib().dtree_gdn_layers_commit(arr, nl, stream()), "layers commit")
    torch.cuda.synchronize()
    for ly, o, b in zip(layers, one, before):
        for n in ("window", "state"):
            assert torch.equal(ly[n], o[n]), n
        assert not torch.equal(ly["state"], b["state"])  # the commit did advance the state
    # into separate destinations: the same results, the sources untouched
    for ly, b in zip(layers, before):
        for n in ("window", "state"):
            ly[n].copy_(b[n])
    dst = [{n: torch.full_like(ly[n], float("nan")) for n in ("window", "state")} for ly in layers]
    arr = (N.GdnArgs * nl)(*[args(ly) for ly in layers])
    for i, d in enumerate(dst):
        arr[i].window_out = d["window"].data_ptr(); arr[i].state_out = d["state"].data_ptr()
    N.check(N.lib().dtree_gdn_layers_commit(arr, nl, stream()), "layers commit into spare buffers")
    torch.cuda.synchronize()
    for ly, d, o, b in zip(layers, dst, one, before):
        for n in ("window", "state"):
            assert torch.equal(d[n], o[n]), n
            assert torch.equal(ly[n], b[n]), n
