"""Qwen3.5 hybrid verify step on the GPU (GatedDeltaNet + gated attention
layers, LM-head argmax, accept walk, KV compaction and the GatedDeltaNet
commit) against the oracle (oracle/qwen35.py) on the same weights, committed
state and tree.

The oracle starts from the device's committed state after the prefill (KV
prefix of the attention layers, conv windows and recurrent states of the
GatedDeltaNet layers), so the check isolates one step; the prefill itself is
checked against the oracle's chain commit separately.

Bars: logits within 2e-2 relative (max |diff| per row <= 2e-2 x max |oracle
logit| of that row); argmax tokens bit-exact on rows whose oracle top-2
margin exceeds that tolerance; accepted path bit-exact up to and including the
first walked node without such a margin; compacted attention cache = the pre-compaction
rows gathered at the accepted indices, bit for bit; committed windows and
states within 2e-2 of the oracle's commit along the device's accepted path."""
import time

import numpy as np
import pytest
import torch

from dtree_hip import Qwen35TreeEngine, Qwen35Weights, tiny_qwen35
from dtree_hip.config import QWEN35_4B
from dtree_hip.synthetic import acceptance_rewrite, make_tree, random_prefix
from oracle import qwen35 as o35
from oracle import tree as otree
from oracle.qwen3 import bf16_to_f32

from gpu_util import bf16_f32, compare_accepted_path, require_path_compared

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _oracle_cfg(c):
    return o35.Qwen35Config(
        hidden=c.hidden_size, layers=c.num_hidden_layers, ffn=c.intermediate_size, heads=c.num_attention_heads,
        kv_heads=c.num_key_value_heads, head_dim=c.head_dim, rope_dims=c.rope_dims,
        lin_k_heads=c.linear_num_key_heads, lin_v_heads=c.linear_num_value_heads, lin_k_dim=c.linear_key_head_dim,
        lin_v_dim=c.linear_value_head_dim, conv_kernel=c.linear_conv_kernel_dim,
        full_attention_interval=c.full_attention_interval, vocab=c.vocab_size, eps=c.rms_norm_eps,
        rope_base=c.rope_theta)


def _oracle_cache(cfg, cache, P):
    """The device's committed state as an oracle cache (fp32)."""
    layers = []
    for li in range(cfg.num_hidden_layers):
        s = cache.slot[li]
        if cfg.is_linear(li):
            layers.append((cache.windows[s].cpu().numpy().copy(), cache.states[s].cpu().double().numpy().copy()))
        else:
            layers.append((bf16_f32(cache.kv.logical_keys(s, P)), bf16_f32(cache.kv.logical_values(s, P))))
    return o35.Qwen35Cache(layers=layers, offset=P)


def _close(got, want, what):
    err = np.abs(np.asarray(got, np.float64) - want).max()
    assert err <= TOL * max(1.0, np.abs(want).max()), f"{what}: max err {err}"


def _check_long_prefill(orc, cfg, cache, prefix, layers, log=print):
    """The long-M prefill at full size against the oracle's causal chain
    (chain_prefill: forward + commit of the whole prompt) over the first
    `layers` layers: each GatedDeltaNet layer's committed window and state and
    each attention layer's K / V at every position."""
    t0 = time.time()
    P = len(prefix)
    _, want = orc.chain_prefill(prefix, layers)
    for li in range(layers):
        s = cache.slot[li]
        if cfg.is_linear(li):
            _close(cache.windows[s].cpu().numpy(), want[li][0], f"prefill window {li}")
            _close(cache.states[s].cpu().numpy(), want[li][1], f"prefill state {li}")
        else:
            _close(bf16_f32(cache.kv.logical_keys(s, P)), want[li][0], f"prefill keys {li}")
            _close(bf16_f32(cache.kv.logical_values(s, P)), want[li][1], f"prefill values {li}")
    log(f"long prefill: {layers} layers' committed state at P={P} match the oracle ({time.time() - t0:.1f}s)")


def _run(cfg, P, layer_ids, dev, norm_jitter=0.1, quant="bf16", log=print, check_prefill=False, budget=24,
         check_long_prefill_layers=0):
    t0 = time.time()
    w = Qwen35Weights.random(cfg, seed=0, device=dev, norm_jitter=norm_jitter, quant=quant)
    eng = Qwen35TreeEngine(cfg, w, max_past=P + 64, layer_ids=layer_ids, max_nodes=budget + 1)
    cache = eng.new_cache()
    prefix = random_prefix(P, cfg.vocab_size, seed=1)
    eng.prefill(cache, prefix)
    torch.cuda.synchronize()
    assert cache.offset == P
    orc = o35.OracleQwen35(_oracle_cfg(cfg), w.host_accessor())
    if check_prefill:
        oc = orc.new_cache()
        chain = [-1] + list(range(P - 1))
        _, _, pend = orc.forward_tree(np.asarray(prefix), np.arange(P), chain, oc)
        orc.commit(oc, pend, chain, list(range(P)))
        for li in cfg.linear_layers:
            s = cache.slot[li]
            _close(cache.windows[s].cpu().numpy(), oc.layers[li][0], f"prefill window {li}")
            _close(cache.states[s].cpu().numpy(), oc.layers[li][1], f"prefill state {li}")
        for li in cfg.attention_layers:
            _close(bf16_f32(cache.kv.logical_keys(cache.slot[li], P)), oc.layers[li][0], f"prefill keys {li}")
    if check_long_prefill_layers:
        _check_long_prefill(orc, cfg, cache, prefix, check_long_prefill_layers, log)
    st = eng.stream_handle()
    tree = make_tree(root_token=prefix[-1] if P else 0, vocab=cfg.vocab_size, seed=2, budget=budget)

    def argmax_at(tr):
        eng.set_step(tr.tokens, tr.positions(P), tr.parents, P)
        eng.launch_forward(cache, st)
        eng.launch_lm_head(st)
        eng.launch_walk(st)
        return eng.read_result().posterior

    path = acceptance_rewrite(tree, argmax_at, p=0.85, seed=3)
    L = tree.size
    log(f"setup {time.time() - t0:.1f}s  L={L} path={path}")

    # dry forward: logits + tree K/V rows before compaction
    eng.set_step(tree.tokens, tree.positions(P), tree.parents, P)
    eng.launch_forward(cache, st)
    eng.launch_lm_head(st, want_logits=True)
    torch.cuda.synchronize()
    logits = eng.logits[:L].cpu().numpy()
    nA = len(cfg.attention_layers)
    tree_k = [bf16_f32(cache.kv.logical_keys(a, P + L))[P:] for a in range(nA)]
    tree_v = [bf16_f32(cache.kv.logical_values(a, P + L))[P:] for a in range(nA)]
    hidden = bf16_f32(eng.hidden[:L]) if layer_ids else None
    oc = _oracle_cache(cfg, cache, P)

    # the real step: graph replay of forward + argmax + walk + compaction + commit
    res = eng.verify(cache, tree.tokens, tree.positions(P), tree.parents, use_graph=True)
    torch.cuda.synchronize()

    t1 = time.time()
    norm, vh, pend = orc.forward_tree(np.asarray(tree.tokens), np.asarray(tree.positions(P)), tree.parents, oc,
                                      layer_ids)
    E = w.host_accessor()(None, "embed")
    ref = np.concatenate([norm @ bf16_to_f32(E[s:s + 16384]).T for s in range(0, E.shape[0], 16384)], axis=1)
    log(f"oracle {time.time() - t1:.1f}s")
    return dict(cfg=cfg, eng=eng, cache=cache, tree=tree, res=res, logits=logits, ref=ref, tree_k=tree_k,
                tree_v=tree_v, hidden=hidden, vh=vh, P=P, L=L, orc=orc, oc=oc, pend=pend)


def _check(r, layer_ids, min_confident=0.5):
    cfg, L, P = r["cfg"], r["L"], r["P"]
    logits, ref, res, tree = r["logits"], r["ref"], r["res"], r["tree"]
    scale = np.abs(ref).max(axis=-1)
    err = np.abs(logits - ref).max(axis=-1)
    assert np.all(err <= TOL * scale), f"logit rel err {float((err / scale).max()):.4f}"
    srt = np.sort(ref, axis=-1)
    margin = srt[:, -1] - srt[:, -2]
    confident = margin > TOL * scale
    # Where every logit of a row is within err of the oracle, a top-2 margin
    # above 2 * err fixes the argmax whatever the logits' scale.
    sure = margin > 2 * err
    o_post = np.argmax(ref, axis=-1)
    post = np.array(res.posterior)
    assert np.array_equal(post[confident], o_post[confident])
    assert np.array_equal(post[sure], o_post[sure])
    assert confident.mean() >= min_confident and sure.mean() > 0.5
    note = (f"max logit err {float((err / scale).max()):.4f} of the row max (bar {TOL}); "
            f"{int(confident.sum())}/{len(confident)} rows confident, {int(sure.sum())} sure")
    r["path_compared"] = compare_accepted_path(res, tree.child_maps, o_post, confident | sure, note=note)
    acc2, bonus2 = otree.follow_verified_tree(tree.child_maps, res.posterior)
    assert res.accepted == acc2 and res.bonus_token == bonus2
    cache, n = r["cache"], len(res.accepted)
    assert cache.offset == P + n
    # attention layers: compaction is a bit-exact gather; tree rows match the oracle
    for a, li in enumerate(cfg.attention_layers):
        kc = bf16_f32(cache.kv.logical_keys(a, P + n))[P:]
        vc = bf16_f32(cache.kv.logical_values(a, P + n))[P:]
        np.testing.assert_array_equal(kc, r["tree_k"][a][res.accepted])
        np.testing.assert_array_equal(vc, r["tree_v"][a][res.accepted])
        _close(r["tree_k"][a], r["pend"][li]["k"], f"tree keys {li}")
        _close(r["tree_v"][a], r["pend"][li]["v"], f"tree values {li}")
    # GatedDeltaNet layers: window / state = the oracle's commit along the same path
    orc, oc = r["orc"], r["oc"]
    orc.commit(oc, r["pend"], tree.parents, res.accepted)
    for li in cfg.linear_layers:
        s = cache.slot[li]
        _close(cache.windows[s].cpu().numpy(), oc.layers[li][0], f"window {li}")
        _close(cache.states[s].cpu().numpy(), oc.layers[li][1], f"state {li}")
    if layer_ids:
        hs = bf16_f32(r["eng"].hidden_sel[:n])
        want = r["vh"][res.accepted]
        assert np.abs(hs - want).max() <= TOL * np.abs(want).max()
        assert np.abs(r["hidden"] - r["vh"]).max() <= TOL * np.abs(r["vh"]).max()
    return res


def test_qwen35_verify_step_tiny_model(gpu_device, attn_kernel):
    cfg = tiny_qwen35()
    r = _run(cfg, P=100, layer_ids=[1, 3], dev=gpu_device, check_prefill=True)
    res = _check(r, [1, 3])
    assert len(res.accepted) >= 1


def test_qwen35_verify_step_tiny_model_q4(gpu_device):
    cfg = tiny_qwen35()
    r = _run(cfg, P=70, layer_ids=[2], dev=gpu_device, quant="q4")
    _check(r, [2])


@pytest.mark.parametrize("quant", ["bf16", "q4"])
def test_qwen35_verify_step_65_nodes(gpu_device, quant, attn_kernel):
    """Draft budget 64 (a 65-node tree, 96 padded rows): attention over three
    32-row query blocks and tree chunks, q4 GEMMs per 32-row block, the
    GatedDeltaNet layer at 96 rows."""
    cfg = tiny_qwen35()
    r = _run(cfg, P=90, layer_ids=[1, 3], dev=gpu_device, quant=quant, budget=64)
    assert r["L"] == 65 and r["eng"].MP == 96
    _check(r, [1, 3])


def test_qwen35_two_steps_graph_matches_eager(gpu_device):
    """Two consecutive verify steps through the captured graph leave the same
    committed state as the same steps launched eagerly."""
    cfg = tiny_qwen35()
    w = Qwen35Weights.random(cfg, seed=5, device=gpu_device, norm_jitter=0.1)
    out = []
    for use_graph in (True, False):
        eng = Qwen35TreeEngine(cfg, w, max_past=128)
        cache = eng.new_cache()
        eng.prefill(cache, random_prefix(40, cfg.vocab_size, seed=6))
        res = []
        for step in range(2):
            tree = make_tree(root_token=7 + step, vocab=cfg.vocab_size, seed=10 + step)
            r = eng.verify(cache, tree.tokens, tree.positions(cache.offset), tree.parents, use_graph=use_graph)
            res.append((r.accepted, r.bonus_token))
        torch.cuda.synchronize()
        out.append((res, cache.windows.cpu(), cache.states.cpu(), cache.offset))
        eng.release_graphs()
    assert out[0][0] == out[1][0] and out[0][3] == out[1][3]
    assert torch.equal(out[0][1], out[1][1]) and torch.equal(out[0][2], out[1][2])


@pytest.mark.parametrize("use_graph", [True, False])
def test_qwen35_uncommitted_step_leaves_state(gpu_device, use_graph):
    """verify(commit=False) leaves the committed windows and states bit for bit
    as they were (its commit goes to the spare pair), so replays accept the
    same path; a kept step afterwards commits exactly what a kept step alone
    would have."""
    cfg = tiny_qwen35()
    w = Qwen35Weights.random(cfg, seed=5, device=gpu_device, norm_jitter=0.1)
    tree = make_tree(root_token=7, vocab=cfg.vocab_size, seed=10)
    out = []
    for preview in (3, 0):
        eng = Qwen35TreeEngine(cfg, w, max_past=128)
        cache = eng.new_cache()
        eng.prefill(cache, random_prefix(40, cfg.vocab_size, seed=6))
        torch.cuda.synchronize()
        P = cache.offset
        win0, st0 = cache.windows.clone(), cache.states.clone()
        first = None
        for _ in range(preview):
            r = eng.verify(cache, tree.tokens, tree.positions(P), tree.parents, use_graph=use_graph, commit=False)
            torch.cuda.synchronize()
            assert cache.offset == P
            assert torch.equal(cache.windows, win0) and torch.equal(cache.states, st0)
            first = first or r
            assert (r.accepted, r.bonus_token) == (first.accepted, first.bonus_token)
        r = eng.verify(cache, tree.tokens, tree.positions(P), tree.parents, use_graph=use_graph, commit=True)
        torch.cuda.synchronize()
        if first is not None:
            assert (r.accepted, r.bonus_token) == (first.accepted, first.bonus_token)
        assert cache.offset == P + len(r.accepted)
        assert not torch.equal(cache.states, st0)
        out.append((r.accepted, cache.windows.cpu(), cache.states.cpu()))
        eng.release_graphs()
    assert out[0][0] == out[1][0]
    assert torch.equal(out[0][1], out[1][1]) and torch.equal(out[0][2], out[1][2])


def test_qwen35_9b_q4_verify_step_prefix_8192_budget_64(gpu_device):
    """Qwen3.5-9B-shaped hybrid (hidden 4096), q4 weights including the tied
    LM head, 8192-token prefix, 65-node tree (draft budget 64)."""
    from dtree_hip.config import QWEN35_9B
    r = _run(QWEN35_9B, P=8192, layer_ids=[1, 15, 30], dev=gpu_device, norm_jitter=0.0, quant="q4", budget=64)
    assert r["L"] == 65
    # The synthetic q4 weights (nibbles 0..15, positive scales) give every
    # embedding row a large common-mode term: at hidden 4096 the top-2 logit
    # margins fall under 2e-2 of the largest logit, so the argmax bar is
    # carried by the measured-error margin (`sure` rows) instead.
    _check(r, [1, 15, 30], min_confident=0.0)
    require_path_compared(r["path_compared"], "Qwen3.5-9B-shaped q4 P=8192")


def test_qwen35_4b_verify_step_prefix_2048(gpu_device):
    """Qwen3.5-4B-shaped hybrid at a 2048-token prefix with a 24-node tree."""
    r = _run(QWEN35_4B, P=2048, layer_ids=[1, 15, 30], dev=gpu_device, norm_jitter=0.0, check_long_prefill_layers=4)
    _check(r, [1, 15, 30])
    require_path_compared(r["path_compared"], "Qwen3.5-4B-shaped bf16 P=2048")
