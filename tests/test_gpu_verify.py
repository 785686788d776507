"""Whole verify step on the GPU (embed, every layer, LM-head argmax, accept
walk, compaction) against the fp32 CPU oracle on the same weights, KV prefix
and tree.

Bars (north-star): logits within 2e-2 relative (max |diff| per row <= 2e-2 x
max |oracle logit| of that row); argmax tokens bit-exact on rows whose oracle
top-2 margin exceeds that tolerance; accepted path bit-exact up to and
including the first walked node without such a margin (the whole path and
the bonus token when every walked row has one); compacted cache = the pre-compaction rows
gathered at the accepted indices, bit for bit."""
import time

import numpy as np
import pytest
import torch

from dtree_hip import Qwen3TreeModel, Qwen3Weights, tiny_qwen3
from dtree_hip.config import QWEN3_4B
from dtree_hip.synthetic import acceptance_rewrite, make_tree, random_prefix
from dtree_hip.weights import W_TILED, W_TILED_F16
from oracle import qwen3 as oq
from oracle import tree as otree

from gpu_util import bf16_f32, compare_accepted_path, require_path_compared

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _oracle_cfg(cfg):
    return oq.Qwen3Config(hidden=cfg.hidden_size, layers=cfg.num_hidden_layers, ffn=cfg.intermediate_size,
                          heads=cfg.num_attention_heads, kv_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                          vocab=cfg.vocab_size, eps=cfg.rms_norm_eps, rope_base=cfg.rope_theta)


def _check_prefill(orc, cfg, prefix, prefix_k, prefix_v, layers, log=print):
    """The device prefill's cache rows (32-row chained tree passes through the
    same kernels, paged) against the oracle's causal forward over the prefix:
    K and V of the first `layers` layers at every position."""
    t0 = time.time()
    P = len(prefix)
    x = orc.embed(np.asarray(prefix, np.int64))
    pos = np.arange(P)
    causal = np.tril(np.ones((P, P), bool))
    empty = np.zeros((0, cfg.num_key_value_heads, cfg.head_dim), np.float32)
    for li in range(layers):
        x, k, v = orc.layer_forward(li, x, empty, empty, pos, causal)
        for got, want, what in ((prefix_k[li], k, "keys"), (prefix_v[li], v, "values")):
            err = np.abs(got - want).max(axis=(1, 2))
            bar = TOL * np.maximum(1.0, np.abs(want).max(axis=(1, 2)))
            assert np.all(err <= bar), f"prefill {what} layer {li}: worst position {int(np.argmax(err / bar))}"
    log(f"prefill K/V of {layers} layers at {P} positions match the oracle ({time.time() - t0:.1f}s)")


def _run(cfg, P, layer_ids, dev, norm_jitter=0.0, log=print, quant="bf16", check_prefill_layers=0,
         layout=W_TILED_F16):
    t0 = time.time()
    if quant == "q4":  # every linear layer and the tied embedding in 4-bit groups of 64
        w = Qwen3Weights.random_q4(cfg, seed=0, device=dev, norm_jitter=norm_jitter)
    else:
        w = Qwen3Weights.random(cfg, seed=0, device=dev, norm_jitter=norm_jitter, layout=layout)
    model = Qwen3TreeModel(cfg, w, max_past=P + 64, layer_ids=layer_ids)
    eng = model.engine
    cache = eng.new_cache()
    prefix = random_prefix(P, cfg.vocab_size, seed=1)
    eng.prefill(cache, prefix)
    assert cache.offset == P
    st = eng.stream_handle()
    tree = make_tree(root_token=prefix[-1] if P else 0, vocab=cfg.vocab_size, seed=2)

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
    tree_k = [bf16_f32(cache.logical_keys(li, P + L))[P:] for li in range(cfg.num_hidden_layers)]
    tree_v = [bf16_f32(cache.logical_values(li, P + L))[P:] for li in range(cfg.num_hidden_layers)]
    hidden = bf16_f32(eng.hidden[:L]) if layer_ids else None
    prefix_k = [bf16_f32(cache.logical_keys(li, P)) for li in range(cfg.num_hidden_layers)]
    prefix_v = [bf16_f32(cache.logical_values(li, P)) for li in range(cfg.num_hidden_layers)]

    # the real step: graph replay of forward + argmax + walk + compaction
    res = eng.verify(cache, tree.tokens, tree.positions(P), tree.parents, use_graph=True)
    torch.cuda.synchronize()

    # oracle on the same weights / prefix / tree
    t1 = time.time()
    orc = oq.OracleQwen3(_oracle_cfg(cfg), w.host_accessor())
    if check_prefill_layers:
        _check_prefill(orc, cfg, prefix, prefix_k, prefix_v, check_prefill_layers, log)
    oc = oq.OracleCache(keys=prefix_k, values=prefix_v)
    ids, pos, mask = otree.compile_tree(tree.tokens[0], P, tree.tokens[1:], tree.depths[1:], tree.visibility, P)
    norm, vh, nk, nv = orc.forward_tree(ids, pos, mask, oc, layer_ids)
    E = w.host_accessor()(None, "embed")
    ref = np.concatenate([norm @ oq.bf16_to_f32(E[s:s + 16384]).T for s in range(0, E.shape[0], 16384)], axis=1)
    log(f"oracle {time.time() - t1:.1f}s")
    return dict(eng=eng, cache=cache, tree=tree, res=res, logits=logits, ref=ref, tree_k=tree_k, tree_v=tree_v,
                nk=nk, nv=nv, hidden=hidden, vh=vh, P=P, L=L)


def _check(r, layer_ids):
    L, P = r["L"], r["P"]
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
    assert confident.mean() > 0.5
    note = (f"max logit err {float((err / scale).max()):.4f} of the row max (bar {TOL}); "
            f"{int(confident.sum())}/{len(confident)} rows confident, {int(sure.sum())} sure")
    r["path_compared"] = compare_accepted_path(res, tree.child_maps, o_post, confident | sure, note=note)
    # device walk == host walk on the device's own posterior
    acc2, bonus2 = otree.follow_verified_tree(tree.child_maps, res.posterior)
    assert res.accepted == acc2 and res.bonus_token == bonus2
    # compaction: rows P..P+n == pre-compaction tree rows at the accepted indices
    cache, n = r["cache"], len(res.accepted)
    assert cache.offset == P + n
    for li in range(len(r["tree_k"])):
        kc = bf16_f32(cache.logical_keys(li, P + n))[P:]
        vc = bf16_f32(cache.logical_values(li, P + n))[P:]
        np.testing.assert_array_equal(kc, r["tree_k"][li][res.accepted])
        np.testing.assert_array_equal(vc, r["tree_v"][li][res.accepted])
        for got, want in ((r["tree_k"][li], r["nk"][li]), (r["tree_v"][li], r["nv"][li])):
            assert np.abs(got - want).max() <= TOL * max(1.0, np.abs(want).max())
    if layer_ids:
        hs = bf16_f32(r["eng"].hidden_sel[:n])
        want = r["vh"][res.accepted]
        assert np.abs(hs - want).max() <= TOL * np.abs(want).max()
        assert np.abs(r["hidden"] - r["vh"]).max() <= TOL * np.abs(r["vh"]).max()
    return res


def test_verify_step_tiny_model(gpu_device, attn_kernel):
    cfg = tiny_qwen3()
    r = _run(cfg, P=100, layer_ids=[0, 1], dev=gpu_device, norm_jitter=0.1, check_prefill_layers=2)
    res = _check(r, [0, 1])
    assert len(res.accepted) >= 1


def test_verify_step_tiny_model_bf16_pairs(gpu_device):
    """bf16 weights in DTREE_W_TILED with the bf16 hi + lo activation pair
    (the layout for checkpoints whose activations exceed fp16's range)."""
    cfg = tiny_qwen3()
    r = _run(cfg, P=100, layer_ids=[0, 1], dev=gpu_device, norm_jitter=0.1, check_prefill_layers=2, layout=W_TILED)
    assert not r["eng"].h16
    res = _check(r, [0, 1])
    assert len(res.accepted) >= 1


def test_verify_step_tiny_model_q4(gpu_device):
    cfg = tiny_qwen3()
    r = _run(cfg, P=100, layer_ids=[0, 1], dev=gpu_device, norm_jitter=0.1, quant="q4")
    res = _check(r, [0, 1])
    assert len(res.accepted) >= 1


def test_verify_step_graph_replays_match_eager(gpu_device, attn_kernel):
    cfg = tiny_qwen3(num_hidden_layers=3)
    w = Qwen3Weights.random(cfg, seed=0, device=gpu_device)
    model = Qwen3TreeModel(cfg, w, max_past=256, layer_ids=[1])
    eng = model.engine
    cache = eng.new_cache()
    eng.prefill(cache, random_prefix(150, cfg.vocab_size, seed=1))
    tree = make_tree(7, cfg.vocab_size, seed=2)
    P = cache.offset
    outs = []
    for mode in ("eager", "graph", "graph", "graph"):
        cache.offset = P
        res = eng.verify(cache, tree.tokens, tree.positions(P), tree.parents, use_graph=(mode == "graph"))
        torch.cuda.synchronize()
        outs.append((res.accepted, res.bonus_token, res.posterior, eng.hidden_sel.clone(),
                     cache.k_pages.clone(), cache.v_pages.clone()))
        _ = torch.randn(1000, device=gpu_device).sum().item()  # eager work between replays
    for o in outs[1:]:
        assert o[0] == outs[0][0] and o[1] == outs[0][1] and o[2] == outs[0][2]
        assert torch.equal(o[3], outs[0][3]) and torch.equal(o[4], outs[0][4]) and torch.equal(o[5], outs[0][5])


def test_verify_step_qwen3_4b_prefix_1024(gpu_device):
    """Full-size verify step: 36 layers, hidden 2560, vocab 151936, P=1024, 25 nodes."""
    r = _run(QWEN3_4B, P=1024, layer_ids=[1, 9, 17, 25, 33], dev=gpu_device, check_prefill_layers=3)
    res = _check(r, [1, 9, 17, 25, 33])
    print("accepted", res.accepted, "bonus", res.bonus_token)
    require_path_compared(r["path_compared"], "Qwen3-4B bf16 P=1024")


def test_verify_step_qwen3_4b_q4_prefix_1024(gpu_device):
    """The q4 workload: the same full-size step with every linear layer and the
    tied LM head quantised to 4-bit groups of 64 (scales |N(0, 0.02)| * 8,
    biases N(0, 0.01)); the oracle runs on the dequantised weights."""
    r = _run(QWEN3_4B, P=1024, layer_ids=[1, 9, 17, 25, 33], dev=gpu_device, quant="q4")
    res = _check(r, [1, 9, 17, 25, 33])
    print("accepted", res.accepted, "bonus", res.bonus_token)
    require_path_compared(r["path_compared"], "Qwen3-4B q4 P=1024")
