"""The DFlash drafter on the GPU (dtree_hip.draft, draft.py:25-367) against
the oracle restatement (oracle/draft.py).

Each drafter call's normed hidden rows must match the fp32 oracle within 2e-2
of the row's largest magnitude (bf16 weights, inputs and output; the same
bar as the verify step's logits), in both cache modes ("kv", the mlx
KVCache; "context-only", the sink + window cache) and both mask modes, over
consecutive calls with trims in between, context batches above the
128-row pass size, and a context-only run long enough to slide the window.
The context K rows the device stored are checked against the oracle cache
too. End to end, the generator with its default random drafter must emit the
target's greedy continuation (speculative decoding at temperature 0 is
lossless whatever the drafter proposes), checked against the fp32 oracle by
teacher forcing as in test_gpu_api.py.
"""
import numpy as np
import pytest
import torch

from oracle import draft as od

from dtree_hip.adapters import load_target_model
from dtree_hip.api import DFlashGenerator
from dtree_hip.config import QWEN3_4B, tiny_qwen3, tiny_qwen35
from dtree_hip.draft import DFlashDraftModel, DraftArgs, random_draft_config
from dtree_hip.runtime import trim_draft_cache

from test_gpu_api import _check_greedy

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _args(H=1024, layers=2, ffn=2048, heads=8, kv=2, n_ids=2, block=16):
    return DraftArgs(model_type="qwen3", hidden_size=H, num_hidden_layers=layers, intermediate_size=ffn,
                     num_attention_heads=heads, rms_norm_eps=1e-6, vocab_size=4096, num_key_value_heads=kv,
                     max_position_embeddings=40960, rope_theta=1e6, head_dim=128, tie_word_embeddings=False,
                     block_size=block, dflash_config={"target_layer_ids": list(range(n_ids)), "mask_token_id": 0})


def _oracle(model: DFlashDraftModel) -> od.OracleDraft:
    a = model.args
    cfg = od.DraftConfig(hidden=a.hidden_size, layers=a.num_hidden_layers, ffn=a.intermediate_size,
                         heads=a.num_attention_heads, kv_heads=a.num_key_value_heads, head_dim=a.head_dim,
                         eps=a.rms_norm_eps, rope_base=a.rope_theta, n_target_layers=len(model.target_layer_ids),
                         block_size=a.block_size)
    return od.OracleDraft(cfg, model.weights.host_accessor())


def _bf16_rows(g, n, width, scale, dev):
    t = torch.from_numpy((g.standard_normal((n, width)) * scale).astype(np.float32)).to(torch.bfloat16)
    return t.to(dev), t.float().numpy()


def _check(got: torch.Tensor, ref: np.ndarray, what) -> float:
    x = got[0].float().cpu().numpy()
    assert x.shape == ref.shape, (what, x.shape, ref.shape)
    scale = np.abs(ref).max(axis=-1)
    err = np.abs(x - ref).max(axis=-1)
    rel = float((err / scale).max())
    assert np.all(err <= TOL * scale), (what, rel)
    return rel


def _run_calls(model, orc, dev, contexts, seed, mode, mask, check_keys=True):
    model.cache_mode = orc.cache_mode = mode
    model.attention_mask_mode = orc.mask_mode = mask
    g = np.random.default_rng(seed)
    H, B = model.args.hidden_size, model.block_size
    width = len(model.target_layer_ids) * H
    cache, ocache = model.make_cache(), orc.make_cache()
    for step, T in enumerate(contexts):
        print(f"draft call mode={mode} mask={mask} step={step} context_rows={T}", flush=True)
        th, th_np = _bf16_rows(g, T, width, 1.0, dev)
        noise, noise_np = _bf16_rows(g, B, H, 0.05, dev)
        got = model(noise_embedding=noise[None], target_hidden=th[None], cache=cache)
        ref = orc.forward(noise_np, th_np, cache=ocache)
        torch.cuda.synchronize()
        rel = _check(got, ref, (mode, mask, step))
        print(f"  max rel err {rel:.2e}", flush=True)
        if check_keys and mode == "kv":
            for li in (0, model.args.num_hidden_layers - 1):
                n = cache.offset
                k = cache.store.logical_keys(li, n).float().cpu().numpy()   # [n, Hkv, D]
                ok = ocache[li].keys[:n]
                assert np.abs(k - ok).max() <= TOL * np.abs(ok).max(), ("keys", li, step)
        trim_draft_cache(cache, B)
        for lc in ocache:
            lc.trim(B)
        assert [lc.offset for lc in cache] == [lc.offset for lc in ocache]


@pytest.mark.parametrize("mask", ["none", "causal"])
@pytest.mark.parametrize("mode", ["kv", "context-only"])
def test_draft_calls_match_oracle(gpu_device, attn_kernel, mode, mask):
    model = DFlashDraftModel.random(_args(), seed=0, max_past=1024, device=gpu_device, norm_jitter=0.1)
    _run_calls(model, _oracle(model), gpu_device, [40, 3, 16, 1, 300], seed=1, mode=mode, mask=mask)


def test_context_only_window_slides(gpu_device):
    """1100 + 130 + 5 context rows: the sink + ring slots must hold the same key
    set as the reference's concatenate-and-trim cache."""
    model = DFlashDraftModel.random(_args(layers=1), seed=2, max_past=4096, device=gpu_device)
    _run_calls(model, _oracle(model), gpu_device, [1100, 130, 5, 64], seed=3, mode="context-only", mask="none")


def test_uncached_call_matches_oracle(gpu_device):
    model = DFlashDraftModel.random(_args(), seed=4, max_past=512, device=gpu_device, norm_jitter=0.1)
    orc = _oracle(model)
    g = np.random.default_rng(5)
    th, th_np = _bf16_rows(g, 21, 2 * 1024, 1.0, gpu_device)
    noise, noise_np = _bf16_rows(g, 16, 1024, 0.05, gpu_device)
    got = model(noise_embedding=noise[None], target_hidden=th[None])
    _check(got, orc.forward(noise_np, th_np), "uncached")
    prep = model.prepare_target_hidden(th[None])
    _check(prep, orc.prepare_target_hidden(th_np), "prepare_target_hidden")


def test_qwen3_4b_shaped_drafter_matches_oracle(gpu_device):
    """The drafter sized for Qwen3-4B (5 layers, hidden 2560, FFN 9728, 32/8
    heads, five target layers -> fc of 12800 inputs), one prefill-sized and
    one step-sized context."""
    args = random_draft_config(QWEN3_4B, "dflash-b16")
    assert args.dflash_config["target_layer_ids"] == [1, 9, 17, 25, 33]
    model = DFlashDraftModel.random(args, seed=6, max_past=1024, device=gpu_device, norm_jitter=0.1)
    _run_calls(model, _oracle(model), gpu_device, [150, 7], seed=7, mode="kv", mask="none", check_keys=False)


@pytest.mark.parametrize("family,decode_mode", [("qwen3", "dtree"), ("qwen3", "dflash"), ("qwen3_5", "dtree"),
                                                ("qwen3_5", "dflash")])
def test_generator_with_random_drafter_is_lossless(gpu_device, monkeypatch, family, decode_mode):
    monkeypatch.delenv("DTREE_QWEN35_TREE_MODE", raising=False)
    cfg = tiny_qwen3() if family == "qwen3" else tiny_qwen35()
    target = load_target_model(cfg, seed=0, max_past=256, device="cuda", norm_jitter=0.1)
    gen = DFlashGenerator(target_model=target, draft_model="random:dflash-b16", seed=3)
    assert gen.draft.cache_mode == ("context-only" if family == "qwen3_5" else "kv")
    rng = np.random.default_rng(8)
    prompt = rng.integers(1, cfg.vocab_size, 30).tolist()
    n_new = 24
    kw = dict(tree_budget=15, verify_mode="parallel-greedy-argmax") if decode_mode == "dtree" else \
        dict(verify_mode="parallel-replay")
    print(f"generate family={family} mode={decode_mode}", flush=True)
    res = gen.generate_from_tokens(prompt, max_new_tokens=n_new, decode_mode=decode_mode, **kw)
    _check_greedy(target, prompt, res.output_tokens, n_new)
