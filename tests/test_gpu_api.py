"""The generator facade (api.py:29-170) and DFlash linear decode
(runtime.py:430-610) on the GPU.

`DFlashGenerator.generate_from_tokens` dispatches decode_mode "dtree" to
dtree_generate and "dflash" to dflash_generate; every verify mode of the
linear decode (stream, chunked, parallel-replay, parallel-lazy-logits,
parallel-greedy-argmax) runs the drafted block as a chain through the HIP
target and commits only the accepted prefix (for the Qwen3.5 hybrid, the
GatedDeltaNet state advances along accepted tokens only). At temperature 0
every emitted token must be the fp32 oracle's greedy continuation (teacher
forced, within the 2e-2 logit tolerance, and exactly its argmax on nearly
every position), whatever the drafter proposes. The drafter is the scripted
one of test_gpu_generate.py (target's own greedy path, one planted error per
step)."""
import numpy as np
import pytest

from dtree_hip.adapters import load_target_model
from dtree_hip.api import DFlashGenerator, DFlashResult, Generator
from dtree_hip.config import tiny_qwen3, tiny_qwen35

from test_gpu_generate import BLOCK, TOL, ScriptedDrafter, _gpu_sequential_greedy, _oracle_teacher_forced

pytestmark = pytest.mark.gpu


def _check_greedy(target, prompt, out, n_new):
    gen = out[len(prompt):]
    assert len(gen) == n_new
    logits = _oracle_teacher_forced(target, out[:-1])[len(prompt) - 1:]
    scale = np.abs(logits).max(axis=-1)
    chosen = logits[np.arange(n_new), gen]
    assert np.all(chosen >= logits.max(axis=-1) - TOL * scale)
    assert np.mean(np.argmax(logits, axis=-1) == np.asarray(gen)) >= 0.9


def _setup(family, seed=5):
    cfg = tiny_qwen3() if family == "qwen3" else tiny_qwen35()
    target = load_target_model(cfg, seed=0, max_past=256, device="cuda", layer_ids=[0, 1],
                               norm_jitter=0.0 if family == "qwen3" else 0.1)
    rng = np.random.default_rng(seed)
    prompt = rng.integers(1, cfg.vocab_size, 40).tolist()
    n_new = 40
    plan = _gpu_sequential_greedy(target, prompt, n_new)
    drafter = ScriptedDrafter(target, prompt + plan)
    drafter.target_layer_ids = [0, 1]
    return target, prompt, n_new, drafter


DFLASH_CASES = [(f, m) for f in ("qwen3", "qwen3_5")
                for m in ("parallel-replay", "parallel-greedy-argmax", "parallel-lazy-logits", "chunked", "stream")]


@pytest.mark.parametrize("family,verify_mode", DFLASH_CASES)
def test_generator_dflash_linear_decode(gpu_device, monkeypatch, family, verify_mode):
    monkeypatch.delenv("DTREE_QWEN35_TREE_MODE", raising=False)
    target, prompt, n_new, drafter = _setup(family)
    gen = DFlashGenerator(target_model=target, draft_model=drafter)
    res = gen.generate_from_tokens(prompt, max_new_tokens=n_new, speculative_tokens=BLOCK, decode_mode="dflash",
                                   verify_mode=verify_mode, verify_chunk_size=3)
    assert isinstance(res, DFlashResult) and res.metrics["decode_mode"] == "dflash"
    assert res.generated_tokens == res.output_tokens[len(prompt):]
    _check_greedy(target, prompt, res.output_tokens, n_new)
    acc = res.metrics["acceptance_lengths"]
    assert max(acc) >= 5 and min(acc) == 1, acc


@pytest.mark.parametrize("family", ["qwen3", "qwen3_5"])
def test_generator_dtree_decode(gpu_device, monkeypatch, family):
    monkeypatch.delenv("DTREE_QWEN35_TREE_MODE", raising=False)
    target, prompt, n_new, drafter = _setup(family, seed=6)
    gen = Generator(target_model=target, draft_model=drafter)
    res = gen.generate_from_tokens(prompt, max_new_tokens=n_new, speculative_tokens=BLOCK, decode_mode="dtree",
                                   tree_budget=12, verify_mode="parallel-greedy-argmax")
    assert res.metrics["decode_mode"] == "dtree"
    _check_greedy(target, prompt, res.output_tokens, n_new)
    with pytest.raises(ValueError):
        gen.generate_from_tokens(prompt, max_new_tokens=4, decode_mode="medusa")
