"""DFlash linear decode (verify of one drafted chain per step) on the HIP target.

Host-side mirror of the reference's runtime.py with the same function names,
arguments, verify modes, metrics and error behaviour, on torch tensors:
  sample_tokens / trim_draft_cache / longest_prefix_match   runtime.py:12-40
  verify_block_stream                    runtime.py:132-158
  verify_block_parallel_replay           runtime.py:161-216
  verify_block_parallel_lazy_logits      runtime.py:219-299
  verify_block_parallel_greedy_argmax    runtime.py:302-354
  verify_block_chunked                   runtime.py:357-427
  dflash_generate                        runtime.py:430-610

A drafted block is verified as a chain-shaped tree (parents -1, 0, 1, ...)
through the target's tree surface: forward_tree_with_hidden_states leaves the
block pending beyond the committed state, and compact_kv_caches with the
accepted prefix commits exactly that prefix. For the Qwen3.5 hybrid this
replaces the reference's rollback tape (qwen35_target.py:23-175,
qwen35_kernels.py:12-391: record the GatedDeltaNet inputs of every block
token, then re-advance the state to the accepted length): the committed
recurrent state and conv window are only ever advanced along accepted
tokens, so nothing has to be rolled back. For Qwen3 the rejected suffix's
K/V rows simply stay beyond the cache offset.
"""
from __future__ import annotations

import time
from typing import Any

import torch

from .dtree_runtime import add_profile_elapsed, profile_start, sample_tokens, stop_position


def trim_draft_cache(cache, num_tokens: int) -> None:
    """runtime.py:22-26: every layer cache that can trim drops the block's rows."""
    if isinstance(cache, dict) or cache is None:
        return
    try:
        layers = list(cache)
    except TypeError:
        return
    for layer_cache in layers:
        trim = getattr(layer_cache, "trim", None)
        if trim is not None:
            trim(num_tokens)


def generated_token_count(output_tokens: list[int], prompt_len: int) -> int:
    return max(len(output_tokens) - prompt_len, 0)


def longest_prefix_match(draft_tokens: list[int], verifier_tokens: list[int]) -> int:
    matched = 0
    for d, v in zip(draft_tokens, verifier_tokens):
        if d != v:
            break
        matched += 1
    return matched


def _chain_inputs(block_tokens: list[int], start: int):
    """Chain-shaped tree over a drafted block: ids [1, B], positions
    start .. start + B - 1, parents -1, 0, .., B - 2, mask [B, start + B]
    (every prefix column, causal over the block)."""
    B = len(block_tokens)
    ids = torch.tensor(block_tokens, dtype=torch.int64)[None]
    pos = torch.arange(start, start + B, dtype=torch.int64)[None]
    parents = [-1] + list(range(B - 1))
    mask = torch.ones((B, start + B), dtype=torch.bool)
    mask[:, start:] = torch.tril(torch.ones((B, B), dtype=torch.bool))
    return ids, pos, parents, mask


def _commit_prefix(target, target_cache, start: int, accepted_inputs: int) -> None:
    target.compact_kv_caches(target_cache, past_length=start, keep_current_indices=list(range(accepted_inputs)))


def verify_block_stream(target, target_cache, block_tokens: list[int], temperature: float,
                        layer_ids: list[int]) -> tuple[int, int, torch.Tensor]:
    """runtime.py:132-158: one committed token per forward."""
    hidden_steps = []
    for idx, token in enumerate(block_tokens):
        logits_step, hidden_step = target.forward_with_hidden_states(torch.tensor([[token]]), target_cache,
                                                                     layer_ids)
        next_token = int(sample_tokens(logits_step[:, -1, :], temperature).reshape(-1)[0].item())
        hidden_steps.append(hidden_step)
        if idx == len(block_tokens) - 1:
            return len(block_tokens), next_token, torch.cat(hidden_steps, dim=1)
        if next_token != block_tokens[idx + 1]:
            return idx + 1, next_token, torch.cat(hidden_steps, dim=1)
    raise RuntimeError("Streaming verifier reached an impossible state.")


def _pending_block(target, target_cache, block_tokens, layer_ids):
    start = target_cache.offset
    ids, pos, parents, mask = _chain_inputs(block_tokens, start)
    norm_hidden, verifier_hidden = target.forward_tree_with_hidden_states(
        ids, target_cache, layer_ids, parents=parents, position_ids=pos, attention_mask=mask)
    return start, norm_hidden, verifier_hidden


def verify_block_parallel_replay(target, target_cache, block_tokens: list[int], draft_block_size: int,
                                 temperature: float, layer_ids: list[int], profile: dict | None = None):
    """runtime.py:161-216: the whole block in one forward, posterior of every
    position, then the accepted prefix is committed."""
    t0 = profile_start(profile)
    start, norm_hidden, verifier_hidden = _pending_block(target, target_cache, block_tokens, layer_ids)
    posterior = sample_tokens(target.lm_head_logits(norm_hidden), temperature)[0].tolist()
    add_profile_elapsed(profile, "verify_forward_logits_time_s", t0)
    t0 = profile_start(profile)
    matched = longest_prefix_match(block_tokens[1:], posterior[:-1])
    accepted_inputs = matched + 1
    add_profile_elapsed(profile, "verify_prefix_time_s", t0)
    t0 = profile_start(profile)
    _commit_prefix(target, target_cache, start, accepted_inputs)
    if accepted_inputs < draft_block_size:
        add_profile_elapsed(profile, "verify_rollback_time_s", t0)
    return accepted_inputs, posterior[matched], verifier_hidden[:, :accepted_inputs, :]


def verify_block_parallel_lazy_logits(target, target_cache, block_tokens: list[int], draft_block_size: int,
                                      temperature: float, layer_ids: list[int], logit_chunk_size: int,
                                      profile: dict | None = None):
    """runtime.py:219-299: one forward, then LM-head rows in chunks until the
    first rejected position."""
    t0 = profile_start(profile)
    start, norm_hidden, verifier_hidden = _pending_block(target, target_cache, block_tokens, layer_ids)
    add_profile_elapsed(profile, "verify_state_time_s", t0)
    matched = 0
    accepted_inputs = draft_block_size
    posterior_token = None
    chunk = max(1, int(logit_chunk_size))
    for c0 in range(0, draft_block_size, chunk):
        c1 = min(c0 + chunk, draft_block_size)
        t0 = profile_start(profile)
        post = sample_tokens(target.lm_head_logits(norm_hidden[:, c0:c1, :]), temperature)[0].tolist()
        add_profile_elapsed(profile, "verify_lazy_logits_time_s", t0)
        t0 = profile_start(profile)
        for li, token in enumerate(post):
            p = c0 + li
            if p == draft_block_size - 1:
                posterior_token, accepted_inputs = token, draft_block_size
                break
            if token == block_tokens[p + 1]:
                matched += 1
                continue
            posterior_token, accepted_inputs = token, matched + 1
            break
        add_profile_elapsed(profile, "verify_prefix_time_s", t0)
        if posterior_token is not None:
            break
    if posterior_token is None:
        raise RuntimeError("Lazy-logit verifier failed to produce a posterior token.")
    t0 = profile_start(profile)
    _commit_prefix(target, target_cache, start, accepted_inputs)
    if accepted_inputs < draft_block_size:
        add_profile_elapsed(profile, "verify_rollback_time_s", t0)
    return accepted_inputs, posterior_token, verifier_hidden[:, :accepted_inputs, :]


def verify_block_parallel_greedy_argmax(target, target_cache, block_tokens: list[int], draft_block_size: int,
                                        temperature: float, layer_ids: list[int], profile: dict | None = None):
    """runtime.py:302-354: greedy argmax of every position. Without profiling
    it runs as the target's fused verify graph over the chain (forward,
    LM-head argmax, walk = longest prefix match, commit of the accepted
    prefix); with profiling, method by method."""
    if temperature >= 1e-5:
        raise ValueError("parallel-greedy-argmax only supports temperature=0.")
    if profile is None and hasattr(target, "verify_tree"):
        start = target_cache.offset
        ids, pos, parents, mask = _chain_inputs(block_tokens, start)
        child_maps: list[dict[int, int]] = [dict() for _ in block_tokens]
        for i in range(1, len(block_tokens)):
            child_maps[i - 1][int(block_tokens[i])] = i
        accepted, posterior_token, hidden = target.verify_tree(ids, target_cache, layer_ids, parents, pos, mask,
                                                               child_maps)
        target.last_verify_compacted = False
        n = len(accepted)
        if hidden is None:
            hidden = torch.zeros(1, n, 0)
        return n, posterior_token, hidden
    t0 = profile_start(profile)
    start, norm_hidden, verifier_hidden = _pending_block(target, target_cache, block_tokens, layer_ids)
    add_profile_elapsed(profile, "verify_state_time_s", t0)
    t0 = profile_start(profile)
    posterior = target.lm_head_argmax(norm_hidden)[0].tolist()
    add_profile_elapsed(profile, "verify_argmax_time_s", t0)
    t0 = profile_start(profile)
    matched = longest_prefix_match(block_tokens[1:], posterior[:-1])
    accepted_inputs = matched + 1
    add_profile_elapsed(profile, "verify_prefix_time_s", t0)
    t0 = profile_start(profile)
    _commit_prefix(target, target_cache, start, accepted_inputs)
    if accepted_inputs < draft_block_size:
        add_profile_elapsed(profile, "verify_rollback_time_s", t0)
    return accepted_inputs, posterior[matched], verifier_hidden[:, :accepted_inputs, :]


def verify_block_chunked(target, target_cache, block_tokens: list[int], draft_block_size: int, temperature: float,
                         layer_ids: list[int], verify_chunk_size: int):
    """runtime.py:357-427: chunks of verify_chunk_size tokens; a chunk that is
    not fully matched commits its accepted prefix and ends the block."""
    hidden_chunks = []
    cursor = 0
    while cursor < draft_block_size:
        end = min(cursor + verify_chunk_size, draft_block_size)
        chunk = block_tokens[cursor:end]
        start, norm_hidden, chunk_hidden = _pending_block(target, target_cache, chunk, layer_ids)
        post = sample_tokens(target.lm_head_logits(norm_hidden), temperature)[0].tolist()
        max_compare = min(len(chunk), draft_block_size - cursor - 1)
        local = 0
        while local < max_compare and post[local] == block_tokens[cursor + local + 1]:
            local += 1
        if local == max_compare:
            _commit_prefix(target, target_cache, start, len(chunk))
            hidden_chunks.append(chunk_hidden)
            if end < draft_block_size:
                cursor = end
                continue
            return draft_block_size, post[-1], torch.cat(hidden_chunks, dim=1)
        accepted_local = local + 1
        _commit_prefix(target, target_cache, start, accepted_local)
        hidden_chunks.append(chunk_hidden[:, :accepted_local, :])
        return cursor + accepted_local, post[local], torch.cat(hidden_chunks, dim=1)
    raise RuntimeError("Chunked verifier reached an impossible state.")


DFLASH_VERIFY_MODES = ("stream", "chunked", "parallel-replay", "parallel-lazy-logits", "parallel-greedy-argmax")


def dflash_generate(target, draft, prompt_tokens, max_new_tokens: int, temperature: float,
                    stop_token_ids: set[int], layer_ids: list[int], speculative_tokens: int | None,
                    verify_mode: str, verify_chunk_size: int, profile: bool = False) -> tuple[list[int], dict]:
    """DFlash decode loop (runtime.py:430-610): draft one block, verify it as a
    chain, commit the accepted prefix plus the target's next token."""
    if verify_mode not in DFLASH_VERIFY_MODES:
        raise ValueError(f"Unknown verify_mode={verify_mode!r}; expected one of {DFLASH_VERIFY_MODES}.")
    target_cache = target.make_cache(speculative_linear_cache=target.adapter.family == "qwen3_5")
    draft_cache = draft.make_cache()
    profile_times: dict[str, float] | None = {} if profile else None
    prompt = [int(t) for t in (prompt_tokens.tolist() if hasattr(prompt_tokens, "tolist") else prompt_tokens)]
    prompt_len = len(prompt)
    total_max_tokens = prompt_len + max_new_tokens
    block_size = draft.block_size if speculative_tokens is None else max(1, min(speculative_tokens, draft.block_size))

    t0 = time.perf_counter()
    logits, target_hidden = target.forward_with_hidden_states(torch.tensor(prompt)[None], target_cache, layer_ids)
    first_token = int(sample_tokens(logits[:, -1, :], temperature).reshape(-1)[0].item())
    if torch.cuda.is_available():
        torch.cuda.synchronize()
    prefill_time = time.perf_counter() - t0

    output_tokens = prompt + [first_token]
    start = prompt_len
    acceptance_lengths: list[int] = []
    decode_start = time.perf_counter()
    while start < total_max_tokens:
        t0 = profile_start(profile_times)
        block_tokens = [output_tokens[start]] + [draft.mask_token_id] * (block_size - 1)
        noise_embedding = target.embed_tokens(torch.tensor(block_tokens)[None])
        draft_hidden = draft(noise_embedding=noise_embedding, target_hidden=target_hidden, cache=draft_cache)
        drafted = sample_tokens(target.lm_head_logits(draft_hidden[:, 1:, :]), temperature)
        trim_draft_cache(draft_cache, block_size)
        block_tokens[1:] = drafted[0].tolist()[: block_size - 1]
        add_profile_elapsed(profile_times, "draft_time_s", t0)

        t0 = profile_start(profile_times)
        if verify_mode == "stream":
            accepted_inputs, posterior_token, verifier_hidden = verify_block_stream(
                target, target_cache, block_tokens, temperature, layer_ids)
        elif verify_mode == "chunked":
            accepted_inputs, posterior_token, verifier_hidden = verify_block_chunked(
                target, target_cache, block_tokens, block_size, temperature, layer_ids, verify_chunk_size)
        elif verify_mode == "parallel-lazy-logits":
            accepted_inputs, posterior_token, verifier_hidden = verify_block_parallel_lazy_logits(
                target, target_cache, block_tokens, block_size, temperature, layer_ids, verify_chunk_size,
                profile_times)
        elif verify_mode == "parallel-greedy-argmax":
            accepted_inputs, posterior_token, verifier_hidden = verify_block_parallel_greedy_argmax(
                target, target_cache, block_tokens, block_size, temperature, layer_ids, profile_times)
        else:
            accepted_inputs, posterior_token, verifier_hidden = verify_block_parallel_replay(
                target, target_cache, block_tokens, block_size, temperature, layer_ids, profile_times)
        acceptance_lengths.append(accepted_inputs)
        target_hidden = verifier_hidden[:, :accepted_inputs, :]
        add_profile_elapsed(profile_times, "verify_time_s", t0)

        t0 = profile_start(profile_times)
        output_tokens = output_tokens[:start]
        output_tokens.extend(block_tokens[:accepted_inputs])
        output_tokens.append(posterior_token)
        start += accepted_inputs
        add_profile_elapsed(profile_times, "bookkeeping_time_s", t0)

        stop_idx = stop_position(output_tokens, prompt_len, stop_token_ids)
        if stop_idx is not None:
            output_tokens = output_tokens[: stop_idx + 1]
            break
        if len(output_tokens) > total_max_tokens:
            output_tokens = output_tokens[:total_max_tokens]
            break

    decode_time = time.perf_counter() - decode_start
    output_tokens = output_tokens[:total_max_tokens]
    generated = generated_token_count(output_tokens, prompt_len)
    total_time = prefill_time + decode_time
    metrics: dict[str, Any] = {
        "decode_mode": "dflash",
        "num_input_tokens": prompt_len,
        "num_output_tokens": generated,
        "prefill_time_s": prefill_time,
        "decode_time_s": decode_time,
        "total_time_s": total_time,
        "prompt_tps": prompt_len / max(prefill_time, 1e-9),
        "generation_tps": generated / max(decode_time, 1e-9),
        "end_to_end_tps": generated / max(total_time, 1e-9),
        "avg_acceptance_length": sum(acceptance_lengths) / max(len(acceptance_lengths), 1),
        "acceptance_lengths": acceptance_lengths,
        "peak_memory_gb": (torch.cuda.max_memory_allocated() / 1e9) if torch.cuda.is_available() else 0.0,
        "target_cache_summary": target.cache_summary(target_cache),
        "speculative_tokens": block_size,
    }
    if profile_times is not None:
        profiled = sum(profile_times.get(k, 0.0) for k in ("draft_time_s", "verify_time_s", "bookkeeping_time_s"))
        metrics["profile"] = {**profile_times, "unattributed_decode_time_s": decode_time - profiled,
                              "steps": len(acceptance_lengths)}
    return output_tokens, metrics
