"""DTree decode runtime (verify half) on the HIP target.

Host-side mirror of the reference's dtree_runtime.py with the same function
names, arguments and error behaviour, operating on torch tensors:
  build_dtree_tree        dtree_runtime.py:82-163
  compile_dtree_tree      dtree_runtime.py:166-192
  follow_verified_tree    dtree_runtime.py:195-208
  lazy_follow_tree_exact  dtree_runtime.py:211-290
  dtree_generate          dtree_runtime.py:293-586
The drafter is an input producer outside this package: any object with
``block_size``, ``mask_token_id``, ``make_cache()`` and
``__call__(noise_embedding=, target_hidden=, cache=)`` can drive
dtree_generate.
"""
from __future__ import annotations

import heapq
import os
import time
from typing import Any

import numpy as np
import torch

DTREE_STAGE_ORDER = (
    "draft_time_s",
    "tree_build_time_s",
    "tree_compile_time_s",
    "verify_time_s",
    "bookkeeping_time_s",
)
DTREE_TREE_BUILD_STAGE_ORDER = (
    "tree_build_copy_time_s",
    "tree_build_heap_time_s",
    "tree_build_visibility_time_s",
)
DTREE_VERIFY_DETAIL_STAGE_ORDER = (
    "verify_tree_forward_time_s",
    "verify_tree_logits_time_s",
    "verify_tree_argmax_time_s",
    "verify_tree_sample_time_s",
)
DTREE_BOOKKEEPING_DETAIL_STAGE_ORDER = (
    "bookkeeping_follow_tree_time_s",
    "bookkeeping_cache_compact_time_s",
    "bookkeeping_hidden_select_time_s",
    "bookkeeping_output_commit_time_s",
)


def empty_dtree_profile() -> dict[str, float]:
    return {
        **{k: 0.0 for k in DTREE_STAGE_ORDER},
        **{k: 0.0 for k in DTREE_TREE_BUILD_STAGE_ORDER},
        **{k: 0.0 for k in DTREE_VERIFY_DETAIL_STAGE_ORDER},
        **{k: 0.0 for k in DTREE_BOOKKEEPING_DETAIL_STAGE_ORDER},
    }


def profile_start(profile: dict[str, float] | None) -> float:
    return time.perf_counter() if profile is not None else 0.0


def add_profile_elapsed(profile: dict[str, float] | None, key: str, start: float) -> None:
    if profile is not None:
        profile[key] = profile.get(key, 0.0) + time.perf_counter() - start


def _sync(t: Any = None) -> None:
    if torch.cuda.is_available():
        torch.cuda.synchronize()


def sample_tokens(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    """runtime.py:12-19: argmax (first index) at temperature 0, else categorical."""
    V = logits.shape[-1]
    flat = logits.reshape(-1, V).float()
    if temperature < 1e-5:
        out = torch.argmax(flat, dim=-1)
    else:
        out = torch.multinomial(torch.softmax(flat / temperature, dim=-1), 1)[:, 0]
    return out.reshape(logits.shape[:-1]).to(torch.int64)


def build_dtree_tree(draft_logits, budget: int, topk: int | None = None):
    """Best-first draft tree over per-depth top-k ranks (dtree_runtime.py:82-163).

    ``topk`` defaults to the reference's ``min(budget, vocab)``; the synthetic
    workloads pass 4 (top-4 branching). Returns (node_token_ids, node_depths,
    parents, child_maps, visibility [L, L] bool, subtimes).
    """
    subtimes = {k: 0.0 for k in DTREE_TREE_BUILD_STAGE_ORDER}
    logits = draft_logits if isinstance(draft_logits, torch.Tensor) else torch.as_tensor(np.asarray(draft_logits))
    if budget <= 0 or logits.shape[0] == 0:
        return [], [], [-1], [dict()], torch.ones((1, 1), dtype=torch.bool), subtimes
    k = min(budget if topk is None else topk, int(logits.shape[-1]))
    depth_limit = int(logits.shape[0])

    t0 = time.perf_counter()
    x = logits.float()
    top_vals, top_ids = torch.topk(x, k, dim=-1, largest=True, sorted=True)
    top_lp = top_vals - torch.logsumexp(x, dim=-1, keepdim=True)
    tok = top_ids.to("cpu", torch.int64).numpy()
    lp = top_lp.to("cpu", torch.float32).numpy()
    subtimes["tree_build_copy_time_s"] = time.perf_counter() - t0

    t0 = time.perf_counter()
    first = float(lp[0, 0])
    heap = [(-first, (0,), 0, 1, 0, first)]
    node_token_ids: list[int] = []
    node_depths: list[int] = []
    parents = [-1]
    child_maps: list[dict[int, int]] = [dict()]
    while heap and len(node_token_ids) < budget:
        _, ranks, parent, depth, rank, logw = heapq.heappop(heap)
        token = int(tok[depth - 1, rank])
        idx = len(node_token_ids) + 1
        node_token_ids.append(token)
        node_depths.append(depth)
        parents.append(parent)
        child_maps.append(dict())
        child_maps[parent][token] = idx
        if rank + 1 < k:
            sib = logw - float(lp[depth - 1, rank]) + float(lp[depth - 1, rank + 1])
            heapq.heappush(heap, (-sib, ranks[:-1] + (rank + 1,), parent, depth, rank + 1, sib))
        if depth < depth_limit:
            child = logw + float(lp[depth, 0])
            heapq.heappush(heap, (-child, ranks + (0,), idx, depth + 1, 0, child))
    subtimes["tree_build_heap_time_s"] = time.perf_counter() - t0

    t0 = time.perf_counter()
    n = 1 + len(node_token_ids)
    vis = np.zeros((n, n), dtype=np.bool_)
    vis[0, 0] = True
    for i in range(1, n):
        vis[i, :i] = vis[parents[i], :i]
        vis[i, i] = True
    subtimes["tree_build_visibility_time_s"] = time.perf_counter() - t0
    return node_token_ids, node_depths, parents, child_maps, torch.from_numpy(vis), subtimes


def compile_dtree_tree(root_token_id: int, start: int, node_token_ids, node_depths, visibility, past_length: int,
                       verify_input_ids_buffer: torch.Tensor, verify_position_ids_buffer: torch.Tensor,
                       attention_mask_buffer: torch.Tensor):
    """Verify inputs for one tree (dtree_runtime.py:166-192): ids [1, L],
    positions start + depth [1, L], mask [L, past_length + L] with every prefix
    column visible and tree columns = ancestor-or-self visibility."""
    tree_tokens = [int(root_token_id), *[int(t) for t in node_token_ids]]
    positions = [int(start), *[int(start) + int(d) for d in node_depths]]
    L = len(tree_tokens)
    ids = verify_input_ids_buffer[:, :L]
    pos = verify_position_ids_buffer[:, :L]
    ids[0, :] = torch.tensor(tree_tokens, dtype=ids.dtype)
    pos[0, :] = torch.tensor(positions, dtype=pos.dtype)
    mask = attention_mask_buffer[:L, : past_length + L]
    mask[:, :past_length] = True
    vis = visibility if isinstance(visibility, torch.Tensor) else torch.as_tensor(np.asarray(visibility))
    mask[:, past_length: past_length + L] = vis.to(mask.device, torch.bool)
    return ids, tree_tokens, pos, mask


def follow_verified_tree(child_maps: list[dict[int, int]], posterior_tokens) -> tuple[list[int], int]:
    accepted = [0]
    cur = 0
    nxt = int(posterior_tokens[cur])
    while nxt in child_maps[cur]:
        cur = child_maps[cur][nxt]
        accepted.append(cur)
        nxt = int(posterior_tokens[cur])
    return accepted, nxt


def lazy_follow_tree_exact(target, target_cache, layer_ids, tree_tokens, child_maps, temperature: float,
                           verify_mode: str, profile_times: dict | None):
    """dtree_runtime.py:211-290: walk one token at a time with real cache updates."""
    if target.adapter.family != "qwen3_5":
        raise NotImplementedError("lazy_follow_tree_exact is only implemented for qwen3_5.")
    model = target.model
    if hasattr(model, "language_model") and hasattr(model.language_model, "model"):
        text_model = model.language_model.model
    elif hasattr(model, "model"):
        text_model = model.model
    else:
        raise AttributeError(f"Unsupported qwen3_5 target model: {type(model)!r}")
    accepted: list[int] = []
    hidden_chunks = []
    cur = 0
    while True:
        t0 = profile_start(profile_times)
        ids = torch.tensor([[tree_tokens[cur]]], dtype=torch.int64)
        norm_hidden, verifier_hidden = text_model.forward_dflash(ids, target_cache, layer_ids)
        add_profile_elapsed(profile_times, "verify_tree_forward_time_s", t0)
        accepted.append(cur)
        hidden_chunks.append(verifier_hidden)
        if verify_mode == "parallel-greedy-argmax":
            t0 = profile_start(profile_times)
            posterior = target.lm_head_argmax(norm_hidden)
            add_profile_elapsed(profile_times, "verify_tree_argmax_time_s", t0)
        else:
            t0 = profile_start(profile_times)
            logits = target.lm_head_logits(norm_hidden)
            add_profile_elapsed(profile_times, "verify_tree_logits_time_s", t0)
            t0 = profile_start(profile_times)
            posterior = sample_tokens(logits, temperature)
            add_profile_elapsed(profile_times, "verify_tree_sample_time_s", t0)
        token = int(posterior.reshape(-1)[0].item())
        nxt = child_maps[cur].get(token)
        if nxt is None:
            return accepted, token, torch.cat(hidden_chunks, dim=1)
        cur = nxt


def stop_position(output_tokens: list[int], prompt_len: int, stop_token_ids: set[int]) -> int | None:
    for i in range(prompt_len, len(output_tokens)):
        if output_tokens[i] in stop_token_ids:
            return i
    return None


def dtree_generate(target, draft, prompt_tokens, max_new_tokens: int, temperature: float,
                   stop_token_ids: set[int], layer_ids: list[int], speculative_tokens: int | None,
                   tree_budget: int | None = None, verify_mode: str = "parallel-replay",
                   profile: bool = False, tree_topk: int | None = None):
    """DTree decode loop (dtree_runtime.py:293-586) over a HIP target."""
    if not target.supports_tree_verification():
        raise NotImplementedError(
            f"DTree is not implemented for target adapter family={target.adapter.family!r}.")
    if verify_mode not in {"parallel-replay", "parallel-greedy-argmax"}:
        raise ValueError("DTree only supports verify_mode='parallel-replay' or 'parallel-greedy-argmax'.")
    if verify_mode == "parallel-greedy-argmax" and temperature >= 1e-5:
        raise ValueError("DTree parallel-greedy-argmax only supports temperature=0.")

    from .runtime import trim_draft_cache

    target_cache = target.make_cache()
    draft_cache = draft.make_cache()
    profile_times = empty_dtree_profile() if profile else None
    prompt = [int(t) for t in (prompt_tokens.tolist() if hasattr(prompt_tokens, "tolist") else prompt_tokens)]
    prompt_len = len(prompt)
    total_max_tokens = prompt_len + max_new_tokens
    block_size = draft.block_size if speculative_tokens is None else max(1, min(speculative_tokens, draft.block_size))
    if block_size <= 1:
        raise ValueError("DTree requires speculative_tokens >= 2.")
    budget = max(tree_budget if tree_budget is not None else block_size - 1, 0)
    max_nodes = 1 + budget
    ids_buf = torch.zeros((1, max_nodes), dtype=torch.int64)
    pos_buf = torch.zeros((1, max_nodes), dtype=torch.int64)
    mask_buf = torch.ones((max_nodes, total_max_tokens + max_nodes), dtype=torch.bool)

    t0 = time.perf_counter()
    logits, target_hidden = target.forward_with_hidden_states(torch.tensor(prompt)[None], target_cache, layer_ids)
    first_token = int(sample_tokens(logits[:, -1, :], temperature).item())
    _sync()
    prefill_time = time.perf_counter() - t0

    output_tokens = prompt + [first_token]
    start = prompt_len
    acceptance_lengths: list[int] = []
    verified_tree_nodes: list[int] = []
    qwen35_tree_mode = os.environ.get("DTREE_QWEN35_TREE_MODE")
    use_lazy = target.adapter.family == "qwen3_5" and qwen35_tree_mode != "full_tree"
    # The fused greedy verify builds the tree on the device unless told otherwise
    # (DTREE_TREE_BUILD=host keeps the host heap of build_dtree_tree).
    device_tree = (not use_lazy and verify_mode == "parallel-greedy-argmax" and profile_times is None
                   and hasattr(target, "verify_tree_from_logits") and os.environ.get("DTREE_TREE_BUILD") != "host")

    decode_start = time.perf_counter()
    while start < total_max_tokens:
        t0 = profile_start(profile_times)
        block = [output_tokens[start]] + [draft.mask_token_id] * (block_size - 1)
        noise = target.embed_tokens(torch.tensor(block)[None])
        draft_hidden = draft(noise_embedding=noise, target_hidden=target_hidden, cache=draft_cache)
        draft_logits = target.lm_head_logits(draft_hidden[:, 1:, :])
        trim_draft_cache(draft_cache, block_size)
        add_profile_elapsed(profile_times, "draft_time_s", t0)

        if device_tree:
            # Tree build, verify-input compile and the fused verify step on the
            # device with one readback (tree kernels write the step descriptor).
            t0 = profile_start(profile_times)
            node_ids, depths, parents, child_maps, accepted, posterior_token, verifier_hidden = \
                target.verify_tree_from_logits(draft_logits[0], budget, tree_topk, block[0], target_cache, layer_ids)
            tree_tokens = [block[0], *node_ids]
            add_profile_elapsed(profile_times, "verify_time_s", t0)
        else:
            t0 = profile_start(profile_times)
            node_ids, depths, parents, child_maps, vis, sub = build_dtree_tree(draft_logits[0], budget,
                                                                               topk=tree_topk)
            add_profile_elapsed(profile_times, "tree_build_time_s", t0)
            if profile_times is not None:
                for k2, v in sub.items():
                    profile_times[k2] += v

            t0 = profile_start(profile_times)
            tree_tokens = [block[0], *node_ids]
            if not use_lazy:
                ids, tree_tokens, pos, mask = compile_dtree_tree(block[0], start, node_ids, depths, vis, start,
                                                                 ids_buf, pos_buf, mask_buf)
            add_profile_elapsed(profile_times, "tree_compile_time_s", t0)

        t0 = profile_start(profile_times)
        if device_tree:
            pass
        elif use_lazy:
            accepted, posterior_token, verifier_hidden = lazy_follow_tree_exact(
                target, target_cache, layer_ids, tree_tokens, child_maps, temperature, verify_mode, profile_times)
        elif verify_mode == "parallel-greedy-argmax" and profile_times is None and hasattr(target, "verify_tree"):
            # Fused path: forward + LM-head argmax + walk + compaction in one graph.
            accepted, posterior_token, verifier_hidden = target.verify_tree(
                ids, target_cache, layer_ids, parents, pos, mask, child_maps)
        else:
            tf = profile_start(profile_times)
            norm_hidden, verifier_hidden = target.forward_tree_with_hidden_states(
                ids, target_cache, layer_ids, parents=parents, position_ids=pos, attention_mask=mask)
            if profile_times is not None:
                _sync()
            add_profile_elapsed(profile_times, "verify_tree_forward_time_s", tf)
            if verify_mode == "parallel-greedy-argmax":
                tf = profile_start(profile_times)
                posterior = target.lm_head_argmax(norm_hidden)
                add_profile_elapsed(profile_times, "verify_tree_argmax_time_s", tf)
            else:
                tf = profile_start(profile_times)
                vlog = target.lm_head_logits(norm_hidden)
                if profile_times is not None:
                    _sync()
                add_profile_elapsed(profile_times, "verify_tree_logits_time_s", tf)
                tf = profile_start(profile_times)
                posterior = sample_tokens(vlog, temperature)
                add_profile_elapsed(profile_times, "verify_tree_sample_time_s", tf)
            posterior_tokens = posterior[0].tolist()
            accepted, posterior_token = follow_verified_tree(child_maps, posterior_tokens)
        add_profile_elapsed(profile_times, "verify_time_s", t0)

        tb = profile_start(profile_times)
        tf = profile_start(profile_times)
        accepted_inputs = len(accepted)
        accepted_token_ids = [tree_tokens[i] for i in accepted]
        add_profile_elapsed(profile_times, "bookkeeping_follow_tree_time_s", tf)
        tf = profile_start(profile_times)
        if not use_lazy and not getattr(target, "last_verify_compacted", False):
            target.compact_kv_caches(target_cache, past_length=start, keep_current_indices=accepted)
            if profile_times is not None:
                _sync()
        add_profile_elapsed(profile_times, "bookkeeping_cache_compact_time_s", tf)
        tf = profile_start(profile_times)
        if use_lazy:
            target_hidden = verifier_hidden
        elif getattr(target, "last_verify_compacted", False):
            target_hidden = verifier_hidden
        else:
            target_hidden = verifier_hidden[:, torch.tensor(accepted, device=verifier_hidden.device), :]
        add_profile_elapsed(profile_times, "bookkeeping_hidden_select_time_s", tf)
        tf = profile_start(profile_times)
        output_tokens = output_tokens[:start]
        output_tokens.extend(accepted_token_ids)
        output_tokens.append(posterior_token)
        start += accepted_inputs
        acceptance_lengths.append(accepted_inputs)
        verified_tree_nodes.append(accepted_inputs if use_lazy else len(tree_tokens))
        add_profile_elapsed(profile_times, "bookkeeping_output_commit_time_s", tf)
        add_profile_elapsed(profile_times, "bookkeeping_time_s", tb)
        if hasattr(target, "last_verify_compacted"):
            target.last_verify_compacted = False

        stop_idx = stop_position(output_tokens, prompt_len, stop_token_ids)
        if stop_idx is not None:
            output_tokens = output_tokens[: stop_idx + 1]
            break
        if len(output_tokens) > total_max_tokens:
            output_tokens = output_tokens[:total_max_tokens]
            break

    decode_time = time.perf_counter() - decode_start
    output_tokens = output_tokens[:total_max_tokens]
    generated = max(len(output_tokens) - prompt_len, 0)
    total_time = prefill_time + decode_time
    metrics = {
        "decode_mode": "dtree",
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
        "avg_verified_tree_nodes": sum(verified_tree_nodes) / max(len(verified_tree_nodes), 1),
        "verified_tree_nodes": verified_tree_nodes,
        "peak_memory_gb": (torch.cuda.max_memory_allocated() / 1e9) if torch.cuda.is_available() else 0.0,
        "target_cache_summary": target.cache_summary(target_cache),
        "speculative_tokens": block_size,
        "tree_budget": budget,
        "verify_mode": verify_mode,
        "tree_build": "device" if device_tree else "host",
    }
    if profile_times is not None:
        profiled = sum(profile_times[k] for k in DTREE_STAGE_ORDER)
        metrics["profile"] = {**profile_times, "unattributed_decode_time_s": decode_time - profiled,
                              "steps": len(acceptance_lengths)}
    return output_tokens, metrics
