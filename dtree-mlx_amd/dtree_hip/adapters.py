"""Target adapters on the HIP verify path.

Mirrors the reference's adapter boundary (adapters.py:88-213 protocol,
Qwen3TargetAdapter adapters.py:451-668, LoadedTargetModel adapters.py:681-819)
with torch tensors in place of mx.array. The tree-verify methods run the HIP
kernels through Qwen3TreeEngine / Qwen35TreeEngine; nothing here computes on
the CPU.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import numpy as np
import torch

from .cache import PagedKVCache, Qwen35Cache
from .config import QWEN3_4B, QWEN35_4B, Qwen35Config, Qwen3Config
from .engine import Qwen3TreeEngine, ancestor_bitsets
from .qwen35_engine import Qwen35TreeEngine
from .weights import Qwen35Weights, Qwen3Weights


class Qwen3TreeModel:
    """A Qwen3 target resident on one GPU (weights + verify engine)."""

    def __init__(self, cfg: Qwen3Config, weights: Qwen3Weights, max_past: int = 4096, layer_ids=(),
                 max_nodes: int = 32, split_k: dict | None = None):
        self.args = cfg
        self.weights = weights
        self.engine = Qwen3TreeEngine(cfg, weights, max_past=max_past, max_nodes=max_nodes,
                                      layer_ids=layer_ids, split_k=split_k)

    @property
    def layers(self):
        return self.weights.layers


class _Qwen35TextModel:
    """The text model's single-token path used by the lazy exact verifier
    (Qwen3_5TextModel.forward_dflash, custom_qwen35_model.py:961-1097): one
    forward per token that commits to the real cache."""

    def __init__(self, owner: "Qwen35TreeModel"):
        self._owner = owner

    def forward_dflash(self, inputs, cache: Qwen35Cache, layer_ids, input_embeddings=None,
                       return_rollback_records: bool = False):
        if input_embeddings is not None or return_rollback_records:
            raise NotImplementedError("forward_dflash takes token ids only here (no rollback records)")
        eng = self._owner.engine
        eng.set_layer_ids(layer_ids)
        toks = _as_list(inputs)
        eng.commit_chain(cache, toks, norm_hidden=True)
        n = len(toks)
        vh = (eng.hidden[:n].clone()[None] if layer_ids
              else torch.zeros(1, n, 0, dtype=torch.bfloat16, device=eng.dev))
        return eng.norm_hidden[:n].clone()[None], vh


class Qwen35TreeModel:
    """A Qwen3.5 hybrid target resident on one GPU (weights + verify engine)."""

    def __init__(self, cfg: Qwen35Config, weights: Qwen35Weights, max_past: int = 4096, layer_ids=(),
                 max_nodes: int = 32, split_k: dict | None = None):
        self.args = cfg
        self.weights = weights
        self.engine = Qwen35TreeEngine(cfg, weights, max_past=max_past, max_nodes=max_nodes,
                                       layer_ids=layer_ids, split_k=split_k)
        self.model = _Qwen35TextModel(self)

    @property
    def layers(self):
        return self.weights.layers


class MLXTargetAdapter:
    """Protocol of adapters.py:88-213 (names kept for drop-in use)."""

    family: str = "unknown"

    def make_cache(self, model, speculative_linear_cache: bool = False):
        raise NotImplementedError

    def embed_tokens(self, model, tokens):
        raise NotImplementedError

    def lm_head_logits(self, model, hidden_states):
        raise NotImplementedError

    def lm_head_argmax(self, model, hidden_states):
        return torch.argmax(self.lm_head_logits(model, hidden_states), dim=-1)

    def forward_with_hidden_states(self, model, inputs, cache, layer_ids, return_rollback_records=False):
        raise NotImplementedError

    def supports_tree_verification(self) -> bool:
        return False

    def forward_tree_with_hidden_states(self, model, inputs, cache, layer_ids, parents, position_ids,
                                        attention_mask):
        raise NotImplementedError(f"{self.family} does not expose explicit tree verification.")

    def cache_summary(self, cache) -> str:
        raise NotImplementedError

    def compact_kv_caches(self, model, cache, past_length: int, keep_current_indices: list[int]) -> None:
        raise NotImplementedError(f"{self.family} does not implement DTree cache compaction.")


def _as_list(x) -> list[int]:
    if isinstance(x, torch.Tensor):
        return [int(v) for v in x.reshape(-1).tolist()]
    return [int(v) for v in np.asarray(x).reshape(-1).tolist()]


def _mask_tree_bitsets(mask: np.ndarray, P: int, L: int) -> np.ndarray:
    """Ancestor bitsets from the tree columns of a [L, P+L] mask; the prefix
    columns must all be visible (dtree_runtime.py:190-191 semantics)."""
    if mask.shape != (L, P + L):
        raise ValueError(f"attention_mask must have shape ({L}, {P + L}), got {tuple(mask.shape)}")
    if P and not mask[:, :P].all():
        raise NotImplementedError("tree verification attends to the whole prefix; masked prefix columns are not supported")
    tree = mask[:, P:]
    out = np.zeros((L, 4), dtype=np.uint32)
    for i in range(L):
        for j in np.nonzero(tree[i])[0]:
            out[i, j // 32] |= np.uint32(1 << (int(j) % 32))
    return out


class Qwen3TargetAdapter(MLXTargetAdapter):
    family = "qwen3"

    def make_cache(self, model: Qwen3TreeModel, speculative_linear_cache: bool = False) -> PagedKVCache:
        del speculative_linear_cache
        return model.engine.new_cache()

    def embed_tokens(self, model: Qwen3TreeModel, tokens) -> torch.Tensor:
        ids = torch.as_tensor(tokens, device=model.weights.device).long()
        return model.weights.embed_rows(ids)

    def _rows(self, model, hidden_states):
        h = hidden_states.reshape(-1, hidden_states.shape[-1])
        return h.to(model.weights.device, torch.bfloat16)

    def lm_head_logits(self, model: Qwen3TreeModel, hidden_states) -> torch.Tensor:
        """adapters.py:489-492 (tied embedding) on the HIP LM-head kernel, fp32 logits."""
        eng = model.engine
        h = self._rows(model, hidden_states)
        outs = []
        st = eng.stream_handle()
        for s in range(0, h.shape[0], eng.MP):
            part = h[s:s + eng.MP]
            eng.lm_in.zero_()
            eng.lm_in[: part.shape[0]].copy_(part)
            eng.launch_lm_head(st, x=eng.lm_in, ss=False, want_logits=True)
            outs.append(eng.logits[: part.shape[0]].clone())
        return torch.cat(outs, 0).reshape(*hidden_states.shape[:-1], -1)

    def lm_head_argmax(self, model: Qwen3TreeModel, hidden_states) -> torch.Tensor:
        """adapters.py:114-118: fused LM head + argmax (first index on ties)."""
        eng = model.engine
        h = self._rows(model, hidden_states)
        st = eng.stream_handle()
        post: list[int] = []
        for s in range(0, h.shape[0], eng.MP):
            part = h[s:s + eng.MP]
            n = part.shape[0]
            eng.lm_in.zero_()
            eng.lm_in[:n].copy_(part)
            eng.launch_lm_head(st, x=eng.lm_in, ss=False)
            eng.set_step([0] * n, [0] * n, [-1] + [0] * (n - 1), 0, aux=True)
            eng.launch_walk(st, aux=True)
            post.extend(eng.read_result().posterior[:n])
        return torch.tensor(post, dtype=torch.int64).reshape(hidden_states.shape[:-1])

    def forward_with_hidden_states(self, model: Qwen3TreeModel, inputs, cache: PagedKVCache, layer_ids,
                                   return_rollback_records: bool = False):
        """Causal forward over the prompt: the long-M GEMM path for 128 tokens
        or more (bf16 weights), else chains of up to max_nodes tokens through
        the tree kernels. Returns the logits of the last position only
        ([1, 1, V], all the callers read) and the verifier hidden states of
        every position."""
        eng = model.engine
        eng.set_layer_ids(layer_ids)
        toks = _as_list(inputs)
        if len(toks) >= 128 and eng.supports_long_prefill():
            logits, hidden = eng.prefill_long(cache, toks)
            target_hidden = (hidden[None] if hidden is not None
                             else torch.zeros(1, len(toks), 0, device=eng.dev))
            if return_rollback_records:
                return logits, target_hidden, {}
            return logits, target_hidden
        hid = []
        for s in range(0, len(toks), eng.max_nodes):
            part = toks[s:s + eng.max_nodes]
            P = cache.offset
            eng.forward_only(cache, part, [P + i for i in range(len(part))], [-1] + list(range(len(part) - 1)))
            cache.offset = P + len(part)
            if layer_ids:
                hid.append(eng.hidden[: len(part)].clone())
        last = len(toks) - 1 - (len(toks) - 1) // eng.max_nodes * eng.max_nodes
        eng.launch_lm_head(eng.stream_handle(), want_logits=True)
        logits = eng.logits[last:last + 1].clone()[None]
        target_hidden = torch.cat(hid, 0)[None] if hid else torch.zeros(1, len(toks), 0, device=eng.dev)
        if return_rollback_records:
            return logits, target_hidden, {}
        return logits, target_hidden

    def supports_tree_verification(self) -> bool:
        return True

    def forward_tree_with_hidden_states(self, model: Qwen3TreeModel, inputs, cache: PagedKVCache, layer_ids,
                                        parents, position_ids, attention_mask):
        """adapters.py:568-597: every layer's tree K/V is appended to the cache
        (offset += L); returns (norm_hidden [1,L,H], verifier_hidden [1,L,n*H])."""
        eng = model.engine
        eng.set_layer_ids(layer_ids)
        toks = _as_list(inputs)
        pos = _as_list(position_ids)
        L, P = len(toks), cache.offset
        mask = attention_mask.cpu().numpy() if isinstance(attention_mask, torch.Tensor) else np.asarray(attention_mask)
        anc = _mask_tree_bitsets(mask.astype(bool), P, L)
        par = list(parents) if parents is not None else [-1] + [0] * (L - 1)
        eng.set_step(toks, pos, par, P, ancestors=anc)
        eng.launch_forward(cache, eng.stream_handle(), norm_hidden=True)
        cache.offset = P + L
        H = model.args.hidden_size
        norm_hidden = eng.norm_hidden[:L].clone()[None]
        vh = eng.hidden[:L].clone()[None] if layer_ids else torch.zeros(1, L, 0, dtype=torch.bfloat16, device=eng.dev)
        del H
        return norm_hidden, vh

    def cache_summary(self, cache: PagedKVCache) -> str:
        return " ".join(f"{i}:kv={cache.offset}" for i in range(len(cache)))

    def compact_kv_caches(self, model: Qwen3TreeModel, cache: PagedKVCache, past_length: int,
                          keep_current_indices: list[int]) -> None:
        """adapters.py:635-668 on the HIP compaction kernel."""
        keep = [int(i) for i in keep_current_indices]
        current = cache.offset - past_length
        if current <= 0:
            return
        if not keep:
            cache.offset = past_length
            return
        if len(keep) == current:
            return
        if any(i < 0 or i >= current for i in keep):
            raise IndexError(f"keep indices must lie in [0, {current})")
        eng = model.engine
        eng.set_step([0] * current, [0] * current, [-1] + [0] * (current - 1), past_length, aux=True, accepted=keep)
        eng.launch_compact(cache, eng.stream_handle(), select_hidden=False, aux=True)
        cache.offset = past_length + len(keep)

    def rewind_kv_caches(self, cache: PagedKVCache, num_tokens: int) -> None:
        cache.offset = max(0, cache.offset - int(num_tokens))

    # ---- fused step (forward + LM-head argmax + walk + compaction) -----------
    def verify_tree(self, model: Qwen3TreeModel, inputs, cache: PagedKVCache, layer_ids, parents, position_ids,
                    attention_mask=None, child_maps=None):
        """Forward + LM-head argmax + walk + compaction as one graph. The
        device derives the ancestor masks from `parents` and walks the tree by
        (parent, token); a given `attention_mask` / `child_maps` must describe
        the same tree (the per-method path reads them instead), else ValueError."""
        eng = model.engine
        eng.set_layer_ids(layer_ids)
        toks, par = _as_list(inputs), [int(p) for p in parents]
        L, P = len(toks), cache.offset
        anc = ancestor_bitsets(par)
        if attention_mask is not None:
            mask = attention_mask.cpu().numpy() if isinstance(attention_mask, torch.Tensor) else np.asarray(attention_mask)
            if not np.array_equal(_mask_tree_bitsets(mask.astype(bool), P, L), anc):
                raise ValueError("attention_mask tree columns differ from the ancestor sets of `parents`")
        if child_maps is not None:
            if len(child_maps) != L:
                raise ValueError(f"child_maps has {len(child_maps)} entries for {L} nodes")
            expect: list[dict[int, int]] = [dict() for _ in range(L)]
            for i in range(1, L):
                expect[par[i]][toks[i]] = i
            if [dict(m) for m in child_maps] != expect:
                raise ValueError("child_maps differ from the (parent, token) children of the tree")
        res = eng.verify(cache, toks, _as_list(position_ids), par, use_graph=True)
        n = len(res.accepted)
        vh = eng.hidden_sel[:n].clone()[None] if layer_ids else None
        return res.accepted, res.bonus_token, vh


    def verify_tree_from_logits(self, model, draft_logits, budget: int, topk, root_token: int, cache, layer_ids):
        """build_dtree_tree + compile_dtree_tree on the device (the tree kernels
        write the step descriptor), then the fused verify step; one readback.
        Returns (node_token_ids, node_depths, parents, child_maps, accepted,
        bonus_token, verifier_hidden). The device tree follows the reference
        order rules exactly given its fp32 log-probs, whose logsumexp is
        summed in another order than the host path's."""
        eng = model.engine
        eng.set_layer_ids(layer_ids)
        res, (ids, depths, parents, child_maps) = eng.verify_from_logits(cache, draft_logits, budget, topk,
                                                                         int(root_token))
        n = len(res.accepted)
        vh = eng.hidden_sel[:n].clone()[None] if layer_ids else None
        return ids, depths, parents, child_maps, res.accepted, res.bonus_token, vh


class Qwen35TargetAdapter(Qwen3TargetAdapter):
    """Qwen3.5 hybrid adapter (adapters.py:257-448): forward_tree leaves the
    committed state untouched and keeps a pending tree state (here: the
    attention layers' tree K/V rows at [P, P + L) beyond the offset and the
    GatedDeltaNet layers' per-node inputs); compact_kv_caches commits it along
    the accepted path and raises without one (adapters.py:433-448)."""

    family = "qwen3_5"

    def __init__(self):
        self._pending_tree_state = None

    def make_cache(self, model: Qwen35TreeModel, speculative_linear_cache: bool = False) -> Qwen35Cache:
        del speculative_linear_cache
        return model.engine.new_cache()

    def forward_with_hidden_states(self, model: Qwen35TreeModel, inputs, cache: Qwen35Cache, layer_ids,
                                   return_rollback_records: bool = False):
        """Prefill (adapters.py:290-307, forward_dflash over the prompt): the
        long-M GEMM path for 128 tokens or more (bf16 weights), else fully
        accepted chains of <= max_nodes tokens through the tree kernels; the
        cache commits either way. Returns the last position's logits
        ([1, 1, V]) and every position's verifier hidden."""
        eng = model.engine
        eng.set_layer_ids(layer_ids)
        toks = _as_list(inputs)
        if len(toks) >= 128 and eng.supports_long_prefill():
            logits, hidden = eng.prefill_long(cache, toks)
            target_hidden = (hidden[None] if hidden is not None
                             else torch.zeros(1, len(toks), 0, device=eng.dev))
            if return_rollback_records:
                return logits, target_hidden, {}
            return logits, target_hidden
        hid = []
        n = 0
        for s in range(0, len(toks), eng.max_nodes):
            part = toks[s:s + eng.max_nodes]
            eng.commit_chain(cache, part)
            n = len(part)
            if layer_ids:
                hid.append(eng.hidden[:n].clone())
        eng.launch_lm_head(eng.stream_handle(), want_logits=True)
        logits = eng.logits[n - 1:n].clone()[None]
        target_hidden = torch.cat(hid, 0)[None] if hid else torch.zeros(1, len(toks), 0, device=eng.dev)
        if return_rollback_records:
            return logits, target_hidden, {}
        return logits, target_hidden

    def forward_tree_with_hidden_states(self, model: Qwen35TreeModel, inputs, cache: Qwen35Cache, layer_ids,
                                        parents, position_ids, attention_mask):
        """adapters.py:411-431 (forward_qwen35_tree_with_hidden_states,
        qwen35_tree.py:629-705): the offset stays at P; the tree is pending."""
        eng = model.engine
        eng.set_layer_ids(layer_ids)
        toks = _as_list(inputs)
        pos = _as_list(position_ids)
        L, P = len(toks), cache.offset
        if parents is None or len(parents) != L:
            raise ValueError(f"tree parent list length must match verify length, got "
                             f"{None if parents is None else len(parents)} vs {L}")
        mask = attention_mask.cpu().numpy() if isinstance(attention_mask, torch.Tensor) else np.asarray(attention_mask)
        anc = _mask_tree_bitsets(mask.astype(bool), P, L)
        eng.set_step(toks, pos, list(parents), P, ancestors=anc)
        eng.launch_forward(cache, eng.stream_handle(), norm_hidden=True)
        self._pending_tree_state = (P, L, [int(p) for p in parents])
        norm_hidden = eng.norm_hidden[:L].clone()[None]
        vh = eng.hidden[:L].clone()[None] if layer_ids else torch.zeros(1, L, 0, dtype=torch.bfloat16, device=eng.dev)
        return norm_hidden, vh

    def compact_kv_caches(self, model: Qwen35TreeModel, cache: Qwen35Cache, past_length: int,
                          keep_current_indices: list[int]) -> None:
        """commit_qwen35_tree_path (qwen35_tree.py:708-732) on the HIP kernels:
        KV compaction of the attention layers, then every GatedDeltaNet layer's
        window / state replayed along the accepted path."""
        if self._pending_tree_state is None:
            raise RuntimeError("Qwen3.5 tree compaction requires pending tree state.")
        P, L, parents = self._pending_tree_state
        self._pending_tree_state = None
        keep = [int(i) for i in keep_current_indices]
        if not keep:
            return
        if keep[0] != 0 or any(parents[b] != a for a, b in zip(keep, keep[1:])):
            raise ValueError("accepted indices must be a root path of the pending tree")
        eng = model.engine
        eng.set_step([0] * L, [0] * L, parents, P, aux=True, accepted=keep)
        eng.launch_compact(cache, eng.stream_handle(), select_hidden=False, aux=True)
        eng._keep_commit(cache, P, len(keep))

    def cache_summary(self, cache: Qwen35Cache) -> str:
        c = cache.cfg
        parts = []
        for i in range(c.num_hidden_layers):
            if c.is_linear(i):
                parts.append(f"{i}:ssm=(1, {c.linear_num_value_heads}, {c.linear_value_head_dim}, "
                             f"{c.linear_key_head_dim})")
            else:
                parts.append(f"{i}:kv={cache.offset}")
        return " ".join(parts)


ADAPTERS: dict[str, type[MLXTargetAdapter]] = {"qwen3": Qwen3TargetAdapter, "qwen3_5": Qwen35TargetAdapter}


def adapter_for_model_type(model_type: str):
    return ADAPTERS.get(model_type)


@dataclass
class LoadedTargetModel:
    """Facade of adapters.py:681-819: delegates every call to the adapter."""

    requested_model: str
    resolved_model_path: Path | None
    model: Any
    tokenizer: Any
    adapter: MLXTargetAdapter
    last_verify_compacted: bool = field(default=False)

    def stop_token_ids(self) -> set[int]:
        if self.tokenizer is not None and hasattr(self.tokenizer, "eos_token_ids"):
            e = self.tokenizer.eos_token_ids
            return {e} if isinstance(e, int) else set(e)
        return set()

    def make_cache(self, speculative_linear_cache: bool = False):
        return self.adapter.make_cache(self.model, speculative_linear_cache=speculative_linear_cache)

    def embed_tokens(self, tokens):
        return self.adapter.embed_tokens(self.model, tokens)

    def lm_head_logits(self, hidden_states):
        return self.adapter.lm_head_logits(self.model, hidden_states)

    def lm_head_argmax(self, hidden_states):
        return self.adapter.lm_head_argmax(self.model, hidden_states)

    def forward_with_hidden_states(self, inputs, cache, layer_ids, return_rollback_records=False):
        return self.adapter.forward_with_hidden_states(self.model, inputs, cache, layer_ids,
                                                       return_rollback_records=return_rollback_records)

    def supports_tree_verification(self) -> bool:
        return self.adapter.supports_tree_verification()

    def forward_tree_with_hidden_states(self, inputs, cache, layer_ids, parents, position_ids, attention_mask):
        return self.adapter.forward_tree_with_hidden_states(self.model, inputs, cache, layer_ids, parents,
                                                            position_ids, attention_mask)

    def cache_summary(self, cache) -> str:
        return self.adapter.cache_summary(cache)

    def compact_kv_caches(self, cache, past_length: int, keep_current_indices: list[int]) -> None:
        self.adapter.compact_kv_caches(self.model, cache, past_length, keep_current_indices)

    def rewind_kv_caches(self, cache, num_tokens: int) -> None:
        self.adapter.rewind_kv_caches(cache, num_tokens)

    def verify_tree(self, inputs, cache, layer_ids, parents, position_ids, attention_mask=None, child_maps=None):
        out = self.adapter.verify_tree(self.model, inputs, cache, layer_ids, parents, position_ids,
                                       attention_mask, child_maps)
        self.last_verify_compacted = True
        return out

    def verify_tree_from_logits(self, draft_logits, budget: int, topk, root_token: int, cache, layer_ids):
        out = self.adapter.verify_tree_from_logits(self.model, draft_logits, budget, topk, root_token, cache,
                                                   layer_ids)
        self.last_verify_compacted = True
        return out


def load_target_model(spec: str | Qwen3Config | Qwen35Config = "random:qwen3-4b", seed: int = 0,
                      max_past: int = 4096, device: str = "cuda", layer_ids=(), norm_jitter: float = 0.0,
                      quant: str = "bf16") -> LoadedTargetModel:
    """Random-init target (no checkpoint download: weights ~ N(0, 0.02), seeded).
    ``spec`` is "random:qwen3-4b", "random:qwen35-4b" or a Qwen3Config /
    Qwen35Config (adapters.py:822-846 resolves a model name instead)."""
    if isinstance(spec, (Qwen3Config, Qwen35Config)):
        cfg, name = spec, "random:custom"
    elif spec in ("random:qwen3-4b", "qwen3-4b"):
        cfg, name = QWEN3_4B, spec
    elif spec in ("random:qwen35-4b", "qwen35-4b"):
        cfg, name = QWEN35_4B, spec
    else:
        raise NotImplementedError(f"Unsupported target {spec!r}: only random-init Qwen3 / Qwen3.5 configs")
    cls = adapter_for_model_type(cfg.model_type)
    if isinstance(cfg, Qwen35Config):
        weights = Qwen35Weights.random(cfg, seed=seed, device=device, norm_jitter=norm_jitter, quant=quant)
        model = Qwen35TreeModel(cfg, weights, max_past=max_past, layer_ids=layer_ids)
    else:
        if quant == "q4":
            weights = Qwen3Weights.random_q4(cfg, seed=seed, device=device, norm_jitter=norm_jitter)
        else:
            weights = Qwen3Weights.random(cfg, seed=seed, device=device, norm_jitter=norm_jitter)
        model = Qwen3TreeModel(cfg, weights, max_past=max_past, layer_ids=layer_ids)
    return LoadedTargetModel(requested_model=name, resolved_model_path=None, model=model, tokenizer=None,
                             adapter=cls())
