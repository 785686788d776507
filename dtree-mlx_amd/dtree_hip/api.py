"""Generator facade over the HIP target (api.py:29-170 of the reference).

`DFlashGenerator` keeps the reference's constructor arguments, methods and
result type. Models are resolved without any download: a target spec is a
`LoadedTargetModel`, a Qwen3 / Qwen3.5 config or "random:qwen3-4b" /
"random:qwen35-4b" (seeded random-init weights); a draft model is any
drafter object with the DFlash drafter interface (block_size,
mask_token_id, target_layer_ids, make_cache(), __call__(noise_embedding=,
target_hidden=, cache=)) or a "random:" spec that builds the HIP DFlash
drafter with random-init weights sized for the target.
"""
from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path
from typing import Any

import torch

from .adapters import LoadedTargetModel, load_target_model
from .dtree_runtime import dtree_generate
from .runtime import dflash_generate

DEFAULT_TARGET_MODEL = "random:qwen3-4b"
DEFAULT_DRAFT_MODEL = "random:dflash-b16"


@dataclass
class DFlashResult:
    text: str
    output_tokens: list[int]
    generated_tokens: list[int]
    metrics: dict[str, Any]


def _resolve_draft(spec, target: LoadedTargetModel, seed: int, quant_bits: int | None):
    if not isinstance(spec, str):
        return spec
    if spec.startswith("random:"):
        from .draft import DFlashDraftModel, random_draft_config

        cfg = random_draft_config(target.model.args, spec.split(":", 1)[1])
        return DFlashDraftModel.random(cfg, target, seed=seed, quant="q4" if quant_bits == 4 else "bf16")
    raise NotImplementedError(f"draft model {spec!r}: only drafter objects and 'random:' specs load offline")


class DFlashGenerator:
    """api.py:29-170: owns a target and a drafter, dispatches generate calls to
    dflash_generate (linear verify) or dtree_generate (tree verify)."""

    def __init__(self, target_model=DEFAULT_TARGET_MODEL, draft_model=DEFAULT_DRAFT_MODEL,
                 draft_attention_mask: str = "auto", target_quant_bits: int | None = None,
                 target_quant_group_size: int = 64, draft_quant_bits: int | None = None,
                 draft_quant_group_size: int = 64, seed: int = 0, *, max_past: int = 4096,
                 device: str = "cuda", tokenizer=None):
        torch.manual_seed(seed)
        if target_quant_bits not in (None, 4) or (target_quant_bits == 4 and target_quant_group_size != 64):
            raise NotImplementedError("target quantisation is 4-bit affine groups of 64 (or none)")
        if draft_quant_bits not in (None, 4) or (draft_quant_bits == 4 and draft_quant_group_size != 64):
            raise NotImplementedError("draft quantisation is 4-bit affine groups of 64 (or none)")
        self.requested_target_model = target_model
        self.requested_draft_model = draft_model
        if isinstance(target_model, LoadedTargetModel):
            if target_quant_bits is not None:
                raise ValueError("target_quant_bits applies to targets built here, not to a loaded target")
            self.target = target_model
        else:
            self.target = load_target_model(target_model, seed=seed, max_past=max_past, device=device,
                                            quant="q4" if target_quant_bits == 4 else "bf16")
        if tokenizer is not None:
            self.target.tokenizer = tokenizer
        self.target_quantization = ({"group_size": 64, "bits": 4} if target_quant_bits == 4 else None)
        self.draft = _resolve_draft(draft_model, self.target, seed, draft_quant_bits)
        self.draft_path = None
        if draft_attention_mask == "auto":
            draft_attention_mask = "none"
        self.draft_attention_mask = draft_attention_mask
        if hasattr(self.draft, "attention_mask_mode"):
            self.draft.attention_mask_mode = draft_attention_mask
        if hasattr(self.draft, "cache_mode"):
            self.draft.cache_mode = "context-only" if self.target.adapter.family == "qwen3_5" else "kv"
        self.draft_quantization = ({"group_size": 64, "bits": 4} if draft_quant_bits == 4 else None)

    @property
    def target_model_path(self) -> Path | None:
        return self.target.resolved_model_path

    def encode_prompt(self, prompt_text: str):
        tok = self.target.tokenizer
        if tok is None:
            raise NotImplementedError("no tokenizer: pass tokenizer= (an object with encode/decode) or use "
                                      "generate_from_tokens")
        return torch.tensor(tok.encode(prompt_text), dtype=torch.int64)

    def _layer_ids(self) -> list[int]:
        ids = getattr(self.draft, "target_layer_ids", None)
        return list(ids) if ids is not None else []

    def generate_from_tokens(self, prompt_tokens, max_new_tokens: int = 256, temperature: float = 0.0,
                             speculative_tokens: int | None = None, decode_mode: str = "dflash",
                             tree_budget: int | None = None, verify_mode: str = "parallel-replay",
                             verify_chunk_size: int = 4, reset_peak_memory: bool = True,
                             skip_special_tokens: bool = False, profile: bool = False) -> DFlashResult:
        if reset_peak_memory and torch.cuda.is_available():
            torch.cuda.reset_peak_memory_stats()
        if decode_mode == "dflash":
            output_tokens, metrics = dflash_generate(
                target=self.target, draft=self.draft, prompt_tokens=prompt_tokens, max_new_tokens=max_new_tokens,
                temperature=temperature, stop_token_ids=self.target.stop_token_ids(), layer_ids=self._layer_ids(),
                speculative_tokens=speculative_tokens, verify_mode=verify_mode,
                verify_chunk_size=verify_chunk_size, profile=profile)
        elif decode_mode == "dtree":
            output_tokens, metrics = dtree_generate(
                target=self.target, draft=self.draft, prompt_tokens=prompt_tokens, max_new_tokens=max_new_tokens,
                temperature=temperature, stop_token_ids=self.target.stop_token_ids(), layer_ids=self._layer_ids(),
                speculative_tokens=speculative_tokens, tree_budget=tree_budget, verify_mode=verify_mode,
                profile=profile)
        else:
            raise ValueError(f"Unknown decode_mode={decode_mode!r}. Expected 'dflash' or 'dtree'.")
        generated_tokens = output_tokens[metrics["num_input_tokens"]:]
        tok = self.target.tokenizer
        text = tok.decode(generated_tokens, skip_special_tokens=skip_special_tokens) if tok is not None else ""
        return DFlashResult(text=text, output_tokens=output_tokens, generated_tokens=generated_tokens,
                            metrics=metrics)

    def generate(self, prompt_text: str, max_new_tokens: int = 256, temperature: float = 0.0,
                 speculative_tokens: int | None = None, decode_mode: str = "dflash", tree_budget: int | None = None,
                 verify_mode: str = "parallel-replay", verify_chunk_size: int = 4, reset_peak_memory: bool = True,
                 skip_special_tokens: bool = False, profile: bool = False) -> DFlashResult:
        return self.generate_from_tokens(
            prompt_tokens=self.encode_prompt(prompt_text), max_new_tokens=max_new_tokens, temperature=temperature,
            speculative_tokens=speculative_tokens, decode_mode=decode_mode, tree_budget=tree_budget,
            verify_mode=verify_mode, verify_chunk_size=verify_chunk_size, reset_peak_memory=reset_peak_memory,
            skip_special_tokens=skip_special_tokens, profile=profile)


# Method-agnostic alias (api.py:170).
Generator = DFlashGenerator
