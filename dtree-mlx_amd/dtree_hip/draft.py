"""DFlash drafter on the HIP kernels (DFlashDraftModel, draft.py:25-367 of the
reference), with the reference's class names, arguments and cache semantics.

A drafter call takes the target's hidden rows of the newly committed tokens
(``target_hidden``, [1, T, n_target_layers * H]) and the embedding of one
block (the root token followed by mask tokens, ``noise_embedding``,
[1, block, H]) and returns the block's normed hidden rows, from which the
target's LM head gives the draft logits (dtree_runtime.py:365-378).

Device path per call:
  context  (T rows, 128 per pass): tile the rows, fc GEMM with the
           hidden_norm fold (RESIDUAL epilogue into a zeroed x), then per
           layer the k/v rows of the fused QKV weight (GEMM, row scale =
           hidden_norm) and dtree_kv_append (k_norm, RoPE at the running
           offset, paged bf16 write; ring slots for the context-only cache);
  block    dtree_rows_in (input_layernorm fold), RoPE table, then the Qwen3
           decoder stack of the verify engine, where attention is the tree
           attention kernel over [context keys ; block] with every block row
           visible to every block query (mask mode "none") or the block's
           lower triangle (mask mode "causal"), and the final RMSNorm.

Cache semantics (draft.py:67-110, 186-257, runtime.py:22-26):
  "kv"            one mlx KVCache per layer: the context rows are appended at
                  the offset, the block's K/V rows are written after them and
                  the offset advances by the block; trim(block) takes it back.
  "context-only"  ContextOnlyDraftKVCache: only context rows are kept, the
                  first 64 and the newest 1024; the block's keys are used
                  but never stored and trim is a no-op. The newest rows live
                  in ring slots, which only reorders keys that the unmasked
                  attention of this mode sums over.
Without a cache (``cache=None``) the reference projects the context keys at
positions 0 .. T-1 and the block after them: exactly what the cached path
does on an empty cache, which this module runs on a temporary one.
"""
from __future__ import annotations

import ctypes as C
import re
from dataclasses import dataclass
from typing import Any

import torch

from . import _native as N
from .cache import PagedKVCache
from .config import Qwen3Config
from .engine import Qwen3TreeEngine
from .weights import Q4Linear, Qwen3Weights, fp16_exact_bf16, q4_random_mlx, q4_to_tiled, tile_weight_f16

CONTEXT_SINK = 64      # ContextOnlyDraftKVCache defaults, draft.py:68
CONTEXT_WINDOW = 1024


@dataclass
class DraftArgs:
    """Drafter config.json fields (draft.py:25-64)."""
    model_type: str
    hidden_size: int
    num_hidden_layers: int
    intermediate_size: int
    num_attention_heads: int
    rms_norm_eps: float
    vocab_size: int
    num_key_value_heads: int
    max_position_embeddings: int
    rope_theta: float
    head_dim: int
    tie_word_embeddings: bool
    attention_bias: bool = False
    attention_dropout: float = 0.0
    rope_scaling: dict | None = None
    block_size: int = 16
    dflash_config: dict | None = None

    @classmethod
    def from_dict(cls, config: dict[str, Any]) -> "DraftArgs":
        keys = set(cls.__dataclass_fields__)
        return cls(**{k: config[k] for k in keys if k in config})

    def stack_config(self) -> Qwen3Config:
        """The decoder-layer geometry as a Qwen3 config (the drafter layers are
        Qwen3 decoder layers with another attention input)."""
        if self.attention_bias:
            raise NotImplementedError("drafter attention with bias terms")
        if self.rope_scaling:
            raise NotImplementedError("drafter RoPE scaling")
        if not self.dflash_config or "target_layer_ids" not in self.dflash_config:
            raise ValueError("dflash_config.target_layer_ids is required")
        return Qwen3Config(hidden_size=self.hidden_size, num_hidden_layers=self.num_hidden_layers,
                           intermediate_size=self.intermediate_size, num_attention_heads=self.num_attention_heads,
                           num_key_value_heads=self.num_key_value_heads, head_dim=self.head_dim, vocab_size=32,
                           rms_norm_eps=self.rms_norm_eps, rope_theta=self.rope_theta, model_type="dflash_draft")


def build_target_layer_ids(num_target_layers: int, count: int) -> list[int]:
    """Target layers whose hidden states feed the drafter: `count` layers
    evenly spaced from layer 1 to layer num_target_layers - 3, ascending and
    distinct (the target concatenates the hidden states of a layer set in
    layer order, adapters.py:506-509), so shallow targets get fewer."""
    if count <= 1 or num_target_layers <= 1:
        return [min(num_target_layers // 2, num_target_layers - 1)]
    start, end = min(1, num_target_layers - 1), max(min(1, num_target_layers - 1), num_target_layers - 3)
    span = end - start
    return sorted({int(round(start + i * span / (count - 1))) for i in range(count)})


def random_draft_config(target_args, spec: str = "dflash-b16") -> DraftArgs:
    """A DFlash drafter sized for ``target_args`` (Qwen3 / Qwen3.5 target
    config): ``dflash-b<block>[-l<layers>]``, default 5 layers, 32 query / 8 KV
    heads of 128, the target's hidden and FFN sizes, vocabulary and RoPE base;
    the mask token is the last vocabulary id."""
    m = re.fullmatch(r"dflash-b(\d+)(?:-l(\d+))?", spec)
    if m is None:
        raise NotImplementedError(f"draft spec {spec!r}: expected 'dflash-b<block>[-l<layers>]'")
    block, layers = int(m.group(1)), int(m.group(2) or 5)
    if not 2 <= block <= N.MAX_NODES:
        raise ValueError(f"draft block size must be in [2, {N.MAX_NODES}]")
    H = target_args.hidden_size
    ffn = getattr(target_args, "intermediate_size", 3 * H)
    heads = 32 if H >= 2048 else max(2, H // 128)
    kv = max(1, heads // 4)
    n_target = target_args.num_hidden_layers
    return DraftArgs(model_type="qwen3", hidden_size=H, num_hidden_layers=layers, intermediate_size=ffn,
                     num_attention_heads=heads, rms_norm_eps=getattr(target_args, "rms_norm_eps", 1e-6),
                     vocab_size=target_args.vocab_size, num_key_value_heads=kv, max_position_embeddings=40960,
                     rope_theta=getattr(target_args, "rope_theta", 1_000_000.0), head_dim=128,
                     tie_word_embeddings=False, block_size=block,
                     dflash_config={"target_layer_ids": build_target_layer_ids(n_target, layers),
                                    "mask_token_id": target_args.vocab_size - 1})


@dataclass
class DFlashWeights:
    """Drafter weights: the decoder stack (Qwen3 layer layout: fused QKV,
    interleaved gate/up), fc [H, n_target * H], hidden_norm and the final norm
    (stack.final_norm)."""
    stack: Qwen3Weights
    fc: Any
    hidden_norm: torch.Tensor

    @property
    def device(self) -> torch.device:
        return self.stack.final_norm.device

    @classmethod
    def random(cls, args: DraftArgs, seed: int = 0, device="cuda", std: float = 0.02, norm_jitter: float = 0.0,
               quant: str = "bf16") -> "DFlashWeights":
        scfg = args.stack_config()
        n_in = len(args.dflash_config["target_layer_ids"]) * args.hidden_size
        dev = torch.device(device)
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed + 7919)
        if quant == "q4":
            stack = Qwen3Weights.random_q4(scfg, seed=seed, device=dev, norm_jitter=norm_jitter)
            fc = Q4Linear(*q4_to_tiled(*q4_random_mlx(args.hidden_size, n_in, gen, dev)))
        elif quant == "bf16":
            stack = Qwen3Weights.random(scfg, seed=seed, device=dev, std=std, norm_jitter=norm_jitter)
            t = torch.empty(args.hidden_size, n_in, dtype=torch.float32, device=dev).normal_(0.0, std, generator=gen)
            fc = tile_weight_f16(fp16_exact_bf16(t))
        else:
            raise NotImplementedError(f"draft weights {quant!r}: bf16 or q4")
        if norm_jitter:
            hn = (1.0 + torch.empty(args.hidden_size, device=dev).normal_(0.0, norm_jitter, generator=gen))
            hidden_norm = hn.to(torch.bfloat16)
        else:
            hidden_norm = torch.ones(args.hidden_size, dtype=torch.bfloat16, device=dev)
        return cls(stack=stack, fc=fc, hidden_norm=hidden_norm)

    def host_accessor(self):
        """(layer, name) -> numpy bf16 bits / fp32 in nn.Linear layout: the
        decoder stack's names plus (None, 'fc' | 'hidden_norm' | 'norm')."""
        get_stack = self.stack.host_accessor()

        def get(layer, name):
            if layer is None:
                if name == "fc":
                    t = self.stack.rowmajor(self.fc)
                elif name == "hidden_norm":
                    t = self.hidden_norm
                elif name == "norm":
                    t = self.stack.final_norm
                else:
                    raise KeyError(name)
                t = t.detach().to("cpu").contiguous()
                return t.numpy() if t.dtype == torch.float32 else t.view(torch.int16).numpy().view("uint16")
            return get_stack(layer, name)

        return get


class DraftLayerCache:
    """One layer of a DFlashDraftCache with the mlx cache surface the
    runtime uses (offset, trim); keys / values read the stored rows back in
    slot order (bf16, [1, Hkv, n, D])."""

    def __init__(self, owner: "DFlashDraftCache", layer: int):
        self._owner = owner
        self.layer = layer
        self.offset = 0

    def trim(self, num_tokens: int) -> int:
        if self._owner.mode == "context-only":
            return 0
        n = min(self.offset, max(int(num_tokens), 0))
        self.offset -= n
        return n

    def fetch(self):
        n = self._owner.stored_length(self.offset)
        st = self._owner.store
        return st.logical_keys(self.layer, n)[None], st.logical_values(self.layer, n)[None]


class DFlashDraftCache:
    """Per-layer drafter caches over one paged store (list-like, as
    DFlashDraftModel.make_cache returns, draft.py:323-326)."""

    def __init__(self, layers: int, kv_heads: int, head_dim: int, mode: str, max_past: int, block: int, device,
                 sink: int = CONTEXT_SINK, window: int = CONTEXT_WINDOW):
        if mode not in ("kv", "context-only"):
            raise ValueError(f"draft cache mode {mode!r}: 'kv' or 'context-only'")
        self.mode = mode
        self.sink, self.window = (sink, window) if mode == "context-only" else (0, 0)
        self.capacity = sink + window if mode == "context-only" else max_past + block
        self.store = PagedKVCache(layers, kv_heads, head_dim, self.capacity, device=device)
        self.layers = [DraftLayerCache(self, i) for i in range(layers)]

    def __len__(self) -> int:
        return len(self.layers)

    def __getitem__(self, i: int) -> DraftLayerCache:
        return self.layers[i]

    def __iter__(self):
        return iter(self.layers)

    @property
    def offset(self) -> int:
        offs = {lc.offset for lc in self.layers}
        if len(offs) != 1:
            raise ValueError("drafter layer caches disagree on their offset")
        return offs.pop()

    def stored_length(self, offset: int | None = None) -> int:
        off = self.offset if offset is None else offset
        return min(off, self.sink + self.window) if self.mode == "context-only" else off


class DFlashDraftEngine(Qwen3TreeEngine):
    """Launches of one drafter call (module docstring)."""

    CTX_ROWS = 128

    def __init__(self, args: DraftArgs, weights: DFlashWeights, max_past: int):
        self.args = args
        self.dw = weights
        self.n_in = len(args.dflash_config["target_layer_ids"]) * args.hidden_size
        if self.n_in % 64:
            raise ValueError("n_target_layers * hidden_size must be a multiple of 64")
        super().__init__(weights.stack.cfg, weights.stack, max_past=max(int(max_past), CONTEXT_SINK + CONTEXT_WINDOW),
                         max_nodes=args.block_size)
        c, CT, dev = self.cfg, self.CTX_ROWS, self.dev
        bf16, f32 = torch.bfloat16, torch.float32
        self.th_rm = torch.zeros(CT, self.n_in, dtype=bf16, device=dev)
        self.th_t = torch.zeros(CT, self.n_in, dtype=self.act_dtype, device=dev)
        self.x_ctx = torch.zeros(CT, c.hidden_size, dtype=f32, device=dev)
        self.ctx_g = torch.zeros(2, CT, c.hidden_size, dtype=self.act_dtype, device=dev)
        self.ss_ctx = torch.zeros(CT // 32, c.hidden_size // 32, 32, dtype=f32, device=dev)
        self.kv = torch.zeros(CT, 2 * c.kv_dim, dtype=f32, device=dev)
        self.noise = torch.zeros(self.MP, c.hidden_size, dtype=bf16, device=dev)
        ws = max(self.lib.dtree_gemm_workspace_bytes(rp, n, k, 0)
                 for rp in (32, 64, 96, 128) for n, k in ((c.hidden_size, self.n_in), (2 * c.kv_dim, c.hidden_size)))
        if ws > self.gemm_ws.numel():
            self.gemm_ws = torch.zeros(ws, dtype=torch.uint8, device=dev)

    def _kv_weight(self, li: int):
        """The k and v rows of the fused QKV weight (a row-block suffix of
        either layout)."""
        w = self.w.layers[li].wqkv
        q = self.cfg.q_dim
        if isinstance(w, Q4Linear):
            return Q4Linear(w.words[q // 32:], w.sb[q // 32:])
        return w[q:]

    def _ctx_gemm(self, name, rows_padded, x, ldx, w, epi, st, **kw) -> None:
        a = self.gemm_args(name, x, ldx, w, epi, **kw)
        a.rows_padded = rows_padded
        N.check(self.lib.dtree_gemm_bf16(C.byref(a), st), f"gemm {name}")

    def prepare_context(self, rows: torch.Tensor, st: int) -> int:
        """fc + hidden_norm fold of up to CTX_ROWS target hidden rows into
        ctx_g / ss_ctx; returns the padded row count."""
        n = rows.shape[0]
        rp = 32 * ((n + 31) // 32)
        self.th_rm[:n].copy_(rows)
        if rp > n:
            self.th_rm[n:rp].zero_()
        tile = self.lib.dtree_tile_weight_f16 if self.h16 else self.lib.dtree_tile_weight
        N.check(tile(self.th_rm.data_ptr(), self.th_t.data_ptr(), rp, self.n_in, st),
                "tile target hidden")
        self.x_ctx[:rp].zero_()
        self._ctx_gemm("fc", rp, self.th_t[:rp], self.n_in, self.dw.fc, N.EPI_RESIDUAL, st, out_f32=self.x_ctx,
                       out_bf16=self.ctx_g, next_norm=self.dw.hidden_norm, ss_out=self.ss_ctx)
        return rp

    def append_context(self, target_hidden: torch.Tensor, cache: DFlashDraftCache) -> None:
        """precompute_context_kv (draft.py:186-206, 334-346) for every layer."""
        c = self.cfg
        T = target_hidden.shape[0]
        if T == 0:
            return
        off = cache.offset
        if cache.mode == "kv" and off + T > self.max_past:
            raise ValueError(f"draft context of {off + T} positions exceeds max_past {self.max_past}")
        st = self.stream_handle()
        store = cache.store
        for s in range(0, T, self.CTX_ROWS):
            rows = target_hidden[s:s + self.CTX_ROWS]
            n = rows.shape[0]
            rp = self.prepare_context(rows, st)
            for li in range(c.num_hidden_layers):
                lw = self.w.layers[li]
                self._ctx_gemm("kv", rp, self.ctx_g, c.hidden_size, self._kv_weight(li), N.EPI_STORE_F32, st,
                               ss_in=self.ss_ctx, out_f32=self.kv)
                N.check(self.lib.dtree_kv_append(
                    self.kv.data_ptr(), self.kv.shape[1], n, off + s, lw.k_norm.data_ptr(), c.rms_norm_eps,
                    c.num_key_value_heads, c.head_dim, c.rope_theta, cache.sink, cache.window,
                    store.k_ptr(li), store.v_ptr(li), store.page_table.data_ptr(), cache.capacity, st),
                    "kv append")
        for lc in cache.layers:
            lc.offset += T

    def draft_block(self, noise: torch.Tensor, cache: DFlashDraftCache, mask_mode: str) -> torch.Tensor:
        """The decoder stack over the block rows; returns the normed hidden
        rows [L, H] (bf16, a fresh tensor)."""
        c = self.cfg
        L = noise.shape[0]
        if not 1 <= L <= self.max_nodes:
            raise ValueError(f"draft block of {L} rows: the drafter takes 1..{self.max_nodes}")
        off = cache.offset
        P = cache.stored_length(off)
        if cache.mode == "context-only" and off == 0:
            raise ValueError("Context-only draft cache is missing precomputed context.")
        if cache.mode == "kv" and off > self.max_past:
            raise ValueError(f"draft cache offset {off} exceeds max_past {self.max_past}")
        causal = mask_mode == "causal" and cache.mode == "kv" and L > 1
        if not causal and L > 32:
            # the tree attention reads tree chunk j only for query blocks >= j
            raise NotImplementedError("unmasked drafter blocks of more than 32 rows")
        chain = [-1] + list(range(L - 1))
        if causal:
            anc = None  # ancestor-or-self of a chain: the lower triangle
        else:
            full = (1 << L) - 1
            row = [(full >> (32 * w)) & 0xFFFFFFFF for w in range(N.MASK_WORDS)]
            anc = [row] * L
        st = self.stream_handle()
        self.set_step([0] * L, [off + i for i in range(L)], chain, P, ancestors=anc)
        self.noise[:L].copy_(noise)
        N.check(self.lib.dtree_rows_in(
            self.noise.data_ptr(), c.hidden_size, L, self.w.layers[0].input_norm.data_ptr(), self.MP, c.hidden_size,
            self.x.data_ptr(), self.xg[0].data_ptr(), self.lo_ptr(self.xg), self.w.layout, self.ss.data_ptr(), st),
            "rows in")
        N.check(self.lib.dtree_rope_table(self.desc.data_ptr(), self.MP, c.head_dim, c.rope_theta,
                                          self.rope_cos.data_ptr(), self.rope_sin.data_ptr(), st), "rope table")
        write = cache.mode == "kv"
        # the context-only store's page table covers its sink + window only
        self.attn_max_past = self.attn_grid_past(P) if write else cache.capacity
        self._launch_layers(cache.store, st, norm_hidden=True, write_cache=write)
        if write:
            for lc in cache.layers:
                lc.offset += L
        return self.norm_hidden[:L].clone()


class DFlashDraftModel:
    """DFlashDraftModel (draft.py:308-367) on the HIP kernels."""

    def __init__(self, args: DraftArgs, weights: DFlashWeights, *, max_past: int = 4096):
        args.stack_config()  # validates the config
        self.args = args
        self.weights = weights
        self.target_layer_ids = list(args.dflash_config["target_layer_ids"])
        self.block_size = int(args.block_size)
        self.mask_token_id = int(args.dflash_config["mask_token_id"])
        self.attention_mask_mode = "none"
        self.cache_mode = "kv"
        self.engine = DFlashDraftEngine(args, weights, max_past)

    @classmethod
    def random(cls, args: DraftArgs, target=None, seed: int = 0, quant: str = "bf16", max_past: int | None = None,
               device=None, norm_jitter: float = 0.0) -> "DFlashDraftModel":
        """Seeded random-init drafter on the target's device (max_past defaults
        to the target engine's)."""
        eng = getattr(getattr(target, "model", None), "engine", None)
        if device is None:
            device = eng.dev if eng is not None else "cuda"
        if max_past is None:
            max_past = eng.max_past if eng is not None else 4096
        w = DFlashWeights.random(args, seed=seed + 1, device=device, quant=quant, norm_jitter=norm_jitter)
        return cls(args, w, max_past=max_past)

    @property
    def num_layers(self) -> int:
        return self.args.num_hidden_layers

    def make_cache(self) -> DFlashDraftCache:
        a = self.args
        return DFlashDraftCache(a.num_hidden_layers, a.num_key_value_heads, a.head_dim, self.cache_mode,
                                self.engine.max_past, self.engine.MP, self.engine.dev)

    def _rows(self, t: torch.Tensor, width: int, what: str) -> torch.Tensor:
        t = torch.as_tensor(t)
        if t.dim() == 3:
            if t.shape[0] != 1:
                raise ValueError(f"{what}: batch size 1 only")
            t = t[0]
        if t.dim() != 2 or t.shape[1] != width:
            raise ValueError(f"{what}: expected [1, n, {width}], got {tuple(t.shape)}")
        return t.to(self.engine.dev, torch.bfloat16).contiguous()

    def prepare_target_hidden(self, target_hidden) -> torch.Tensor:
        """hidden_norm(fc(target_hidden)) (draft.py:331-332), bf16 [1, T, H]."""
        eng = self.engine
        th = self._rows(target_hidden, eng.n_in, "target_hidden")
        H = self.args.hidden_size
        st = eng.stream_handle()
        outs = []
        for s in range(0, th.shape[0], eng.CTX_ROWS):
            rows = th[s:s + eng.CTX_ROWS]
            rp = eng.prepare_context(rows, st)
            out = torch.empty(rp, H, dtype=torch.bfloat16, device=eng.dev)
            N.check(eng.lib.dtree_rownorm(eng.x_ctx.data_ptr(), H, rp, H, eng.ss_ctx.data_ptr(), H // 32,
                                          self.weights.hidden_norm.data_ptr(), self.args.rms_norm_eps,
                                          out.data_ptr(), H, st), "rownorm")
            outs.append(out[: rows.shape[0]])
        return torch.cat(outs, 0)[None] if outs else torch.zeros(1, 0, H, dtype=torch.bfloat16, device=eng.dev)

    def precompute_context_kv(self, target_hidden, cache: DFlashDraftCache | None) -> None:
        """draft.py:334-346 (takes the raw target hidden rows; fc and
        hidden_norm are applied on the way)."""
        if cache is None:
            return
        self._check_cache(cache)
        self.engine.append_context(self._rows(target_hidden, self.engine.n_in, "target_hidden"), cache)

    def _check_cache(self, cache) -> None:
        if not isinstance(cache, DFlashDraftCache):
            raise TypeError("drafter caches come from DFlashDraftModel.make_cache()")
        if cache.store.k_pages.device != self.engine.dev:
            raise ValueError("drafter cache lives on another device")

    def __call__(self, noise_embedding, target_hidden, cache: DFlashDraftCache | None = None) -> torch.Tensor:
        """draft.py:349-364 -> normed hidden [1, block, H] (bf16)."""
        noise = self._rows(noise_embedding, self.args.hidden_size, "noise_embedding")
        if cache is None:
            # Context at positions 0 .. T-1 and the block after it (draft.py:243-258)
            # is the cached computation on an empty cache.
            saved = self.cache_mode
            self.cache_mode = "kv"
            try:
                cache = self.make_cache()
            finally:
                self.cache_mode = saved
        self.precompute_context_kv(target_hidden, cache)
        return self.engine.draft_block(noise, cache, self.attention_mask_mode)[None]
