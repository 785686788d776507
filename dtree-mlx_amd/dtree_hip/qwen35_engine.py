"""Qwen3.5 hybrid tree-verify executor (forward_qwen35_tree_with_hidden_states
+ commit_qwen35_tree_path, qwen35_tree.py:629-732, on the HIP kernels).

One step:
  embed (+ first input RMSNorm fold, RoPE table for the 64 rotary dims)
  GatedDeltaNet layer (qwen35_tree.py:329-480):
    in_proj GEMM [qkv | z | b | a] (row scale = input RMSNorm)   -> proj fp32
    prep: tree conv1d + SiLU, q/k RMS scaling, g, beta              -> q k v g beta
    tree recurrence from the committed state (node states in LDS)  -> y
    gated RMSNorm (y, z)                                           -> bf16 pair
    out_proj GEMM + residual (+ post-attention RMSNorm fold)
  gated attention layer (qwen35_tree.py:552-626):
    QKV GEMM (q_proj [q | gate] per head, k_proj, v_proj)          -> fp32
    tree attention (q/k norm, partial RoPE, cache append, mask, sigmoid gate)
    o_proj GEMM + residual (+ post-attention RMSNorm fold)
  MLP: gate/up GEMM + SwiGLU, down GEMM + residual (+ next RMSNorm fold)
  LM head + argmax, accept walk, KV compaction of the attention layers and
  the commit of every GatedDeltaNet layer along the accepted path.

The reference keeps a pending state and commits it in compact_kv_caches
(adapters.py:411-448); here the attention layers append the tree K/V at
[P, P + L) during the forward (compaction moves the accepted rows to
[P, P + n)), and the GatedDeltaNet layers keep their per-node inputs in
per-layer buffers that the commit replays along the accepted path.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _native as N
from .cache import Qwen35Cache
from .engine import TreeEngineBase
from .weights import W_TILED, W_TILED_F16, GdnLayerWeights


class Qwen35TreeEngine(TreeEngineBase):
    # The register-resident GatedDeltaNet recurrence holds trees of up to 96
    # nodes (head dim 128); larger ones fit no recurrence kernel.
    max_nodes_limit = 96

    def _alloc_layer_buffers(self) -> None:
        c, MP, dev = self.cfg, self.MP, self.dev
        f32, bf16 = torch.float32, torch.bfloat16
        nG = len(c.linear_layers)
        Hv = c.linear_num_value_heads
        # Per GatedDeltaNet layer: the projection and the prepped recurrence
        # inputs of every node, kept until the commit after the walk.
        self.proj = torch.zeros(nG, MP, c.in_proj_dim, dtype=f32, device=dev)
        self.gq = torch.zeros(nG, MP, c.key_dim, dtype=f32, device=dev)
        self.gk = torch.zeros(nG, MP, c.key_dim, dtype=f32, device=dev)
        self.gv = torch.zeros(nG, MP, c.value_dim, dtype=f32, device=dev)
        self.gg = torch.zeros(nG, MP, Hv, dtype=f32, device=dev)
        self.gbeta = torch.zeros(nG, MP, Hv, dtype=f32, device=dev)
        self.gy = torch.zeros(MP, c.value_dim, dtype=f32, device=dev)
        self.gout = torch.zeros(2, MP, c.value_dim, dtype=self.act_dtype, device=dev)
        self.qkv = torch.zeros(MP, c.attn_qkv_dim, dtype=f32, device=dev)
        self.attn = torch.zeros(2, MP, c.q_dim, dtype=self.act_dtype, device=dev)
        self.act = torch.zeros(2, MP, c.intermediate_size, dtype=self.act_dtype, device=dev)
        self.rope_cos = torch.zeros(MP, c.rope_dims // 2, dtype=f32, device=dev)
        self.rope_sin = torch.zeros(MP, c.rope_dims // 2, dtype=f32, device=dev)
        aws = self.lib.dtree_attention_workspace_bytes(c.num_attention_heads, c.head_dim, self.max_past, self.MP)
        self.attn_ws = torch.zeros(aws, dtype=torch.uint8, device=dev)

    def _gemm_shapes(self):
        c = self.cfg
        H, F = c.hidden_size, c.intermediate_size
        return {"in": (c.in_proj_dim, H), "out": (H, c.value_dim), "qkv": (c.attn_qkv_dim, H),
                "o": (H, c.q_dim), "gu": (2 * F, H), "down": (H, F)}

    def set_step(self, tokens, positions, parents, past_length: int, stream=None, ancestors=None,
                 aux: bool = False, accepted=None) -> None:
        # Trees past 32 nodes run the depth-first recurrence, whose state stack
        # holds a bounded nesting of branching nodes: reject deeper ones here.
        if len(parents) > 32:
            arr = (C.c_int32 * len(parents))(*[int(p) for p in parents])
            N.check(self.lib.dtree_gdn_tree_check(arr, len(parents)), "GatedDeltaNet tree")
        super().set_step(tokens, positions, parents, past_length, stream=stream, ancestors=ancestors, aux=aux,
                         accepted=accepted)

    def new_cache(self, page_order=None) -> Qwen35Cache:
        return Qwen35Cache(self.cfg, self.max_past + self.max_nodes, device=self.dev, page_order=page_order)

    # ---- launches ----------------------------------------------------------------
    def gdn_args(self, li: int, cache: Qwen35Cache) -> N.GdnArgs:
        c = self.cfg
        gi = cache.slot[li]
        lw: GdnLayerWeights = self.w.layers[li]
        a = N.GdnArgs()
        a.desc = self.desc.data_ptr(); a.rows_padded = self.MP
        a.num_k_heads = c.linear_num_key_heads; a.num_v_heads = c.linear_num_value_heads
        a.head_k_dim = c.linear_key_head_dim; a.head_v_dim = c.linear_value_head_dim
        a.conv_keep = c.linear_conv_kernel_dim - 1
        a.proj = self.proj[gi].data_ptr(); a.ld_proj = c.in_proj_dim
        a.window = cache.windows[gi].data_ptr(); a.conv_w = lw.conv_w.data_ptr()
        a.A_log = lw.A_log.data_ptr(); a.dt_bias = lw.dt_bias.data_ptr()
        a.state = cache.states[gi].data_ptr()
        a.q = self.gq[gi].data_ptr(); a.k = self.gk[gi].data_ptr(); a.v = self.gv[gi].data_ptr()
        a.g = self.gg[gi].data_ptr(); a.beta = self.gbeta[gi].data_ptr()
        a.y = self.gy.data_ptr()
        a.norm_w = lw.gnorm.data_ptr(); a.eps = c.rms_norm_eps
        a.out = self.gout[0].data_ptr(); a.out_lo = self.lo_ptr(self.gout)
        a.out_layout = self.w.layout; a.ld_out = c.value_dim
        return a

    def _attention(self, li, cache: Qwen35Cache, st, write_cache=True):
        c = self.cfg
        ai = cache.slot[li]
        lw = self.w.layers[li]
        kv = cache.kv
        a = N.AttnArgs()
        a.qkv = self.qkv.data_ptr(); a.ld_qkv = self.qkv.shape[1]
        a.q_norm = lw.q_norm.data_ptr(); a.k_norm = lw.k_norm.data_ptr(); a.eps = c.rms_norm_eps
        a.rope_cos = self.rope_cos.data_ptr(); a.rope_sin = self.rope_sin.data_ptr()
        a.k_pages = kv.k_ptr(ai); a.v_pages = kv.v_ptr(ai); a.page_table = kv.page_table.data_ptr()
        a.desc = self.desc.data_ptr()
        a.out = self.attn[0].data_ptr(); a.out_lo = self.lo_ptr(self.attn); a.ld_out = self.attn.shape[-1]
        a.out_layout = self.w.layout
        a.num_heads = c.num_attention_heads; a.num_kv_heads = c.num_key_value_heads; a.head_dim = c.head_dim
        a.rows_padded = self.MP; a.scale = c.head_dim ** -0.5
        a.max_past_length = self.attn_grid_past(self._step_past); a.write_cache = 1 if write_cache else 0
        a.workspace = self.attn_ws.data_ptr(); a.workspace_bytes = self.attn_ws.numel()
        a.rope_dims = c.rope_dims; a.gated = 1
        N.check(self.lib.dtree_tree_attention(C.byref(a), st), "tree attention")

    def launch_forward(self, cache: Qwen35Cache, st: int, norm_hidden: bool = False) -> None:
        """embed + all layers; attention-layer tree K/V land in the cache at
        [P, P + L); GatedDeltaNet per-node inputs stay in the layer buffers."""
        c = self.cfg
        H = c.hidden_size
        if cache.capacity < self.max_past + self.max_nodes:
            raise ValueError("cache capacity is smaller than max_past + max_nodes")
        emb, emb_layout, emb_sb = self._embedding()
        N.check(self.lib.dtree_embed(
            self.desc.data_ptr(), emb, emb_layout, emb_sb, c.vocab_size, H,
            self.w.layers[0].input_norm.data_ptr(), self.MP,
            self.x.data_ptr(), self.xg[0].data_ptr(), self.lo_ptr(self.xg), self.w.layout, self.ss.data_ptr(),
            c.rope_dims, c.rope_theta, self.rope_cos.data_ptr(), self.rope_sin.data_ptr(), st), "embed")
        slot = {li: i for i, li in enumerate(self.layer_ids)}
        nL = c.num_hidden_layers
        for li in range(nL):
            lw = self.w.layers[li]
            nxt = self.w.layers[li + 1].input_norm if li + 1 < nL else self.w.final_norm
            if c.is_linear(li):
                gi = cache.slot[li]
                self._gemm("in", self.xg, H, lw.w_in, N.EPI_STORE_F32, st, ss_in=self.ss, out_f32=self.proj[gi])
                ga = self.gdn_args(li, cache)
                # one launch for trees of up to 32 nodes, else prep + recurrence
                N.check(self.lib.dtree_gdn_layer_prep_recurrence(C.byref(ga), st), "gdn prep + recurrence")
                N.check(self.lib.dtree_gdn_layer_gated_norm(C.byref(ga), st), "gdn gated norm")
                self._gemm("out", self.gout, c.value_dim, lw.w_out, N.EPI_RESIDUAL, st, out_f32=self.x,
                           out_bf16=self.xg, next_norm=lw.post_norm, ss_out=self.ss)
            else:
                self._gemm("qkv", self.xg, H, lw.wqkv, N.EPI_STORE_F32, st, ss_in=self.ss, out_f32=self.qkv)
                self._attention(li, cache, st)
                self._gemm("o", self.attn, c.q_dim, lw.wo, N.EPI_RESIDUAL, st, out_f32=self.x, out_bf16=self.xg,
                           next_norm=lw.post_norm, ss_out=self.ss)
            self._gemm("gu", self.xg, H, lw.wgu, N.EPI_SWIGLU, st, ss_in=self.ss, out_bf16=self.act)
            hid, ldh = 0, 0
            if li in slot:
                hid = self.hidden.data_ptr() + 2 * slot[li] * H
                ldh = self.hidden.shape[1]
            self._gemm("down", self.act, c.intermediate_size, lw.wd, N.EPI_RESIDUAL, st, out_f32=self.x,
                       out_bf16=self.xg, next_norm=nxt, ss_out=self.ss, hidden_out=hid, ld_hidden=ldh)
        if norm_hidden:
            N.check(self.lib.dtree_rownorm(self.x.data_ptr(), H, self.MP, H, self.ss.data_ptr(), H // 32,
                                           self.w.final_norm.data_ptr(), c.rms_norm_eps,
                                           self.norm_hidden.data_ptr(), H, st), "rownorm")
        self.launch_attention_status(self.attn_ws, st)

    def launch_compact(self, cache: Qwen35Cache, st: int, select_hidden: bool = True, aux: bool = False) -> None:
        """commit_qwen35_tree_path: KV compaction of the attention layers (+ the
        hidden-state select), then every GatedDeltaNet layer's window / state
        replayed along desc.accepted."""
        c = self.cfg
        d = self.desc_aux if aux else self.desc
        kv = cache.kv
        N.check(self.lib.dtree_compact(
            d.data_ptr(), kv.k_pages.data_ptr(), kv.v_pages.data_ptr(), kv.layer_stride, kv.layers,
            c.num_key_value_heads, c.head_dim, kv.page_table.data_ptr(),
            self.hidden.data_ptr() if select_hidden else None, self.hidden.shape[1],
            self.hidden_sel.data_ptr() if select_hidden else None, st), "compact")
        self._commit_gdn(cache, st, d)

    def _commit_gdn(self, cache: Qwen35Cache, st: int, desc: torch.Tensor) -> None:
        """Every GatedDeltaNet layer's commit in one launch
        (dtree_gdn_layers_commit), from the committed windows / states into
        the cache's spare pair; cache.flip() keeps it."""
        layers = list(cache.gdn_layers)
        if not layers:
            return
        arr = (N.GdnArgs * len(layers))()
        for i, li in enumerate(layers):
            arr[i] = self.gdn_args(li, cache)
            arr[i].desc = desc.data_ptr()
            gi = cache.slot[li]
            arr[i].window_out = cache.windows_next[gi].data_ptr()
            arr[i].state_out = cache.states_next[gi].data_ptr()
        N.check(self.lib.dtree_gdn_layers_commit(arr, len(layers), st), "gdn commit")

    def _graph_key(self, cache: Qwen35Cache):
        # The graph reads the committed pair and writes the spare one, so each
        # buffer parity has its own graph (and each attention grid size).
        return (id(cache), cache.parity, self.attn_grid_past(self._step_past))

    def _keep_commit(self, cache: Qwen35Cache, past_length: int, n_accepted: int) -> None:
        cache.offset = past_length + n_accepted
        cache.flip()

    def commit_chain(self, cache: Qwen35Cache, tokens, norm_hidden: bool = False) -> None:
        """Forward a causal chain of <= max_nodes tokens and commit all of it:
        the attention K/V rows stay where the forward wrote them, every
        GatedDeltaNet window / state advances along the whole chain."""
        n = len(tokens)
        P = cache.offset
        if not 1 <= n <= self.max_nodes:
            raise ValueError(f"a chain holds 1..{self.max_nodes} tokens, got {n}")
        if P + n > self.max_past:
            raise ValueError("chain beyond max_past")
        st = self.stream_handle()
        self.set_step(tokens, [P + i for i in range(n)], [-1] + list(range(n - 1)), P, accepted=list(range(n)))
        self.launch_forward(cache, st, norm_hidden=norm_hidden)
        self._commit_gdn(cache, st, self.desc)
        self._keep_commit(cache, P, n)

    def prefill(self, cache: Qwen35Cache, tokens, chunk: int | None = None) -> None:
        """Causal prefill through the tree path: fully accepted chains of up to
        max_nodes tokens."""
        chunk = chunk or self.max_nodes
        toks = [int(t) for t in tokens]
        for s in range(0, len(toks), chunk):
            self.commit_chain(cache, toks[s:s + chunk])

    # ---- prompt prefill on the long-M GEMM (forward_dflash,
    # custom_qwen35_model.py:961-1097, via adapters.py:290-307) ---------------------
    def supports_long_prefill(self) -> bool:
        return self.w.layout in (W_TILED, W_TILED_F16)  # bf16 or q4 group-64 weights

    def _prefill_buffers(self, rows: int) -> dict:
        pf = getattr(self, "_pf", None)
        if pf is not None and pf["rows"] >= rows and pf["nh"] == max(1, len(self.layer_ids)):
            return pf
        self._pf = None  # release the smaller set first
        c, dev = self.cfg, self.dev
        H, F = c.hidden_size, c.intermediate_size
        Hv = c.linear_num_value_heads
        f32, bf16 = torch.float32, torch.bfloat16
        nh = max(1, len(self.layer_ids))
        pf = dict(rows=rows, nh=nh,
                  tokens=torch.zeros(rows, dtype=torch.int32, device=dev),
                  x=torch.zeros(rows, H, dtype=f32, device=dev),
                  xg=torch.zeros(2, rows, H, dtype=self.act_dtype, device=dev),
                  ss=torch.zeros(rows // 32, H // 32, 32, dtype=f32, device=dev),
                  proj=torch.zeros(rows, c.in_proj_dim, dtype=f32, device=dev),
                  q=torch.zeros(rows, c.key_dim, dtype=f32, device=dev),
                  k=torch.zeros(rows, c.key_dim, dtype=f32, device=dev),
                  v=torch.zeros(rows, c.value_dim, dtype=f32, device=dev),
                  g=torch.zeros(rows, Hv, dtype=f32, device=dev),
                  beta=torch.zeros(rows, Hv, dtype=f32, device=dev),
                  y=torch.zeros(rows, c.value_dim, dtype=f32, device=dev),
                  gout=torch.zeros(2, rows, c.value_dim, dtype=self.act_dtype, device=dev),
                  qkv=torch.zeros(rows, c.attn_qkv_dim, dtype=f32, device=dev),
                  attn=torch.zeros(2, rows, c.q_dim, dtype=self.act_dtype, device=dev),
                  act=torch.zeros(2, rows, F, dtype=self.act_dtype, device=dev),
                  hidden=torch.zeros(rows, nh * H, dtype=bf16, device=dev),
                  cos=torch.zeros(rows, c.rope_dims // 2, dtype=f32, device=dev),
                  sin=torch.zeros(rows, c.rope_dims // 2, dtype=f32, device=dev),
                  descs=torch.zeros(rows // 128, C.sizeof(N.StepDesc), dtype=torch.uint8, device=dev),
                  attn_ws=torch.zeros(self.lib.dtree_attention_workspace_bytes(c.num_attention_heads, c.head_dim,
                                                                               self.max_past, 128),
                                      dtype=torch.uint8, device=dev))
        self._pf = pf
        return pf

    def _chain_gdn_args(self, li: int, cache: Qwen35Cache, pf: dict, rows: int) -> N.GdnArgs:
        c = self.cfg
        gi = cache.slot[li]
        lw: GdnLayerWeights = self.w.layers[li]
        a = N.GdnArgs()
        a.desc = None; a.rows_padded = rows
        a.num_k_heads = c.linear_num_key_heads; a.num_v_heads = c.linear_num_value_heads
        a.head_k_dim = c.linear_key_head_dim; a.head_v_dim = c.linear_value_head_dim
        a.conv_keep = c.linear_conv_kernel_dim - 1
        a.proj = pf["proj"].data_ptr(); a.ld_proj = c.in_proj_dim
        a.window = cache.windows[gi].data_ptr(); a.conv_w = lw.conv_w.data_ptr()
        a.A_log = lw.A_log.data_ptr(); a.dt_bias = lw.dt_bias.data_ptr()
        a.state = cache.states[gi].data_ptr()
        a.q = pf["q"].data_ptr(); a.k = pf["k"].data_ptr(); a.v = pf["v"].data_ptr()
        a.g = pf["g"].data_ptr(); a.beta = pf["beta"].data_ptr(); a.y = pf["y"].data_ptr()
        a.norm_w = lw.gnorm.data_ptr(); a.eps = c.rms_norm_eps
        a.out = pf["gout"][0].data_ptr(); a.out_lo = self.lo_ptr(pf["gout"])
        a.out_layout = self.w.layout; a.ld_out = c.value_dim
        return a

    def prefill_long(self, cache: Qwen35Cache, tokens, want_logits: bool = True):
        """Causal forward over the prompt with the long-M GEMM, committing as it
        goes (forward_dflash over the prompt): per segment of up to
        PREFILL_SEGMENT tokens, embed, then per GatedDeltaNet layer the in_proj
        GEMM, the chain prep + recurrence + gated norm (dtree_gdn_layer_chain:
        the committed window and state advance over the segment) and out_proj;
        per attention layer the fused QKV GEMM, gated attention per 128-row
        chunk (appending its K/V rows) and o_proj; then the MLP. Returns the
        fp32 logits of the last position ([1, 1, V]) if asked and the verifier
        hidden rows of every position ([n, n_ids * H] bf16 or None)."""
        if not self.supports_long_prefill():
            raise NotImplementedError("the long-M prefill runs tiled weights")
        c = self.cfg
        H, D = c.hidden_size, c.head_dim
        toks = [int(t) for t in tokens]
        if not toks:
            raise ValueError("empty prompt")
        if any(t < 0 or t >= c.vocab_size for t in toks):
            raise ValueError("token id outside the vocabulary")
        if cache.offset + len(toks) > self.max_past:
            raise ValueError(f"prefill of {len(toks)} tokens beyond max_past {self.max_past}")
        st = self.stream_handle()
        emb, emb_layout, emb_sb = self._embedding()
        slot = {li: i for i, li in enumerate(self.layer_ids)}
        hid_parts = []
        seg = self.PREFILL_SEGMENT
        kv = cache.kv
        for s0 in range(0, len(toks), seg):
            part = toks[s0:s0 + seg]
            n = len(part)
            rows = 128 * ((n + 127) // 128)
            pf = self._prefill_buffers(max(rows, seg if len(toks) > seg else rows))
            P0 = cache.offset
            pf["tokens"][:n].copy_(torch.tensor(part, dtype=torch.int32))
            nch = rows // 128
            N.check(self.lib.dtree_embed_tokens(
                pf["tokens"].data_ptr(), n, emb, emb_layout, emb_sb, c.vocab_size, H,
                self.w.layers[0].input_norm.data_ptr(), rows, pf["x"].data_ptr(), pf["xg"][0].data_ptr(),
                self.lo_ptr(pf["xg"]), self.w.layout, pf["ss"].data_ptr(), st), "embed tokens")
            dstride = self._prefill_chunks(pf, P0, n, rows, c.rope_dims, st)
            nL = c.num_hidden_layers
            for li in range(nL):
                lw = self.w.layers[li]
                nxt = self.w.layers[li + 1].input_norm if li + 1 < nL else self.w.final_norm
                if c.is_linear(li):
                    self._long_gemm("in", pf["xg"], H, lw.w_in, N.EPI_STORE_F32, rows, st, ss_in=pf["ss"],
                                    out_f32=pf["proj"])
                    ga = self._chain_gdn_args(li, cache, pf, rows)
                    N.check(self.lib.dtree_gdn_layer_chain(C.byref(ga), n, st), "gdn chain")
                    self._long_gemm("out", pf["gout"], c.value_dim, lw.w_out, N.EPI_RESIDUAL, rows, st,
                                    out_f32=pf["x"], out_bf16=pf["xg"], next_norm=lw.post_norm, ss_out=pf["ss"])
                else:
                    ai = cache.slot[li]
                    self._long_gemm("qkv", pf["xg"], H, lw.wqkv, N.EPI_STORE_F32, rows, st, ss_in=pf["ss"],
                                    out_f32=pf["qkv"])
                    for ch in range(nch):
                        a = N.AttnArgs()
                        a.qkv = pf["qkv"][128 * ch].data_ptr(); a.ld_qkv = c.attn_qkv_dim
                        a.q_norm = lw.q_norm.data_ptr(); a.k_norm = lw.k_norm.data_ptr(); a.eps = c.rms_norm_eps
                        a.rope_cos = pf["cos"][128 * ch].data_ptr(); a.rope_sin = pf["sin"][128 * ch].data_ptr()
                        a.k_pages = kv.k_ptr(ai); a.v_pages = kv.v_ptr(ai); a.page_table = kv.page_table.data_ptr()
                        a.desc = pf["descs"].data_ptr() + ch * dstride
                        a.out = pf["attn"][0, 128 * ch].data_ptr()
                        a.out_lo = self.lo_ptr(pf["attn"], 2 * 128 * ch * c.q_dim)
                        a.ld_out = c.q_dim; a.out_layout = self.w.layout
                        a.num_heads = c.num_attention_heads; a.num_kv_heads = c.num_key_value_heads
                        a.head_dim = D; a.rows_padded = 128; a.scale = D ** -0.5
                        a.max_past_length = self.attn_grid_past(P0 + 128 * ch); a.write_cache = 1
                        a.workspace = pf["attn_ws"].data_ptr(); a.workspace_bytes = pf["attn_ws"].numel()
                        a.rope_dims = c.rope_dims; a.gated = 1
                        N.check(self.lib.dtree_tree_attention(C.byref(a), st), "prefill attention")
                    self._long_gemm("o", pf["attn"], c.q_dim, lw.wo, N.EPI_RESIDUAL, rows, st, out_f32=pf["x"],
                                    out_bf16=pf["xg"], next_norm=lw.post_norm, ss_out=pf["ss"])
                self._long_gemm("gu", pf["xg"], H, lw.wgu, N.EPI_SWIGLU, rows, st, ss_in=pf["ss"],
                                out_bf16=pf["act"])
                hid, ldh = 0, 0
                if li in slot:
                    hid = pf["hidden"].data_ptr() + 2 * slot[li] * H
                    ldh = pf["hidden"].shape[1]
                self._long_gemm("down", pf["act"], c.intermediate_size, lw.wd, N.EPI_RESIDUAL, rows, st,
                                out_f32=pf["x"], out_bf16=pf["xg"], next_norm=nxt, ss_out=pf["ss"],
                                hidden_out=hid, ld_hidden=ldh)
            cache.offset = P0 + n
            if self.layer_ids:
                hid_parts.append(pf["hidden"][:n].clone())
        self.launch_attention_status(pf["attn_ws"], st)
        logits = self._prefill_logits(pf, n, st) if want_logits else None
        hidden = torch.cat(hid_parts, 0) if hid_parts else None
        return logits, hidden
