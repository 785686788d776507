"""Qwen3 tree-verify executor: launches the HIP kernels of one verify step.

One step (dtree_runtime.py:410-537 for the Qwen3 target):
  embed(+input RMSNorm fold, RoPE table)
  for every layer:
    QKV GEMM (row scale = input RMSNorm)      -> qkv fp32
    tree attention (q/k norm, RoPE, cache append, ancestor mask) -> attn bf16
    O GEMM + residual (+ post-attention RMSNorm fold)
    gate/up GEMM + SwiGLU (row scale = post-attention RMSNorm) -> act bf16
    down GEMM + residual (+ next RMSNorm fold, optional hidden capture)
  LM head + argmax candidates, argmax reduction + accept walk, KV/hidden compaction.

The launch sequence only depends on device-resident step data (P, L, tree),
so it can be captured once into a HIP graph and replayed for every step.
"""
from __future__ import annotations

import ctypes as C
import weakref
from dataclasses import dataclass

import numpy as np
import torch

from . import _native as N
from .cache import PagedKVCache
from .config import Qwen3Config
from .weights import W_TILED, W_TILED_F16, Q4Linear, Qwen3Weights, tile_weight, tile_weight_f16


_HIP = None


def _hip():
    """The HIP runtime (already loaded by torch) for the per-step descriptor and
    result copies: one call each instead of a tensor copy through the
    dispatcher, on the step's critical path between two verify steps."""
    global _HIP
    if _HIP is None:
        h = None
        for name in ("libamdhip64.so", "libamdhip64.so.7", "libamdhip64.so.6"):
            try:
                h = C.CDLL(name)
                break
            except OSError:
                continue
        if h is None:
            raise RuntimeError("the HIP runtime (libamdhip64.so) is not loadable")
        h.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
        h.hipMemcpyAsync.restype = C.c_int
        h.hipStreamSynchronize.argtypes = [C.c_void_p]
        h.hipStreamSynchronize.restype = C.c_int
        _HIP = h
    return _HIP


_H2D, _D2H = 1, 2  # hipMemcpyHostToDevice, hipMemcpyDeviceToHost


def _hip_check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: HIP error {rc}")


def ancestor_bitsets(parents) -> np.ndarray:
    """[L, MASK_WORDS] uint32 ancestor-or-self bitsets (parents[i] < i, root -1)."""
    L = len(parents)
    if L > N.MAX_NODES:
        raise ValueError(f"at most {N.MAX_NODES} tree nodes are supported, got {L}")
    masks = [0] * L  # one Python integer per node: cheaper than L numpy row copies
    for i in range(L):
        p = int(parents[i])
        if i == 0:
            if p != -1:
                raise ValueError(f"tree root parent must be -1, got {p}")
            masks[0] = 1
        elif p < 0 or p >= i:
            raise ValueError(f"tree parent index must precede child, got parents[{i}]={p}")
        else:
            masks[i] = masks[p] | (1 << i)
    raw = b"".join(m.to_bytes(4 * N.MASK_WORDS, "little") for m in masks)
    return np.frombuffer(raw, dtype="<u4").reshape(L, N.MASK_WORDS).copy()


def mask_to_parents(tree_mask: np.ndarray) -> list[int]:
    """Parents from an ancestor-or-self visibility matrix [L, L] (rows topological)."""
    L = tree_mask.shape[0]
    parents = [-1]
    for i in range(1, L):
        anc = [j for j in range(i) if tree_mask[i, j]]
        if not tree_mask[i, i]:
            raise ValueError("tree visibility must include the diagonal")
        if not anc:
            raise ValueError(f"node {i} sees no ancestor; the root must be visible to every node")
        p = max(anc)
        expect = tree_mask[p, :i].copy()
        expect[p] = True
        if not np.array_equal(expect, tree_mask[i, :i]):
            raise ValueError("tree visibility rows must be ancestor-or-self sets (parent row + self)")
        parents.append(p)
    return parents


@dataclass
class StepResult:
    accepted: list[int]
    bonus_token: int
    posterior: list[int]


class TreeEngineBase:
    """Buffers and launches shared by the Qwen3 and Qwen3.5 verify steps: the
    device step descriptor, GEMM arguments, the LM head + argmax, the accept
    walk, result readback and the HIP graph of the whole step. Subclasses
    provide the layer stack (launch_forward), the cache and its compaction."""

    max_nodes_limit = N.MAX_NODES
    # GEMMs that read only the high bf16 plane of their split-pair input. The
    # fused QKV projection: q and k pass through their RMSNorm and attention
    # averages over keys, so its input rounded to bf16 moves the full
    # Qwen3-4B step's logits from 0.09 % to 0.12 % of the row maximum (every
    # other class costs ~1 %: gate/up 1.45 %, down 0.98 %, o_proj 1.05 %, the
    # hybrid's in_proj 1.25 %), and the projection, bound by what each CU
    # loads, reads a third fewer bytes.
    HI_ONLY = frozenset({"qkv"})

    def __init__(self, cfg, weights, max_past: int, max_nodes: int = 32, layer_ids=(), split_k: dict | None = None):
        cfg.validate()
        if not 1 <= max_nodes <= self.max_nodes_limit:
            raise NotImplementedError(f"trees of 1 .. {self.max_nodes_limit} nodes per verify step")
        self.cfg = cfg
        self.w = weights
        self.lib = N.lib()
        self.dev = weights.device
        self.max_past = int(max_past)
        self.max_nodes = max_nodes
        # Tree rows padded to whole 32-row MFMA blocks (32, 64, 96 or 128).
        self.MP = 32 * ((max_nodes + 31) // 32)
        self.layer_ids = list(layer_ids)
        H, V = cfg.hidden_size, cfg.vocab_size
        MP, dev = self.MP, self.dev
        f32, bf16 = torch.float32, torch.bfloat16
        # GEMM inputs: with DTREE_W_TILED_F16 weights one fp16 plane (plane 0
        # of the plane buffers; plane 1 stays unused), else split pairs
        # [hi, lo] of bf16 planes (value = hi + lo).
        self.h16 = weights.layout == W_TILED_F16
        self.act_dtype = torch.float16 if self.h16 else bf16
        # q4 group-64 models run on the high bf16 plane alone (bf16
        # activations, as the reference's quantised matmuls take them): half
        # the activation bytes and MFMA passes of the split pair.
        self.hi_only = self.h16 or getattr(weights, "quant", "bf16") == "q4"
        self.x = torch.zeros(MP, H, dtype=f32, device=dev)
        self.xg = torch.zeros(2, MP, H, dtype=self.act_dtype, device=dev)
        # RMSNorm statistics: per 32-row block, per 32-column tile, per row
        self.ss = torch.zeros(MP // 32, H // 32, 32, dtype=f32, device=dev)
        self.norm_hidden = torch.zeros(MP, H, dtype=bf16, device=dev)
        nh = max(1, len(self.layer_ids))
        self.hidden = torch.zeros(MP, nh * H, dtype=bf16, device=dev)
        self.hidden_sel = torch.zeros(MP, nh * H, dtype=bf16, device=dev)
        self.logits = None
        self.split_k = dict(split_k or {})
        self._alloc_layer_buffers()
        shapes = self._gemm_shapes()
        ws = max(self.lib.dtree_gemm_workspace_bytes(MP, n, k, self.split_k.get(name, 0))
                 for name, (n, k) in shapes.items())
        self.gemm_ws = torch.zeros(ws, dtype=torch.uint8, device=dev)
        self.n_cand = self.lib.dtree_lmhead_candidate_blocks(V, MP)
        self.cand = torch.zeros(self.lib.dtree_lmhead_candidates_bytes(MP), dtype=torch.uint8, device=dev)
        self.desc_pinned = torch.zeros(C.sizeof(N.StepDesc), dtype=torch.uint8).pin_memory()
        self.desc = torch.zeros(C.sizeof(N.StepDesc), dtype=torch.uint8, device=dev)
        self.desc_aux_pinned = torch.zeros(C.sizeof(N.StepDesc), dtype=torch.uint8).pin_memory()
        # record views of the pinned descriptors: the host fills them in place
        self._desc_rec = self.desc_pinned.numpy().view(N.STEP_DESC_DTYPE)[0]
        self._desc_aux_rec = self.desc_aux_pinned.numpy().view(N.STEP_DESC_DTYPE)[0]
        for rec in (self._desc_rec, self._desc_aux_rec):
            rec["parents"][:] = -1
        self.desc_aux = torch.zeros(C.sizeof(N.StepDesc), dtype=torch.uint8, device=dev)
        self._desc_event = torch.cuda.Event()
        self._aux_event = torch.cuda.Event()
        self._desc_event.record()
        self._aux_event.record()
        self.lm_in = torch.zeros(self.MP, H, dtype=bf16, device=dev)
        # walk result [n, bonus, L, accepted[MAX], posterior[MAX]] + the attention
        # status word (dtree_attention_status), read back together
        self.result = torch.zeros(4 + 2 * N.MAX_NODES, dtype=torch.int32, device=dev)
        self.result_host = torch.zeros(4 + 2 * N.MAX_NODES, dtype=torch.int32).pin_memory()
        self._result_np = self.result_host.numpy()
        self._step_past = 0  # P of the step the descriptor holds (host copy)
        self._graphs: dict = {}
        self._dead_graphs: list = []
        self._tree_ws = None
        self.tree_out = torch.zeros(1 + 3 * N.MAX_NODES, dtype=torch.int32, device=dev)
        self.tree_out_host = torch.zeros(1 + 3 * N.MAX_NODES, dtype=torch.int32).pin_memory()

    def _alloc_layer_buffers(self) -> None:
        raise NotImplementedError

    def _gemm_shapes(self) -> dict:
        raise NotImplementedError

    def new_cache(self, page_order=None):
        raise NotImplementedError

    def launch_forward(self, cache, st: int, norm_hidden: bool = False) -> None:
        raise NotImplementedError

    def launch_compact(self, cache, st: int, select_hidden: bool = True, aux: bool = False) -> None:
        raise NotImplementedError

    @staticmethod
    def stream_handle(stream=None) -> int:
        s = torch.cuda.current_stream() if stream is None else stream
        return s.cuda_stream

    # ---- step descriptor -------------------------------------------------------
    def set_step(self, tokens, positions, parents, past_length: int, stream=None, ancestors=None,
                 aux: bool = False, accepted=None) -> None:
        """Fill the device step descriptor (``aux`` selects the second one used by
        stand-alone argmax / compaction calls, so the step's own stays intact)."""
        L = len(tokens)
        if not 1 <= L <= self.max_nodes:
            raise ValueError(f"tree must have 1..{self.max_nodes} nodes, got {L}")
        if len(positions) != L or len(parents) != L:
            raise ValueError("tokens, positions and parents must have the same length")
        if past_length < 0 or past_length > self.max_past:
            raise ValueError(f"past_length {past_length} outside [0, {self.max_past}]")
        anc = ancestor_bitsets(parents) if ancestors is None else np.asarray(ancestors, dtype=np.uint32)
        toks = np.asarray(tokens, dtype=np.int64).reshape(L)
        bad = np.nonzero((toks < 0) | (toks >= self.cfg.vocab_size))[0]
        if bad.size:
            raise ValueError(f"token id {int(toks[bad[0]])} outside the vocabulary")
        pinned, dst, ev, rec = ((self.desc_aux_pinned, self.desc_aux, self._aux_event, self._desc_aux_rec) if aux
                                else (self.desc_pinned, self.desc, self._desc_event, self._desc_rec))
        ev.synchronize()  # the previous upload from this pinned buffer has finished
        if not aux:
            self._step_past = int(past_length)
        rec["past_length"] = int(past_length)
        rec["num_nodes"] = L
        rec["n_accepted"] = 0 if accepted is None else len(accepted)
        rec["bonus_token"] = -1
        if accepted is not None and len(accepted):
            rec["accepted"][: len(accepted)] = np.asarray(accepted, dtype=np.int64)
        rec["tokens"][:L] = toks
        rec["tokens"][L:] = 0
        rec["positions"][:L] = np.asarray(positions, dtype=np.int64)
        rec["positions"][L:] = 0
        rec["parents"][:L] = np.asarray(parents, dtype=np.int64)
        rec["parents"][L:] = -1
        rec["ancestors"][:L] = anc
        rec["ancestors"][L:] = 0
        s = torch.cuda.current_stream() if stream is None else stream
        _hip_check(_hip().hipMemcpyAsync(dst.data_ptr(), pinned.data_ptr(), pinned.numel(), _H2D, s.cuda_stream),
                   "step descriptor upload")
        ev.record(s)

    # ---- launches ----------------------------------------------------------------
    def gemm_args(self, name, x, ldx, w, epi, *, ss_in=None, out_f32=None, out_bf16=None, next_norm=None,
                  ss_out=None, hidden_out=0, ld_hidden=0) -> N.GemmArgs:
        n, k = w.shape
        a = N.GemmArgs()
        if x.dim() == 3:  # plane buffers: [fp16] (tiled) or split pair [hi, lo]
            a.x = x[0].data_ptr(); a.x_lo = None if name in self.HI_ONLY else self.lo_ptr(x)
        else:
            a.x = x.data_ptr()
        a.ldx = ldx; a.rows_padded = self.MP
        # Internal activations share the weights' layout (tiled: contiguous
        # kilobyte loads for both GEMM operands).
        if isinstance(w, Q4Linear):  # q4 group-64 weights (w_scales = scale/bias pairs)
            a.w = w.words.data_ptr(); a.w_scales = w.sb.data_ptr(); a.w_layout = N.W_Q4G64
        else:
            a.w = w.data_ptr(); a.w_layout = self.w.layout
        a.x_layout = self.w.layout; a.n = n; a.k = k
        a.epilogue = epi; a.split_k = self.split_k.get(name, 0)
        a.ss_in = ss_in.data_ptr() if ss_in is not None else None
        a.ss_tiles = self.cfg.hidden_size // 32 if ss_in is not None else 0
        a.norm_dim = self.cfg.hidden_size; a.eps = self.cfg.rms_norm_eps
        if out_f32 is not None:
            a.out_f32 = out_f32.data_ptr(); a.ld_out_f32 = out_f32.shape[1]
        if out_bf16 is not None:
            if out_bf16.dim() == 3:
                a.out_bf16 = out_bf16[0].data_ptr(); a.out_lo = self.lo_ptr(out_bf16)
            else:
                a.out_bf16 = out_bf16.data_ptr()
            a.ld_out_bf16 = out_bf16.shape[-1]
            a.out_layout = self.w.layout
        a.next_norm = next_norm.data_ptr() if next_norm is not None else None
        a.ss_out = ss_out.data_ptr() if ss_out is not None else None
        a.hidden_out = hidden_out or None; a.ld_hidden = ld_hidden
        a.workspace = self.gemm_ws.data_ptr(); a.workspace_bytes = self.gemm_ws.numel()
        return a

    def lo_ptr(self, t: torch.Tensor, offset_bytes: int = 0):
        """Low plane of a plane buffer: none on the fp16 path (one plane) and
        for q4 models (the high bf16 plane alone)."""
        return None if self.hi_only else t[1].data_ptr() + offset_bytes

    def _embedding(self):
        """(pointer, layout, scale/bias pointer) of the tied embedding."""
        e = self.w.embed
        if isinstance(e, Q4Linear):
            return e.words.data_ptr(), N.W_Q4G64, e.sb.data_ptr()
        return e.data_ptr(), self.w.layout, None

    def _gemm(self, name, x, ldx, w, epi, st, **kw):
        a = self.gemm_args(name, x, ldx, w, epi, **kw)
        N.check(self.lib.dtree_gemm_bf16(C.byref(a), st), f"gemm {name}")

    # ---- prompt prefill on the long-M GEMM: pieces shared by both models -------
    PREFILL_SEGMENT = 1024  # prompt rows per pass through the layer stack (a multiple of 128)

    def _long_gemm(self, name, x, k, w, epi, rows, st, **kw):
        a = self.gemm_args(name, x, k, w, epi, **kw)
        a.rows_padded = rows
        N.check(self.lib.dtree_gemm_long(C.byref(a), st), f"long gemm {name}")

    def _prefill_chunks(self, pf: dict, P0: int, n: int, rows: int, rope_dims: int, st: int) -> int:
        """Step descriptors of a segment's 128-row causal chunks (chain trees
        over the cached prefix: chunk ch holds positions P0 + 128 ch ..) and
        their RoPE tables over rope_dims dims; returns the descriptor stride."""
        nch = rows // 128
        recs = np.zeros(nch, dtype=N.STEP_DESC_DTYPE)
        for ch in range(nch):
            L = min(128, n - 128 * ch)
            r = recs[ch]
            r["past_length"] = P0 + 128 * ch
            r["num_nodes"] = L
            r["bonus_token"] = -1
            r["positions"][:L] = np.arange(P0 + 128 * ch, P0 + 128 * ch + L)
            r["parents"][:] = -1
            r["parents"][1:L] = np.arange(L - 1)
            r["ancestors"][:L] = ancestor_bitsets([-1] + list(range(L - 1)))
        pf["descs"][:nch].copy_(torch.from_numpy(recs.view(np.uint8).reshape(nch, -1)))
        dstride = pf["descs"].shape[1]
        for ch in range(nch):
            N.check(self.lib.dtree_rope_table(pf["descs"].data_ptr() + ch * dstride, 128, rope_dims,
                                              self.cfg.rope_theta, pf["cos"][128 * ch].data_ptr(),
                                              pf["sin"][128 * ch].data_ptr(), st), "rope table")
        return dstride

    def _prefill_logits(self, pf: dict, n: int, st: int) -> torch.Tensor:
        """fp32 logits [1, 1, V] of a segment's last row (its xg / ss rows hold
        the final RMSNorm's input)."""
        c = self.cfg
        H = c.hidden_size
        emb, emb_layout, emb_sb = self._embedding()
        b, r = (n - 1) // 32, (n - 1) % 32
        if self.logits is None:
            self.logits = torch.zeros(self.MP, c.vocab_size, dtype=torch.float32, device=self.dev)
        xo = b * 32 * H
        N.check(self.lib.dtree_lmhead_argmax(
            pf["xg"][0].data_ptr() + 2 * xo, self.lo_ptr(pf["xg"], 2 * xo), self.w.layout, H, 32, emb,
            emb_layout, emb_sb, c.vocab_size, H, pf["ss"][b].data_ptr(), H // 32, c.rms_norm_eps,
            self.logits.data_ptr(), self.cand.data_ptr(), st), "prefill lm head")
        return self.logits[r:r + 1].clone()[None]

    def launch_lm_head(self, st: int, x=None, ss=True, want_logits=False) -> None:
        c = self.cfg
        logits_ptr = None
        if want_logits:
            if self.logits is None:
                self.logits = torch.zeros(self.MP, c.vocab_size, dtype=torch.float32, device=self.dev)
            logits_ptr = self.logits.data_ptr()
        if x is None:
            xin = self.xg
        elif self.w.layout in (W_TILED, W_TILED_F16):  # caller rows are row-major [MP, H]
            self._lm_tiled = tile_weight_f16(x) if self.h16 else tile_weight(x)
            xin = self._lm_tiled
        else:
            xin = x
        hi, lo = (xin[0].data_ptr(), self.lo_ptr(xin)) if xin.dim() == 3 else (xin.data_ptr(), None)
        emb, emb_layout, emb_sb = self._embedding()
        N.check(self.lib.dtree_lmhead_argmax(
            hi, lo, self.w.layout, xin.shape[-1], self.MP, emb, emb_layout, emb_sb, c.vocab_size, c.hidden_size,
            self.ss.data_ptr() if ss else None, c.hidden_size // 32 if ss else 0, c.rms_norm_eps,
            logits_ptr, self.cand.data_ptr(), st), "lm head")

    STATUS_SLOT = 3 + 2 * N.MAX_NODES

    def launch_attention_status(self, ws: torch.Tensor, st: int) -> None:
        """ORs the attention workspace's error word into the result's status
        slot (checked by read_result) and clears it."""
        N.check(self.lib.dtree_attention_status(ws.data_ptr(), self.result.data_ptr() + 4 * self.STATUS_SLOT, st),
                "attention status")

    def launch_walk(self, st: int, aux: bool = False) -> None:
        d = self.desc_aux if aux else self.desc
        N.check(self.lib.dtree_accept_walk(d.data_ptr(), self.cand.data_ptr(), self.n_cand, self.MP,
                                           self.result.data_ptr(), st), "accept walk")

    def launch_verify(self, cache: PagedKVCache, st: int) -> None:
        self.launch_forward(cache, st)
        self.launch_lm_head(st)
        self.launch_walk(st)
        self.launch_compact(cache, st)

    # ---- host-facing steps -----------------------------------------------------
    def set_layer_ids(self, layer_ids) -> None:
        ids = list(layer_ids)
        if ids == self.layer_ids:
            return
        H = self.cfg.hidden_size
        self.layer_ids = ids
        nh = max(1, len(ids))
        self.hidden = torch.zeros(self.MP, nh * H, dtype=torch.bfloat16, device=self.dev)
        self.hidden_sel = torch.zeros(self.MP, nh * H, dtype=torch.bfloat16, device=self.dev)
        self.release_graphs()

    # ---- draft tree on the device (dtree_runtime.py:82-192) ----------------------
    def launch_tree_build(self, draft_logits: torch.Tensor, budget: int, topk: int | None, root_token: int,
                          past_length: int, st: int) -> None:
        """build_dtree_tree + compile_dtree_tree into the step descriptor: the
        verify launches can follow on the stream without a host round trip."""
        x = draft_logits
        if x.dim() != 2 or x.dtype != torch.float32 or x.device != self.dev or not x.is_contiguous():
            x = x.reshape(-1, x.shape[-1]).to(self.dev, torch.float32).contiguous()
        D, V = x.shape
        budget = max(int(budget), 0)
        if 1 + budget > self.max_nodes:
            raise ValueError(f"tree budget {budget} needs {1 + budget} nodes; the engine holds {self.max_nodes}")
        if not 0 <= int(root_token) < self.cfg.vocab_size:
            raise ValueError(f"root token {root_token} outside the vocabulary")
        if past_length < 0 or past_length > self.max_past:
            raise ValueError(f"past_length {past_length} outside [0, {self.max_past}]")
        k = min(budget if topk is None else int(topk), V) if budget > 0 and D > 0 else 1
        ws_ptr, ws_bytes = None, 0
        if budget > 0 and D > 0:
            need = self.lib.dtree_tree_build_workspace_bytes(D, V, k)
            if self._tree_ws is None or self._tree_ws.numel() < need:
                self._tree_ws = torch.zeros(need, dtype=torch.uint8, device=self.dev)
            ws_ptr, ws_bytes = self._tree_ws.data_ptr(), self._tree_ws.numel()
        self._desc_event.synchronize()  # no host upload into the descriptor is still in flight
        self._step_past = int(past_length)
        N.check(self.lib.dtree_tree_build(x.data_ptr(), V, D, V, k, budget, int(root_token), int(past_length),
                                          ws_ptr, ws_bytes, self.desc.data_ptr(), self.tree_out.data_ptr(), None,
                                          None, st), "tree build")

    def tree_lists(self, root_token: int):
        """(node_token_ids, node_depths, parents, child_maps) of the last device
        tree, from the copy read_result(tree=True) fetched."""
        t = self.tree_out_host.numpy()
        n, M = int(t[0]), N.MAX_NODES
        ids = t[1:1 + n].tolist()
        depths = t[1 + M:1 + M + n].tolist()
        parents = [-1] + t[1 + 2 * M:1 + 2 * M + n].tolist()
        child_maps: list[dict[int, int]] = [dict() for _ in range(n + 1)]
        for i in range(1, n + 1):
            child_maps[parents[i]][ids[i - 1]] = i
        return ids, depths, parents, child_maps

    def verify_from_logits(self, cache, draft_logits, budget: int, topk: int | None, root_token: int,
                           use_graph: bool = True, commit: bool = True):
        """Tree build on the device, then the verify step, then one readback of
        the walk result and the tree. Returns (StepResult, tree lists)."""
        P = cache.offset
        st = self.stream_handle()
        self.launch_tree_build(draft_logits, budget, topk, root_token, P, st)
        if use_graph:
            self.graph_launch(cache, st)
        else:
            self.launch_verify(cache, st)
        res = self.read_result(tree=True)
        if commit:
            self._keep_commit(cache, P, len(res.accepted))
        return res, self.tree_lists(root_token)

    def _keep_commit(self, cache, past_length: int, n_accepted: int) -> None:
        """The host keeps a verify step's commit: the offset advances over the
        accepted rows that compaction moved to [P, P + n)."""
        cache.offset = past_length + n_accepted

    def read_result(self, stream=None, tree: bool = False) -> StepResult:
        s = torch.cuda.current_stream() if stream is None else stream
        h = _hip()
        _hip_check(h.hipMemcpyAsync(self.result_host.data_ptr(), self.result.data_ptr(),
                                    self.result_host.numel() * 4, _D2H, s.cuda_stream), "walk result copy")
        if tree:
            _hip_check(h.hipMemcpyAsync(self.tree_out_host.data_ptr(), self.tree_out.data_ptr(),
                                        self.tree_out_host.numel() * 4, _D2H, s.cuda_stream), "tree copy")
        _hip_check(h.hipStreamSynchronize(s.cuda_stream), "walk result wait")
        r = self._result_np
        if r[self.STATUS_SLOT]:
            self.result[self.STATUS_SLOT:].zero_()
            raise N.DtreeError("tree attention: a split's bounded wait gave up (DTREE_E_ATTN_WAIT); this step's "
                               "attention output is incomplete and must be recomputed")
        n, bonus, L = int(r[0]), int(r[1]), int(r[2])
        return StepResult(accepted=r[3:3 + n].tolist(), bonus_token=bonus,
                          posterior=r[3 + N.MAX_NODES:3 + N.MAX_NODES + L].tolist())

    def verify(self, cache: PagedKVCache, tokens, positions, parents, use_graph: bool = True,
               commit: bool = True) -> StepResult:
        """Full verify step on the current stream; returns the walk result and
        (commit=True) advances cache.offset by the accepted count."""
        P = cache.offset
        self.set_step(tokens, positions, parents, P)
        st = self.stream_handle()
        if use_graph:
            self.graph_launch(cache, st)
        else:
            self.launch_verify(cache, st)
        res = self.read_result()
        if commit:
            self._keep_commit(cache, P, len(res.accepted))
        return res

    def forward_only(self, cache: PagedKVCache, tokens, positions, parents, norm_hidden=False) -> None:
        self.set_step(tokens, positions, parents, cache.offset)
        self.launch_forward(cache, self.stream_handle(), norm_hidden=norm_hidden)

    def prefill(self, cache: PagedKVCache, tokens, chunk: int | None = None) -> None:
        """Causal prefill: the long-M path (prefill_long) for prompts of 128
        tokens or more where the engine has one, else chains of up to
        max_nodes tokens through the tree path."""
        toks = [int(t) for t in tokens]
        if chunk is None and len(toks) >= 128 and getattr(self, "supports_long_prefill", lambda: False)():
            self.prefill_long(cache, toks, want_logits=False)
            return
        chunk = chunk or self.max_nodes
        for s in range(0, len(toks), chunk):
            part = toks[s:s + chunk]
            P = cache.offset
            if P + len(part) > self.max_past:
                raise ValueError("prefill beyond max_past")
            self.forward_only(cache, part, [P + i for i in range(len(part))], [-1] + list(range(len(part) - 1)))
            cache.offset = P + len(part)

    # ---- HIP graph of the verify step ------------------------------------------
    # A captured graph holds the raw device pointers of one cache (K/V pages,
    # page table), so it is only ever replayed for that cache object: entries
    # are keyed by id() and hold a weak reference that is checked on lookup
    # (a new cache may reuse a dead one's id). When a cache dies its graph is
    # queued and destroyed at the next launch, after the stream has drained
    # (the finalizer itself may run at any point, e.g. during another capture).
    # Prefix lengths an attention grid is sized for: the step's P rounded up
    # to one of these (never past max_past), so the attention design and its
    # split count follow the prefix the step has, not the longest prefix the
    # engine may grow to (a 1024-key step of an engine sized for 4096 keys
    # runs the 1024-key grid). Graphs are kept per grid size.
    ATTN_GRID_PAST = (256, 512, 1024, 1536, 2048, 3072, 4096, 6144, 8192, 12288, 16384)

    def attn_grid_past(self, past_length: int) -> int:
        for b in self.ATTN_GRID_PAST:
            if past_length <= b:
                return min(b, self.max_past)
        return self.max_past

    def _graph_key(self, cache):
        return (id(cache), self.attn_grid_past(self._step_past))

    def _graph_for(self, cache: PagedKVCache) -> int:
        self._destroy_pending()
        key = self._graph_key(cache)
        ent = self._graphs.get(key)
        if ent is not None:
            ref, g = ent
            if ref() is cache:
                return g
            self._graphs.pop(key)
            self._dead_graphs.append(g)
            self._destroy_pending()
        return self.capture_verify(cache)

    def _destroy_pending(self) -> None:
        if not self._dead_graphs:
            return
        torch.cuda.synchronize(self.dev)
        while self._dead_graphs:
            self.lib.dtree_graph_destroy(C.c_void_p(self._dead_graphs.pop()))

    def graph_launch(self, cache: PagedKVCache, st: int) -> None:
        g = self._graph_for(cache)
        N.check(self.lib.dtree_graph_launch(C.c_void_p(g), st), "graph launch")

    def capture_verify(self, cache: PagedKVCache) -> int:
        side = torch.cuda.Stream(device=self.dev)
        side.wait_stream(torch.cuda.current_stream())
        h = side.cuda_stream
        N.check(self.lib.dtree_graph_begin(h), "graph begin")
        try:
            self.launch_verify(cache, h)
        except Exception:
            ex = C.c_void_p()
            self.lib.dtree_graph_end(h, C.byref(ex))
            raise
        ex = C.c_void_p()
        N.check(self.lib.dtree_graph_end(h, C.byref(ex)), "graph end")
        torch.cuda.current_stream().wait_stream(side)
        key, graphs, dead = self._graph_key(cache), self._graphs, self._dead_graphs

        def on_cache_dead(_ref, key=key, graphs=graphs, dead=dead):
            ent = graphs.get(key)
            if ent is not None and ent[0] is _ref:
                graphs.pop(key)
                dead.append(ent[1])

        self._graphs[key] = (weakref.ref(cache, on_cache_dead), ex.value)
        return ex.value

    def release_graphs(self) -> None:
        self._dead_graphs.extend(g for _, g in self._graphs.values())
        self._graphs.clear()
        self._destroy_pending()

    def __del__(self):
        try:
            self.release_graphs()
        except Exception:
            pass


class Qwen3TreeEngine(TreeEngineBase):
    """Qwen3 tree-verify executor (module docstring)."""

    def _alloc_layer_buffers(self) -> None:
        c, MP, dev = self.cfg, self.MP, self.dev
        f32, bf16 = torch.float32, torch.bfloat16
        self.qkv = torch.zeros(MP, c.qkv_dim, dtype=f32, device=dev)
        self.attn = torch.zeros(2, MP, c.q_dim, dtype=self.act_dtype, device=dev)
        self.act = torch.zeros(2, MP, c.intermediate_size, dtype=self.act_dtype, device=dev)
        self.rope_cos = torch.zeros(MP, c.head_dim // 2, dtype=f32, device=dev)
        self.rope_sin = torch.zeros(MP, c.head_dim // 2, dtype=f32, device=dev)
        aws = self.lib.dtree_attention_workspace_bytes(c.num_attention_heads, c.head_dim, self.max_past, self.MP)
        self.attn_ws = torch.zeros(aws, dtype=torch.uint8, device=dev)
        # Prefix length the attention grid is sized for (launch_forward sets it
        # from the step's P); the cache's page table must cover it (the
        # kernels read page entries before P is known).
        self.attn_max_past = self.max_past

    # ---- sizes ---------------------------------------------------------------
    def _gemm_shapes(self):
        c = self.cfg
        H, F = c.hidden_size, c.intermediate_size
        return {"qkv": (c.qkv_dim, H), "o": (H, c.q_dim), "gu": (2 * F, H), "down": (H, F)}

    def new_cache(self, page_order=None) -> PagedKVCache:
        c = self.cfg
        return PagedKVCache(c.num_hidden_layers, c.num_key_value_heads, c.head_dim,
                            self.max_past + self.max_nodes, device=self.dev, page_order=page_order)

    def _attention(self, li, cache: PagedKVCache, st, write_cache=True):
        c = self.cfg
        lw = self.w.layers[li]
        a = N.AttnArgs()
        a.qkv = self.qkv.data_ptr(); a.ld_qkv = self.qkv.shape[1]
        a.q_norm = lw.q_norm.data_ptr(); a.k_norm = lw.k_norm.data_ptr(); a.eps = c.rms_norm_eps
        a.rope_cos = self.rope_cos.data_ptr(); a.rope_sin = self.rope_sin.data_ptr()
        a.k_pages = cache.k_ptr(li); a.v_pages = cache.v_ptr(li); a.page_table = cache.page_table.data_ptr()
        a.desc = self.desc.data_ptr()
        a.out = self.attn[0].data_ptr(); a.out_lo = self.lo_ptr(self.attn); a.ld_out = self.attn.shape[-1]
        a.out_layout = self.w.layout
        a.num_heads = c.num_attention_heads; a.num_kv_heads = c.num_key_value_heads; a.head_dim = c.head_dim
        a.rows_padded = self.MP; a.scale = c.head_dim ** -0.5
        a.max_past_length = self.attn_max_past; a.write_cache = 1 if write_cache else 0
        a.workspace = self.attn_ws.data_ptr(); a.workspace_bytes = self.attn_ws.numel()
        N.check(self.lib.dtree_tree_attention(C.byref(a), st), "tree attention")

    def launch_forward(self, cache: PagedKVCache, st: int, norm_hidden: bool = False) -> None:
        """embed + all layers; tree K/V rows land in the cache at [P, P+L)."""
        c = self.cfg
        H = c.hidden_size
        if cache.capacity < self.max_past + self.max_nodes:
            raise ValueError("cache capacity is smaller than max_past + max_nodes")
        emb, emb_layout, emb_sb = self._embedding()
        N.check(self.lib.dtree_embed(
            self.desc.data_ptr(), emb, emb_layout, emb_sb, c.vocab_size, H,
            self.w.layers[0].input_norm.data_ptr(),
            self.MP,
            self.x.data_ptr(), self.xg[0].data_ptr(), self.lo_ptr(self.xg), self.w.layout, self.ss.data_ptr(),
            c.head_dim, c.rope_theta,
            self.rope_cos.data_ptr(), self.rope_sin.data_ptr(), st), "embed")
        self.attn_max_past = self.attn_grid_past(self._step_past)
        self._launch_layers(cache, st, norm_hidden=norm_hidden)
        self.launch_attention_status(self.attn_ws, st)

    def _launch_layers(self, cache: PagedKVCache, st: int, norm_hidden: bool = False, write_cache: bool = True) -> None:
        """The decoder layers over the rows already in x / xg / ss (and the RoPE
        table), then the optional final-norm output."""
        c = self.cfg
        H = c.hidden_size
        slot = {li: i for i, li in enumerate(self.layer_ids)}
        nL = c.num_hidden_layers
        for li in range(nL):
            lw = self.w.layers[li]
            nxt = self.w.layers[li + 1].input_norm if li + 1 < nL else self.w.final_norm
            self._gemm("qkv", self.xg, H, lw.wqkv, N.EPI_STORE_F32, st, ss_in=self.ss, out_f32=self.qkv)
            self._attention(li, cache, st, write_cache=write_cache)
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

    # ---- prompt prefill on the long-M GEMM (adapters.py:494-533) ---------------
    def supports_long_prefill(self) -> bool:
        return self.w.layout in (W_TILED, W_TILED_F16)  # bf16 or q4 group-64 weights

    def _prefill_buffers(self, rows: int) -> dict:
        pf = getattr(self, "_pf", None)
        if pf is not None and pf["rows"] >= rows and pf["nh"] == max(1, len(self.layer_ids)):
            return pf
        c, dev = self.cfg, self.dev
        H, F, D = c.hidden_size, c.intermediate_size, c.head_dim
        f32, bf16 = torch.float32, torch.bfloat16
        nh = max(1, len(self.layer_ids))
        pf = dict(rows=rows, nh=nh,
                  tokens=torch.zeros(rows, dtype=torch.int32, device=dev),
                  x=torch.zeros(rows, H, dtype=f32, device=dev),
                  xg=torch.zeros(2, rows, H, dtype=self.act_dtype, device=dev),
                  ss=torch.zeros(rows // 32, H // 32, 32, dtype=f32, device=dev),
                  qkv=torch.zeros(rows, c.qkv_dim, dtype=f32, device=dev),
                  attn=torch.zeros(2, rows, c.q_dim, dtype=self.act_dtype, device=dev),
                  act=torch.zeros(2, rows, F, dtype=self.act_dtype, device=dev),
                  hidden=torch.zeros(rows, nh * H, dtype=bf16, device=dev),
                  cos=torch.zeros(rows, D // 2, dtype=f32, device=dev),
                  sin=torch.zeros(rows, D // 2, dtype=f32, device=dev),
                  descs=torch.zeros(rows // 128, C.sizeof(N.StepDesc), dtype=torch.uint8, device=dev),
                  attn_ws=torch.zeros(self.lib.dtree_attention_workspace_bytes(c.num_attention_heads, D,
                                                                               self.max_past, 128),
                                      dtype=torch.uint8, device=dev))
        self._pf = pf
        return pf

    def prefill_long(self, cache: PagedKVCache, tokens, want_logits: bool = True):
        """Causal forward over the prompt with the long-M GEMM: per segment of
        up to PREFILL_SEGMENT tokens, embed, then per layer the fused QKV GEMM,
        attention per 128-row chunk (a chain "tree" over the cached prefix,
        appending its K/V rows), o_proj, gate/up and down_proj. Returns the
        fp32 logits of the last position ([1, 1, V]) if asked and the
        verifier hidden rows of every position ([n, n_ids * H] bf16 or None)."""
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
            dstride = self._prefill_chunks(pf, P0, n, rows, D, st)
            nL = c.num_hidden_layers
            for li in range(nL):
                lw = self.w.layers[li]
                nxt = self.w.layers[li + 1].input_norm if li + 1 < nL else self.w.final_norm
                self._long_gemm("qkv", pf["xg"], H, lw.wqkv, N.EPI_STORE_F32, rows, st, ss_in=pf["ss"],
                                out_f32=pf["qkv"])
                for ch in range(nch):
                    a = N.AttnArgs()
                    a.qkv = pf["qkv"][128 * ch].data_ptr(); a.ld_qkv = c.qkv_dim
                    a.q_norm = lw.q_norm.data_ptr(); a.k_norm = lw.k_norm.data_ptr(); a.eps = c.rms_norm_eps
                    a.rope_cos = pf["cos"][128 * ch].data_ptr(); a.rope_sin = pf["sin"][128 * ch].data_ptr()
                    a.k_pages = cache.k_ptr(li); a.v_pages = cache.v_ptr(li)
                    a.page_table = cache.page_table.data_ptr()
                    a.desc = pf["descs"].data_ptr() + ch * dstride
                    a.out = pf["attn"][0, 128 * ch].data_ptr()
                    a.out_lo = self.lo_ptr(pf["attn"], 2 * 128 * ch * c.q_dim)
                    a.ld_out = c.q_dim; a.out_layout = self.w.layout
                    a.num_heads = c.num_attention_heads; a.num_kv_heads = c.num_key_value_heads; a.head_dim = D
                    a.rows_padded = 128; a.scale = D ** -0.5
                    a.max_past_length = self.attn_grid_past(P0 + 128 * ch); a.write_cache = 1
                    a.workspace = pf["attn_ws"].data_ptr(); a.workspace_bytes = pf["attn_ws"].numel()
                    N.check(self.lib.dtree_tree_attention(C.byref(a), st), "prefill attention")
                self._long_gemm("o", pf["attn"], c.q_dim, lw.wo, N.EPI_RESIDUAL, rows, st, out_f32=pf["x"],
                                out_bf16=pf["xg"], next_norm=lw.post_norm, ss_out=pf["ss"])
                self._long_gemm("gu", pf["xg"], H, lw.wgu, N.EPI_SWIGLU, rows, st, ss_in=pf["ss"], out_bf16=pf["act"])
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

    def launch_compact(self, cache: PagedKVCache, st: int, select_hidden: bool = True, aux: bool = False) -> None:
        c = self.cfg
        d = self.desc_aux if aux else self.desc
        N.check(self.lib.dtree_compact(
            d.data_ptr(), cache.k_pages.data_ptr(), cache.v_pages.data_ptr(), cache.layer_stride,
            c.num_hidden_layers, c.num_key_value_heads, c.head_dim, cache.page_table.data_ptr(),
            self.hidden.data_ptr() if select_hidden else None, self.hidden.shape[1],
            self.hidden_sel.data_ptr() if select_hidden else None, st), "compact")

