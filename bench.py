"""Tree-verify step benchmark on one MI355X.

Workload (default): one DTree verify step of a random-init Qwen3-4B-shaped bf16
model (36 layers, hidden 2560, FFN 9728, GQA 32/8, head_dim 128, vocab
151936) at a 1024-token prefix with a 24-node draft tree (25 rows incl. the
root): every layer, LM-head argmax per node, greedy accept walk and KV
compaction, replayed as one HIP graph. Inputs (weights, KV prefix, tree) are
resident in HBM before timing; each timed step uploads the 4.6 KB step
descriptor, replays the graph and reads the walk result back.

--model qwen35-4b runs the Qwen3.5-4B-shaped hybrid instead (32 layers: 24
GatedDeltaNet + 8 gated attention, hidden 2560, prefix 2048 by default):
GatedDeltaNet tree recurrence from the committed fp32 state, gated
head_dim-256 tree attention, LM-head argmax, walk, KV compaction and the
GatedDeltaNet commit along the accepted path, as one HIP graph.
--model qwen35-9b runs the Qwen3.5-9B-shaped hybrid (hidden 4096, FFN 12288)
with q4 weights, an 8192-token prefix and draft budget 64 (65-node trees) by
default.

Prints ONE JSON line (rank 0). Progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "dtree-mlx_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBPS = 8000.0
# Timed and warmup steps of every extra workload line: the headline's
# defaults, since a 30-step run after 5 warmup steps reads 2-4 % slower
# than a 100-step run of the same step in the same process.
CONFIG_STEPS, CONFIG_WARMUP = 100, 10


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def graph_timed(lib, st: int, launch, n: int, reps: int) -> float:
    """Average device time of one launch: `reps` launches (launch(r % n,
    stream), rotating over n argument sets) captured into one HIP graph on a
    side stream and replayed on `st` between two HIP events. Launching from
    the host instead would time the host's launch rate for kernels shorter
    than one ctypes + HIP launch (~10 us), as the step's graph never does."""
    import ctypes as C

    import torch

    from dtree_hip import _native as N

    for r in range(n):
        launch(r, st)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    h = side.cuda_stream
    N.check(lib.dtree_graph_begin(h), "graph begin")
    try:
        for r in range(reps):
            launch(r % n, h)
    finally:
        ex = C.c_void_p()
        rc = lib.dtree_graph_end(h, C.byref(ex))
    N.check(rc, "graph end")
    torch.cuda.current_stream().wait_stream(side)
    try:
        N.check(lib.dtree_graph_launch(ex, st), "graph launch")  # warm replay
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        N.check(lib.dtree_graph_launch(ex, st), "graph launch")
        e1.record()
        e1.synchronize()
    finally:
        lib.dtree_graph_destroy(ex)
    return e0.elapsed_time(e1) * 1e3 / reps


def weight_bytes(params: int, quant: str) -> int:
    """bf16: 2 B per weight; q4 group-64: half a byte plus a bf16 scale and bias per 64."""
    return params * 2 if quant == "bf16" else params // 2 + params // 64 * 4


def algorithmic_bytes(cfg, P: int, L: int, quant: str = "bf16") -> dict:
    """Minimum HBM bytes of one verify step (weights once, KV prefix read, tree KV write)."""
    H, F, V, D = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.head_dim
    nl = cfg.num_hidden_layers
    lin = weight_bytes(nl * cfg.layer_linear_params(), quant)
    lm = weight_bytes(V * H, quant)
    norms = (nl * (2 * H + 2 * D) + H) * 2
    emb = weight_bytes(L * H, quant)
    kv_read = nl * 2 * cfg.num_key_value_heads * P * D * 2
    kv_write = nl * 2 * cfg.num_key_value_heads * L * D * 2
    total = lin + lm + norms + emb + kv_read + kv_write
    return dict(linear=lin, lm_head=lm, norms=norms, embed_rows=emb, kv_prefix_read=kv_read,
                tree_kv_write=kv_write, total=total)


def cpu_baseline(cfg, weights, cache, tree, P, warmup=2, steps=10):
    """The fp32 numpy oracle of the same verify step (the CPU restatement:
    every layer's tree block over the same KV prefix, the tied LM head and
    argmax, the greedy walk and the KV compaction), timed on the host cores as
    whole steps: `warmup` untimed steps, then the median of `steps` timed ones."""
    import numpy as np

    from oracle import qwen3 as oq
    from oracle import tree as otree

    try:
        from threadpoolctl import threadpool_info
        cores = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        cores = os.cpu_count() or 1
    t_setup = time.perf_counter()
    ocfg = oq.Qwen3Config(hidden=cfg.hidden_size, layers=cfg.num_hidden_layers, ffn=cfg.intermediate_size,
                          heads=cfg.num_attention_heads, kv_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                          vocab=cfg.vocab_size, eps=cfg.rms_norm_eps, rope_base=cfg.rope_theta)
    acc = weights.host_accessor()
    names = ("input_norm", "q", "k", "v", "q_norm", "k_norm", "o", "post_norm", "gate", "up", "down")
    W = {(li, n): oq.bf16_to_f32(acc(li, n)) for li in range(cfg.num_hidden_layers) for n in names}
    W[(None, "embed")] = oq.bf16_to_f32(acc(None, "embed"))
    W[(None, "final_norm")] = oq.bf16_to_f32(acc(None, "final_norm"))
    orc = oq.OracleQwen3(ocfg, lambda li, n: W[(li, n)])
    ids, pos, mask = otree.compile_tree(tree.tokens[0], P, tree.tokens[1:], tree.depths[1:], tree.visibility, P)
    kp = [cache.logical_keys(li, P).float().cpu().numpy() for li in range(cfg.num_hidden_layers)]
    vp = [cache.logical_values(li, P).float().cpu().numpy() for li in range(cfg.num_hidden_layers)]
    oc = oq.OracleCache(keys=kp, values=vp)
    E = W[(None, "embed")]
    t_setup = time.perf_counter() - t_setup

    def step():
        norm, vh, nk, nv = orc.forward_tree(ids, pos, mask, oc, [1, 9, 17, 25, 33])
        post = np.argmax(norm @ E.T, axis=-1)
        acc_idx, _ = otree.follow_verified_tree(tree.child_maps, post.tolist())
        for li in range(cfg.num_hidden_layers):  # KV compaction: cache rows of the accepted path
            np.concatenate([kp[li], nk[li][acc_idx]]), np.concatenate([vp[li], nv[li][acc_idx]])
        return vh[acc_idx]

    for _ in range(warmup):
        step()
    times = []
    for _ in range(steps):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    t_step = float(np.median(times))
    return {"value": 1.0 / t_step, "unit": "steps/s", "cores": int(cores), "kind": "port",
            "sample": (f"CPU restatement (fp32 numpy oracle of the whole verify step: {cfg.num_hidden_layers} tree "
                       f"blocks, LM head + argmax, walk, KV compaction) on the same weights, prefix and tree; "
                       f"{warmup} warm-up + median of {steps} whole steps ({t_step:.3f} s/step; setup "
                       f"{t_setup:.0f} s)")}


def time_kernels(eng, cfg, w, cache, st, P: int, L: int, reps: int, quant: str = "bf16") -> dict:
    """Average launch duration of every kernel of the step, timed live with HIP
    events on the launch stream (torch's current stream), each kernel class
    rotating over the 36 layers' weights so every launch streams from HBM.
    Must run after the timed region: re-running the residual GEMMs keeps
    adding into the residual stream. Algorithmic bytes per launch count each
    weight once and activations in bf16."""
    import ctypes as C

    import torch

    from dtree_hip import _native as N

    H, F, V, D = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.head_dim
    Hq, Hkv, nl = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.num_hidden_layers
    qkv_n = (Hq + 2 * Hkv) * D
    lib = eng.lib
    gemm = lib.dtree_gemm_bf16

    def layer_args(li):
        lw = w.layers[li]
        nxt = w.layers[li + 1].input_norm if li + 1 < nl else w.final_norm
        return {
            "qkv": eng.gemm_args("qkv", eng.xg, H, lw.wqkv, N.EPI_STORE_F32, ss_in=eng.ss, out_f32=eng.qkv),
            "o": eng.gemm_args("o", eng.attn, cfg.q_dim, lw.wo, N.EPI_RESIDUAL, out_f32=eng.x, out_bf16=eng.xg,
                               next_norm=lw.post_norm, ss_out=eng.ss),
            "gu": eng.gemm_args("gu", eng.xg, H, lw.wgu, N.EPI_SWIGLU, ss_in=eng.ss, out_bf16=eng.act),
            "down": eng.gemm_args("down", eng.act, F, lw.wd, N.EPI_RESIDUAL, out_f32=eng.x, out_bf16=eng.xg,
                                  next_norm=nxt, ss_out=eng.ss),
        }

    args = [layer_args(li) for li in range(nl)]
    keep = [args]

    def timed(launch) -> float:
        return graph_timed(lib, st, launch, nl, reps)

    refs = {k: [C.byref(args[li][k]) for li in range(nl)] for k in ("qkv", "o", "gu", "down")}
    us = {k: timed(lambda r, s, k=k: gemm(refs[k][r], s)) for k in refs}
    us["attention"] = timed(lambda r, s: eng._attention(r, cache, s))
    us["lm_head"] = timed(lambda r, s: eng.launch_lm_head(s))
    keep.append(refs)

    wb = lambda params: weight_bytes(params, quant)  # noqa: E731
    b = {
        "qkv": wb(qkv_n * H) + L * H * 2 + L * qkv_n * 2,
        "o": wb(H * cfg.q_dim) + L * cfg.q_dim * 2 + L * H * 2,
        "gu": wb(2 * F * H) + L * H * 2 + L * F * 2,
        "down": wb(H * F) + L * F * 2 + L * H * 2,
        "attention": 2 * Hkv * P * D * 2 + 2 * Hkv * L * D * 2 + L * qkv_n * 2 + L * cfg.q_dim * 2,
        "lm_head": wb(V * H) + L * H * 2,
    }
    q4 = "true" if quant == "q4" else "false"
    out = {}

    def entry(kernel, n, t_us, nbytes):
        return {"kernel": kernel, "launches_per_step": n, "avg_launch_us": t_us,
                "algorithmic_bytes_per_launch": int(nbytes), "achieved_gbps": nbytes / (t_us * 1e-6) / 1e9}

    lo = not eng.hi_only  # q4 models and fp16 weights read one activation plane
    out["qkv_gemm"] = entry(gemm_kernel_name(qkv_n, H, 0, quant, lo=lo and "qkv" not in eng.HI_ONLY, h16=eng.h16),
                            nl, us["qkv"], b["qkv"])
    out["attention"] = entry(attention_kernel_name(eng.attn_grid_past(P), 128, 128, False, eng.MP), nl, us["attention"],
                             b["attention"])
    out["o_gemm"] = entry(gemm_kernel_name(H, cfg.q_dim, 1, quant, lo=lo, h16=eng.h16), nl, us["o"], b["o"])
    out["down_gemm"] = entry(gemm_kernel_name(H, F, 1, quant, lo=lo, h16=eng.h16), nl, us["down"], b["down"])
    out["gate_up_gemm"] = entry(gemm_kernel_name(2 * F, H, 2, quant, lo=lo, h16=eng.h16), nl, us["gu"], b["gu"])
    out["lm_head"] = entry(lmhead_kernel_name(quant, eng.MP, eng.h16, lo=lo), 1, us["lm_head"], b["lm_head"])
    return out


def algorithmic_bytes35(cfg, P: int, L: int, quant: str = "bf16") -> dict:
    """Minimum HBM bytes of one hybrid verify step: every weight once, the KV
    prefix of the attention layers, the committed GatedDeltaNet windows and
    states read and the committed ones written, tree KV rows written."""
    H, F, V, D = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.head_dim
    nG, nA = len(cfg.linear_layers), len(cfg.attention_layers)
    Hv = cfg.linear_num_value_heads
    gdn_params = (cfg.conv_dim + cfg.value_dim + 2 * Hv) * H + H * cfg.value_dim
    attn_params = cfg.attn_qkv_dim * H + H * cfg.q_dim
    mlp_params = 3 * H * F
    lin = weight_bytes(nG * gdn_params + nA * attn_params + cfg.num_hidden_layers * mlp_params, quant)
    small = nG * (cfg.linear_conv_kernel_dim * cfg.conv_dim * 4 + 2 * Hv * 4 + cfg.linear_value_head_dim * 2)
    lm = weight_bytes(V * H, quant)
    norms = (cfg.num_hidden_layers * 2 * H + nA * 2 * D + H) * 2
    emb = weight_bytes(L * H, quant)
    kv_read = nA * 2 * cfg.num_key_value_heads * P * D * 2
    kv_write = nA * 2 * cfg.num_key_value_heads * L * D * 2
    state = nG * (Hv * cfg.linear_value_head_dim * cfg.linear_key_head_dim
                  + (cfg.linear_conv_kernel_dim - 1) * cfg.conv_dim) * 4
    total = lin + small + lm + norms + emb + kv_read + kv_write + 2 * state
    return dict(linear=lin, gdn_small=small, lm_head=lm, norms=norms, embed_rows=emb, kv_prefix_read=kv_read,
                tree_kv_write=kv_write, gdn_state_read=state, gdn_state_write=state, total=total)


def cpu_baseline35(cfg, weights, cache, tree, P, min_seconds=15.0):
    """The oracle (fp32 numpy, GatedDeltaNet recurrence in fp64) of the same
    hybrid step on the host cores, on a bounded sample: the first
    GatedDeltaNet layer and the first attention layer (repeated), and a
    quarter of the LM head, scaled linearly to the whole step."""
    import numpy as np

    from oracle import qwen35 as o35
    from oracle.qwen3 import bf16_to_f32, rms_norm

    try:
        from threadpoolctl import threadpool_info
        cores = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        cores = os.cpu_count() or 1
    ocfg = o35.Qwen35Config(
        hidden=cfg.hidden_size, layers=cfg.num_hidden_layers, ffn=cfg.intermediate_size,
        heads=cfg.num_attention_heads, kv_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
        rope_dims=cfg.rope_dims, lin_k_heads=cfg.linear_num_key_heads, lin_v_heads=cfg.linear_num_value_heads,
        lin_k_dim=cfg.linear_key_head_dim, lin_v_dim=cfg.linear_value_head_dim,
        conv_kernel=cfg.linear_conv_kernel_dim, full_attention_interval=cfg.full_attention_interval,
        vocab=cfg.vocab_size, eps=cfg.rms_norm_eps, rope_base=cfg.rope_theta)
    acc = weights.host_accessor()
    lg, la = cfg.linear_layers[0], cfg.attention_layers[0]
    gdn_names = ("input_norm", "in_qkv", "in_z", "in_b", "in_a", "conv", "A_log", "dt_bias", "gnorm", "out",
                 "post_norm", "gate", "up", "down")
    attn_names = ("input_norm", "q", "k", "v", "q_norm", "k_norm", "o", "post_norm", "gate", "up", "down")
    W = {(lg, n): np.asarray(acc(lg, n)) for n in gdn_names}
    W.update({(la, n): np.asarray(acc(la, n)) for n in attn_names})
    orc = o35.OracleQwen35(ocfg, lambda li, n: W[(li, n)])
    s = cache.slot
    win = cache.windows[s[lg]].cpu().numpy()
    state = cache.states[s[lg]].cpu().double().numpy()
    kp = cache.kv.logical_keys(s[la], P).float().cpu().numpy()
    vp = cache.kv.logical_values(s[la], P).float().cpu().numpy()
    pos = np.asarray(tree.positions(P))
    mask = o35.tree_mask(tree.parents, P)
    x0 = bf16_to_f32(acc(None, "embed")[np.asarray(tree.tokens)])
    tg, ta = [], []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        x, _ = orc.gdn_layer(lg, x0, win, state, tree.parents)
        t1 = time.perf_counter()
        x, _ = orc.attn_layer(la, x, kp, vp, pos, mask)
        t2 = time.perf_counter()
        tg.append(t1 - t0)
        ta.append(t2 - t1)
        if time.perf_counter() - t_start > min_seconds or len(tg) >= 200:
            break
    E = acc(None, "embed")
    q = E.shape[0] // 4
    Eq = bf16_to_f32(E[:q])
    h = rms_norm(x, np.ones(cfg.hidden_size, np.float32), cfg.rms_norm_eps)
    lm_t = []
    for _ in range(3):
        t0 = time.perf_counter()
        np.argmax(h @ Eq.T, axis=-1)
        lm_t.append(time.perf_counter() - t0)
    t_g, t_a = float(np.median(tg)), float(np.median(ta))
    t_step = (t_g * len(cfg.linear_layers) + t_a * len(cfg.attention_layers)
              + float(np.median(lm_t)) * (E.shape[0] / q))
    return {"value": 1.0 / t_step, "unit": "steps/s", "cores": int(cores), "kind": "port",
            "sample": (f"oracle: 1 GatedDeltaNet + 1 attention layer x {len(tg)} passes (median "
                       f"{t_g * 1e3:.1f} / {t_a * 1e3:.1f} ms) + 1/4 of the LM head, scaled linearly to one "
                       f"step ({t_step:.2f} s)")}


def time_kernels35(eng, cfg, w, cache, st, P: int, L: int, reps: int, quant: str = "bf16") -> dict:
    """Average launch duration of every kernel class of the hybrid step (HIP
    events on the launch stream), rotating over the layers of that class so
    each launch streams its own weights. Runs after the timed region (the
    residual GEMMs keep adding into the residual stream)."""
    import ctypes as C

    import torch

    from dtree_hip import _native as N

    H, F, V, D = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.head_dim
    lib = eng.lib
    gemm = lib.dtree_gemm_bf16
    G, A = cfg.linear_layers, cfg.attention_layers
    args = {"in": [], "out": [], "gdn": [], "qkv": [], "o": [], "gu": [], "down": []}
    for li in G:
        lw = w.layers[li]
        gi = cache.slot[li]
        args["in"].append(eng.gemm_args("in", eng.xg, H, lw.w_in, N.EPI_STORE_F32, ss_in=eng.ss,
                                        out_f32=eng.proj[gi]))
        args["out"].append(eng.gemm_args("out", eng.gout, cfg.value_dim, lw.w_out, N.EPI_RESIDUAL, out_f32=eng.x,
                                         out_bf16=eng.xg, next_norm=lw.post_norm, ss_out=eng.ss))
        args["gdn"].append(eng.gdn_args(li, cache))
    for li in A:
        lw = w.layers[li]
        args["qkv"].append(eng.gemm_args("qkv", eng.xg, H, lw.wqkv, N.EPI_STORE_F32, ss_in=eng.ss,
                                         out_f32=eng.qkv))
        args["o"].append(eng.gemm_args("o", eng.attn, cfg.q_dim, lw.wo, N.EPI_RESIDUAL, out_f32=eng.x,
                                       out_bf16=eng.xg, next_norm=lw.post_norm, ss_out=eng.ss))
    for li in range(cfg.num_hidden_layers):
        lw = w.layers[li]
        nxt = w.layers[li + 1].input_norm if li + 1 < cfg.num_hidden_layers else w.final_norm
        args["gu"].append(eng.gemm_args("gu", eng.xg, H, lw.wgu, N.EPI_SWIGLU, ss_in=eng.ss, out_bf16=eng.act))
        args["down"].append(eng.gemm_args("down", eng.act, F, lw.wd, N.EPI_RESIDUAL, out_f32=eng.x,
                                          out_bf16=eng.xg, next_norm=nxt, ss_out=eng.ss))
    refs = {k: [C.byref(a) for a in v] for k, v in args.items()}

    def timed(launch, n) -> float:
        return graph_timed(lib, st, launch, n, reps)

    us = {k: timed(lambda r, s, k=k: gemm(refs[k][r], s), len(refs[k])) for k in ("in", "out", "qkv", "o", "gu",
                                                                                     "down")}
    g = refs["gdn"]
    us["prep"] = timed(lambda r, s: lib.dtree_gdn_layer_prep(g[r], s), len(g))
    us["recurrence"] = timed(lambda r, s: lib.dtree_gdn_layer_recurrence(g[r], s), len(g))
    # trees of up to 32 nodes with 128-dim heads run prep and recurrence as one
    # launch in the step (dtree_gdn_layer_prep_recurrence)
    fused = eng.MP == 32 and cfg.linear_key_head_dim == 128 and cfg.linear_value_head_dim == 128
    if fused:
        us["prep_recurrence"] = timed(lambda r, s: lib.dtree_gdn_layer_prep_recurrence(g[r], s), len(g))
    us["gated_norm"] = timed(lambda r, s: lib.dtree_gdn_layer_gated_norm(g[r], s), len(g))
    # every layer's commit in one launch, as the step runs it
    g_all = (N.GdnArgs * len(args["gdn"]))(*args["gdn"])
    for i, li in enumerate(G):  # into the spare pair, as the step's commit writes
        g_all[i].window_out = cache.windows_next[cache.slot[li]].data_ptr()
        g_all[i].state_out = cache.states_next[cache.slot[li]].data_ptr()
    us["commit"] = timed(lambda r, s: lib.dtree_gdn_layers_commit(g_all, len(args["gdn"]), s), 1)
    us["attention"] = timed(lambda r, s: eng._attention(A[r], cache, s), len(A))
    us["lm_head"] = timed(lambda r, s: eng.launch_lm_head(s), 1)

    wb = lambda params: weight_bytes(params, quant)  # noqa: E731
    Hv, Dk, Dv = cfg.linear_num_value_heads, cfg.linear_key_head_dim, cfg.linear_value_head_dim
    C_ = cfg.conv_dim
    state_b = Hv * Dv * Dk * 4
    b = {
        "in": wb(cfg.in_proj_dim * H) + L * H * 2 + L * cfg.in_proj_dim * 4,
        "out": wb(H * cfg.value_dim) + L * cfg.value_dim * 2 + L * H * 2,
        "qkv": wb(cfg.attn_qkv_dim * H) + L * H * 2 + L * cfg.attn_qkv_dim * 4,
        "o": wb(H * cfg.q_dim) + L * cfg.q_dim * 2 + L * H * 2,
        "gu": wb(2 * F * H) + L * H * 2 + L * F * 2,
        "down": wb(H * F) + L * F * 2 + L * H * 2,
        "prep": L * (C_ + 2 * Hv) * 4 + cfg.linear_conv_kernel_dim * C_ * 4 + L * (C_ + 2 * Hv) * 4,
        "recurrence": state_b + L * (2 * cfg.key_dim + cfg.value_dim + 2 * Hv) * 4 + L * cfg.value_dim * 4,
        "gated_norm": 2 * L * cfg.value_dim * 4 + L * cfg.value_dim * 2,
        "commit": 2 * state_b,
        "attention": 2 * cfg.num_key_value_heads * P * D * 2 + 2 * cfg.num_key_value_heads * L * D * 2
        + L * cfg.attn_qkv_dim * 4 + L * cfg.q_dim * 2,
        "lm_head": wb(V * H) + L * H * 2,
    }
    q4 = "true" if quant == "q4" else "false"
    nG, nA, nL = len(G), len(A), cfg.num_hidden_layers

    def entry(kernel, n, t_us, nbytes):
        return {"kernel": kernel, "launches_per_step": n, "avg_launch_us": t_us,
                "algorithmic_bytes_per_launch": int(nbytes), "achieved_gbps": nbytes / (t_us * 1e-6) / 1e9}

    kn = lambda n, k, epi, lo=not eng.hi_only: gemm_kernel_name(n, k, epi, quant, rows=eng.MP, lo=lo,  # noqa: E731
                                                                h16=eng.h16)
    out = {
        "in_proj_gemm": entry(kn(cfg.in_proj_dim, H, 0), nG, us["in"], b["in"]),
        "out_proj_gemm": entry(kn(H, cfg.value_dim, 1), nG, us["out"], b["out"]),
        "attn_qkv_gemm": entry(kn(cfg.attn_qkv_dim, H, 0, not eng.hi_only and "qkv" not in eng.HI_ONLY), nA, us["qkv"],
                               b["qkv"]),
        "o_gemm": entry(kn(H, cfg.q_dim, 1), nA, us["o"], b["o"]),
        "gate_up_gemm": entry(kn(2 * F, H, 2), nL, us["gu"], b["gu"]),
        "down_gemm": entry(kn(H, F, 1), nL, us["down"], b["down"]),
        "gdn_prep": entry(f"gdn_prep_kernel<{cfg.linear_conv_kernel_dim - 1}, 128>", nG, us["prep"], b["prep"]),
        "gdn_recurrence": entry(gdn_recurrence_name(eng.MP, 0), nG,
                                us["recurrence"], b["recurrence"]),
        "gdn_gated_norm": entry("gdn_gated_norm_kernel<128>", nG, us["gated_norm"], b["gated_norm"]),
        "gdn_commit": entry("gdn_commit_layers_kernel<128>", 1, us["commit"], nG * b["commit"]),
        "attention": entry(attention_kernel_name(eng.attn_grid_past(P), 256, 64, True, eng.MP), nA, us["attention"],
                           b["attention"]),
        "lm_head": entry(lmhead_kernel_name(quant, eng.MP, eng.h16, lo=not eng.hi_only), 1, us["lm_head"],
                         b["lm_head"]),
    }
    if fused:
        for k in ("gdn_prep", "gdn_recurrence"):
            out[k]["launches_per_step"] = 0
            out[k]["note"] = "timed alone; the step runs it inside gdn_prep_recurrence"
        # the recurrence's bytes (its inputs are now the raw conv / b / a columns,
        # of the same size), the conv taps and window, and q / k / v / g / beta
        # written for the commit
        out["gdn_prep_recurrence"] = entry(gdn_recurrence_name(eng.MP, cfg.linear_conv_kernel_dim - 1), nG,
                                           us["prep_recurrence"],
                                           b["recurrence"] + (2 * cfg.linear_conv_kernel_dim - 1) * C_ * 4
                                           + L * (C_ + 2 * Hv) * 4)
    return out



def gdn_recurrence_name(rows: int, keep: int) -> str:
    """GatedDeltaNet tree recurrence kernel (gdn.hip): the matrix form for up
    to 32 rows (with the input prep fused when keep > 0) and in 32-node blocks
    up to 96 rows; DTREE_GDN_KERNEL=reg keeps the node-by-node kernels, =dfs
    the depth-first kernel past 32 rows."""
    node_by_node = os.environ.get("DTREE_GDN_KERNEL") in ("reg", "dfs")
    if rows <= 32:
        if os.environ.get("DTREE_GDN_KERNEL") == "reg":
            return f"gdn_prep_reg_kernel<{keep}>" if keep else "gdn_tree_reg_kernel<32>"
        return f"gdn_tree_chunk_kernel<{keep}>"
    return "gdn_tree_dfs_kernel" if node_by_node or rows > 96 else "gdn_tree_blocks_kernel"


def attention_kernel_name(max_past: int, D: int, R: int, gated: bool, MP: int) -> str:
    """Tree-attention kernel the library dispatches (attention.hip): the
    per-KV-group design above a 1536-key prefix grid, the per-head one below;
    DTREE_ATTN_KERNEL forces either."""
    forced = os.environ.get("DTREE_ATTN_KERNEL")
    group = forced == "group" or (forced != "head" and max_past > 1536)
    g = "true" if gated else "false"
    return f"gqa_tree_attn_kernel<{D}, {R}, {g}, 4>" if group else f"tree_attn_kernel<{D}, {R}, {g}, {1 if MP == 32 else 4}>"


def lmhead_kernel_name(quant: str, rows: int, h16: bool = False, lo: bool = True) -> str:
    """LM-head kernel (gemm.hip, dtree_lmhead_argmax): the one-pass q4 kernel's
    argmax epilogue for a q4 embedding (vocabularies up to 262144; `lo` False:
    the high activation plane alone), else the persistent LM head (`h16`: fp16
    tiled embedding and one fp16 activation plane)."""
    if quant == "q4":
        return f"q4m_gemm_kernel<{'true' if lo else 'false'}, 16, {rows // 32}, 4>"
    mb = rows // 32
    lo, h = ("false", ", true") if h16 else ("true", "")
    return (f"lmhead_kernel<{mb}, {2 if mb == 1 else (2 if mb == 2 else 1)}, {2 if mb == 1 else 1}, {lo}, true, "
            f"{'true' if quant == 'q4' else 'false'}{h}>")


def gemm_kernel_name(n: int, k: int, epi: int, quant: str, cus: int = 256, rows: int = 32,
                     lo: bool = True, h16: bool = False) -> str:
    """Kernel the library picks for a tiled GEMM with split_k 0 (gemm.hip,
    dtree_gemm_bf16); `lo` False for a projection that reads only the high
    activation plane (the first template argument); `h16` for fp16 tiled
    weights with one fp16 activation plane (no low plane, the last template
    argument true). q4 over 64-128 rows: the one-pass kernel, two 64-column
    blocks per workgroup unless a 4-block tiling still covers half the CUs,
    three when that fills at least an eighth more of the CUs.
    32 rows, bf16 or q4: three workgroups per 32-column tile (one per part of
    K) at K >= 4096 and N % 256 == 0 when 3 N / 32 fit the CUs, two at K = 4096
    when 2 N / 32 do; else one per tile at K <= 4096 and N / 32 <= CUs (q4:
    at K <= 4096 whatever N); else stream-K (q4: two workgroups per CU when
    there are at least 20 64 x 64 units per CU)."""
    L = "true" if lo and not h16 else "false"
    h = ", true" if h16 else ""
    if quant == "q4" and rows > 32:
        nblk, nkb = n // 64, k // 64

        def plan(cw):
            tiles = -(-nblk // cw)
            parts = max(1, min(cus // tiles, nkb // (2 if cw == 2 else 1)))
            return tiles * parts

        cw = 4 if nblk % 4 == 0 and 2 * (nblk // 4) >= cus else 2
        if plan(3) >= plan(cw) + cus // 8:
            cw = 3
        return f"q4m_gemm_kernel<{L}, {epi}, {rows // 32}, {cw}>"
    dp = "dp_gemm_kernel" if quant == "bf16" else "dpq_gemm_kernel"
    if k >= 4096 and n % 256 == 0:
        if (n // 32) * 3 <= cus:
            return f"{dp}<{L}, {epi}, 3{h}>"
        if k == 4096 and (n // 32) * 2 <= cus:
            return f"{dp}<{L}, {epi}, 2{h}>"
    if k <= 4096 and (n // 32 <= cus or quant == "q4"):
        return f"{dp}<{L}, {epi}, 1{h}>"
    if quant == "q4" and (n // 64) * (k // 64) >= 20 * cus:
        return f"sk2_gemm_kernel<{L}, {epi}>"
    return f"sk_gemm_kernel<{L}, {epi}, {'true' if quant == 'q4' else 'false'}{h}>"


def copy_probe(mib: int) -> None:
    """Five copies of `mib` MiB between two device buffers: each dispatch reads
    and writes exactly mib MiB, which calibrates the profiler's FETCH_SIZE and
    WRITE_SIZE counters against known traffic."""
    import torch

    n = mib << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] copy probe: 5 x {mib} MiB")


MODEL_NAMES = {"qwen3-4b": "Qwen3-4B", "qwen35-4b": "Qwen3.5-4B-shaped hybrid",
               "qwen35-9b": "Qwen3.5-9B-shaped hybrid"}


def prefill_bench(eng, P: int, reps: int = 3, hybrid: bool = False, label: str = "Qwen3-4B bf16") -> dict:
    """Prompt prefill of P random tokens into a fresh cache: the long-M path
    (128 x 128 MFMA tiles, attention per 128-row chunk; for the hybrid the
    GatedDeltaNet layers as a chain recurrence over the prompt) against the
    chain path (max_nodes-token tree passes). Algorithmic FLOPs: 2 * P *
    linear parameters (the kernels do twice that: hi and lo activation
    planes)."""
    import torch

    from dtree_hip.synthetic import random_prefix

    c = eng.cfg
    toks = random_prefix(P, c.vocab_size, seed=7)
    times = []
    for _ in range(reps + 1):
        cache = eng.new_cache()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        eng.prefill_long(cache, toks)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
        del cache
    long_ms = min(times[1:]) * 1e3
    cache = eng.new_cache()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    eng.prefill(cache, toks, chunk=eng.max_nodes)
    torch.cuda.synchronize()
    chain_ms = (time.perf_counter() - t0) * 1e3
    del cache
    if hybrid:
        nG, nA = len(c.linear_layers), len(c.attention_layers)
        params = (nG * (c.in_proj_dim * c.hidden_size + c.hidden_size * c.value_dim)
                  + nA * (c.attn_qkv_dim * c.hidden_size + c.hidden_size * c.q_dim)
                  + c.num_hidden_layers * 3 * c.hidden_size * c.intermediate_size)
        what = (f"{label} prompt prefill, {P} tokens ({nG} GatedDeltaNet layers: chain recurrence, committed "
                f"window and state; {nA} attention layers: K/V into the paged cache)")
    else:
        params = c.layer_linear_params() * c.num_hidden_layers
        what = f"{label} prompt prefill, {P} tokens ({c.num_hidden_layers} layers, K/V into the paged cache)"
    flops = 2.0 * P * params
    return {"workload": what,
            "long_path_ms": round(long_ms, 3), "chain_path_ms": round(chain_ms, 3),
            "long_path_tflops_algorithmic": round(flops / (long_ms * 1e-3) / 1e12, 1),
            "tokens_per_s": round(P / (long_ms * 1e-3), 1)}


def decode_step_bench(target_model, cache, P: int, budget: int, steps: int = 30) -> dict:
    """Latency of the rest of a DTree decode step around the verify, at the
    verify workload's shapes: the DFlash drafter call (Qwen3-4B-sized drafter,
    5 layers; 16-row block after a 5-row context append, then the block trim),
    the target's LM head over the 15 draft rows (fp32 logits), the draft tree
    built on the device from those logits (3 launches) against the host heap
    of build_dtree_tree, and the whole step: drafter + LM head + device tree +
    verify graph + one readback. Random-init drafter: the acceptance it gets is
    not meaningful, the latencies are."""
    import torch

    from dtree_hip.adapters import Qwen3TargetAdapter
    from dtree_hip.draft import DFlashDraftModel, random_draft_config
    from dtree_hip.dtree_runtime import build_dtree_tree
    from dtree_hip.runtime import trim_draft_cache

    eng = target_model.engine
    cfg = target_model.args
    dev = eng.dev
    args = random_draft_config(cfg, "dflash-b16")
    draft = DFlashDraftModel.random(args, seed=11, max_past=P + 64, device=dev)
    dcache = draft.make_cache()
    H = cfg.hidden_size
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    ctx0 = (torch.randn(1, P, 5 * H, generator=g, device=dev)).to(torch.bfloat16)
    draft(noise_embedding=torch.zeros(1, 16, H, dtype=torch.bfloat16, device=dev), target_hidden=ctx0, cache=dcache)
    trim_draft_cache(dcache, 16)
    ctx = (torch.randn(1, 5, 5 * H, generator=g, device=dev)).to(torch.bfloat16)
    noise = target_model.weights.embed_rows(torch.tensor([7] + [args.dflash_config["mask_token_id"]] * 15,
                                                         device=dev))[None]
    adapter = Qwen3TargetAdapter()
    base_off = dcache.offset

    def one_draft():
        for lc in dcache:
            lc.offset = base_off
        h = draft(noise_embedding=noise, target_hidden=ctx, cache=dcache)
        trim_draft_cache(dcache, 16)
        return h

    def timed(fn, n):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            out = fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n * 1e3, out

    draft_ms, dh = timed(one_draft, steps)
    lm_ms, logits = timed(lambda: adapter.lm_head_logits(target_model, dh[:, 1:, :]), steps)
    x = logits[0].contiguous()
    st = eng.stream_handle()
    tb_ms, _ = timed(lambda: eng.launch_tree_build(x, budget, 4, 7, P, st), steps * 4)
    host_ms, _ = timed(lambda: build_dtree_tree(x, budget, topk=4), steps)

    def full():
        h = one_draft()
        lg = adapter.lm_head_logits(target_model, h[:, 1:, :])
        return eng.verify_from_logits(cache, lg[0], budget, 4, 7, commit=False)

    step_ms, _ = timed(full, steps)
    del draft, dcache
    return {"workload": "DTree decode step pieces around the verify (Qwen3-4B target, DFlash drafter sized for it, "
                        f"prefix {P}, budget {budget}, top-4)",
            "draft_call_ms": round(draft_ms, 4), "lm_head_15_rows_ms": round(lm_ms, 4),
            "tree_build_device_ms": round(tb_ms, 4), "tree_build_host_ms": round(host_ms, 4),
            "whole_step_ms": round(step_ms, 4), "steps": steps}


def run_workload(model: str, quant: str, P: int, budget: int, steps: int, warmup: int, kernel_reps: int = 0,
                 with_cpu: bool = False, with_decode: bool = False, with_prefill: bool = False,
                 max_past: int | None = None) -> dict:
    """Builds the random-init model, prefills P tokens, builds the seeded tree
    (acceptance pass at p = 0.85 on the device argmax) and times `steps`
    verify steps (descriptor upload, graph replay, result read back) after
    `warmup` untimed ones. Optionally times every kernel class and the CPU
    restatement. Frees the model before returning."""
    import torch

    from dtree_hip import Qwen35TreeEngine, Qwen35Weights, Qwen3TreeModel, Qwen3Weights
    from dtree_hip.config import QWEN3_4B, QWEN35_4B, QWEN35_9B
    from dtree_hip.synthetic import acceptance_rewrite, make_tree, random_prefix

    dev = torch.device("cuda:0")
    hybrid = model.startswith("qwen35")
    cfg = {"qwen3-4b": QWEN3_4B, "qwen35-4b": QWEN35_4B, "qwen35-9b": QWEN35_9B}[model]
    max_nodes = budget + 1
    max_past = P + 64 if max_past is None else max_past
    t0 = time.time()
    if hybrid:
        w = Qwen35Weights.random(cfg, seed=0, device=dev, quant=quant)
        eng = Qwen35TreeEngine(cfg, w, max_past=max_past, layer_ids=[1, 9, 17, 25, 30], max_nodes=max_nodes)
    else:
        if quant == "q4":
            w = Qwen3Weights.random_q4(cfg, seed=0, device=dev)
        else:
            w = Qwen3Weights.random(cfg, seed=0, device=dev)
        tmodel = Qwen3TreeModel(cfg, w, max_past=max_past, layer_ids=[1, 9, 17, 25, 33], max_nodes=max_nodes)
        eng = tmodel.engine
    cache = eng.new_cache()
    prefix = random_prefix(P, cfg.vocab_size, seed=1)
    eng.prefill(cache, prefix)
    torch.cuda.synchronize()
    log(f"[bench] {model} {quant} P={P}: weights + prefill {time.time() - t0:.1f}s")
    st = eng.stream_handle()
    tree = make_tree(prefix[-1], cfg.vocab_size, budget=budget, depth=15, topk=4, seed=2)

    def argmax_at(tr):
        eng.set_step(tr.tokens, tr.positions(P), tr.parents, P)
        eng.launch_forward(cache, st)
        eng.launch_lm_head(st)
        eng.launch_walk(st)
        return eng.read_result().posterior

    acceptance_rewrite(tree, argmax_at, p=0.85, seed=3)
    L = tree.size
    pos, par, toks = tree.positions(P), tree.parents, tree.tokens
    log(f"[bench] tree L={L} max depth={max(tree.depths)}")
    # commit=False: every step verifies the same tree against the same
    # committed state (the hybrid's commit writes the cache's spare state
    # buffers), so each replay is the seeded step and accepts the same path.
    first = eng.verify(cache, toks, pos, par, use_graph=True, commit=False)
    for _ in range(max(warmup - 1, 0)):
        res = eng.verify(cache, toks, pos, par, use_graph=True, commit=False)
        if res.accepted != first.accepted:
            raise RuntimeError(f"warmup step accepted {res.accepted}, the first step {first.accepted}")
    torch.cuda.synchronize()
    log(f"[bench] warmup done, accepted={first.accepted}")
    results = []
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for _ in range(steps):
        results.append(eng.verify(cache, toks, pos, par, use_graph=True, commit=False))
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    for i, r in enumerate(results):
        if r.accepted != first.accepted or r.bonus_token != first.bonus_token:
            raise RuntimeError(f"timed step {i} accepted {r.accepted} (bonus {r.bonus_token}), the first step "
                               f"{first.accepted} (bonus {first.bonus_token})")
    res = results[-1]
    accepted_lens = [len(r.accepted) for r in results]
    ms = elapsed / steps * 1e3
    ab = algorithmic_bytes35(cfg, P, L, quant) if hybrid else algorithmic_bytes(cfg, P, L, quant)
    gbps = ab["total"] / (ms * 1e-3) / 1e9
    mean_acc = sum(accepted_lens) / len(accepted_lens)
    log(f"[bench] {model} {quant}: {ms:.3f} ms/step  {steps / elapsed:.1f} steps/s  {gbps:.0f} GB/s")
    out = {"cfg": cfg, "P": P, "L": L, "ms": ms, "steps_per_s": steps / elapsed, "gbps": gbps,
           "algorithmic_bytes": ab["total"], "mean_accepted": mean_acc, "accepted": res.accepted}
    if kernel_reps:
        out["kernels"] = (time_kernels35 if hybrid else time_kernels)(eng, cfg, w, cache, st, P, L, kernel_reps,
                                                                      quant)
    if (with_decode and quant == "bf16") or with_prefill:
        t0 = time.time()
        label = f"{MODEL_NAMES[model]} {'bf16' if quant == 'bf16' else 'q4 group-64'}"
        out["prefill"] = prefill_bench(eng, P, reps=1 if P > 4096 else 3, hybrid=hybrid, label=label)
        log(f"[bench] prefill {out['prefill']} ({time.time() - t0:.1f}s)")
    if with_decode and not hybrid:
        t0 = time.time()
        out["decode"] = decode_step_bench(tmodel, cache, P, budget)
        log(f"[bench] decode step pieces {out['decode']} ({time.time() - t0:.1f}s)")
    if with_cpu:
        t0 = time.time()
        out["cpu"] = (cpu_baseline35 if hybrid else cpu_baseline)(cfg, w, cache, tree, P)
        log(f"[bench] cpu baseline {out['cpu']['value']:.3f} steps/s ({time.time() - t0:.1f}s)")
    eng.release_graphs()
    del eng, w, cache
    if not hybrid:
        del tmodel
    import gc

    gc.collect()
    torch.cuda.empty_cache()
    return out


def lazy_hop_bench(P: int = 2048, hops: int = CONFIG_STEPS, warmup: int = CONFIG_WARMUP) -> dict:
    """The reference's default Qwen3.5 verifier (lazy_follow_tree_exact,
    dtree_runtime.py:211-290) walks the tree one token at a time; one hop is
    text_model.forward_dflash over one token (every layer, committing the
    GatedDeltaNet state and the attention K/V), the LM-head argmax and the
    host read of the token. Timed here on the Qwen3.5-4B-shaped hybrid with q4
    group-64 weights after a P-token prefill, hop after hop as the walk runs
    them (the prefix grows by one per hop)."""
    import torch

    from dtree_hip.adapters import Qwen35TargetAdapter, Qwen35TreeModel
    from dtree_hip.config import QWEN35_4B
    from dtree_hip.synthetic import random_prefix
    from dtree_hip.weights import Qwen35Weights

    dev = torch.device("cuda:0")
    cfg = QWEN35_4B
    layer_ids = [1, 9, 17, 25, 30]
    w = Qwen35Weights.random(cfg, seed=0, device=dev, quant="q4")
    model = Qwen35TreeModel(cfg, w, max_past=P + hops + warmup + 64, layer_ids=layer_ids)
    adapter = Qwen35TargetAdapter()
    cache = adapter.make_cache(model)
    model.engine.prefill(cache, random_prefix(P, cfg.vocab_size, seed=1))
    text = model.model
    tok = 7

    def hop(t):
        norm_hidden, _ = text.forward_dflash(torch.tensor([[t]]), cache, layer_ids)
        return int(adapter.lm_head_argmax(model, norm_hidden).reshape(-1)[0].item())

    for _ in range(warmup):
        tok = hop(tok)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(hops):
        tok = hop(tok)
    ms = (time.perf_counter() - t0) / hops * 1e3
    model.engine.release_graphs()
    del model, w, cache
    torch.cuda.empty_cache()
    return {"workload": f"Qwen3.5-4B-shaped hybrid q4 group-64, lazy exact verifier: one single-token hop "
                        f"(forward_dflash over 1 token with commit, LM-head argmax, host read) at prefix {P}",
            "ms_per_hop": round(ms, 4), "hops": hops,
            "reference_m2max_ms_per_hop": 14.38}


def dflash_block_bench(P: int = 1024, block: int = 16, steps: int = 30, warmup: int = 5) -> dict:
    """DFlash linear verification in the parallel-greedy-argmax mode
    (runtime.py:302-354): a drafted block of 16 tokens verified in one
    forward as a chain, LM-head argmax of every row, the longest matching
    prefix and its commit, on the Qwen3-4B-shaped bf16 target at prefix P.
    Each timed call starts from the same prefix (the offset is reset; the
    rows past it are rewritten by the next call)."""
    import torch

    from dtree_hip import Qwen3TreeModel, Qwen3Weights
    from dtree_hip.adapters import LoadedTargetModel, Qwen3TargetAdapter
    from dtree_hip.config import QWEN3_4B
    from dtree_hip.runtime import verify_block_parallel_greedy_argmax
    from dtree_hip.synthetic import random_prefix

    dev = torch.device("cuda:0")
    cfg = QWEN3_4B
    layer_ids = [1, 9, 17, 25, 33]
    w = Qwen3Weights.random(cfg, seed=0, device=dev)
    model = Qwen3TreeModel(cfg, w, max_past=P + 64, layer_ids=layer_ids, max_nodes=block)
    target = LoadedTargetModel(requested_model="random:qwen3-4b", resolved_model_path=None, model=model,
                               tokenizer=None, adapter=Qwen3TargetAdapter())
    cache = target.make_cache()
    model.engine.prefill(cache, random_prefix(P, cfg.vocab_size, seed=1))
    blk = random_prefix(block, cfg.vocab_size, seed=9)
    acc = []

    def one():
        cache.offset = P
        n, post, _ = verify_block_parallel_greedy_argmax(target, cache, blk, block, 0.0, layer_ids)
        acc.append(n)

    for _ in range(warmup):
        one()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        one()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps * 1e3
    model.engine.release_graphs()
    del model, w, cache, target
    torch.cuda.empty_cache()
    return {"workload": f"DFlash parallel-greedy-argmax block verify (Qwen3-4B bf16 target, {block}-token block as a "
                        f"chain, LM-head argmax, prefix match, commit) at prefix {P}",
            "ms_per_step": round(ms, 4), "steps": steps, "accepted_last": acc[-1]}


def attention_layer_bench(P: int = 512, sets: int = 128, reps: int = 1280) -> dict:
    """One Qwen3-4B-shaped tree-attention layer (32 query / 8 KV heads,
    head_dim 128, bf16 paged KV prefix of P positions ~ N(0, 0.5), 25-node
    seeded tree), launched back to back over `sets` distinct layer-sized
    buffer sets (their K/V prefixes together exceed the 256 MB MALL), timed
    with HIP events on the launch stream."""
    import ctypes as C

    import numpy as np
    import torch

    from dtree_hip import _native as N
    from dtree_hip.cache import PagedKVCache
    from dtree_hip.engine import ancestor_bitsets
    from dtree_hip.synthetic import make_tree

    dev = torch.device("cuda:0")
    lib = N.lib()
    Hq, Hkv, D, MP = 32, 8, 128, 32
    tree = make_tree(7, 151936, budget=24, depth=15, topk=4, seed=2)
    L = tree.size
    g = torch.Generator(device=dev).manual_seed(4)
    cache = PagedKVCache(sets, Hkv, D, P + MP, device=dev)
    cache.k_pages.normal_(0.0, 0.5, generator=g)
    cache.v_pages.normal_(0.0, 0.5, generator=g)
    qkv = torch.randn(sets, MP, (Hq + 2 * Hkv) * D, generator=g, device=dev)
    qn = torch.ones(D, dtype=torch.bfloat16, device=dev)
    d = N.StepDesc()
    d.past_length, d.num_nodes = P, L
    anc = ancestor_bitsets(tree.parents)
    for i in range(L):
        d.tokens[i], d.positions[i], d.parents[i] = tree.tokens[i], tree.positions(P)[i], tree.parents[i]
        for wd in range(N.MASK_WORDS):
            d.ancestors[i][wd] = int(anc[i, wd])
    N.check(lib.dtree_step_desc_validate(C.byref(d), MP, P, 151936), "attention bench descriptor")
    desc = torch.frombuffer(bytearray(bytes(d)), dtype=torch.uint8).to(dev)
    cos = torch.zeros(MP, D // 2, device=dev)
    sin = torch.zeros(MP, D // 2, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    N.check(lib.dtree_rope_table(desc.data_ptr(), MP, D, 1e6, cos.data_ptr(), sin.data_ptr(), st), "rope table")
    out = torch.zeros(2, MP, Hq * D, dtype=torch.float16, device=dev)
    ws = torch.zeros(lib.dtree_attention_workspace_bytes(Hq, D, P, MP), dtype=torch.uint8, device=dev)
    args = []
    for s_ in range(sets):
        a = N.AttnArgs()
        a.qkv = qkv[s_].data_ptr(); a.ld_qkv = qkv.shape[-1]
        a.q_norm = qn.data_ptr(); a.k_norm = qn.data_ptr(); a.eps = 1e-6
        a.rope_cos = cos.data_ptr(); a.rope_sin = sin.data_ptr()
        a.k_pages = cache.k_ptr(s_); a.v_pages = cache.v_ptr(s_); a.page_table = cache.page_table.data_ptr()
        a.desc = desc.data_ptr()
        a.out = out[0].data_ptr(); a.out_lo = None; a.ld_out = Hq * D; a.out_layout = N.W_TILED_F16
        a.num_heads = Hq; a.num_kv_heads = Hkv; a.head_dim = D; a.rows_padded = MP; a.scale = D ** -0.5
        a.max_past_length = P; a.write_cache = 0
        a.workspace = ws.data_ptr(); a.workspace_bytes = ws.numel()
        args.append(a)
    refs = [C.byref(a) for a in args]
    for r in range(sets):
        N.check(lib.dtree_tree_attention(refs[r], st), "attention")
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for r in range(reps):
        lib.dtree_tree_attention(refs[r % sets], st)
    e1.record()
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    # algorithmic bytes: Q (L x 32 heads x 128, bf16), K/V prefix + tree (P + L keys x 8 heads x 128 x 2),
    # ancestor bitsets (4 B per node), output (L x 4096 bf16)
    nbytes = L * Hq * D * 2 + 2 * Hkv * (P + L) * D * 2 + 4 * L + L * Hq * D * 2
    del cache, qkv, out, ws
    torch.cuda.empty_cache()
    return {"workload": f"one Qwen3-4B tree-attention layer, prefix {P}, {L}-node tree, 32/8 heads, head_dim 128",
            "avg_launch_us": round(us, 3), "algorithmic_bytes_per_launch": int(nbytes),
            "achieved_gbps": round(nbytes / (us * 1e-6) / 1e9, 1), "buffer_sets": sets, "launches": reps}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--model", choices=["qwen3-4b", "qwen35-4b", "qwen35-9b"], default="qwen3-4b",
                    help="qwen35-4b / qwen35-9b: the Qwen3.5-shaped GatedDeltaNet / attention hybrids")
    ap.add_argument("--prefix", type=int, default=None,
                    help="prefix tokens (default 1024; 2048 for qwen35-4b, 8192 for qwen35-9b)")
    ap.add_argument("--budget", type=int, default=None, help="draft budget (default 24; 64 for qwen35-9b)")
    ap.add_argument("--quant", choices=["bf16", "q4"], default=None,
                    help="q4: every linear layer and the tied LM head in 4-bit affine groups of 64 "
                         "(default bf16; q4 for qwen35-9b)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other workloads' lines (single attention layer, q4, Qwen3.5 hybrids)")
    ap.add_argument("--kernel-reps", type=int, default=108)
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 5 device copies of MIB MiB (the known-size kernel that scales the "
                         "FETCH_SIZE / WRITE_SIZE counters) and exit")
    a = ap.parse_args()
    if a.copy_probe:
        copy_probe(a.copy_probe)
        return
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (the verify step is not sharded across GPUs); got --gpus {a.gpus}",
              file=sys.stderr)
        sys.exit(2)

    hybrid = a.model.startswith("qwen35")
    big = a.model == "qwen35-9b"
    P = a.prefix if a.prefix is not None else {"qwen3-4b": 1024, "qwen35-4b": 2048, "qwen35-9b": 8192}[a.model]
    if a.budget is None:
        a.budget = 64 if big else 24
    if a.quant is None:
        a.quant = "q4" if big else "bf16"
    r = run_workload(a.model, a.quant, P, a.budget, a.steps, a.warmup, kernel_reps=a.kernel_reps,
                     with_cpu=not a.no_cpu_baseline, with_decode=not a.no_configs)
    cfg, L, ms, gbps = r["cfg"], r["L"], r["ms"], r["gbps"]
    kernels = r["kernels"]
    for name, kd in kernels.items():
        log(f"[bench] {name:10s} {kd['avg_launch_us']:7.1f} us/launch x {kd['launches_per_step']:2d}  "
            f"{kd['achieved_gbps']:6.0f} GB/s  ({kd['kernel']})")
    dom = max(kernels, key=lambda k: kernels[k]["avg_launch_us"] * kernels[k]["launches_per_step"])
    kd = kernels[dom]
    traffic = None
    tag = ("_qwen35" if hybrid else "") + ("_q4" if a.quant == "q4" else "")
    tf = ROOT / "profiles" / f"{dom}{tag}_traffic.json"
    if tf.exists():
        try:
            traffic = json.loads(tf.read_text()).get("hbm_bytes_per_launch")
        except Exception:
            traffic = None

    configs = None
    if not a.no_configs and a.model == "qwen3-4b" and a.quant == "bf16" and P == 1024 and a.budget == 24:
        configs = {}
        if "decode" in r:
            configs["decode_step_qwen3_4b_p1024"] = r["decode"]
        if "prefill" in r:
            configs["prefill_qwen3_4b_p1024"] = r["prefill"]
        t0 = time.time()
        configs["attention_layer_p512"] = attention_layer_bench(P=512)
        log(f"[bench] attention layer P=512: {configs['attention_layer_p512']}")
        # the same step on an engine sized for the generator's default max_past
        rr = run_workload("qwen3-4b", "bf16", 1024, 24, steps=CONFIG_STEPS, warmup=CONFIG_WARMUP, max_past=4096,
                          kernel_reps=54)
        configs["qwen3_4b_bf16_p1024_max_past_4096"] = {
            "workload": "Qwen3-4B bf16 tree-verify step, prefix 1024, 25-node tree, engine and cache sized for "
                        "max_past 4096 (DFlashGenerator's default)",
            "ms_per_step": round(rr["ms"], 4), "steps_per_s": round(rr["steps_per_s"], 3),
            "attention": {k: (round(v, 2) if isinstance(v, float) else v)
                          for k, v in rr["kernels"]["attention"].items()}, "steps": CONFIG_STEPS}
        log(f"[bench] max_past 4096: {configs['qwen3_4b_bf16_p1024_max_past_4096']}")
        configs["dflash_block_verify_qwen3_4b_p1024"] = dflash_block_bench()
        log(f"[bench] dflash block verify: {configs['dflash_block_verify_qwen3_4b_p1024']}")
        for key, (m, q, pp, bb) in {"qwen3_4b_q4_p1024": ("qwen3-4b", "q4", 1024, 24),
                                    "qwen35_4b_bf16_p2048": ("qwen35-4b", "bf16", 2048, 24),
                                    "qwen35_9b_q4_p8192_budget64": ("qwen35-9b", "q4", 8192, 64)}.items():
            rr = run_workload(m, q, pp, bb, steps=CONFIG_STEPS, warmup=CONFIG_WARMUP, with_prefill=True)
            configs["prefill_" + key.replace("_budget64", "")] = rr["prefill"]
            configs[key] = {"workload": f"{MODEL_NAMES[m]} {'bf16' if q == 'bf16' else 'q4 group-64'} tree-verify "
                                        f"step, prefix {pp}, {rr['L']}-node tree",
                            "ms_per_step": round(rr["ms"], 4), "steps_per_s": round(rr["steps_per_s"], 3),
                            "hbm_gbps": round(rr["gbps"], 1), "hbm_frac_of_peak": round(rr["gbps"] / HBM_PEAK_GBPS, 4),
                            "algorithmic_bytes_per_step": rr["algorithmic_bytes"],
                            "tokens_per_s": round(rr["steps_per_s"] * rr["mean_accepted"], 2),
                            "mean_accepted": rr["mean_accepted"], "accepted": rr["accepted"], "steps": CONFIG_STEPS}
        configs["lazy_hop_qwen35_4b_q4_p2048"] = lazy_hop_bench()
        log(f"[bench] lazy hop: {configs['lazy_hop_qwen35_4b_q4_p2048']}")
        log(f"[bench] other workloads {time.time() - t0:.1f}s")

    model_name = MODEL_NAMES[a.model]
    qname = "bf16" if a.quant == "bf16" else "q4 group-64"
    if hybrid:
        workload = (f"{model_name} {qname} tree-verify step (24 GatedDeltaNet + 8 gated attention layers, "
                    "LM-head argmax, walk, KV compaction, GatedDeltaNet commit)")
    else:
        workload = f"{model_name} {qname} tree-verify step (36 layers, LM-head argmax, walk, compaction)"
    out = {
        "metric": f"tree-verify steps/s + HBM GB/s (% of peak), {a.budget}-node tree, {model_name} {qname}",
        "value": round(r["steps_per_s"], 3),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if a.quant == "bf16" else "q4g64 weights, bf16 activations",
        "data": ("synthetic: random-init weights N(0,0.02), uniform prefix ids, seeded Gumbel draft tree"
                 if a.quant == "bf16" else
                 "synthetic: q4 nibbles uniform 0..15, scales |N(0,0.02)|*8, biases N(0,0.01), uniform prefix ids, "
                 "seeded Gumbel draft tree"),
        "config": {"workload": workload,
                   "prefix": P, "tree_nodes": L, "draft_budget": a.budget,
                   "layers": cfg.num_hidden_layers, "hidden": cfg.hidden_size, "vocab": cfg.vocab_size},
        "hbm_gbps": round(gbps, 1),
        "hbm_frac_of_peak": round(gbps / HBM_PEAK_GBPS, 4),
        "algorithmic_bytes_per_step": r["algorithmic_bytes"],
        "tokens_per_s": round(r["steps_per_s"] * r["mean_accepted"], 2),
        "mean_accepted": r["mean_accepted"],
        "roofline": {"kernel": f"{kd['kernel']} ({dom})", "bound": "hbm",
                     "achieved": round(kd["achieved_gbps"], 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(kd["achieved_gbps"] / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "avg_launch_us": round(kd["avg_launch_us"], 2),
                     "algorithmic_bytes_per_launch": kd["algorithmic_bytes_per_launch"]},
        "kernels": {k: {kk: (round(vv, 2) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in kernels.items()},
        "cpu_baseline": r.get("cpu"),
        "configs": configs,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
