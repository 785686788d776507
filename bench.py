"""Tree-verify step benchmark on one MI355X.

Workload (default): one DTree verify step of a random-init Qwen3-4B-shaped bf16
model (36 layers, hidden 2560, FFN 9728, GQA 32/8, head_dim 128, vocab
151936) at a 1024-token prefix with a 24-node draft tree (25 rows incl. the
root): every layer, LM-head argmax per node, greedy accept walk and KV
compaction, replayed as one HIP graph. Inputs (weights, KV prefix, tree) are
resident in HBM before timing; each timed step uploads the 4.6 KB step
descriptor, replays the graph and reads the walk result back.

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


def log(*a):
    print(*a, file=sys.stderr, flush=True)


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


def cpu_baseline(cfg, weights, cache, tree, P, sample_layers=4, min_seconds=15.0):
    """The fp32 numpy oracle of the same verify step, timed on the host cores on
    a bounded sample: `sample_layers` of the 36 tree blocks (repeated) and a
    quarter of the LM head, scaled linearly to the whole step."""
    import numpy as np

    from oracle import qwen3 as oq
    from oracle import tree as otree

    try:
        from threadpoolctl import threadpool_info
        cores = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        cores = os.cpu_count() or 1
    ocfg = oq.Qwen3Config(hidden=cfg.hidden_size, layers=cfg.num_hidden_layers, ffn=cfg.intermediate_size,
                          heads=cfg.num_attention_heads, kv_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                          vocab=cfg.vocab_size, eps=cfg.rms_norm_eps, rope_base=cfg.rope_theta)
    acc = weights.host_accessor()
    names = ("input_norm", "q", "k", "v", "q_norm", "k_norm", "o", "post_norm", "gate", "up", "down")
    W = {(li, n): oq.bf16_to_f32(acc(li, n)) for li in range(sample_layers) for n in names}
    orc = oq.OracleQwen3(ocfg, lambda li, n: W[(li, n)])
    ids, pos, mask = otree.compile_tree(tree.tokens[0], P, tree.tokens[1:], tree.depths[1:], tree.visibility, P)
    kp = [cache.logical_keys(li, P).float().cpu().numpy() for li in range(sample_layers)]
    vp = [cache.logical_values(li, P).float().cpu().numpy() for li in range(sample_layers)]
    x0 = oq.bf16_to_f32(acc(None, "embed")[ids])
    per_layer = []
    t_start = time.perf_counter()
    while True:
        x = x0
        for li in range(sample_layers):
            t0 = time.perf_counter()
            x, _, _ = orc.layer_forward(li, x, kp[li], vp[li], pos, mask)
            per_layer.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > min_seconds or len(per_layer) >= 400 * sample_layers:
            break
    E = acc(None, "embed")
    q = E.shape[0] // 4
    Eq = oq.bf16_to_f32(E[:q])
    h = oq.rms_norm(x, np.ones(cfg.hidden_size, np.float32), cfg.rms_norm_eps)
    lm_t = []
    for _ in range(3):
        t0 = time.perf_counter()
        np.argmax(h @ Eq.T, axis=-1)
        lm_t.append(time.perf_counter() - t0)
    t_layer = float(np.median(per_layer))
    t_step = t_layer * cfg.num_hidden_layers + float(np.median(lm_t)) * (E.shape[0] / q)
    return {"value": 1.0 / t_step, "unit": "steps/s", "cores": int(cores), "kind": "port",
            "sample": (f"fp32 numpy oracle: {sample_layers} of {cfg.num_hidden_layers} tree blocks x "
                       f"{len(per_layer) // sample_layers} passes (median {t_layer * 1e3:.1f} ms/block) + 1/4 of "
                       f"the LM head, scaled linearly to one step ({t_step:.2f} s)")}


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
        for r in range(nl):
            launch(r)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for r in range(reps):
            launch(r % nl)
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    refs = {k: [C.byref(args[li][k]) for li in range(nl)] for k in ("qkv", "o", "gu", "down")}
    us = {k: timed(lambda r, k=k: gemm(refs[k][r], st)) for k in refs}
    us["attention"] = timed(lambda r: eng._attention(r, cache, st))
    us["lm_head"] = timed(lambda r: eng.launch_lm_head(st))
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

    out["qkv_gemm"] = entry(f"sk_gemm_kernel<true, 0, {q4}>", nl, us["qkv"], b["qkv"])
    out["attention"] = entry("tree_attn_kernel<128>", nl, us["attention"], b["attention"])
    # o_proj and down_proj share one instantiation (residual epilogue): its
    # average launch is the mean of the two shapes, as the profiler reports.
    out["residual_gemm"] = entry(f"sk_gemm_kernel<true, 1, {q4}>", 2 * nl, (us["o"] + us["down"]) / 2,
                                 (b["o"] + b["down"]) / 2)
    out["gate_up_gemm"] = entry(f"sk_gemm_kernel<true, 2, {q4}>", nl, us["gu"], b["gu"])
    out["lm_head"] = entry(f"lmhead_kernel<1, 2, 2, true, true, {q4}>", 1, us["lm_head"], b["lm_head"])
    out["residual_gemm"]["shapes_us"] = {"o_proj": us["o"], "down_proj": us["down"]}
    return out


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--prefix", type=int, default=1024)
    ap.add_argument("--budget", type=int, default=24)
    ap.add_argument("--quant", choices=["bf16", "q4"], default="bf16",
                    help="q4: every linear layer and the tied LM head in 4-bit affine groups of 64")
    ap.add_argument("--no-cpu-baseline", action="store_true")
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

    import torch

    from dtree_hip import Qwen3TreeModel, Qwen3Weights
    from dtree_hip import _native as N
    from dtree_hip.config import QWEN3_4B
    from dtree_hip.synthetic import acceptance_rewrite, make_tree, random_prefix

    dev = torch.device("cuda:0")
    cfg = QWEN3_4B
    P = a.prefix
    t0 = time.time()
    if a.quant == "q4":
        w = Qwen3Weights.random_q4(cfg, seed=0, device=dev)
    else:
        w = Qwen3Weights.random(cfg, seed=0, device=dev)
    model = Qwen3TreeModel(cfg, w, max_past=P + 64, layer_ids=[1, 9, 17, 25, 33])
    eng = model.engine
    cache = eng.new_cache()
    prefix = random_prefix(P, cfg.vocab_size, seed=1)
    eng.prefill(cache, prefix)
    torch.cuda.synchronize()
    log(f"[bench] weights + prefill {time.time() - t0:.1f}s")
    st = eng.stream_handle()
    tree = make_tree(prefix[-1], cfg.vocab_size, budget=a.budget, depth=15, topk=4, seed=2)

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

    for _ in range(a.warmup):
        res = eng.verify(cache, toks, pos, par, use_graph=True, commit=False)
    torch.cuda.synchronize()
    log(f"[bench] warmup done, accepted={res.accepted}")

    accepted_lens = []
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for _ in range(a.steps):
        res = eng.verify(cache, toks, pos, par, use_graph=True, commit=False)
        accepted_lens.append(len(res.accepted))
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    ms = elapsed / a.steps * 1e3
    steps_per_s = a.steps / elapsed
    ab = algorithmic_bytes(cfg, P, L, a.quant)
    gbps = ab["total"] / (ms * 1e-3) / 1e9
    log(f"[bench] {ms:.3f} ms/step  {steps_per_s:.1f} steps/s  {gbps:.0f} GB/s")

    kernels = time_kernels(eng, cfg, w, cache, st, P, L, a.kernel_reps, a.quant)
    for name, kd in kernels.items():
        log(f"[bench] {name:10s} {kd['avg_launch_us']:7.1f} us/launch x {kd['launches_per_step']:2d}  "
            f"{kd['achieved_gbps']:6.0f} GB/s  ({kd['kernel']})")
    dom = max(kernels, key=lambda k: kernels[k]["avg_launch_us"] * kernels[k]["launches_per_step"])
    kd = kernels[dom]
    traffic = None
    tf = ROOT / "profiles" / (f"{dom}_traffic.json" if a.quant == "bf16" else f"{dom}_q4_traffic.json")
    if tf.exists():
        try:
            traffic = json.loads(tf.read_text()).get("hbm_bytes_per_launch")
        except Exception:
            traffic = None

    cpu = None
    if not a.no_cpu_baseline:
        t0 = time.time()
        cpu = cpu_baseline(cfg, w, cache, tree, P)
        log(f"[bench] cpu baseline {cpu['value']:.3f} steps/s ({time.time() - t0:.1f}s)")

    mean_acc = sum(accepted_lens) / len(accepted_lens)
    out = {
        "metric": ("tree-verify steps/s + HBM GB/s (% of peak), 24-node tree, Qwen3-4B bf16" if a.quant == "bf16"
                   else "tree-verify steps/s + HBM GB/s (% of peak), 24-node tree, Qwen3-4B q4 group-64"),
        "value": round(steps_per_s, 3),
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
        "config": {"workload": (f"Qwen3-4B-shaped {'bf16' if a.quant == 'bf16' else 'q4 group-64'} tree-verify step "
                                "(36 layers, LM-head argmax, walk, compaction)"),
                   "prefix": P, "tree_nodes": L, "draft_budget": a.budget,
                   "layers": cfg.num_hidden_layers, "hidden": cfg.hidden_size, "vocab": cfg.vocab_size},
        "hbm_gbps": round(gbps, 1),
        "hbm_frac_of_peak": round(gbps / HBM_PEAK_GBPS, 4),
        "algorithmic_bytes_per_step": ab["total"],
        "tokens_per_s": round(steps_per_s * mean_acc, 2),
        "mean_accepted": mean_acc,
        "roofline": {"kernel": f"{kd['kernel']} ({dom})", "bound": "hbm",
                     "achieved": round(kd["achieved_gbps"], 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(kd["achieved_gbps"] / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "avg_launch_us": round(kd["avg_launch_us"], 2),
                     "algorithmic_bytes_per_launch": kd["algorithmic_bytes_per_launch"]},
        "kernels": {k: {kk: (round(vv, 2) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in kernels.items()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
