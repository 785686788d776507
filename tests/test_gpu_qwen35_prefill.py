"""Prompt prefill of the Qwen3.5 hybrid on the long-M path (forward_dflash over
the prompt, custom_qwen35_model.py:961-1097, reached through
Qwen35TargetAdapter.forward_with_hidden_states, adapters.py:290-307) against
the oracle.

* dtree_gemm_long with a 64-column last tile (n % 128 == 64, the in_proj
  shape; fp32 store only) against a float64 product.
* dtree_gdn_layer_chain (one GatedDeltaNet layer over a prompt chain that
  continues a committed window and state, GatedDeltaNet.__call__,
  custom_qwen35_model.py:823-878) against the oracle's conv, q/k/v/g/beta,
  recurrence, gated norm and commit, for chains shorter and longer than the
  conv window.
* Qwen35TreeEngine.prefill_long on the tiny hybrid against the oracle's
  causal forward + commit: every GatedDeltaNet layer's committed window and
  state, every attention layer's cached K/V rows, the verifier hidden rows
  and the last position's logits (2e-2 bar); one segment, several segments,
  a prompt continuing a prefix the chain path wrote, q4 group-64 weights,
  and the adapter taking the long path.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from oracle import gdn as ogdn
from oracle import qwen35 as o35

from dtree_hip import Qwen35TreeEngine, Qwen35Weights, tiny_qwen35
from dtree_hip import _native as N
from dtree_hip.adapters import load_target_model
from dtree_hip.synthetic import random_prefix
from dtree_hip.weights import tile_weight
from gpu_util import bf16_f32
from test_gpu_qwen35 import _oracle_cfg

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _stream():
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("rows,L,n,k", [(128, 100, 1600, 512), (256, 200, 320, 256)])
@pytest.mark.parametrize("lo", [False, True])
def test_gemm_long_64_column_tail(gpu_device, rows, L, n, k, lo):
    g = np.random.default_rng(n + rows + lo)
    dev = gpu_device
    xf = np.zeros((rows, k), np.float32)
    xf[:L] = g.standard_normal((L, k))
    hi = torch.from_numpy(xf).to(torch.bfloat16)
    lo_t = (torch.from_numpy(xf) - hi.float()).to(torch.bfloat16)
    xin = hi.double().numpy() + (lo_t.double().numpy() if lo else 0.0)
    w = torch.from_numpy(g.standard_normal((n, k)).astype(np.float32) * 0.05).to(torch.bfloat16)
    xt, xlt, wt = tile_weight(hi.to(dev)), tile_weight(lo_t.to(dev)), tile_weight(w.to(dev))
    ss = torch.from_numpy(np.abs(g.standard_normal((rows // 32, k // 32, 32))).astype(np.float32) + 0.5).to(dev)
    out = torch.full((rows, n + 64), 7.0, device=dev)  # the column past n must stay untouched
    a = N.GemmArgs()
    a.x = xt.data_ptr(); a.x_lo = xlt.data_ptr() if lo else None
    a.x_layout = a.w_layout = N.W_TILED; a.ldx = k; a.rows_padded = rows
    a.w = wt.data_ptr(); a.n = n; a.k = k
    a.ss_in = ss.data_ptr(); a.ss_tiles = k // 32; a.norm_dim = k; a.eps = 1e-6
    a.out_f32 = out.data_ptr(); a.ld_out_f32 = n + 64
    a.epilogue = N.EPI_STORE_F32
    N.check(N.lib().dtree_gemm_long(C.byref(a), _stream()), "gemm_long")
    torch.cuda.synchronize()
    rs = 1.0 / np.sqrt(ss.cpu().numpy().transpose(0, 2, 1).reshape(rows, k // 32).sum(1) / k + 1e-6)
    ref = (xin @ w.double().numpy().T) * rs[:, None]
    got = out.cpu().numpy()
    assert np.abs(got[:, :n] - ref).max() <= 2e-4 * max(1.0, np.abs(ref).max())
    assert np.all(got[:, n:] == 7.0)
    # the other epilogues keep n % 128 == 0
    a.epilogue = N.EPI_RESIDUAL
    assert N.lib().dtree_gemm_long(C.byref(a), _stream()) != 0


def _chain_case(T, seed, dev):
    cfg = tiny_qwen35()
    w = Qwen35Weights.random(cfg, seed=0, device=dev, norm_jitter=0.1)
    orc = o35.OracleQwen35(_oracle_cfg(cfg), w.host_accessor())
    li = cfg.linear_layers[0]
    g = np.random.default_rng(seed)
    Hv, Dv = cfg.linear_num_value_heads, cfg.linear_value_head_dim
    Cc = 2 * cfg.key_dim + cfg.value_dim
    keep = cfg.linear_conv_kernel_dim - 1
    rows = 32 * ((T + 31) // 32)
    proj = np.zeros((rows, cfg.in_proj_dim), np.float32)
    proj[:T] = g.standard_normal((T, cfg.in_proj_dim)).astype(np.float32)
    window = (0.5 * g.standard_normal((keep, Cc))).astype(np.float32)
    state = (0.1 * g.standard_normal((Hv, Dv, cfg.linear_key_head_dim))).astype(np.float32)
    return cfg, w, orc, li, proj, window, state, rows


@pytest.mark.parametrize("T", [1, 2, 37, 300])
def test_gdn_layer_chain_matches_oracle(gpu_device, T):
    dev = gpu_device
    cfg, w, orc, li, proj, window, state, rows = _chain_case(T, 11 + T, dev)
    lw = w.layers[li]
    Hv, Dv = cfg.linear_num_value_heads, cfg.linear_value_head_dim
    Cc = 2 * cfg.key_dim + cfg.value_dim
    f32 = dict(dtype=torch.float32, device=dev)
    d = dict(proj=torch.from_numpy(proj).to(dev), window=torch.from_numpy(window).to(dev),
             state=torch.from_numpy(state).to(dev),
             q=torch.zeros(rows, cfg.key_dim, **f32), k=torch.zeros(rows, cfg.key_dim, **f32),
             v=torch.zeros(rows, cfg.value_dim, **f32), g=torch.zeros(rows, Hv, **f32),
             beta=torch.zeros(rows, Hv, **f32), y=torch.zeros(rows, cfg.value_dim, **f32),
             out=torch.zeros(2, rows, cfg.value_dim, dtype=torch.bfloat16, device=dev))
    a = N.GdnArgs()
    a.desc = None; a.rows_padded = rows
    a.num_k_heads = cfg.linear_num_key_heads; a.num_v_heads = Hv
    a.head_k_dim = cfg.linear_key_head_dim; a.head_v_dim = Dv
    a.conv_keep = cfg.linear_conv_kernel_dim - 1
    a.proj = d["proj"].data_ptr(); a.ld_proj = cfg.in_proj_dim
    a.window = d["window"].data_ptr(); a.conv_w = lw.conv_w.data_ptr()
    a.A_log = lw.A_log.data_ptr(); a.dt_bias = lw.dt_bias.data_ptr(); a.state = d["state"].data_ptr()
    a.q = d["q"].data_ptr(); a.k = d["k"].data_ptr(); a.v = d["v"].data_ptr()
    a.g = d["g"].data_ptr(); a.beta = d["beta"].data_ptr(); a.y = d["y"].data_ptr()
    a.norm_w = lw.gnorm.data_ptr(); a.eps = cfg.rms_norm_eps
    a.out = d["out"][0].data_ptr(); a.out_lo = d["out"][1].data_ptr()
    a.out_layout = N.W_ROWMAJOR; a.ld_out = cfg.value_dim
    print(f"gdn chain T={T}", flush=True)
    N.check(N.lib().dtree_gdn_layer_chain(C.byref(a), T, _stream()), "gdn chain")
    torch.cuda.synchronize()

    chain = [-1] + list(range(T - 1))
    xin = proj[:T, :Cc]
    z = proj[:T, Cc:Cc + cfg.value_dim]
    b = proj[:T, Cc + cfg.value_dim:Cc + cfg.value_dim + Hv]
    av = proj[:T, Cc + cfg.value_dim + Hv:Cc + cfg.value_dim + 2 * Hv]
    conv_out, _ = ogdn.tree_conv1d(xin, window, orc.w(li, "conv"), chain)
    q, k, v, gg, beta = orc.gdn_inputs(li, conv_out, av, b)
    y, states = ogdn.tree_gated_delta(q, k, v, gg, beta, state, chain)
    o = orc.gated_norm(li, y, z.reshape(T, Hv, Dv)).reshape(T, -1)
    win, st = ogdn.commit(xin, window, q, k, v, gg, beta, state, chain, list(range(T)))

    def close(got, want, what, tol=1e-4):
        err = np.abs(np.asarray(got, np.float64) - want).max()
        assert err <= tol * max(1.0, np.abs(want).max()), f"{what}: max err {err}"

    close(d["q"][:T].cpu().numpy(), q.reshape(T, -1), "q")
    close(d["k"][:T].cpu().numpy(), k.reshape(T, -1), "k")
    close(d["g"][:T].cpu().numpy(), gg, "g")
    close(d["y"][:T].cpu().numpy(), y.reshape(T, -1), "y", 1e-3)
    close(d["state"].cpu().numpy(), st, "committed state", 1e-3)
    # the window is a copy of conv inputs (or of the old window): exact
    assert np.array_equal(d["window"].cpu().numpy(), win.astype(np.float32))
    got_o = bf16_f32(d["out"][0])[:T] + bf16_f32(d["out"][1])[:T]
    close(got_o, o, "gated norm", 1e-3)
    assert np.all(bf16_f32(d["out"][0])[T:] == 0)


def _oracle_prefill(cfg, w, toks, layer_ids):
    orc = o35.OracleQwen35(_oracle_cfg(cfg), w.host_accessor())
    oc = orc.new_cache()
    T = len(toks)
    chain = [-1] + list(range(T - 1))
    norm, vh, pend = orc.forward_tree(np.asarray(toks), np.arange(T), chain, oc, layer_ids=layer_ids)
    orc.commit(oc, pend, chain, list(range(T)))
    return orc, oc, vh, orc.lm_head_logits(norm[-1:])[0]


def _close(got, want, what):
    err = np.abs(np.asarray(got, np.float64) - want).max()
    assert err <= TOL * max(1.0, np.abs(want).max()), f"{what}: max err {err}"


def _check_cache(cfg, cache, oc, T):
    for li in range(cfg.num_hidden_layers):
        s = cache.slot[li]
        if cfg.is_linear(li):
            _close(cache.windows[s].cpu().numpy(), oc.layers[li][0], f"window {li}")
            _close(cache.states[s].cpu().numpy(), oc.layers[li][1], f"state {li}")
        else:
            _close(bf16_f32(cache.kv.logical_keys(s, T)), oc.layers[li][0], f"keys {li}")
            _close(bf16_f32(cache.kv.logical_values(s, T)), oc.layers[li][1], f"values {li}")


@pytest.mark.parametrize("T,segment,head", [(300, 1024, 0), (600, 256, 0), (260, 1024, 40)])
def test_qwen35_prefill_long_matches_oracle(gpu_device, attn_kernel, T, segment, head):
    cfg = tiny_qwen35()
    w = Qwen35Weights.random(cfg, seed=0, device=gpu_device, norm_jitter=0.1)
    layer_ids = [1, 3]
    eng = Qwen35TreeEngine(cfg, w, max_past=T + 64, layer_ids=layer_ids, max_nodes=25)
    eng.PREFILL_SEGMENT = segment
    toks = random_prefix(T, cfg.vocab_size, seed=T)
    cache = eng.new_cache()
    print(f"qwen35 prefill T={T} segment={segment} chain head={head}", flush=True)
    if head:
        eng.prefill(cache, toks[:head])  # the chain path
    logits, hidden = eng.prefill_long(cache, toks[head:])
    torch.cuda.synchronize()
    assert cache.offset == T
    _, oc, vh, last_logits = _oracle_prefill(cfg, w, toks, layer_ids)
    _check_cache(cfg, cache, oc, T)
    _close(bf16_f32(hidden), vh[head:], "verifier hidden")
    lg = logits[0, 0].cpu().numpy()
    assert np.abs(lg - last_logits).max() <= TOL * np.abs(last_logits).max()


def test_qwen35_prefill_long_q4_matches_oracle(gpu_device):
    """The hybrid's long-M prefill with q4 group-64 weights (every linear
    layer and the tied embedding) against the oracle on the dequantised
    weights."""
    cfg = tiny_qwen35()
    w = Qwen35Weights.random(cfg, seed=0, device=gpu_device, norm_jitter=0.1, quant="q4")
    layer_ids = [1, 3]
    eng = Qwen35TreeEngine(cfg, w, max_past=364, layer_ids=layer_ids, max_nodes=25)
    eng.PREFILL_SEGMENT = 256
    T = 300
    toks = random_prefix(T, cfg.vocab_size, seed=T)
    cache = eng.new_cache()
    logits, hidden = eng.prefill_long(cache, toks)
    torch.cuda.synchronize()
    assert cache.offset == T
    _, oc, vh, last_logits = _oracle_prefill(cfg, w, toks, layer_ids)
    _check_cache(cfg, cache, oc, T)
    _close(bf16_f32(hidden), vh, "verifier hidden")
    lg = logits[0, 0].cpu().numpy()
    assert np.abs(lg - last_logits).max() <= TOL * np.abs(last_logits).max()


def test_qwen35_adapter_prefill_takes_the_long_path(gpu_device, monkeypatch):
    cfg = tiny_qwen35()
    target = load_target_model(cfg, seed=0, max_past=512, device="cuda", norm_jitter=0.1)
    eng = target.model.engine
    calls = []
    orig = eng.prefill_long
    monkeypatch.setattr(eng, "prefill_long", lambda *a, **k: calls.append(1) or orig(*a, **k))
    toks = random_prefix(200, cfg.vocab_size, seed=3)
    cache = target.make_cache()
    logits, th = target.forward_with_hidden_states(torch.tensor(toks)[None], cache, [1])
    torch.cuda.synchronize()
    assert calls and cache.offset == 200 and tuple(th.shape) == (1, 200, cfg.hidden_size)
    _, oc, vh, last_logits = _oracle_prefill(cfg, target.model.weights, toks, [1])
    _check_cache(cfg, cache, oc, 200)
    _close(bf16_f32(th[0]), vh, "verifier hidden")
    lg = logits[0, -1].cpu().numpy()
    assert np.abs(lg - last_logits).max() <= TOL * np.abs(last_logits).max()
