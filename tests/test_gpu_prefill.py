"""Prompt prefill on the long-M path (adapters.py:494-533) against the oracle.

* dtree_gemm_long (128 x 128 MFMA tiles over any multiple of 128 rows) in
  every epilogue, with and without the low activation plane, tiled and
  row-major outputs, against a float64 product (2e-4 of the output scale,
  as the skinny GEMMs); with q4 group-64 weights against the float64 q4
  product (the fp32 store, a 64-column last tile, residual and SwiGLU).
* Qwen3TreeEngine.prefill_long on the tiny model against the oracle's causal
  forward: every cached K / V row of every layer, the verifier hidden rows
  and the last position's logits within the 2e-2 bar; one segment with a
  ragged last 128-row chunk, several segments, and a prompt that continues
  a prefix the chain path wrote; q4 group-64 weights; the adapter's
  forward_with_hidden_states taking the long path.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from oracle import q4 as o4
from oracle import qwen3 as oq

from dtree_hip import _native as N
from dtree_hip import Qwen3TreeModel, Qwen3Weights, tiny_qwen3
from dtree_hip.adapters import load_target_model
from dtree_hip.synthetic import random_prefix
from dtree_hip.weights import interleave_gate_up, q4_to_tiled, tile_weight

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _bf(t):
    return t.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("rows,L", [(128, 128), (384, 300)])
@pytest.mark.parametrize("epi", ["f32", "bf16", "residual", "swiglu"])
@pytest.mark.parametrize("lo", [False, True])
@pytest.mark.parametrize("out_tiled", [False, True])
def test_gemm_long_matches_float64(gpu_device, rows, L, epi, lo, out_tiled):
    g = np.random.default_rng(rows + L + 7 * lo + 3 * out_tiled + len(epi))
    n, k = (512, 384) if epi != "swiglu" else (768, 384)
    dev = gpu_device
    xf = np.zeros((rows, k), np.float32)
    xf[:L] = g.standard_normal((L, k))
    hi = torch.from_numpy(xf).to(torch.bfloat16)
    lo_t = (torch.from_numpy(xf) - hi.float()).to(torch.bfloat16)
    xin = _bf(hi) + (_bf(lo_t) if lo else 0.0)
    if epi == "swiglu":
        gate = torch.from_numpy(g.standard_normal((n // 2, k)).astype(np.float32) * 0.05).to(torch.bfloat16)
        up = torch.from_numpy(g.standard_normal((n // 2, k)).astype(np.float32) * 0.05).to(torch.bfloat16)
        w = interleave_gate_up(gate, up)
    else:
        w = torch.from_numpy(g.standard_normal((n, k)).astype(np.float32) * 0.05).to(torch.bfloat16)
    a = N.GemmArgs()
    xt = tile_weight(hi.to(dev))
    xlt = tile_weight(lo_t.to(dev))
    wt = tile_weight(w.to(dev))
    a.x = xt.data_ptr(); a.x_lo = xlt.data_ptr() if lo else None
    a.x_layout = a.w_layout = N.W_TILED; a.ldx = k; a.rows_padded = rows
    a.w = wt.data_ptr(); a.n = n; a.k = k
    a.out_layout = N.W_TILED if out_tiled else N.W_ROWMAJOR
    ss = None
    if epi in ("f32", "bf16", "swiglu"):
        ss = torch.from_numpy(np.abs(g.standard_normal((rows // 32, k // 32, 32))).astype(np.float32) + 0.5).to(dev)
        a.ss_in = ss.data_ptr(); a.ss_tiles = k // 32; a.norm_dim = k; a.eps = 1e-6
        rs = 1.0 / np.sqrt(ss.cpu().numpy().transpose(0, 2, 1).reshape(rows, k // 32).sum(1) / k + 1e-6)
    else:
        rs = np.ones(rows)
    width = n // 2 if epi == "swiglu" else n
    out_f32 = torch.zeros(rows, n, device=dev)
    out_bf = torch.zeros(2, rows, width, dtype=torch.bfloat16, device=dev)
    a.out_f32 = out_f32.data_ptr(); a.ld_out_f32 = n
    a.out_bf16 = out_bf[0].data_ptr(); a.out_lo = out_bf[1].data_ptr(); a.ld_out_bf16 = width
    hid = torch.zeros(rows, n, dtype=torch.bfloat16, device=dev)
    ss_out = torch.zeros(rows // 32, n // 32, 32, device=dev)
    gn = torch.from_numpy((1 + 0.1 * g.standard_normal(n)).astype(np.float32)).to(torch.bfloat16).to(dev)
    res0 = np.zeros((rows, n), np.float32)
    if epi == "residual":
        res0[:L] = g.standard_normal((L, n))
        out_f32.copy_(torch.from_numpy(res0))
        a.next_norm = gn.data_ptr(); a.ss_out = ss_out.data_ptr(); a.hidden_out = hid.data_ptr(); a.ld_hidden = n
    a.epilogue = {"f32": N.EPI_STORE_F32, "bf16": N.EPI_STORE_BF16, "residual": N.EPI_RESIDUAL,
                  "swiglu": N.EPI_SWIGLU}[epi]
    N.check(N.lib().dtree_gemm_long(C.byref(a), _stream()), "gemm_long")
    torch.cuda.synchronize()
    y = (xin @ _bf(w).T) * rs[:, None]

    def unt(t):  # bf16 [rows, width] in the output layout -> row-major fp64
        t = t.view(torch.int16).contiguous()
        if out_tiled:
            from dtree_hip.weights import untile_weight
            t = untile_weight(t.view(torch.bfloat16)).view(torch.int16)
        return t.view(torch.bfloat16).float().cpu().numpy().astype(np.float64)

    if epi == "f32":
        got, ref = out_f32.cpu().numpy(), y
    elif epi == "bf16":
        got, ref = unt(out_bf[0]) + unt(out_bf[1]), y
    elif epi == "residual":
        got, ref = out_f32.cpu().numpy(), res0.astype(np.float64) + y
        xg = unt(out_bf[0]) + unt(out_bf[1])
        np.testing.assert_allclose(xg, got * _bf(gn)[None], rtol=1e-5, atol=1e-5)
        exp_ss = (got.astype(np.float64) ** 2).reshape(rows // 32, 32, n // 32, 32).sum(-1).transpose(0, 2, 1)
        np.testing.assert_allclose(ss_out.cpu().numpy(), exp_ss, rtol=1e-5, atol=1e-5)
        assert torch.equal(hid.cpu(), torch.from_numpy(got).to(torch.bfloat16))
    else:
        gt = y[:, 0::1].reshape(rows, n // 32, 2, 16)[:, :, 0, :].reshape(rows, n // 2)
        upv = y.reshape(rows, n // 32, 2, 16)[:, :, 1, :].reshape(rows, n // 2)
        got, ref = unt(out_bf[0]) + unt(out_bf[1]), gt / (1 + np.exp(-gt)) * upv
    assert np.abs(got - ref).max() <= 2e-4 * max(1.0, np.abs(ref).max())
    assert np.all(got[L:] == 0) if epi != "residual" else True


def _q4_torch(wq, s, b):
    return (torch.from_numpy(np.ascontiguousarray(wq).view(np.int32)),
            torch.from_numpy(np.ascontiguousarray(s).view(np.int16)).view(torch.bfloat16),
            torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16))


@pytest.mark.parametrize("rows,L", [(128, 100), (256, 200)])
@pytest.mark.parametrize("epi", ["f32", "f32_tail", "residual", "swiglu"])
@pytest.mark.parametrize("lo", [False, True])
def test_gemm_long_q4_matches_float64(gpu_device, rows, L, epi, lo):
    """dtree_gemm_long with q4 group-64 weights (the nibble trick and the
    per-group scale / bias fix-up on 128 x 128 tiles) against the float64 q4
    product; f32_tail: n % 128 == 64."""
    g = np.random.default_rng(rows + L + 5 * lo + len(epi))
    dev = gpu_device
    k = 384
    n = {"f32": 512, "f32_tail": 320, "residual": 512, "swiglu": 768}[epi]
    xf = np.zeros((rows, k), np.float32)
    xf[:L] = g.standard_normal((L, k))
    hi = torch.from_numpy(xf).to(torch.bfloat16)
    lo_t = (torch.from_numpy(xf) - hi.float()).to(torch.bfloat16)
    xin = _bf(hi) + (_bf(lo_t) if lo else 0.0)
    if epi == "swiglu":
        F = n // 2
        gq, gs, gb = o4.random_q4(F, k, g)
        uq, us, ub = o4.random_q4(F, k, g)
        wq2 = interleave_gate_up(*[torch.from_numpy(np.ascontiguousarray(t).view(np.int32)) for t in (gq, uq)])
        s2 = interleave_gate_up(*[torch.from_numpy(np.ascontiguousarray(t).view(np.int16)) for t in (gs, us)])
        b2 = interleave_gate_up(*[torch.from_numpy(np.ascontiguousarray(t).view(np.int16)) for t in (gb, ub)])
        wt, sb = q4_to_tiled(wq2, s2.view(torch.bfloat16), b2.view(torch.bfloat16))
        gate = o4.q4_matmul(xin, gq, oq.bf16_to_f32(gs), oq.bf16_to_f32(gb))
        up = o4.q4_matmul(xin, uq, oq.bf16_to_f32(us), oq.bf16_to_f32(ub))
    else:
        wq, ws, wb = o4.random_q4(n, k, g)
        wt, sb = q4_to_tiled(*_q4_torch(wq, ws, wb))
        y = o4.q4_matmul(xin, wq, oq.bf16_to_f32(ws), oq.bf16_to_f32(wb))
    wt, sb = wt.to(dev), sb.to(dev)
    a = N.GemmArgs()
    xt, xlt = tile_weight(hi.to(dev)), tile_weight(lo_t.to(dev))
    a.x = xt.data_ptr(); a.x_lo = xlt.data_ptr() if lo else None
    a.x_layout = N.W_TILED; a.ldx = k; a.rows_padded = rows
    a.w = wt.data_ptr(); a.w_scales = sb.data_ptr(); a.w_layout = N.W_Q4G64; a.n = n; a.k = k
    a.out_layout = N.W_ROWMAJOR
    width = n // 2 if epi == "swiglu" else n
    out_f32 = torch.zeros(rows, n, device=dev)
    out_bf = torch.zeros(2, rows, width, dtype=torch.bfloat16, device=dev)
    a.out_f32 = out_f32.data_ptr(); a.ld_out_f32 = n
    a.out_bf16 = out_bf[0].data_ptr(); a.out_lo = out_bf[1].data_ptr(); a.ld_out_bf16 = width
    rs = np.ones(rows)
    if epi != "residual":
        ss = torch.from_numpy(np.abs(g.standard_normal((rows // 32, k // 32, 32))).astype(np.float32) + 0.5).to(dev)
        a.ss_in = ss.data_ptr(); a.ss_tiles = k // 32; a.norm_dim = k; a.eps = 1e-6
        rs = 1.0 / np.sqrt(ss.cpu().numpy().transpose(0, 2, 1).reshape(rows, k // 32).sum(1) / k + 1e-6)
    res0 = np.zeros((rows, n), np.float32)
    gn = torch.ones(n, dtype=torch.bfloat16, device=dev)
    ss_out = torch.zeros(rows // 32, n // 32, 32, device=dev)
    if epi == "residual":
        res0[:L] = g.standard_normal((L, n))
        out_f32.copy_(torch.from_numpy(res0))
        a.next_norm = gn.data_ptr(); a.ss_out = ss_out.data_ptr()
    a.epilogue = {"f32": N.EPI_STORE_F32, "f32_tail": N.EPI_STORE_F32, "residual": N.EPI_RESIDUAL,
                  "swiglu": N.EPI_SWIGLU}[epi]
    print(f"q4 long gemm rows={rows} n={n} k={k} epi={epi} lo={lo}", flush=True)
    N.check(N.lib().dtree_gemm_long(C.byref(a), _stream()), "gemm_long q4")
    torch.cuda.synchronize()
    if epi == "swiglu":
        gt, upv = gate * rs[:, None], up * rs[:, None]
        ref = gt / (1 + np.exp(-np.clip(gt, -80, 80))) * upv
        got = _bf(out_bf[0]) + _bf(out_bf[1])
    elif epi == "residual":
        ref, got = res0.astype(np.float64) + y, out_f32.cpu().numpy()
    else:
        ref, got = y * rs[:, None], out_f32.cpu().numpy()
    assert np.abs(got - ref).max() <= 2e-4 * max(1.0, np.abs(ref).max())


def _oracle(cfg, w):
    ocfg = oq.Qwen3Config(hidden=cfg.hidden_size, layers=cfg.num_hidden_layers, ffn=cfg.intermediate_size,
                          heads=cfg.num_attention_heads, kv_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                          vocab=cfg.vocab_size, eps=cfg.rms_norm_eps, rope_base=cfg.rope_theta)
    return oq.OracleQwen3(ocfg, w.host_accessor())


def _oracle_causal(orc, cfg, toks, layer_ids):
    """Per-layer K/V at every position, the verifier hidden rows and the last
    position's logits of the causal forward over `toks`."""
    T = len(toks)
    x = orc.embed(np.asarray(toks, np.int64))
    empty = np.zeros((0, cfg.num_key_value_heads, cfg.head_dim), np.float32)
    ks, vs, hid = [], [], []
    for li in range(cfg.num_hidden_layers):
        x, k, v = orc.layer_forward(li, x, empty, empty, np.arange(T), np.tril(np.ones((T, T), bool)))
        ks.append(k)
        vs.append(v)
        if li in layer_ids:
            hid.append(x)
    norm = oq.rms_norm(x[-1:], orc.w(None, "final_norm"), cfg.rms_norm_eps)
    return ks, vs, np.concatenate(hid, -1) if hid else None, orc.lm_head_logits(norm)[0]


def _check_rows(got, want, what):
    err = np.abs(got - want).max(axis=tuple(range(1, got.ndim)))
    bar = TOL * np.maximum(1.0, np.abs(want).max(axis=tuple(range(1, want.ndim))))
    assert np.all(err <= bar), f"{what}: worst row {int(np.argmax(err / bar))} ({float((err / bar).max()):.3f} of the bar)"


@pytest.mark.parametrize("T,segment,head", [(300, 1024, 0), (600, 256, 0), (400, 1024, 70)])
def test_prefill_long_matches_oracle(gpu_device, attn_kernel, T, segment, head):
    cfg = tiny_qwen3()
    w = Qwen3Weights.random(cfg, seed=0, device=gpu_device, norm_jitter=0.1)
    layer_ids = [0, 1]
    eng = Qwen3TreeModel(cfg, w, max_past=T + 64, layer_ids=layer_ids).engine
    eng.PREFILL_SEGMENT = segment
    toks = random_prefix(T, cfg.vocab_size, seed=T)
    cache = eng.new_cache()
    print(f"prefill T={T} segment={segment} chain head={head}", flush=True)
    if head:
        eng.prefill(cache, toks[:head])  # < 128 tokens: the chain path
    logits, hidden = eng.prefill_long(cache, toks[head:])
    torch.cuda.synchronize()
    assert cache.offset == T
    orc = _oracle(cfg, w)
    ks, vs, hid, last_logits = _oracle_causal(orc, cfg, toks, layer_ids)
    for li in range(cfg.num_hidden_layers):
        _check_rows(cache.logical_keys(li, T).float().cpu().numpy(), ks[li], f"keys layer {li}")
        _check_rows(cache.logical_values(li, T).float().cpu().numpy(), vs[li], f"values layer {li}")
    _check_rows(hidden.float().cpu().numpy(), hid[head:], "verifier hidden")
    lg = logits[0, 0].cpu().numpy()
    assert np.abs(lg - last_logits).max() <= TOL * np.abs(last_logits).max()


def test_prefill_long_q4_matches_oracle(gpu_device):
    """The long-M prefill with q4 group-64 weights (every linear layer and the
    tied embedding) against the oracle on the dequantised weights."""
    cfg = tiny_qwen3()
    w = Qwen3Weights.random_q4(cfg, seed=0, device=gpu_device, norm_jitter=0.1)
    layer_ids = [0, 1]
    eng = Qwen3TreeModel(cfg, w, max_past=364, layer_ids=layer_ids).engine
    eng.PREFILL_SEGMENT = 256
    T = 300
    toks = random_prefix(T, cfg.vocab_size, seed=T)
    cache = eng.new_cache()
    logits, hidden = eng.prefill_long(cache, toks)
    torch.cuda.synchronize()
    assert cache.offset == T
    orc = _oracle(cfg, w)
    ks, vs, hid, last_logits = _oracle_causal(orc, cfg, toks, layer_ids)
    for li in range(cfg.num_hidden_layers):
        _check_rows(cache.logical_keys(li, T).float().cpu().numpy(), ks[li], f"keys layer {li}")
        _check_rows(cache.logical_values(li, T).float().cpu().numpy(), vs[li], f"values layer {li}")
    _check_rows(hidden.float().cpu().numpy(), hid, "verifier hidden")
    lg = logits[0, 0].cpu().numpy()
    assert np.abs(lg - last_logits).max() <= TOL * np.abs(last_logits).max()


def test_adapter_prefill_takes_the_long_path(gpu_device, monkeypatch):
    cfg = tiny_qwen3()
    target = load_target_model(cfg, seed=0, max_past=512, device="cuda", norm_jitter=0.1)
    eng = target.model.engine
    calls = []
    orig = eng.prefill_long
    monkeypatch.setattr(eng, "prefill_long", lambda *a, **k: calls.append(1) or orig(*a, **k))
    toks = random_prefix(200, cfg.vocab_size, seed=3)
    cache = target.make_cache()
    logits, th = target.forward_with_hidden_states(torch.tensor(toks)[None], cache, [1])
    assert calls and cache.offset == 200 and tuple(th.shape) == (1, 200, cfg.hidden_size)
    orc = _oracle(cfg, target.model.weights)
    _, _, hid, last_logits = _oracle_causal(orc, cfg, toks, [1])
    lg = logits[0, -1].cpu().numpy()
    assert np.abs(lg - last_logits).max() <= TOL * np.abs(last_logits).max()
    _check_rows(th[0].float().cpu().numpy(), hid, "verifier hidden")
