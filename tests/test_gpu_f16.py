"""The DTREE_W_TILED_F16 path: fp16 tiled weights and one fp16 activation
plane (the format of the bf16 workloads' engines), kernel by kernel against
float64 references on the same fp16 inputs.

* dtree_tile_weight_f16 against the host tile_weight_f16 (order and the
  bf16 -> fp16 conversion, exact from 2^-17 to 65504);
* the 32-row GEMM in every schedule (stream-K, one workgroup per tile, two /
  three per tile) and epilogue, the 64-128-row kernel, the long-M prefill
  GEMM and the LM head: fp32 outputs within 1e-4 of the float64 product of
  the fp16 operands, fp16 activation outputs within fp16 rounding (2^-11
  relative), the low-plane pointer ignored, no low plane written, and
  deterministic reductions;
* attention and the GatedDeltaNet gated norm writing DTREE_W_TILED_F16: the
  fp16 plane equals their bf16-pair output (hi + lo) rounded to fp16.
"""
import ctypes as C

import numpy as np
import pytest
import torch

from dtree_hip import _native as N
from dtree_hip.weights import interleave_gate_up, tile_weight, tile_weight_f16, untile_weight

from gpu_util import stream

pytestmark = pytest.mark.gpu


def _f64(t: torch.Tensor) -> np.ndarray:
    return t.double().cpu().numpy()


def _x16(rows, L, k, g, dev, scale=1.0):
    xf = np.zeros((rows, k), np.float32)
    xf[:L] = g.standard_normal((L, k)) * scale
    x16 = torch.from_numpy(xf).to(torch.float16)
    return tile_weight_f16(x16.to(dev)), _f64(x16)


def _w(n, k, g, scale=0.05):
    return torch.from_numpy(g.standard_normal((n, k)).astype(np.float32) * scale).to(torch.bfloat16)


def test_tile_weight_f16_kernel_matches_host(gpu_device):
    g = np.random.default_rng(41)
    wf = g.standard_normal((96, 320)).astype(np.float32)
    wf[0, :8] = [2.0 ** -17, -(2.0 ** -17) * 1.5, 2.0 ** -20 * 1.25, 3e-9, 65504.0, -65504.0, 1e6, -1e30]
    w = torch.from_numpy(wf).to(torch.bfloat16).to(gpu_device)
    dst = torch.empty(96, 320, dtype=torch.float16, device=gpu_device)
    N.check(N.lib().dtree_tile_weight_f16(w.data_ptr(), dst.data_ptr(), 96, 320, stream()), "tile f16")
    torch.cuda.synchronize()
    host = tile_weight_f16(w)
    assert host.dtype == torch.float16 and torch.equal(dst, host)
    back = untile_weight(dst).float()
    wv = w.float()
    exact = (wv.abs() >= 2.0 ** -17) & (wv.abs() <= 65504)
    assert torch.equal(back[exact], wv[exact])
    assert back[0, 6].item() == 65504.0 and back[0, 7].item() == -65504.0
    # same order as the bf16 tiling
    assert torch.equal(untile_weight(tile_weight(w)), w)


def _args(xt, wt, n, k, rows, epi, ws, sched=0):
    a = N.GemmArgs()
    a.x = xt.data_ptr(); a.x_lo = xt.data_ptr()  # a low plane handed over anyway: must be ignored
    a.x_layout = a.w_layout = N.W_TILED_F16; a.ldx = k; a.rows_padded = rows
    a.w = wt.data_ptr(); a.n = n; a.k = k; a.epilogue = epi; a.split_k = sched
    a.workspace = ws.data_ptr(); a.workspace_bytes = ws.numel()
    return a


SHAPES = [(64, 64), (4096, 64), (64, 9728), (6144, 2560), (2560, 4096), (19456, 2560), (2560, 9728)]


@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("sched", [-4, -3, -2, -1, 0])
def test_f16_gemm_store_f32(gpu_device, n, k, sched):
    if sched in (-3, -4) and (n % 256 or k < 64 * (2 if sched == -3 else 3)):
        pytest.skip("the split per-tile schedules need n % 256 == 0 and k >= 64 * parts")
    g = np.random.default_rng(n + k - sched)
    xt, xin = _x16(32, 25, k, g, gpu_device)
    w = _w(n, k, g)
    wt = tile_weight_f16(w.to(gpu_device))
    ss = torch.from_numpy(np.abs(g.standard_normal((3, 32))).astype(np.float32) + 0.5).to(gpu_device)
    ws = torch.zeros(N.lib().dtree_gemm_workspace_bytes(32, n, k, 0), dtype=torch.uint8, device=gpu_device)
    outs = []
    for _ in range(2):
        out = torch.zeros(32, n, device=gpu_device)
        a = _args(xt, wt, n, k, 32, N.EPI_STORE_F32, ws, sched)
        a.ss_in = ss.data_ptr(); a.ss_tiles = 3; a.norm_dim = k; a.eps = 1e-6
        a.out_f32 = out.data_ptr(); a.ld_out_f32 = n
        N.check(N.lib().dtree_gemm_bf16(C.byref(a), stream()), "f16 gemm")
        outs.append(out)
    torch.cuda.synchronize()
    rs = 1.0 / np.sqrt(ss.cpu().numpy().sum(0) / k + 1e-6)
    ref = (xin @ _f64(w).T) * rs[:, None]
    got = outs[0].cpu().numpy()
    assert np.abs(got - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())
    assert torch.equal(outs[0], outs[1])
    assert int(ws[: (n // 32) * 4].view(torch.int32).abs().sum()) == 0


@pytest.mark.parametrize("rows", [32, 64, 96, 128])
@pytest.mark.parametrize("epi", ["residual", "swiglu", "store"])
def test_f16_gemm_epilogues(gpu_device, rows, epi):
    """Residual + next-norm statistics + hidden capture, SwiGLU and the
    activation store into DTREE_W_TILED_F16 outputs (one fp16 plane; the
    low-plane pointer is ignored and the buffer behind it untouched)."""
    g = np.random.default_rng(rows * 3 + len(epi))
    L = rows - 7
    n, k = (640, 1024) if epi != "swiglu" else (1536, 512)
    xt, xin = _x16(rows, L, k, g, gpu_device)
    if epi == "swiglu":
        gate, up = _w(n // 2, k, g), _w(n // 2, k, g)
        w = interleave_gate_up(gate, up)
    else:
        w = _w(n, k, g)
    wt = tile_weight_f16(w.to(gpu_device))
    width = n // 2 if epi == "swiglu" else n
    out = torch.zeros(2, rows * width, dtype=torch.float16, device=gpu_device)
    ws = torch.zeros(N.lib().dtree_gemm_workspace_bytes(rows, n, k, 0), dtype=torch.uint8, device=gpu_device)
    a = _args(xt, wt, n, k, rows, {"residual": N.EPI_RESIDUAL, "swiglu": N.EPI_SWIGLU,
                                   "store": N.EPI_STORE_BF16}[epi], ws)
    a.out_bf16 = out[0].data_ptr(); a.out_lo = out[1].data_ptr(); a.ld_out_bf16 = width
    a.out_layout = N.W_TILED_F16
    rs = np.ones(rows)
    if epi != "residual":
        ss_np = (np.abs(g.standard_normal((rows // 32, k // 32, 32))) + 0.5).astype(np.float32)
        ss = torch.from_numpy(ss_np).to(gpu_device)
        a.ss_in = ss.data_ptr(); a.ss_tiles = k // 32; a.norm_dim = k; a.eps = 1e-6
        rs = 1.0 / np.sqrt(ss_np.transpose(0, 2, 1).reshape(rows, k // 32).sum(1) / k + 1e-6)
    else:
        res = torch.zeros(rows, n)
        res[:L] = torch.from_numpy(g.standard_normal((L, n)).astype(np.float32))
        res = res.to(gpu_device)
        res0 = _f64(res)
        gn = torch.from_numpy((1 + 0.1 * g.standard_normal(n)).astype(np.float32)).to(torch.bfloat16).to(gpu_device)
        sso = torch.zeros(rows // 32, n // 32, 32, device=gpu_device)
        hid = torch.zeros(rows, n, dtype=torch.bfloat16, device=gpu_device)
        a.out_f32 = res.data_ptr(); a.ld_out_f32 = n
        a.next_norm = gn.data_ptr(); a.ss_out = sso.data_ptr(); a.hidden_out = hid.data_ptr(); a.ld_hidden = n
    print(f"f16 gemm epilogue={epi} rows={rows}", flush=True)
    N.check(N.lib().dtree_gemm_bf16(C.byref(a), stream()), "f16 gemm epilogue")
    torch.cuda.synchronize()
    got16 = _f64(untile_weight(out[0].view(rows, width)))
    assert not out[1].any()  # no low plane
    wf = _f64(w)
    if epi == "residual":
        ref = res0 + xin @ wf.T
        got = res.cpu().numpy()
        assert np.abs(got - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())
        want = got * _f64(gn.float())[None]
        assert np.all(np.abs(got16 - want) <= (2 ** -11 + 2 ** -20) * np.abs(want) + 2 ** -25)  # one fp16 rounding of x * g
        exp_ss = (got.astype(np.float64) ** 2).reshape(rows // 32, 32, n // 32, 32).sum(-1).transpose(0, 2, 1)
        np.testing.assert_allclose(sso.cpu().numpy(), exp_ss, rtol=1e-5, atol=1e-5)
        assert torch.equal(hid.cpu(), torch.from_numpy(got).to(torch.bfloat16))
    elif epi == "swiglu":
        gt = (xin @ _f64(gate).T) * rs[:, None]
        u = (xin @ _f64(up).T) * rs[:, None]
        ref = gt / (1 + np.exp(-gt)) * u
        assert np.abs(got16 - ref).max() <= 2 ** -10 * np.abs(ref).max() + 1e-6
    else:
        ref = (xin @ wf.T) * rs[:, None]
        assert np.abs(got16 - ref).max() <= 2 ** -10 * np.abs(ref).max() + 1e-6


def test_f16_gemm_rejects_mixed_layouts(gpu_device):
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device=gpu_device)
    a = N.GemmArgs()
    a.x = buf.data_ptr(); a.x_layout = N.W_TILED_F16; a.ldx = 64; a.rows_padded = 32
    a.w = buf.data_ptr(); a.w_layout = N.W_TILED; a.n = 64; a.k = 64
    a.epilogue = N.EPI_STORE_F32; a.out_f32 = buf.data_ptr(); a.ld_out_f32 = 64
    a.workspace = buf.data_ptr(); a.workspace_bytes = buf.numel()
    assert N.lib().dtree_gemm_bf16(C.byref(a), stream()) != 0
    assert b"TILED_F16" in N.lib().dtree_last_error()
    a.w_layout = N.W_Q4G64
    assert N.lib().dtree_gemm_bf16(C.byref(a), stream()) != 0


@pytest.mark.parametrize("rows,L", [(128, 128), (384, 300)])
@pytest.mark.parametrize("epi", ["f32", "residual", "swiglu"])
def test_f16_gemm_long(gpu_device, rows, L, epi):
    """The long-M prefill GEMM on fp16 operands: 128 x 128 tiles, fp32 and
    fp16-plane outputs against float64."""
    g = np.random.default_rng(rows + L + len(epi))
    n, k = (512, 384) if epi != "swiglu" else (768, 384)
    xt, xin = _x16(rows, L, k, g, gpu_device)
    if epi == "swiglu":
        gate, up = _w(n // 2, k, g), _w(n // 2, k, g)
        w = interleave_gate_up(gate, up)
    else:
        w = _w(n, k, g)
    wt = tile_weight_f16(w.to(gpu_device))
    a = N.GemmArgs()
    a.x = xt.data_ptr(); a.x_layout = a.w_layout = N.W_TILED_F16; a.ldx = k; a.rows_padded = rows
    a.w = wt.data_ptr(); a.n = n; a.k = k; a.out_layout = N.W_TILED_F16
    rs = np.ones(rows)
    if epi != "residual":
        ss_np = (np.abs(g.standard_normal((rows // 32, k // 32, 32))) + 0.5).astype(np.float32)
        ss = torch.from_numpy(ss_np).to(gpu_device)
        a.ss_in = ss.data_ptr(); a.ss_tiles = k // 32; a.norm_dim = k; a.eps = 1e-6
        rs = 1.0 / np.sqrt(ss_np.transpose(0, 2, 1).reshape(rows, k // 32).sum(1) / k + 1e-6)
    width = n // 2 if epi == "swiglu" else n
    out16 = torch.zeros(rows * width, dtype=torch.float16, device=gpu_device)
    wf = _f64(w)
    if epi == "f32":
        out = torch.zeros(rows, n, device=gpu_device)
        a.epilogue = N.EPI_STORE_F32; a.out_f32 = out.data_ptr(); a.ld_out_f32 = n
    elif epi == "residual":
        res = torch.zeros(rows, n)
        res[:L] = torch.from_numpy(g.standard_normal((L, n)).astype(np.float32))
        res = res.to(gpu_device)
        res0 = _f64(res)
        gn = torch.ones(n, dtype=torch.bfloat16, device=gpu_device)
        sso = torch.zeros(rows // 32, n // 32, 32, device=gpu_device)
        a.epilogue = N.EPI_RESIDUAL; a.out_f32 = res.data_ptr(); a.ld_out_f32 = n
        a.out_bf16 = out16.data_ptr(); a.ld_out_bf16 = n; a.next_norm = gn.data_ptr(); a.ss_out = sso.data_ptr()
    else:
        a.epilogue = N.EPI_SWIGLU; a.out_bf16 = out16.data_ptr(); a.ld_out_bf16 = width
    N.check(N.lib().dtree_gemm_long(C.byref(a), stream()), "f16 long gemm")
    torch.cuda.synchronize()
    if epi == "f32":
        ref = (xin @ wf.T) * rs[:, None]
        assert np.abs(out.cpu().numpy() - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())
    elif epi == "residual":
        ref = res0 + xin @ wf.T
        got = res.cpu().numpy()
        assert np.abs(got - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())
        got16 = _f64(untile_weight(out16.view(rows, n)))
        assert np.all(np.abs(got16 - got) <= (2 ** -11 + 2 ** -20) * np.abs(got) + 2 ** -25)
    else:
        gt = (xin @ _f64(gate).T) * rs[:, None]
        u = (xin @ _f64(up).T) * rs[:, None]
        ref = gt / (1 + np.exp(-gt)) * u
        got16 = _f64(untile_weight(out16.view(rows, width)))
        assert np.abs(got16 - ref).max() <= 2 ** -10 * np.abs(ref).max() + 1e-6


@pytest.mark.parametrize("rows", [32, 96])
def test_f16_lmhead(gpu_device, rows):
    """The LM head on the fp16 embedding and activation plane: logits against
    float64, the walk's posterior = the argmax of the logits."""
    from gpu_util import device_desc
    g = np.random.default_rng(31 + rows)
    V, H = 8192, 1024
    L = rows - 5
    xt, xin = _x16(rows, L, H, g, gpu_device)
    E = _w(V, H, g, 0.02)
    Et = tile_weight_f16(E.to(gpu_device))
    lib = N.lib()
    cand = torch.zeros(lib.dtree_lmhead_candidates_bytes(rows), dtype=torch.uint8, device=gpu_device)
    logits = torch.zeros(rows, V, device=gpu_device)
    N.check(lib.dtree_lmhead_argmax(xt.data_ptr(), xt.data_ptr(), N.W_TILED_F16, H, rows, Et.data_ptr(),
                                    N.W_TILED_F16, None, V, H, None, 0, 1e-6, logits.data_ptr(), cand.data_ptr(),
                                    stream()), "f16 lm head")
    parents = [-1] + [(i - 1) // 2 for i in range(1, L)]
    desc = device_desc([0] * L, list(range(L)), parents, 0, gpu_device)
    res = torch.zeros(3 + 2 * N.MAX_NODES, dtype=torch.int32, device=gpu_device)
    N.check(lib.dtree_accept_walk(desc.data_ptr(), cand.data_ptr(), lib.dtree_lmhead_candidate_blocks(V, rows), rows,
                                  res.data_ptr(), stream()), "walk")
    torch.cuda.synchronize()
    ref = xin[:L] @ _f64(E).T
    got = logits[:L].cpu().numpy()
    assert np.abs(got - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())
    r = res.cpu().numpy()
    assert list(r[3 + N.MAX_NODES:3 + N.MAX_NODES + L]) == list(np.argmax(got, axis=-1))


@pytest.mark.parametrize("kernel", ["head", "group"])
@pytest.mark.parametrize("P,MP,L", [(700, 32, 25), (300, 96, 65)])
def test_f16_attention_output(gpu_device, monkeypatch, kernel, P, MP, L):
    """Tree attention writing DTREE_W_TILED_F16: its fp16 plane equals the
    bf16-pair output (hi + lo, DTREE_W_TILED) of the same launch inputs to
    within one fp16 rounding, rows past the tree are zero, no low plane is
    written."""
    from gpu_util import device_desc, random_tree
    from dtree_hip.cache import PagedKVCache
    monkeypatch.setenv("DTREE_ATTN_KERNEL", kernel)
    g = np.random.default_rng(P + MP)
    Hq, Hkv, D = 32, 8, 128
    parents = random_tree(L, seed=9)
    cache = PagedKVCache(1, Hkv, D, P + MP, device=gpu_device)
    if P:
        cache.write_logical(0, torch.from_numpy((g.standard_normal((P, Hkv, D)) * 0.5).astype(np.float32)),
                            torch.from_numpy((g.standard_normal((P, Hkv, D)) * 0.5).astype(np.float32)))
    qkv = np.zeros((MP, (Hq + 2 * Hkv) * D), np.float32)
    qkv[:L] = g.standard_normal((L, (Hq + 2 * Hkv) * D))
    qkv_t = torch.from_numpy(qkv).to(gpu_device)
    depth = [0] * L
    for i in range(1, L):
        depth[i] = depth[parents[i]] + 1
    desc = device_desc([0] * L, [P + d for d in depth], parents, P, gpu_device)
    cos = torch.zeros(MP, D // 2, device=gpu_device)
    sin = torch.zeros(MP, D // 2, device=gpu_device)
    N.check(N.lib().dtree_rope_table(desc.data_ptr(), MP, D, 1e6, cos.data_ptr(), sin.data_ptr(), stream()))
    ws = torch.zeros(N.lib().dtree_attention_workspace_bytes(Hq, D, P, MP), dtype=torch.uint8, device=gpu_device)
    outs = {}
    for layout, dt in ((N.W_TILED, torch.bfloat16), (N.W_TILED_F16, torch.float16)):
        o = torch.full((2, MP, Hq * D), 3.0, dtype=dt, device=gpu_device)
        a = N.AttnArgs()
        a.qkv = qkv_t.data_ptr(); a.ld_qkv = qkv.shape[1]; a.q_norm = None; a.k_norm = None; a.eps = 1e-6
        a.rope_cos = cos.data_ptr(); a.rope_sin = sin.data_ptr()
        a.k_pages = cache.k_ptr(0); a.v_pages = cache.v_ptr(0); a.page_table = cache.page_table.data_ptr()
        a.desc = desc.data_ptr(); a.out = o[0].data_ptr(); a.out_lo = o[1].data_ptr(); a.ld_out = Hq * D
        a.out_layout = layout
        a.num_heads = Hq; a.num_kv_heads = Hkv; a.head_dim = D; a.rows_padded = MP; a.scale = D ** -0.5
        a.max_past_length = P; a.write_cache = 1 if layout == N.W_TILED else 0
        a.workspace = ws.data_ptr(); a.workspace_bytes = ws.numel()
        N.check(N.lib().dtree_tree_attention(C.byref(a), stream()), "attention")
        outs[layout] = o
    torch.cuda.synchronize()
    pair = outs[N.W_TILED]
    full = _f64(untile_weight(pair[0].view(MP, Hq * D))) + _f64(untile_weight(pair[1].view(MP, Hq * D)))
    got = _f64(untile_weight(outs[N.W_TILED_F16][0].view(MP, Hq * D)))
    assert np.all(np.abs(got - full) <= (2 ** -11 + 2 ** -16) * np.abs(full) + 2 ** -24)
    assert not got[L:].any()
    assert torch.all(outs[N.W_TILED_F16][1] == 3.0)  # the low-plane buffer is not touched


def test_f16_gated_norm_output(gpu_device):
    """dtree_gdn_layer_gated_norm into DTREE_W_TILED_F16: the fp16 plane equals
    the bf16-pair output (hi + lo) of the same inputs rounded to fp16."""
    from gpu_util import device_desc
    g = np.random.default_rng(17)
    Hk, Hv, D, MP, L = 16, 32, 128, 32, 25
    C_ = 2 * Hk * D + Hv * D
    ld = C_ + Hv * D + 2 * Hv
    dev = gpu_device
    desc = device_desc([0] * L, list(range(L)), [-1] + list(range(L - 1)), 0, dev)
    y = torch.from_numpy(g.standard_normal((MP, Hv * D)).astype(np.float32)).to(dev)
    proj = torch.from_numpy(g.standard_normal((MP, ld)).astype(np.float32)).to(dev)
    nw = torch.from_numpy((1 + 0.1 * g.standard_normal(D)).astype(np.float32)).to(torch.bfloat16).to(dev)
    outs = {}
    for layout in (N.W_TILED, N.W_TILED_F16):
        dt = torch.float16 if layout == N.W_TILED_F16 else torch.bfloat16
        o = torch.zeros(2, MP, Hv * D, dtype=dt, device=dev)
        a = N.GdnArgs()
        a.desc = desc.data_ptr(); a.rows_padded = MP; a.num_k_heads = Hk; a.num_v_heads = Hv
        a.head_k_dim = D; a.head_v_dim = D; a.conv_keep = 3
        a.proj = proj.data_ptr(); a.ld_proj = ld; a.y = y.data_ptr(); a.norm_w = nw.data_ptr(); a.eps = 1e-6
        a.out = o[0].data_ptr(); a.out_lo = o[1].data_ptr(); a.out_layout = layout; a.ld_out = Hv * D
        N.check(N.lib().dtree_gdn_layer_gated_norm(C.byref(a), stream()), "gated norm")
        outs[layout] = o
    torch.cuda.synchronize()
    pair = outs[N.W_TILED]
    full = untile_weight(pair[0]).float() + untile_weight(pair[1]).float()
    got = untile_weight(outs[N.W_TILED_F16][0]).float()
    assert torch.all((got - full).abs() <= (2 ** -11 + 2 ** -16) * full.abs() + 2 ** -24)
    assert not outs[N.W_TILED_F16][1].any()
