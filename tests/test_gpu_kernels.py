"""Kernel-level parity on the GPU through the C ABI, against the CPU oracle /
fp32 references. Tolerances: fp32-accumulated GEMM outputs rtol 1e-4 (only
the summation order differs); bf16 outputs within 1 bf16 ulp-ish (rtol 1e-2);
attention vs the fp32 oracle within 2e-2 of the row scale (bf16 operands)."""
import ctypes as C

import numpy as np
import pytest
import torch

from dtree_hip import _native as N
from dtree_hip.cache import PagedKVCache
from dtree_hip.weights import tile_weight
from oracle import qwen3 as oq
from oracle import tree as otree

from gpu_util import bf16_f32, device_desc, random_tree, read_desc, stream, tree_mask

pytestmark = pytest.mark.gpu


def _gemm(x, w, epi, split, ws, **kw):
    """w is row-major; tiled=True hands the kernel its DTREE_W_TILED copy."""
    a = N.GemmArgs()
    if kw.get("tiled"):  # tiled copies are freed stream-ordered, after the launch below
        w = tile_weight(w)
        x = tile_weight(x)
        a.w_layout = a.x_layout = N.W_TILED
    a.x = x.data_ptr(); a.ldx = x.shape[1]; a.rows_padded = x.shape[0]
    a.w = w.data_ptr(); a.n = w.shape[0]; a.k = w.shape[1]
    a.epilogue = epi; a.split_k = split
    ss = kw.get("ss_in")
    a.ss_in = ss.data_ptr() if ss is not None else None
    # statistics [rows/32][tiles][32] (or [tiles][32] for 32 rows)
    a.ss_tiles = (ss.shape[-2] if ss.dim() == 3 else ss.shape[0]) if ss is not None else 0
    a.norm_dim = kw.get("norm_dim", 1); a.eps = 1e-6
    for name in ("out_f32", "out_bf16"):
        t = kw.get(name)
        if t is not None:
            setattr(a, name, t.data_ptr()); setattr(a, "ld_" + name, t.stride(0))
    nn = kw.get("next_norm")
    a.next_norm = nn.data_ptr() if nn is not None else None
    so = kw.get("ss_out")
    a.ss_out = so.data_ptr() if so is not None else None
    hid = kw.get("hidden_out")
    if hid is not None:
        a.hidden_out = hid.data_ptr(); a.ld_hidden = hid.stride(0)
    a.workspace = ws.data_ptr(); a.workspace_bytes = ws.numel()
    N.check(N.lib().dtree_gemm_bf16(C.byref(a), stream()), "gemm")


def _rows(MP, L, K, g, dev, scale=1.0):
    x = torch.zeros(MP, K)
    x[:L] = torch.from_numpy(g.standard_normal((L, K)).astype(np.float32)) * scale
    return x.to(torch.bfloat16).to(dev)


@pytest.mark.parametrize("MP,L", [(32, 25), (32, 32), (64, 40), (96, 65), (128, 128)])
@pytest.mark.parametrize("split", [1, 3, 8])
@pytest.mark.parametrize("tiled", [False, True])
def test_gemm_store_f32_rowscale(gpu_device, MP, L, split, tiled):
    g = np.random.default_rng(MP + split)
    N_, K = 256, 1024
    x = _rows(MP, L, K, g, gpu_device)
    w = torch.from_numpy(g.standard_normal((N_, K)).astype(np.float32) * 0.05).to(torch.bfloat16).to(gpu_device)
    ss = torch.from_numpy(np.abs(g.standard_normal((MP // 32, 5, 32))).astype(np.float32)).to(gpu_device)
    out = torch.zeros(MP, N_, device=gpu_device)
    ws = torch.zeros(N.lib().dtree_gemm_workspace_bytes(MP, N_, K, split), dtype=torch.uint8, device=gpu_device)
    _gemm(x, w, N.EPI_STORE_F32, split, ws, ss_in=ss, norm_dim=K, out_f32=out, tiled=tiled)
    torch.cuda.synchronize()
    rs = 1.0 / np.sqrt(ss.cpu().numpy().sum(1).reshape(MP) / K + 1e-6)  # row m = 32 * block + lane
    ref = (bf16_f32(x).astype(np.float64) @ bf16_f32(w).T.astype(np.float64)) * rs[:, None]
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-4, atol=1e-4)
    assert int(ws[: (N_ // 32) * 4].view(torch.int32).abs().sum()) == 0  # counters self-reset
    out2 = torch.zeros_like(out)
    _gemm(x, w, N.EPI_STORE_F32, split, ws, ss_in=ss, norm_dim=K, out_f32=out2)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)  # deterministic split-K reduction


@pytest.mark.parametrize("MP", [32, 64, 128])
def test_gemm_split_pair_input_and_output(gpu_device, MP):
    """X = hi + lo (split bf16 pair) multiplies like an fp32 X; the split output
    hi + lo carries the fp32 result to ~2^-16 relative."""
    g = np.random.default_rng(31 + MP)
    L, N_, K = MP - 5, 128, 512
    xf = np.zeros((MP, K), np.float32)
    xf[:L] = g.standard_normal((L, K))
    hi = torch.from_numpy(xf).to(torch.bfloat16)
    lo = (torch.from_numpy(xf) - hi.float()).to(torch.bfloat16)
    x2 = torch.stack([hi, lo]).to(gpu_device)
    w = torch.from_numpy(g.standard_normal((N_, K)).astype(np.float32) * 0.05).to(torch.bfloat16).to(gpu_device)
    out = torch.zeros(2, MP, N_, dtype=torch.bfloat16, device=gpu_device)
    ws = torch.zeros(N.lib().dtree_gemm_workspace_bytes(MP, N_, K, 2), dtype=torch.uint8, device=gpu_device)
    a = N.GemmArgs()
    a.x = x2[0].data_ptr(); a.x_lo = x2[1].data_ptr(); a.ldx = K; a.rows_padded = MP
    a.w = w.data_ptr(); a.n = N_; a.k = K; a.epilogue = N.EPI_STORE_BF16; a.split_k = 2
    a.out_bf16 = out[0].data_ptr(); a.out_lo = out[1].data_ptr(); a.ld_out_bf16 = N_
    a.workspace = ws.data_ptr(); a.workspace_bytes = ws.numel()
    N.check(N.lib().dtree_gemm_bf16(C.byref(a), stream()), "gemm")
    torch.cuda.synchronize()
    ref = (hi.double() + lo.double()).numpy() @ bf16_f32(w).T.astype(np.float64)
    got = out[0].double().cpu().numpy() + out[1].double().cpu().numpy()
    assert np.abs(got - ref).max() <= 2e-5 * np.abs(ref).max()
    # hi-only would be ~100x worse: the low half is really used
    ref_hi = hi.double().numpy() @ bf16_f32(w).T.astype(np.float64)
    assert np.abs(ref_hi - ref).max() > 10 * np.abs(got - ref).max()


def test_tile_weight_kernel_matches_host_layout(gpu_device):
    g = np.random.default_rng(41)
    w = torch.from_numpy(g.standard_normal((96, 320)).astype(np.float32)).to(torch.bfloat16).to(gpu_device)
    dst = torch.empty_like(w)
    N.check(N.lib().dtree_tile_weight(w.data_ptr(), dst.data_ptr(), 96, 320, stream()))
    torch.cuda.synchronize()
    assert torch.equal(dst, tile_weight(w))


def test_gemm_shapes_share_one_workspace(gpu_device):
    """Regression: a split-K GEMM with few column tiles followed by one with many
    tiles on the same workspace (the layer sequence QKV -> gate/up). The first
    one's partials must not land on the second one's tile counters."""
    g = np.random.default_rng(21)
    MP, L, K = 32, 25, 1024
    x = _rows(MP, L, K, g, gpu_device)
    w_small = torch.from_numpy(g.standard_normal((1536, K)).astype(np.float32) * 0.05).to(torch.bfloat16).to(gpu_device)
    w_big = torch.from_numpy(g.standard_normal((4096, K)).astype(np.float32) * 0.05).to(torch.bfloat16).to(gpu_device)
    ws = torch.zeros(N.lib().dtree_gemm_workspace_bytes(MP, 4096, K, 4), dtype=torch.uint8, device=gpu_device)
    out_s = torch.zeros(MP, 1536, device=gpu_device)
    out_b = torch.zeros(MP, 4096, device=gpu_device)
    for _ in range(2):
        _gemm(x, w_small, N.EPI_STORE_F32, 4, ws, out_f32=out_s)
        _gemm(x, w_big, N.EPI_STORE_F32, 4, ws, out_f32=out_b)
    torch.cuda.synchronize()
    xf = bf16_f32(x).astype(np.float64)
    np.testing.assert_allclose(out_s.cpu().numpy(), xf @ bf16_f32(w_small).T, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(out_b.cpu().numpy(), xf @ bf16_f32(w_big).T, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("split", [1, 4])
def test_gemm_residual_epilogue(gpu_device, split):
    g = np.random.default_rng(7)
    MP, L, N_, K = 32, 25, 512, 768
    x = _rows(MP, L, K, g, gpu_device)
    w = torch.from_numpy(g.standard_normal((N_, K)).astype(np.float32) * 0.05).to(torch.bfloat16).to(gpu_device)
    res = torch.zeros(MP, N_)
    res[:L] = torch.from_numpy(g.standard_normal((L, N_)).astype(np.float32))
    res = res.to(gpu_device)
    res0 = res.clone()
    gn = torch.from_numpy((1 + 0.1 * g.standard_normal(N_)).astype(np.float32)).to(torch.bfloat16).to(gpu_device)
    xg = torch.zeros(MP, N_, dtype=torch.bfloat16, device=gpu_device)
    ss = torch.zeros(N_ // 32, MP, device=gpu_device)
    hid = torch.zeros(MP, 3 * N_, dtype=torch.bfloat16, device=gpu_device)
    ws = torch.zeros(N.lib().dtree_gemm_workspace_bytes(MP, N_, K, split), dtype=torch.uint8, device=gpu_device)
    _gemm(x, w, N.EPI_RESIDUAL, split, ws, out_f32=res, out_bf16=xg, next_norm=gn, ss_out=ss,
          hidden_out=hid[:, N_:])
    torch.cuda.synchronize()
    ref = res0.cpu().numpy().astype(np.float64) + bf16_f32(x).astype(np.float64) @ bf16_f32(w).T.astype(np.float64)
    got = res.cpu().numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)
    assert np.all(got[L:] == 0)
    exp_xg = (torch.from_numpy(got) * gn.float().cpu()).to(torch.bfloat16)
    assert torch.equal(xg.cpu(), exp_xg)
    exp_ss = (got.astype(np.float64) ** 2).reshape(MP, N_ // 32, 32).sum(-1).T
    np.testing.assert_allclose(ss.cpu().numpy(), exp_ss, rtol=1e-5, atol=1e-5)
    assert torch.equal(hid[:, N_:2 * N_].cpu(), torch.from_numpy(got).to(torch.bfloat16))
    assert int(hid[:, :N_].float().abs().sum()) == 0 and int(hid[:, 2 * N_:].float().abs().sum()) == 0


def test_gemm_swiglu_epilogue(gpu_device):
    g = np.random.default_rng(9)
    MP, L, F, K = 32, 25, 384, 512
    x = _rows(MP, L, K, g, gpu_device)
    gate = torch.from_numpy(g.standard_normal((F, K)).astype(np.float32) * 0.05).to(torch.bfloat16)
    up = torch.from_numpy(g.standard_normal((F, K)).astype(np.float32) * 0.05).to(torch.bfloat16)
    from dtree_hip.weights import interleave_gate_up
    wgu = interleave_gate_up(gate, up).to(gpu_device)
    ss = torch.from_numpy(np.abs(g.standard_normal((3, MP))).astype(np.float32) + 0.5).to(gpu_device)
    act = torch.zeros(MP, F, dtype=torch.bfloat16, device=gpu_device)
    ws = torch.zeros(N.lib().dtree_gemm_workspace_bytes(MP, 2 * F, K, 2), dtype=torch.uint8, device=gpu_device)
    _gemm(x, wgu, N.EPI_SWIGLU, 2, ws, ss_in=ss, norm_dim=K, out_bf16=act)
    torch.cuda.synchronize()
    rs = 1.0 / np.sqrt(ss.cpu().numpy().sum(0) / K + 1e-6)
    xf = bf16_f32(x).astype(np.float64)
    gt = (xf @ gate.float().numpy().T) * rs[:, None]
    u = (xf @ up.float().numpy().T) * rs[:, None]
    ref = gt / (1 + np.exp(-gt)) * u
    np.testing.assert_allclose(bf16_f32(act), ref, rtol=1e-2, atol=1e-3)


# ---- 32-row tiled paths: stream-K (split_k -2), one workgroup per tile
# (split_k -1) and two or three per tile, one per part of K (split_k -3 / -4,
# n % 256 == 0); split_k 0 picks one of them per shape.
# Shapes chosen for the stream-K schedule: one unit; one K block over many
# column blocks (workgroups touching several blocks); one column block over 152
# K blocks (one block shared by 152 workgroups); and the Qwen3-4B layer shapes.
SK_SHAPES = [(64, 64), (4096, 64), (19456, 64), (64, 9728), (256, 1024), (6144, 2560), (2560, 4096),
             (19456, 2560), (2560, 9728)]
SCHEDULES = [-4, -3, -2, -1, 0]


def _skip_unsupported(n, k, sched):
    parts = {-3: 2, -4: 3}.get(sched)  # workgroups per 32-column tile
    if parts and (n % 256 or k < 64 * parts):
        pytest.skip("the split per-tile schedules need n % 256 == 0 and k >= 64 * parts")


def _sk_args(xt, xlo_t, wt, n, k, epi, ws, sched=0):
    a = N.GemmArgs()
    a.x = xt.data_ptr(); a.x_lo = xlo_t.data_ptr() if xlo_t is not None else None
    a.x_layout = a.w_layout = N.W_TILED; a.ldx = k; a.rows_padded = 32
    a.w = wt.data_ptr(); a.n = n; a.k = k; a.epilogue = epi; a.split_k = sched
    a.workspace = ws.data_ptr(); a.workspace_bytes = ws.numel()
    return a


@pytest.mark.parametrize("n,k", SK_SHAPES)
@pytest.mark.parametrize("lo", [False, True])
@pytest.mark.parametrize("sched", SCHEDULES)
def test_sk_gemm_store_f32(gpu_device, n, k, lo, sched):
    _skip_unsupported(n, k, sched)
    g = np.random.default_rng(n + k + lo)
    L = 25
    xf = np.zeros((32, k), np.float32)
    xf[:L] = g.standard_normal((L, k))
    hi = torch.from_numpy(xf).to(torch.bfloat16)
    lo_t = (torch.from_numpy(xf) - hi.float()).to(torch.bfloat16) if lo else None
    w = torch.from_numpy(g.standard_normal((n, k)).astype(np.float32) * 0.05).to(torch.bfloat16)
    ss = torch.from_numpy(np.abs(g.standard_normal((3, 32))).astype(np.float32) + 0.5).to(gpu_device)
    xt = tile_weight(hi.to(gpu_device))
    xlt = tile_weight(lo_t.to(gpu_device)) if lo else None
    wt = tile_weight(w.to(gpu_device))
    ws = torch.zeros(N.lib().dtree_gemm_workspace_bytes(32, n, k, 0), dtype=torch.uint8, device=gpu_device)
    outs = []
    for _ in range(2):
        out = torch.zeros(32, n, device=gpu_device)
        a = _sk_args(xt, xlt, wt, n, k, N.EPI_STORE_F32, ws, sched)
        a.ss_in = ss.data_ptr(); a.ss_tiles = 3; a.norm_dim = k; a.eps = 1e-6
        a.out_f32 = out.data_ptr(); a.ld_out_f32 = n
        N.check(N.lib().dtree_gemm_bf16(C.byref(a), stream()), "gemm")
        outs.append(out)
    torch.cuda.synchronize()
    rs = 1.0 / np.sqrt(ss.cpu().numpy().sum(0) / k + 1e-6)
    xin = hi.double() + (lo_t.double() if lo else 0)
    ref = (xin.numpy() @ bf16_f32(w).T.astype(np.float64)) * rs[:, None]
    got = outs[0].cpu().numpy()
    assert np.abs(got - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())
    assert torch.equal(outs[0], outs[1])  # fixed reduction order
    assert int(ws[: (n // 32) * 4].view(torch.int32).abs().sum()) == 0  # counters self-reset


@pytest.mark.parametrize("n,k", [(512, 768), (2560, 4096), (2560, 9728)])
@pytest.mark.parametrize("sched", SCHEDULES)
def test_sk_gemm_residual_epilogue(gpu_device, n, k, sched):
    _skip_unsupported(n, k, sched)
    g = np.random.default_rng(n + 3 * k)
    L = 25
    x = _rows(32, L, k, g, gpu_device)
    w = torch.from_numpy(g.standard_normal((n, k)).astype(np.float32) * 0.05).to(torch.bfloat16).to(gpu_device)
    res = torch.zeros(32, n)
    res[:L] = torch.from_numpy(g.standard_normal((L, n)).astype(np.float32))
    res = res.to(gpu_device)
    res0 = res.clone()
    gn = torch.from_numpy((1 + 0.1 * g.standard_normal(n)).astype(np.float32)).to(torch.bfloat16).to(gpu_device)
    xg = torch.zeros(32, n, dtype=torch.bfloat16, device=gpu_device)
    ss = torch.zeros(n // 32, 32, device=gpu_device)
    hid = torch.zeros(32, n, dtype=torch.bfloat16, device=gpu_device)
    ws = torch.zeros(N.lib().dtree_gemm_workspace_bytes(32, n, k, 0), dtype=torch.uint8, device=gpu_device)
    _gemm(x, w, N.EPI_RESIDUAL, sched, ws, out_f32=res, out_bf16=xg, next_norm=gn, ss_out=ss, hidden_out=hid,
          tiled=True)
    torch.cuda.synchronize()
    ref = res0.cpu().numpy().astype(np.float64) + bf16_f32(x).astype(np.float64) @ bf16_f32(w).T.astype(np.float64)
    got = res.cpu().numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)
    assert np.all(got[L:] == 0)
    assert torch.equal(xg.cpu(), (torch.from_numpy(got) * gn.float().cpu()).to(torch.bfloat16))
    exp_ss = (got.astype(np.float64) ** 2).reshape(32, n // 32, 32).sum(-1).T
    np.testing.assert_allclose(ss.cpu().numpy(), exp_ss, rtol=1e-5, atol=1e-5)
    assert torch.equal(hid.cpu(), torch.from_numpy(got).to(torch.bfloat16))


@pytest.mark.parametrize("F,k", [(384, 512), (9728, 2560)])
@pytest.mark.parametrize("sched", SCHEDULES)
def test_sk_gemm_swiglu_epilogue(gpu_device, F, k, sched):
    _skip_unsupported(2 * F, k, sched)
    g = np.random.default_rng(F + k)
    L = 25
    x = _rows(32, L, k, g, gpu_device)
    gate = torch.from_numpy(g.standard_normal((F, k)).astype(np.float32) * 0.05).to(torch.bfloat16)
    up = torch.from_numpy(g.standard_normal((F, k)).astype(np.float32) * 0.05).to(torch.bfloat16)
    from dtree_hip.weights import interleave_gate_up
    wgu = interleave_gate_up(gate, up).to(gpu_device)
    ss = torch.from_numpy(np.abs(g.standard_normal((3, 32))).astype(np.float32) + 0.5).to(gpu_device)
    act = torch.zeros(32, F, dtype=torch.bfloat16, device=gpu_device)
    ws = torch.zeros(N.lib().dtree_gemm_workspace_bytes(32, 2 * F, k, 0), dtype=torch.uint8, device=gpu_device)
    _gemm(x, wgu, N.EPI_SWIGLU, sched, ws, ss_in=ss, norm_dim=k, out_bf16=act, tiled=True)
    torch.cuda.synchronize()
    rs = 1.0 / np.sqrt(ss.cpu().numpy().sum(0) / k + 1e-6)
    xf = bf16_f32(x).astype(np.float64)
    gt = (xf @ gate.float().numpy().T) * rs[:, None]
    u = (xf @ up.float().numpy().T) * rs[:, None]
    ref = gt / (1 + np.exp(-gt)) * u
    np.testing.assert_allclose(bf16_f32(act), ref, rtol=1e-2, atol=1e-3)


def _attention(qkv, cache, layer, desc, out, ws, Hq, Hkv, max_past, cos, sin, qn, kn, write=1, MP=32):
    a = N.AttnArgs()
    a.qkv = qkv.data_ptr(); a.ld_qkv = qkv.shape[1]
    a.q_norm = qn.data_ptr() if qn is not None else None
    a.k_norm = kn.data_ptr() if kn is not None else None
    a.eps = 1e-6
    a.rope_cos = cos.data_ptr(); a.rope_sin = sin.data_ptr()
    a.k_pages = cache.k_ptr(layer); a.v_pages = cache.v_ptr(layer); a.page_table = cache.page_table.data_ptr()
    a.desc = desc.data_ptr(); a.out = out.data_ptr(); a.ld_out = out.shape[1]
    a.num_heads = Hq; a.num_kv_heads = Hkv; a.head_dim = 128; a.rows_padded = MP
    a.scale = 128 ** -0.5; a.max_past_length = max_past; a.write_cache = write
    a.workspace = ws.data_ptr(); a.workspace_bytes = ws.numel()
    N.check(N.lib().dtree_tree_attention(C.byref(a), stream()), "attention")


def _attention_case(dev, P, parents, Hq=32, Hkv=8, seed=0, permute_pages=True, max_past=None, MP=32):
    g = np.random.default_rng(seed)
    D = 128
    L = len(parents)
    max_past = max(P, 64) if max_past is None else max_past
    n_pages = (max_past + MP + 63) // 64
    order = torch.from_numpy(g.permutation(n_pages).astype(np.int32)) if permute_pages else None
    cache = PagedKVCache(1, Hkv, D, max_past + MP, device=dev, page_order=order)
    kpre = (g.standard_normal((P, Hkv, D)) * 0.5).astype(np.float32)
    vpre = (g.standard_normal((P, Hkv, D)) * 0.5).astype(np.float32)
    if P:
        cache.write_logical(0, torch.from_numpy(kpre), torch.from_numpy(vpre))
    cache.offset = P
    qkv = np.zeros((MP, (Hq + 2 * Hkv) * D), np.float32)
    qkv[:L] = g.standard_normal((L, (Hq + 2 * Hkv) * D)).astype(np.float32)
    qn = (1 + 0.1 * g.standard_normal(D)).astype(np.float32)
    kn = (1 + 0.1 * g.standard_normal(D)).astype(np.float32)
    depth = [0] * L
    for i in range(1, L):
        depth[i] = depth[parents[i]] + 1
    pos = [P + d for d in depth]
    desc = device_desc([0] * L, pos, parents, P, dev)
    cos = torch.zeros(MP, 64, device=dev)
    sin = torch.zeros(MP, 64, device=dev)
    N.check(N.lib().dtree_rope_table(desc.data_ptr(), MP, D, 1e6, cos.data_ptr(), sin.data_ptr(), stream()))
    qn_t = torch.from_numpy(qn).to(torch.bfloat16).to(dev)
    kn_t = torch.from_numpy(kn).to(torch.bfloat16).to(dev)
    # stale rows past the tree: the kernel must zero them
    out = torch.full((MP, Hq * D), 7.0, dtype=torch.bfloat16, device=dev)
    ws = torch.zeros(N.lib().dtree_attention_workspace_bytes(Hq, D, max_past, MP), dtype=torch.uint8, device=dev)
    qkv_t = torch.from_numpy(qkv).to(dev)
    _attention(qkv_t, cache, 0, desc, out, ws, Hq, Hkv, max_past, cos, sin, qn_t, kn_t, MP=MP)
    torch.cuda.synchronize()

    # oracle: q/k norm (bf16 norm weights), RoPE, masked SDPA over [prefix ; tree]
    qnf, knf = bf16_f32(qn_t), bf16_f32(kn_t)
    q = oq.rms_norm(qkv[:L, : Hq * D].reshape(L, Hq, D), qnf, 1e-6)
    k = oq.rms_norm(qkv[:L, Hq * D:(Hq + Hkv) * D].reshape(L, Hkv, D), knf, 1e-6)
    v = qkv[:L, (Hq + Hkv) * D:].reshape(L, Hkv, D)
    q = oq.rope(q, np.array(pos), 1e6)
    k = oq.rope(k, np.array(pos), 1e6)
    kp = oq.bf16_to_f32(oq.f32_to_bf16_bits(kpre))
    vp = oq.bf16_to_f32(oq.f32_to_bf16_bits(vpre))
    ref = oq.sdpa(q, np.concatenate([kp, k]), np.concatenate([vp, v]), tree_mask(parents, P), D ** -0.5)
    return cache, out, ref.reshape(L, Hq * D), k, v, ws


@pytest.mark.parametrize("P", [0, 1, 100, 128, 129, 512, 1000])
@pytest.mark.parametrize("shape", ["chain25", "star25", "random25", "single", "chain32"])
def test_tree_attention_matches_oracle(gpu_device, P, shape, attn_kernel):
    L = {"chain25": 25, "star25": 25, "random25": 25, "single": 1, "chain32": 32}[shape]
    if shape.startswith("chain"):
        parents = [-1] + list(range(L - 1))
    elif shape == "star25":
        parents = [-1] + [0] * (L - 1)
    elif shape == "single":
        parents = [-1]
    else:
        parents = random_tree(L, seed=P + 11)
    cache, out, ref, k, v, ws = _attention_case(gpu_device, P, parents, seed=P + L)
    got = bf16_f32(out)
    scale = np.abs(ref).max()
    assert np.abs(got[:L] - ref).max() <= 2e-2 * scale, np.abs(got[:L] - ref).max() / scale
    assert np.all(got[L:] == 0)
    # tree K/V appended at [P, P+L): K = bf16(rope(k_norm(k))), V = bf16(v)
    kc = bf16_f32(cache.logical_keys(0, P + L))[P:]
    vc = bf16_f32(cache.logical_values(0, P + L))[P:]
    np.testing.assert_allclose(kc, k, rtol=1e-2, atol=1e-2)
    np.testing.assert_array_equal(vc, oq.bf16_to_f32(oq.f32_to_bf16_bits(v)))
    Hq = 32
    assert int(ws[:4].view(torch.int32).item()) == 0  # error word clear
    assert int(ws[64: 64 + Hq * 4].view(torch.int32).abs().sum()) == 0  # counters self-reset


@pytest.mark.parametrize("P,max_past,noalloc", [(1000, 1024, False), (1000, 1024, True), (3000, 4096, False)])
def test_group_attention_give_up_is_reported(gpu_device, monkeypatch, P, max_past, noalloc):
    """The per-KV-group kernel's bounded split wait, made to give up from the
    host (DTREE_TEST_SPIN_LIMIT=0: a split that is not the last to arrive
    stops waiting at once; every workgroup still runs to its end):
    dtree_attention_status reports it and clears the word, the counters are
    back at zero, and the next launch with the normal bound is correct and
    reports nothing. Also through the allocation-free entry point (whose
    32 MiB scratch holds the grid for 1024 keys)."""
    monkeypatch.setenv("DTREE_ATTN_KERNEL", "group")
    parents = random_tree(25, seed=3)
    cache, out, ref, k, v, ws = _attention_case(gpu_device, P, parents, seed=5, max_past=max_past)
    lib = N.lib()
    status = torch.zeros(1, dtype=torch.int32, device=gpu_device)
    ws_ptr = None if noalloc else ws.data_ptr()

    def launch():
        a = N.AttnArgs()
        qkv = launch.qkv
        a.qkv = qkv.data_ptr(); a.ld_qkv = qkv.shape[1]
        a.q_norm = None; a.k_norm = None; a.eps = 1e-6
        a.rope_cos = launch.cos.data_ptr(); a.rope_sin = launch.sin.data_ptr()
        a.k_pages = cache.k_ptr(0); a.v_pages = cache.v_ptr(0); a.page_table = cache.page_table.data_ptr()
        a.desc = launch.desc.data_ptr(); a.out = out.data_ptr(); a.ld_out = out.shape[1]
        a.num_heads = 32; a.num_kv_heads = 8; a.head_dim = 128; a.rows_padded = 32
        a.scale = 128 ** -0.5; a.max_past_length = max_past; a.write_cache = 0
        a.workspace = ws.data_ptr(); a.workspace_bytes = ws.numel()
        f = lib.dtree_tree_attention_noalloc if noalloc else lib.dtree_tree_attention
        N.check(f(C.byref(a), stream()), "attention")
        N.check(lib.dtree_attention_status(ws_ptr, status.data_ptr(), stream()), "attention status")
        torch.cuda.synchronize()

    g = np.random.default_rng(9)
    launch.qkv = torch.from_numpy(g.standard_normal((32, (32 + 16) * 128)).astype(np.float32)).to(gpu_device)
    depth = [0] * 25
    for i in range(1, 25):
        depth[i] = depth[parents[i]] + 1
    launch.desc = device_desc([0] * 25, [P + d for d in depth], parents, P, gpu_device)
    launch.cos = torch.zeros(32, 64, device=gpu_device)
    launch.sin = torch.zeros(32, 64, device=gpu_device)
    N.check(lib.dtree_rope_table(launch.desc.data_ptr(), 32, 128, 1e6, launch.cos.data_ptr(), launch.sin.data_ptr(),
                                 stream()))
    launch()
    assert int(status.item()) == 0
    want = out.clone()
    monkeypatch.setenv("DTREE_TEST_SPIN_LIMIT", "0")
    out.fill_(7.0)
    launch()
    assert int(status.item()) == 1, "a give-up was not reported"
    monkeypatch.delenv("DTREE_TEST_SPIN_LIMIT")
    status.zero_()
    launch()
    assert int(status.item()) == 0  # the word was cleared, nothing new
    assert torch.equal(out, want)
    if not noalloc:
        assert int(ws[:4096].view(torch.int32).abs().sum()) == 0  # error word and counters at zero


@pytest.mark.parametrize("P,max_past", [(300, 300), (512, 512), (1000, 1024), (1500, 1536), (1750, 1792),
                                        (1000, 4096)])
def test_head_attention_flag_exchange_matches_counter_combine(gpu_device, monkeypatch, P, max_past):
    """The per-head kernel's flag exchange (2..8 splits; every split combines
    the output units u with u % splits == split from its partners' (value,
    flag) pairs) against the last-arriver combine (DTREE_ATTN_EXCHANGE=counter)
    and the oracle; the launch raises every head's epoch by exactly one
    (launches in a row on one workspace: the give-up test below). The last
    case's grid is sized for 4096 keys, whose partials would be combined by a
    second launch: its 1000-key step still takes the exchange (five splits)
    and the second launch finds nothing to do."""
    monkeypatch.setenv("DTREE_ATTN_KERNEL", "head")
    parents = random_tree(25, seed=P)
    Hq = 32
    monkeypatch.setenv("DTREE_ATTN_EXCHANGE", "counter")
    _, out_cnt, ref, *_ = _attention_case(gpu_device, P, parents, seed=P + 3, max_past=max_past)
    monkeypatch.delenv("DTREE_ATTN_EXCHANGE")
    cache, out_ll, ref2, k, v, ws = _attention_case(gpu_device, P, parents, seed=P + 3, max_past=max_past)
    np.testing.assert_array_equal(ref, ref2)
    epochs = ws[4096: 4096 + 4 * Hq].view(torch.int32)
    assert torch.all(epochs == 1), epochs
    got = bf16_f32(out_ll)[:25]
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() <= 2e-2 * scale
    # same partials, same split-order sum: at most one bf16 rounding apart
    diff = np.abs(got - bf16_f32(out_cnt)[:25])
    assert diff.max() <= 2 ** -7 * np.abs(got).max(), diff.max()


@pytest.mark.parametrize("noalloc", [False, True])
def test_head_attention_give_up_is_reported(gpu_device, monkeypatch, noalloc):
    """The flag exchange's bounded wait, made to give up before its first poll
    (DTREE_TEST_SPIN_LIMIT=-1; every workgroup still runs to its end): the
    status query reports it, clears the word and moves every head's epoch
    2^16 ahead; the next launch with the normal bound is correct and reports
    nothing. Also through the allocation-free entry point."""
    monkeypatch.setenv("DTREE_ATTN_KERNEL", "head")
    P, max_past, Hq = 1000, 1024, 32
    parents = random_tree(25, seed=4)
    cache, out, ref, k, v, ws = _attention_case(gpu_device, P, parents, seed=6, max_past=max_past)
    lib = N.lib()
    status = torch.zeros(1, dtype=torch.int32, device=gpu_device)
    ws_ptr = None if noalloc else ws.data_ptr()
    g = np.random.default_rng(10)
    qkv = torch.from_numpy(g.standard_normal((32, (Hq + 16) * 128)).astype(np.float32)).to(gpu_device)
    depth = [0] * 25
    for i in range(1, 25):
        depth[i] = depth[parents[i]] + 1
    desc = device_desc([0] * 25, [P + d for d in depth], parents, P, gpu_device)
    cos = torch.zeros(32, 64, device=gpu_device)
    sin = torch.zeros(32, 64, device=gpu_device)
    N.check(lib.dtree_rope_table(desc.data_ptr(), 32, 128, 1e6, cos.data_ptr(), sin.data_ptr(), stream()))

    def launch():
        a = N.AttnArgs()
        a.qkv = qkv.data_ptr(); a.ld_qkv = qkv.shape[1]
        a.q_norm = None; a.k_norm = None; a.eps = 1e-6
        a.rope_cos = cos.data_ptr(); a.rope_sin = sin.data_ptr()
        a.k_pages = cache.k_ptr(0); a.v_pages = cache.v_ptr(0); a.page_table = cache.page_table.data_ptr()
        a.desc = desc.data_ptr(); a.out = out.data_ptr(); a.ld_out = out.shape[1]
        a.num_heads = Hq; a.num_kv_heads = 8; a.head_dim = 128; a.rows_padded = 32
        a.scale = 128 ** -0.5; a.max_past_length = max_past; a.write_cache = 0
        a.workspace = ws.data_ptr(); a.workspace_bytes = ws.numel()
        f = lib.dtree_tree_attention_noalloc if noalloc else lib.dtree_tree_attention
        N.check(f(C.byref(a), stream()), "attention")
        N.check(lib.dtree_attention_status(ws_ptr, status.data_ptr(), stream()), "attention status")
        torch.cuda.synchronize()

    launch()
    assert int(status.item()) == 0
    want = out.clone()
    if not noalloc:
        e0 = ws[4096: 4096 + 4 * Hq].view(torch.int32).clone()
    monkeypatch.setenv("DTREE_TEST_SPIN_LIMIT", "-1")
    out.fill_(7.0)
    launch()
    assert int(status.item()) == 1, "a give-up was not reported"
    if not noalloc:
        e1 = ws[4096: 4096 + 4 * Hq].view(torch.int32)
        assert torch.all(e1 >= e0 + (1 << 16)), (e0, e1)
    monkeypatch.delenv("DTREE_TEST_SPIN_LIMIT")
    status.zero_()
    launch()
    assert int(status.item()) == 0  # the word was cleared, nothing new
    assert torch.equal(out, want)
    if not noalloc:
        assert int(ws[:4].view(torch.int32).item()) == 0


@pytest.mark.parametrize("P", [0, 129, 1000])
@pytest.mark.parametrize("MP,L,shape", [(64, 40, "random"), (96, 65, "random"), (96, 65, "chain"),
                                        (96, 65, "star"), (96, 33, "random"), (128, 128, "random")])
def test_tree_attention_more_than_32_nodes(gpu_device, P, MP, L, shape, attn_kernel):
    """Trees of 33..128 nodes: query blocks of 32 rows, tree chunks of 32
    keys masked by ancestor word w (nodes 32w..32w+31), cache rows appended
    once, rows past the tree zero."""
    parents = {"random": random_tree(L, seed=P + L), "chain": [-1] + list(range(L - 1)),
               "star": [-1] + [0] * (L - 1)}[shape]
    cache, out, ref, k, v, ws = _attention_case(gpu_device, P, parents, seed=P + L + MP, MP=MP)
    got = bf16_f32(out)
    assert np.abs(got[:L] - ref).max() <= 2e-2 * np.abs(ref).max()
    assert np.all(got[L:] == 0)
    kc = bf16_f32(cache.logical_keys(0, P + L))[P:]
    vc = bf16_f32(cache.logical_values(0, P + L))[P:]
    np.testing.assert_allclose(kc, k, rtol=1e-2, atol=1e-2)
    np.testing.assert_array_equal(vc, oq.bf16_to_f32(oq.f32_to_bf16_bits(v)))
    assert int(ws[: 64 + 32 * (MP // 32) * 4].view(torch.int32).abs().sum()) == 0  # counters self-reset


@pytest.mark.parametrize("P,max_past,MP,L", [(0, 64, 32, 25), (100, 128, 32, 25), (300, 2000, 32, 25),
                                             (1000, 4096, 32, 25), (4000, 4096, 32, 25), (3000, 4096, 96, 65)])
def test_tree_attention_long_prefix_separate_combine(gpu_device, P, max_past, MP, L, attn_kernel):
    """Grids sized for long prefixes combine the workgroup partials in a
    launch of their own (more than 128 KB of partials per head), also for
    several query blocks; short descriptors (one split) still write the
    output from the main kernel."""
    parents = random_tree(L, seed=P + 3)
    cache, out, ref, k, v, ws = _attention_case(gpu_device, P, parents, Hq=8, Hkv=2, seed=P + 1, max_past=max_past,
                                                MP=MP)
    got = bf16_f32(out)
    assert np.abs(got[:L] - ref).max() <= 2e-2 * np.abs(ref).max()
    assert np.all(got[L:] == 0)
    _, out2, *_ = _attention_case(gpu_device, P, parents, Hq=8, Hkv=2, seed=P + 1, max_past=max_past, MP=MP)
    assert torch.equal(out, out2)


def _gated_attention_case(dev, P, parents, max_past, Hq=8, Hkv=2, seed=0, MP=32):
    """Qwen3.5 gated attention: head_dim 256, per head [q | gate] in the QKV
    row, q/k RMSNorm, RoPE on the first 64 dims (base 1e5), output times
    sigmoid(gate) (qwen35_tree.py:503-540)."""
    from oracle import qwen35 as o35
    g = np.random.default_rng(seed)
    D, RD = 256, 64
    L = len(parents)
    cache = PagedKVCache(1, Hkv, D, max_past + MP, device=dev,
                         page_order=torch.from_numpy(g.permutation((max_past + MP + 63) // 64).astype(np.int32)))
    kpre = (g.standard_normal((P, Hkv, D)) * 0.5).astype(np.float32)
    vpre = (g.standard_normal((P, Hkv, D)) * 0.5).astype(np.float32)
    if P:
        cache.write_logical(0, torch.from_numpy(kpre), torch.from_numpy(vpre))
    cache.offset = P
    W = 2 * Hq * D + 2 * Hkv * D
    qkv = np.zeros((MP, W), np.float32)
    qkv[:L] = g.standard_normal((L, W)).astype(np.float32)
    qn = (1 + 0.1 * g.standard_normal(D)).astype(np.float32)
    kn = (1 + 0.1 * g.standard_normal(D)).astype(np.float32)
    depth = [0] * L
    for i in range(1, L):
        depth[i] = depth[parents[i]] + 1
    pos = [P + d for d in depth]
    desc = device_desc([0] * L, pos, parents, P, dev)
    cos = torch.zeros(MP, RD // 2, device=dev)
    sin = torch.zeros(MP, RD // 2, device=dev)
    N.check(N.lib().dtree_rope_table(desc.data_ptr(), MP, RD, 1e5, cos.data_ptr(), sin.data_ptr(), stream()))
    qn_t = torch.from_numpy(qn).to(torch.bfloat16).to(dev)
    kn_t = torch.from_numpy(kn).to(torch.bfloat16).to(dev)
    out = torch.full((MP, Hq * D), 7.0, dtype=torch.bfloat16, device=dev)
    ws = torch.zeros(N.lib().dtree_attention_workspace_bytes(Hq, D, max_past, MP), dtype=torch.uint8, device=dev)
    qkv_t = torch.from_numpy(qkv).to(dev)
    a = N.AttnArgs()
    a.qkv = qkv_t.data_ptr(); a.ld_qkv = W
    a.q_norm = qn_t.data_ptr(); a.k_norm = kn_t.data_ptr(); a.eps = 1e-6
    a.rope_cos = cos.data_ptr(); a.rope_sin = sin.data_ptr()
    a.k_pages = cache.k_ptr(0); a.v_pages = cache.v_ptr(0); a.page_table = cache.page_table.data_ptr()
    a.desc = desc.data_ptr(); a.out = out.data_ptr(); a.ld_out = Hq * D
    a.num_heads = Hq; a.num_kv_heads = Hkv; a.head_dim = D; a.rows_padded = MP
    a.scale = D ** -0.5; a.max_past_length = max_past; a.write_cache = 1
    a.workspace = ws.data_ptr(); a.workspace_bytes = ws.numel()
    a.rope_dims = RD; a.gated = 1
    N.check(N.lib().dtree_tree_attention(C.byref(a), stream()), "attention")
    torch.cuda.synchronize()
    qg = qkv[:L, : 2 * Hq * D].reshape(L, Hq, 2 * D)
    q, gate = qg[..., :D], qg[..., D:].reshape(L, Hq * D)
    k = qkv[:L, 2 * Hq * D:(2 * Hq + Hkv) * D].reshape(L, Hkv, D)
    v = qkv[:L, (2 * Hq + Hkv) * D:].reshape(L, Hkv, D)
    q = o35.partial_rope(oq.rms_norm(q, bf16_f32(qn_t), 1e-6), np.array(pos), RD, 1e5)
    k = o35.partial_rope(oq.rms_norm(k, bf16_f32(kn_t), 1e-6), np.array(pos), RD, 1e5)
    kp = oq.bf16_to_f32(oq.f32_to_bf16_bits(kpre))
    vp = oq.bf16_to_f32(oq.f32_to_bf16_bits(vpre))
    ref = oq.sdpa(q, np.concatenate([kp, k]), np.concatenate([vp, v]), tree_mask(parents, P), D ** -0.5)
    ref = ref.reshape(L, Hq * D) / (1.0 + np.exp(-gate))
    return out, ref


@pytest.mark.parametrize("P,max_past,MP,L", [(0, 64, 32, 25), (100, 128, 32, 25), (700, 2048, 32, 25),
                                             (2000, 2048, 32, 25), (0, 64, 96, 65), (1500, 2048, 96, 65)])
def test_gated_attention_head_dim_256(gpu_device, P, max_past, MP, L, attn_kernel):
    """The Qwen3.5 geometry directly against the oracle: staged query rows
    (one query block) and per-wave rows (more than 32 nodes), with the
    in-kernel combine (short grids) and the separate combine launch
    (max_past 2048: 17 splits of 32 KB per head)."""
    parents = random_tree(L, seed=P + 7)
    out, ref = _gated_attention_case(gpu_device, P, parents, max_past, seed=P + 2, MP=MP)
    got = bf16_f32(out)
    assert np.abs(got[:L] - ref).max() <= 2e-2 * np.abs(ref).max()
    assert np.all(got[L:] == 0)
    out2, _ = _gated_attention_case(gpu_device, P, parents, max_past, seed=P + 2, MP=MP)
    assert torch.equal(out, out2)


def test_tree_attention_gqa_small_and_deterministic(gpu_device, attn_kernel):
    parents = random_tree(25, seed=5)
    cache, out, ref, *_ = _attention_case(gpu_device, 300, parents, Hq=8, Hkv=2, seed=4, max_past=2000)
    got = bf16_f32(out)
    assert np.abs(got[:25] - ref).max() <= 2e-2 * np.abs(ref).max()
    cache2, out2, *_ = _attention_case(gpu_device, 300, parents, Hq=8, Hkv=2, seed=4, max_past=2000)
    assert torch.equal(out, out2)


def _lmhead(x, E, dev, logits=None, ss=None, layout=0):
    MP = x.shape[0]
    lib = N.lib()
    cand = torch.zeros(lib.dtree_lmhead_candidates_bytes(MP), dtype=torch.uint8, device=dev)
    if layout == N.W_TILED:
        x = tile_weight(x)
    N.check(lib.dtree_lmhead_argmax(x.data_ptr(), None, layout, x.shape[1], MP, E.data_ptr(), layout, None,
                                    E.shape[0], E.shape[1],
                                    ss.data_ptr() if ss is not None else None, ss.shape[0] if ss is not None else 0,
                                    1e-6, logits.data_ptr() if logits is not None else None, cand.data_ptr(),
                                    stream()))
    return cand, lib.dtree_lmhead_candidate_blocks(E.shape[0], MP)


def _walk(cand, nblocks, desc, dev, rows=32):
    res = torch.zeros(3 + 2 * N.MAX_NODES, dtype=torch.int32, device=dev)
    N.check(N.lib().dtree_accept_walk(desc.data_ptr(), cand.data_ptr(), nblocks, rows, res.data_ptr(), stream()))
    torch.cuda.synchronize()
    r = res.cpu().numpy()
    n, bonus, L = int(r[0]), int(r[1]), int(r[2])
    return list(r[3:3 + n]), bonus, list(r[3 + N.MAX_NODES:3 + N.MAX_NODES + L])


@pytest.mark.parametrize("V", [4096, 151936])
@pytest.mark.parametrize("tiled", [False, True])
def test_lmhead_argmax_and_logits(gpu_device, V, tiled):
    g = np.random.default_rng(V)
    H, L = 2560, 25
    x = _rows(32, L, H, g, gpu_device)
    E = torch.from_numpy((g.standard_normal((V, H)) * 0.02).astype(np.float32)).to(torch.bfloat16).to(gpu_device)
    logits = torch.zeros(32, V, device=gpu_device)
    if tiled:
        cand, nb = _lmhead(x, tile_weight(E), gpu_device, logits=logits, layout=N.W_TILED)
    else:
        cand, nb = _lmhead(x, E, gpu_device, logits=logits)
    desc = device_desc([0] * L, [0] * L, [-1] + [0] * (L - 1), 0, gpu_device)
    _, _, post = _walk(cand, nb, desc, gpu_device)
    ref = bf16_f32(x)[:L] @ bf16_f32(E).T
    np.testing.assert_allclose(logits.cpu().numpy()[:L], ref, rtol=1e-4, atol=1e-4)
    srt = np.sort(ref, axis=-1)
    margin = srt[:, -1] - srt[:, -2]
    want = np.argmax(ref, axis=-1)
    for m in range(L):
        if margin[m] > 1e-3:
            assert post[m] == want[m]
    assert post == list(np.argmax(logits.cpu().numpy()[:L], axis=-1))


@pytest.mark.parametrize("tiled", [False, True])
def test_lmhead_argmax_96_rows(gpu_device, tiled):
    """65 tree rows (rows_padded 96, three 32-row blocks of candidates): every
    row's argmax through the walk equals the fp64 product's where the top-2
    margin is clear, and the RMSNorm statistics of every block apply."""
    g = np.random.default_rng(965)
    V, H, L, MP = 4096, 1024, 65, 96
    x = _rows(MP, L, H, g, gpu_device)
    E = torch.from_numpy((g.standard_normal((V, H)) * 0.02).astype(np.float32)).to(torch.bfloat16).to(gpu_device)
    ss_np = np.abs(g.standard_normal((MP // 32, H // 32, 32))).astype(np.float32) + 0.5
    ss = torch.from_numpy(ss_np).to(gpu_device)
    logits = torch.zeros(MP, V, device=gpu_device)
    lib = N.lib()
    cand = torch.zeros(lib.dtree_lmhead_candidates_bytes(MP), dtype=torch.uint8, device=gpu_device)
    xin, Ein = (tile_weight(x), tile_weight(E)) if tiled else (x, E)
    lay = N.W_TILED if tiled else N.W_ROWMAJOR
    N.check(lib.dtree_lmhead_argmax(xin.data_ptr(), None, lay, H, MP, Ein.data_ptr(), lay, None, V, H,
                                    ss.data_ptr(), H // 32, 1e-6, logits.data_ptr(), cand.data_ptr(), stream()),
            "lmhead 96")
    nb = lib.dtree_lmhead_candidate_blocks(V, MP)
    parents = [-1] + [(i - 1) // 2 for i in range(1, L)]
    desc = device_desc([0] * L, list(range(L)), parents, 0, gpu_device)
    _, _, post = _walk(cand, nb, desc, gpu_device, rows=MP)
    rs = 1.0 / np.sqrt(ss_np.sum(1).reshape(MP) / H + 1e-6)
    ref = (bf16_f32(x).astype(np.float64) @ bf16_f32(E).T.astype(np.float64)) * rs[:, None]
    np.testing.assert_allclose(logits.cpu().numpy()[:L], ref[:L], rtol=1e-4, atol=1e-4)
    assert post == list(np.argmax(logits.cpu().numpy()[:L], axis=-1))
    srt = np.sort(ref[:L], axis=-1)
    clear = srt[:, -1] - srt[:, -2] > 1e-3
    assert np.array_equal(np.asarray(post)[clear], np.argmax(ref[:L], axis=-1)[clear])


def test_lmhead_first_index_on_tie(gpu_device):
    # tests/test_adapters.py:51-81: rows 0 and 70 of the head equal -> index 0
    V, H = 128, 64
    E = torch.zeros(V, H)
    E[0] = 1.0
    E[70] = 1.0
    E = E.to(torch.bfloat16).to(gpu_device)
    x = torch.zeros(32, H, dtype=torch.bfloat16, device=gpu_device)
    x[0] = 1.0
    cand, nb = _lmhead(x, E, gpu_device)
    desc = device_desc([0], [0], [-1], 0, gpu_device)
    _, _, post = _walk(cand, nb, desc, gpu_device)
    assert post == [0]
    # tie across workgroups: 151936-wide vocab, equal rows at 5 and 151900
    V = 151936
    E = torch.zeros(V, H)
    E[151900] = 1.0
    E[5] = 1.0
    E = E.to(torch.bfloat16).to(gpu_device)
    cand, nb = _lmhead(x, E, gpu_device)
    _, _, post = _walk(cand, nb, desc, gpu_device)
    assert post == [5]


@pytest.mark.parametrize("seed", range(4))
def test_walk_and_compaction_match_oracle(gpu_device, seed):
    g = np.random.default_rng(seed)
    L, V, H = 25, 64, 64
    parents = random_tree(L, seed)
    # distinct tokens among siblings
    tokens = [int(g.integers(0, V))]
    for i in range(1, L):
        used = {tokens[j] for j in range(1, i) if parents[j] == parents[i]}
        t = int(g.integers(0, V))
        while t in used:
            t = int(g.integers(0, V))
        tokens.append(t)
    child_maps = [dict() for _ in range(L)]
    for i in range(1, L):
        child_maps[parents[i]][tokens[i]] = i
    # posterior: follow a random path by making argmax = some child token, then stop
    post = [int(g.integers(0, V)) for _ in range(L)]
    cur = 0
    while True:
        ch = [j for j in range(1, L) if parents[j] == cur]
        if not ch or g.random() < 0.15:
            break
        nxt = ch[int(g.integers(0, len(ch)))]
        post[cur] = tokens[nxt]
        cur = nxt
    # identity LM head: x rows one-hot at the posterior token
    E = torch.eye(V, H).to(torch.bfloat16).to(gpu_device)
    x = torch.zeros(32, H)
    for m in range(L):
        x[m, post[m]] = 1.0
    x = x.to(torch.bfloat16).to(gpu_device)
    cand, nb = _lmhead(x, E, gpu_device)
    P = 70 + seed
    depth = [0] * L
    for i in range(1, L):
        depth[i] = depth[parents[i]] + 1
    desc = device_desc(tokens, [P + d for d in depth], parents, P, gpu_device)
    acc, bonus, got_post = _walk(cand, nb, desc, gpu_device)
    o_acc, o_bonus = otree.follow_verified_tree(child_maps, post)
    assert got_post == post
    assert acc == o_acc and bonus == o_bonus
    d = read_desc(desc)
    assert d.n_accepted == len(acc) and list(d.accepted[: len(acc)]) == acc

    # compaction of 3 layers x 2 kv heads, permuted pages; hidden select
    layers, Hkv, D = 3, 2, 128
    order = torch.from_numpy(g.permutation(4).astype(np.int32))
    cache = PagedKVCache(layers, Hkv, D, 256, device=gpu_device, page_order=order)
    before_k, before_v = [], []
    for li in range(layers):
        k = torch.from_numpy(g.standard_normal((P + L, Hkv, D)).astype(np.float32))
        v = torch.from_numpy(g.standard_normal((P + L, Hkv, D)).astype(np.float32))
        cache.write_logical(li, k, v)
        before_k.append(bf16_f32(cache.logical_keys(li, P + L)))
        before_v.append(bf16_f32(cache.logical_values(li, P + L)))
    hid = torch.from_numpy(g.standard_normal((32, 96)).astype(np.float32)).to(torch.bfloat16).to(gpu_device)
    hsel = torch.zeros(32, 96, dtype=torch.bfloat16, device=gpu_device)
    N.check(N.lib().dtree_compact(desc.data_ptr(), cache.k_pages.data_ptr(), cache.v_pages.data_ptr(),
                                  cache.layer_stride, layers, Hkv, D, cache.page_table.data_ptr(), hid.data_ptr(),
                                  96, hsel.data_ptr(), stream()))
    torch.cuda.synchronize()
    n = len(acc)
    for li in range(layers):
        ek = oq.compact(before_k[li], P, acc)
        ev = oq.compact(before_v[li], P, acc)
        np.testing.assert_array_equal(bf16_f32(cache.logical_keys(li, P + n)), ek)
        np.testing.assert_array_equal(bf16_f32(cache.logical_values(li, P + n)), ev)
        # rows past the kept range are untouched unless overwritten by the move
        np.testing.assert_array_equal(bf16_f32(cache.logical_keys(li, P + L))[P + n:], before_k[li][P + n:])
    assert torch.equal(hsel[:n].cpu(), hid[acc].cpu())


def test_cross_xcd_exchange_paths(gpu_device, monkeypatch, attn_kernel):
    """The dispatcher places workgroups round-robin over the XCDs, so the
    exchanges normally read partials from the local L2. DTREE_TEST_OFF_XCD=1
    makes every workgroup count as off its expected XCD: partials are then
    read past the L2 (the path taken if placement ever differs) and must give
    the same bits."""
    L = 25

    def gemms():
        outs = []
        for n, k, sched in [(19456 // 4, 2560, -2), (2560, 4096, -3), (2560, 9728, -2)]:
            x = _rows(32, L, k, g, gpu_device)
            w = torch.from_numpy(g.standard_normal((n, k)).astype(np.float32) * 0.05).to(torch.bfloat16)
            w = w.to(gpu_device)
            out = torch.zeros(32, n, device=gpu_device)
            ws = torch.zeros(N.lib().dtree_gemm_workspace_bytes(32, n, k, 0), dtype=torch.uint8, device=gpu_device)
            _gemm(x, w, N.EPI_STORE_F32, sched, ws, out_f32=out, tiled=True)
            outs.append(out)
        torch.cuda.synchronize()
        return outs

    g = np.random.default_rng(77)
    native = gemms()
    parents = random_tree(25, seed=9)
    _, a_native, *_ = _attention_case(gpu_device, 1000, parents, seed=5)
    monkeypatch.setenv("DTREE_TEST_OFF_XCD", "1")
    g = np.random.default_rng(77)
    off = gemms()
    _, a_off, ref, *_ = _attention_case(gpu_device, 1000, parents, seed=5)
    monkeypatch.delenv("DTREE_TEST_OFF_XCD")
    for a, b in zip(native, off):
        assert torch.equal(a, b)
    assert torch.equal(a_native, a_off)
    assert np.abs(bf16_f32(a_off)[:25] - ref).max() <= 2e-2 * np.abs(ref).max()
