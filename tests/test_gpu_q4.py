"""q4 group-64 affine GEMM (DTREE_W_Q4G64, adapters.py:63-71 semantics) on the
GPU against the float64 q4 oracle (oracle/q4.py), through the C-ABI.

Weights are synthetic as in the q4 workload: nibbles uniform in [0, 15],
scales |N(0, 0.02)| * 8, biases N(0, 0.01), scales/biases bf16. The kernel
multiplies raw nibbles on MFMA (as 128 + q in bf16, exact) and applies
s * acc + (b - 128 s) * sum(x) per group; its fp32 accumulation is the only
rounding, so the bar is 2e-4 of the output's magnitude."""
import ctypes as C

import numpy as np
import pytest
import torch

from gpu_util import bf16_f32, stream
from oracle import q4 as o4
from oracle.qwen3 import bf16_to_f32

from dtree_hip import _native as N
from dtree_hip.weights import interleave_gate_up, q4_to_tiled, tile_weight

pytestmark = pytest.mark.gpu

SHAPES = [(64, 64), (4096, 64), (64, 9728), (256, 1024), (6144, 2560), (2560, 4096), (19456, 2560), (2560, 9728)]


def _to_torch(wq, s, b):
    return (torch.from_numpy(np.ascontiguousarray(wq).view(np.int32)),
            torch.from_numpy(np.ascontiguousarray(s).view(np.int16)).view(torch.bfloat16),
            torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16))


def _x(L, k, g, dev, lo):
    xf = np.zeros((32, k), np.float32)
    xf[:L] = g.standard_normal((L, k))
    hi = torch.from_numpy(xf).to(torch.bfloat16)
    lo_t = (torch.from_numpy(xf) - hi.float()).to(torch.bfloat16)
    xin = hi.double() + (lo_t.double() if lo else 0)
    return tile_weight(hi.to(dev)), (tile_weight(lo_t.to(dev)) if lo else None), xin.numpy()


def _args(xt, xlt, wt, sb, n, k, epi, ws):
    a = N.GemmArgs()
    a.x = xt.data_ptr(); a.x_lo = xlt.data_ptr() if xlt is not None else None
    a.x_layout = N.W_TILED; a.ldx = k; a.rows_padded = 32
    a.w = wt.data_ptr(); a.w_layout = N.W_Q4G64; a.w_scales = sb.data_ptr()
    a.n = n; a.k = k; a.epilogue = epi; a.split_k = 0
    a.workspace = ws.data_ptr(); a.workspace_bytes = ws.numel()
    return a


@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("lo", [False, True])
def test_q4_gemm_store_f32(gpu_device, n, k, lo):
    g = np.random.default_rng(n * 7 + k + lo)
    wq, s, b = o4.random_q4(n, k, g)
    wt, sb = q4_to_tiled(*_to_torch(wq, s, b))
    wt, sb = wt.to(gpu_device), sb.to(gpu_device)
    xt, xlt, xin = _x(25, k, g, gpu_device, lo)
    ss = torch.from_numpy(np.abs(g.standard_normal((3, 32))).astype(np.float32) + 0.5).to(gpu_device)
    ws = torch.zeros(N.lib().dtree_gemm_workspace_bytes(32, n, k, 0), dtype=torch.uint8, device=gpu_device)
    outs = []
    for _ in range(2):
        out = torch.zeros(32, n, device=gpu_device)
        a = _args(xt, xlt, wt, sb, n, k, N.EPI_STORE_F32, ws)
        a.ss_in = ss.data_ptr(); a.ss_tiles = 3; a.norm_dim = k; a.eps = 1e-6
        a.out_f32 = out.data_ptr(); a.ld_out_f32 = n
        N.check(N.lib().dtree_gemm_bf16(C.byref(a), stream()), "q4 gemm")
        outs.append(out)
    torch.cuda.synchronize()
    rs = 1.0 / np.sqrt(ss.cpu().numpy().sum(0) / k + 1e-6)
    ref = o4.q4_matmul(xin, wq, bf16_to_f32(s), bf16_to_f32(b)) * rs[:, None]
    got = outs[0].cpu().numpy()
    assert np.abs(got - ref).max() <= 2e-4 * np.abs(ref).max()
    assert torch.equal(outs[0], outs[1])
    assert int(ws[: (n // 64) * 4].view(torch.int32).abs().sum()) == 0


def test_q4_gemm_residual_and_swiglu(gpu_device):
    g = np.random.default_rng(77)
    H, F, L = 512, 768, 25
    # residual (o_proj / down_proj shape class): x += y, xg = split(x * g), ss
    wq, s, b = o4.random_q4(H, F, g)
    wt, sb = q4_to_tiled(*_to_torch(wq, s, b))
    xt, xlt, xin = _x(L, F, g, gpu_device, True)
    res = torch.zeros(32, H)
    res[:L] = torch.from_numpy(g.standard_normal((L, H)).astype(np.float32))
    res = res.to(gpu_device)
    res0 = res.clone()
    gn = torch.from_numpy((1 + 0.1 * g.standard_normal(H)).astype(np.float32)).to(torch.bfloat16).to(gpu_device)
    xg = torch.zeros(32, H, dtype=torch.bfloat16, device=gpu_device)
    ss = torch.zeros(H // 32, 32, device=gpu_device)
    ws = torch.zeros(N.lib().dtree_gemm_workspace_bytes(32, 2 * F, H, 0) + (1 << 20), dtype=torch.uint8,
                     device=gpu_device)
    a = _args(xt, xlt, wt.to(gpu_device), sb.to(gpu_device), H, F, N.EPI_RESIDUAL, ws)
    a.out_f32 = res.data_ptr(); a.ld_out_f32 = H
    a.out_bf16 = xg.data_ptr(); a.ld_out_bf16 = H; a.next_norm = gn.data_ptr(); a.ss_out = ss.data_ptr()
    N.check(N.lib().dtree_gemm_bf16(C.byref(a), stream()), "q4 residual")
    torch.cuda.synchronize()
    ref = res0.cpu().double().numpy() + o4.q4_matmul(xin, wq, bf16_to_f32(s), bf16_to_f32(b))
    got = res.cpu().numpy()
    assert np.abs(got - ref).max() <= 2e-4 * np.abs(ref).max()
    assert torch.equal(xg.cpu(), (torch.from_numpy(got) * gn.float().cpu()).to(torch.bfloat16))
    np.testing.assert_allclose(ss.cpu().numpy(), (got.astype(np.float64) ** 2).reshape(32, H // 32, 32).sum(-1).T,
                               rtol=1e-5, atol=1e-5)

    # SwiGLU: gate / up interleaved in 16-row groups, q4 on both
    gq, gs, gb = o4.random_q4(F, H, g)
    uq, us, ub = o4.random_q4(F, H, g)
    wq2 = interleave_gate_up(*[torch.from_numpy(np.ascontiguousarray(t).view(np.int32)) for t in (gq, uq)])
    s2 = interleave_gate_up(*[torch.from_numpy(np.ascontiguousarray(t).view(np.int16)) for t in (gs, us)])
    b2 = interleave_gate_up(*[torch.from_numpy(np.ascontiguousarray(t).view(np.int16)) for t in (gb, ub)])
    wt2, sb2 = q4_to_tiled(wq2, s2.view(torch.bfloat16), b2.view(torch.bfloat16))
    xt, xlt, xin = _x(L, H, g, gpu_device, True)
    rsq = torch.from_numpy(np.abs(g.standard_normal((2, 32))).astype(np.float32) + 0.5).to(gpu_device)
    act = torch.zeros(32, F, dtype=torch.bfloat16, device=gpu_device)
    a = _args(xt, xlt, wt2.to(gpu_device), sb2.to(gpu_device), 2 * F, H, N.EPI_SWIGLU, ws)
    a.ss_in = rsq.data_ptr(); a.ss_tiles = 2; a.norm_dim = H; a.eps = 1e-6
    a.out_bf16 = act.data_ptr(); a.ld_out_bf16 = F
    N.check(N.lib().dtree_gemm_bf16(C.byref(a), stream()), "q4 swiglu")
    torch.cuda.synchronize()
    rs = 1.0 / np.sqrt(rsq.cpu().numpy().sum(0) / H + 1e-6)
    gt = o4.q4_matmul(xin, gq, bf16_to_f32(gs), bf16_to_f32(gb)) * rs[:, None]
    up = o4.q4_matmul(xin, uq, bf16_to_f32(us), bf16_to_f32(ub)) * rs[:, None]
    ref = gt / (1 + np.exp(-np.clip(gt, -80, 80))) * up
    # bf16 output: 1e-2 relative, plus an absolute floor scaled to the output's
    # magnitude (q4 activations here reach ~1e5)
    assert np.all(np.abs(bf16_f32(act) - ref) <= 1e-2 * np.abs(ref) + 1e-5 * np.abs(ref).max())


def _q4_layer_case(epi, g, dev):
    """Qwen3-4B layer shapes: down_proj with the residual epilogue (N 2560,
    K 9728; automatically three per-tile workgroups, one per part of K) and
    gate/up with SwiGLU (N 19456, K 2560; automatically one workgroup per
    tile, 608 of them; split_k -2 forces the two-per-CU stream-K kernel)."""
    L = 25
    if epi == N.EPI_RESIDUAL:
        n, k = 2560, 9728
        wq, s, b = o4.random_q4(n, k, g)
        wt, sb = q4_to_tiled(*_to_torch(wq, s, b))
        ref_w = [(wq, s, b)]
    else:
        F, k = 9728, 2560
        n = 2 * F
        gq, gs, gb = o4.random_q4(F, k, g)
        uq, us, ub = o4.random_q4(F, k, g)
        wq2 = interleave_gate_up(*[torch.from_numpy(np.ascontiguousarray(t).view(np.int32)) for t in (gq, uq)])
        s2 = interleave_gate_up(*[torch.from_numpy(np.ascontiguousarray(t).view(np.int16)) for t in (gs, us)])
        b2 = interleave_gate_up(*[torch.from_numpy(np.ascontiguousarray(t).view(np.int16)) for t in (gb, ub)])
        wt, sb = q4_to_tiled(wq2, s2.view(torch.bfloat16), b2.view(torch.bfloat16))
        ref_w = [(gq, gs, gb), (uq, us, ub)]
    xt, xlt, xin = _x(L, k, g, dev, True)
    return n, k, wt.to(dev), sb.to(dev), xt, xlt, xin, ref_w


def _run_q4_layer(epi, n, k, wt, sb, xt, xlt, g_seed, dev, split_k=0):
    g = np.random.default_rng(g_seed)
    ws = torch.zeros(N.lib().dtree_gemm_workspace_bytes(32, n, k, 0), dtype=torch.uint8, device=dev)
    a = _args(xt, xlt, wt, sb, n, k, epi, ws)
    a.split_k = split_k
    out = {}
    if epi == N.EPI_RESIDUAL:
        res = torch.zeros(32, n)
        res[:25] = torch.from_numpy(g.standard_normal((25, n)).astype(np.float32))
        out["res0"] = res.clone()
        out["res"] = res.to(dev)
        out["gn"] = torch.from_numpy((1 + 0.1 * g.standard_normal(n)).astype(np.float32)).to(torch.bfloat16).to(dev)
        out["xg"] = torch.zeros(32, n, dtype=torch.bfloat16, device=dev)
        out["ss"] = torch.zeros(n // 32, 32, device=dev)
        a.out_f32 = out["res"].data_ptr(); a.ld_out_f32 = n
        a.out_bf16 = out["xg"].data_ptr(); a.ld_out_bf16 = n
        a.next_norm = out["gn"].data_ptr(); a.ss_out = out["ss"].data_ptr()
    else:
        out["rsq"] = torch.from_numpy(np.abs(g.standard_normal((k // 32, 32))).astype(np.float32) + 0.5).to(dev)
        out["act"] = torch.zeros(32, n // 2, dtype=torch.bfloat16, device=dev)
        a.ss_in = out["rsq"].data_ptr(); a.ss_tiles = k // 32; a.norm_dim = k; a.eps = 1e-6
        a.out_bf16 = out["act"].data_ptr(); a.ld_out_bf16 = n // 2
    N.check(N.lib().dtree_gemm_bf16(C.byref(a), stream()), "q4 layer gemm")
    torch.cuda.synchronize()
    out["ws"] = ws
    return out


# split_k 0: the automatic schedule (residual: dpq_gemm_kernel, three parts;
# SwiGLU: dpq_gemm_kernel, one workgroup per tile); -2 forces stream-K
# (sk2_gemm_kernel at these unit counts); -1 / -4 force the per-tile q4 kernel
# with one / three parts of K.
@pytest.mark.parametrize("epi,split_k", [(N.EPI_RESIDUAL, 0), (N.EPI_RESIDUAL, -2), (N.EPI_RESIDUAL, -1),
                                         (N.EPI_SWIGLU, 0), (N.EPI_SWIGLU, -2), (N.EPI_SWIGLU, -4)])
def test_q4_layer_shapes(gpu_device, epi, split_k):
    g = np.random.default_rng(91 + epi)
    n, k, wt, sb, xt, xlt, xin, ref_w = _q4_layer_case(epi, g, gpu_device)
    print(f"q4 layer shape n={n} k={k} epi={epi} split_k={split_k}", flush=True)
    runs = [_run_q4_layer(epi, n, k, wt, sb, xt, xlt, 5, gpu_device, split_k) for _ in range(2)]
    if epi == N.EPI_RESIDUAL:
        wq, s, b = ref_w[0]
        ref = runs[0]["res0"].double().numpy() + o4.q4_matmul(xin, wq, bf16_to_f32(s), bf16_to_f32(b))
        got = runs[0]["res"].cpu().numpy()
        assert np.abs(got - ref).max() <= 2e-4 * np.abs(ref).max()
        assert torch.equal(runs[0]["xg"].cpu(), (torch.from_numpy(got) * runs[0]["gn"].float().cpu()).to(torch.bfloat16))
        for key in ("res", "xg", "ss"):
            assert torch.equal(runs[0][key], runs[1][key]), key
    else:
        rs = 1.0 / np.sqrt(runs[0]["rsq"].cpu().numpy().sum(0) / k + 1e-6)
        (gq, gs, gb), (uq, us, ub) = ref_w
        gt = o4.q4_matmul(xin, gq, bf16_to_f32(gs), bf16_to_f32(gb)) * rs[:, None]
        up = o4.q4_matmul(xin, uq, bf16_to_f32(us), bf16_to_f32(ub)) * rs[:, None]
        ref = gt / (1 + np.exp(-np.clip(gt, -80, 80))) * up
        assert np.all(np.abs(bf16_f32(runs[0]["act"]) - ref) <= 1e-2 * np.abs(ref) + 1e-5 * np.abs(ref).max())
        assert torch.equal(runs[0]["act"], runs[1]["act"])
    for r in runs:  # counters self-reset
        assert int(r["ws"][: (n // 64) * 4].view(torch.int32).abs().sum()) == 0


@pytest.mark.parametrize("split_k", [0, -2])
def test_q4_partials_read_past_the_l2(gpu_device, monkeypatch, split_k):
    """DTREE_TEST_OFF_XCD=1 makes every workgroup count as off its expected
    XCD, so the per-tile q4 kernel's parts (split_k 0) and the two-per-CU
    stream-K kernel (split_k -2) read their partial tiles past the L2; the
    bits must equal the native run's."""
    g = np.random.default_rng(123)
    n, k, wt, sb, xt, xlt, xin, _ = _q4_layer_case(N.EPI_RESIDUAL, g, gpu_device)
    native = _run_q4_layer(N.EPI_RESIDUAL, n, k, wt, sb, xt, xlt, 6, gpu_device, split_k)
    monkeypatch.setenv("DTREE_TEST_OFF_XCD", "1")
    off = _run_q4_layer(N.EPI_RESIDUAL, n, k, wt, sb, xt, xlt, 6, gpu_device, split_k)
    monkeypatch.delenv("DTREE_TEST_OFF_XCD")
    for key in ("res", "xg", "ss"):
        assert torch.equal(native[key], off[key]), key


def _xrows(MP, L, k, g, dev, hi_only=False):
    """MP tiled activation rows (L nonzero) as the split pair; the float64
    input the kernel sees (hi + lo, or hi alone without the low plane)."""
    xf = np.zeros((MP, k), np.float32)
    xf[:L] = g.standard_normal((L, k))
    hi = torch.from_numpy(xf).to(torch.bfloat16)
    lo = (torch.from_numpy(xf) - hi.float()).to(torch.bfloat16)
    xin = hi.double().numpy() + (0 if hi_only else lo.double().numpy())
    return tile_weight(hi.to(dev)), tile_weight(lo.to(dev)), xin


def _x96(L, k, g, dev):
    return _xrows(96, L, k, g, dev)


def test_q4_gemm_96_rows(gpu_device):
    """65 tree rows (rows_padded 96): the q4 GEMM makes one pass over the
    weights for all three row blocks (q4m_gemm_kernel). Row-block-major
    statistics in and out, residual + next norm into a tiled output, against
    the q4 oracle on every row."""
    g = np.random.default_rng(96)
    H, F, L, MP = 512, 768, 65, 96
    ws = torch.zeros(max(N.lib().dtree_gemm_workspace_bytes(MP, n, k, 0) for n, k in ((F, H), (H, F))),
                     dtype=torch.uint8, device=gpu_device)
    # fp32 store with a row scale from [3][H/32][32] statistics
    wq, s, b = o4.random_q4(F, H, g)
    wt, sb = q4_to_tiled(*_to_torch(wq, s, b))
    xt, xlt, xin = _x96(L, H, g, gpu_device)
    ss_np = (np.abs(g.standard_normal((3, H // 32, 32))) + 0.5).astype(np.float32)
    ss = torch.from_numpy(ss_np).to(gpu_device)
    out = torch.zeros(MP, F, device=gpu_device)
    a = _args(xt, xlt, wt.to(gpu_device), sb.to(gpu_device), F, H, N.EPI_STORE_F32, ws)
    a.rows_padded = MP
    a.ss_in = ss.data_ptr(); a.ss_tiles = H // 32; a.norm_dim = H; a.eps = 1e-6
    a.out_f32 = out.data_ptr(); a.ld_out_f32 = F
    N.check(N.lib().dtree_gemm_bf16(C.byref(a), stream()), "q4 gemm 96 rows")
    torch.cuda.synchronize()
    rs = 1.0 / np.sqrt(ss_np.sum(1).reshape(MP) / H + 1e-6)
    ref = o4.q4_matmul(xin, wq, bf16_to_f32(s), bf16_to_f32(b)) * rs[:, None]
    got = out.cpu().numpy()
    assert np.abs(got - ref).max() <= 2e-4 * np.abs(ref).max()
    assert not got[L:].any()
    # residual + next-norm statistics, tiled xg output
    wq, s, b = o4.random_q4(H, F, g)
    wt, sb = q4_to_tiled(*_to_torch(wq, s, b))
    xt, xlt, xin = _x96(L, F, g, gpu_device)
    res = torch.zeros(MP, H)
    res[:L] = torch.from_numpy(g.standard_normal((L, H)).astype(np.float32))
    res = res.to(gpu_device)
    res0 = res.cpu().double().numpy()
    gn = torch.from_numpy((1 + 0.1 * g.standard_normal(H)).astype(np.float32)).to(torch.bfloat16).to(gpu_device)
    xg = torch.zeros(2, MP * H, dtype=torch.bfloat16, device=gpu_device)
    sso = torch.zeros(3, H // 32, 32, device=gpu_device)
    a = _args(xt, xlt, wt.to(gpu_device), sb.to(gpu_device), H, F, N.EPI_RESIDUAL, ws)
    a.rows_padded = MP
    a.out_f32 = res.data_ptr(); a.ld_out_f32 = H
    a.out_bf16 = xg[0].data_ptr(); a.out_lo = xg[1].data_ptr(); a.ld_out_bf16 = H; a.out_layout = N.W_TILED
    a.next_norm = gn.data_ptr(); a.ss_out = sso.data_ptr()
    N.check(N.lib().dtree_gemm_bf16(C.byref(a), stream()), "q4 residual 96 rows")
    torch.cuda.synchronize()
    ref = res0 + o4.q4_matmul(xin, wq, bf16_to_f32(s), bf16_to_f32(b))
    got = res.cpu().numpy()
    assert np.abs(got - ref).max() <= 2e-4 * np.abs(ref).max()
    from dtree_hip.weights import untile_weight
    xg_rows = untile_weight(xg[0].view(MP, H)).float() + untile_weight(xg[1].view(MP, H)).float()
    want = torch.from_numpy(got) * gn.float().cpu()
    assert torch.allclose(xg_rows.cpu(), want, rtol=2 ** -15, atol=1e-30)
    exp_ss = (got.astype(np.float64) ** 2).reshape(3, 32, H // 32, 32).sum(-1).transpose(0, 2, 1)
    np.testing.assert_allclose(sso.cpu().numpy(), exp_ss, rtol=1e-5, atol=1e-5)


# One-pass q4 GEMM over 64-128 rows (q4m_gemm_kernel). Shapes chosen for its
# plans on a 256-CU device: (768, 512) two 64-column blocks per workgroup
# over several K parts; (320, 1024) a ragged last tile (5 blocks in tiles of
# 2); (32768, 128) four blocks per workgroup in two K parts; (4096, 4096) the
# 9B out_proj class (two per workgroup, eight K parts); (12352, 256) 193
# blocks (in_proj's ragged width) in two parts; (24576, 128) and (24448, 128)
# three blocks per workgroup in two parts (the 9B gate/up plan), the second
# with a ragged last tile (382 blocks).
Q4M_SHAPES = [(768, 512), (320, 1024), (32768, 128), (4096, 4096), (12352, 256), (24576, 128), (24448, 128)]


@pytest.mark.parametrize("n,k", Q4M_SHAPES)
@pytest.mark.parametrize("MP", [64, 96, 128])
def test_q4_one_pass_store_f32(gpu_device, n, k, MP):
    g = np.random.default_rng(n + k + MP)
    L = MP - 31
    lo = MP != 64  # both activation-plane variants
    wq, s, b = o4.random_q4(n, k, g)
    wt, sb = q4_to_tiled(*_to_torch(wq, s, b))
    wt, sb = wt.to(gpu_device), sb.to(gpu_device)
    xt, xlt, xin = _xrows(MP, L, k, g, gpu_device, hi_only=not lo)
    ss_np = (np.abs(g.standard_normal((MP // 32, k // 32, 32))) + 0.5).astype(np.float32)
    ss = torch.from_numpy(ss_np).to(gpu_device)
    ws = torch.zeros(N.lib().dtree_gemm_workspace_bytes(MP, n, k, 0), dtype=torch.uint8, device=gpu_device)
    outs = []
    for _ in range(2):
        out = torch.zeros(MP, n, device=gpu_device)
        a = _args(xt, xlt if lo else None, wt, sb, n, k, N.EPI_STORE_F32, ws)
        a.rows_padded = MP
        a.ss_in = ss.data_ptr(); a.ss_tiles = k // 32; a.norm_dim = k; a.eps = 1e-6
        a.out_f32 = out.data_ptr(); a.ld_out_f32 = n
        print(f"q4 one pass n={n} k={k} rows={MP}", flush=True)
        N.check(N.lib().dtree_gemm_bf16(C.byref(a), stream()), "q4 one pass")
        outs.append(out)
    torch.cuda.synchronize()
    rs = 1.0 / np.sqrt(ss_np.transpose(0, 2, 1).reshape(MP, k // 32).sum(1) / k + 1e-6)
    ref = o4.q4_matmul(xin, wq, bf16_to_f32(s), bf16_to_f32(b)) * rs[:, None]
    got = outs[0].cpu().numpy()
    assert np.abs(got - ref).max() <= 2e-4 * np.abs(ref).max()
    assert not got[L:].any()
    assert torch.equal(outs[0], outs[1])  # fixed reduction order
    assert int(ws[:65536].view(torch.int32).abs().sum()) == 0  # counters self-reset


# (n, k, rows): eight K parts with fewer pairs than parts (the 9B out_proj
# class), two parts owning several pairs each (the 9B gate/up plan), four
# parts, and eight parts over a ragged last tile.
Q4M_PART_CASES = [(4096, 4096, 96), (24576, 128, 96), (768, 512, 64), (320, 1024, 128)]


@pytest.mark.parametrize("n,k,MP", Q4M_PART_CASES)
def test_q4_one_pass_parts_combine(gpu_device, monkeypatch, n, k, MP):
    """The K parts of a one-pass tile combine in a distributed way: pair i
    (64-column block, 32-row block) is added and finished by part i % P once
    every part has published, or by the last part to arrive when its owner's
    bounded wait gave up. Forced from the host (DTREE_TEST_SPIN_LIMIT=-1: no
    owner polls, so the last arriver claims every pair; 0: one poll each),
    every variant gives the same bits through the residual + next-norm +
    hidden-capture epilogue, matches the q4 oracle, and leaves the tile
    counters at zero."""
    from dtree_hip.weights import untile_weight
    g = np.random.default_rng(n + 3 * k + MP)
    L = MP - 29
    wq, s, b = o4.random_q4(n, k, g)
    wt, sb = q4_to_tiled(*_to_torch(wq, s, b))
    wt, sb = wt.to(gpu_device), sb.to(gpu_device)
    xt, _, xin = _xrows(MP, L, k, g, gpu_device, hi_only=True)
    res0 = torch.zeros(MP, n)
    res0[:L] = torch.from_numpy(g.standard_normal((L, n)).astype(np.float32))
    gn = torch.from_numpy((1 + 0.1 * g.standard_normal(n)).astype(np.float32)).to(torch.bfloat16).to(gpu_device)
    ws = torch.zeros(N.lib().dtree_gemm_workspace_bytes(MP, n, k, 0), dtype=torch.uint8, device=gpu_device)
    runs = []
    for limit in (None, "-1", "0", None):
        if limit is None:
            monkeypatch.delenv("DTREE_TEST_SPIN_LIMIT", raising=False)
        else:
            monkeypatch.setenv("DTREE_TEST_SPIN_LIMIT", limit)
        res = res0.clone().to(gpu_device)
        outb = torch.zeros(MP * n, dtype=torch.bfloat16, device=gpu_device)
        sso = torch.zeros(MP // 32, n // 32, 32, device=gpu_device)
        hid = torch.zeros(MP, n, dtype=torch.bfloat16, device=gpu_device)
        a = _args(xt, None, wt, sb, n, k, N.EPI_RESIDUAL, ws)
        a.rows_padded = MP
        a.out_f32 = res.data_ptr(); a.ld_out_f32 = n
        a.out_bf16 = outb.data_ptr(); a.out_lo = None; a.ld_out_bf16 = n; a.out_layout = N.W_TILED
        a.next_norm = gn.data_ptr(); a.ss_out = sso.data_ptr(); a.hidden_out = hid.data_ptr(); a.ld_hidden = n
        print(f"q4 one pass parts n={n} k={k} rows={MP} spin limit={limit}", flush=True)
        N.check(N.lib().dtree_gemm_bf16(C.byref(a), stream()), "q4 one pass parts")
        torch.cuda.synchronize()
        assert int(ws[:65536].view(torch.int32).abs().sum()) == 0  # counters cleared by the last release
        runs.append((res.cpu(), outb.cpu(), sso.cpu(), hid.cpu()))
    monkeypatch.delenv("DTREE_TEST_SPIN_LIMIT", raising=False)
    for other in runs[1:]:
        for x, y in zip(runs[0], other):
            assert torch.equal(x, y)
    got = runs[0][0].numpy()
    ref = res0.double().numpy() + o4.q4_matmul(xin, wq, bf16_to_f32(s), bf16_to_f32(b))
    assert np.abs(got - ref).max() <= 2e-4 * np.abs(ref).max()
    assert not got[L:].any()
    got_b = untile_weight(runs[0][1].view(MP, n)).float().numpy()
    np.testing.assert_allclose(got_b, got * bf16_f32(gn)[None], rtol=2 ** -8, atol=1e-30)  # one bf16 plane


@pytest.mark.parametrize("epi", ["residual", "swiglu", "bf16"])
@pytest.mark.parametrize("MP", [64, 96, 128])
def test_q4_one_pass_epilogues(gpu_device, epi, MP):
    """Residual + next-norm statistics + hidden capture, SwiGLU and the split
    bf16 store over 64-128 rows, tiled bf16 outputs, against the q4 oracle."""
    from dtree_hip.weights import untile_weight
    g = np.random.default_rng(7 * MP + len(epi))
    L = MP - 31
    n, k = (640, 1024) if epi != "swiglu" else (1536, 512)
    if epi == "swiglu":
        F = n // 2
        gq, gs, gb = o4.random_q4(F, k, g)
        uq, us, ub = o4.random_q4(F, k, g)
        wq2 = interleave_gate_up(*[torch.from_numpy(np.ascontiguousarray(t).view(np.int32)) for t in (gq, uq)])
        s2 = interleave_gate_up(*[torch.from_numpy(np.ascontiguousarray(t).view(np.int16)) for t in (gs, us)])
        b2 = interleave_gate_up(*[torch.from_numpy(np.ascontiguousarray(t).view(np.int16)) for t in (gb, ub)])
        wt, sb = q4_to_tiled(wq2, s2.view(torch.bfloat16), b2.view(torch.bfloat16))
    else:
        wq, s, b = o4.random_q4(n, k, g)
        wt, sb = q4_to_tiled(*_to_torch(wq, s, b))
    wt, sb = wt.to(gpu_device), sb.to(gpu_device)
    xt, xlt, xin = _xrows(MP, L, k, g, gpu_device)
    ws = torch.zeros(N.lib().dtree_gemm_workspace_bytes(MP, n, k, 0), dtype=torch.uint8, device=gpu_device)
    width = n // 2 if epi == "swiglu" else n
    outb = torch.zeros(2, MP * width, dtype=torch.bfloat16, device=gpu_device)
    a = _args(xt, xlt, wt, sb, n, k, {"residual": N.EPI_RESIDUAL, "swiglu": N.EPI_SWIGLU,
                                      "bf16": N.EPI_STORE_BF16}[epi], ws)
    a.rows_padded = MP
    a.out_bf16 = outb[0].data_ptr(); a.out_lo = outb[1].data_ptr(); a.ld_out_bf16 = width
    a.out_layout = N.W_TILED
    rs = np.ones(MP)
    if epi != "residual":
        ss_np = (np.abs(g.standard_normal((MP // 32, k // 32, 32))) + 0.5).astype(np.float32)
        ss = torch.from_numpy(ss_np).to(gpu_device)
        a.ss_in = ss.data_ptr(); a.ss_tiles = k // 32; a.norm_dim = k; a.eps = 1e-6
        rs = 1.0 / np.sqrt(ss_np.transpose(0, 2, 1).reshape(MP, k // 32).sum(1) / k + 1e-6)
    else:
        res = torch.zeros(MP, n)
        res[:L] = torch.from_numpy(g.standard_normal((L, n)).astype(np.float32))
        res = res.to(gpu_device)
        res0 = res.cpu().double().numpy()
        gn = torch.from_numpy((1 + 0.1 * g.standard_normal(n)).astype(np.float32)).to(torch.bfloat16).to(gpu_device)
        sso = torch.zeros(MP // 32, n // 32, 32, device=gpu_device)
        hid = torch.zeros(MP, n, dtype=torch.bfloat16, device=gpu_device)
        a.out_f32 = res.data_ptr(); a.ld_out_f32 = n
        a.next_norm = gn.data_ptr(); a.ss_out = sso.data_ptr(); a.hidden_out = hid.data_ptr(); a.ld_hidden = n
    print(f"q4 one pass epilogue={epi} rows={MP}", flush=True)
    N.check(N.lib().dtree_gemm_bf16(C.byref(a), stream()), "q4 one pass")
    torch.cuda.synchronize()
    got_b = (untile_weight(outb[0].view(MP, width)).float() + untile_weight(outb[1].view(MP, width)).float()).cpu().numpy()
    if epi == "residual":
        ref = res0 + o4.q4_matmul(xin, wq, bf16_to_f32(s), bf16_to_f32(b))
        got = res.cpu().numpy()
        assert np.abs(got - ref).max() <= 2e-4 * np.abs(ref).max()
        assert not got[L:].any()
        np.testing.assert_allclose(got_b, got * bf16_f32(gn)[None], rtol=2 ** -15, atol=1e-30)
        exp_ss = (got.astype(np.float64) ** 2).reshape(MP // 32, 32, n // 32, 32).sum(-1).transpose(0, 2, 1)
        np.testing.assert_allclose(sso.cpu().numpy(), exp_ss, rtol=1e-5, atol=1e-5)
        assert torch.equal(hid.cpu(), torch.from_numpy(got).to(torch.bfloat16))
    elif epi == "swiglu":
        gt = o4.q4_matmul(xin, gq, bf16_to_f32(gs), bf16_to_f32(gb)) * rs[:, None]
        up = o4.q4_matmul(xin, uq, bf16_to_f32(us), bf16_to_f32(ub)) * rs[:, None]
        ref = gt / (1 + np.exp(-np.clip(gt, -80, 80))) * up
        assert np.abs(got_b - ref).max() <= 2e-4 * np.abs(ref).max()
    else:
        ref = o4.q4_matmul(xin, wq, bf16_to_f32(s), bf16_to_f32(b)) * rs[:, None]
        assert np.abs(got_b - ref).max() <= 2e-4 * np.abs(ref).max()
    assert int(ws[:65536].view(torch.int32).abs().sum()) == 0


def test_q4_rejects_bad_arguments(gpu_device):
    a = N.GemmArgs()
    buf = torch.zeros(1 << 16, dtype=torch.uint8, device=gpu_device)
    a.x = buf.data_ptr(); a.x_layout = N.W_TILED; a.ldx = 64; a.rows_padded = 32
    a.w = buf.data_ptr(); a.w_layout = N.W_Q4G64; a.w_scales = None; a.n = 64; a.k = 64
    a.epilogue = N.EPI_STORE_F32; a.out_f32 = buf.data_ptr(); a.ld_out_f32 = 64
    a.workspace = buf.data_ptr(); a.workspace_bytes = buf.numel()
    assert N.lib().dtree_gemm_bf16(C.byref(a), stream()) != 0  # no scales
    a.w_scales = buf.data_ptr(); a.split_k = 2
    assert N.lib().dtree_gemm_bf16(C.byref(a), stream()) != 0  # q4 is stream-K only


def test_q4_lmhead_argmax_and_logits(gpu_device):
    """Fused q4 LM head (quantised tied embedding): logits against the q4
    oracle, argmax first index on ties, including a tie across workgroups."""
    g = np.random.default_rng(91)
    V, H, L = 151936, 2560, 25
    wq, s, b = o4.random_q4(V, H, g)
    # two equal rows far apart -> equal logits; the smaller index must win.
    # Their scales are the largest, so their norm is too and (Cauchy-Schwarz)
    # row 3 = 4 E[5] peaks there.
    from oracle.qwen3 import f32_to_bf16_bits
    s[5] = f32_to_bf16_bits(np.full(s.shape[1], 0.5, np.float32))
    wq[151900] = wq[5]; s[151900] = s[5]; b[151900] = b[5]
    wt, sb = q4_to_tiled(*_to_torch(wq, s, b))
    wt, sb = wt.to(gpu_device), sb.to(gpu_device)
    xf = np.zeros((32, H), np.float32)
    xf[:L] = g.standard_normal((L, H))
    E5 = o4.dequantize(wq[5:6], bf16_to_f32(s[5:6]), bf16_to_f32(b[5:6]))[0]
    xf[3] = E5.astype(np.float32) * 4.0  # row 3 peaks at tokens 5 and 151900
    hi = torch.from_numpy(xf).to(torch.bfloat16)
    lo = (torch.from_numpy(xf) - hi.float()).to(torch.bfloat16)
    xt, xlt = tile_weight(hi.to(gpu_device)), tile_weight(lo.to(gpu_device))
    lib = N.lib()
    cand = torch.zeros(lib.dtree_lmhead_candidates_bytes(32), dtype=torch.uint8, device=gpu_device)
    logits = torch.zeros(32, V, device=gpu_device)
    N.check(lib.dtree_lmhead_argmax(xt.data_ptr(), xlt.data_ptr(), N.W_TILED, H, 32, wt.data_ptr(), N.W_Q4G64,
                                    sb.data_ptr(), V, H, None, 0, 1e-6, logits.data_ptr(), cand.data_ptr(),
                                    stream()), "q4 lmhead")
    torch.cuda.synchronize()
    xin = hi.double().numpy() + lo.double().numpy()
    ref = np.concatenate([o4.q4_matmul(xin[:L], wq[r:r + 8192], bf16_to_f32(s[r:r + 8192]),
                                       bf16_to_f32(b[r:r + 8192])) for r in range(0, V, 8192)], axis=1)
    got = logits[:L].cpu().numpy()
    assert np.abs(got - ref).max() <= 2e-4 * np.abs(ref).max()
    c = cand.view(torch.int32).view(-1, 32, 2)[: lib.dtree_lmhead_candidate_blocks(V, 32)].cpu().numpy()
    vals, idx = c[..., 0].view(np.float32), c[..., 1]
    best = []
    for m in range(L):
        order = np.lexsort((idx[:, m], -vals[:, m]))
        best.append(int(idx[order[0], m]))
    exact = np.argmax(got, axis=-1)
    assert best == exact.tolist()
    assert best[3] == 5


@pytest.mark.parametrize("MP", [32, 96])
def test_q4_lmhead_vocab_past_the_one_pass_grid(gpu_device, MP):
    """A vocabulary of more than 4 x 64 x 1024 entries does not fit the one-pass
    kernel's candidate grid: the 32-row kernel runs once per row block
    instead. Logits and first-index argmax against the q4 oracle."""
    g = np.random.default_rng(17 + MP)
    V, H, L = 4 * 64 * 1024 + 128, 128, MP - 7
    wq, s, b = o4.random_q4(V, H, g)
    # Row 3's scales (2.0, twelve standard deviations past the random ones)
    # give it the largest norm, so x = 4 E[3] peaks there (Cauchy-Schwarz);
    # row V - 40 copies it: a tie across workgroups.
    from oracle.qwen3 import f32_to_bf16_bits
    s[3] = f32_to_bf16_bits(np.full(s.shape[1], 2.0, np.float32))
    wq[V - 40] = wq[3]; s[V - 40] = s[3]; b[V - 40] = b[3]
    wt, sb = q4_to_tiled(*_to_torch(wq, s, b))
    wt, sb = wt.to(gpu_device), sb.to(gpu_device)
    xf = np.zeros((MP, H), np.float32)
    xf[:L] = g.standard_normal((L, H))
    xf[1] = o4.dequantize(wq[3:4], bf16_to_f32(s[3:4]), bf16_to_f32(b[3:4]))[0].astype(np.float32) * 4.0
    hi = torch.from_numpy(xf).to(torch.bfloat16)
    lo = (torch.from_numpy(xf) - hi.float()).to(torch.bfloat16)
    xt, xlt = tile_weight(hi.to(gpu_device)), tile_weight(lo.to(gpu_device))
    lib = N.lib()
    cand = torch.zeros(lib.dtree_lmhead_candidates_bytes(MP), dtype=torch.uint8, device=gpu_device)
    logits = torch.zeros(MP, V, device=gpu_device)
    print(f"q4 lmhead V={V} H={H} MP={MP}", flush=True)
    N.check(lib.dtree_lmhead_argmax(xt.data_ptr(), xlt.data_ptr(), N.W_TILED, H, MP, wt.data_ptr(), N.W_Q4G64,
                                    sb.data_ptr(), V, H, None, 0, 1e-6, logits.data_ptr(), cand.data_ptr(),
                                    stream()), "q4 lmhead")
    torch.cuda.synchronize()
    xin = hi.double().numpy() + lo.double().numpy()
    ref = o4.q4_matmul(xin[:L], wq, bf16_to_f32(s), bf16_to_f32(b))
    got = logits[:L].cpu().numpy()
    assert np.abs(got - ref).max() <= 2e-4 * np.abs(ref).max()
    blocks = lib.dtree_lmhead_candidate_blocks(V, MP)
    c = cand.view(torch.int32)[: (MP // 32) * blocks * 64].view(MP // 32, blocks, 32, 2).cpu().numpy()
    best = []
    for m in range(L):
        cb = c[m // 32, :, m % 32]
        vals, idx = cb[:, 0].view(np.float32), cb[:, 1]
        best.append(int(idx[np.lexsort((idx, -vals))[0]]))
    assert best == np.argmax(got, axis=-1).tolist()
    assert best[1] == 3


def test_q4_lmhead_96_rows_through_walk(gpu_device):
    """q4 LM head over 65 tree rows (one pass over the embedding for the three
    row blocks): the walk's posterior over all 65 rows equals the argmax of
    the returned logits, which match the q4 oracle."""
    g = np.random.default_rng(965)
    V, H, L, MP = 8192, 1024, 65, 96
    wq, s, b = o4.random_q4(V, H, g)
    wt, sb = q4_to_tiled(*_to_torch(wq, s, b))
    xt, xlt, xin = _x96(L, H, g, gpu_device)
    lib = N.lib()
    cand = torch.zeros(lib.dtree_lmhead_candidates_bytes(MP), dtype=torch.uint8, device=gpu_device)
    logits = torch.zeros(MP, V, device=gpu_device)
    N.check(lib.dtree_lmhead_argmax(xt.data_ptr(), xlt.data_ptr(), N.W_TILED, H, MP, wt.to(gpu_device).data_ptr(),
                                    N.W_Q4G64, sb.to(gpu_device).data_ptr(), V, H, None, 0, 1e-6,
                                    logits.data_ptr(), cand.data_ptr(), stream()), "q4 lmhead 96")
    from gpu_util import device_desc
    parents = [-1] + [(i - 1) // 3 for i in range(1, L)]
    desc = device_desc([0] * L, list(range(L)), parents, 0, gpu_device)
    res = torch.zeros(3 + 2 * N.MAX_NODES, dtype=torch.int32, device=gpu_device)
    N.check(lib.dtree_accept_walk(desc.data_ptr(), cand.data_ptr(), lib.dtree_lmhead_candidate_blocks(V, MP), MP,
                                  res.data_ptr(), stream()), "walk 96")
    torch.cuda.synchronize()
    ref = o4.q4_matmul(xin[:L], wq, bf16_to_f32(s), bf16_to_f32(b))
    got = logits[:L].cpu().numpy()
    assert np.abs(got - ref).max() <= 2e-4 * np.abs(ref).max()
    r = res.cpu().numpy()
    post = list(r[3 + N.MAX_NODES:3 + N.MAX_NODES + L])
    assert int(r[2]) == L and post == list(np.argmax(got, axis=-1))


@pytest.mark.parametrize("MP", [64, 96, 128])
def test_q4_lmhead_one_pass_ties_ragged_vocab(gpu_device, MP):
    """The one-pass q4 LM head (q4m_gemm_kernel's argmax epilogue) over 64-128
    rows: a vocabulary whose last 256-column tile is ragged (42 64-column
    blocks), the final RMSNorm row scale, no logits buffer, and an exact tie
    between vocab rows 300 and 2600 (different tiles; identical words, scale
    0, bias 20, activations >= 0, so the two are every row's maximum): the
    walk's posterior is the first index, 300, on every row."""
    from gpu_util import device_desc
    from oracle.qwen3 import f32_to_bf16_bits
    g = np.random.default_rng(MP + 5)
    V, H, L = 2688, 512, MP - 31
    wq, s, b = o4.random_q4(V, H, g)
    wq[2600] = wq[300]
    s[300] = s[2600] = 0
    b[300] = b[2600] = f32_to_bf16_bits(np.float32([20.0]))[0]
    wt, sb = q4_to_tiled(*_to_torch(wq, s, b))
    wt, sb = wt.to(gpu_device), sb.to(gpu_device)
    xf = np.zeros((MP, H), np.float32)
    xf[:L] = np.abs(g.standard_normal((L, H)))
    hi = torch.from_numpy(xf).to(torch.bfloat16)
    lo = (torch.from_numpy(xf) - hi.float()).to(torch.bfloat16)
    xt, xlt = tile_weight(hi.to(gpu_device)), tile_weight(lo.to(gpu_device))
    xin = hi.double().numpy() + lo.double().numpy()
    ss_np = (np.abs(g.standard_normal((MP // 32, H // 32, 32))) + 0.5).astype(np.float32)
    ss = torch.from_numpy(ss_np).to(gpu_device)
    rs = 1.0 / np.sqrt(ss_np.transpose(0, 2, 1).reshape(MP, H // 32).sum(1) / H + 1e-6)
    lib = N.lib()
    blocks = lib.dtree_lmhead_candidate_blocks(V, MP)
    parents = [-1] + list(range(L - 1))
    desc = device_desc([0] * L, list(range(L)), parents, 0, gpu_device)
    posts = []
    logits = torch.zeros(MP, V, device=gpu_device)
    for want_logits in (False, True):
        cand = torch.full((lib.dtree_lmhead_candidates_bytes(MP),), 0x55, dtype=torch.uint8, device=gpu_device)
        print(f"q4 one-pass lm head rows={MP} logits={want_logits}", flush=True)
        N.check(lib.dtree_lmhead_argmax(xt.data_ptr(), xlt.data_ptr(), N.W_TILED, H, MP, wt.data_ptr(), N.W_Q4G64,
                                        sb.data_ptr(), V, H, ss.data_ptr(), H // 32, 1e-6,
                                        logits.data_ptr() if want_logits else None, cand.data_ptr(), stream()),
                "q4 lmhead one pass")
        res = torch.zeros(3 + 2 * N.MAX_NODES, dtype=torch.int32, device=gpu_device)
        N.check(lib.dtree_accept_walk(desc.data_ptr(), cand.data_ptr(), blocks, MP, res.data_ptr(), stream()), "walk")
        torch.cuda.synchronize()
        r = res.cpu().numpy()
        posts.append(list(r[3 + N.MAX_NODES:3 + N.MAX_NODES + L]))
    assert posts[0] == posts[1] == [300] * L
    ref = o4.q4_matmul(xin[:L], wq, bf16_to_f32(s), bf16_to_f32(b)) * rs[:L, None]
    got = logits[:L].cpu().numpy()
    assert np.abs(got - ref).max() <= 2e-4 * np.abs(ref).max()
    assert np.array_equal(got[:, 300], got[:, 2600])


def test_q4_embedding_gather(gpu_device):
    """dtree_embed on a q4 embedding: x rows = scale * q + bias of each token."""
    from gpu_util import device_desc
    g = np.random.default_rng(5)
    V, H, L = 4096, 1024, 25
    wq, s, b = o4.random_q4(V, H, g)
    wt, sb = q4_to_tiled(*_to_torch(wq, s, b))
    toks = g.integers(0, V, L).tolist()
    desc = device_desc(toks, list(range(L)), [-1] + list(range(L - 1)), 0, gpu_device)
    nw = torch.ones(H, dtype=torch.bfloat16, device=gpu_device)
    x = torch.zeros(32, H, device=gpu_device)
    xg = torch.zeros(32, H, dtype=torch.bfloat16, device=gpu_device)
    ss = torch.zeros(H // 32, 32, device=gpu_device)
    N.check(N.lib().dtree_embed(desc.data_ptr(), wt.to(gpu_device).data_ptr(), N.W_Q4G64,
                                sb.to(gpu_device).data_ptr(), V, H, nw.data_ptr(), 32, x.data_ptr(),
                                xg.data_ptr(), None, N.W_ROWMAJOR, ss.data_ptr(), 128, 1e6, None, None, stream()),
            "q4 embed")
    torch.cuda.synchronize()
    ref = o4.dequantize(wq[toks], bf16_to_f32(s[toks]), bf16_to_f32(b[toks]))
    got = x.cpu().numpy()
    assert np.abs(got[:L] - ref).max() <= 1e-6 * np.abs(ref).max()
    assert np.all(got[L:] == 0)
