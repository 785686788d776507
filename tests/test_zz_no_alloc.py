"""dtree_tree_attention_noalloc (the allocation-free variant with a static
device scratch array) against dtree_tree_attention with a caller workspace:
same inputs, same kernels, so outputs and cache rows must agree bit for bit,
on two calls in a row (the second with a smaller tree and prefix, in a shorter
grid), for both attention designs; shapes beyond the scratch array are
rejected before any launch."""
import ctypes as C

import numpy as np
import pytest
import torch

from dtree_hip import _native as N
from dtree_hip.cache import PagedKVCache

from gpu_util import device_desc, random_tree, stream

pytestmark = pytest.mark.gpu


def _case(dev, P, L, max_past, seed, Hq=32, Hkv=8, D=128, MP=32):
    g = np.random.default_rng(seed)
    parents = random_tree(L, seed=seed)
    depth = [0] * L
    for i in range(1, L):
        depth[i] = depth[parents[i]] + 1
    desc = device_desc([0] * L, [P + d for d in depth], parents, P, dev)
    kpre = torch.from_numpy((g.standard_normal((P, Hkv, D)) * 0.5).astype(np.float32))
    vpre = torch.from_numpy((g.standard_normal((P, Hkv, D)) * 0.5).astype(np.float32))
    caches = []
    for _ in range(2):
        cache = PagedKVCache(1, Hkv, D, max_past + MP, device=dev)
        if P:
            cache.write_logical(0, kpre, vpre)
        caches.append(cache)
    qkv = torch.zeros(MP, (Hq + 2 * Hkv) * D, device=dev)
    qkv[:L] = torch.from_numpy(g.standard_normal((L, (Hq + 2 * Hkv) * D)).astype(np.float32)).to(dev)
    cos = torch.zeros(MP, D // 2, device=dev)
    sin = torch.zeros(MP, D // 2, device=dev)
    N.check(N.lib().dtree_rope_table(desc.data_ptr(), MP, D, 1e6, cos.data_ptr(), sin.data_ptr(), stream()))
    norm = torch.from_numpy((1 + 0.1 * g.standard_normal(D)).astype(np.float32)).to(torch.bfloat16).to(dev)
    return dict(desc=desc, caches=caches, qkv=qkv, cos=cos, sin=sin, norm=norm, Hq=Hq, Hkv=Hkv, D=D, MP=MP,
                max_past=max_past)


def _args(c, cache, out, ws=None):
    a = N.AttnArgs()
    a.qkv = c["qkv"].data_ptr(); a.ld_qkv = c["qkv"].shape[1]
    a.q_norm = c["norm"].data_ptr(); a.k_norm = c["norm"].data_ptr(); a.eps = 1e-6
    a.rope_cos = c["cos"].data_ptr(); a.rope_sin = c["sin"].data_ptr()
    a.k_pages = cache.k_ptr(0); a.v_pages = cache.v_ptr(0); a.page_table = cache.page_table.data_ptr()
    a.desc = c["desc"].data_ptr()
    a.out = out[0].data_ptr(); a.out_lo = out[1].data_ptr(); a.ld_out = c["Hq"] * c["D"]; a.out_layout = N.W_TILED
    a.num_heads = c["Hq"]; a.num_kv_heads = c["Hkv"]; a.head_dim = c["D"]; a.rows_padded = c["MP"]
    a.scale = c["D"] ** -0.5; a.max_past_length = c["max_past"]; a.write_cache = 1
    if ws is not None:
        a.workspace = ws.data_ptr(); a.workspace_bytes = ws.numel()
    return a


def test_noalloc_attention_matches_workspace_entry(gpu_device, attn_kernel):
    lib = N.lib()
    assert lib.dtree_tree_attention_noalloc_max_bytes() == 32 << 20
    for P, L, max_past, seed in [(1000, 25, 1088, 3), (300, 10, 400, 4)]:  # second call: smaller input
        c = _case(gpu_device, P, L, max_past, seed)
        outs = []
        for k, cache in enumerate(c["caches"]):
            out = torch.full((2, c["MP"], c["Hq"] * c["D"]), 7.0, dtype=torch.bfloat16, device=gpu_device)
            if k == 0:
                ws = torch.zeros(lib.dtree_attention_workspace_bytes(c["Hq"], c["D"], max_past, c["MP"]),
                                 dtype=torch.uint8, device=gpu_device)
                N.check(lib.dtree_tree_attention(C.byref(_args(c, cache, out, ws)), stream()), "attention")
            else:
                N.check(lib.dtree_tree_attention_noalloc(C.byref(_args(c, cache, out)), stream()),
                        "attention (no alloc)")
            outs.append(out)
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1]), (P, L)
        assert torch.equal(c["caches"][0].k_pages, c["caches"][1].k_pages)
        assert torch.equal(c["caches"][0].v_pages, c["caches"][1].v_pages)
        # The output is in the tiled layout, so rows are not contiguous slices: check the
        # whole buffer was written (no fill value left) and holds finite values.
        assert bool(torch.isfinite(outs[1].float()).all())
        assert int((outs[1] == 7.0).sum()) == 0


def test_noalloc_attention_rejects_shapes_beyond_the_scratch(gpu_device, attn_kernel):
    lib = N.lib()
    c = _case(gpu_device, 0, 1, 64, 5)
    out = torch.zeros(2, c["MP"], c["Hq"] * c["D"], dtype=torch.bfloat16, device=gpu_device)
    a = _args(c, c["caches"][0], out)
    a.max_past_length = 16384  # needs far more than 32 MiB of partials
    assert lib.dtree_tree_attention_noalloc(C.byref(a), stream()) == N.E_WORKSPACE
    assert b"32 MiB" in lib.dtree_last_error()
