"""The C-ABI library loads and exports every entry point include/dtree_hip.h
declares; argument validation fails with DTREE_E_ARG before any launch.
CPU only (no kernel runs)."""
import ctypes as C
import re
from pathlib import Path

import pytest

from dtree_hip import _native as N

HEADER = Path(__file__).resolve().parents[1] / "include" / "dtree_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dtree_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for must in ("dtree_gemm_bf16", "dtree_tree_attention", "dtree_lmhead_argmax", "dtree_accept_walk",
                 "dtree_compact", "dtree_embed", "dtree_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = N.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(declared_functions()) <= set(N.SIGNATURES), "ctypes signatures must cover the header"


def test_abi_version_and_descriptor_layout():
    lib = N.lib()
    assert lib.dtree_abi_version() == N.ABI_VERSION
    assert lib.dtree_step_desc_bytes() == C.sizeof(N.StepDesc) == 16 + 128 * 4 * 3 + 128 * 16 + 128 * 4 * 2


def test_argument_validation_without_gpu():
    lib = N.lib()
    a = N.GemmArgs()
    assert lib.dtree_gemm_bf16(C.byref(a), None) == -1
    assert b"null" in lib.dtree_last_error()
    a.x = 16; a.w = 16; a.n = 40; a.k = 64; a.ldx = 64; a.rows_padded = 32
    assert lib.dtree_gemm_bf16(C.byref(a), None) == -1
    assert b"multiple of 64" in lib.dtree_last_error()
    a.n = 64; a.rows_padded = 48
    assert lib.dtree_gemm_bf16(C.byref(a), None) == -1
    assert b"rows_padded" in lib.dtree_last_error()
    att = N.AttnArgs()
    assert lib.dtree_tree_attention(C.byref(att), None) == -1
    assert lib.dtree_accept_walk(None, None, 1, 32, None, None) == -1
    with pytest.raises(N.DtreeError):
        N.check(-1, "probe")


def test_workspace_queries():
    lib = N.lib()
    # split-K 1 needs only the fixed tile-counter region
    assert lib.dtree_gemm_workspace_bytes(32, 2560, 4096, 1) == 65536
    # split-K 8: counters + 80 tiles * 8 splits * 32x32 fp32
    assert lib.dtree_gemm_workspace_bytes(32, 2560, 4096, 8) == 65536 + 80 * 8 * 32 * 32 * 4
    assert lib.dtree_lmhead_candidate_blocks(151936, 32) == 1024
    assert lib.dtree_lmhead_candidate_blocks(4096, 32) == 64
    assert lib.dtree_lmhead_candidate_blocks(4096, 128) == 128
    # attention: the larger of the two designs' workspaces. Both start with a
    # 4 KB header (error word, exchange-table place, counters) and, for 32-row
    # trees, the per-head flag exchange region: one epoch word per head
    # (256-byte aligned block), then 8 slots per head of 512 bytes of row
    # statistics and 4 * D / 32 units of 2 KB of (value, flag) pairs.
    def ll_bytes(Hq, D, MP):
        if MP != 32:
            return 0
        return ((Hq * 4 + 255) // 256) * 256 + Hq * 8 * (512 + 4 * (D // 32) * 2048)

    # Per-head kernel: + one partial per head per workgroup for the
    # last-arriver / separate combine; head_dim 128 gives the tree chunks a
    # workgroup of its own (prefix 1024 = 16 pages -> 1 + 4 workgroups per
    # head), head_dim 256 packs four chunks per workgroup, tree chunks last.
    def head_ws(Hq, D, P, MP):
        nt = MP // 32
        ck = 64 if D == 128 else 32
        npre = (P + ck - 1) // ck
        splits = 1 + (npre + 3) // 4 if D == 128 else (nt + npre + 3) // 4
        return 4096 + ll_bytes(Hq, D, MP) + Hq * nt * splits * (32 * D + 64) * 4

    # Per-KV-group kernel: + at most one partial (32 rows x head_dim fp32 +
    # row max / sum) per head, query block and split, with at most one split
    # per prefix chunk plus the tree split.
    def group_ws(Hq, D, P, MP):
        nt = MP // 32
        ck = 64 if D == 128 else 32
        return 4096 + ll_bytes(Hq, D, MP) + Hq * nt * (1 + (P + ck - 1) // ck) * ((D // 32) * 64 * 16 + 64) * 4

    for Hq, D, P, MP in [(32, 128, 1024, 32), (32, 128, 0, 32), (16, 256, 2048, 32), (32, 128, 1024, 96),
                         (16, 256, 8192, 96)]:
        want = max(head_ws(Hq, D, P, MP), group_ws(Hq, D, P, MP))
        assert lib.dtree_attention_workspace_bytes(Hq, D, P, MP) == want, (Hq, D, P, MP)
    assert head_ws(32, 128, 1024, 96) == 4096 + 32 * 3 * 5 * (32 * 128 + 64) * 4
    assert ll_bytes(32, 128, 32) == 256 + 32 * 8 * 33280
    assert lib.dtree_attention_workspace_bytes(32, 128, 1024, 48) == 0


def test_struct_sizes_match_the_library():
    lib = N.lib()
    assert lib.dtree_gemm_args_bytes() == C.sizeof(N.GemmArgs)
    assert lib.dtree_attn_args_bytes() == C.sizeof(N.AttnArgs)
    assert lib.dtree_gdn_args_bytes() == C.sizeof(N.GdnArgs)


def test_attention_and_gdn_layer_validation_without_gpu():
    lib = N.lib()
    att = N.AttnArgs()
    for f in ("qkv", "rope_cos", "rope_sin", "k_pages", "v_pages", "page_table", "desc", "out", "workspace"):
        setattr(att, f, 256)
    att.num_heads, att.num_kv_heads, att.rows_padded = 16, 4, 32
    att.head_dim, att.rope_dims, att.gated = 256, 256, 0  # head_dim 256 is compiled gated with rope_dims 64 only
    assert lib.dtree_tree_attention(C.byref(att), None) == -1
    assert b"geometries" in lib.dtree_last_error()
    att.rope_dims, att.gated, att.ld_qkv = 64, 1, 16 * 512  # k / v columns missing
    assert lib.dtree_tree_attention(C.byref(att), None) == -1
    assert b"ld_qkv" in lib.dtree_last_error()
    g = N.GdnArgs()
    assert lib.dtree_gdn_layer_prep(C.byref(g), None) == -1
    g.desc, g.rows_padded, g.num_k_heads, g.num_v_heads, g.conv_keep = 256, 32, 16, 32, 3
    g.head_k_dim, g.head_v_dim = 64, 128
    assert lib.dtree_gdn_layer_recurrence(C.byref(g), None) == -1
    assert b"head dims" in lib.dtree_last_error()
    g.head_k_dim = 128
    for f in ("proj", "window", "conv_w", "A_log", "dt_bias", "q", "k", "v", "g", "beta"):
        setattr(g, f, 256)
    g.ld_proj = 8192 + 4096  # b and a columns missing
    assert lib.dtree_gdn_layer_prep(C.byref(g), None) == -1
    assert b"ld_proj" in lib.dtree_last_error()
    # commit destinations: both or neither, and never a partial overlap
    g.ld_proj = 8192 + 4096 + 64
    g.state = 1 << 32
    g.window_out = 1 << 33
    assert lib.dtree_gdn_layer_commit(C.byref(g), None) == -1
    assert b"together" in lib.dtree_last_error()
    g.state_out = (1 << 32) + 4096
    assert lib.dtree_gdn_layer_commit(C.byref(g), None) == -1
    assert b"overlaps" in lib.dtree_last_error()


def _desc(parents, tokens=None, P=10):
    from dtree_hip import _native as N
    from dtree_hip.engine import ancestor_bitsets

    d = N.StepDesc()
    L = len(parents)
    d.past_length, d.num_nodes = P, L
    anc = ancestor_bitsets(parents)
    for i in range(L):
        d.parents[i] = parents[i]
        d.tokens[i] = (tokens or [3] * L)[i]
        d.positions[i] = P + i
        for w in range(N.MASK_WORDS):
            d.ancestors[i][w] = int(anc[i, w])
    return d


def test_host_tree_validation():
    """dtree_validate_parents / dtree_step_desc_validate (host only, no device
    work): DTREE_E_TREE for non-topological parents, a wrong root, more nodes
    than allowed or ancestor sets that are not the parent's plus the node;
    DTREE_E_ARG for out-of-range tokens, past lengths and accepted indices."""
    import ctypes as C

    from dtree_hip import _native as N

    lib = N.lib()
    ok = (C.c_int32 * 5)(-1, 0, 0, 1, 2)
    assert lib.dtree_validate_parents(ok, 5) == 0
    for bad in ((0, 0, 0), (-1, 1, 0), (-1, 0, 2), (-1, -1, 0)):
        arr = (C.c_int32 * 3)(*bad)
        assert lib.dtree_validate_parents(arr, 3) == N.E_TREE, bad
    assert lib.dtree_validate_parents(ok, 0) == N.E_TREE
    d = _desc([-1, 0, 0, 1, 2])
    assert lib.dtree_step_desc_validate(C.byref(d), 32, 100, 50) == 0
    assert lib.dtree_step_desc_validate(C.byref(d), 4, 100, 50) == N.E_TREE      # more nodes than max_nodes
    assert lib.dtree_step_desc_validate(C.byref(d), 32, 5, 50) == N.E_ARG        # past_length > max_past
    d.ancestors[3][0] = 0b1001                                                    # node 3 without its parent 1
    assert lib.dtree_step_desc_validate(C.byref(d), 32, 100, 50) == N.E_TREE
    assert b"ancestors[3]" in lib.dtree_last_error()
    d = _desc([-1, 0, 0], tokens=[1, 2, 50])
    assert lib.dtree_step_desc_validate(C.byref(d), 32, 100, 50) == N.E_ARG
    d = _desc([-1, 0, 0])
    d.n_accepted, d.accepted[0], d.accepted[1] = 2, 0, 3
    assert lib.dtree_step_desc_validate(C.byref(d), 32, 100, 50) == N.E_ARG
    d.accepted[1] = 2
    assert lib.dtree_step_desc_validate(C.byref(d), 32, 100, 50) == 0


def test_gdn_tree_check_bounds_the_nested_branching():
    """dtree_gdn_tree_check: trees of more than 32 nodes run the depth-first
    recurrence, whose state stack holds 31 nested branching nodes. A
    caterpillar (path node j also carries a leaf, so it has j branching
    ancestors) with 31 branching nodes passes, with 32 it is DTREE_E_TREE;
    32-node trees always pass; malformed parents are DTREE_E_TREE too."""
    lib = N.lib()

    def check(par):
        arr = (C.c_int32 * len(par))(*par)
        return lib.dtree_gdn_tree_check(arr, len(par))

    def caterpillar(n):
        par = [-1]
        for j in range(n):
            par += [2 * j, 2 * j]
        return par

    assert check(caterpillar(31)) == 0
    assert check(caterpillar(32)) == -3
    assert b"nested branching" in lib.dtree_last_error()
    assert check(caterpillar(15) + [30]) == 0  # 32 nodes: the register-resident recurrence
    assert check([-1] + list(range(95))) == 0  # a 96-node chain has no branching node
    assert check([-1, 0, 5]) == -3  # parent after the child

