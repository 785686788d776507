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
    # attention: head counters (256-byte aligned) + one partial per head per
    # 4-chunk workgroup; prefix 1024 = tree + 16 pages = 5 workgroups per head
    assert lib.dtree_attention_workspace_bytes(32, 128, 1024) == 256 + 32 * 5 * (32 * 128 + 64) * 4
    assert lib.dtree_attention_workspace_bytes(32, 128, 0) == 256 + 32 * 1 * (32 * 128 + 64) * 4
