"""ctypes binding of libdtree_hip.so (the C ABI declared in include/dtree_hip.h).

The library is loaded from this package directory. There is no fallback: if
it is missing or stale the import of any compute entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libdtree_hip.so"

MAX_NODES = 128
MASK_WORDS = 4
PAGE = 64
ABI_VERSION = 8

E_OK, E_ARG, E_HIP, E_TREE, E_WORKSPACE = 0, -1, -2, -3, -4

EPI_STORE_F32 = 0
EPI_RESIDUAL = 1
EPI_SWIGLU = 2
EPI_STORE_BF16 = 3

W_ROWMAJOR = 0
W_TILED = 1
W_TILED_F16 = 3  # tiled fp16 weights + one fp16 activation plane
W_Q4G64 = 2


class DtreeError(RuntimeError):
    pass


class StepDesc(C.Structure):
    _fields_ = [
        ("past_length", C.c_int32),
        ("num_nodes", C.c_int32),
        ("n_accepted", C.c_int32),
        ("bonus_token", C.c_int32),
        ("tokens", C.c_int32 * MAX_NODES),
        ("positions", C.c_int32 * MAX_NODES),
        ("parents", C.c_int32 * MAX_NODES),
        ("ancestors", (C.c_uint32 * MASK_WORDS) * MAX_NODES),
        ("accepted", C.c_int32 * MAX_NODES),
        ("posterior", C.c_int32 * MAX_NODES),
    ]


# The same record as a numpy dtype (the host fills a pinned copy in place).
STEP_DESC_DTYPE = np.dtype([
    ("past_length", "<i4"), ("num_nodes", "<i4"), ("n_accepted", "<i4"), ("bonus_token", "<i4"),
    ("tokens", "<i4", (MAX_NODES,)), ("positions", "<i4", (MAX_NODES,)), ("parents", "<i4", (MAX_NODES,)),
    ("ancestors", "<u4", (MAX_NODES, MASK_WORDS)), ("accepted", "<i4", (MAX_NODES,)),
    ("posterior", "<i4", (MAX_NODES,)),
])
assert STEP_DESC_DTYPE.itemsize == C.sizeof(StepDesc)


class GemmArgs(C.Structure):
    _fields_ = [
        ("x", C.c_void_p), ("x_lo", C.c_void_p), ("x_layout", C.c_int32), ("ldx", C.c_int32),
        ("rows_padded", C.c_int32),
        ("w", C.c_void_p), ("w_layout", C.c_int32), ("n", C.c_int32), ("k", C.c_int32),
        ("epilogue", C.c_int32), ("split_k", C.c_int32),
        ("ss_in", C.c_void_p), ("ss_tiles", C.c_int32), ("norm_dim", C.c_int32), ("eps", C.c_float),
        ("out_f32", C.c_void_p), ("ld_out_f32", C.c_int32),
        ("out_bf16", C.c_void_p), ("out_lo", C.c_void_p), ("out_layout", C.c_int32), ("ld_out_bf16", C.c_int32),
        ("next_norm", C.c_void_p), ("ss_out", C.c_void_p),
        ("hidden_out", C.c_void_p), ("ld_hidden", C.c_int32),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
        ("w_scales", C.c_void_p),
    ]


class AttnArgs(C.Structure):
    _fields_ = [
        ("qkv", C.c_void_p), ("ld_qkv", C.c_int32),
        ("q_norm", C.c_void_p), ("k_norm", C.c_void_p), ("eps", C.c_float),
        ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p),
        ("k_pages", C.c_void_p), ("v_pages", C.c_void_p), ("page_table", C.c_void_p),
        ("desc", C.c_void_p),
        ("out", C.c_void_p), ("out_lo", C.c_void_p), ("ld_out", C.c_int32), ("out_layout", C.c_int32),
        ("num_heads", C.c_int32), ("num_kv_heads", C.c_int32), ("head_dim", C.c_int32),
        ("rows_padded", C.c_int32),
        ("scale", C.c_float),
        ("max_past_length", C.c_int32),
        ("write_cache", C.c_int32),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
        ("rope_dims", C.c_int32), ("gated", C.c_int32),
    ]


class GdnArgs(C.Structure):
    _fields_ = [
        ("desc", C.c_void_p), ("rows_padded", C.c_int32),
        ("num_k_heads", C.c_int32), ("num_v_heads", C.c_int32), ("head_k_dim", C.c_int32),
        ("head_v_dim", C.c_int32), ("conv_keep", C.c_int32),
        ("proj", C.c_void_p), ("ld_proj", C.c_int32),
        ("window", C.c_void_p), ("conv_w", C.c_void_p), ("A_log", C.c_void_p), ("dt_bias", C.c_void_p),
        ("state", C.c_void_p),
        ("q", C.c_void_p), ("k", C.c_void_p), ("v", C.c_void_p), ("g", C.c_void_p), ("beta", C.c_void_p),
        ("y", C.c_void_p),
        ("norm_w", C.c_void_p), ("eps", C.c_float),
        ("out", C.c_void_p), ("out_lo", C.c_void_p), ("out_layout", C.c_int32), ("ld_out", C.c_int32),
        ("window_out", C.c_void_p), ("state_out", C.c_void_p),
    ]


_vp, _i32, _f32, _sz = C.c_void_p, C.c_int32, C.c_float, C.c_size_t

# name -> (restype, argtypes)
SIGNATURES = {
    "dtree_last_error": (C.c_char_p, []),
    "dtree_abi_version": (C.c_int, []),
    "dtree_step_desc_bytes": (_sz, []),
    "dtree_validate_parents": (C.c_int, [_vp, _i32]),
    "dtree_step_desc_validate": (C.c_int, [_vp, _i32, _i32, _i32]),
    "dtree_gemm_args_bytes": (_sz, []),
    "dtree_attn_args_bytes": (_sz, []),
    "dtree_gemm_workspace_bytes": (_sz, [C.c_int, C.c_int, C.c_int, C.c_int]),
    "dtree_gemm_bf16": (C.c_int, [C.POINTER(GemmArgs), _vp]),
    "dtree_embed": (C.c_int, [_vp, _vp, _i32, _vp, _i32, _i32, _vp, _i32, _vp, _vp, _vp, _i32, _vp, _i32, _f32, _vp,
                              _vp, _vp]),
    "dtree_rope_table": (C.c_int, [_vp, _i32, _i32, _f32, _vp, _vp, _vp]),
    "dtree_attention_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32]),
    "dtree_tree_attention": (C.c_int, [C.POINTER(AttnArgs), _vp]),
    "dtree_tree_attention_noalloc_max_bytes": (_sz, []),
    "dtree_tree_attention_noalloc": (C.c_int, [C.POINTER(AttnArgs), _vp]),
    "dtree_attention_status": (C.c_int, [_vp, _vp, _vp]),
    "dtree_lmhead_candidates_bytes": (_sz, [_i32]),
    "dtree_lmhead_candidate_blocks": (C.c_int, [_i32, _i32]),
    "dtree_lmhead_argmax": (C.c_int, [_vp, _vp, _i32, _i32, _i32, _vp, _i32, _vp, _i32, _i32, _vp, _i32, _f32, _vp,
                                      _vp, _vp]),
    "dtree_tile_weight": (C.c_int, [_vp, _vp, _i32, _i32, _vp]),
    "dtree_tile_weight_f16": (C.c_int, [_vp, _vp, _i32, _i32, _vp]),
    "dtree_accept_walk": (C.c_int, [_vp, _vp, _i32, _i32, _vp, _vp]),
    "dtree_compact": (C.c_int, [_vp, _vp, _vp, _sz, _i32, _i32, _i32, _vp, _vp, _i32, _vp, _vp]),
    "dtree_rownorm": (C.c_int, [_vp, _i32, _i32, _i32, _vp, _i32, _vp, _f32, _vp, _i32, _vp]),
    "dtree_tree_build_workspace_bytes": (_sz, [_i32, _i32, _i32]),
    "dtree_tree_build": (C.c_int, [_vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _sz, _vp, _vp, _vp, _vp,
                                   _vp]),
    "dtree_gemm_long": (C.c_int, [C.POINTER(GemmArgs), _vp]),
    "dtree_embed_tokens": (C.c_int, [_vp, _i32, _vp, _i32, _vp, _i32, _i32, _vp, _i32, _vp, _vp, _vp, _i32, _vp, _vp]),
    "dtree_rows_in": (C.c_int, [_vp, _i32, _i32, _vp, _i32, _i32, _vp, _vp, _vp, _i32, _vp, _vp]),
    "dtree_kv_append": (C.c_int, [_vp, _i32, _i32, _i32, _vp, _f32, _i32, _i32, _f32, _i32, _i32, _vp, _vp, _vp, _i32,
                                  _vp]),
    "dtree_gdn_tree_conv": (C.c_int, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _vp]),
    "dtree_gdn_tree_recurrence": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp,
                                            _vp]),
    "dtree_gdn_commit": (C.c_int, [_vp, _vp, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32,
                                   _vp]),
    "dtree_gdn_args_bytes": (_sz, []),
    "dtree_gdn_tree_check": (C.c_int, [_vp, _i32]),
    "dtree_gdn_layer_prep": (C.c_int, [C.POINTER(GdnArgs), _vp]),
    "dtree_gdn_layer_recurrence": (C.c_int, [C.POINTER(GdnArgs), _vp]),
    "dtree_gdn_layer_prep_recurrence": (C.c_int, [C.POINTER(GdnArgs), _vp]),
    "dtree_gdn_layers_commit": (C.c_int, [C.POINTER(GdnArgs), _i32, _vp]),
    "dtree_gdn_layer_gated_norm": (C.c_int, [C.POINTER(GdnArgs), _vp]),
    "dtree_gdn_layer_commit": (C.c_int, [C.POINTER(GdnArgs), _vp]),
    "dtree_gdn_layer_chain": (C.c_int, [C.POINTER(GdnArgs), C.c_int32, _vp]),
    "dtree_graph_begin": (C.c_int, [_vp]),
    "dtree_graph_end": (C.c_int, [_vp, C.POINTER(C.c_void_p)]),
    "dtree_graph_launch": (C.c_int, [_vp, _vp]),
    "dtree_graph_destroy": (C.c_int, [_vp]),
}

_LIB: C.CDLL | None = None


def lib() -> C.CDLL:
    """Load the native library (raises if it is missing or has another ABI)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise DtreeError(
            f"native library {LIB_PATH} is missing; build it with "
            "`python dtree-mlx_amd/build_native.py` (or __graft_entry__.build())")
    h = C.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(h, name)
        fn.restype = res
        fn.argtypes = args
    if h.dtree_abi_version() != ABI_VERSION:
        raise DtreeError("libdtree_hip.so ABI version mismatch; rebuild it")
    for fn, struct in (("dtree_step_desc_bytes", StepDesc), ("dtree_gemm_args_bytes", GemmArgs),
                       ("dtree_attn_args_bytes", AttnArgs), ("dtree_gdn_args_bytes", GdnArgs)):
        if getattr(h, fn)() != C.sizeof(struct):
            raise DtreeError(f"{struct.__name__} layout mismatch between Python and the library")
    _LIB = h
    return h


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = lib().dtree_last_error().decode(errors="replace")
        raise DtreeError(f"{what or 'dtree call'} failed ({rc}): {msg}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)
