"""ctypes binding of libd2sd.so (C ABI declared in include/d2sd.h).

The library is loaded at import; a missing library raises ImportError — there
is no fallback path.  Device work additionally requires ROCm device tensors.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libd2sd.so"
TORCH_LIB_PATH = Path(__file__).resolve().parent / "libd2sd_torch.so"

D2SD_OK = 0
D2SD_ERR_WORKSPACE = 3
D2SD_KV_BF16 = 0
D2SD_KV_FP8_E4M3 = 1
D2SD_MASK_NONE = 0
D2SD_MASK_CAUSAL = 1
D2SD_MASK_TREE = 2
D2SD_DTYPE_BF16 = 0
D2SD_DTYPE_F32 = 1

# Every symbol include/d2sd.h declares.
EXPORTED_SYMBOLS = (
    "d2sd_last_error",
    "d2sd_version",
    "d2sd_merge_state_in_place",
    "d2sd_single_prefill_workspace_size",
    "d2sd_single_prefill_with_kv_cache",
    "d2sd_local_attention_merge",
    "d2sd_graph_begin_capture",
    "d2sd_graph_end_capture",
    "d2sd_graph_launch",
    "d2sd_graph_destroy",
    "d2sd_cascade_plan",
    "d2sd_cascade_run",
    "d2sd_cascade_attention",
    "d2sd_cascade_merge",
    "d2sd_cascade_scratch_bytes",
    "d2sd_cascade_run_noalloc",
    "d2sd_paged_kv_append",
    "d2sd_greedy_accept_workspace_size",
    "d2sd_greedy_accept",
    "d2sd_sample_accept",
    "d2sd_qk_norm_rope",
    "d2sd_d3_tree_build",
)


class PlanDesc(C.Structure):
    _fields_ = [
        ("num_reqs", C.c_int),
        ("qo_indptr", C.POINTER(C.c_int32)),
        ("prefix_len", C.POINTER(C.c_int32)),
        ("page_indptr", C.POINTER(C.c_int32)),
        ("prefix_tok_indptr", C.POINTER(C.c_int32)),
        ("num_qo_heads", C.c_int),
        ("num_kv_heads", C.c_int),
        ("head_dim", C.c_int),
        ("window_left", C.c_int),
        ("kv_dtype", C.c_int),
        ("page_size", C.c_int),
        ("num_cus", C.c_int),
        ("max_splits", C.c_int),
        ("waves_per_block", C.c_int),
        ("dynamic_prefix", C.c_int),
        ("prefix_split", C.POINTER(C.c_int32)),
        ("prefix2_tok_indptr", C.POINTER(C.c_int32)),
    ]


class PlanInfo(C.Structure):
    _fields_ = [
        ("num_items", C.c_int),
        ("num_merges", C.c_int),
        ("waves_per_block", C.c_int),
        ("rows_per_tile", C.c_int),
        ("num_slots", C.c_int),
        ("plan_ints", C.c_int),
        ("workspace_bytes", C.c_size_t),
        ("max_splits_used", C.c_int),
        ("num_reqs", C.c_int),
        ("num_qo_heads", C.c_int),
        ("num_kv_heads", C.c_int),
        ("head_dim", C.c_int),
        ("kv_dtype", C.c_int),
        ("page_size", C.c_int),
        ("num_groups", C.c_int),
        ("dynamic_prefix", C.c_int),
        ("window_left", C.c_int),
        ("prefix_extent", C.c_int64),
        ("max_qo_len", C.c_int),
        ("fused", C.c_int),
        ("two_segment", C.c_int),
        ("prefix2_extent", C.c_int64),
    ]


class RunArgs(C.Structure):
    _fields_ = [
        ("plan", C.c_void_p),
        ("q", C.c_void_p),
        ("q_stride_n", C.c_int64),
        ("q_stride_h", C.c_int64),
        ("k_suffix", C.c_void_p),
        ("v_suffix", C.c_void_p),
        ("suffix_stride_n", C.c_int64),
        ("suffix_stride_h", C.c_int64),
        ("mask_mode", C.c_int),
        ("mask_words", C.c_int),
        ("tree_mask", C.c_void_p),
        ("k_prefix", C.c_void_p),
        ("v_prefix", C.c_void_p),
        ("prefix_stride_tok", C.c_int64),
        ("prefix_stride_head", C.c_int64),
        ("prefix_stride_page", C.c_int64),
        ("page_size", C.c_int),
        ("page_table", C.c_void_p),
        ("prefix_extent", C.c_int64),
        ("prefix_len", C.c_void_p),
        ("k_scale", C.c_void_p),
        ("v_scale", C.c_void_p),
        ("sinks", C.c_void_p),
        ("out", C.c_void_p),
        ("o_stride_n", C.c_int64),
        ("o_stride_h", C.c_int64),
        ("lse", C.c_void_p),
        ("lse_stride_n", C.c_int64),
        ("sm_scale", C.c_float),
        ("lse_base2", C.c_int),
        ("workspace", C.c_void_p),
        ("workspace_bytes", C.c_size_t),
        ("k_prefix2", C.c_void_p),
        ("v_prefix2", C.c_void_p),
        ("prefix2_stride_tok", C.c_int64),
        ("prefix2_stride_head", C.c_int64),
        ("prefix2_extent", C.c_int64),
        ("k2_scale", C.c_void_p),
        ("v2_scale", C.c_void_p),
    ]


class KvAppendArgs(C.Structure):
    _fields_ = [
        ("num_layers", C.c_int),
        ("num_kv_heads", C.c_int),
        ("head_dim", C.c_int),
        ("page_size", C.c_int),
        ("prefix_len", C.c_int),
        ("num_accepted", C.c_int),
        ("num_rows", C.c_int),
        ("pool_pages", C.c_int),
        ("page_table_len", C.c_int),
        ("node_ids", C.c_void_p),
        ("page_table", C.c_void_p),
        ("k_new", C.c_void_p),
        ("v_new", C.c_void_p),
        ("k_pool", C.c_void_p),
        ("v_pool", C.c_void_p),
        ("new_stride_n", C.c_int64),
        ("new_stride_h", C.c_int64),
        ("pool_stride_page", C.c_int64),
        ("pool_stride_head", C.c_int64),
        ("pool_stride_tok", C.c_int64),
        ("num_accepted_dev", C.c_void_p),
        ("prefix_len_dev", C.c_void_p),
        ("advance_prefix", C.c_int),
        ("pool_dtype", C.c_int),
        ("k_scale", C.c_void_p),
        ("v_scale", C.c_void_p),
    ]


class QkRopeArgs(C.Structure):
    _fields_ = [
        ("q", C.c_void_p),
        ("k", C.c_void_p),
        ("q_stride_n", C.c_int64),
        ("q_stride_h", C.c_int64),
        ("k_stride_n", C.c_int64),
        ("k_stride_h", C.c_int64),
        ("q_norm", C.c_void_p),
        ("k_norm", C.c_void_p),
        ("cos", C.c_void_p),
        ("sin", C.c_void_p),
        ("cs_stride", C.c_int64),
        ("eps", C.c_float),
        ("num_tokens", C.c_int),
        ("num_qo_heads", C.c_int),
        ("num_kv_heads", C.c_int),
        ("head_dim", C.c_int),
        ("half_cos", C.c_int),
    ]


class TreeArgs(C.Structure):
    _fields_ = [
        ("conf", C.c_void_p),
        ("conf_dtype", C.c_int),
        ("block_size", C.c_int),
        ("block_size_2", C.c_int),
        ("topk", C.c_int),
        ("capacity", C.c_int),
        ("rows_cap", C.c_int),
        ("mask_words", C.c_int),
        ("num_nodes", C.c_void_p),
        ("num_rows", C.c_void_p),
        ("parents", C.c_void_p),
        ("node_index", C.c_void_p),
        ("tree_mask", C.c_void_p),
        ("shared", C.c_void_p),
        ("rates", C.c_void_p),
    ]


class AcceptArgs(C.Structure):
    _fields_ = [
        ("num_rows", C.c_int),
        ("row_len", C.c_int),
        ("num_nodes", C.c_int),
        ("vocab", C.c_int),
        ("logits_dtype", C.c_int),
        ("logits", C.c_void_p),
        ("logits_stride", C.c_int64),
        ("node_index", C.c_void_p),
        ("draft_ids", C.c_void_p),
        ("accept_ids", C.c_void_p),
        ("accept_nodes", C.c_void_p),
        ("result", C.c_void_p),
        ("workspace", C.c_void_p),
        ("workspace_bytes", C.c_size_t),
    ]


class SampleAcceptArgs(C.Structure):
    _fields_ = [
        ("walk", AcceptArgs),
        ("temperature", C.c_float),
        ("seed", C.c_uint64),
        ("rng_step", C.c_void_p),
        ("node_tokens", C.c_void_p),
    ]


# int32 entries per attention item / merge item in the host plan
PLAN_ITEM_INTS = 16
PLAN_MERGE_INTS = 8


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()' "
            "or python d2-sd_amd/d2sd/_build.py)")
    # global: libd2sd_torch.so (torch.ops.d2sd) links this same instance by soname
    lib = C.CDLL(str(LIB_PATH), mode=C.RTLD_GLOBAL)
    vp, i64, i32, f32, sz = C.c_void_p, C.c_int64, C.c_int, C.c_float, C.c_size_t
    lib.d2sd_last_error.restype = C.c_char_p
    lib.d2sd_last_error.argtypes = []
    lib.d2sd_version.restype = C.c_char_p
    lib.d2sd_version.argtypes = []
    lib.d2sd_merge_state_in_place.restype = i32
    lib.d2sd_merge_state_in_place.argtypes = [vp, i64, i64, vp, i64, vp, i64, i64, vp, i64, i32, i32, i32, i32, vp]
    lib.d2sd_single_prefill_workspace_size.restype = sz
    lib.d2sd_single_prefill_workspace_size.argtypes = [i32, i32, i32, i32, i32, i32]
    lib.d2sd_single_prefill_with_kv_cache.restype = i32
    lib.d2sd_single_prefill_with_kv_cache.argtypes = [
        vp, i64, i64, vp, vp, i64, i64, vp, i64, i64, vp, i32, i32, i32, i32, i32, i32, i32, f32, i32, vp, sz, vp]
    lib.d2sd_local_attention_merge.restype = i32
    lib.d2sd_local_attention_merge.argtypes = [
        vp, i64, i64, i64, vp, vp, i64, i64, i64, vp, i64, i64, i64, vp, i64, i64,
        i32, i32, i32, i32, i32, i32, f32, vp, i32, vp]
    lib.d2sd_graph_begin_capture.restype = i32
    lib.d2sd_graph_begin_capture.argtypes = [vp]
    lib.d2sd_graph_end_capture.restype = i32
    lib.d2sd_graph_end_capture.argtypes = [vp, C.POINTER(C.c_void_p)]
    lib.d2sd_graph_launch.restype = i32
    lib.d2sd_graph_launch.argtypes = [vp, vp]
    lib.d2sd_graph_destroy.restype = i32
    lib.d2sd_graph_destroy.argtypes = [vp]
    lib.d2sd_cascade_plan.restype = i32
    lib.d2sd_cascade_plan.argtypes = [C.POINTER(PlanDesc), C.POINTER(C.c_int32), sz, C.POINTER(PlanInfo)]
    lib.d2sd_cascade_scratch_bytes.restype = sz
    lib.d2sd_cascade_scratch_bytes.argtypes = []
    for name in ("d2sd_cascade_run", "d2sd_cascade_attention", "d2sd_cascade_merge", "d2sd_cascade_run_noalloc"):
        fn = getattr(lib, name)
        fn.restype = i32
        fn.argtypes = [C.POINTER(PlanInfo), C.POINTER(RunArgs), vp]
    lib.d2sd_paged_kv_append.restype = i32
    lib.d2sd_paged_kv_append.argtypes = [C.POINTER(KvAppendArgs), vp]
    lib.d2sd_greedy_accept_workspace_size.restype = sz
    lib.d2sd_greedy_accept_workspace_size.argtypes = [i32, i32]
    lib.d2sd_greedy_accept.restype = i32
    lib.d2sd_greedy_accept.argtypes = [C.POINTER(AcceptArgs), vp]
    lib.d2sd_sample_accept.restype = i32
    lib.d2sd_sample_accept.argtypes = [C.POINTER(SampleAcceptArgs), vp]
    lib.d2sd_d3_tree_build.restype = i32
    lib.d2sd_d3_tree_build.argtypes = [C.POINTER(TreeArgs), vp]
    lib.d2sd_qk_norm_rope.restype = i32
    lib.d2sd_qk_norm_rope.argtypes = [C.POINTER(QkRopeArgs), vp]
    return lib


lib = _load()


def _load_torch_ops() -> None:
    """Registers torch.ops.d2sd.* (libd2sd_torch.so, built with libd2sd.so)."""
    import torch
    if not TORCH_LIB_PATH.exists():
        raise ImportError(f"{TORCH_LIB_PATH} is missing: build it first (d2-sd_amd/d2sd/_build.py)")
    torch.ops.load_library(str(TORCH_LIB_PATH))


_load_torch_ops()


def check(rc: int, what: str) -> None:
    if rc != D2SD_OK:
        msg = lib.d2sd_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def version() -> str:
    return lib.d2sd_version().decode()
