"""ctypes declarations of include/kvrecall.h (libkvrecall.so).

The library is the product: it must be built in-tree and load, or every entry
point here raises.  There is no fallback implementation.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libkvrecall.so")
HEADER = os.path.join(ROOT, "include", "kvrecall.h")

# enums
(OK, ERR_INVALID, ERR_NONFINITE, ERR_RANGE, ERR_BUDGET, ERR_WORKSPACE, ERR_HIP, ERR_SCORES, ERR_UNSUPPORTED,
 ERR_GRAPH) = range(10)
MEDIA_OVERLAP, MEDIA_IN_ORDER = 0, 1
HALF_NONE, HALF_SUM, HALF_MAX = 0, 1, 2
GROUP_SELECT_PAGES = 4096
FIXED_BITMAP_PAGES = 524288
GRAPH_MAX_PAGES = 8192
FMT_F16, FMT_Q8_0, FMT_Q4_1, FMT_F32, FMT_BF16, FMT_Q4_0, FMT_Q5_0 = range(7)
AGG_MEAN, AGG_MAX, AGG_MAX_LOGIT = range(3)
TIE_LOWER_FIRST, TIE_HIGHER_FIRST = range(2)
GATHER_COPY, GATHER_DEQUANT_F16, GATHER_REQUANT_Q8_0, GATHER_ROPE_FWHT = range(4)
ENGINE_AUTO, ENGINE_KERNEL, ENGINE_SDMA = range(3)
OPT_GATHER_WORKGROUPS, OPT_GATHER_CHUNK_ROWS, OPT_GATHER_THREADS, OPT_ATTN_PAGE_GROUP = 1, 2, 3, 4
MAX_INLINE_MANDATORY = 64
MAX_PLANES = 8
STACK_GROUP = 4
ATTENTION_ROWS = 64
NOALLOC_SCRATCH_BYTES = 16 << 20
NOALLOC_MAX_LANES = 1024

_P = C.c_void_p
_u32, _u64, _sz, _i = C.c_uint32, C.c_uint64, C.c_size_t, C.c_int


class KeyHistory(C.Structure):
    _fields_ = [("data", _P), ("format", _i), ("tokens", _u64), ("kv_heads", _u32),
                ("head_dim", _u32), ("page_tokens", _u32), ("lanes", _u32), ("lane_stride", _sz)]


class Query(C.Structure):
    _fields_ = [("data", _P), ("scalar", _i), ("rows", _u32), ("query_heads", _u32),
                ("kv_heads", _u32), ("head_dim", _u32), ("row_stride", _sz), ("head_stride", _sz),
                ("dim_stride", _sz), ("lane_stride", _sz), ("attention_scale", C.c_float)]


class Rope(C.Structure):
    _fields_ = [("head_dim", _u32), ("n_rot", _u32), ("theta", _P), ("fwht", _u32), ("pos_base", C.c_int64)]


class Plane(C.Structure):
    _fields_ = [("history", _P), ("format", _i), ("width", _u32), ("tokens", _u64), ("mode", _i),
                ("slots", _P), ("host_lane_stride", _sz), ("slot_lane_stride", _sz),
                ("rope", C.POINTER(Rope)), ("page_stride", _sz)]


class PagePolicy(C.Structure):
    _fields_ = [("fixed", _P), ("n_fixed", _u32), ("groups", _P), ("n_groups", _u32), ("preferred", _P),
                ("preferred_count", _P), ("preferred_stride", _u32)]


class Media(C.Structure):
    _fields_ = [("ranges", _P), ("n_ranges", _u32), ("page_tokens", _u32), ("total_tokens", _u64)]


class LayerRecall(C.Structure):
    _fields_ = [("keys", C.POINTER(KeyHistory)), ("summaries", _P), ("means", _P), ("pages", _u32),
                ("page_tokens", _u32), ("lanes", _u32), ("query", C.POINTER(Query)),
                ("score_mask", _P), ("aggregation", _i), ("k", _u32), ("tie_rule", _i),
                ("mandatory", C.POINTER(_u32)), ("n_mandatory", _u32), ("scores", _P),
                ("selected", _P), ("count", _P), ("planes", C.POINTER(Plane)), ("n_planes", _u32),
                ("engine", _i), ("force_mfma", _i), ("summary_begin", _P), ("summary_end", _P),
                ("select_end", _P), ("policy", C.POINTER(PagePolicy)), ("half_fold", _i)]


class AttentionSample(C.Structure):
    _fields_ = [("q", _P), ("q_format", _i), ("q_row_stride", _sz), ("q_head_stride", _sz),
                ("k", _P), ("k_format", _i), ("k_row_stride", _sz), ("k_head_stride", _sz),
                ("mask", _P), ("mask_format", _i), ("mask_row_stride", _sz), ("head_dim", _u32),
                ("query_heads", _u32), ("kv_heads", _u32), ("tokens", _u32), ("page_tokens", _u32),
                ("scale", C.c_float), ("softcap", C.c_float), ("rows", C.POINTER(_u32)), ("n_rows", _u32),
                ("mask_rows", C.POINTER(_u32))]


class PageGraph(C.Structure):
    _fields_ = [("n_rows", _u32), ("n_edges", _u32), ("row_source", _P), ("row_begin", _P),
                ("edge_target", _P), ("edge_mass", _P), ("neighbor_weight", _P)]


_SIGNATURES = {
    "kvr_create": (_i, [_i, C.POINTER(_P)]),
    "kvr_destroy": (_i, [_P]),
    "kvr_last_error": (C.c_char_p, []),
    "kvr_status_string": (C.c_char_p, [_i]),
    "kvr_check": (_i, [_P, _P]),
    "kvr_set_option": (_i, [_P, _i, C.c_int64]),
    "kvr_select_stream": (_P, [_P]),
    "kvr_copy_stream": (_P, [_P]),
    "kvr_workspace_bytes": (_sz, [_u32, _u32, _u32, _u32, _u32, _u32]),
    "kvr_bind_workspace": (_i, [_P, _P, _sz]),
    "kvr_device_bytes": (_sz, [_P]),
    "kvr_summary_build": (_i, [_P, C.POINTER(KeyHistory), _P, _P, _P]),
    "kvr_summary_accumulate": (_i, [_P, _P, _P, _u32, _P, _i, _u64, _u32, _u32, _u32, _sz, _sz, _sz, _P]),
    "kvr_summary_finalize": (_i, [_P, _P, _P, _u32, _u32, _P, _P, _P]),
    "kvr_score": (_i, [_P, C.POINTER(Query), _P, _u32, _u32, _P, _i, _u32, _i, _P, _i, _P]),
    "kvr_select_topk": (_i, [_P, _P, _u32, _u32, _u32, C.POINTER(_u32), _u32, _i, _i, _P, _P, _P]),
    "kvr_fold_half_pages": (_i, [_P, _P, _u32, _u32, _P, _i, _P, _P]),
    "kvr_select_pages": (_i, [_P, _P, _u32, _u32, _u32, C.POINTER(PagePolicy), _i, _i, _P, _P, _P]),
    "kvr_media_page_groups": (_i, [C.POINTER(Media), _u32, _i, C.POINTER(_u32), C.POINTER(_u32)]),
    "kvr_query_fixed_pages": (_i, [_u32, _u32, _u32, _u32, C.POINTER(Media), C.POINTER(_u32), _u32,
                                   C.POINTER(_u32), C.POINTER(_u32)]),
    "kvr_topk_fixed_pages": (_i, [_u32, _u32, _u32, _u32, C.POINTER(_u32), _u32, C.POINTER(_u32), C.POINTER(_u32)]),
    "kvr_media_fixed_pages": (_i, [_u32, _u32, _u32, C.POINTER(Media), C.POINTER(_u32), _u32, C.POINTER(_u32),
                                   C.POINTER(_u32)]),
    "kvr_stage_in": (_i, [_P, C.POINTER(Plane), _u32, _u32, _u32, _P, _P, _u32, _i, _P]),
    "kvr_recall_layer": (_i, [_P, C.POINTER(LayerRecall), _P, _P]),
    "kvr_recall_stack": (_i, [_P, C.POINTER(LayerRecall), _u32, _P, _P]),
    "kvr_recall_layer_noalloc": (_i, [_P, C.POINTER(LayerRecall), _P, _P]),
    "kvr_attention_workspace_bytes": (_sz, [_u32, _u32, _u32]),
    "kvr_attention_page_mass": (_i, [_P, C.POINTER(AttentionSample), _P, _P]),
    "kvr_propagate_scores": (_i, [_P, _P, _u32, _u32, _P, C.POINTER(PageGraph), C.c_double, _P]),
    "kvr_lrfu_preview": (_i, [_P, _P, _u32, _u32, _P, _u32, C.c_double, C.c_double, _P, _P]),
    "kvr_propagate_lrfu": (_i, [_P, _P, _u32, _u32, _P, C.POINTER(PageGraph), C.c_double, _P, _u32, C.c_double,
                                C.c_double, _P, _P]),
    "kvr_d2d_batched": (_i, [_P, C.POINTER(_P), C.POINTER(_P), C.POINTER(_sz), _u32, _P]),
    "kvr_host_alloc": (_i, [_sz, C.POINTER(_P)]),
    "kvr_host_free": (_i, [_P]),
    "kvr_h2d_peak_gbps": (_i, [_P, _sz, _i, C.POINTER(C.c_double)]),
    "kvr_h2d_read_peak_gbps": (_i, [_P, _sz, _i, C.POINTER(C.c_double)]),
    "kvr_synth_normal_f16": (_i, [_P, _u64, _u64, _u64, _P, _P]),
    "kvr_synth_scaled_normal_f16": (_i, [_P, _u64, _u64, _u64, _u32, _P, _P, _P]),
    "kvr_synth_normal_f32": (_i, [_P, _u64, _u64, _u64, _P, _P]),
    "kvr_synth_q8_0": (_i, [_P, _u64, _u64, _u64, C.c_float, C.c_float, _P, _P]),
    "kvr_synth_q4_1": (_i, [_P, _u64, _u64, _u64, C.c_float, C.c_float, C.c_float, C.c_float, _P, _P]),
    "kvr_synth_normal_q8_0": (_i, [_P, _u64, _u64, _u64, _P, _P]),
}


def header_symbols() -> list[str]:
    """Entry points declared in include/kvrecall.h."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kvr_[a-z0-9_]+)\s*\(", text)))


class KvrError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"kvrecall status {status}: {message}")
        self.status = status


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build()")
        handle = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status != OK:
        raise KvrError(status, lib().kvr_last_error().decode())
