"""ctypes bindings for the checkers: the C restatement (liboracle.so) and,
where it was built, the reference's own host library (_ref/libkvmem_ref.so).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, by __graft_entry__.smoke()
and by bench.py's CPU-baseline leg; the product package never imports it.
Array arguments are numpy arrays; results come back as numpy arrays.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OK, ERR_ARG, ERR_NONFINITE, ERR_RANGE, ERR_BUDGET = 0, 1, 2, 3, 4
AGG_MEAN, AGG_MAX, AGG_MAX_LOGIT = 0, 1, 2
TIE_LOWER_FIRST, TIE_HIGHER_FIRST = 0, 1
FMT_F16, FMT_Q8_0, FMT_Q4_1, FMT_F32, FMT_BF16, FMT_Q4_0, FMT_Q5_0 = range(7)
GATHER_COPY, GATHER_DEQUANT_F16, GATHER_REQUANT_Q8_0 = 0, 1, 2
QK, Q8_0_BYTES, Q4_1_BYTES, Q4_0_BYTES, Q5_0_BYTES = 32, 34, 20, 18, 22

_P = C.c_void_p
_u8, _u16, _u32, _u64 = C.c_uint8, C.c_uint16, C.c_uint32, C.c_uint64


class OracleError(RuntimeError):
    def __init__(self, code: int, what: str = ""):
        super().__init__(f"oracle status {code}{': ' + what if what else ''}")
        self.code = code


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(_P)


def _load_oracle() -> C.CDLL:
    path = os.path.join(HERE, "liboracle.so")
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built; run __graft_entry__.build()")
    lib = C.CDLL(path)
    sig = {
        "orc_f32_to_f16": (_u16, [C.c_float]),
        "orc_f16_to_f32": (C.c_float, [_u16]),
        "orc_recall_fp16": (C.c_int, [C.c_float, _P]),
        "orc_page_count": (_u32, [_u64, _u32]),
        "orc_query_score_frame": (C.c_int, [_u64, _u32, _u32, _u32, _u32, _P, _u32, _P, _P, _P, _P]),
        "orc_row_bytes": (C.c_size_t, [C.c_int, _u32]),
        "orc_page_summaries": (C.c_int, [_P, C.c_int, _u64, _u32, _u32, _P, _P]),
        "orc_page_softmax_scores": (C.c_int, [_P, _P, _P, _u32, _u32, _u32, _u32, _u32, _u32, _P,
                                              C.c_float, C.c_int, _P]),
        "orc_page_logits": (C.c_int, [_P, _P, _u32, _u32, _u32, _u32, _u32, C.c_float, _P]),
        "orc_pick_scored_blocks": (C.c_int, [_P, _u32, _P, _u32, _u32, C.c_int, C.c_int, _P, _P]),
        "orc_layerwise_fold": (C.c_int, [_P, _u32, _P, C.c_int, _P]),
        "orc_media_group": (None, [_u32, _u32, _u32, _P, _u32, _P, _P]),
        "orc_query_fixed_blocks": (C.c_int, [_u32, _u32, _u32, _u32, _P, _u32, _u64, _u32, _P, _u32, _P, _P]),
        "orc_pick_scored_grouped": (C.c_int, [_P, _u32, _P, _u32, _u32, C.c_int, C.c_int, _P, _u32, _u32, _P, _P]),
        "orc_pick_topk_ungrouped": (C.c_int, [_P, _u32, _u32, _u32, _u32, _P, _u32, _P, _P]),
        "orc_constrain_media": (C.c_int, [_P, _u32, _P, _u32, _u32, _u32, _P, _u32, _u64, _u32, _P, _u32, _P, _P]),
        "orc_dequant_q8_0": (None, [_P, _P]),
        "orc_dequant_q4_1": (None, [_P, _P]),
        "orc_quant_q8_0": (None, [_P, _P]),
        "orc_dequant_q4_0": (None, [_P, _P]),
        "orc_quant_q4_0": (None, [_P, _P]),
        "orc_rope_sincos": (None, [C.c_float, _P, _P]),
        "orc_rope_neox_row": (None, [_P, _u32, _u32, _u32, _P, C.c_float]),
        "orc_fwht_row": (None, [_P, _u32, _u32]),
        "orc_rope_fwht_rows": (C.c_int, [_P, C.c_int, _u32, _u32, C.c_int64, _u32, _u32, _P, _u32, _P]),
        "orc_rope_fwht_rows_variant": (C.c_int, [_P, C.c_int, _u32, _u32, C.c_int64, _u32, _u32, _P, _u32,
                                                 C.c_int, _P]),
        "orc_gather_rope": (C.c_int, [_P, C.c_int, _u32, _u64, _u32, _P, _u32, _u32, _u32, _P, _u32,
                                      C.c_int64, _P]),
        "orc_dequant_q5_0": (None, [_P, _P]),
        "orc_attention_page_mass": (C.c_int, [_P, C.c_int, C.c_size_t, C.c_size_t, _P, C.c_int, C.c_size_t,
                                              C.c_size_t, _P, C.c_int, C.c_size_t, _u32, _u32, _u32, _u32,
                                              _u32, C.c_float, C.c_float, _P, _u32, _P]),
        "orc_gather_row_bytes": (C.c_size_t, [C.c_int, C.c_int, _u32]),
        "orc_gather": (C.c_int, [_P, C.c_int, _u32, _u64, _u32, _P, _u32, C.c_int, _P]),
        "orc_span_coefficients": (C.c_int, [_P, _P, _P, _u32, _u32, _u32, C.c_double, _P]),
        "orc_propagate_scores": (C.c_int, [_P, _P, _u32, _u32, _P, _P, _P, _P, _P, C.c_double, _P]),
        "orc_lrfu_preview": (C.c_int, [_P, _u32, _P, _u32, C.c_double, C.c_double, _P]),
        "orc_synth_bits": (_u64, [_u64, _u64, _u64]),
        "orc_synth_normal": (C.c_double, [_u64, _u64, _u64]),
        "orc_synth_uniform": (C.c_float, [_u64, _u64, _u64, C.c_float, C.c_float]),
        "orc_synth_normal_f16": (None, [_u64, _u64, _u64, _P]),
        "orc_synth_scaled_normal_f16": (None, [_u64, _u64, _u64, _u32, _P, _P]),
        "orc_synth_normal_f32": (None, [_u64, _u64, _u64, _P]),
        "orc_synth_uniform_f32": (None, [_u64, _u64, _u64, C.c_float, C.c_float, _P]),
        "orc_synth_q8_0": (None, [_u64, _u64, _u64, C.c_float, C.c_float, _P]),
        "orc_synth_q4_1": (None, [_u64, _u64, _u64, C.c_float, C.c_float, C.c_float, C.c_float, _P]),
        "orc_synth_normal_q8_0": (None, [_u64, _u64, _u64, _P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def _load_ref() -> Optional[C.CDLL]:
    path = os.path.join(HERE, "_ref", "libkvmem_ref.so")
    if not os.path.exists(path):
        return None
    lib = C.CDLL(path)
    sig = {
        "ref_last_error": (C.c_char_p, []),
        "ref_recall_fp16": (C.c_int, [C.c_float, _P]),
        "ref_query_score_frame": (C.c_int, [_u64, _u32, _u32, _u32, _u32, _P, _u32, _P, _P, _P, _P]),
        "ref_scores_f16_keys": (C.c_int, [_P, _u32, _u64, _u32, _u32, _u32, _P, _P, _u32, _u32,
                                          C.c_float, C.c_int, _P, _P, _P]),
        "ref_scores_f32_keys": (C.c_int, [_P, _u32, _u64, _u32, _u32, _u32, _P, _P, _u32, _u32,
                                          C.c_float, C.c_int, _P, _P, _P]),
        "ref_scores_from_sums": (C.c_int, [_P, _u32, _u32, _u32, _u32, _u32, _P, _P, _u32, _u32,
                                           C.c_float, C.c_int, _P, _P]),
        "ref_layerwise_scores_f16_keys": (C.c_int, [_P, _u32, _u32, _u64, _u32, _u32, _u32, _P,
                                                    _u32, _u32, C.c_float, _P]),
        "ref_pick_scored_blocks": (C.c_int, [_P, _u32, _P, _u32, _u32, C.c_int, _P, _P]),
        "ref_layerwise_tile_scores_f16_keys": (C.c_int, [_P, _u32, _u32, _u64, _u32, _u32, _u32, _u32, _P, _u32,
                                                         _u32, C.c_float, C.c_int, _P, _P]),
        "ref_query_fixed_blocks": (C.c_int, [_u64, _u32, _u32, _u32, _u32, _P, _u32, _P, _u32, _P, _P]),
        "ref_pick_scored_grouped": (C.c_int, [_P, _u64, _u32, _P, _u32, _P, _u32, _u32, C.c_int, _P, _P]),
        "ref_pick_topk_blocks": (C.c_int, [_P, _u64, _u32, _u32, _u32, _u32, _P, _u32, _P, _u32, _P, _P]),
        "ref_propagate_query_scores": (C.c_int, [_P, _u32, _P, _u32, _u32, _P, _P, _P, _P, _u32, _P, _P, _P,
                                                 C.c_double, C.c_double, _P]),
        "ref_graph_accept": (C.c_int, [_u32, _u64, _u32, _P, _P, _P, _P, _u32, _u32, _u32, _P, _P, _P, _P, _P]),
        "ref_lrfu_preview": (C.c_int, [_P, _u32, _P, _u32, C.c_double, C.c_double, _P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load_oracle()
ref = _load_ref()


def _check(code: int) -> None:
    if code != OK:
        raise OracleError(code)


def _ref_check(code: int) -> None:
    if code != 0:
        raise OracleError(code, ref.ref_last_error().decode())


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# ---- conversions -----------------------------------------------------------

def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32).ravel()
    return np.array([lib.orc_f32_to_f16(float(v)) for v in x], dtype=np.uint16)


def recall_fp16(value: float) -> float:
    out = C.c_float()
    _check(lib.orc_recall_fp16(value, C.byref(out)))
    return out.value


def query_score_frame(accepted: int, block_tokens: int, budget: int, sink: int, recent: int,
                      fixed: Sequence[int] = (), use_ref: bool = False):
    n = lib.orc_page_count(accepted, block_tokens)
    starts = np.zeros(max(n, 1), np.uint64)
    counts = np.zeros(max(n, 1), np.uint32)
    smask = np.zeros(max(n, 1), np.uint8)
    tmask = np.zeros(max(n, 1), np.uint8)
    pins = _c(list(fixed) or [0], np.uint32)
    fn = ref.ref_query_score_frame if use_ref else lib.orc_query_score_frame
    code = fn(accepted, block_tokens, budget, sink, recent, _ptr(pins), len(fixed),
              _ptr(starts), _ptr(counts), _ptr(smask), _ptr(tmask))
    (_ref_check if use_ref else _check)(code)
    return starts[:n], counts[:n], smask[:n], tmask[:n]


# ---- summaries and scores --------------------------------------------------

def row_bytes(fmt: int, width: int) -> int:
    return lib.orc_row_bytes(fmt, width)


def page_summaries(keys: np.ndarray, fmt: int, tokens: int, width: int, page_tokens: int):
    """Per-page (sums, means), float32 [pages][width], for one layer."""
    pages = lib.orc_page_count(tokens, page_tokens)
    sums = np.zeros((pages, width), np.float32)
    means = np.zeros((pages, width), np.float32)
    keys = np.ascontiguousarray(keys)
    _check(lib.orc_page_summaries(_ptr(keys), fmt, tokens, width, page_tokens, _ptr(sums), _ptr(means)))
    return sums, means


def page_softmax_scores(means: np.ndarray, query: np.ndarray, layer_rows: Sequence[int],
                        query_heads: int, kv_heads: int, head_dim: int, aggregation: int,
                        score_mask: Optional[np.ndarray] = None, scale: float = 0.0) -> np.ndarray:
    """means [L][P][Hkv*D] float32; query [L][R][Hq][D] float32 -> double [P]."""
    means = _c(means, np.float32)
    query = _c(query, np.float32)
    layers, pages = means.shape[0], means.shape[1]
    rows = query.shape[1]
    lr = _c(layer_rows, np.uint32)
    out = np.zeros(pages, np.float64)
    mask = None if score_mask is None else _c(score_mask, np.uint8)
    _check(lib.orc_page_softmax_scores(_ptr(means), _ptr(query), _ptr(lr), layers, rows,
                                       query_heads, kv_heads, head_dim, pages, _ptr(mask),
                                       scale, aggregation, _ptr(out)))
    return out


def page_logits(means: np.ndarray, query: np.ndarray, query_heads: int, kv_heads: int,
                head_dim: int, scale: float = 0.0) -> np.ndarray:
    """means [P][Hkv*D]; query [R][Hq][D] -> double [R*Hq][P]."""
    means = _c(means, np.float32)
    query = _c(query, np.float32)
    pages, rows = means.shape[0], query.shape[0]
    out = np.zeros((rows * query_heads, pages), np.float64)
    _check(lib.orc_page_logits(_ptr(means), _ptr(query), rows, query_heads, kv_heads, head_dim,
                               pages, scale, _ptr(out)))
    return out


def pick_scored_blocks(scores: np.ndarray, budget: int, mandatory: Sequence[int] = (),
                       tie_rule: int = TIE_LOWER_FIRST, signed_scores: bool = False) -> np.ndarray:
    scores = _c(scores, np.float64)
    n = scores.shape[0]
    pins = _c(list(mandatory) or [0], np.uint32)
    out = np.zeros(max(n, 1), np.uint32)
    n_out = C.c_uint32()
    _check(lib.orc_pick_scored_blocks(_ptr(scores), n, _ptr(pins), len(mandatory), budget,
                                      tie_rule, int(signed_scores), _ptr(out), C.byref(n_out)))
    return out[: n_out.value].copy()


# ---- half-page layerwise scores ------------------------------------------------

def layerwise_fold(mass: np.ndarray, score_mask: Optional[np.ndarray] = None, keep_halves: bool = False) -> np.ndarray:
    """layerwise_tile_scores' fold of 2*count half masses (left + right), or
    layerwise_max_page_scores (the larger half)."""
    mass = _c(mass, np.float64)
    count = mass.shape[0] // 2
    out = np.zeros(max(count, 1), np.float64)
    mask = None if score_mask is None else _c(score_mask, np.uint8)
    _check(lib.orc_layerwise_fold(_ptr(mass), count, _ptr(mask), int(keep_halves), _ptr(out)))
    return out[:count].copy()


def half_page_scores(keys: np.ndarray, tokens: int, width: int, mean_tokens: int, query: np.ndarray,
                     query_heads: int, kv_heads: int, head_dim: int, keep_halves: bool = False,
                     score_mask: Optional[np.ndarray] = None, scale: float = 0.0) -> np.ndarray:
    """One layer's transport-page scores from Mean-K records every
    mean_tokens tokens: the softmax over every half page, then the fold.
    query [rows][Hq][D] float32."""
    _, means = page_summaries(keys, FMT_F16 if keys.dtype == np.uint16 else FMT_Q8_0, tokens, width, mean_tokens)
    pages = means.shape[0] // 2
    mask2 = None if score_mask is None else np.repeat(np.asarray(score_mask, np.uint8), 2)
    q = np.asarray(query, np.float32)
    mass = page_softmax_scores(means[None], q[None], [q.shape[0]], query_heads, kv_heads, head_dim, AGG_MEAN,
                               mask2, scale)
    return layerwise_fold(mass, score_mask, keep_halves)


def ref_layerwise_tile_scores_f16_keys(keys: np.ndarray, layer: int, tokens: int, kv_heads: int, head_dim: int,
                                       mean_tokens: int, page_tokens: int, query: np.ndarray, query_heads: int,
                                       keep_halves: bool = False, score_mask: Optional[np.ndarray] = None,
                                       scale: float = 0.0) -> np.ndarray:
    keys = _c(keys, np.uint16)
    query = _c(query, np.float32)
    pages = (tokens + page_tokens - 1) // page_tokens
    out = np.zeros(pages, np.float64)
    mask = None if score_mask is None else _c(score_mask, np.uint8)
    _ref_check(ref.ref_layerwise_tile_scores_f16_keys(_ptr(keys), keys.shape[0], layer, tokens, kv_heads, head_dim,
                                                      mean_tokens, page_tokens, _ptr(query), query.shape[0],
                                                      query_heads, scale, int(keep_halves), _ptr(mask), _ptr(out)))
    return out


# ---- page policies (media groups, fixed pages) --------------------------------
# Media ranges are token ranges: a sequence of (first, end) pairs.

def _ranges(ranges) -> np.ndarray:
    return _c(np.asarray(list(ranges) or [(0, 0)], np.uint32).reshape(-1, 2), np.uint32)


def media_group(page: int, pages: int, page_tokens: int, ranges) -> tuple:
    """scored_media_group: the page range [begin, end) kept with `page`."""
    r = _ranges(ranges)
    b, e = C.c_uint32(), C.c_uint32()
    lib.orc_media_group(page, pages, page_tokens, _ptr(r), len(ranges), C.byref(b), C.byref(e))
    return b.value, e.value


def _out(n: int):
    return np.zeros(max(n, 1), np.uint32), C.c_uint32()


def query_fixed_blocks(pages: int, budget: int, sink: int, recent: int, ranges, total_tokens: int,
                       page_tokens: int, mandatory: Sequence[int] = ()) -> np.ndarray:
    r, m = _ranges(ranges), _c(list(mandatory) or [0], np.uint32)
    out, n_out = _out(pages)
    _check(lib.orc_query_fixed_blocks(pages, budget, sink, recent, _ptr(r), len(ranges), total_tokens, page_tokens,
                                      _ptr(m), len(mandatory), _ptr(out), C.byref(n_out)))
    return out[: n_out.value].copy()


def pick_scored_grouped(scores: np.ndarray, budget: int, mandatory: Sequence[int] = (), ranges=(),
                        page_tokens: int = 256, tie_rule: int = TIE_HIGHER_FIRST,
                        signed_scores: bool = False) -> np.ndarray:
    scores = _c(scores, np.float64)
    n = scores.shape[0]
    r, m = _ranges(ranges), _c(list(mandatory) or [0], np.uint32)
    out, n_out = _out(n)
    _check(lib.orc_pick_scored_grouped(_ptr(scores), n, _ptr(m), len(mandatory), budget, tie_rule,
                                       int(signed_scores), _ptr(r), len(ranges), page_tokens, _ptr(out),
                                       C.byref(n_out)))
    return out[: n_out.value].copy()


def pick_topk_ungrouped(scores: np.ndarray, budget: int, sink: int = 0, recent: int = 0,
                        mandatory: Sequence[int] = ()) -> np.ndarray:
    scores = _c(scores, np.float64)
    n = scores.shape[0]
    m = _c(list(mandatory) or [0], np.uint32)
    out, n_out = _out(n)
    _check(lib.orc_pick_topk_ungrouped(_ptr(scores), n, budget, sink, recent, _ptr(m), len(mandatory), _ptr(out),
                                       C.byref(n_out)))
    return out[: n_out.value].copy()


def constrain_media(selected: Sequence[int], scores: np.ndarray, budget: int, sink: int, ranges, total_tokens: int,
                    page_tokens: int, mandatory: Sequence[int] = ()) -> np.ndarray:
    scores = _c(scores, np.float64)
    n = scores.shape[0]
    sel = _c(list(selected) or [0], np.uint32)
    r, m = _ranges(ranges), _c(list(mandatory) or [0], np.uint32)
    out, n_out = _out(n)
    _check(lib.orc_constrain_media(_ptr(sel), len(selected), _ptr(scores), n, budget, sink, _ptr(r), len(ranges),
                                   total_tokens, page_tokens, _ptr(m), len(mandatory), _ptr(out), C.byref(n_out)))
    return out[: n_out.value].copy()


def pick_topk_blocks(scores: np.ndarray, budget: int, sink: int, recent: int, ranges, total_tokens: int,
                     page_tokens: int, mandatory: Sequence[int] = ()) -> np.ndarray:
    """KvMemStore::pick_topk_blocks: the ungrouped pick, then constrain_media."""
    sel = pick_topk_ungrouped(scores, budget, sink, recent, mandatory)
    return constrain_media(sel, scores, budget, sink, ranges, total_tokens, page_tokens, mandatory)


def ref_query_fixed_blocks(total_tokens: int, page_tokens: int, budget: int, sink: int, recent: int, ranges,
                           mandatory: Sequence[int] = ()) -> np.ndarray:
    r, m = _ranges(ranges), _c(list(mandatory) or [0], np.uint32)
    out, n_out = _out(int(-(-total_tokens // page_tokens)))
    _ref_check(ref.ref_query_fixed_blocks(total_tokens, page_tokens, budget, sink, recent, _ptr(r), len(ranges),
                                          _ptr(m), len(mandatory), _ptr(out), C.byref(n_out)))
    return out[: n_out.value].copy()


def ref_pick_scored_grouped(scores: np.ndarray, total_tokens: int, page_tokens: int, ranges, budget: int,
                            mandatory: Sequence[int] = (), signed_scores: bool = False) -> np.ndarray:
    scores = _c(scores, np.float64)
    r, m = _ranges(ranges), _c(list(mandatory) or [0], np.uint32)
    out, n_out = _out(scores.shape[0])
    _ref_check(ref.ref_pick_scored_grouped(_ptr(scores), total_tokens, page_tokens, _ptr(r), len(ranges), _ptr(m),
                                           len(mandatory), budget, int(signed_scores), _ptr(out), C.byref(n_out)))
    return out[: n_out.value].copy()


def ref_pick_topk_blocks(scores: np.ndarray, total_tokens: int, page_tokens: int, budget: int, sink: int,
                         recent: int, ranges, mandatory: Sequence[int] = ()) -> np.ndarray:
    scores = _c(scores, np.float64)
    r, m = _ranges(ranges), _c(list(mandatory) or [0], np.uint32)
    out, n_out = _out(scores.shape[0])
    _ref_check(ref.ref_pick_topk_blocks(_ptr(scores), total_tokens, page_tokens, budget, sink, recent, _ptr(r),
                                        len(ranges), _ptr(m), len(mandatory), _ptr(out), C.byref(n_out)))
    return out[: n_out.value].copy()


# ---- graph propagation and LRFU --------------------------------------------

class PageGraph:
    """A graph flattened by page: row r moves evidence from page
    row_source[r] to pages edge_target[row_begin[r]:row_begin[r+1]] in
    proportion to edge_mass."""

    def __init__(self, rows=()):
        """rows: iterable of (source_page, [(target_page, mass), ...])."""
        rows = list(rows)
        self.row_source = np.array([r[0] for r in rows], np.uint32)
        begin = [0]
        for _, edges in rows:
            begin.append(begin[-1] + len(edges))
        self.row_begin = np.array(begin, np.uint32)
        self.edge_target = np.array([t for _, e in rows for t, _ in e], np.uint32)
        self.edge_mass = np.array([m for _, e in rows for _, m in e], np.float64)

    @classmethod
    def from_arrays(cls, row_source, row_begin, edge_target, edge_mass):
        g = cls()
        g.row_source = _c(row_source, np.uint32)
        g.row_begin = _c(row_begin, np.uint32)
        g.edge_target = _c(edge_target, np.uint32)
        g.edge_mass = _c(edge_mass, np.float64)
        return g

    @property
    def n_rows(self) -> int:
        return int(self.row_source.size)

    @property
    def n_edges(self) -> int:
        return int(self.row_begin[-1])


def span_coefficients(spans, block_tokens: int, pages: int, cross: float = 0.25) -> np.ndarray:
    """spans: [(begin, end, end_known)] message spans -> [pages-1] weights."""
    b = _c([s[0] for s in spans] or [0], np.uint64)
    e = _c([s[1] for s in spans] or [0], np.uint64)
    k = _c([int(s[2]) for s in spans] or [0], np.uint8)
    out = np.ones(max(pages - 1, 1), np.float64)
    _check(lib.orc_span_coefficients(_ptr(b), _ptr(e), _ptr(k), len(spans), block_tokens, pages, cross, _ptr(out)))
    return out[: max(pages - 1, 0)]


def propagate_scores(raw: np.ndarray, graph: Optional[PageGraph] = None, alpha: float = 0.2,
                     mask: Optional[np.ndarray] = None, neighbor_weight: Optional[np.ndarray] = None) -> np.ndarray:
    raw = _c(raw, np.float64)
    n = raw.size
    g = graph or PageGraph()
    m = None if mask is None else _c(mask, np.uint8)
    nw = None if neighbor_weight is None else _c(neighbor_weight, np.float64)
    out = np.zeros(n, np.float64)
    _check(lib.orc_propagate_scores(_ptr(raw), _ptr(m), n, g.n_rows, _ptr(g.row_source), _ptr(g.row_begin),
                                    _ptr(g.edge_target), _ptr(g.edge_mass), _ptr(nw), alpha, _ptr(out)))
    return out


def lrfu_preview(scores: np.ndarray, history: Optional[np.ndarray] = None, lam: float = 0.5,
                 top_fraction: float = 0.9) -> np.ndarray:
    scores = _c(scores, np.float64)
    h = _c(history if history is not None else [0.0], np.float64)
    nh = 0 if history is None else h.size
    out = np.zeros(scores.size, np.float64)
    _check(lib.orc_lrfu_preview(_ptr(scores), scores.size, _ptr(h), nh, lam, top_fraction, _ptr(out)))
    return out


# ---- block formats and gather ---------------------------------------------

def dequant_q8_0(block: np.ndarray) -> np.ndarray:
    block = _c(block, np.uint8)
    y = np.zeros(QK, np.float32)
    lib.orc_dequant_q8_0(_ptr(block), _ptr(y))
    return y


def dequant_q4_1(block: np.ndarray) -> np.ndarray:
    block = _c(block, np.uint8)
    y = np.zeros(QK, np.float32)
    lib.orc_dequant_q4_1(_ptr(block), _ptr(y))
    return y


def dequant_q4_0(block: np.ndarray) -> np.ndarray:
    block = _c(block, np.uint8)
    y = np.zeros(QK, np.float32)
    lib.orc_dequant_q4_0(_ptr(block), _ptr(y))
    return y


def dequant_q5_0(block: np.ndarray) -> np.ndarray:
    block = _c(block, np.uint8)
    y = np.zeros(QK, np.float32)
    lib.orc_dequant_q5_0(_ptr(block), _ptr(y))
    return y


def attention_page_mass(q: np.ndarray, q_fmt: int, q_row_stride: int, q_head_stride: int,
                        k: np.ndarray, k_fmt: int, k_row_stride: int, k_head_stride: int,
                        mask: np.ndarray, mask_fmt: int, mask_row_stride: int, head_dim: int,
                        query_heads: int, kv_heads: int, tokens: int, page_tokens: int,
                        scale: float, softcap: float, rows: Sequence[int]) -> np.ndarray:
    """Masses [len(rows)][pages] (float64).  q, k, mask are the operands' raw
    bytes (uint8 views) with byte strides, as the device entry point takes."""
    q, k, mask = _c(q.view(np.uint8), np.uint8), _c(k.view(np.uint8), np.uint8), _c(mask.view(np.uint8), np.uint8)
    r = _c(np.asarray(rows), np.uint32)
    pages = (tokens + page_tokens - 1) // page_tokens
    out = np.zeros((len(r), pages), np.float64)
    _check(lib.orc_attention_page_mass(_ptr(q), q_fmt, q_row_stride, q_head_stride, _ptr(k), k_fmt,
                                       k_row_stride, k_head_stride, _ptr(mask), mask_fmt, mask_row_stride,
                                       head_dim, query_heads, kv_heads, tokens, page_tokens, scale, softcap,
                                       _ptr(r), len(r), _ptr(out)))
    return out


def quant_q4_0(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.zeros(Q4_0_BYTES, np.uint8)
    lib.orc_quant_q4_0(_ptr(x), _ptr(out))
    return out


def rope_sincos(angle: float):
    s, c = C.c_float(), C.c_float()
    lib.orc_rope_sincos(angle, C.byref(s), C.byref(c))
    return s.value, c.value


def rope_neox_row(row: np.ndarray, head_dim: int, n_rot: int, theta: np.ndarray, pos: float) -> np.ndarray:
    r = np.array(row, np.float32)
    th = _c(theta, np.float32)
    lib.orc_rope_neox_row(_ptr(r), r.size, head_dim, n_rot, _ptr(th), pos)
    return r


def fwht_row(row: np.ndarray, n: int) -> np.ndarray:
    r = np.array(row, np.float32)
    lib.orc_fwht_row(_ptr(r), r.size, n)
    return r


def rope_fwht_rows(rows: np.ndarray, fmt: int, width: int, n: int, pos0: int, head_dim: int, n_rot: int,
                   theta: np.ndarray, fwht: int) -> np.ndarray:
    rows = _c(rows, np.uint8)
    th = _c(theta if theta is not None else np.zeros(1), np.float32)
    out = np.zeros_like(rows)
    _check(lib.orc_rope_fwht_rows(_ptr(rows), fmt, width, n, pos0, head_dim, n_rot, _ptr(th), fwht, _ptr(out)))
    return out


VAR_UNFUSED_ROT, VAR_UNFUSED_Q4, VAR_SIN_UP, VAR_SIN_DOWN, VAR_COS_UP, VAR_COS_DOWN, VAR_RNE = \
    1, 2, 4, 8, 16, 32, 64


def rope_fwht_rows_variant(rows: np.ndarray, fmt: int, width: int, n: int, pos0: int, head_dim: int, n_rot: int,
                           theta: np.ndarray, fwht: int, variant: int) -> np.ndarray:
    """The transform with other floating-point choices (VAR_* bits), for
    sensitivity tests: unfused rotation or q4_0 multiply-add, sin/cos one ulp
    off, ties to even in the requantizers."""
    rows = _c(rows, np.uint8)
    th = _c(theta if theta is not None else np.zeros(1), np.float32)
    out = np.zeros_like(rows)
    _check(lib.orc_rope_fwht_rows_variant(_ptr(rows), fmt, width, n, pos0, head_dim, n_rot, _ptr(th), fwht,
                                          variant, _ptr(out)))
    return out


def gather_rope(history: np.ndarray, fmt: int, width: int, tokens: int, page_tokens: int,
                selected: Sequence[int], head_dim: int, n_rot: int, theta: np.ndarray, fwht: int,
                pos_base: int = 0, slots: Optional[np.ndarray] = None) -> np.ndarray:
    """Slots [k][page_tokens][row] of the raw-K transform gather; rows past a
    partial last page keep `slots`' bytes (zero by default)."""
    h = _c(history, np.uint8)
    sel = _c(np.asarray(selected), np.uint32)
    th = _c(theta if theta is not None else np.zeros(1), np.float32)
    row = width // QK * (Q8_0_BYTES if fmt == FMT_Q8_0 else Q4_0_BYTES)
    out = np.zeros(len(sel) * page_tokens * row, np.uint8) if slots is None else np.array(slots, np.uint8)
    _check(lib.orc_gather_rope(_ptr(h), fmt, width, tokens, page_tokens, _ptr(sel), len(sel), head_dim, n_rot,
                               _ptr(th), fwht, pos_base, _ptr(out)))
    return out


def quant_q8_0(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.zeros(Q8_0_BYTES, np.uint8)
    lib.orc_quant_q8_0(_ptr(x), _ptr(out))
    return out


def gather_row_bytes(src_fmt: int, mode: int, width: int) -> int:
    return lib.orc_gather_row_bytes(src_fmt, mode, width)


def gather(history: np.ndarray, src_fmt: int, width: int, tokens: int, page_tokens: int,
           selected: Sequence[int], mode: int, slots: Optional[np.ndarray] = None) -> np.ndarray:
    history = np.ascontiguousarray(history).view(np.uint8)
    sel = _c(list(selected) or [0], np.uint32)
    drow = gather_row_bytes(src_fmt, mode, width)
    if slots is None:
        slots = np.zeros(max(len(selected), 1) * page_tokens * drow, np.uint8)
    _check(lib.orc_gather(_ptr(history), src_fmt, width, tokens, page_tokens, _ptr(sel),
                          len(selected), mode, _ptr(slots)))
    return slots


# ---- synthetic inputs ------------------------------------------------------

def synth_normal_f16(seed: int, stream: int, count: int) -> np.ndarray:
    out = np.zeros(count, np.uint16)
    lib.orc_synth_normal_f16(seed, stream, count, _ptr(out))
    return out


def synth_scaled_normal_f16(seed: int, stream: int, rows: int, scale: np.ndarray) -> np.ndarray:
    scale = _c(scale, np.float32)
    out = np.zeros(rows * scale.shape[0], np.uint16)
    lib.orc_synth_scaled_normal_f16(seed, stream, rows, scale.shape[0], _ptr(scale), _ptr(out))
    return out


def synth_normal_f32(seed: int, stream: int, count: int) -> np.ndarray:
    out = np.zeros(count, np.float32)
    lib.orc_synth_normal_f32(seed, stream, count, _ptr(out))
    return out


def synth_uniform_f32(seed: int, stream: int, count: int, lo: float, hi: float) -> np.ndarray:
    out = np.zeros(count, np.float32)
    lib.orc_synth_uniform_f32(seed, stream, count, lo, hi, _ptr(out))
    return out


def synth_q8_0(seed: int, stream: int, blocks: int, d_lo: float, d_hi: float) -> np.ndarray:
    out = np.zeros(blocks * Q8_0_BYTES, np.uint8)
    lib.orc_synth_q8_0(seed, stream, blocks, d_lo, d_hi, _ptr(out))
    return out


def synth_q4_1(seed: int, stream: int, blocks: int, d_lo: float, d_hi: float, m_lo: float,
               m_hi: float) -> np.ndarray:
    out = np.zeros(blocks * Q4_1_BYTES, np.uint8)
    lib.orc_synth_q4_1(seed, stream, blocks, d_lo, d_hi, m_lo, m_hi, _ptr(out))
    return out


def synth_normal_q8_0(seed: int, stream: int, blocks: int) -> np.ndarray:
    out = np.zeros(blocks * Q8_0_BYTES, np.uint8)
    lib.orc_synth_normal_q8_0(seed, stream, blocks, _ptr(out))
    return out


# ---- reference build (oracle/_ref) -----------------------------------------

def ref_available() -> bool:
    return ref is not None


def ref_recall_fp16(value: float) -> float:
    out = C.c_float()
    _ref_check(ref.ref_recall_fp16(value, C.byref(out)))
    return out.value


def ref_scores_f16_keys(keys: np.ndarray, tokens: int, kv_heads: int, head_dim: int,
                        page_tokens: int, query: np.ndarray, layer_rows: Sequence[int],
                        query_heads: int, aggregation: int, scale: float = 0.0,
                        score_mask: Optional[np.ndarray] = None, want_scores: bool = True):
    """keys uint16 [L][T][Hkv*D]; query [L][R][Hq][D] -> (means [L][P][W], scores [P])."""
    keys = _c(keys, np.uint16)
    query = _c(query, np.float32)
    layers, rows = keys.shape[0], query.shape[1]
    width = kv_heads * head_dim
    pages = (tokens + page_tokens - 1) // page_tokens
    means = np.zeros((layers, pages, width), np.float32)
    scores = np.zeros(pages, np.float64)
    lr = _c(layer_rows, np.uint32)
    mask = None if score_mask is None else _c(score_mask, np.uint8)
    _ref_check(ref.ref_scores_f16_keys(_ptr(keys), layers, tokens, kv_heads, head_dim, page_tokens,
                                       _ptr(query), _ptr(lr), rows, query_heads, scale, aggregation,
                                       _ptr(mask), _ptr(means), _ptr(scores) if want_scores else None))
    return means, scores


def ref_scores_f32_keys(keys: np.ndarray, tokens: int, kv_heads: int, head_dim: int,
                        page_tokens: int, query: np.ndarray, layer_rows: Sequence[int],
                        query_heads: int, aggregation: int, scale: float = 0.0):
    keys = _c(keys, np.float32)
    query = _c(query, np.float32)
    layers, rows = keys.shape[0], query.shape[1]
    width = kv_heads * head_dim
    pages = (tokens + page_tokens - 1) // page_tokens
    means = np.zeros((layers, pages, width), np.float32)
    scores = np.zeros(pages, np.float64)
    lr = _c(layer_rows, np.uint32)
    _ref_check(ref.ref_scores_f32_keys(_ptr(keys), layers, tokens, kv_heads, head_dim, page_tokens,
                                       _ptr(query), _ptr(lr), rows, query_heads, scale, aggregation,
                                       None, _ptr(means), _ptr(scores)))
    return means, scores


def ref_scores_from_sums(sums: np.ndarray, kv_heads: int, head_dim: int, page_tokens: int,
                         query: np.ndarray, layer_rows: Sequence[int], query_heads: int,
                         aggregation: int, scale: float = 0.0,
                         score_mask: Optional[np.ndarray] = None) -> np.ndarray:
    sums = _c(sums, np.float32)
    query = _c(query, np.float32)
    layers, pages = sums.shape[0], sums.shape[1]
    rows = query.shape[1]
    scores = np.zeros(pages, np.float64)
    lr = _c(layer_rows, np.uint32)
    mask = None if score_mask is None else _c(score_mask, np.uint8)
    _ref_check(ref.ref_scores_from_sums(_ptr(sums), layers, pages, kv_heads, head_dim, page_tokens,
                                        _ptr(query), _ptr(lr), rows, query_heads, scale,
                                        aggregation, _ptr(mask), _ptr(scores)))
    return scores


def ref_layerwise_scores_f16_keys(keys: np.ndarray, layer: int, tokens: int, kv_heads: int,
                                  head_dim: int, page_tokens: int, query: np.ndarray,
                                  query_heads: int, scale: float = 0.0) -> np.ndarray:
    keys = _c(keys, np.uint16)
    query = _c(query, np.float32)
    pages = (tokens + page_tokens - 1) // page_tokens
    scores = np.zeros(pages, np.float64)
    _ref_check(ref.ref_layerwise_scores_f16_keys(_ptr(keys), keys.shape[0], layer, tokens, kv_heads,
                                                 head_dim, page_tokens, _ptr(query), query.shape[0],
                                                 query_heads, scale, _ptr(scores)))
    return scores


def ref_pick_scored_blocks(scores: np.ndarray, budget: int, mandatory: Sequence[int] = (),
                           signed_scores: bool = False) -> np.ndarray:
    scores = _c(scores, np.float64)
    n = scores.shape[0]
    pins = _c(list(mandatory) or [0], np.uint32)
    out = np.zeros(max(n, 1), np.uint32)
    n_out = C.c_uint32()
    _ref_check(ref.ref_pick_scored_blocks(_ptr(scores), n, _ptr(pins), len(mandatory), budget,
                                          int(signed_scores), _ptr(out), C.byref(n_out)))
    return out[: n_out.value].copy()


def ref_propagate_query_scores(raw: np.ndarray, graph: Optional[PageGraph] = None, alpha: float = 0.2,
                               mask: Optional[np.ndarray] = None, block_tokens: int = 64, spans=None,
                               cross: float = 0.25) -> np.ndarray:
    """The reference's propagate_query_scores on a page-indexed frame and
    graph (spans None: no message spans)."""
    raw = _c(raw, np.float64)
    n = raw.size
    g = graph or PageGraph()
    m = None if mask is None else _c(mask, np.uint8)
    sp = spans or []
    b = _c([s[0] for s in sp] or [0], np.uint64)
    e = _c([s[1] for s in sp] or [0], np.uint64)
    k = _c([int(s[2]) for s in sp] or [0], np.uint8)
    out = np.zeros(n, np.float64)
    _ref_check(ref.ref_propagate_query_scores(_ptr(raw), n, _ptr(m), block_tokens, g.n_rows, _ptr(g.row_source),
                                              _ptr(g.row_begin), _ptr(g.edge_target), _ptr(g.edge_mass),
                                              0xFFFFFFFF if spans is None else len(sp), _ptr(b), _ptr(e), _ptr(k),
                                              alpha, cross, _ptr(out)))
    return out


def ref_graph_accept(block_tokens: int, end: int, samples, topk: int = 4) -> PageGraph:
    """samples: [(source_position, [(target_token_position, mass), ...])] ->
    the rows propagation reads after one prepare_graph_accept over [0, end)."""
    pos = _c([s[0] for s in samples] or [0], np.uint64)
    begin = [0]
    for _, mass in samples:
        begin.append(begin[-1] + len(mass))
    sb = _c(begin, np.uint32)
    tg = _c([t for _, ms in samples for t, _ in ms] or [0], np.uint64)
    ma = _c([w for _, ms in samples for _, w in ms] or [0], np.float64)
    max_rows = end // block_tokens + 1
    max_edges = max_rows * topk
    rs = np.zeros(max_rows, np.uint32)
    rb = np.zeros(max_rows + 1, np.uint32)
    et = np.zeros(max(max_edges, 1), np.uint32)
    em = np.zeros(max(max_edges, 1), np.float64)
    nr = C.c_uint32()
    _ref_check(ref.ref_graph_accept(block_tokens, end, len(samples), _ptr(pos), _ptr(sb), _ptr(tg), _ptr(ma), topk,
                                    max_rows, max_edges, C.byref(nr), _ptr(rs), _ptr(rb), _ptr(et), _ptr(em)))
    r = nr.value
    ne = int(rb[r])
    return PageGraph.from_arrays(rs[:r], rb[:r + 1], et[:ne], em[:ne])


def ref_lrfu_preview(scores: np.ndarray, history: Optional[np.ndarray] = None, lam: float = 0.5,
                     top_fraction: float = 0.9) -> np.ndarray:
    scores = _c(scores, np.float64)
    h = _c(history if history is not None else [0.0], np.float64)
    nh = 0 if history is None else h.size
    out = np.zeros(scores.size, np.float64)
    _ref_check(ref.ref_lrfu_preview(_ptr(h), nh, _ptr(scores), scores.size, lam, top_fraction, _ptr(out)))
    return out
