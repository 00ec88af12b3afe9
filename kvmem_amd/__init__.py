"""kvmem_amd -- MI355X-native KVMem recall hot path.

The product is the C ABI in include/kvrecall.h, implemented by the in-tree
libkvrecall.so (HIP kernels for gfx950).  This module is a thin Python view
of that ABI used by tests and the benchmark: device buffers are torch CUDA
tensors (plumbing only), pinned host history is allocated by the library.
Every call goes through the native library; if it is missing or fails to
load, calls raise.
"""
from __future__ import annotations

import ctypes as C
import math
from typing import Optional, Sequence

import numpy as np

from . import _capi
from ._capi import (AGG_MAX, AGG_MAX_LOGIT, AGG_MEAN, ENGINE_AUTO, ENGINE_KERNEL, ENGINE_SDMA,
                    FMT_BF16, FMT_F16, FMT_F32, FMT_Q4_0, FMT_Q4_1, FMT_Q5_0, FMT_Q8_0, GATHER_COPY,
                    GATHER_DEQUANT_F16, GATHER_REQUANT_Q8_0, GATHER_ROPE_FWHT, TIE_HIGHER_FIRST,
                    TIE_LOWER_FIRST, KvrError, check, lib)

__all__ = [
    "Context", "PinnedBuffer", "KvrError", "row_bytes", "gather_row_bytes",
    "AGG_MEAN", "AGG_MAX", "AGG_MAX_LOGIT", "TIE_LOWER_FIRST", "TIE_HIGHER_FIRST",
    "FMT_F16", "FMT_Q8_0", "FMT_Q4_1", "FMT_F32", "FMT_BF16", "FMT_Q4_0", "FMT_Q5_0",
    "GATHER_COPY", "GATHER_DEQUANT_F16", "GATHER_REQUANT_Q8_0", "GATHER_ROPE_FWHT",
    "ENGINE_AUTO", "ENGINE_KERNEL", "ENGINE_SDMA",
]

_SCALAR_BYTES = {FMT_F32: 4, FMT_F16: 2, FMT_BF16: 2}


def row_bytes(fmt: int, width: int) -> int:
    if fmt == FMT_F16:
        return width * 2
    if fmt == FMT_Q8_0:
        return width // 32 * 34
    if fmt == FMT_Q4_1:
        return width // 32 * 20
    if fmt == FMT_Q4_0:
        return width // 32 * 18
    raise ValueError(f"no row format {fmt}")


def gather_row_bytes(fmt: int, mode: int, width: int) -> int:
    if mode == GATHER_DEQUANT_F16:
        return width * 2
    return row_bytes(fmt, width)


def _ptr(t) -> Optional[int]:
    if t is None:
        return None
    if isinstance(t, int):
        return t
    if isinstance(t, PinnedBuffer):
        return t.ptr
    return t.data_ptr()


class PinnedBuffer:
    """Page-locked, device-mapped host memory from kvr_host_alloc."""

    def __init__(self, nbytes: int):
        p = C.c_void_p()
        check(lib().kvr_host_alloc(nbytes, C.byref(p)))
        self.ptr = p.value
        self.nbytes = nbytes

    def numpy(self, dtype=np.uint8) -> np.ndarray:
        buf = (C.c_uint8 * self.nbytes).from_address(self.ptr)
        return np.frombuffer(buf, dtype=np.uint8).view(dtype)

    def free(self) -> None:
        if self.ptr:
            check(lib().kvr_host_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def make_query(t, scalar: int, rows: int, query_heads: int, kv_heads: int, head_dim: int,
               lanes: int = 1, attention_scale: float = 0.0, strides: Optional[Sequence[int]] = None):
    """Query descriptor; `strides` = (row, head, dim, lane) in elements, default dense
    [lanes][rows][query_heads][head_dim]."""
    el = _SCALAR_BYTES[scalar]
    if strides is None:
        strides = (query_heads * head_dim, head_dim, 1, rows * query_heads * head_dim)
    q = _capi.Query()
    q.data = _ptr(t)
    q.scalar = scalar
    q.rows, q.query_heads, q.kv_heads, q.head_dim = rows, query_heads, kv_heads, head_dim
    q.row_stride, q.head_stride, q.dim_stride, q.lane_stride = (s * el for s in strides)
    q.attention_scale = attention_scale
    q._keep = t  # the device buffer lives as long as the descriptor
    return q


def make_keys(t, fmt: int, tokens: int, kv_heads: int, head_dim: int, page_tokens: int,
              lanes: int = 1, lane_stride: int = 0):
    k = _capi.KeyHistory()
    k.data = _ptr(t)
    k.format = fmt
    k.tokens, k.kv_heads, k.head_dim, k.page_tokens = tokens, kv_heads, head_dim, page_tokens
    k.lanes, k.lane_stride = lanes, lane_stride
    k._keep = t
    return k


def make_page_graph(n_rows=0, n_edges=0, row_source=None, row_begin=None, edge_target=None, edge_mass=None,
                    neighbor_weight=None) -> "_capi.PageGraph":
    """A kvr_page_graph over device arrays (the caller keeps them alive)."""
    return _capi.PageGraph(n_rows, n_edges, _ptr(row_source), _ptr(row_begin), _ptr(edge_target),
                           _ptr(edge_mass), _ptr(neighbor_weight))


def make_plane(history, fmt: int, width: int, tokens: int, mode: int, slots,
               host_lane_stride: int = 0, slot_lane_stride: int = 0, rope: Optional[dict] = None,
               history_offset: int = 0, page_stride: int = 0):
    """rope (for GATHER_ROPE_FWHT): dict(head_dim, n_rot, theta (device
    float32 tensor of n_rot/2 values), fwht, pos_base).  Record sources:
    history_offset = the plane's offset in a record, page_stride = the
    record size."""
    p = _capi.Plane()
    p.history = _ptr(history) + history_offset
    p.page_stride = page_stride
    p.format, p.width, p.tokens, p.mode = fmt, width, tokens, mode
    p.slots = _ptr(slots)
    p.host_lane_stride, p.slot_lane_stride = host_lane_stride, slot_lane_stride
    keep = [history, slots]
    if rope is not None:
        r = _capi.Rope(rope["head_dim"], rope.get("n_rot", 0), _ptr(rope.get("theta")), rope.get("fwht", 0),
                       rope.get("pos_base", 0))
        p.rope = C.pointer(r)
        keep += [r, rope.get("theta")]
    p._keep = tuple(keep)
    return p


# ---- page policies (host helpers of include/kvrecall.h, no device work) ----

def _media(ranges, page_tokens: int, total_tokens: int):
    arr = np.ascontiguousarray(np.asarray(list(ranges) or [(0, 0)], np.uint32).reshape(-1, 2))
    m = _capi.Media(arr.ctypes.data, len(ranges), page_tokens, total_tokens)
    m._keep = arr
    return m


def _u32_arr(values):
    return (C.c_uint32 * max(1, len(values)))(*values)


def media_page_groups(ranges, page_tokens: int, total_tokens: int, pages: int, merge: int = 0) -> np.ndarray:
    """kvr_media_page_groups: disjoint ascending [begin, end) page ranges,
    shape [n][2] (merge 0: ranges sharing a page join; 1: in list order)."""
    m = _media(ranges, page_tokens, total_tokens)
    out = (C.c_uint32 * max(2, 2 * len(ranges)))()
    n = C.c_uint32()
    check(lib().kvr_media_page_groups(C.byref(m), pages, merge, out, C.byref(n)))
    return np.frombuffer(out, np.uint32)[: 2 * n.value].reshape(-1, 2).copy()


def query_fixed_pages(pages: int, budget: int, sink: int, recent: int, ranges=(), page_tokens: int = 256,
                      total_tokens: int = 0, mandatory: Sequence[int] = ()) -> np.ndarray:
    """kvr_query_fixed_pages (KvMemStore::query_fixed_blocks)."""
    m = _media(ranges, page_tokens, total_tokens)
    out = (C.c_uint32 * max(1, pages))()
    n = C.c_uint32()
    check(lib().kvr_query_fixed_pages(pages, budget, sink, recent, C.byref(m), _u32_arr(mandatory), len(mandatory),
                                      out, C.byref(n)))
    return np.frombuffer(out, np.uint32)[: n.value].copy()


def topk_fixed_pages(pages: int, budget: int, sink: int, recent: int, mandatory: Sequence[int] = ()) -> np.ndarray:
    """kvr_topk_fixed_pages (the kept part of pick_topk_ungrouped)."""
    out = (C.c_uint32 * max(1, pages))()
    n = C.c_uint32()
    check(lib().kvr_topk_fixed_pages(pages, budget, sink, recent, _u32_arr(mandatory), len(mandatory), out,
                                     C.byref(n)))
    return np.frombuffer(out, np.uint32)[: n.value].copy()


def media_fixed_pages(pages: int, budget: int, sink: int, ranges, page_tokens: int, total_tokens: int,
                      mandatory: Sequence[int] = ()) -> np.ndarray:
    """kvr_media_fixed_pages (the kept part of constrain_media)."""
    m = _media(ranges, page_tokens, total_tokens)
    out = (C.c_uint32 * max(1, pages))()
    n = C.c_uint32()
    check(lib().kvr_media_fixed_pages(pages, budget, sink, C.byref(m), _u32_arr(mandatory), len(mandatory), out,
                                      C.byref(n)))
    return np.frombuffer(out, np.uint32)[: n.value].copy()


def make_policy(fixed=None, n_fixed: int = 0, groups=None, n_groups: int = 0, preferred=None,
                preferred_count=None, preferred_stride: int = 0) -> "_capi.PagePolicy":
    """A kvr_page_policy over device arrays (the descriptor keeps them alive)."""
    p = _capi.PagePolicy(_ptr(fixed), n_fixed, _ptr(groups), n_groups, _ptr(preferred), _ptr(preferred_count),
                         preferred_stride)
    p._keep = (fixed, groups, preferred, preferred_count)
    return p


class Context:
    """One kvr_context: a GPU, two streams, a workspace."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        check(lib().kvr_create(device, C.byref(h)))
        self.handle = h.value
        self.device = device

    def close(self) -> None:
        if self.handle:
            check(lib().kvr_destroy(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- streams / status ---------------------------------------------------
    @property
    def select_stream(self) -> int:
        return lib().kvr_select_stream(self.handle)

    @property
    def copy_stream(self) -> int:
        return lib().kvr_copy_stream(self.handle)

    def check(self, stream: Optional[int] = None) -> None:
        check(lib().kvr_check(self.handle, stream))

    def status(self, stream: Optional[int] = None) -> int:
        return lib().kvr_check(self.handle, stream)

    def set_option(self, option: int, value: int) -> None:
        check(lib().kvr_set_option(self.handle, option, value))

    # -- workspace ----------------------------------------------------------
    @staticmethod
    def workspace_bytes(lanes, pages, rows, query_heads, kv_heads, head_dim) -> int:
        return lib().kvr_workspace_bytes(lanes, pages, rows, query_heads, kv_heads, head_dim)

    def bind_workspace(self, t, nbytes: int) -> None:
        check(lib().kvr_bind_workspace(self.handle, _ptr(t), nbytes))

    def device_bytes(self) -> int:
        return lib().kvr_device_bytes(self.handle)

    # -- summaries ----------------------------------------------------------
    def summary_build(self, keys, means=None, summaries=None, stream=None) -> None:
        check(lib().kvr_summary_build(self.handle, C.byref(keys), _ptr(means), _ptr(summaries), stream))

    def summary_accumulate(self, sums, counts, page_tokens, k, scalar, pos0, n, kv_heads, head_dim,
                           strides_el: Sequence[int], stream=None) -> None:
        el = _SCALAR_BYTES[scalar]
        ts, hs, ds = (s * el for s in strides_el)
        check(lib().kvr_summary_accumulate(self.handle, _ptr(sums), _ptr(counts), page_tokens, _ptr(k),
                                           scalar, pos0, n, kv_heads, head_dim, ts, hs, ds, stream))

    def summary_finalize(self, sums, counts, pages, width, means=None, summaries=None, stream=None) -> None:
        check(lib().kvr_summary_finalize(self.handle, _ptr(sums), _ptr(counts), pages, width, _ptr(means),
                                         _ptr(summaries), stream))

    # -- scoring / selection ----------------------------------------------
    def score(self, query, summaries, pages, scores, aggregation=AGG_MEAN, lanes=1, score_mask=None,
              active_layers=1, accumulate=False, force_mfma=0, stream=None) -> None:
        check(lib().kvr_score(self.handle, C.byref(query), _ptr(summaries), lanes, pages, _ptr(score_mask),
                              aggregation, active_layers, int(accumulate), _ptr(scores), force_mfma, stream))

    def select_topk(self, scores, pages, k, selected, count, lanes=1, mandatory: Sequence[int] = (),
                    tie_rule=TIE_LOWER_FIRST, signed_scores=False, stream=None) -> None:
        arr = (C.c_uint32 * max(1, len(mandatory)))(*mandatory)
        check(lib().kvr_select_topk(self.handle, _ptr(scores), lanes, pages, k, arr, len(mandatory), tie_rule,
                                    int(signed_scores), _ptr(selected), _ptr(count), stream))

    def fold_half_pages(self, halves, pages, scores, rule, lanes=1, score_mask=None, stream=None) -> None:
        """kvr_fold_half_pages: [lanes][2*pages] half masses -> [lanes][pages]."""
        check(lib().kvr_fold_half_pages(self.handle, _ptr(halves), lanes, pages, _ptr(score_mask), rule,
                                        _ptr(scores), stream))

    def select_pages(self, scores, pages, k, selected, count, policy=None, lanes=1, tie_rule=TIE_LOWER_FIRST,
                     signed_scores=False, stream=None) -> None:
        """kvr_select_pages with a make_policy() descriptor (or None)."""
        check(lib().kvr_select_pages(self.handle, _ptr(scores), lanes, pages, k,
                                     None if policy is None else C.byref(policy), tie_rule, int(signed_scores),
                                     _ptr(selected), _ptr(count), stream))

    # -- graph propagation and LRFU -------------------------------------------
    def propagate_scores(self, scores, pages, graphs: Sequence = (), alpha=0.2, transport_mask=None, lanes=1,
                         stream=None) -> None:
        """graphs: one _capi.PageGraph per lane (make_page_graph), or none."""
        arr = (_capi.PageGraph * max(1, len(graphs)))(*graphs) if graphs else None
        check(lib().kvr_propagate_scores(self.handle, _ptr(scores), lanes, pages, _ptr(transport_mask), arr,
                                         alpha, stream))

    def lrfu_preview(self, scores, pages, candidate, history=None, history_pages=0, lam=0.5, top_fraction=0.9,
                     lanes=1, stream=None) -> None:
        check(lib().kvr_lrfu_preview(self.handle, _ptr(scores), lanes, pages, _ptr(history), history_pages, lam,
                                     top_fraction, _ptr(candidate), stream))

    def propagate_lrfu(self, scores, pages, candidate, graphs: Sequence = (), alpha=0.2, transport_mask=None,
                       history=None, history_pages=0, lam=0.5, top_fraction=0.9, lanes=1, stream=None) -> None:
        arr = (_capi.PageGraph * max(1, len(graphs)))(*graphs) if graphs else None
        check(lib().kvr_propagate_lrfu(self.handle, _ptr(scores), lanes, pages, _ptr(transport_mask), arr, alpha,
                                       _ptr(history), history_pages, lam, top_fraction, _ptr(candidate), stream))

    # -- stage-in -----------------------------------------------------------
    def stage_in(self, planes: Sequence, page_tokens, selected, count, k, lanes=1, engine=ENGINE_AUTO,
                 stream=None) -> None:
        arr = (_capi.Plane * max(1, len(planes)))(*planes)
        check(lib().kvr_stage_in(self.handle, arr, len(planes), lanes, page_tokens, _ptr(selected),
                                 _ptr(count), k, engine, stream))

    @staticmethod
    def layer_recall(*, query, summaries, scores, selected, count, k, keys=None, means=None,
                     pages=0, page_tokens=0, lanes=0, score_mask=None, aggregation=AGG_MEAN,
                     tie_rule=TIE_LOWER_FIRST, mandatory: Sequence[int] = (), planes: Sequence = (),
                     engine=ENGINE_AUTO, force_mfma=0, summary_events=(None, None),
                     select_end=None, policy=None, half_fold=0) -> "_capi.LayerRecall":
        """A kvr_layer_recall descriptor (holding what it points to), for
        callers that issue the same layer many times."""
        d = _capi.LayerRecall()
        if keys is not None:
            d.keys = C.pointer(keys)
        d.summaries, d.means = _ptr(summaries), _ptr(means)
        d.pages, d.page_tokens, d.lanes = pages, page_tokens, lanes
        d.query = C.pointer(query)
        d.score_mask = _ptr(score_mask)
        d.aggregation, d.k, d.tie_rule = aggregation, k, tie_rule
        mand = (C.c_uint32 * max(1, len(mandatory)))(*mandatory)
        d.mandatory, d.n_mandatory = mand, len(mandatory)
        d.scores, d.selected, d.count = _ptr(scores), _ptr(selected), _ptr(count)
        parr = (_capi.Plane * max(1, len(planes)))(*planes)
        d.planes, d.n_planes = parr, len(planes)
        d.engine, d.force_mfma = engine, force_mfma
        d.summary_begin, d.summary_end = summary_events
        d.select_end = select_end
        if policy is not None:
            d.policy = C.pointer(policy)
        d.half_fold = half_fold
        d._keep = (keys, query, summaries, means, score_mask, scores, selected, count, mand, parr, list(planes),
                   policy)
        return d

    def recall(self, desc, select_stream=None, copy_stream=None) -> None:
        """kvr_recall_layer on a prebuilt descriptor."""
        check(lib().kvr_recall_layer(self.handle, C.byref(desc), select_stream, copy_stream))

    def recall_noalloc(self, desc, select_stream=None, copy_stream=None) -> None:
        """kvr_recall_layer_noalloc on a prebuilt descriptor: the same layer
        with its logits and counters in the library's static device scratch."""
        check(lib().kvr_recall_layer_noalloc(self.handle, C.byref(desc), select_stream, copy_stream))

    def recall_layer(self, *, select_stream=None, copy_stream=None, **kw) -> None:
        self.recall(self.layer_recall(**kw), select_stream, copy_stream)

    def recall_stack(self, descs: Sequence, select_stream=None, copy_stream=None):
        """kvr_recall_stack over prebuilt descriptors (Context.layer_recall).
        Returns the descriptor array, which the caller keeps until the work
        has run."""
        arr = (_capi.LayerRecall * len(descs))(*descs)
        arr._keep = list(descs)
        check(lib().kvr_recall_stack(self.handle, arr, len(descs), select_stream, copy_stream))
        return arr

    def attention_page_mass(self, *, q, q_format: int, q_row_stride: int, q_head_stride: int, k, k_format: int,
                            k_row_stride: int, k_head_stride: int, mask, mask_format: int, mask_row_stride: int,
                            head_dim: int, query_heads: int, kv_heads: int, tokens: int, page_tokens: int,
                            scale: float, softcap: float, rows: Sequence[int], mass, stream=None,
                            mask_rows: Optional[Sequence[int]] = None) -> None:
        """kvr_attention_page_mass: device tensors (or addresses) with byte
        strides; `mass` is float32 [len(rows)][pages] on the device."""
        r = (C.c_uint32 * max(1, len(rows)))(*rows)
        mr = None if mask_rows is None else (C.c_uint32 * max(1, len(mask_rows)))(*mask_rows)
        a = _capi.AttentionSample(_ptr(q), q_format, q_row_stride, q_head_stride, _ptr(k), k_format, k_row_stride,
                                  k_head_stride, _ptr(mask), mask_format, mask_row_stride, head_dim, query_heads,
                                  kv_heads, tokens, page_tokens, scale, softcap,
                                  C.cast(r, C.POINTER(C.c_uint32)), len(rows),
                                  None if mr is None else C.cast(mr, C.POINTER(C.c_uint32)))
        check(lib().kvr_attention_page_mass(self.handle, C.byref(a), _ptr(mass), stream))

    @staticmethod
    def attention_workspace_bytes(n_rows: int, query_heads: int, pages: int) -> int:
        return lib().kvr_attention_workspace_bytes(n_rows, query_heads, pages)

    def d2d_batched(self, srcs: Sequence[int], dsts: Sequence[int], sizes: Sequence[int], stream=None) -> None:
        n = len(srcs)
        s = (C.c_void_p * max(1, n))(*srcs)
        d = (C.c_void_p * max(1, n))(*dsts)
        z = (C.c_size_t * max(1, n))(*sizes)
        check(lib().kvr_d2d_batched(self.handle, s, d, z, n, stream))

    # -- measurement / synthetic inputs ----------------------------------
    def h2d_peak_gbps(self, nbytes: int = 1 << 30, reps: int = 5) -> float:
        out = C.c_double()
        check(lib().kvr_h2d_peak_gbps(self.handle, nbytes, reps, C.byref(out)))
        return out.value

    def h2d_read_peak_gbps(self, nbytes: int = 1 << 30, reps: int = 5) -> float:
        """A kernel's zero-copy read rate of pinned host memory (GB/s)."""
        out = C.c_double()
        check(lib().kvr_h2d_read_peak_gbps(self.handle, nbytes, reps, C.byref(out)))
        return out.value

    def h2d_ceiling_gbps(self, nbytes: int = 1 << 30, reps: int = 5) -> dict:
        """Both host-link probes; the ceiling is the larger."""
        copy, read = self.h2d_peak_gbps(nbytes, reps), self.h2d_read_peak_gbps(nbytes, reps)
        return {"copy_GBps": round(copy, 3), "kernel_read_GBps": round(read, 3), "ceiling_GBps": round(max(copy, read), 3)}

    def synth_normal_f16(self, seed, sid, count, out, stream=None):
        check(lib().kvr_synth_normal_f16(self.handle, seed, sid, count, _ptr(out), stream))

    def synth_scaled_normal_f16(self, seed, sid, rows, width, scale, out, stream=None):
        check(lib().kvr_synth_scaled_normal_f16(self.handle, seed, sid, rows, width, _ptr(scale), _ptr(out),
                                                stream))

    def synth_normal_f32(self, seed, sid, count, out, stream=None):
        check(lib().kvr_synth_normal_f32(self.handle, seed, sid, count, _ptr(out), stream))

    def synth_q8_0(self, seed, sid, blocks, d_lo, d_hi, out, stream=None):
        check(lib().kvr_synth_q8_0(self.handle, seed, sid, blocks, d_lo, d_hi, _ptr(out), stream))

    def synth_q4_1(self, seed, sid, blocks, d_lo, d_hi, m_lo, m_hi, out, stream=None):
        check(lib().kvr_synth_q4_1(self.handle, seed, sid, blocks, d_lo, d_hi, m_lo, m_hi, _ptr(out), stream))

    def synth_normal_q8_0(self, seed, sid, blocks, out, stream=None):
        check(lib().kvr_synth_normal_q8_0(self.handle, seed, sid, blocks, _ptr(out), stream))


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
