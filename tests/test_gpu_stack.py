"""kvr_recall_stack: a layer stack gives exactly the bytes of one
kvr_recall_layer call per layer (summaries, scores, selections, counts,
slots), on the fused path (layer l's softmax/selection inside layer l+1's
summary launch) and on the fallback, with device-side operand errors kept to
their own layer, and recorded into a graph."""
import numpy as np
import pytest
import torch

import kvmem_amd as K
import oracle as O
from gpu_util import dev, host, zeros
from kvmem_amd.hip import Graph, runtime

pytestmark = pytest.mark.gpu
SEED = 42
OUTS = ("s16", "scores", "sel", "cnt", "ks", "vs")


def _pinned(arr):
    raw = np.ascontiguousarray(arr).view(np.uint8).ravel()
    p = K.PinnedBuffer(raw.size)
    p.numpy()[:] = raw
    return p


class Stack:
    """n layers of fp16 history (resident K, pinned K/V) and their outputs."""

    def __init__(self, n, T=32768, HQ=32, HKV=8, D=128, PT=256, R=1, KSEL=16, resident=(), sid=900):
        self.n, self.T, self.HQ, self.HKV, self.D, self.PT, self.R, self.KSEL = n, T, HQ, HKV, D, PT, R, KSEL
        W = HKV * D
        self.W, self.P = W, T // PT
        self.layers = []
        for l in range(n):
            keys = O.synth_normal_f16(SEED, sid + 3 * l, T * W)
            vals = O.synth_normal_f16(SEED, sid + 3 * l + 1, T * W)
            q = O.synth_normal_f16(SEED, sid + 3 * l + 2, R * HQ * D)
            b = dict(keys=keys, q=q, kd=dev(keys), qd=dev(q), pk=_pinned(keys), pv=_pinned(vals),
                     resident=l in resident)
            if b["resident"]:
                _, m = O.page_summaries(keys, O.FMT_F16, T, W, PT)
                b["s16"] = dev(m.ravel().astype(np.float16).view(np.uint16))
            self.layers.append(b)
        self.alloc()

    def alloc(self):
        for b in self.layers:
            if not b["resident"]:
                b["s16"] = zeros(self.P * self.W, np.uint16)
            b.update(scores=zeros(self.P, np.float64), sel=zeros(self.KSEL, np.uint32), cnt=zeros(1, np.uint32),
                     ks=zeros(self.KSEL * self.PT * self.W, np.uint16),
                     vs=zeros(self.KSEL * self.PT * self.W, np.uint16))

    def descs(self, agg=K.AGG_MEAN, mandatory=(), tie=K.TIE_LOWER_FIRST, force_mfma=0):
        out = []
        for b in self.layers:
            planes = [K.make_plane(b["pk"], K.FMT_F16, self.W, self.T, K.GATHER_COPY, b["ks"]),
                      K.make_plane(b["pv"], K.FMT_F16, self.W, self.T, K.GATHER_COPY, b["vs"])]
            kw = dict(keys=None, pages=self.P, page_tokens=self.PT) if b["resident"] else \
                dict(keys=K.make_keys(b["kd"], K.FMT_F16, self.T, self.HKV, self.D, self.PT))
            out.append(K.Context.layer_recall(
                summaries=b["s16"], query=K.make_query(b["qd"], K.FMT_F16, self.R, self.HQ, self.HKV, self.D),
                scores=b["scores"], selected=b["sel"], count=b["cnt"], k=self.KSEL, aggregation=agg,
                tie_rule=tie, mandatory=mandatory, planes=planes, force_mfma=force_mfma, **kw))
        return out

    def outputs(self):
        return [{n: host(b[n], np.uint8).copy() for n in OUTS} for b in self.layers]

    def clear(self):
        for b in self.layers:
            for n in OUTS:
                if n != "s16" or not b["resident"]:
                    b[n].zero_()
        torch.cuda.synchronize()

    def free(self):
        for b in self.layers:
            b["pk"].free()
            b["pv"].free()


def _same(a, b):
    for l, (x, y) in enumerate(zip(a, b)):
        for n in OUTS:
            assert np.array_equal(x[n], y[n]), (l, n)


def _per_layer_then_stack(ctx, st, **kw):
    for d in st.descs(**kw):
        ctx.recall(d)
    ctx.check()
    eager = st.outputs()
    st.clear()
    keep = ctx.recall_stack(st.descs(**kw))
    ctx.check()
    del keep
    return eager, st.outputs()


@pytest.mark.parametrize("agg", [K.AGG_MEAN, K.AGG_MAX, K.AGG_MAX_LOGIT])
def test_stack_equals_layers(ctx, agg):
    st = Stack(5, resident=(2,))
    try:
        eager, stacked = _per_layer_then_stack(ctx, st, agg=agg, mandatory=(0, 3), tie=K.TIE_HIGHER_FIRST)
        _same(eager, stacked)
        for b, o in zip(st.layers, stacked):  # and the oracle on the selections
            _, m = O.page_summaries(b["keys"], O.FMT_F16, st.T, st.W, st.PT)
            qf = b["q"].view(np.float16).astype(np.float32).reshape(1, st.R, st.HQ, st.D)
            s = O.page_softmax_scores(m[None], qf, [st.R], st.HQ, st.HKV, st.D, agg)
            assert np.array_equal(o["sel"].view(np.uint32), O.pick_scored_blocks(s, st.KSEL, (0, 3),
                                                                                  O.TIE_HIGHER_FIRST))
    finally:
        st.free()


@pytest.mark.parametrize("fmt,hkv,d", [(K.FMT_Q8_0, 8, 128), (K.FMT_Q8_0, 2, 256), (K.FMT_Q8_0, 2, 128),
                                        (K.FMT_F16, 8, 128), (K.FMT_F16, 2, 64)])
def test_stack_keys_partial_last_page(ctx, fmt, hkv, d):
    """Stacks of q8_0 and fp16 key histories whose last page is partial
    (156 of 256 rows), with widths whose waves cover exactly one page (1024
    and 512 channels: rows read through a buffer resource, pad rows past the
    layer's end read as zeros) and narrower ones (256 and 128 channels:
    per-lane clamped rows): five layers (a group of four, then one), equal to
    one kvr_recall_layer per layer and to the oracle's summaries and
    selections."""
    n, T, PT, KSEL = 5, 8192 - 100, 256, 8
    HQ, W = 4 * hkv, hkv * d
    P = -(-T // PT)
    layers = []
    for l in range(n):
        if fmt == K.FMT_Q8_0:
            keys = O.synth_normal_q8_0(SEED, 700 + 2 * l, T * W // 32)
        else:
            keys = O.synth_normal_f16(SEED, 700 + 2 * l, T * W)
        q = O.synth_normal_f16(SEED, 701 + 2 * l, HQ * d)
        layers.append(dict(keys=keys, q=q, kd=dev(keys), qd=dev(q), s16=zeros(P * W, np.uint16),
                           scores=zeros(P, np.float64), sel=zeros(KSEL, np.uint32), cnt=zeros(1, np.uint32)))
    names = ("s16", "scores", "sel", "cnt")

    def descs():
        return [K.Context.layer_recall(
            keys=K.make_keys(b["kd"], fmt, T, hkv, d, PT), summaries=b["s16"],
            query=K.make_query(b["qd"], K.FMT_F16, 1, HQ, hkv, d), scores=b["scores"], selected=b["sel"],
            count=b["cnt"], k=KSEL, aggregation=K.AGG_MEAN) for b in layers]

    def outputs():
        return [{x: host(b[x], np.uint8).copy() for x in names} for b in layers]

    for desc in descs():
        ctx.recall(desc)
    ctx.check()
    eager = outputs()
    for b in layers:
        for x in names:
            b[x].zero_()
    torch.cuda.synchronize()
    keep = ctx.recall_stack(descs())
    ctx.check()
    del keep
    stacked = outputs()
    for l, (b, e, st) in enumerate(zip(layers, eager, stacked)):
        for x in names:
            assert np.array_equal(e[x], st[x]), (l, x)
        _, m = O.page_summaries(b["keys"], fmt, T, W, PT)
        assert np.array_equal(st["s16"].view(np.float16), m.ravel().astype(np.float16)), l
        qf = b["q"].view(np.float16).astype(np.float32).reshape(1, 1, HQ, d)
        s = O.page_softmax_scores(m[None], qf, [1], HQ, hkv, d, K.AGG_MEAN)
        assert np.array_equal(st["sel"].view(np.uint32), O.pick_scored_blocks(s, KSEL)), l


def test_stack_long_rows_and_single_layer(ctx):
    """4096 resident pages per layer (the tail's keys in LDS, rows in memory
    passes), and a one-layer stack."""
    st = Stack(3, T=4096 * 16, HQ=16, HKV=2, D=256, PT=16, KSEL=48, resident=(0, 1, 2), sid=950)
    try:
        eager, stacked = _per_layer_then_stack(ctx, st)
        _same(eager, stacked)
    finally:
        st.free()
    one = Stack(1, sid=960)
    try:
        eager, stacked = _per_layer_then_stack(ctx, one)
        _same(eager, stacked)
    finally:
        one.free()


@pytest.mark.parametrize("agg", [K.AGG_MEAN, K.AGG_MAX])
def test_stack_long_rows_from_keys(ctx, agg):
    """2048 pages per layer from key histories: the softmax workgroups
    compute the logits of long rows into memory, not LDS."""
    st = Stack(5, T=2048 * 16, HQ=8, HKV=2, D=64, PT=16, KSEL=32, sid=940)
    try:
        eager, stacked = _per_layer_then_stack(ctx, st, agg=agg, mandatory=(1, 2047))
        _same(eager, stacked)
    finally:
        st.free()


def test_stack_matrix_core_fallback(ctx):
    """rows*group >= 16 takes the matrix-core logits: the stack runs layer by layer."""
    st = Stack(3, T=8192, HQ=40, HKV=8, R=4, KSEL=8, sid=970)
    try:
        eager, stacked = _per_layer_then_stack(ctx, st)
        _same(eager, stacked)
    finally:
        st.free()


def test_stack_operand_error_stays_in_its_layer(ctx):
    st = Stack(4, sid=980)
    try:
        for d in st.descs():
            ctx.recall(d)
        ctx.check()
        good = st.outputs()
        st.clear()
        bad = st.layers[1]["q"].copy()
        bad[7] = 0x7C00  # fp16 +inf
        st.layers[1]["qd"].copy_(dev(bad))
        torch.cuda.synchronize()
        keep = ctx.recall_stack(st.descs())
        with pytest.raises(K.KvrError) as e:
            ctx.check()
        assert e.value.status == K._capi.ERR_NONFINITE
        del keep
        got = st.outputs()
        assert got[1]["cnt"].view(np.uint32)[0] == 0
        for l in (0, 2, 3):
            for n in OUTS:
                assert np.array_equal(got[l][n], good[l][n]), (l, n)
    finally:
        st.free()


def test_stack_in_a_graph(ctx):
    st = Stack(4, sid=990)
    hip = runtime()
    try:
        descs = st.descs()
        keep = ctx.recall_stack(descs)  # eager once: sizes the workspace
        ctx.check()
        eager = st.outputs()
        g = Graph(hip, ctx.select_stream).begin()
        try:
            keep2 = ctx.recall_stack(descs)
            join = hip.event()
            hip.record(join, ctx.copy_stream)
            hip.wait(ctx.select_stream, join)
        except Exception:
            g.abort()
            raise
        g.end()
        try:
            for rep in range(3):
                st.clear()
                g.replay()
                ctx.check()
                _same(eager, st.outputs())
                ctx.recall(descs[0])  # eager work between replays
                ctx.check()
        finally:
            g.close()
            hip.destroy_event(join)
        del keep, keep2
    finally:
        st.free()
