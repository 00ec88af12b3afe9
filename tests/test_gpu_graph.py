"""Recall recorded into a HIP graph and replayed: every replay equals the
eager call on the same buffers, replays read the buffers' current contents,
device-side operand errors raised in a replay reach kvr_check once, and the
calls that cannot be captured refuse before recording anything."""
import numpy as np
import pytest
import torch

import kvmem_amd as K
import oracle as O
from gpu_util import dev, host, zeros
from kvmem_amd.hip import Graph, runtime

pytestmark = pytest.mark.gpu
SEED = 42
T, HQ, HKV, D, PT, KSEL, LAYERS = 32768, 32, 8, 128, 256, 16, 2
W = HKV * D
PAGES = T // PT


def _pinned(arr):
    raw = np.ascontiguousarray(arr).view(np.uint8).ravel()
    p = K.PinnedBuffer(raw.size)
    p.numpy()[:] = raw
    return p


@pytest.fixture(scope="module")
def stack():
    """Two layers of fp16 history, resident K and pinned K/V, with outputs."""
    layers = []
    for l in range(LAYERS):
        keys = O.synth_normal_f16(SEED, 600 + l, T * W)
        vals = O.synth_normal_f16(SEED, 610 + l, T * W)
        q = O.synth_normal_f16(SEED, 620 + l, HQ * D)
        layers.append(dict(keys=keys, vals=vals, q=q, kd=dev(keys), qd=dev(q), pk=_pinned(keys),
                           pv=_pinned(vals), s16=zeros(PAGES * W, np.uint16),
                           scores=zeros(PAGES, np.float64), sel=zeros(KSEL, np.uint32),
                           cnt=zeros(1, np.uint32), ks=zeros(KSEL * PT * W, np.uint16),
                           vs=zeros(KSEL * PT * W, np.uint16)))
    yield layers
    for b in layers:
        b["pk"].free()
        b["pv"].free()


def _enqueue(ctx, layers, engine=K.ENGINE_KERNEL):
    for b in layers:
        planes = [K.make_plane(b["pk"], K.FMT_F16, W, T, K.GATHER_COPY, b["ks"]),
                  K.make_plane(b["pv"], K.FMT_F16, W, T, K.GATHER_COPY, b["vs"])]
        ctx.recall_layer(keys=K.make_keys(b["kd"], K.FMT_F16, T, HKV, D, PT), summaries=b["s16"],
                         query=K.make_query(b["qd"], K.FMT_F16, 1, HQ, HKV, D), scores=b["scores"],
                         selected=b["sel"], count=b["cnt"], k=KSEL, aggregation=K.AGG_MEAN,
                         planes=planes, engine=engine)


def _outputs(layers):
    return [{n: host(b[n], np.uint8).copy() for n in ("s16", "scores", "sel", "cnt", "ks", "vs")}
            for b in layers]


def _clear(layers):
    for b in layers:
        for n in ("s16", "scores", "sel", "cnt", "ks", "vs"):
            b[n].zero_()
    torch.cuda.synchronize()


def _capture(ctx, layers):
    hip = runtime()
    g = Graph(hip, ctx.select_stream).begin()
    try:
        _enqueue(ctx, layers)
        join = hip.event()
        hip.record(join, ctx.copy_stream)  # join the copy stream back
        hip.wait(ctx.select_stream, join)
    except Exception:
        g.abort()
        raise
    g.end()
    hip.destroy_event(join)
    return g


def _expect_oracle(b):
    _, means = O.page_summaries(b["keys"], O.FMT_F16, T, W, PT)
    qf = b["q"].view(np.float16).astype(np.float32).reshape(1, 1, HQ, D)
    return O.pick_scored_blocks(O.page_softmax_scores(means[None], qf, [1], HQ, HKV, D, O.AGG_MEAN), KSEL)


def test_graph_replays_match_eager(ctx, stack):
    _enqueue(ctx, stack)       # eager; also sizes the workspace before capture
    ctx.check()
    eager = _outputs(stack)
    for b, e in zip(stack, eager):
        assert np.array_equal(e["sel"].view(np.uint32), _expect_oracle(b))
    _clear(stack)
    g = _capture(ctx, stack)
    try:
        # capture recorded work without running it
        assert not any(host(b["cnt"], np.uint32)[0] for b in stack)
        for rep in range(3):
            _clear(stack)
            g.replay()
            ctx.check()
            got = _outputs(stack)
            for l in range(LAYERS):
                for n in eager[l]:
                    assert np.array_equal(got[l][n], eager[l][n]), (rep, l, n)
            # eager work on the same context between replays
            _enqueue(ctx, stack[:1])
            ctx.check()
    finally:
        g.close()


def test_graph_reads_live_buffers(ctx, stack):
    """A replay after the query buffers change scores the new queries."""
    _enqueue(ctx, stack)
    ctx.check()
    g = _capture(ctx, stack)
    saved = [b["qd"].clone() for b in stack]
    try:
        for b, l in zip(stack, range(LAYERS)):
            q2 = O.synth_normal_f16(SEED, 700 + l, HQ * D)
            b["qd"].copy_(dev(q2))
            b["q_new"] = q2
        torch.cuda.synchronize()
        g.replay()
        ctx.check()
        for b in stack:
            qf = b["q_new"].view(np.float16).astype(np.float32).reshape(1, 1, HQ, D)
            _, means = O.page_summaries(b["keys"], O.FMT_F16, T, W, PT)
            s = O.page_softmax_scores(means[None], qf, [1], HQ, HKV, D, O.AGG_MEAN)
            got = host(b["sel"], np.uint32)
            assert np.array_equal(got, O.pick_scored_blocks(s, KSEL))
            assert np.array_equal(host(b["ks"], np.uint8),
                                  O.gather(b["keys"].view(np.uint8), O.FMT_F16, W, T, PT, got, O.GATHER_COPY))
    finally:
        for b, q in zip(stack, saved):
            b["qd"].copy_(q)
        torch.cuda.synchronize()
        g.close()


def test_graph_replay_error_is_reported_once(ctx, stack):
    """A non-finite query in a replay empties that layer's selection and is
    reported by the next kvr_check; the following good replay is clean."""
    _enqueue(ctx, stack)
    ctx.check()
    g = _capture(ctx, stack)
    saved = stack[0]["qd"].clone()
    try:
        bad = stack[0]["q"].copy()
        bad[5] = 0x7E00  # fp16 NaN
        stack[0]["qd"].copy_(dev(bad))
        torch.cuda.synchronize()
        g.replay()
        with pytest.raises(K.KvrError) as e:
            ctx.check()
        assert e.value.status == K._capi.ERR_NONFINITE
        assert host(stack[0]["cnt"], np.uint32)[0] == 0
        stack[0]["qd"].copy_(saved)
        torch.cuda.synchronize()
        g.replay()
        ctx.check()
        for b in stack:
            assert host(b["cnt"], np.uint32)[0] == KSEL
            assert np.array_equal(host(b["sel"], np.uint32), _expect_oracle(b))
    finally:
        stack[0]["qd"].copy_(saved)
        torch.cuda.synchronize()
        g.close()


def test_dma_engine_refuses_capture(ctx, stack):
    _enqueue(ctx, stack[:1])
    ctx.check()
    hip = runtime()
    g = Graph(hip, ctx.select_stream).begin()
    try:
        with pytest.raises(K.KvrError) as e:
            _enqueue(ctx, stack[:1], engine=K.ENGINE_SDMA)
        assert "captured" in str(e.value)
    finally:
        g.abort()
    ctx.check()


def test_workspace_growth_refuses_capture(stack):
    """A fresh context has no workspace: growing it inside a capture fails
    with KVR_ERR_WORKSPACE instead of allocating."""
    c2 = K.Context(0)
    hip = runtime()
    g = Graph(hip, c2.select_stream).begin()
    try:
        with pytest.raises(K.KvrError) as e:
            _enqueue(c2, stack[:1])
        assert e.value.status == K._capi.ERR_WORKSPACE
    finally:
        g.abort()
    c2.close()


def test_timing_events_refuse_capture(ctx, stack):
    """Summary timing events would not be re-recorded by replays: refused."""
    _enqueue(ctx, stack[:1])
    ctx.check()
    hip = runtime()
    ev = (hip.event(), hip.event())
    b = stack[0]
    g = Graph(hip, ctx.select_stream).begin()
    try:
        with pytest.raises(K.KvrError) as e:
            ctx.recall_layer(keys=K.make_keys(b["kd"], K.FMT_F16, T, HKV, D, PT), summaries=b["s16"],
                             query=K.make_query(b["qd"], K.FMT_F16, 1, HQ, HKV, D), scores=b["scores"],
                             selected=b["sel"], count=b["cnt"], k=KSEL, summary_events=ev)
        assert "captured" in str(e.value)
    finally:
        g.abort()
    for x in ev:
        hip.destroy_event(x)
    ctx.check()
