"""kvr_recall_layer_noalloc (logits and counters in the library's static
device scratch) against kvr_recall_layer on the same inputs: two calls in a
row, the second smaller and on the matrix-core path, each compared bit for
bit with the allocating entry point and with the oracle's selection; then a
call too large for the scratch is refused before any launch."""
import numpy as np
import pytest

import kvmem_amd as K
import oracle as O
from kvmem_amd import _capi
from gpu_util import dev, host, zeros

pytestmark = pytest.mark.gpu
SEED = 42


def _pinned(arr):
    raw = np.ascontiguousarray(arr).view(np.uint8).ravel()
    p = K.PinnedBuffer(raw.size)
    p.numpy()[:] = raw
    return p


def _run(ctx, noalloc, *, kd, kfmt, T, lanes, HQ, HKV, D, PT, rows, q, agg, KSEL, mandatory, pv, vfmt, vmode):
    W = HKV * D
    pages = (T + PT - 1) // PT
    s16 = zeros(lanes * pages * W, np.uint16)
    scores = zeros(lanes * pages, np.float64)
    sel = zeros(lanes * KSEL, np.uint32)
    cnt = zeros(lanes, np.uint32)
    slots = zeros(lanes * KSEL * PT * K.gather_row_bytes(vfmt, vmode, W), np.uint8)
    planes = [K.make_plane(pv, vfmt, W, T, vmode, slots)]
    desc = ctx.layer_recall(keys=K.make_keys(kd, kfmt, T, HKV, D, PT, lanes=lanes),
                            summaries=s16, query=K.make_query(q, K.FMT_F32, rows, HQ, HKV, D, lanes=lanes),
                            scores=scores, selected=sel, count=cnt, k=KSEL, aggregation=agg,
                            mandatory=mandatory, planes=planes, engine=K.ENGINE_KERNEL)
    (ctx.recall_noalloc if noalloc else ctx.recall)(desc)
    ctx.check()
    return (host(s16, np.uint16), host(scores, np.float64), host(sel, np.uint32), host(cnt, np.uint32),
            host(slots, np.uint8))


def _compare(ctx, **kw):
    ref = _run(ctx, False, **kw)
    got = _run(ctx, True, **kw)
    for name, a, b in zip(("summaries", "scores", "selected", "count", "slots"), got, ref):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"{name} differ from kvr_recall_layer"
    return got


def test_noalloc_matches_recall_layer(ctx):
    # call 1: fp16 keys, 65536 tokens, one query row (vector scoring), Mean,
    # two mandatory pages, fp16 V copied
    T, HQ, HKV, D, PT, KSEL = 65536, 32, 8, 128, 256, 16
    W = HKV * D
    keys = O.synth_normal_f16(SEED, 500, T * W)
    vals = O.synth_normal_f16(SEED, 501, T * W)
    q = O.synth_normal_f32(SEED, 502, HQ * D)
    pv = _pinned(vals)
    s16, sc, sel, cnt, _ = _compare(ctx, kd=dev(keys), kfmt=K.FMT_F16, T=T, lanes=1, HQ=HQ, HKV=HKV, D=D, PT=PT,
                                    rows=1, q=dev(q), agg=K.AGG_MEAN, KSEL=KSEL, mandatory=(3, 200), pv=pv,
                                    vfmt=K.FMT_F16, vmode=K.GATHER_COPY)
    _, means = O.page_summaries(keys, O.FMT_F16, T, W, PT)
    expect = O.page_softmax_scores(means[None], q.reshape(1, 1, HQ, D), [1], HQ, HKV, D, O.AGG_MEAN)
    assert np.array_equal(sel, O.pick_scored_blocks(expect, KSEL, (3, 200)))
    assert float(np.max(np.abs(sc - expect) / expect)) <= 1e-9
    pv.free()

    # call 2, smaller: two lanes of 16384 q8_0 tokens, 4 query rows x 40/8
    # heads (matrix-core logits: packed queries in the scratch too), Max,
    # 4-bit V dequantized on gather
    T, HQ, HKV, D, PT, KSEL, LANES, ROWS = 16384, 40, 8, 128, 256, 8, 2, 4
    W = HKV * D
    kq = O.synth_q8_0(SEED, 510, LANES * T * W // 32, 0.01, 0.05)
    vq = O.synth_q4_1(SEED, 511, LANES * T * W // 32, 0.01, 0.05, -0.4, 0.0)
    q = O.synth_normal_f32(SEED, 512, LANES * ROWS * HQ * D)
    pv = _pinned(vq)
    _, sc, sel, cnt, _ = _compare(ctx, kd=dev(kq), kfmt=K.FMT_Q8_0, T=T, lanes=LANES, HQ=HQ, HKV=HKV, D=D, PT=PT,
                                  rows=ROWS, q=dev(q), agg=K.AGG_MAX, KSEL=KSEL, mandatory=(), pv=pv,
                                  vfmt=K.FMT_Q4_1, vmode=K.GATHER_DEQUANT_F16)
    rowb = W // 32 * 34
    for lane in range(LANES):
        lk = kq[lane * T * rowb:(lane + 1) * T * rowb]
        _, means = O.page_summaries(lk, O.FMT_Q8_0, T, W, PT)
        ql = q[lane * ROWS * HQ * D:(lane + 1) * ROWS * HQ * D].reshape(1, ROWS, HQ, D)
        expect = O.page_softmax_scores(means[None], ql, [ROWS], HQ, HKV, D, O.AGG_MAX)
        pages = means.shape[0]
        assert np.array_equal(sel[lane * KSEL:(lane + 1) * KSEL], O.pick_scored_blocks(expect, KSEL))
        assert float(np.max(np.abs(sc[lane * pages:(lane + 1) * pages] - expect) / expect)) <= 1e-9
    assert np.array_equal(cnt, [KSEL, KSEL])
    pv.free()


def test_noalloc_refuses_what_does_not_fit(ctx):
    # 64 rows x 64 heads x 1024 pages of binary64 logits = 32 MiB > 16 MiB
    HQ, HKV, D, PT, ROWS, PAGES = 64, 8, 128, 256, 64, 1024
    s16 = zeros(16, np.uint16)
    q = zeros(ROWS * HQ * D, np.float32)
    scores, sel, cnt = zeros(PAGES, np.float64), zeros(4, np.uint32), zeros(1, np.uint32)
    desc = ctx.layer_recall(summaries=s16, pages=PAGES, page_tokens=PT,
                            query=K.make_query(q, K.FMT_F32, ROWS, HQ, HKV, D), scores=scores, selected=sel,
                            count=cnt, k=4)
    with pytest.raises(K.KvrError) as e:
        ctx.recall_noalloc(desc)
    assert e.value.status == _capi.ERR_WORKSPACE
    ctx.check()
    # the DMA engine stages through allocations: refused with planes
    slots = zeros(4 * PT * 16, np.uint8)
    pv = K.PinnedBuffer(PAGES * PT * 16)
    desc = ctx.layer_recall(summaries=s16, pages=4, page_tokens=PT,
                            query=K.make_query(q, K.FMT_F32, 1, HQ, HKV, D), scores=scores, selected=sel,
                            count=cnt, k=4, planes=[K.make_plane(pv, K.FMT_F16, 8, 4 * PT, K.GATHER_COPY, slots)],
                            engine=K.ENGINE_SDMA)
    with pytest.raises(K.KvrError) as e:
        ctx.recall_noalloc(desc)
    assert e.value.status == _capi.ERR_UNSUPPORTED
    pv.free()
