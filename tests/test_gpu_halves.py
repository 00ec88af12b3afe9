"""Half-page layerwise recall on the device (summaries every half transport
page, one softmax over the halves, folded in the softmax tail) against the
oracle: one layer, a fused stack, resident summaries and the standalone
fold, with the reference suite's known answers run on the device."""
import math

import numpy as np
import pytest

import kvmem_amd as K
import oracle as O
from kvmem_amd import _capi
from gpu_util import dev, host, zeros

pytestmark = pytest.mark.gpu
SEED = 42
REL = 1e-9


def _rel(a, b):
    return float(np.max(np.abs(a - b) / np.maximum(np.abs(b), 1e-300)))


def _pinned(arr):
    raw = np.ascontiguousarray(arr).view(np.uint8).ravel()
    p = K.PinnedBuffer(raw.size)
    p.numpy()[:] = raw
    return p


@pytest.mark.parametrize("fold", [_capi.HALF_SUM, _capi.HALF_MAX])
def test_half_page_layer_and_stack(ctx, fold):
    T, HQ, HKV, D, MT, KSEL = 65536, 32, 8, 128, 128, 16  # Mean-K every 128 tokens, pages of 256
    W, PT = HKV * D, 2 * MT
    P = T // PT
    keys = O.synth_normal_f16(SEED, 800, T * W)
    vals = O.synth_normal_f16(SEED, 801, T * W)
    q = O.synth_normal_f32(SEED, 802, 2 * HQ * D).reshape(2, HQ, D)
    mask = np.ones(P, np.uint8)
    mask[[0, 5, P - 1]] = 0
    keep = fold == _capi.HALF_MAX
    expect = O.half_page_scores(keys, T, W, MT, q, HQ, HKV, D, keep, mask)
    mand = (0, P - 1)
    sel_expect = O.pick_scored_blocks(expect, KSEL, mand, O.TIE_HIGHER_FIRST)
    kd, qd, md = dev(keys), dev(q), dev(mask)
    pv = _pinned(vals)

    def layer():
        out = dict(s16=zeros(2 * P * W, np.uint16), sc=zeros(P, np.float64), sel=zeros(KSEL, np.uint32),
                   cnt=zeros(1, np.uint32), vs=zeros(KSEL * PT * W, np.uint16))
        d = ctx.layer_recall(keys=K.make_keys(kd, K.FMT_F16, T, HKV, D, MT), summaries=out["s16"],
                             query=K.make_query(qd, K.FMT_F32, 2, HQ, HKV, D), scores=out["sc"],
                             selected=out["sel"], count=out["cnt"], k=KSEL, score_mask=md,
                             tie_rule=K.TIE_HIGHER_FIRST, mandatory=mand, half_fold=fold,
                             planes=[K.make_plane(pv, K.FMT_F16, W, T, K.GATHER_COPY, out["vs"])])
        return d, out

    def verify(out):
        assert _rel(host(out["sc"], np.float64), expect) <= REL
        got = host(out["sel"], np.uint32)[: int(host(out["cnt"], np.uint32)[0])]
        assert np.array_equal(got, sel_expect)
        vx = O.gather(vals.view(np.uint8), O.FMT_F16, W, T, PT, got, O.GATHER_COPY)
        assert np.array_equal(host(out["vs"], np.uint8), vx)

    d, out = layer()
    ctx.recall(d)
    ctx.check()
    verify(out)
    descs = [layer() for _ in range(5)]  # five identical layers: groups of four and one
    arr = ctx.recall_stack([x[0] for x in descs])
    ctx.check()
    for _, o in descs:
        verify(o)
    del arr
    # resident half-page summaries, vector and matrix-core logits
    s16 = out["s16"]
    for force in (-1, 1):
        sc, sel, cnt = zeros(P, np.float64), zeros(KSEL, np.uint32), zeros(1, np.uint32)
        ctx.recall_layer(summaries=s16, pages=2 * P, page_tokens=MT, query=K.make_query(qd, K.FMT_F32, 2, HQ, HKV, D),
                         scores=sc, selected=sel, count=cnt, k=KSEL, score_mask=md, tie_rule=K.TIE_HIGHER_FIRST,
                         mandatory=mand, half_fold=fold, force_mfma=force)
        ctx.check()
        assert _rel(host(sc, np.float64), expect) <= REL
        assert np.array_equal(host(sel, np.uint32)[: int(host(cnt, np.uint32)[0])], sel_expect)
    pv.free()


def _device_kat(ctx, means, q, mask, fold, k, mand=()):
    """Resident fp32 half means padded to head_dim 8 (zeros), scale 1."""
    halves, dims = means.shape
    s16 = np.zeros((halves, 8), np.float16)
    s16[:, :dims] = means
    rows = q.shape[0]
    qq = np.zeros((rows, 1, 8), np.float32)
    qq[:, 0, :dims] = q
    P = halves // 2
    sc, sel, cnt = zeros(P, np.float64), zeros(k, np.uint32), zeros(1, np.uint32)
    ctx.recall_layer(summaries=dev(s16.view(np.uint16)), pages=halves, page_tokens=4,
                     query=K.make_query(dev(qq), K.FMT_F32, rows, 1, 1, 8, attention_scale=1.0), scores=sc,
                     selected=sel, count=cnt, k=k, score_mask=None if mask is None else dev(mask),
                     tie_rule=K.TIE_HIGHER_FIRST, mandatory=mand, half_fold=fold)
    ctx.check()
    return host(sc, np.float64), host(sel, np.uint32)[: int(host(cnt, np.uint32)[0])]


def test_known_answers_on_device(ctx):
    # layerwise_selection_test.cpp:104-131: half pages keep short evidence
    means = np.array([100, 100, 8, -8, 2, 2], np.float32).reshape(6, 1)
    sc, sel = _device_kat(ctx, means, np.ones((1, 1), np.float32), np.array([0, 1, 1], np.uint8), _capi.HALF_SUM,
                          2, (0,))
    strong, moderate = math.exp(8) + math.exp(-8), 2 * math.exp(2)
    assert sc[0] == 0 and abs(sc[1] - strong / (strong + moderate)) < 1e-12
    assert sel.tolist() == [0, 1]
    # :133-160: the strongest half after the whole Query
    left, right = [1, -4, .75, .75], [-4, 1, .75, .75]
    means = np.array([[left[i], right[i]] for i in range(4)], np.float32)
    q2 = np.array([[1, 0], [0, 1]], np.float32)
    assert _device_kat(ctx, means, q2[:1], None, _capi.HALF_SUM, 1)[1].tolist() == [1]
    assert _device_kat(ctx, means, q2[:1], None, _capi.HALF_MAX, 1)[1].tolist() == [0]
    sc, sel = _device_kat(ctx, means, q2, None, _capi.HALF_MAX, 1)
    z = math.exp(1) + math.exp(-4) + 2 * math.exp(.75)
    assert abs(sc[0] - (math.exp(1) + math.exp(-4)) / z) < 1e-12 and abs(sc[1] - 2 * math.exp(.75) / z) < 1e-12
    assert sel.tolist() == [1]


def test_standalone_fold_of_tiled_halves(ctx):
    """A Query scored tile by tile over the halves (kvr_score accumulating),
    then folded by kvr_fold_half_pages: max at the end of the Query."""
    T, HQ, HKV, D, MT = 16384, 8, 2, 64, 64
    W, P = HKV * D, T // (2 * MT)
    keys = O.synth_normal_f16(SEED, 810, T * W)
    q = O.synth_normal_f32(SEED, 811, 3 * HQ * D).reshape(3, HQ, D)
    _, means = O.page_summaries(keys, O.FMT_F16, T, W, MT)
    s16 = dev(means.astype(np.float16).view(np.uint16))  # RNE to binary16, as recall_fp16
    halves = zeros(2 * P, np.float64)
    for r in range(3):  # three tiles of one row each
        ctx.score(K.make_query(dev(q[r]), K.FMT_F32, 1, HQ, HKV, D), s16, 2 * P, halves, accumulate=r > 0)
    for rule, keep in ((_capi.HALF_MAX, True), (_capi.HALF_SUM, False)):
        out = zeros(P, np.float64)
        ctx.fold_half_pages(halves, P, out, rule)
        ctx.check()
        expect = O.half_page_scores(keys, T, W, MT, q, HQ, HKV, D, keep)
        assert _rel(host(out, np.float64), expect) <= REL
    # invalid halves: a negative mass
    bad = dev(np.array([0.5, -0.25, 0.1, 0.1]))
    out = zeros(2, np.float64)
    ctx.fold_half_pages(bad, 2, out, _capi.HALF_SUM)
    assert ctx.status() == _capi.ERR_SCORES
    ctx.check()
