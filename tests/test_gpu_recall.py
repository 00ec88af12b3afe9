"""One-call recall (kvr_recall_layer) end to end against the oracle:
summaries -> scores -> selection -> gather, on the shapes of the workloads
(the CPU-runnable 32K-token case at full size, the others downsized)."""
import numpy as np
import pytest

import kvmem_amd as K
import oracle as O
from gpu_util import dev, host, zeros

pytestmark = pytest.mark.gpu
SEED = 42
REL = 1e-9


def _rel_err(a, b):
    return float(np.max(np.abs(np.asarray(a) - b) / np.maximum(np.abs(b), 1e-300)))


def _pinned(arr):
    raw = np.ascontiguousarray(arr).view(np.uint8).ravel()
    p = K.PinnedBuffer(raw.size)
    p.numpy()[:] = raw
    return p


@pytest.mark.parametrize("agg", [K.AGG_MAX, K.AGG_MAX_LOGIT, K.AGG_MEAN])
@pytest.mark.parametrize("engine", [K.ENGINE_KERNEL, K.ENGINE_SDMA])
def test_single_layer_32k_recall(ctx, agg, engine):
    """32768 tokens, Hq 32 / Hkv 8, D 128, page 256 (128 pages), top-16,
    K = N(0,1) x per-channel U(0.5, 2), fp16 query [32 x 128]."""
    T, HQ, HKV, D, PT, KSEL = 32768, 32, 8, 128, 256, 16
    W = HKV * D
    cscale = O.synth_uniform_f32(SEED, 100, W, 0.5, 2.0)
    keys = O.synth_scaled_normal_f16(SEED, 101, T, cscale)
    vals = O.synth_normal_f16(SEED, 102, T * W)
    q16 = O.synth_normal_f16(SEED, 103, HQ * D)
    qf = q16.view(np.float16).astype(np.float32).reshape(1, 1, HQ, D)
    _, means = O.page_summaries(keys, O.FMT_F16, T, W, PT)
    expect = O.page_softmax_scores(means[None], qf, [1], HQ, HKV, D, agg)
    pages = means.shape[0]

    kd = dev(keys)
    pk, pv = _pinned(keys), _pinned(vals)
    for tie in (K.TIE_LOWER_FIRST, K.TIE_HIGHER_FIRST):
        sel_expect = O.pick_scored_blocks(expect, KSEL, (), tie)
        s16 = zeros(pages * W, np.uint16)
        m32 = zeros(pages * W, np.float32)
        scores = zeros(pages, np.float64)
        sel = zeros(KSEL, np.uint32)
        cnt = zeros(1, np.uint32)
        ks = zeros(KSEL * PT * W, np.uint16)
        vs = zeros(KSEL * PT * W, np.uint16)
        planes = [K.make_plane(pk, K.FMT_F16, W, T, K.GATHER_COPY, ks),
                  K.make_plane(pv, K.FMT_F16, W, T, K.GATHER_COPY, vs)]
        ctx.recall_layer(keys=K.make_keys(kd, K.FMT_F16, T, HKV, D, PT), summaries=s16, means=m32,
                         query=K.make_query(dev(q16), K.FMT_F16, 1, HQ, HKV, D), scores=scores,
                         selected=sel, count=cnt, k=KSEL, aggregation=agg, tie_rule=tie,
                         planes=planes, engine=engine)
        ctx.check()
        assert np.array_equal(host(m32, np.uint32), means.ravel().view(np.uint32))
        assert _rel_err(host(scores, np.float64), expect) <= REL
        assert host(cnt, np.uint32)[0] == KSEL
        got_sel = host(sel, np.uint32)
        assert np.array_equal(got_sel, sel_expect)
        kx = O.gather(keys.view(np.uint8), O.FMT_F16, W, T, PT, got_sel, O.GATHER_COPY)
        vx = O.gather(vals.view(np.uint8), O.FMT_F16, W, T, PT, got_sel, O.GATHER_COPY)
        assert np.array_equal(host(ks, np.uint8), kx)
        assert np.array_equal(host(vs, np.uint8), vx)
    pk.free()
    pv.free()


def test_quantized_k8v4_recall(ctx):
    """q8_0 K / 4-bit (q4_1 layout) V history, summaries from dequantized K,
    top-k pages dequantized to fp16 on gather (downsized: 16384 tokens)."""
    T, HQ, HKV, D, PT, KSEL = 16384, 32, 8, 128, 256, 8
    W = HKV * D
    kq = O.synth_q8_0(SEED, 110, T * W // 32, 0.01, 0.05)
    vq = O.synth_q4_1(SEED, 111, T * W // 32, 0.01, 0.05, -0.4, 0.0)
    q = O.synth_normal_f32(SEED, 112, HQ * D)
    _, means = O.page_summaries(kq, O.FMT_Q8_0, T, W, PT)
    expect = O.page_softmax_scores(means[None], q.reshape(1, 1, HQ, D), [1], HQ, HKV, D, O.AGG_MEAN)
    sel_expect = O.pick_scored_blocks(expect, KSEL)
    pages = means.shape[0]
    pk, pv = _pinned(kq), _pinned(vq)
    s16 = zeros(pages * W, np.uint16)
    scores = zeros(pages, np.float64)
    sel = zeros(KSEL, np.uint32)
    cnt = zeros(1, np.uint32)
    ks = zeros(KSEL * PT * W, np.uint16)
    vs = zeros(KSEL * PT * W, np.uint16)
    kr = zeros(KSEL * PT * K.row_bytes(K.FMT_Q8_0, W), np.uint8)
    planes = [K.make_plane(pk, K.FMT_Q8_0, W, T, K.GATHER_DEQUANT_F16, ks),
              K.make_plane(pv, K.FMT_Q4_1, W, T, K.GATHER_DEQUANT_F16, vs),
              K.make_plane(pk, K.FMT_Q8_0, W, T, K.GATHER_REQUANT_Q8_0, kr)]
    ctx.recall_layer(keys=K.make_keys(dev(kq), K.FMT_Q8_0, T, HKV, D, PT), summaries=s16,
                     query=K.make_query(dev(q), K.FMT_F32, 1, HQ, HKV, D), scores=scores,
                     selected=sel, count=cnt, k=KSEL, planes=planes)
    ctx.check()
    assert _rel_err(host(scores, np.float64), expect) <= REL
    got = host(sel, np.uint32)
    assert np.array_equal(got, sel_expect)
    assert np.array_equal(host(ks, np.uint8), O.gather(kq, O.FMT_Q8_0, W, T, PT, got, O.GATHER_DEQUANT_F16))
    assert np.array_equal(host(vs, np.uint8), O.gather(vq, O.FMT_Q4_1, W, T, PT, got, O.GATHER_DEQUANT_F16))
    assert np.array_equal(host(kr, np.uint8), O.gather(kq, O.FMT_Q8_0, W, T, PT, got, O.GATHER_REQUANT_Q8_0))
    pk.free()
    pv.free()


@pytest.mark.parametrize("mfma", [1, -1])
def test_multilane_batched_recall(ctx, mfma):
    """Eight lanes scored in one launch; Hq 40 / Hkv 8 with 4 query rows per
    lane (20 rows per kv-head, the matrix-core path), top-k per lane
    (downsized: 8192 tokens per lane)."""
    L, T, HQ, HKV, D, PT, R, KSEL = 8, 8192, 40, 8, 128, 256, 4, 8
    W = HKV * D
    keys = O.synth_normal_f16(SEED, 120, L * T * W)
    vals = O.synth_normal_f16(SEED, 121, L * T * W)
    q = O.synth_normal_f32(SEED, 122, L * R * HQ * D)
    pages = T // PT
    exp_scores, exp_sel = [], []
    for l in range(L):
        _, means = O.page_summaries(keys[l * T * W:(l + 1) * T * W], O.FMT_F16, T, W, PT)
        s = O.page_softmax_scores(means[None], q[l * R * HQ * D:(l + 1) * R * HQ * D].reshape(1, R, HQ, D),
                                  [R], HQ, HKV, D, O.AGG_MEAN)
        exp_scores.append(s)
        exp_sel.append(O.pick_scored_blocks(s, KSEL))
    pk, pv = _pinned(keys), _pinned(vals)
    s16 = zeros(L * pages * W, np.uint16)
    scores = zeros(L * pages, np.float64)
    sel = zeros(L * KSEL, np.uint32)
    cnt = zeros(L, np.uint32)
    ks = zeros(L * KSEL * PT * W, np.uint16)
    vs = zeros(L * KSEL * PT * W, np.uint16)
    planes = [K.make_plane(pk, K.FMT_F16, W, T, K.GATHER_COPY, ks),
              K.make_plane(pv, K.FMT_F16, W, T, K.GATHER_COPY, vs)]
    ctx.recall_layer(keys=K.make_keys(dev(keys), K.FMT_F16, T, HKV, D, PT, lanes=L), summaries=s16,
                     query=K.make_query(dev(q), K.FMT_F32, R, HQ, HKV, D, lanes=L), scores=scores,
                     selected=sel, count=cnt, k=KSEL, planes=planes, force_mfma=mfma)
    ctx.check()
    got_s = host(scores, np.float64).reshape(L, pages)
    got = host(sel, np.uint32).reshape(L, KSEL)
    kslots = host(ks, np.uint8).reshape(L, -1)
    for l in range(L):
        assert _rel_err(got_s[l], exp_scores[l]) <= REL
        assert np.array_equal(got[l], exp_sel[l])
        lane_keys = keys[l * T * W:(l + 1) * T * W].view(np.uint8)
        assert np.array_equal(kslots[l], O.gather(lane_keys, O.FMT_F16, W, T, PT, got[l], O.GATHER_COPY))
    pk.free()
    pv.free()


@pytest.mark.parametrize("agg", [K.AGG_MEAN, K.AGG_MAX])
def test_multilane_small_layer_fused(ctx, agg):
    """Two lanes of a small fp16 layer (16 pages each, 4096 summary lanes of 2
    channels in one-wave workgroups) with packed fp16 queries: fp16
    summaries bit-exact, scores and selections per lane against the oracle."""
    L, T, HQ, HKV, D, PT, R, KSEL = 2, 4096, 32, 8, 128, 256, 1, 5
    W, pages = HKV * D, T // PT
    keys = O.synth_normal_f16(SEED, 130, L * T * W)
    q = O.synth_normal_f16(SEED, 131, L * R * HQ * D)
    s16 = zeros(L * pages * W, np.uint16)
    scores = zeros(L * pages, np.float64)
    sel = zeros(L * KSEL, np.uint32)
    cnt = zeros(L, np.uint32)
    ctx.recall_layer(keys=K.make_keys(dev(keys), K.FMT_F16, T, HKV, D, PT, lanes=L), summaries=s16,
                     query=K.make_query(dev(q), K.FMT_F16, R, HQ, HKV, D, lanes=L), scores=scores,
                     selected=sel, count=cnt, k=KSEL, aggregation=agg)
    ctx.check()
    got16 = host(s16, np.uint16).reshape(L, pages * W)
    got_s = host(scores, np.float64).reshape(L, pages)
    got = host(sel, np.uint32).reshape(L, KSEL)
    for l in range(L):
        _, means = O.page_summaries(keys[l * T * W:(l + 1) * T * W], O.FMT_F16, T, W, PT)
        assert np.array_equal(got16[l], means.astype(np.float16).view(np.uint16).ravel()), l
        qf = q[l * R * HQ * D:(l + 1) * R * HQ * D].view(np.float16).astype(np.float32).reshape(1, R, HQ, D)
        s = O.page_softmax_scores(means[None], qf, [R], HQ, HKV, D, agg)
        assert _rel_err(got_s[l], s) <= REL, l
        assert np.array_equal(got[l], O.pick_scored_blocks(s, KSEL)), l


def test_layerwise_pipeline_resident_summaries(ctx):
    """Layerwise recall over resident summaries: score layer l+1 on the select
    stream while layer l's pages stream in on the copy stream.  Hq 16 / Hkv 2,
    D 256, q8_0 K / fp16 V history (downsized: 4 layers x 32768 tokens, top-8)."""
    LAYERS, T, HQ, HKV, D, PT, KSEL = 4, 32768, 16, 2, 256, 256, 8
    W = HKV * D
    pages = T // PT
    per_layer = []
    for l in range(LAYERS):
        kq = O.synth_normal_q8_0(SEED, 130 + l, T * W // 32)
        v = O.synth_normal_f16(SEED, 140 + l, T * W)
        q = O.synth_normal_f32(SEED, 150 + l, HQ * D)
        _, means = O.page_summaries(kq, O.FMT_Q8_0, T, W, PT)
        s = O.page_softmax_scores(means[None], q.reshape(1, 1, HQ, D), [1], HQ, HKV, D, O.AGG_MEAN)
        per_layer.append((kq, v, q, means, s, O.pick_scored_blocks(s, KSEL)))
    bufs = []
    for kq, v, q, means, s, _ in per_layer:
        bufs.append(dict(pk=_pinned(kq), pv=_pinned(v), s16=dev(means.ravel().astype(np.float16).view(np.uint16)),
                         q=dev(q), scores=zeros(pages, np.float64), sel=zeros(KSEL, np.uint32),
                         cnt=zeros(1, np.uint32), ks=zeros(KSEL * PT * W, np.uint16),
                         vs=zeros(KSEL * PT * W, np.uint16)))
    for l, b in enumerate(bufs):
        planes = [K.make_plane(b["pk"], K.FMT_Q8_0, W, T, K.GATHER_DEQUANT_F16, b["ks"]),
                  K.make_plane(b["pv"], K.FMT_F16, W, T, K.GATHER_COPY, b["vs"])]
        ctx.recall_layer(query=K.make_query(b["q"], K.FMT_F32, 1, HQ, HKV, D), summaries=b["s16"],
                         pages=pages, page_tokens=PT, scores=b["scores"], selected=b["sel"],
                         count=b["cnt"], k=KSEL, planes=planes)
    ctx.check()
    for (kq, v, q, means, s, sel_expect), b in zip(per_layer, bufs):
        assert _rel_err(host(b["scores"], np.float64), s) <= REL
        got = host(b["sel"], np.uint32)
        assert np.array_equal(got, sel_expect)
        assert np.array_equal(host(b["ks"], np.uint8),
                              O.gather(kq, O.FMT_Q8_0, W, T, PT, got, O.GATHER_DEQUANT_F16))
        assert np.array_equal(host(b["vs"], np.uint8), O.gather(v.view(np.uint8), O.FMT_F16, W, T, PT, got,
                                                                O.GATHER_COPY))
        b["pk"].free()
        b["pv"].free()


def test_borrowed_workspace_never_grows(ctx):
    """A borrowed workspace (page_softmax_cuda.hpp:16-17) serves calls that fit
    and rejects a larger call before launching anything."""
    import kvmem_amd
    pages, rows, dim, qh, kvh = 128, 1, 128, 32, 8
    c2 = kvmem_amd.Context(0)
    need = c2.workspace_bytes(1, pages, rows, qh, kvh, dim)
    ws = zeros(need, np.uint8)
    c2.bind_workspace(ws, need)
    means = O.synth_normal_f32(SEED, 160, pages * kvh * dim).reshape(1, pages, kvh * dim) * np.float32(0.1)
    q = O.synth_normal_f32(SEED, 161, rows * qh * dim).reshape(1, rows, qh, dim)
    expect = O.page_softmax_scores(means, q, [rows], qh, kvh, dim, O.AGG_MEAN)
    s16 = dev(means[0].astype(np.float16).view(np.uint16))
    out = zeros(pages, np.float64)
    c2.score(K.make_query(dev(q[0]), K.FMT_F32, rows, qh, kvh, dim), s16, pages, out)
    c2.check()
    assert _rel_err(host(out, np.float64), expect) <= REL
    with pytest.raises(K.KvrError) as e:
        c2.score(K.make_query(dev(np.zeros((4, qh, dim), np.float32)), K.FMT_F32, 4, qh, kvh, dim), s16, pages, out)
    assert e.value.status == K._capi.ERR_WORKSPACE
    assert c2.device_bytes() >= need
    c2.close()
