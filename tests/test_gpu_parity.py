"""GPU parity of the HIP recall path against the oracle, through the C ABI.

Bar: bit-exact for summaries (binary32 means and their fp16 operands),
selections (both tie rules) and gathered bytes; binary64 scores within
1e-9 relative of the oracle (1e-3).
"""
import numpy as np
import pytest

import kvmem_amd as K
import oracle as O
from gpu_util import dev, host, sync, zeros

pytestmark = pytest.mark.gpu
SEED = 42
REL = 1e-9  # binary64 logits/softmax: differences come from summation order only


def _rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b) / np.maximum(np.abs(b), 1e-300))) if a.size else 0.0


# ---------------------------------------------------------------------------
# seeded generator: device == oracle, bit for bit
# ---------------------------------------------------------------------------
def test_synth_matches_oracle(ctx):
    n = 200_003
    t = zeros(n, np.uint16)
    ctx.synth_normal_f16(SEED, 7, n, t)
    f = zeros(n, np.float32)
    ctx.synth_normal_f32(SEED, 8, n, f)
    blocks = 5001
    q8 = zeros(blocks * 34, np.uint8)
    ctx.synth_q8_0(SEED, 9, blocks, 0.01, 0.05, q8)
    q41 = zeros(blocks * 20, np.uint8)
    ctx.synth_q4_1(SEED, 10, blocks, 0.01, 0.05, -0.4, 0.0, q41)
    nq8 = zeros(blocks * 34, np.uint8)
    ctx.synth_normal_q8_0(SEED, 11, blocks, nq8)
    scale = O.synth_uniform_f32(SEED, 12, 1024, 0.5, 2.0)
    sd = dev(scale)
    sc = zeros(300 * 1024, np.uint16)
    ctx.synth_scaled_normal_f16(SEED, 13, 300, 1024, sd, sc)
    ctx.check()
    assert np.array_equal(host(t, np.uint16), O.synth_normal_f16(SEED, 7, n))
    assert np.array_equal(host(f, np.uint32), O.synth_normal_f32(SEED, 8, n).view(np.uint32))
    assert np.array_equal(host(q8, np.uint8), O.synth_q8_0(SEED, 9, blocks, 0.01, 0.05))
    assert np.array_equal(host(q41, np.uint8), O.synth_q4_1(SEED, 10, blocks, 0.01, 0.05, -0.4, 0.0))
    assert np.array_equal(host(nq8, np.uint8), O.synth_normal_q8_0(SEED, 11, blocks))
    assert np.array_equal(host(sc, np.uint16), O.synth_scaled_normal_f16(SEED, 13, 300, scale))


# ---------------------------------------------------------------------------
# page summaries
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("tokens,page_tokens,kvh,dim", [
    (5000, 256, 8, 128),   # ragged last page
    (1024, 128, 2, 64),
    (777, 32, 1, 8),
    (256, 256, 2, 256),    # one page
    (33, 1, 1, 16),        # one token per page
])
def test_summary_f16_bit_exact(ctx, tokens, page_tokens, kvh, dim):
    w = kvh * dim
    keys = O.synth_normal_f16(SEED, 1, tokens * w)
    _, means = O.page_summaries(keys, O.FMT_F16, tokens, w, page_tokens)
    pages = means.shape[0]
    m = zeros(pages * w, np.float32)
    s16 = zeros(pages * w, np.uint16)
    ctx.summary_build(K.make_keys(dev(keys), K.FMT_F16, tokens, kvh, dim, page_tokens), m, s16)
    ctx.check()
    assert np.array_equal(host(m, np.uint32), means.ravel().view(np.uint32))
    assert np.array_equal(host(s16, np.uint16), means.ravel().astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("tokens,page_tokens,kvh,dim", [(4000, 256, 8, 128), (700, 64, 2, 256), (130, 32, 1, 64),
                                                        (1000, 24, 4, 64)])
def test_summary_q8_0_bit_exact(ctx, tokens, page_tokens, kvh, dim):
    w = kvh * dim
    keys = O.synth_q8_0(SEED, 2, tokens * w // 32, 0.01, 0.05)
    _, means = O.page_summaries(keys, O.FMT_Q8_0, tokens, w, page_tokens)
    pages = means.shape[0]
    m = zeros(pages * w, np.float32)
    s16 = zeros(pages * w, np.uint16)
    ctx.summary_build(K.make_keys(dev(keys), K.FMT_Q8_0, tokens, kvh, dim, page_tokens), m, s16)
    ctx.check()
    assert np.array_equal(host(m, np.uint32), means.ravel().view(np.uint32))
    assert np.array_equal(host(s16, np.uint16), means.ravel().astype(np.float16).view(np.uint16))


def test_summary_lanes(ctx):
    lanes, tokens, kvh, dim, pt = 3, 1000, 2, 128, 128
    w = kvh * dim
    keys = O.synth_normal_f16(SEED, 3, lanes * tokens * w)
    expect = np.concatenate([O.page_summaries(keys[l * tokens * w:(l + 1) * tokens * w], O.FMT_F16,
                                              tokens, w, pt)[1].ravel() for l in range(lanes)])
    m = zeros(expect.size, np.float32)
    ctx.summary_build(K.make_keys(dev(keys), K.FMT_F16, tokens, kvh, dim, pt, lanes=lanes), m, None)
    ctx.check()
    assert np.array_equal(host(m, np.uint32), expect.view(np.uint32))


# ---------------------------------------------------------------------------
# scoring: logits + softmax + aggregation
# ---------------------------------------------------------------------------
def _score_inputs(pages, rows, dim, qheads, kvheads, layers=1, closed_form=True):
    """Closed-form operands of graph_recall_cuda_test.cpp:25,29 (sums of 4
    tokens written per page; query values in sixty-fourths)."""
    w = kvheads * dim
    if closed_form:
        b = np.arange(pages)[:, None]
        d = np.arange(w)[None, :]
        sums = np.stack([((b * 13 + d * 7 + l * 11) % 101 - 50).astype(np.float32) / np.float32(16)
                         for l in range(layers)])
        means = sums * np.float32(0.25)
        qd = np.arange(layers * rows * qheads * dim)
        query = (((qd * 17) % 127 - 63).astype(np.float32) / np.float32(32)).reshape(layers, rows, qheads, dim)
    else:
        means = O.synth_normal_f32(SEED, 4, layers * pages * w).reshape(layers, pages, w) * np.float32(0.1)
        query = O.synth_normal_f32(SEED, 5, layers * rows * qheads * dim).reshape(layers, rows, qheads, dim)
    return means.astype(np.float32), query.astype(np.float32)


SHAPES = [  # (pages, rows, dim, qheads, kvheads): graph_recall_cuda_test.cpp:18-19 and the configs
    (7, 129, 256, 8, 2),
    (8192, 2, 64, 4, 1),
    (8193, 2, 64, 4, 1),
    (128, 1, 128, 32, 8),
    (1024, 4, 128, 40, 8),
    (4096, 1, 256, 16, 2),
]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("agg", [K.AGG_MEAN, K.AGG_MAX, K.AGG_MAX_LOGIT])
@pytest.mark.parametrize("mfma", [-1, 1])
def test_score_matches_oracle(ctx, shape, agg, mfma):
    pages, rows, dim, qh, kvh = shape
    means, query = _score_inputs(pages, rows, dim, qh, kvh, closed_form=pages != 4096)
    expect = O.page_softmax_scores(means, query, [rows], qh, kvh, dim, agg)
    s16 = dev(means[0].astype(np.float16).view(np.uint16))
    q = dev(query[0])
    out = zeros(pages, np.float64)
    ctx.score(K.make_query(q, K.FMT_F32, rows, qh, kvh, dim), s16, pages, out, aggregation=agg,
              force_mfma=mfma)
    ctx.check()
    got = host(out, np.float64)
    assert _rel_err(got, expect) <= REL
    heads = qh if agg == K.AGG_MEAN else kvh
    assert abs(got.sum() - rows) <= rows * 1e-12 * max(1, heads)


@pytest.mark.parametrize("pages", [300, 3000])
def test_score_mask_and_accumulate(ctx, pages):
    """Masked scores accumulated over two layers: rows in registers (300
    pages; Max units in one workgroup with the terms in LDS) and long rows
    (3000 pages; Mean through the units' statistics and page slices)."""
    rows, dim, qh, kvh, layers = 3, 64, 8, 2, 2
    means, query = _score_inputs(pages, rows, dim, qh, kvh, layers=layers, closed_form=False)
    mask = (np.arange(pages) % 7 != 3).astype(np.uint8)
    for agg in (K.AGG_MEAN, K.AGG_MAX):
        expect = O.page_softmax_scores(means, query, [rows, rows], qh, kvh, dim, agg, score_mask=mask)
        out = zeros(pages, np.float64)
        md = dev(mask)
        for l in range(layers):
            s16 = dev(means[l].astype(np.float16).view(np.uint16))
            ctx.score(K.make_query(dev(query[l]), K.FMT_F32, rows, qh, kvh, dim), s16, pages, out,
                      aggregation=agg, score_mask=md, active_layers=layers, accumulate=l > 0)
            ctx.check()
        got = host(out, np.float64)
        assert _rel_err(got, expect) <= REL
        assert np.all(got[mask == 0] == 0)


@pytest.mark.parametrize("pages", [3000, 5000, 9000])
@pytest.mark.parametrize("agg", [K.AGG_MEAN, K.AGG_MAX, K.AGG_MAX_LOGIT])
def test_scored_selection_long_rows(ctx, pages, agg):
    """Softmax rows held in registers (<= 4096 pages), in memory passes with
    keys in LDS (<= 8192) and with keys recomputed from scores (> 8192), each
    through softmax -> aggregation -> selection in one call, with a mask and
    mandatory pages."""
    rows, dim, qh, kvh, k, pt = 2, 64, 8, 2, 64, 16
    means, query = _score_inputs(pages, rows, dim, qh, kvh, closed_form=False)
    mask = (np.arange(pages) % 11 != 5).astype(np.uint8)
    mand = (0, pages - 1)
    expect = O.page_softmax_scores(means, query, [rows], qh, kvh, dim, agg, score_mask=mask)
    s16 = dev(means[0].astype(np.float16).view(np.uint16))
    qd, md = dev(query[0]), dev(mask)  # held: the descriptors keep raw pointers
    out = zeros(pages, np.float64)
    sel = zeros(k, np.uint32)
    cnt = zeros(1, np.uint32)
    ctx.recall_layer(query=K.make_query(qd, K.FMT_F32, rows, qh, kvh, dim), summaries=s16,
                     pages=pages, page_tokens=pt, scores=out, selected=sel, count=cnt, k=k,
                     aggregation=agg, score_mask=md, mandatory=mand, tie_rule=K.TIE_LOWER_FIRST)
    ctx.check()
    got = host(out, np.float64)
    assert _rel_err(got, expect) <= REL
    assert host(cnt, np.uint32)[0] == k
    assert np.array_equal(host(sel, np.uint32), O.pick_scored_blocks(expect, k, mand, O.TIE_LOWER_FIRST))


@pytest.mark.parametrize("pages,agg", [(200, K.AGG_MAX), (3000, K.AGG_MEAN), (3000, K.AGG_MAX)])
@pytest.mark.parametrize("tie", [K.TIE_LOWER_FIRST, K.TIE_HIGHER_FIRST])
def test_multi_lane_selection(ctx, pages, agg, tie):
    """Three lanes of different summaries and queries through one call: short
    Max rows (softmax units and tail in one workgroup per lane), long Mean rows
    (units' statistics, then page slices and tail) and long Max rows, with a
    score mask and mandatory pages; every lane against the oracle."""
    lanes, rows, dim, qh, kvh, k, pt = 3, 2, 64, 8, 2, 24, 16
    means, query = _score_inputs(pages, rows, dim, qh, kvh, layers=lanes, closed_form=False)
    mask = (np.arange(pages) % 13 != 6).astype(np.uint8)
    mand = (1, pages - 2)
    s16 = dev(means.astype(np.float16).view(np.uint16).ravel())
    qd, md = dev(query.ravel()), dev(mask)
    out = zeros(lanes * pages, np.float64)
    sel = zeros(lanes * k, np.uint32)
    cnt = zeros(lanes, np.uint32)
    ctx.recall_layer(query=K.make_query(qd, K.FMT_F32, rows, qh, kvh, dim, lanes=lanes), summaries=s16,
                     pages=pages, page_tokens=pt, lanes=lanes, scores=out, selected=sel, count=cnt, k=k,
                     aggregation=agg, score_mask=md, mandatory=mand, tie_rule=tie)
    ctx.check()
    got = host(out, np.float64).reshape(lanes, pages)
    gsel = host(sel, np.uint32).reshape(lanes, k)
    assert np.array_equal(host(cnt, np.uint32), [k] * lanes)
    for l in range(lanes):
        expect = O.page_softmax_scores(means[l:l + 1], query[l:l + 1], [rows], qh, kvh, dim, agg, score_mask=mask)
        assert _rel_err(got[l], expect) <= REL, l
        assert np.array_equal(gsel[l], O.pick_scored_blocks(expect, k, mand, tie)), l


@pytest.mark.parametrize("pages,rows,dim,qh,kvh", [(300, 4, 96, 8, 2), (77, 16, 36, 4, 4)])
def test_mfma_other_head_dims(ctx, pages, rows, dim, qh, kvh):
    """Head dims the matrix-core path handles with a run-time k-range (the
    vector path needs dim/8 to be a power of two)."""
    means, query = _score_inputs(pages, rows, dim, qh, kvh, closed_form=False)
    expect = O.page_softmax_scores(means, query, [rows], qh, kvh, dim, K.AGG_MEAN)
    s16 = dev(means[0].astype(np.float16).view(np.uint16))
    q = dev(query[0])
    out = zeros(pages, np.float64)
    ctx.score(K.make_query(q, K.FMT_F32, rows, qh, kvh, dim), s16, pages, out, force_mfma=1)
    ctx.check()
    assert _rel_err(host(out, np.float64), expect) <= REL


def test_mfma_and_vector_logits_agree(ctx):
    pages, rows, dim, qh, kvh = 1024, 4, 128, 40, 8
    means, query = _score_inputs(pages, rows, dim, qh, kvh, closed_form=False)
    s16 = dev(means[0].astype(np.float16).view(np.uint16))
    q = dev(query[0])
    a = zeros(pages, np.float64)
    b = zeros(pages, np.float64)
    qd = K.make_query(q, K.FMT_F32, rows, qh, kvh, dim)
    ctx.score(qd, s16, pages, a, force_mfma=1)
    ctx.score(qd, s16, pages, b, force_mfma=-1)
    ctx.check()
    assert _rel_err(host(a, np.float64), host(b, np.float64)) <= 1e-12


@pytest.mark.parametrize("scalar", [K.FMT_F32, K.FMT_F16, K.FMT_BF16])
def test_query_scalars_and_strides(ctx, scalar):
    """Native-Q layouts (layerwise_scoring_cuda_test.cpp:37-148): token-major and
    head-major strides in f32/f16/bf16 give the same scores as dense f32 rows."""
    pages, rows, dim, qh, kvh = 200, 3, 64, 8, 2
    means, query = _score_inputs(pages, rows, dim, qh, kvh, closed_form=False)
    q32 = query[0]
    if scalar == K.FMT_F16:
        qs = q32.astype(np.float16)
        qref = qs.astype(np.float32)
        raw = qs.view(np.uint16)
    elif scalar == K.FMT_BF16:
        bits = (q32.view(np.uint32) >> 16).astype(np.uint16)
        qref = (bits.astype(np.uint32) << 16).view(np.float32)
        raw = bits
    else:
        qref = q32
        raw = q32
    expect = O.page_softmax_scores(means, qref[None], [rows], qh, kvh, dim, K.AGG_MEAN)
    s16 = dev(means[0].astype(np.float16).view(np.uint16))
    # head-major physical layout [qh][rows][dim]
    hm = np.ascontiguousarray(np.transpose(raw, (1, 0, 2)))
    for t, strides in ((raw, None), (hm, (dim, rows * dim, 1, 0))):
        out = zeros(pages, np.float64)
        ctx.score(K.make_query(dev(t), scalar, rows, qh, kvh, dim, strides=strides), s16, pages, out)
        ctx.check()
        assert _rel_err(host(out, np.float64), expect) <= REL


# ---------------------------------------------------------------------------
# selection
# ---------------------------------------------------------------------------
def _select(ctx, scores, k, lanes=1, mandatory=(), tie=K.TIE_LOWER_FIRST, signed=False):
    pages = scores.size // lanes
    sd = dev(scores.astype(np.float64))
    sel = zeros(lanes * k, np.uint32)
    cnt = zeros(lanes, np.uint32)
    ctx.select_topk(sd, pages, k, sel, cnt, lanes=lanes, mandatory=mandatory, tie_rule=tie,
                    signed_scores=signed)
    status = ctx.status()
    return status, host(sel, np.uint32).reshape(lanes, k), host(cnt, np.uint32)


@pytest.mark.parametrize("tie", [K.TIE_LOWER_FIRST, K.TIE_HIGHER_FIRST])
def test_select_matches_oracle(ctx, tie):
    rng = np.random.default_rng(SEED)
    for pages, k in ((1000, 37), (512, 32), (4096, 48), (33, 33), (40, 100), (1, 1), (32769, 64)):
        scores = rng.random(pages)
        scores[rng.choice(pages, pages // 5)] = scores[0]  # many exact ties
        for mand in ((), (min(3, pages - 1),), tuple(range(min(k, pages, 5)))):
            st, sel, cnt = _select(ctx, scores, k, mandatory=mand, tie=tie)
            assert st == 0
            expect = O.pick_scored_blocks(scores, k, mand, tie)
            assert cnt[0] == expect.size
            assert np.array_equal(sel[0, :cnt[0]], expect)


@pytest.mark.parametrize("tie", [K.TIE_LOWER_FIRST, K.TIE_HIGHER_FIRST])
def test_select_long_rows_edges(ctx, tie):
    """Rows over 1024 pages (workgroup selection) at the LDS and mandatory-mask
    boundaries, all-equal scores, a budget taken whole by mandatory pages,
    and a budget above the candidate count."""
    rng = np.random.default_rng(SEED + 1)
    mand20 = lambda pages: tuple(sorted(set(rng.choice(pages, 20, replace=False).tolist())))
    for pages in (1025, 8192, 8193, 16384, 16385):
        scores = np.round(rng.random(pages), 3)  # ~1000 distinct values: heavy ties
        for k, mand in ((64, ()), (64, mand20(pages)), (20, mand20(pages)), (pages - 3, (0, 1))):
            st, sel, cnt = _select(ctx, scores, k, mandatory=mand, tie=tie)
            assert st == 0
            expect = O.pick_scored_blocks(scores, k, mand, tie)
            assert cnt[0] == expect.size, (pages, k, len(mand))
            assert np.array_equal(sel[0, :cnt[0]], expect), (pages, k, len(mand))
    for pages in (3000, 20000):
        flat = np.full(pages, 0.25)
        for k, mand in ((50, ()), (50, (7, pages - 1))):
            st, sel, cnt = _select(ctx, flat, k, mandatory=mand, tie=tie)
            assert st == 0
            assert np.array_equal(sel[0, :cnt[0]], O.pick_scored_blocks(flat, k, mand, tie))


def test_select_reference_tie_rule(ctx):
    """layerwise_selection_test.cpp:184-194: equal mass over six pages with a
    budget of two keeps {4, 5} under the reference (higher id first) rule."""
    st, sel, cnt = _select(ctx, np.full(6, 1 / 6), 2, tie=K.TIE_HIGHER_FIRST)
    assert st == 0 and cnt[0] == 2 and list(sel[0]) == [4, 5]
    st, sel, cnt = _select(ctx, np.full(6, 1 / 6), 2, tie=K.TIE_LOWER_FIRST)
    assert st == 0 and list(sel[0]) == [0, 1]


def test_select_signed_and_invalid(ctx):
    """graph_recall_test.cpp:101-105: signed order {-.8,-.2,-.5} keeps {1,2};
    the unsigned picker rejects negative scores."""
    st, sel, cnt = _select(ctx, np.array([-.8, -.2, -.5]), 2, tie=K.TIE_HIGHER_FIRST, signed=True)
    assert st == 0 and list(sel[0, :cnt[0]]) == [1, 2]
    st, sel, cnt = _select(ctx, np.array([-.8, -.2, -.5]), 2)
    assert st == K._capi.ERR_SCORES and cnt[0] == 0
    st, sel, cnt = _select(ctx, np.array([0.1, np.nan, 0.3]), 2, signed=True)
    assert st == K._capi.ERR_SCORES and cnt[0] == 0


def test_select_lanes(ctx):
    rng = np.random.default_rng(1)
    lanes, pages, k = 8, 1024, 64
    scores = rng.random(lanes * pages)
    st, sel, cnt = _select(ctx, scores, k, lanes=lanes)
    assert st == 0
    for l in range(lanes):
        assert np.array_equal(sel[l], O.pick_scored_blocks(scores[l * pages:(l + 1) * pages], k))


def test_select_rejects_bad_mandatory(ctx):
    with pytest.raises(K.KvrError) as e:
        _select(ctx, np.ones(10), 2, mandatory=(0, 1, 2))
    assert e.value.status == K._capi.ERR_BUDGET
    with pytest.raises(K.KvrError) as e:
        _select(ctx, np.ones(10), 2, mandatory=(10,))
    assert e.value.status == K._capi.ERR_INVALID


# ---------------------------------------------------------------------------
# stage-in gather
# ---------------------------------------------------------------------------
GATHER_CASES = [  # (format, mode, width)
    (K.FMT_F16, K.GATHER_COPY, 1024),
    (K.FMT_F16, K.GATHER_DEQUANT_F16, 512),
    (K.FMT_Q8_0, K.GATHER_COPY, 1024),
    (K.FMT_Q8_0, K.GATHER_DEQUANT_F16, 1024),
    (K.FMT_Q8_0, K.GATHER_DEQUANT_F16, 512),
    (K.FMT_Q8_0, K.GATHER_REQUANT_Q8_0, 1024),
    (K.FMT_Q4_1, K.GATHER_DEQUANT_F16, 1024),
    (K.FMT_Q4_1, K.GATHER_COPY, 1024),
]


def _history(fmt, tokens, width, sid):
    if fmt == K.FMT_F16:
        return O.synth_normal_f16(SEED, sid, tokens * width).view(np.uint8)
    if fmt == K.FMT_Q8_0:
        return O.synth_q8_0(SEED, sid, tokens * width // 32, 0.01, 0.05)
    return O.synth_q4_1(SEED, sid, tokens * width // 32, 0.01, 0.05, -0.4, 0.0)


@pytest.mark.parametrize("engine", [K.ENGINE_KERNEL, K.ENGINE_SDMA])
@pytest.mark.parametrize("fmt,mode,width", GATHER_CASES)
def test_gather_bit_exact(ctx, fmt, mode, width, engine):
    tokens, pt, k = 3000, 256, 5  # 12 pages, the last one short (184 rows)
    hist = _history(fmt, tokens, width, 20 + fmt)
    pin = K.PinnedBuffer(hist.size)
    pin.numpy()[:] = hist
    sel = np.array([0, 3, 4, 9, 11], np.uint32)
    drow = K.gather_row_bytes(fmt, mode, width)
    fill = np.full(k * pt * drow, 0xA5, np.uint8)
    expect = O.gather(hist, fmt, width, tokens, pt, sel, mode, slots=fill.copy())
    slots = dev(fill)
    seld = dev(sel)
    cnt = dev(np.array([k], np.uint32))
    plane = K.make_plane(pin, fmt, width, tokens, mode, slots)
    ctx.stage_in([plane], pt, seld, cnt, k, engine=engine)
    ctx.check()
    assert np.array_equal(host(slots, np.uint8), expect)
    pin.free()


def test_gather_respects_count_and_lanes(ctx):
    lanes, tokens, width, pt, k = 3, 2048, 512, 128, 6
    hist = _history(K.FMT_Q8_0, lanes * tokens, width, 30)
    pin = K.PinnedBuffer(hist.size)
    pin.numpy()[:] = hist
    rb = K.row_bytes(K.FMT_Q8_0, width)
    sel = np.array([[1, 2, 5, 8, 9, 15], [0, 1, 2, 3, 4, 5], [10, 11, 12, 13, 14, 15]], np.uint32)
    counts = np.array([6, 2, 0], np.uint32)
    drow = width * 2
    fill = np.full(lanes * k * pt * drow, 0x5A, np.uint8)
    expect = fill.copy().reshape(lanes, -1)
    for l in range(lanes):
        lane_hist = hist[l * tokens * rb:(l + 1) * tokens * rb]
        expect[l] = O.gather(lane_hist, K.FMT_Q8_0, width, tokens, pt, sel[l, :counts[l]],
                             K.GATHER_DEQUANT_F16, slots=expect[l].copy())
    slots = dev(fill)
    plane = K.make_plane(pin, K.FMT_Q8_0, width, tokens, K.GATHER_DEQUANT_F16, slots)
    ctx.stage_in([plane], pt, dev(sel.ravel()), dev(counts), k, lanes=lanes)
    ctx.check()
    assert np.array_equal(host(slots, np.uint8), expect.ravel())
    pin.free()


def test_gather_rejects_pageable_history(ctx):
    hist = np.zeros(1024 * 256 * 2, np.uint8)
    slots = zeros(1024 * 256 * 2, np.uint8)
    plane = K.make_plane(hist.ctypes.data, K.FMT_F16, 1024, 256, K.GATHER_COPY, slots)
    with pytest.raises(K.KvrError):
        ctx.stage_in([plane], 256, dev(np.zeros(1, np.uint32)), dev(np.ones(1, np.uint32)), 1)


# ---------------------------------------------------------------------------
# capture-side running sums
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("scalar", [K.FMT_F32, K.FMT_F16, K.FMT_BF16])
def test_capture_accumulate_matches_sequential_sums(ctx, scalar):
    pt, kvh, dim, n = 128, 2, 64, 1000
    w = kvh * dim
    x = O.synth_normal_f32(SEED, 40, n * w).reshape(n, kvh, dim)
    if scalar == K.FMT_F16:
        raw = x.astype(np.float16)
        vals = raw.astype(np.float32)
        raw = raw.view(np.uint16)
    elif scalar == K.FMT_BF16:
        raw = (x.view(np.uint32) >> 16).astype(np.uint16)
        vals = (raw.astype(np.uint32) << 16).view(np.float32)
    else:
        raw = x
        vals = x
    vals = vals.reshape(n, w)
    pages = (n + pt - 1) // pt
    acc = np.zeros((pages, w), np.float32)
    cnt = np.zeros(pages, np.uint32)
    for t in range(n):
        acc[t // pt] += vals[t]
        cnt[t // pt] += 1
    means = acc * (np.float32(1) / cnt.astype(np.float32))[:, None]
    sums = zeros(pages * w, np.float32)
    counts = zeros(pages, np.uint32)
    kd = dev(raw)
    el = 4 if scalar == K.FMT_F32 else 2
    for lo, hi in ((0, 300), (300, 301), (301, 700), (700, n)):
        ptr = kd.data_ptr() + lo * w * el
        ctx.summary_accumulate(sums, counts, pt, ptr, scalar, lo, hi - lo, kvh, dim, (w, dim, 1))
    m = zeros(pages * w, np.float32)
    s16 = zeros(pages * w, np.uint16)
    ctx.summary_finalize(sums, counts, pages, w, m, s16)
    ctx.check()
    assert np.array_equal(host(counts, np.uint32), cnt)
    assert np.array_equal(host(sums, np.uint32), acc.ravel().view(np.uint32))
    assert np.array_equal(host(m, np.uint32), means.ravel().view(np.uint32))
    assert np.array_equal(host(s16, np.uint16), means.ravel().astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------------------
# operand errors
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("bad,status", [(np.nan, 2), (np.inf, 2), (70000.0, 3)])
def test_operand_errors_empty_selection(ctx, bad, status):
    pages, rows, dim, qh, kvh = 64, 1, 64, 4, 1
    means, query = _score_inputs(pages, rows, dim, qh, kvh, closed_form=False)
    query[0, 0, 1, 5] = bad
    s16 = dev(means[0].astype(np.float16).view(np.uint16))
    out = zeros(pages, np.float64)
    sel = zeros(8, np.uint32)
    cnt = dev(np.array([99], np.uint32))
    ctx.recall_layer(query=K.make_query(dev(query[0]), K.FMT_F32, rows, qh, kvh, dim), summaries=s16,
                     pages=pages, page_tokens=16, scores=out, selected=sel, count=cnt, k=8)
    assert ctx.status() == status
    assert host(cnt, np.uint32)[0] == 0
    # the next call is clean again
    query[0, 0, 1, 5] = 0.5
    ctx.recall_layer(query=K.make_query(dev(query[0]), K.FMT_F32, rows, qh, kvh, dim), summaries=s16,
                     pages=pages, page_tokens=16, scores=out, selected=sel, count=cnt, k=8)
    assert ctx.status() == 0
    assert host(cnt, np.uint32)[0] == 8


@pytest.mark.parametrize("wgs,chunk,threads", [(1, 1, 64), (7, 3, 128), (64, 8, 256), (1000, 64, 64), (0, 0, 0)])
def test_gather_options_do_not_change_bytes(ctx, wgs, chunk, threads):
    """The persistent gather's grid bound, chunk size and workgroup size
    change only the schedule: every setting writes the same slots (decoding
    and copying planes, partial last pages and partial last batches)."""
    tokens, width, pt, k = 2100, 1024, 256, 6
    hist = _history(K.FMT_Q8_0, tokens, width, 50)
    hist16 = _history(K.FMT_F16, tokens, width, 51)
    pin = K.PinnedBuffer(hist.size)
    pin.numpy()[:] = hist
    pin16 = K.PinnedBuffer(hist16.size)
    pin16.numpy()[:] = hist16
    sel = np.array([0, 2, 3, 5, 7, 8], np.uint32)
    expect = O.gather(hist, K.FMT_Q8_0, width, tokens, pt, sel, O.GATHER_DEQUANT_F16)
    expect_rq = O.gather(hist, K.FMT_Q8_0, width, tokens, pt, sel, O.GATHER_REQUANT_Q8_0)
    expect16 = O.gather(hist16, K.FMT_F16, width, tokens, pt, sel, O.GATHER_COPY)
    slots = zeros(expect.size, np.uint8)
    rq = zeros(expect_rq.size, np.uint8)
    cp = zeros(expect16.size, np.uint8)
    ctx.set_option(K._capi.OPT_GATHER_WORKGROUPS, wgs)
    ctx.set_option(K._capi.OPT_GATHER_CHUNK_ROWS, chunk)
    ctx.set_option(K._capi.OPT_GATHER_THREADS, threads)
    try:
        planes = [K.make_plane(pin, K.FMT_Q8_0, width, tokens, K.GATHER_DEQUANT_F16, slots),
                  K.make_plane(pin, K.FMT_Q8_0, width, tokens, K.GATHER_REQUANT_Q8_0, rq),
                  K.make_plane(pin16, K.FMT_F16, width, tokens, K.GATHER_COPY, cp)]
        ctx.stage_in(planes, pt, dev(sel), dev(np.array([k], np.uint32)), k)
        ctx.check()
        ctx.stage_in(planes[2:], pt, dev(sel), dev(np.array([k], np.uint32)), k)  # copy-only defaults
        ctx.check()
    finally:
        ctx.set_option(K._capi.OPT_GATHER_WORKGROUPS, 0)
        ctx.set_option(K._capi.OPT_GATHER_CHUNK_ROWS, 0)
        ctx.set_option(K._capi.OPT_GATHER_THREADS, 0)
    assert np.array_equal(host(slots, np.uint8), expect)
    assert np.array_equal(host(rq, np.uint8), expect_rq)
    assert np.array_equal(host(cp, np.uint8), expect16)
    pin.free()
    pin16.free()
