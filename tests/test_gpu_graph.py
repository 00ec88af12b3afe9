"""GPU parity of kvr_propagate_scores and kvr_lrfu_preview (graph
propagation and the LRFU preview between scoring and selection) against the
oracle, through the C ABI.

Bars: LRFU candidates bit-exact (the same binary64 operations, no
contraction); propagated scores within 1e-12 of the evidence total (the
device adds its transfers as integers in units of <= 2^-61 of the total, the
reference one by one in its hash map's order), the same bits on every run,
and exact where the reference is exact (alpha 0, no positive evidence,
pages outside the transport mask).  Covered: the reference's known answers
(kvmem/tests/graph_recall_test.cpp:107-126, 167-188, 312-322;
kvmem_store_test.cpp:1178-1200), random graphs with masks and span
coefficients up to KVR_GRAPH_MAX_PAGES pages, several lanes, history shorter
and longer than the frame, ties at the threshold, the selection that follows
(signed scores, higher id first, as RecallPolicy::query), and every error.
"""
import numpy as np
import pytest

import kvmem_amd as K
import oracle as O
from gpu_util import dev, host, sync, zeros

pytestmark = pytest.mark.gpu


class DevGraph:
    """An O.PageGraph uploaded, plus optional neighbor weights."""

    def __init__(self, g: O.PageGraph, nw=None):
        self.g = g
        self.t = [dev(g.row_source if g.n_rows else np.zeros(1, np.uint32)),
                  dev(g.row_begin if g.row_begin.size else np.zeros(1, np.uint32)),
                  dev(g.edge_target if g.n_edges else np.zeros(1, np.uint32)),
                  dev(g.edge_mass if g.n_edges else np.zeros(1))]
        self.nw = None if nw is None else dev(np.asarray(nw, np.float64))
        self.s = K.make_page_graph(g.n_rows, g.n_edges, *self.t, neighbor_weight=self.nw)


def propagate(ctx, raw, graphs, alpha=.2, mask=None):
    """raw [lanes][pages]; graphs: one DevGraph per lane (or None)."""
    raw = np.asarray(raw, np.float64).reshape(len(graphs), -1)
    lanes, pages = raw.shape
    sc = dev(raw.ravel())
    md = None if mask is None else dev(np.asarray(mask, np.uint8).ravel())
    ctx.propagate_scores(sc, pages, [g.s if g else K.make_page_graph() for g in graphs], alpha, md, lanes)
    ctx.check()
    sync()
    return host(sc, np.float64).reshape(lanes, pages)


def lrfu(ctx, scores, history=None, lam=.5, f=.9, in_place=False):
    scores = np.asarray(scores, np.float64)
    scores = scores.reshape(1, -1) if scores.ndim == 1 else scores
    lanes, pages = scores.shape
    sc = dev(scores.ravel())
    cd = sc if in_place else zeros(scores.size, np.float64)
    h = None if history is None else np.asarray(history, np.float64).reshape(lanes, -1)
    hd = None if h is None else dev(h.ravel())
    ctx.lrfu_preview(sc, pages, cd, hd, 0 if h is None else h.shape[1], lam, f, lanes)
    ctx.check()
    sync()
    return host(cd, np.float64).reshape(lanes, pages)


def tol(raw, mask=None):
    pos = np.maximum(raw, 0)
    if mask is not None:
        pos = pos[np.asarray(mask, bool)]
    return 1e-12 * max(1.0, pos.sum())


def test_known_answers(ctx):
    g = DevGraph(O.PageGraph([(1, [(0, .8)]), (2, [(1, 1.0)])]))
    np.testing.assert_allclose(propagate(ctx, [1, 0, 1], [g])[0], [.95, .2, .85], atol=1e-15)
    np.testing.assert_allclose(propagate(ctx, [8, 0, 1], [g], mask=[0, 1, 1])[0], [8, .15, .85], atol=1e-14)
    t = DevGraph(O.PageGraph([(2, [(0, 1.0)])]))
    raw = np.array([.8, -.2, .4])
    np.testing.assert_allclose(propagate(ctx, raw, [t], alpha=.4)[0], [.8, -.08, .28], atol=1e-15)
    assert np.array_equal(propagate(ctx, raw, [t], alpha=0)[0], raw)
    neg = np.array([-.8, -.2, -.4])
    assert np.array_equal(propagate(ctx, neg, [t], alpha=1)[0], neg)
    np.testing.assert_allclose(propagate(ctx, raw, [t], alpha=.4, mask=[1, 1, 0])[0], [.72, -.12, .4], atol=1e-15)
    w = O.span_coefficients([(0, 64, True), (64, 192, True)], 64, 3)
    np.testing.assert_allclose(propagate(ctx, [1, 0, 0], [DevGraph(O.PageGraph(), w)])[0][:2], [.9875, .0125],
                               atol=1e-15)
    # LRFU
    assert np.array_equal(lrfu(ctx, [-.8, -.6, -.2, -.2], lam=0, f=.5)[0], [-.8, -.6, -.2, -.2])
    first = lrfu(ctx, [.1, .2, .6, .8], lam=.5, f=.5)[0]
    assert np.array_equal(first, [0, 0, .6, .8])
    np.testing.assert_allclose(lrfu(ctx, [-.8, -.2, .4, .8], first, lam=.5, f=.5)[0], [-.8, -.2, .7, 1.2],
                               atol=1e-12)


def random_case(rng, n, rows_frac=1.0):
    raw = rng.standard_normal(n) * float(10.0 ** rng.integers(-2, 3))
    rows = []
    for s in rng.choice(n, size=max(1, int(n * rows_frac)) if n > 1 else 1, replace=False):
        k = int(rng.integers(0, 5))
        tg = rng.integers(0, n, k)
        rows.append((int(s), [(int(t), float(m)) for t, m in zip(tg, rng.uniform(0, 1, k))]))
    return raw, O.PageGraph(rows)


@pytest.mark.parametrize("pages", [2, 255, 256, 257, 1000, 4096, 8192])
def test_random_graphs(ctx, pages):
    rng = np.random.default_rng(pages)
    lanes = 3
    raws, graphs, dgs, nws = [], [], [], []
    for l in range(lanes):
        raw, g = random_case(rng, pages, (0.0, .3, 1.0)[l])
        nw = None if l == 0 else np.where(rng.uniform(size=pages - 1) < .2, .25, 1.0)
        raws.append(raw)
        graphs.append(g)
        nws.append(nw)
        dgs.append(DevGraph(g, nw))
    mask = (rng.uniform(size=(lanes, pages)) < .85).astype(np.uint8)
    mask[0] = 1
    got = propagate(ctx, np.stack(raws), dgs, alpha=.3, mask=mask)
    again = propagate(ctx, np.stack(raws), dgs, alpha=.3, mask=mask)
    assert np.array_equal(got.view(np.uint64), again.view(np.uint64)), "not deterministic"
    for l in range(lanes):
        want = O.propagate_scores(raws[l], graphs[l], .3, mask[l], nws[l])
        np.testing.assert_allclose(got[l], want, rtol=0, atol=tol(raws[l], mask[l]))
        off = mask[l] == 0
        # pages outside the mask keep their score (a -0.0 becomes +0.0, as in the reference)
        assert np.array_equal(got[l][off], np.maximum(np.minimum(raws[l][off], 0), raws[l][off]))


@pytest.mark.parametrize("pages", [1, 7, 256, 1000, 8192])
def test_lrfu_bit_exact(ctx, pages):
    rng = np.random.default_rng(500 + pages)
    lanes = 2
    s = np.round(rng.standard_normal((lanes, pages)), 2)  # ties at the threshold
    for f in (.1, .5, .9, .95, 1.0):
        for hp in (0, pages // 2, pages + 3):
            h = rng.standard_normal((lanes, hp)) if hp else None
            lam = float(rng.uniform(0, 1))
            got = lrfu(ctx, s, h, lam, f)
            for l in range(lanes):
                want = O.lrfu_preview(s[l], None if h is None else h[l], lam, f)
                np.testing.assert_array_equal(got[l].view(np.uint64), want.view(np.uint64))
    # in place (candidate = scores), all scores equal, and signed zeros
    z = np.array([[0.0, -0.0, 0.0, -0.0, -1.0, 2.0]])
    np.testing.assert_array_equal(lrfu(ctx, z, lam=.3, f=.5, in_place=True)[0].view(np.uint64),
                                  O.lrfu_preview(z[0], None, .3, .5).view(np.uint64))
    e = np.full((1, 100), 0.25)
    np.testing.assert_array_equal(lrfu(ctx, e, lam=0, f=.3)[0], O.lrfu_preview(e[0], None, 0, .3))


def test_propagate_lrfu_select_pipeline(ctx):
    """RecallPolicy::query (backends/radiance/adapter/recall_policy.hpp:104-130):
    scores -> propagate -> LRFU preview -> (score desc, id desc) top budget."""
    rng = np.random.default_rng(77)
    pages, k = 4096, 48
    raw, g = random_case(rng, pages, .5)
    raw = raw / np.abs(raw).sum()
    hist = O.lrfu_preview(rng.standard_normal(pages) * 1e-3, None, .5, .9)
    sc = propagate(ctx, raw, [DevGraph(g)], alpha=.2)[0]
    cand = lrfu(ctx, sc, hist, .5, .9)[0]
    want_c = O.lrfu_preview(O.propagate_scores(raw, g, .2), hist, .5, .9)
    np.testing.assert_allclose(cand, want_c, rtol=0, atol=3e-12)
    cd = dev(cand)
    sel, cnt = zeros(k, np.uint32), zeros(1, np.uint32)
    ctx.select_topk(cd, pages, k, sel, cnt, tie_rule=K.TIE_HIGHER_FIRST, signed_scores=True)
    ctx.check()
    sync()
    want = O.pick_scored_blocks(cand, k, tie_rule=O.TIE_HIGHER_FIRST, signed_scores=True)
    np.testing.assert_array_equal(host(sel, np.uint32)[:host(cnt, np.uint32)[0]], want)
    assert np.array_equal(want, O.pick_scored_blocks(want_c, k, tie_rule=O.TIE_HIGHER_FIRST, signed_scores=True))


def test_fused_launch_matches_the_two_calls(ctx):
    rng = np.random.default_rng(88)
    lanes, pages = 2, 3000
    raws, dgs = [], []
    for _ in range(lanes):
        raw, g = random_case(rng, pages, .6)
        raws.append(raw)
        dgs.append(DevGraph(g, np.where(rng.uniform(size=pages - 1) < .1, .25, 1.0)))
    raw = np.stack(raws)
    mask = (rng.uniform(size=(lanes, pages)) < .9).astype(np.uint8)
    hist = rng.standard_normal((lanes, pages - 100))
    want_s = propagate(ctx, raw, dgs, alpha=.25, mask=mask)
    want_c = lrfu(ctx, want_s, hist, .4, .8)
    sc, cd = dev(raw.ravel()), zeros(raw.size, np.float64)
    ctx.propagate_lrfu(sc, pages, cd, [g.s for g in dgs], .25, dev(mask.ravel()), dev(hist.ravel()), pages - 100,
                       .4, .8, lanes)
    ctx.check()
    sync()
    assert np.array_equal(host(sc, np.float64).reshape(lanes, pages).view(np.uint64), want_s.view(np.uint64))
    assert np.array_equal(host(cd, np.float64).reshape(lanes, pages).view(np.uint64), want_c.view(np.uint64))
    # a propagation error writes neither output of its lane
    bad = raw.copy()
    bad[1, 5] = np.nan
    sc, cd = dev(bad.ravel()), zeros(raw.size, np.float64)
    ctx.propagate_lrfu(sc, pages, cd, [g.s for g in dgs], .25, None, None, 0, .4, .8, lanes)
    with pytest.raises(K.KvrError) as e:
        ctx.check()
    assert e.value.status == K._capi.ERR_SCORES
    assert not host(cd, np.float64).reshape(lanes, pages)[1].any()
    assert np.array_equal(host(sc, np.float64).reshape(lanes, pages)[1].view(np.uint64), bad[1].view(np.uint64))


def test_errors(ctx):
    g = DevGraph(O.PageGraph([(0, [(1, .5)])]))
    raw = np.array([1.0, np.nan, 2.0])
    sc = dev(raw)
    ctx.propagate_scores(sc, 3, [g.s])
    with pytest.raises(K.KvrError) as e:
        ctx.check()
    assert e.value.status == K._capi.ERR_SCORES
    assert np.array_equal(host(sc, np.float64)[[0, 2]], [1.0, 2.0])  # untouched

    def graph_error(gr):
        s = dev(np.array([1.0, 1.0, 1.0]))
        ctx.propagate_scores(s, 3, [gr.s])
        with pytest.raises(K.KvrError) as e:
            ctx.check()
        assert e.value.status == K._capi.ERR_GRAPH
        assert np.array_equal(host(s, np.float64), [1.0, 1.0, 1.0])

    graph_error(DevGraph(O.PageGraph([(0, [(1, -1.0)])])))
    graph_error(DevGraph(O.PageGraph([(0, [(1, np.inf)])])))
    graph_error(DevGraph(O.PageGraph(), [1.5, 1.0]))
    bad = O.PageGraph.from_arrays([0], [1, 0], [1], [1.0])  # row_begin decreasing
    gb = DevGraph(O.PageGraph([(0, [(1, 1.0)])]))
    gb.t[1] = dev(bad.row_begin)
    gb.s = K.make_page_graph(1, 1, *gb.t)
    graph_error(gb)

    big = zeros(K._capi.GRAPH_MAX_PAGES + 1, np.float64)
    with pytest.raises(K.KvrError) as e:
        ctx.propagate_scores(big, K._capi.GRAPH_MAX_PAGES + 1)
    assert e.value.status == K._capi.ERR_UNSUPPORTED
    with pytest.raises(K.KvrError) as e:
        ctx.propagate_scores(dev(np.ones(3)), 3, alpha=1.5)
    assert e.value.status == K._capi.ERR_INVALID
    cd = zeros(3, np.float64)
    for lam, f in ((-.1, .5), (1.1, .5), (.5, 0.0), (.5, 1.5)):
        with pytest.raises(K.KvrError) as e:
            ctx.lrfu_preview(dev(np.ones(3)), 3, cd, lam=lam, top_fraction=f)
        assert e.value.status == K._capi.ERR_INVALID
    ctx.lrfu_preview(dev(np.array([1.0, np.inf, 0.0])), 3, cd)
    with pytest.raises(K.KvrError) as e:
        ctx.check()
    assert e.value.status == K._capi.ERR_SCORES
    assert not host(cd, np.float64).any()
