"""Pins the oracle's graph propagation and LRFU preview without the GPU.

* propagate_query_scores (kvmem/src/host/graph_recall.cpp:494-552): the
  known answers of the reference's own tests -- graph lifecycle
  (kvmem/tests/graph_recall_test.cpp:107-126), the explicit transport matrix,
  alpha 0, negative scores and a masked node (:167-188) and message locality
  (:312-322) -- then mass conservation and an independent dense
  transport-matrix restatement on random graphs;
* LrfuHistory::preview (kvmem/include/kvmem/lrfu.hpp:57-79): the known
  answers of kvmem/tests/kvmem_store_test.cpp:1178-1206 and a brute-force
  gate by sorted rank;
* and, where oracle/_ref is built, the reference's own functions on the same
  inputs (propagation to 1e-12 of the evidence total, LRFU bit for bit, and
  graph rows built by the reference's prepare_graph_accept).
"""
import numpy as np
import pytest

import oracle as O

ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")

ALL = None  # every page a transport node


def close(a, b, tol=1e-12):
    np.testing.assert_allclose(a, b, rtol=0, atol=tol)


# graph_recall_test.cpp:107-126, block_tokens 64: the sample at 64 seals as
# row (page 1 -> page 0, mass .8) once [65, 128) is accepted, the sample at
# 128 as (page 2 -> page 1, mass 1) at 192.
LIFECYCLE = [(1, [(0, .8)]), (2, [(1, 1.0)])]


def test_lifecycle_known_answers():
    g = O.PageGraph(LIFECYCLE)
    out = O.propagate_scores([1, 0, 1], g)
    close(out, [.95, .2, .85])
    close(out.sum(), 2.0)
    # the first page fixed (not a transport node)
    close(O.propagate_scores([8, 0, 1], g, mask=[0, 1, 1]), [8, .15, .85])


@ref
def test_lifecycle_rows_from_the_reference_accept():
    g = O.ref_graph_accept(64, 192, [(64, [(0, .8), (64, .2)]), (128, [(64, 1.0)])])
    want = O.PageGraph(LIFECYCLE)
    np.testing.assert_array_equal(g.row_source, want.row_source)
    np.testing.assert_array_equal(g.row_begin, want.row_begin)
    np.testing.assert_array_equal(g.edge_target, want.edge_target)
    close(g.edge_mass, want.edge_mass, 1e-15)


def test_transport_matrix_known_answers():
    # graph_recall_test.cpp:167-188: three adjacent pages, page 2 has an
    # accepted edge to page 0; columns of the transport matrix are sources
    g = O.PageGraph([(2, [(0, 1.0)])])
    raw = np.array([.8, -.2, .4])
    out = O.propagate_scores(raw, g, alpha=.4)
    close(out, [.8, -.08, .28])
    close(out.sum(), 1.0)
    assert np.array_equal(O.propagate_scores(raw, g, alpha=0), raw)  # exact bypass
    neg = np.array([-.8, -.2, -.4])
    assert np.array_equal(O.propagate_scores(neg, g, alpha=1), neg)
    close(O.propagate_scores(raw, g, alpha=.4, mask=[1, 1, 0]), [.72, -.12, .4])
    for bad in (np.nan, np.inf):
        with pytest.raises(O.OracleError):
            O.propagate_scores([0, bad, 0], g, alpha=.4)
    with pytest.raises(O.OracleError):
        O.propagate_scores([0, np.nan, 0], g, alpha=0)  # checked before the bypass


def test_message_locality_known_answers():
    # graph_recall_test.cpp:312-322: a boundary between pages 0 and 1 gives
    # the cross weight .25
    w = O.span_coefficients([(0, 64, True), (64, 192, True)], 64, 3)
    np.testing.assert_array_equal(w, [.25, 1.0])
    out = O.propagate_scores([1, 0, 0], alpha=.2, neighbor_weight=w)
    close(out[:2], [.9875, .0125])
    w = O.span_coefficients([(0, 192, True)], 64, 3)
    close(O.propagate_scores([1, 0, 0], alpha=.2, neighbor_weight=w)[:2], [.95, .05])
    # an open span's end is no boundary; a known one is
    np.testing.assert_array_equal(O.span_coefficients([(0, 64, False)], 64, 4), [1, 1, 1])
    np.testing.assert_array_equal(O.span_coefficients([(0, 64, True)], 64, 4), [.25, 1, 1])


def random_graph(rng, n, rows, fanout=4, self_edges=True):
    srcs = rng.choice(n, size=min(rows, n), replace=False)
    out = []
    for s in srcs:
        k = int(rng.integers(0, fanout + 1))
        tg = rng.integers(0, n, k)
        if self_edges and k:
            tg[0] = s
        out.append((int(s), [(int(t), float(m)) for t, m in zip(tg, rng.uniform(0, 1, k))]))
    return O.PageGraph(out)


def dense_restatement(raw, g, alpha, mask, nw):
    """out = min(raw, 0) + T max(raw, 0) with T built column by column."""
    n = raw.size
    node = np.ones(n, bool) if mask is None else np.asarray(mask, bool)
    pos = np.where(node, np.maximum(raw, 0), 0)
    if node.sum() <= 1 or pos.sum() == 0 or alpha == 0:
        return raw.copy()
    T = np.zeros((n, n))
    for i in np.flatnonzero(node):
        for j in (i - 1, i + 1):
            if 0 <= j < n and node[j]:
                c = 1.0 if nw is None else nw[min(i, j)]
                T[j, i] += alpha * .25 * c
                T[i, i] -= alpha * .25 * c
    for r in range(g.n_rows):
        s = g.row_source[r]
        if not node[s]:
            continue
        e = range(g.row_begin[r], g.row_begin[r + 1])
        den = sum(g.edge_mass[x] for x in e if g.edge_target[x] != s and node[g.edge_target[x]])
        if not den:
            continue
        for x in e:
            t = g.edge_target[x]
            if t != s and node[t]:
                T[t, s] += alpha * .5 * g.edge_mass[x] / den
                T[s, s] -= alpha * .5 * g.edge_mass[x] / den
    out = raw + T @ pos
    return np.maximum(np.minimum(raw, 0), out)


@pytest.mark.parametrize("seed", range(6))
def test_dense_restatement_and_conservation(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(2, 300))
    raw = rng.standard_normal(n)
    g = random_graph(rng, n, n // 2)
    mask = None if seed % 2 else (rng.uniform(size=n) < .8).astype(np.uint8)
    nw = None if seed % 3 else np.where(rng.uniform(size=n - 1) < .3, .25, 1.0)
    alpha = float(rng.uniform(.05, 1))
    out = O.propagate_scores(raw, g, alpha=alpha, mask=mask, neighbor_weight=nw)
    total = np.maximum(raw, 0)[mask.astype(bool) if mask is not None else slice(None)].sum()
    close(out, dense_restatement(raw, g, alpha, mask, nw), 1e-12 * max(1, total))
    close(out.sum(), raw.sum(), 1e-12 * max(1, total))  # transfers conserve mass
    assert (out >= np.minimum(raw, 0)).all()


def test_rejects_invalid_graph_mass():
    g = O.PageGraph([(0, [(1, -1.0)])])
    with pytest.raises(O.OracleError):
        O.propagate_scores([1, 1], g)
    with pytest.raises(O.OracleError):
        O.propagate_scores([1, 1], O.PageGraph([(0, [(1, np.inf)])]))


@ref
@pytest.mark.parametrize("seed", range(8))
def test_propagation_matches_reference(seed):
    rng = np.random.default_rng(100 + seed)
    n = int(rng.integers(2, 2000))
    bt = 64
    raw = rng.standard_normal(n) * (10.0 ** rng.integers(-3, 4))
    g = random_graph(rng, n, n)
    mask = None if seed % 2 else (rng.uniform(size=n) < .7).astype(np.uint8)
    spans = None
    nw = None
    if seed % 3 == 0:
        cuts = np.sort(rng.choice(np.arange(1, n), size=min(n - 1, 8), replace=False)) * bt
        edges = [0] + [int(c) for c in cuts] + [n * bt]
        spans = [(edges[i], edges[i + 1] + int(rng.integers(0, 2)) * 17, bool(rng.integers(0, 2)))
                 for i in range(len(edges) - 1)]
        nw = O.span_coefficients(spans, bt, n, .25)
    out = O.propagate_scores(raw, g, alpha=.2, mask=mask, neighbor_weight=nw)
    want = O.ref_propagate_query_scores(raw, g, alpha=.2, mask=mask, block_tokens=bt, spans=spans)
    total = np.maximum(raw, 0)[mask.astype(bool) if mask is not None else slice(None)].sum()
    close(out, want, 1e-12 * max(1, total))


@ref
def test_accept_built_graph_matches_reference():
    rng = np.random.default_rng(7)
    bt, end = 16, 16 * 200
    samples = []
    for p in sorted(rng.choice(end, 150, replace=False)):
        blocks = np.arange(0, p // bt + 1) * bt
        tg = rng.choice(blocks, size=min(6, blocks.size), replace=False)
        m = rng.uniform(0, 1, tg.size)
        samples.append((int(p), [(int(t), float(x)) for t, x in zip(tg, m / m.sum())]))
    g = O.ref_graph_accept(bt, end, samples, topk=4)
    assert g.n_rows > 50
    raw = rng.standard_normal(end // bt)
    close(O.propagate_scores(raw, g), O.ref_propagate_query_scores(raw, g, block_tokens=bt), 1e-12 * 200)


# ---------------------------------------------------------------------------
# LRFU
# ---------------------------------------------------------------------------
def test_lrfu_known_answers():
    # kvmem_store_test.cpp:1178-1179
    np.testing.assert_array_equal(O.lrfu_preview([-.8, -.6, -.2, -.2], lam=0, top_fraction=.5),
                                  [-.8, -.6, -.2, -.2])
    # :1184-1192: negative scores and fraction 1 pass through; order kept
    for x in ([-.8, -.6, -.2, -.2], [-.8, -.2, 0, .2, .6, .8], [-.8, 0, 0, 0], [0, .2, .6, .8]):
        for f in (.1, .5, .9, 1.):
            out = O.lrfu_preview(x, lam=0, top_fraction=f)
            for i, v in enumerate(x):
                if v < 0 or f == 1:
                    assert out[i] == v
                if i:
                    assert out[i] >= out[i - 1]
    # :1195-1200: hits, decay, negative evidence outside the hit set
    first = O.lrfu_preview([.1, .2, .6, .8], lam=.5, top_fraction=.5)
    np.testing.assert_array_equal(first, [0, 0, .6, .8])
    second = O.lrfu_preview([-.8, -.2, .4, .8], first, lam=.5, top_fraction=.5)
    close(second, [-.8, -.2, .7, 1.2])


@pytest.mark.parametrize("seed", range(5))
def test_lrfu_brute_force_gate(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 500))
    s = np.round(rng.standard_normal(n), 1)  # many ties
    h = rng.standard_normal(n // 2)
    lam, f = float(rng.uniform(0, 1)), float(rng.choice([.1, .37, .5, .9, 1.0]))
    out = O.lrfu_preview(s, h, lam, f)
    thr = -np.inf if f == 1 else np.sort(s)[min(n - 1, int((1 - f) * n))]
    hist = np.concatenate([h, np.zeros(n - h.size)])
    np.testing.assert_array_equal(out, lam * hist + np.where(s >= thr, s, np.minimum(s, 0)))


@ref
@pytest.mark.parametrize("seed", range(6))
def test_lrfu_matches_reference_bitwise(seed):
    rng = np.random.default_rng(50 + seed)
    n = int(rng.integers(1, 3000))
    s = rng.standard_normal(n) * 0.01
    if seed % 2:
        s = np.round(s, 3)
    h = rng.standard_normal(int(rng.integers(0, n + 5))) if seed % 3 else None
    lam, f = float(rng.uniform(0, 1)), float(rng.choice([.1, .5, .9, .95, 1.0]))
    out = O.lrfu_preview(s, h, lam, f)
    want = O.ref_lrfu_preview(s, h, lam, f)
    np.testing.assert_array_equal(out.view(np.uint64), want.view(np.uint64))
