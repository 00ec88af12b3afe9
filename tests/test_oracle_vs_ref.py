"""The oracle against the reference's own host library (oracle/_ref, built
from the reference sources by oracle/Makefile) on randomized inputs.
Skipped where the reference build is absent (the GPU host)."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no reference sources)")
SEED = 7


def test_recall_fp16_random():
    rng = np.random.default_rng(SEED)
    xs = np.concatenate([rng.standard_normal(4000) * s for s in (1e-7, 1e-4, 1, 1e3, 4e4)]).astype(np.float32)
    for x in xs:
        try:
            a = O.recall_fp16(float(x))
        except O.OracleError:
            a = None
        try:
            b = O.ref_recall_fp16(float(x))
        except O.OracleError:
            b = None
        assert (a is None) == (b is None)
        if a is not None:
            assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32)


@pytest.mark.parametrize("tokens,pt,kvh,dim,rows,qh,agg", [
    (1000, 128, 2, 64, 3, 8, O.AGG_MEAN),
    (1000, 128, 2, 64, 3, 8, O.AGG_MAX),
    (777, 32, 1, 32, 1, 4, O.AGG_MAX),
    (4096, 256, 8, 128, 1, 32, O.AGG_MAX),
    (2048, 256, 8, 128, 4, 40, O.AGG_MEAN),
])
def test_summaries_and_scores_f16(tokens, pt, kvh, dim, rows, qh, agg):
    layers = 2
    w = kvh * dim
    keys = O.synth_normal_f16(SEED, 1, layers * tokens * w).reshape(layers, tokens, w)
    q = O.synth_normal_f32(SEED, 2, layers * rows * qh * dim).reshape(layers, rows, qh, dim)
    lr = [rows, max(1, rows - 1)]
    rm, rs = O.ref_scores_f16_keys(keys, tokens, kvh, dim, pt, q, lr, qh, agg)
    om = np.stack([O.page_summaries(keys[l], O.FMT_F16, tokens, w, pt)[1] for l in range(layers)])
    assert np.array_equal(om.view(np.uint32), rm.view(np.uint32))
    os_ = O.page_softmax_scores(om, q, lr, qh, kvh, dim, agg)
    assert np.array_equal(os_, rs)


def test_summaries_f32_prefill_path():
    layers, tokens, kvh, dim, pt = 1, 900, 2, 32, 128
    w = kvh * dim
    k = O.synth_normal_f32(SEED, 3, layers * tokens * w).reshape(layers, tokens, w)
    rm, _ = O.ref_scores_f32_keys(k, tokens, kvh, dim, pt, np.zeros((1, 1, 2, dim), np.float32), [1], 2,
                                  O.AGG_MEAN)
    for p in range(rm.shape[1]):
        rows = k[0, p * pt:min(tokens, (p + 1) * pt)]
        acc = np.zeros(w, np.float32)
        for r in rows:
            acc = (acc + r).astype(np.float32)
        assert np.array_equal((acc * (np.float32(1) / np.float32(len(rows)))).view(np.uint32),
                              rm[0, p].view(np.uint32))


@pytest.mark.parametrize("blocks,rows,dim,qh,kvh", [(7, 129, 256, 8, 2), (8193, 2, 64, 4, 1), (32769, 1, 64, 2, 1)])
@pytest.mark.parametrize("agg", [O.AGG_MEAN, O.AGG_MAX])
def test_cuda_qualification_shapes(blocks, rows, dim, qh, kvh, agg):
    """graph_recall_cuda_test.cpp:18-35 closed-form inputs, two layers, sink
    and recent masked by the frame (budget 3, sink 1, recent 1)."""
    layers = 2
    w = kvh * dim
    b = np.arange(blocks)[:, None]
    d = np.arange(w)[None, :]
    sums = np.stack([((b * 13 + d * 7 + l * 11) % 101 - 50).astype(np.float32) / np.float32(16)
                     for l in range(layers)])
    qd = np.arange(layers * rows * qh * dim)
    query = (((qd * 17) % 127 - 63).astype(np.float32) / np.float32(32)).reshape(layers, rows, qh, dim)
    _, _, mask, _ = O.query_score_frame(blocks * 4, 4, 3, 1, 1, [0, blocks - 1])
    expect = O.ref_scores_from_sums(sums, kvh, dim, 4, query, [rows, rows], qh, agg, score_mask=mask)
    got = O.page_softmax_scores(sums * np.float32(0.25), query, [rows, rows], qh, kvh, dim, agg, score_mask=mask)
    assert np.array_equal(got, expect)


def test_layerwise_current_query():
    layers, tokens, kvh, dim, pt, rows, qh = 3, 1024, 2, 64, 128, 4, 16
    w = kvh * dim
    keys = O.synth_normal_f16(SEED, 4, layers * tokens * w).reshape(layers, tokens, w)
    q = O.synth_normal_f32(SEED, 5, rows * qh * dim).reshape(rows, qh, dim)
    for layer in range(layers):
        rs = O.ref_layerwise_scores_f16_keys(keys, layer, tokens, kvh, dim, pt, q, qh)
        _, m = O.page_summaries(keys[layer], O.FMT_F16, tokens, w, pt)
        assert np.array_equal(O.page_softmax_scores(m[None], q[None], [rows], qh, kvh, dim, O.AGG_MEAN), rs)


def test_pick_random_with_pins():
    rng = np.random.default_rng(SEED)
    for trial in range(100):
        n = int(rng.integers(1, 3000))
        budget = int(rng.integers(1, 100))
        s = rng.random(n)
        s[rng.choice(n, n // 3)] = s[int(rng.integers(0, n))]
        mand = [int(x) for x in rng.choice(n, min(n, budget, int(rng.integers(0, 4))), replace=False)]
        assert np.array_equal(O.pick_scored_blocks(s, budget, mand, O.TIE_HIGHER_FIRST),
                              O.ref_pick_scored_blocks(s, budget, mand))
