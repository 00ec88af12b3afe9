"""Half-page layerwise scores (Mean-K records every half transport page):
the oracle's softmax over the halves and its fold, pinned by the reference
suite's known answers (layerwise_selection_test.cpp:104-160) and by the
reference's own layerwise_tile_scores / layerwise_max_page_scores."""
import math

import numpy as np
import pytest

import oracle as O


def test_half_pages_keep_short_evidence():
    # :104-131: one dim, q = 1; half means 100,100 | 8,-8 | 2,2; the first
    # page is the sink (outside the softmax); budget 2.
    means = np.array([100, 100, 8, -8, 2, 2], np.float32).reshape(6, 1)
    mask = np.array([0, 1, 1], np.uint8)
    mass = O.page_softmax_scores(means[None], np.ones((1, 1, 1, 1), np.float32), [1], 1, 1, 1, O.AGG_MEAN,
                                 np.repeat(mask, 2))
    page = O.layerwise_fold(mass, mask)
    strong, moderate = math.exp(8) + math.exp(-8), 2 * math.exp(2)
    assert page[0] == 0
    assert abs(page[1] - strong / (strong + moderate)) < 1e-12
    assert abs(page[2] - moderate / (strong + moderate)) < 1e-12
    assert O.pick_scored_blocks(page, 2, [0], O.TIE_HIGHER_FIRST).tolist() == [0, 1]
    # whole-page means average the strong half away: page 2 wins
    coarse = means.reshape(3, 2).mean(axis=1, dtype=np.float32).reshape(3, 1)
    whole = O.page_softmax_scores(coarse[None], np.ones((1, 1, 1, 1), np.float32), [1], 1, 1, 1, O.AGG_MEAN, mask)
    assert O.pick_scored_blocks(whole, 2, [0], O.TIE_HIGHER_FIRST).tolist() == [0, 2]


def _strongest_half_case(rows):
    # :133-160: two pages of two halves; dims encode logits [1,-4,.75,.75]
    # and [-4,1,.75,.75]; query rows (1,0) and (0,1)
    left, right = [1, -4, .75, .75], [-4, 1, .75, .75]
    means = np.array([[left[i], right[i]] for i in range(4)], np.float32)
    q = np.array([[[1, 0]], [[0, 1]]], np.float32)[:rows]
    return O.page_softmax_scores(means[None], q[None], [rows], 1, 1, 2, O.AGG_MEAN, None, 1.0)


def test_strongest_half_after_the_whole_query():
    z = math.exp(1) + math.exp(-4) + 2 * math.exp(.75)
    e0, e1 = (math.exp(1) + math.exp(-4)) / z, 2 * math.exp(.75) / z
    one = _strongest_half_case(1)
    assert O.pick_scored_blocks(O.layerwise_fold(one), 1, (), O.TIE_HIGHER_FIRST).tolist() == [1]  # sum
    assert O.pick_scored_blocks(O.layerwise_fold(one, keep_halves=True), 1, (), O.TIE_HIGHER_FIRST).tolist() == [0]
    both = O.layerwise_fold(_strongest_half_case(2), keep_halves=True)
    assert abs(both[0] - e0) < 1e-12 and abs(both[1] - e1) < 1e-12
    assert O.pick_scored_blocks(both, 1, (), O.TIE_HIGHER_FIRST).tolist() == [1]


def test_fold_rejects_invalid_mass():
    with pytest.raises(O.OracleError):
        O.layerwise_fold(np.array([0.5, -0.1]))
    with pytest.raises(O.OracleError):
        O.layerwise_fold(np.array([0.5, np.inf]))
    with pytest.raises(O.OracleError):
        O.layerwise_fold(np.array([0.2, 0.0, 0.3, 0.5]), np.array([0, 1], np.uint8))  # mass on a masked page


@pytest.mark.skipif(not O.ref_available(), reason="reference build (oracle/_ref) not present")
@pytest.mark.parametrize("keep", [False, True])
def test_half_page_scores_vs_reference(keep):
    rng = np.random.default_rng(31 + keep)
    for trial in range(6):
        kvh, d = [(1, 8), (2, 16), (4, 32)][trial % 3]
        group = int(rng.choice([1, 2, 4]))
        hq, mean_t = kvh * group, int(rng.choice([2, 4, 16]))
        pages = int(rng.integers(2, 40))
        tokens, w = pages * 2 * mean_t, kvh * d
        keys = O.synth_normal_f16(50 + trial, 1, tokens * w)
        rows = int(rng.integers(1, 4))
        q = O.synth_normal_f32(50 + trial, 2, rows * hq * d).reshape(rows, hq, d)
        mask = (rng.random(pages) > 0.2).astype(np.uint8)
        mask[0] = 1
        ours = O.half_page_scores(keys, tokens, w, mean_t, q, hq, kvh, d, keep, mask)
        ref = O.ref_layerwise_tile_scores_f16_keys(keys.reshape(1, -1), 0, tokens, kvh, d, mean_t, 2 * mean_t,
                                                   q.reshape(rows, -1), hq, keep, mask)
        assert np.array_equal(ours, ref)
