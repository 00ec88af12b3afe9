"""The oracle's page policies around the scored pick (query_fixed_blocks,
pick_scored_blocks with media groups, pick_topk_ungrouped, constrain_media)
pinned by the reference test suite's known answers and by the reference's
own KvMemStore compiled into oracle/_ref, on random stores with media
ranges (sorted, overlapping, unsorted, past the end, empty)."""
import numpy as np
import pytest

import oracle as O

BT = 32  # block tokens of the known-answer stores


def _has(sel, ids):
    return all(i in set(sel.tolist()) for i in ids)


# ---- known answers (kvmem/tests/kvmem_store_test.cpp) -----------------------

def test_topk_mandatory_inside_budget():
    # :434-459: budget 4, sink 1; scores 2:100 3:90 4:80 8:-10 9:-20, mandatory {8, 9}
    s = np.zeros(10)
    s[2], s[3], s[4], s[8], s[9] = 100, 90, 80, -10, -20
    sel = O.pick_topk_blocks(s, 4, 1, 0, (), 10 * BT, BT, (8, 9))
    assert len(sel) == 4 and _has(sel, (0, 2, 8, 9)) and 3 not in sel


def test_topk_mandatory_overlap_and_recent_best_effort():
    # :462-478: budget 4, sink 2, recent 3, mandatory {0, 0, 5} -> {0, 1, 5, 9}
    sel = O.pick_topk_blocks(np.zeros(10), 4, 2, 3, (), 10 * BT, BT, (0, 0, 5))
    assert sel.tolist() == [0, 1, 5, 9]


def test_topk_mandatory_overflow_trims_newest():
    # :481-497: budget 4, sink 1, recent 2, mandatory {1, 2, 3, 4} -> {0, 2, 3, 4}
    sel = O.pick_topk_blocks(np.zeros(10), 4, 1, 2, (), 10 * BT, BT, (1, 2, 3, 4))
    assert sel.tolist() == [0, 2, 3, 4]


def test_media_groups_with_shared_boundary():
    # :1080-1107: two images sharing block 6 form one group 4..8
    ranges = [(4 * BT + 3, 6 * BT + 9), (6 * BT + 10, 9 * BT)]
    for mand in ((), (11,)):
        assert O.pick_topk_blocks(np.zeros(12), 6, 1, 0, ranges, 12 * BT, BT, mand).tolist() == [0, 4, 5, 6, 7, 8]
    ranges = [(2 * BT + 1, 4 * BT), (9 * BT, 11 * BT)]
    sel = O.pick_topk_blocks(np.zeros(12), 6, 1, 0, ranges, 12 * BT, BT, (11,)).tolist()
    assert (2 in sel) == (3 in sel) and 9 in sel and 10 in sel


def test_media_suffix_over_budget():
    # :1109-1130
    ranges = [(2 * BT + 1, 4 * BT), (6 * BT + 1, 8 * BT)]
    for mand in ((8, 9, 10, 11), (11, 8, 10, 9, 8), (7, 9, 10, 11), (3, 8, 9, 10, 11)):
        assert O.pick_topk_blocks(np.zeros(12), 6, 1, 0, ranges, 12 * BT, BT, mand).tolist() == [0, 6, 7, 9, 10, 11]
    with pytest.raises(O.OracleError):
        O.pick_topk_blocks(np.zeros(12), 6, 1, 0, [(2 * BT, 8 * BT)], 12 * BT, BT, (11,))


def test_media_group_is_the_transitive_union():
    # pages 1-2 and 2-4 share page 2; 6-7 is apart; page 5 is alone
    ranges = [(6 * BT, 8 * BT), (1 * BT, 3 * BT), (2 * BT + 5, 5 * BT)]
    for p in range(1, 5):
        assert O.media_group(p, 10, BT, ranges) == (1, 5)
    assert O.media_group(5, 10, BT, ranges) == (5, 6)
    assert O.media_group(7, 10, BT, ranges) == (6, 8)
    # a range past the last page is clipped; an empty range joins nothing
    assert O.media_group(9, 10, BT, [(9 * BT, 40 * BT), (3 * BT, 3 * BT)]) == (9, 10)
    assert O.media_group(3, 10, BT, [(3 * BT, 3 * BT)]) == (3, 4)


def test_grouped_pick_skips_groups_that_do_not_fit():
    # budget 4: page 7 (best) pulls its group 5..8 (3 pages) in; page 1 next;
    # the group 2..4 (second best page 3) no longer fits and is skipped
    s = np.array([0.0, 5, 1, 8, 1, 2, 2, 9, 0, 0])
    ranges = [(5 * BT, 8 * BT), (2 * BT, 5 * BT)]
    assert O.pick_scored_grouped(s, 4, (), ranges, BT).tolist() == [1, 5, 6, 7]
    # a mandatory page brings its whole group (2..4) and must fit; page 7's
    # group then no longer fits, page 1 takes the last place
    assert O.pick_scored_grouped(s, 4, (3,), ranges, BT).tolist() == [1, 2, 3, 4]
    with pytest.raises(O.OracleError):
        O.pick_scored_grouped(s, 2, (3,), ranges, BT)


def test_query_fixed_blocks_known_cases():
    # budget covering every page: all pages
    assert O.query_fixed_blocks(8, 8, 1, 2, (), 8 * BT, BT).tolist() == list(range(8))
    assert O.query_fixed_blocks(8, 0, 1, 2, (), 8 * BT, BT).tolist() == list(range(8))
    # sink 1, last media range's first page (with its group), mandatory,
    # then recent pages while they fit
    got = O.query_fixed_blocks(20, 6, 1, 4, [(3 * BT, 5 * BT)], 20 * BT, BT, (10,))
    assert got.tolist() == [0, 3, 4, 10, 18, 19]
    with pytest.raises(O.OracleError):
        O.query_fixed_blocks(20, 2, 1, 0, [(3 * BT, 5 * BT)], 20 * BT, BT)


# ---- against the reference's KvMemStore ------------------------------------

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="reference build (oracle/_ref) not present")


def _random_ranges(rng, total, pt):
    kind = rng.integers(0, 5)
    n = int(rng.integers(0, 5))
    ranges = []
    for _ in range(n):
        a = int(rng.integers(0, total + pt))
        b = a + int(rng.integers(-pt, 6 * pt))
        ranges.append((a, max(0, b)))
    if kind == 0:
        ranges.sort()
    elif kind == 1 and ranges:
        ranges.append((ranges[0][0] + 1, ranges[0][1] + 3 * pt))  # overlapping
    return ranges


def _random_case(rng):
    pt = int(rng.choice([1, 4, 16, 32]))
    n = int(rng.integers(1, 40))
    total = (n - 1) * pt + int(rng.integers(1, pt + 1))
    budget = int(rng.integers(0, n + 3))
    sink, recent = int(rng.integers(0, 4)), int(rng.integers(0, 6))
    mand = [int(x) for x in rng.integers(0, n, size=int(rng.integers(0, 5)))]
    scores = np.round(rng.normal(size=n) * 2) / 2 if rng.integers(0, 2) else rng.normal(size=n)
    return pt, n, total, budget, sink, recent, _random_ranges(rng, total, pt), mand, scores


def _both(f_oracle, f_ref):
    """Equal results, or both raise."""
    try:
        a = f_oracle()
    except O.OracleError:
        a = None
    try:
        b = f_ref()
    except O.OracleError:
        b = None
    assert (a is None) == (b is None), (a, b)
    if a is not None:
        assert a.tolist() == b.tolist()
    return a


@needs_ref
def test_media_group_matches_reference_picks():
    # the grouped pick of a single best page equals the reference's group
    rng = np.random.default_rng(7)
    for _ in range(300):
        pt, n, total, _, _, _, ranges, _, _ = _random_case(rng)
        p = int(rng.integers(0, n))
        b, e = O.media_group(p, n, pt, ranges)
        s = np.zeros(n)
        s[p] = 1.0
        got = O.ref_pick_scored_grouped(s, total, pt, ranges, e - b)
        assert got.tolist() == list(range(b, e))


@needs_ref
def test_query_fixed_blocks_vs_reference():
    rng = np.random.default_rng(11)
    for _ in range(600):
        pt, n, total, budget, sink, recent, ranges, mand, _ = _random_case(rng)
        _both(lambda: O.query_fixed_blocks(n, budget, sink, recent, ranges, total, pt, mand),
              lambda: O.ref_query_fixed_blocks(total, pt, budget, sink, recent, ranges, mand))


@needs_ref
def test_pick_scored_grouped_vs_reference():
    rng = np.random.default_rng(13)
    for _ in range(600):
        pt, n, total, budget, sink, recent, ranges, mand, scores = _random_case(rng)
        budget = max(1, budget)
        signed = bool(rng.integers(0, 2))
        if not signed:
            scores = np.abs(scores)
        _both(lambda: O.pick_scored_grouped(scores, budget, mand, ranges, pt, O.TIE_HIGHER_FIRST, signed),
              lambda: O.ref_pick_scored_grouped(scores, total, pt, ranges, budget, mand, signed))


@needs_ref
def test_pick_topk_blocks_vs_reference():
    rng = np.random.default_rng(17)
    for _ in range(600):
        pt, n, total, budget, sink, recent, ranges, mand, scores = _random_case(rng)
        _both(lambda: O.pick_topk_blocks(scores, budget, sink, recent, ranges, total, pt, mand),
              lambda: O.ref_pick_topk_blocks(scores, total, pt, budget, sink, recent, ranges, mand))


@needs_ref
def test_query_fixed_then_grouped_pick_vs_reference():
    # the recall path: pick_scored_blocks(scores, query_fixed_blocks(mandatory))
    rng = np.random.default_rng(19)
    for _ in range(400):
        pt, n, total, budget, sink, recent, ranges, mand, scores = _random_case(rng)
        budget = max(1, budget)
        try:
            fixed = O.ref_query_fixed_blocks(total, pt, budget, sink, recent, ranges, mand)
        except O.OracleError:
            continue
        _both(lambda: O.pick_scored_grouped(scores, budget, fixed, ranges, pt, O.TIE_HIGHER_FIRST, True),
              lambda: O.ref_pick_scored_grouped(scores, total, pt, ranges, budget, fixed, True))
