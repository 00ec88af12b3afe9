"""The C ABI's host-side page policies (kvr_media_page_groups,
kvr_query_fixed_pages, kvr_topk_fixed_pages, kvr_media_fixed_pages) against
the oracle and the reference suite's known answers.  No device work: these
run on the host before the device pick."""
import numpy as np
import pytest

import kvmem_amd as K
import oracle as O
from kvmem_amd import _capi
from test_oracle_policy import _random_case

BT = 32


def test_overlap_groups_match_scored_media_group():
    rng = np.random.default_rng(3)
    for _ in range(400):
        pt, n, total, _, _, _, ranges, _, _ = _random_case(rng)
        groups = K.media_page_groups(ranges, pt, total, n, _capi.MEDIA_OVERLAP)
        # disjoint, ascending, nonempty
        assert all(b < e for b, e in groups)
        assert all(groups[i][1] <= groups[i + 1][0] for i in range(len(groups) - 1))
        for p in range(n):
            inside = [(int(b), int(e)) for b, e in groups if b <= p < e]
            assert (inside[0] if inside else (p, p + 1)) == O.media_group(p, n, pt, ranges)


def test_in_order_groups_known_cases():
    # sorted ranges: one group each; a range starting inside the previous
    # group extends its end; past the history's end or empty: dropped
    ranges = [(2 * BT + 1, 4 * BT), (3 * BT, 6 * BT), (8 * BT, 9 * BT), (40 * BT, 41 * BT), (9 * BT, 9 * BT)]
    g = K.media_page_groups(ranges, BT, 12 * BT, 12, _capi.MEDIA_IN_ORDER)
    assert g.tolist() == [[2, 6], [8, 9]]
    # out of order: an earlier-starting range merges into the last group's end only
    g = K.media_page_groups([(5 * BT, 7 * BT), (1 * BT, 9 * BT)], BT, 12 * BT, 12, _capi.MEDIA_IN_ORDER)
    assert g.tolist() == [[5, 9]]


def _both(f_product, f_oracle):
    try:
        a = f_product()
    except K.KvrError as e:
        a = e.status
    try:
        b = f_oracle()
    except O.OracleError as e:
        b = {O.ERR_BUDGET: _capi.ERR_BUDGET, O.ERR_ARG: _capi.ERR_INVALID}[e.code]
    if isinstance(a, int) or isinstance(b, int):
        assert a == b, (a, b)
    else:
        assert a.tolist() == b.tolist()


def test_query_fixed_pages_vs_oracle():
    rng = np.random.default_rng(5)
    for _ in range(600):
        pt, n, total, budget, sink, recent, ranges, mand, _ = _random_case(rng)
        _both(lambda: K.query_fixed_pages(n, budget, sink, recent, ranges, pt, total, mand),
              lambda: O.query_fixed_blocks(n, budget, sink, recent, ranges, total, pt, mand))


def test_topk_fixed_pages_known_answers():
    # kvmem_store_test.cpp:462-478 and :481-497 (no scores involved when the
    # kept part fills the budget)
    assert K.topk_fixed_pages(10, 4, 2, 3, (0, 0, 5)).tolist() == [0, 1, 5, 9]
    assert K.topk_fixed_pages(10, 4, 1, 2, (1, 2, 3, 4)).tolist() == [0, 2, 3, 4]
    # :434-459: sink 1 + mandatory {8, 9}; the device fills one more page
    assert K.topk_fixed_pages(10, 4, 1, 0, (8, 9)).tolist() == [0, 8, 9]
    # everything fits: every page
    assert K.topk_fixed_pages(5, 5, 1, 1, ()).tolist() == list(range(5))
    assert K.topk_fixed_pages(5, 0, 1, 1, ()).tolist() == list(range(5))
    # ids past the history are ignored
    assert K.topk_fixed_pages(10, 4, 0, 0, (3, 77)).tolist() == [3]


def test_topk_fixed_pages_then_fill_is_the_ungrouped_pick():
    # the kept part, then the best remaining scores (higher id first) = the
    # oracle's pick_topk_ungrouped
    rng = np.random.default_rng(9)
    for _ in range(300):
        pt, n, total, budget, sink, recent, _, mand, scores = _random_case(rng)
        kept = K.topk_fixed_pages(n, budget, sink, recent, mand)
        if budget == 0 or n <= budget:
            assert kept.tolist() == list(range(n))
            continue
        filled = O.pick_scored_blocks(scores, budget, kept.tolist(), O.TIE_HIGHER_FIRST, signed_scores=True)
        assert filled.tolist() == O.pick_topk_ungrouped(scores, budget, sink, recent, mand).tolist()


def test_media_fixed_pages_known_answers():
    # kvmem_store_test.cpp:1109-1124: sink 1 and the last image (6, 7)
    # required, then mandatory pages newest first while they fit
    ranges = [(2 * BT + 1, 4 * BT), (6 * BT + 1, 8 * BT)]
    for mand in ((8, 9, 10, 11), (11, 8, 10, 9, 8), (3, 8, 9, 10, 11)):
        assert K.media_fixed_pages(12, 6, 1, ranges, BT, 12 * BT, mand).tolist() == [0, 6, 7, 9, 10, 11]
    # :1125-1130: a single image that cannot fit whole
    with pytest.raises(K.KvrError) as e:
        K.media_fixed_pages(12, 6, 1, [(2 * BT, 8 * BT)], BT, 12 * BT, (11,))
    assert e.value.status == _capi.ERR_BUDGET
    # :1080-1107: the shared-boundary image group 4..8 is required
    ranges = [(4 * BT + 3, 6 * BT + 9), (6 * BT + 10, 9 * BT)]
    assert K.media_fixed_pages(12, 6, 1, ranges, BT, 12 * BT, (11,)).tolist() == [0, 4, 5, 6, 7, 8]


def test_host_helpers_reject_bad_arguments():
    with pytest.raises(K.KvrError):
        K.query_fixed_pages(10, 4, 0, 0, (), BT, 10 * BT, (10,))  # mandatory outside the pages
    with pytest.raises(K.KvrError):
        K.media_page_groups([(0, 5)], 0, 10, 4)  # zero page tokens
