"""Device page selection against the oracle: mandatory lists of any length
(inline, uploaded, or a device list; short and long rows), the device-side
budget check, media-grouped picks (KvMemStore::pick_scored_blocks with media
ranges, after query_fixed_blocks), the two-pass pick_topk_blocks
(pick_topk_ungrouped, then constrain_media), and one layer of recall with a
grouped policy."""
import numpy as np
import pytest

import kvmem_amd as K
import oracle as O
from kvmem_amd import _capi
from gpu_util import dev, host, zeros

pytestmark = pytest.mark.gpu
SEED = 42


def _scores(rng, n, ties=True, signed=False):
    s = rng.normal(size=n)
    if ties:
        s = np.round(s * 3) / 3
    return s if signed else np.abs(s)


def _pick(ctx, scores, k, mandatory=(), tie=K.TIE_LOWER_FIRST, signed=False):
    n = scores.shape[0]
    sel, cnt = zeros(k, np.uint32), zeros(1, np.uint32)
    ctx.select_topk(dev(scores), n, k, sel, cnt, mandatory=mandatory, tie_rule=tie, signed_scores=signed)
    ctx.check()
    c = int(host(cnt, np.uint32)[0])
    return host(sel, np.uint32)[:c]


@pytest.mark.parametrize("n,k,n_mand", [(1024, 150, 100), (4096, 300, 257), (16384, 2000, 1500), (40000, 600, 300)])
def test_long_mandatory_lists(ctx, n, k, n_mand):
    """More than 64 mandatory pages (uploaded), one-wave rows and
    workgroup rows with keys in LDS or re-read (the bitmap in dynamic LDS)."""
    rng = np.random.default_rng(n + k)
    s = _scores(rng, n)
    mand = [int(x) for x in rng.integers(0, n, size=n_mand)]
    for tie in (K.TIE_LOWER_FIRST, K.TIE_HIGHER_FIRST):
        got = _pick(ctx, s, k, mand, tie)
        assert np.array_equal(got, O.pick_scored_blocks(s, k, mand, tie))


def test_short_mandatory_lists_unchanged(ctx):
    rng = np.random.default_rng(1)
    s = _scores(rng, 512)
    mand = [5, 9, 9, 500]
    assert np.array_equal(_pick(ctx, s, 32, mand), O.pick_scored_blocks(s, 32, mand))


def test_device_fixed_list_and_budget_check(ctx):
    rng = np.random.default_rng(2)
    n, k, lanes = 2048, 64, 3
    s = np.concatenate([_scores(rng, n) for _ in range(lanes)])
    fixed = np.array([7, 7, 3000, 11, 1999, 0, 11], np.uint32)  # repeats and an id past the row
    sel, cnt = zeros(lanes * k, np.uint32), zeros(lanes, np.uint32)
    fd = dev(fixed)
    ctx.select_pages(dev(s), n, k, sel, cnt, policy=K.make_policy(fixed=fd, n_fixed=len(fixed)), lanes=lanes)
    ctx.check()
    got, c = host(sel, np.uint32).reshape(lanes, k), host(cnt, np.uint32)
    for lane in range(lanes):
        expect = O.pick_scored_blocks(s[lane * n:(lane + 1) * n], k, [0, 7, 11, 1999])
        assert np.array_equal(got[lane][: c[lane]], expect)
    # more distinct fixed pages than the budget: empty selection, KVR_ERR_BUDGET
    over = dev(np.arange(0, 2 * (k + 1), 2, dtype=np.uint32))  # k + 1 distinct pages
    ctx.select_pages(dev(s), n, k, sel, cnt, policy=K.make_policy(fixed=over, n_fixed=k + 1), lanes=lanes)
    assert ctx.status() == _capi.ERR_BUDGET
    assert (host(cnt, np.uint32) == 0).all()
    ctx.check()


def _random_policy_case(rng):
    pt = int(rng.choice([16, 64, 256]))
    n = int(rng.integers(2, 4097))
    total = (n - 1) * pt + int(rng.integers(1, pt + 1))
    budget = int(rng.integers(1, max(2, n // 3)))
    sink, recent = int(rng.integers(0, 3)), int(rng.integers(0, 8))
    ranges = []
    for _ in range(int(rng.integers(0, 12))):
        a = int(rng.integers(0, total))
        ranges.append((a, a + int(rng.integers(1, 12 * pt))))
    if rng.integers(0, 2):
        ranges.sort()
    mand = [int(x) for x in rng.integers(0, n, size=int(rng.integers(0, 6)))]
    return pt, n, total, budget, sink, recent, ranges, mand


def test_grouped_pick_after_query_fixed_pages(ctx):
    """The recall path's pick_scored_blocks(scores, query_fixed_blocks(m)) with
    media groups, against the oracle, on rows of up to 4096 pages."""
    rng = np.random.default_rng(SEED)
    done = 0
    while done < 40:
        pt, n, total, budget, sink, recent, ranges, mand = _random_policy_case(rng)
        try:
            fixed = K.query_fixed_pages(n, budget, sink, recent, ranges, pt, total, mand)
        except K.KvrError:
            continue
        groups = K.media_page_groups(ranges, pt, total, n, _capi.MEDIA_OVERLAP)
        signed = bool(rng.integers(0, 2))
        s = _scores(rng, n, signed=signed)
        for tie in (K.TIE_HIGHER_FIRST, K.TIE_LOWER_FIRST):
            expect = O.pick_scored_grouped(s, budget, fixed.tolist(), ranges, pt, tie, signed)
            k = budget
            sel, cnt = zeros(k, np.uint32), zeros(1, np.uint32)
            fd = dev(fixed if len(fixed) else np.zeros(1, np.uint32))
            gd = dev(groups.ravel() if len(groups) else np.zeros(2, np.uint32))
            pol = K.make_policy(fixed=fd, n_fixed=len(fixed), groups=gd, n_groups=len(groups))
            ctx.select_pages(dev(s), n, k, sel, cnt, policy=pol, tie_rule=tie, signed_scores=signed)
            ctx.check()
            got = host(sel, np.uint32)[: int(host(cnt, np.uint32)[0])]
            assert np.array_equal(got, expect), (n, budget, ranges, fixed.tolist())
        done += 1


def test_pick_topk_blocks_two_passes(ctx):
    """pick_topk_blocks on the device: the ungrouped pick (host kept pages +
    device fill), then constrain_media (host kept pages + a grouped device
    pick with the first pass's pages preferred), against the oracle."""
    rng = np.random.default_rng(7)
    done = 0
    while done < 40:
        pt, n, total, budget, sink, recent, ranges, mand = _random_policy_case(rng)
        s = _scores(rng, n, signed=True)
        try:
            expect = O.pick_topk_blocks(s, budget, sink, recent, ranges, total, pt, mand)
        except O.OracleError:
            continue
        kept = K.topk_fixed_pages(n, budget, sink, recent, mand)
        sel1, cnt1 = zeros(budget, np.uint32), zeros(1, np.uint32)
        kd = dev(kept)
        sd = dev(s)
        ctx.select_pages(sd, n, budget, sel1, cnt1, policy=K.make_policy(fixed=kd, n_fixed=len(kept)),
                         tie_rule=K.TIE_HIGHER_FIRST, signed_scores=True)
        first = O.pick_topk_ungrouped(s, budget, sink, recent, mand)
        ctx.check()
        assert np.array_equal(host(sel1, np.uint32)[: int(host(cnt1, np.uint32)[0])], first)
        if ranges and n > budget:
            fixed2 = K.media_fixed_pages(n, budget, sink, ranges, pt, total, mand)
            groups = K.media_page_groups(ranges, pt, total, n, _capi.MEDIA_IN_ORDER)
            sel2, cnt2 = zeros(budget, np.uint32), zeros(1, np.uint32)
            f2 = dev(fixed2 if len(fixed2) else np.zeros(1, np.uint32))
            g2 = dev(groups.ravel() if len(groups) else np.zeros(2, np.uint32))
            pol = K.make_policy(fixed=f2, n_fixed=len(fixed2), groups=g2, n_groups=len(groups), preferred=sel1,
                                preferred_count=cnt1, preferred_stride=budget)
            ctx.select_pages(sd, n, budget, sel2, cnt2, policy=pol, tie_rule=K.TIE_HIGHER_FIRST, signed_scores=True)
            ctx.check()
            got = host(sel2, np.uint32)[: int(host(cnt2, np.uint32)[0])]
        else:
            got = first
        assert np.array_equal(got, expect), (n, budget, sink, recent, ranges, mand)
        done += 1


def test_recall_layer_with_groups_and_long_mandatory(ctx):
    """One layer end to end (summaries -> scores -> grouped pick), then the
    fused tail with an uploaded mandatory list, in a layer and in a stack."""
    T, HQ, HKV, D, PT, KSEL = 65536, 32, 8, 128, 256, 48
    W, P = HKV * D, T // PT
    keys = O.synth_normal_f16(SEED, 700, T * W)
    q = O.synth_normal_f32(SEED, 701, HQ * D)
    _, means = O.page_summaries(keys, O.FMT_F16, T, W, PT)
    expect_scores = O.page_softmax_scores(means[None], q.reshape(1, 1, HQ, D), [1], HQ, HKV, D, O.AGG_MEAN)
    kd, qd = dev(keys), dev(q)
    ranges = [(10 * PT + 5, 14 * PT), (13 * PT, 20 * PT), (100 * PT, 103 * PT)]
    fixed = K.query_fixed_pages(P, KSEL, 1, 4, ranges, PT, T, (50,))
    groups = K.media_page_groups(ranges, PT, T, P, _capi.MEDIA_OVERLAP)
    fd, gd = dev(fixed), dev(groups.ravel())

    def run(k, policy=None, mandatory=()):
        s16, sc = zeros(P * W, np.uint16), zeros(P, np.float64)
        sel, cnt = zeros(k, np.uint32), zeros(1, np.uint32)
        ctx.recall_layer(keys=K.make_keys(kd, K.FMT_F16, T, HKV, D, PT), summaries=s16,
                         query=K.make_query(qd, K.FMT_F32, 1, HQ, HKV, D), scores=sc, selected=sel, count=cnt,
                         k=k, tie_rule=K.TIE_HIGHER_FIRST, policy=policy, mandatory=mandatory)
        ctx.check()
        got_s = host(sc, np.float64)
        assert float(np.max(np.abs(got_s - expect_scores) / expect_scores)) <= 1e-9
        return got_s, host(sel, np.uint32)[: int(host(cnt, np.uint32)[0])]

    # media groups: the selection is its own launch after the softmax
    got_s, got = run(KSEL, K.make_policy(fixed=fd, n_fixed=len(fixed), groups=gd, n_groups=len(groups)))
    assert np.array_equal(got, O.pick_scored_grouped(got_s, KSEL, fixed.tolist(), ranges, PT, O.TIE_HIGHER_FIRST))
    # 80 distinct mandatory pages (> 64: uploaded), budget 96, fused tail
    mand = list(range(0, 160, 2))
    got_s, got = run(96, mandatory=mand)
    assert np.array_equal(got, O.pick_scored_blocks(got_s, 96, mand, O.TIE_HIGHER_FIRST))
    # a stack of five layers, each with its own long list (one upload)
    descs, outs = [], []
    for layer in range(5):
        lm = [int(x) for x in range(layer, layer + 3 * 70, 3)]
        sc, sel, cnt = zeros(P, np.float64), zeros(96, np.uint32), zeros(1, np.uint32)
        descs.append(ctx.layer_recall(keys=K.make_keys(kd, K.FMT_F16, T, HKV, D, PT),
                                      summaries=zeros(P * W, np.uint16),
                                      query=K.make_query(qd, K.FMT_F32, 1, HQ, HKV, D), scores=sc, selected=sel,
                                      count=cnt, k=96, tie_rule=K.TIE_HIGHER_FIRST, mandatory=lm))
        outs.append((lm, sc, sel, cnt))
    arr = ctx.recall_stack(descs)
    ctx.check()
    for lm, sc, sel, cnt in outs:
        got_s = host(sc, np.float64)
        assert float(np.max(np.abs(got_s - expect_scores) / expect_scores)) <= 1e-9
        got = host(sel, np.uint32)[: int(host(cnt, np.uint32)[0])]
        assert np.array_equal(got, O.pick_scored_blocks(got_s, 96, lm, O.TIE_HIGHER_FIRST))
    del arr
