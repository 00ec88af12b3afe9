"""The oracle against known answers and closed forms (CPU only).

Known answers restate the reference's own tests (cited); closed forms come
from the mathematics (softmax of hand-computed logits, exact block products,
brute-force ranking), chosen so that a dropped term, a swapped index or a
wrong tie direction fails at least one of them.
"""
import math

import numpy as np
import pytest

import oracle as O


def close(a, b, tol=1e-12):
    assert abs(a - b) <= tol, (a, b)


# ---- fp16 boundary ---------------------------------------------------------
def test_recall_fp16_known_answers():
    """graph_recall_test.cpp:57-61."""
    close(O.recall_fp16(1.00048828125), 1.0)
    close(O.recall_fp16(1.00146484375), 1.001953125)
    close(O.recall_fp16(2.0 ** -24), 2.0 ** -24)
    close(O.recall_fp16(2.0 ** -25), 0.0)
    with pytest.raises(O.OracleError) as e:
        O.recall_fp16(65536.0)
    assert e.value.code == O.ERR_RANGE
    with pytest.raises(O.OracleError) as e:
        O.recall_fp16(float("nan"))
    assert e.value.code == O.ERR_NONFINITE
    close(O.recall_fp16(65519.0), 65504.0)
    with pytest.raises(O.OracleError):
        O.recall_fp16(65520.0)


def test_f16_conversions_exhaustive():
    """Every binary16 value survives f16 -> f32 -> f16, decodes like numpy's
    IEEE conversion, and every midpoint between neighbours rounds to even."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    as32 = np.array([O.lib.orc_f16_to_f32(int(b)) for b in bits], np.float32)
    ref = bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(as32[finite].view(np.uint32), ref[finite].view(np.uint32))
    back = O.f32_to_f16_bits(as32[finite])
    assert np.array_equal(back, bits[finite])
    # midpoints of consecutive positive finite halves (0x0000..0x7bff)
    lo = np.arange(0, 0x7bff, dtype=np.uint16).view(np.float16).astype(np.float64)
    hi = np.arange(1, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)  # exact in binary32
    got = O.f32_to_f16_bits(mid)
    expect = mid.astype(np.float16).view(np.uint16)  # numpy rounds to nearest even
    assert np.array_equal(got, expect)
    assert np.all(got % 2 == 0)


# ---- frames ------------------------------------------------------------------
def test_query_score_frame_known_answers():
    """graph_recall_test.cpp:23-31."""
    _, _, sm, tm = O.query_score_frame(12, 4, 2, 0, 0, [2])
    assert sm.tolist() == [1, 1, 1] and tm.tolist() == [1, 1, 0]
    _, counts, sm, tm = O.query_score_frame(11, 4, 4, 1, 1, [0, 2])
    assert sm.tolist() == [1, 1, 1] and tm.tolist() == [0, 0, 0] and counts[-1] == 3
    _, _, sm, _ = O.query_score_frame(12, 4, 2, 1, 1, [0, 2])
    assert sm.tolist() == [0, 1, 0]


# ---- page summaries ----------------------------------------------------------
def test_summary_sequential_sum_closed_form():
    """Integer-valued fp16 keys: every partial sum is exact, so the mean is
    sum/n exactly; a ragged last page divides by its own count."""
    tokens, w, pt = 10, 32, 4
    vals = (np.arange(tokens * w) % 7 - 3).astype(np.float16).reshape(tokens, w)
    sums, means = O.page_summaries(vals.view(np.uint16), O.FMT_F16, tokens, w, pt)
    v = vals.astype(np.float64)
    for p, (a, b) in enumerate(((0, 4), (4, 8), (8, 10))):
        assert np.array_equal(sums[p], v[a:b].sum(0))
        assert np.array_equal(means[p], (v[a:b].sum(0) * np.float32(1.0 / (b - a))).astype(np.float32))


def test_summary_order_is_token_order():
    """Rows [2^-10, 60000, -60000]: summed in token order the 2^-10 is lost
    against 60000 (binary32 ulp 2^-8) and the page sums to 0; summed in
    reverse (or with the large pair first) it survives as 2^-10."""
    w = 32
    rows = np.zeros((3, w), np.float16)
    rows[0, :] = 0.0009765625
    rows[1, :] = 60000.0
    rows[2, :] = -60000.0
    sums, means = O.page_summaries(rows.view(np.uint16), O.FMT_F16, 3, w, 3)
    assert np.all(sums[0] == 0.0)
    rev = np.float32(np.float32(np.float32(-60000.0) + np.float32(60000.0)) + np.float32(0.0009765625))
    assert rev == np.float32(0.0009765625)


def test_q8_0_summary_uses_exact_products():
    w, tokens = 64, 3
    blk = np.zeros((tokens, w // 32, 34), np.uint8)
    d = np.float16(0.03125)
    for t in range(tokens):
        for b in range(w // 32):
            blk[t, b, :2] = np.frombuffer(d.tobytes(), np.uint8)
            blk[t, b, 2:] = (np.arange(32) - 16 + t).astype(np.int8).view(np.uint8)
    sums, means = O.page_summaries(blk.ravel(), O.FMT_Q8_0, tokens, w, 4)
    q = np.array([(np.arange(32) - 16 + t) for t in range(tokens)], np.float64)
    expect = np.tile(q.sum(0) * 0.03125, 2)
    assert np.array_equal(sums[0], expect.astype(np.float32))


# ---- page softmax ------------------------------------------------------------
def _three_page_case():
    # RawKvStore({1,2,0,4}); sums {8,0},{0,4},{40,0} over 4 tokens -> means /4
    means = np.array([[[2, 0], [0, 1], [10, 0]]], np.float32)
    query = np.array([[[[2, 0]], [[0, 2]]]], np.float32)  # rows 2, Hq 1, D 2
    return means, query


def test_mean_softmax_known_answer():
    """graph_recall_test.cpp:32-56 with its long-double reference."""
    means, query = _three_page_case()
    got = O.page_softmax_scores(means, query, [2], 1, 1, 2, O.AGG_MEAN)
    s2 = math.sqrt(2)
    expect = np.zeros(3)
    for line in ([4 / s2, 0, 20 / s2], [0, 2 / s2, 0]):
        e = np.exp(np.array(line, np.longdouble))
        expect += (e / e.sum()).astype(np.float64)
    for i in range(3):
        close(got[i], expect[i])
    assert got[1] > got[0]
    close(got.sum(), 2.0)
    masked = O.page_softmax_scores(means, query, [2], 1, 1, 2, O.AGG_MEAN, score_mask=np.array([1, 1, 0]))
    assert masked[0] > masked[1] and masked[2] == 0
    empty = O.page_softmax_scores(means, query, [2], 1, 1, 2, O.AGG_MEAN, score_mask=np.zeros(3))
    assert np.all(empty == 0)


def test_gqa_two_layers_and_large_domains():
    """graph_recall_test.cpp:63-84."""
    means = np.array([[[1], [-1]], [[1], [-1]]], np.float32)
    query = np.array([[[[1], [-1]]], [[[2], [-2]]]], np.float32)
    got = O.page_softmax_scores(means, query, [1, 1], 2, 1, 1, O.AGG_MEAN)
    close(got[0], 0.5)
    close(got[1], 0.5)
    for n in (8192, 8193, 32768, 32769):
        m = np.ones((1, n, 1), np.float32)
        s = O.page_softmax_scores(m, np.ones((1, 1, 1, 1), np.float32), [1], 1, 1, 1, O.AGG_MEAN)
        close(s[0], 1 / n)
        close(s[-1], 1 / n)
        close(s.sum(), 1.0, 2e-12)


def test_max_aggregation_closed_form():
    """graph_recall_test.cpp:85-96: mirrored head distributions."""
    means = np.array([[[1, 0], [0, 1], [-1, -1]]], np.float32)
    query = np.array([[[[2, 0], [0, 2]], [[2, 0], [0, 2]]]], np.float32)  # rows 2, Hq 2, Hkv 1
    got = O.page_softmax_scores(means, query, [2], 2, 1, 2, O.AGG_MAX)
    a, b, c = math.exp(math.sqrt(2)), 1.0, math.exp(-math.sqrt(2))
    maximum, negative = a / (a + b + c), c / (a + b + c)
    mass = 2 * maximum + negative
    close(got[0], 2 * maximum / mass)
    close(got[1], 2 * maximum / mass)
    close(got[2], 2 * negative / mass)


def test_max_logit_variant_closed_form():
    """Literal 'max over the group's logits, then softmax': head logits (1, 0)
    and (0, 2) give group logits (1, 2) -> softmax (e, e^2)/(e + e^2); the
    max-of-probabilities rule gives a different answer on the same input."""
    means = np.array([[[1, 0], [0, 1]]], np.float32)
    query = np.array([[[[1, 0], [0, 2]]]], np.float32)
    got = O.page_softmax_scores(means, query, [1], 2, 1, 2, O.AGG_MAX_LOGIT, scale=1.0)
    e1, e2 = math.e, math.e ** 2
    close(got[0], e1 / (e1 + e2))
    close(got[1], e2 / (e1 + e2))
    other = O.page_softmax_scores(means, query, [1], 2, 1, 2, O.AGG_MAX, scale=1.0)
    assert abs(other[0] - got[0]) > 1e-3


def test_logit_head_to_group_mapping():
    """Query head h reads kv-head h // (Hq/Hkv): swapping the two kv-heads'
    summaries must swap which heads see the large logit."""
    means = np.zeros((1, 1, 4), np.float32)
    means[0, 0, :2] = [1, 0]   # kv-head 0
    means[0, 0, 2:] = [0, 3]   # kv-head 1
    query = np.zeros((1, 4, 2), np.float32)  # rows 1, Hq 4, D 2
    query[:, :, :] = [1, 1]
    lg = O.page_logits(means[0], query, 4, 2, 2, scale=1.0)
    assert lg[:, 0].tolist() == [1.0, 1.0, 3.0, 3.0]


# ---- selection ---------------------------------------------------------------
def _brute(scores, budget, mandatory, higher_first):
    kept = list(dict.fromkeys(mandatory))
    key = (lambda i: (-scores[i], -i)) if higher_first else (lambda i: (-scores[i], i))
    for i in sorted(range(len(scores)), key=key):
        if len(kept) >= budget:
            break
        if i not in kept:
            kept.append(i)
    return sorted(kept)


def test_pick_brute_force_and_ties():
    rng = np.random.default_rng(3)
    for trial in range(200):
        n = int(rng.integers(1, 40))
        budget = int(rng.integers(1, 45))
        s = rng.integers(0, 5, n).astype(np.float64) / 4  # heavy ties
        mand = [int(x) for x in rng.choice(n, min(n, int(rng.integers(0, 3))), replace=False)]
        if len(mand) > budget:
            mand = mand[:budget]
        for tie, hf in ((O.TIE_LOWER_FIRST, False), (O.TIE_HIGHER_FIRST, True)):
            assert O.pick_scored_blocks(s, budget, mand, tie).tolist() == _brute(s, budget, mand, hf)


def test_pick_tie_rule_known_answer():
    """layerwise_selection_test.cpp:184-194: equal mass over six pages, budget 2."""
    eq = np.full(6, 1 / 6)
    assert O.pick_scored_blocks(eq, 2, (), O.TIE_HIGHER_FIRST).tolist() == [4, 5]
    assert O.pick_scored_blocks(eq, 2, (), O.TIE_LOWER_FIRST).tolist() == [0, 1]


def test_pick_rejections():
    """graph_recall_test.cpp:101-105 and kvmem_store.cpp:425-437."""
    s = np.array([-.8, -.2, -.5])
    assert O.pick_scored_blocks(s, 2, (), O.TIE_HIGHER_FIRST, signed_scores=True).tolist() == [1, 2]
    with pytest.raises(O.OracleError):
        O.pick_scored_blocks(s, 2)
    with pytest.raises(O.OracleError) as e:
        O.pick_scored_blocks(np.ones(5), 1, (0, 1))
    assert e.value.code == O.ERR_BUDGET
    with pytest.raises(O.OracleError):
        O.pick_scored_blocks(np.ones(5), 0)


# ---- block formats and gather ------------------------------------------------
def test_q8_0_dequant_closed_form():
    d = np.float16(0.0213)
    qs = (np.arange(32) * 8 - 128).astype(np.int8)
    blk = np.concatenate([np.frombuffer(d.tobytes(), np.uint8), qs.view(np.uint8)])
    y = O.dequant_q8_0(blk)
    assert np.array_equal(y, qs.astype(np.float32) * np.float32(d))


def test_q4_1_dequant_closed_form():
    d, m = np.float16(0.0377), np.float16(-0.311)
    nib = np.arange(32) % 16
    qs = (nib[:16] | (nib[16:] << 4)).astype(np.uint8)  # low nibble -> j, high -> j+16
    blk = np.concatenate([np.frombuffer(d.tobytes(), np.uint8), np.frombuffer(m.tobytes(), np.uint8), qs])
    y = O.dequant_q4_1(blk)
    expect = (nib.astype(np.float32) * np.float32(d)).astype(np.float32) + np.float32(m)
    assert np.array_equal(y, expect.astype(np.float32))


def test_q8_0_quant_closed_form():
    k = np.arange(-127, 128, 8).astype(np.float32)
    x = np.zeros(32, np.float32)
    x[: k.size] = k * np.float32(0.5)
    x[31] = np.float32(127 * 0.5)
    blk = O.quant_q8_0(x)
    assert np.frombuffer(blk[:2].tobytes(), np.float16)[0] == np.float16(0.5)
    q = blk[2:].view(np.int8).astype(np.float32)
    assert np.array_equal(q, x * 2)
    zero = O.quant_q8_0(np.zeros(32, np.float32))
    assert np.all(zero == 0)


def test_gather_layout():
    """Slot i holds page selected[i] (ascending ids), valid rows only."""
    tokens, w, pt = 10, 32, 4  # pages: [0,4) [4,8) [8,10)
    hist = (np.arange(tokens * w) % 251).astype(np.uint16)
    slots = O.gather(hist.view(np.uint8), O.FMT_F16, w, tokens, pt, [0, 2], O.GATHER_COPY,
                     slots=np.full(2 * pt * w * 2, 0xEE, np.uint8))
    sl = slots.view(np.uint16).reshape(2 * pt, w)
    h = hist.reshape(tokens, w)
    assert np.array_equal(sl[0:4], h[0:4])
    assert np.array_equal(sl[4:6], h[8:10])
    assert np.all(sl[6:8] == 0xEEEE)
    with pytest.raises(O.OracleError):
        O.gather(hist.view(np.uint8), O.FMT_F16, w, tokens, pt, [2, 0], O.GATHER_COPY)


def test_synth_moments():
    """The shared generator's normals: Box-Muller pairs (normals 2j, 2j+1 =
    R cos, R sin of 2 pi u2 from draws 2j, 2j+1), its ln, sqrt, sin and cos
    built from +, -, *, / only.  Checked against numpy's log, sqrt, cos and
    sin on the same 53-bit uniforms (a wrong series term, reduction,
    quadrant or draw index fails it), then N(0,1) by moments, tails and a
    Kolmogorov-Smirnov test."""
    from scipy import stats
    n = 200_000
    x = O.synth_normal_f32(1, 2, n).astype(np.float64)
    pairs = 2000
    r1 = np.array([O.lib.orc_synth_bits(1, 2, 2 * j) for j in range(pairs)], np.uint64)
    r2 = np.array([O.lib.orc_synth_bits(1, 2, 2 * j + 1) for j in range(pairs)], np.uint64)
    u1 = ((r1 >> np.uint64(11)) + np.uint64(1)).astype(np.float64) * 2.0 ** -53
    u2 = (r2 >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    radius = np.sqrt(-2 * np.log(u1))
    want = np.empty(2 * pairs)
    want[0::2] = radius * np.cos(2 * np.pi * u2)
    want[1::2] = radius * np.sin(2 * np.pi * u2)
    np.testing.assert_allclose(x[:2 * pairs], want, rtol=1e-6, atol=1e-7)
    # every quarter turn is hit (the sign pattern of cos and sin)
    quarter = (u2 * 4).astype(int)
    assert set(quarter.tolist()) == {0, 1, 2, 3}
    assert abs(x.mean()) < 0.01 and abs(x.var() - 1) < 0.01
    assert 0.0022 < np.mean(np.abs(x) > 3) < 0.0033  # 2 * (1 - Phi(3)) = 0.0027
    assert stats.kstest(x, "norm").pvalue > 1e-3
    u = O.synth_uniform_f32(1, 3, 100_000, 0.5, 2.0)
    assert u.min() >= 0.5 and u.max() < 2.0 and abs(u.mean() - 1.25) < 0.01
    q = O.synth_q8_0(1, 4, 1000, 0.01, 0.05).reshape(1000, 34)
    codes = q[:, 2:].view(np.int8)
    assert codes.min() == -127 and codes.max() == 127
