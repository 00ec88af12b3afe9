"""The oracle reproduces the golden vectors written from the reference's own
host library (tests/golden/make_golden.py).  CPU only; runs without the
reference sources."""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def test_recall_fp16_vectors():
    g = load("recall_fp16.npz")
    for x, out, ok in zip(g["x"], g["out"], g["ok"]):
        if ok:
            got = O.recall_fp16(float(x))
            assert np.float32(got).view(np.uint32) == np.float32(out).view(np.uint32), x
        else:
            with pytest.raises(O.OracleError):
                O.recall_fp16(float(x))


def test_frame_vectors():
    for row in json.load(open(os.path.join(GOLD, "frames.json"))):
        acc, bt, budget, sink, recent, fixed = row["args"]
        s, c, sm, tm = O.query_score_frame(acc, bt, budget, sink, recent, fixed)
        assert s.tolist() == row["starts"] and c.tolist() == row["counts"]
        assert sm.tolist() == row["score_mask"] and tm.tolist() == row["transport_mask"]


def test_summary_vectors():
    g = load("summaries.npz")
    layers, tokens, kvh, dim, pt = (int(v) for v in g["geometry"])
    w = kvh * dim
    for l in range(layers):
        _, m = O.page_summaries(g["k16"][l], O.FMT_F16, tokens, w, pt)
        assert np.array_equal(m.view(np.uint32), g["means16"][l].view(np.uint32))
    # binary32 rows through the prefill mean-K path: same sequential sums
    for l in range(layers):
        k = g["k32"][l]
        pages = (tokens + pt - 1) // pt
        for p in range(pages):
            rows = k[p * pt:min(tokens, (p + 1) * pt)]
            acc = np.zeros(w, np.float32)
            for r in rows:
                acc = (acc + r).astype(np.float32)
            mean = acc * (np.float32(1) / np.float32(len(rows)))
            assert np.array_equal(mean.view(np.uint32), g["means32"][l, p].view(np.uint32))


def test_score_vectors():
    g = load("scores.npz")
    i = 0
    while f"shape{i}" in g:
        pages, rows, dim, qh, kvh = (int(v) for v in g[f"shape{i}"])
        means = g[f"sums{i}"] * np.float32(0.25)
        lr = [rows, rows - 1 if rows > 1 else rows]
        for agg in (O.AGG_MEAN, O.AGG_MAX):
            for use_mask in (0, 1):
                got = O.page_softmax_scores(means, g[f"query{i}"], lr, qh, kvh, dim, agg,
                                            score_mask=g[f"mask{i}"] if use_mask else None)
                assert np.array_equal(got, g[f"s{i}_agg{agg}_mask{use_mask}"])
        i += 1
    assert i == 3


def test_layerwise_vectors():
    g = load("layerwise.npz")
    layers, layer, tokens, kvh, dim, pt, rows, qh = (int(v) for v in g["geometry"])
    _, m = O.page_summaries(g["keys"][layer], O.FMT_F16, tokens, kvh * dim, pt)
    got = O.page_softmax_scores(m[None], g["query"][None], [rows], qh, kvh, dim, O.AGG_MEAN)
    assert np.array_equal(got, g["scores"])


def test_pick_vectors():
    g = load("pick.npz")
    i = 0
    while f"scores{i}" in g:
        got = O.pick_scored_blocks(g[f"scores{i}"], int(g[f"budget{i}"][0]), g[f"mandatory{i}"].tolist(),
                                   O.TIE_HIGHER_FIRST)
        assert np.array_equal(got, g[f"picked{i}"])
        i += 1
    assert i >= 6


def test_single_layer_32k_full_size():
    """The 32768-token case end to end on the oracle: generated inputs hash to
    the recorded values, summaries hash equal, scores equal bit for bit, and
    both tie rules give the reference's top-16 (no exact ties here)."""
    g = json.load(open(os.path.join(GOLD, "single_layer_32k.json")))
    T, HQ, HKV, D, PT, K, seed = (g[k] for k in ("tokens", "query_heads", "kv_heads", "head_dim",
                                                 "page_tokens", "top_k", "seed"))
    W = HKV * D
    cscale = O.synth_uniform_f32(seed, 100, W, 0.5, 2.0)
    keys = O.synth_scaled_normal_f16(seed, 101, T, cscale)
    q16 = O.synth_normal_f16(seed, 103, HQ * D)
    assert hashlib.sha256(keys.tobytes()).hexdigest() == g["keys_sha256"]
    assert hashlib.sha256(q16.tobytes()).hexdigest() == g["query_sha256"]
    _, means = O.page_summaries(keys, O.FMT_F16, T, W, PT)
    assert hashlib.sha256(means.tobytes()).hexdigest() == g["means_sha256"]
    qf = q16.view(np.float16).astype(np.float32).reshape(1, 1, HQ, D)
    scores = O.page_softmax_scores(means[None], qf, [1], HQ, HKV, D, O.AGG_MAX)
    expect = np.array([float.fromhex(v) for v in g["scores"]])
    assert np.array_equal(scores, expect)
    for tie in (O.TIE_HIGHER_FIRST, O.TIE_LOWER_FIRST):
        assert O.pick_scored_blocks(scores, K, (), tie).tolist() == g["picked_higher_first"]
