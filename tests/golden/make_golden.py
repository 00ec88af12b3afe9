#!/usr/bin/env python3
"""Write the golden vectors under tests/golden/ from the reference's own
host library (oracle/_ref/libkvmem_ref.so, compiled from the reference
sources by oracle/Makefile).  Run in a container that has the reference
build; the committed .npz/.json files are data only (inputs + expected
outputs), loadable without it:

    make -C oracle ref && python tests/golden/make_golden.py

Fixtures
  recall_fp16.npz      recall_fp16 on boundary and random binary32 values
  frames.json          query_score_frame on small frames
  summaries.npz        mean_k of fp16 and binary32 key rows (ragged pages)
  scores.npz           page_softmax_scores Mean/Max on small explicit inputs
  layerwise.npz        layerwise_mean_key_scores (single-layer current Q)
  pick.npz             KvMemStore::pick_scored_blocks with ties and pins
  single_layer_32k.json  the 32768-token single-layer case at full size:
                       generator seed, sha256 of the generated K and Q bytes,
                       reference scores (Max aggregation) and top-16 pages
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle as O  # noqa: E402

SEED = 42


def recall_vectors():
    rng = np.random.default_rng(SEED)
    special = np.array([1.00048828125, 1.00146484375, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.5,
                        65504.0, 65519.99, 65520.0, 65536.0, -65519.0, 6.1035156e-05, 6.0975552e-05,
                        5.9604645e-08, -2.9802322e-08, 0.0, -0.0, 1e-30, -1e-30, np.inf, -np.inf, np.nan],
                       np.float32)
    rnd = np.concatenate([rng.standard_normal(3000).astype(np.float32),
                          (rng.standard_normal(1000) * 1e-5).astype(np.float32),
                          (rng.standard_normal(1000) * 3e4).astype(np.float32)])
    x = np.concatenate([special, rnd])
    out = np.zeros_like(x)
    ok = np.zeros(x.size, np.uint8)
    for i, v in enumerate(x):
        try:
            out[i] = O.ref_recall_fp16(float(v))
            ok[i] = 1
        except O.OracleError:
            ok[i] = 0
    np.savez(os.path.join(HERE, "recall_fp16.npz"), x=x, out=out, ok=ok)


def frame_vectors():
    cases = [(12, 4, 2, 0, 0, [2]), (11, 4, 4, 1, 1, [0, 2]), (12, 4, 2, 1, 1, [0, 2]),
             (1000, 64, 4, 2, 3, []), (5, 1, 10, 0, 0, []), (256, 256, 1, 0, 0, [0])]
    rows = []
    for acc, bt, budget, sink, recent, fixed in cases:
        s, c, sm, tm = O.query_score_frame(acc, bt, budget, sink, recent, fixed, use_ref=True)
        rows.append(dict(args=[acc, bt, budget, sink, recent, fixed], starts=s.tolist(), counts=c.tolist(),
                         score_mask=sm.tolist(), transport_mask=tm.tolist()))
    json.dump(rows, open(os.path.join(HERE, "frames.json"), "w"), indent=0)


def summary_vectors():
    layers, tokens, kvh, dim, pt = 2, 300, 2, 16, 128
    w = kvh * dim
    k16 = O.synth_normal_f16(SEED, 500, layers * tokens * w).reshape(layers, tokens, w)
    m16, _ = O.ref_scores_f16_keys(k16, tokens, kvh, dim, pt, np.zeros((layers, 1, 4, dim), np.float32),
                                   [1, 1], 4, O.AGG_MEAN, want_scores=False)
    k32 = O.synth_normal_f32(SEED, 501, layers * tokens * w).reshape(layers, tokens, w)
    m32, _ = O.ref_scores_f32_keys(k32, tokens, kvh, dim, pt, np.zeros((layers, 1, 4, dim), np.float32),
                                   [1, 1], 4, O.AGG_MEAN)
    np.savez(os.path.join(HERE, "summaries.npz"), k16=k16, means16=m16, k32=k32, means32=m32,
             geometry=np.array([layers, tokens, kvh, dim, pt]))


def score_vectors():
    out = {}
    shapes = [(9, 3, 16, 8, 2), (40, 2, 32, 4, 4), (17, 1, 8, 6, 3)]
    for i, (pages, rows, dim, qh, kvh) in enumerate(shapes):
        w = kvh * dim
        sums = (O.synth_normal_f32(SEED, 600 + i, 2 * pages * w) * np.float32(4)).reshape(2, pages, w)
        query = O.synth_normal_f32(SEED, 700 + i, 2 * rows * qh * dim).reshape(2, rows, qh, dim)
        mask = (np.arange(pages) % 5 != 1).astype(np.uint8)
        for agg in (O.AGG_MEAN, O.AGG_MAX):
            for use_mask in (0, 1):
                s = O.ref_scores_from_sums(sums, kvh, dim, 4, query, [rows, rows - 1 if rows > 1 else rows],
                                           qh, agg, score_mask=mask if use_mask else None)
                out[f"s{i}_agg{agg}_mask{use_mask}"] = s
        out[f"sums{i}"] = sums
        out[f"query{i}"] = query
        out[f"mask{i}"] = mask
        out[f"shape{i}"] = np.array([pages, rows, dim, qh, kvh])
    np.savez(os.path.join(HERE, "scores.npz"), **out)


def layerwise_vectors():
    layers, tokens, kvh, dim, pt, rows, qh = 2, 640, 2, 32, 128, 3, 8
    w = kvh * dim
    keys = O.synth_normal_f16(SEED, 800, layers * tokens * w).reshape(layers, tokens, w)
    q = O.synth_normal_f32(SEED, 801, rows * qh * dim).reshape(rows, qh, dim)
    s = O.ref_layerwise_scores_f16_keys(keys, 1, tokens, kvh, dim, pt, q, qh)
    np.savez(os.path.join(HERE, "layerwise.npz"), keys=keys, query=q, scores=s,
             geometry=np.array([layers, 1, tokens, kvh, dim, pt, rows, qh]))


def pick_vectors():
    rng = np.random.default_rng(SEED)
    out = {}
    cases = [(6, 2, ()), (300, 20, (5, 17)), (300, 20, ()), (1000, 64, (0, 999, 500)), (50, 50, (1,)),
             (7, 3, (6,))]
    for i, (n, budget, mand) in enumerate(cases):
        s = rng.random(n)
        if i == 0:
            s[:] = 1.0 / 6
        else:
            s[rng.choice(n, n // 4)] = s[0]
        out[f"scores{i}"] = s
        out[f"budget{i}"] = np.array([budget])
        out[f"mandatory{i}"] = np.array(mand, np.uint32)
        out[f"picked{i}"] = O.ref_pick_scored_blocks(s, budget, mand)
    np.savez(os.path.join(HERE, "pick.npz"), **out)


def single_layer_32k():
    T, HQ, HKV, D, PT, K = 32768, 32, 8, 128, 256, 16
    W = HKV * D
    cscale = O.synth_uniform_f32(SEED, 100, W, 0.5, 2.0)
    keys = O.synth_scaled_normal_f16(SEED, 101, T, cscale)
    q16 = O.synth_normal_f16(SEED, 103, HQ * D)
    qf = q16.view(np.float16).astype(np.float32).reshape(1, 1, HQ, D)
    means, scores = O.ref_scores_f16_keys(keys.reshape(1, T, W), T, HKV, D, PT, qf, [1], HQ, O.AGG_MAX)
    picked = O.ref_pick_scored_blocks(scores, K)
    doc = dict(
        tokens=T, query_heads=HQ, kv_heads=HKV, head_dim=D, page_tokens=PT, top_k=K, seed=SEED,
        generator=dict(channel_scale="synth_uniform_f32(seed, 100, 1024, 0.5, 2.0)",
                       keys="synth_scaled_normal_f16(seed, 101, 32768, channel_scale)",
                       query="synth_normal_f16(seed, 103, 4096)"),
        keys_sha256=hashlib.sha256(keys.tobytes()).hexdigest(),
        query_sha256=hashlib.sha256(q16.tobytes()).hexdigest(),
        means_sha256=hashlib.sha256(means.tobytes()).hexdigest(),
        aggregation="max", scores=[float.hex(float(v)) for v in scores],
        picked_higher_first=picked.tolist())
    json.dump(doc, open(os.path.join(HERE, "single_layer_32k.json"), "w"), indent=1)


if __name__ == "__main__":
    if not O.ref_available():
        sys.exit("oracle/_ref is not built: make -C oracle ref")
    recall_vectors()
    frame_vectors()
    summary_vectors()
    score_vectors()
    layerwise_vectors()
    pick_vectors()
    single_layer_32k()
    print("golden vectors written to", HERE)
