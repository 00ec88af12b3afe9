"""The recall workloads at their full per-layer / per-lane sizes against the
oracle: summaries, scores (binary64, rel 1e-9), selections under both tie
rules, and gathered bytes.  Inputs come from the device generator, which is
bit-identical to the oracle's (tests/test_oracle_kat.py pins that), copied to
pinned host memory: the history of the stage-in and the oracle's input.

  128K layer   131072 tokens, Hq 32 / Hkv 8, D 128, fp16 K/V, 512 pages, top-32
  k8v4         131072 tokens, q8_0 K + q4_1-layout V, dequantized on gather
  8 lanes      8 x 262144 tokens, Hq 40 / Hkv 8, 4 query rows (matrix cores), top-64
  1M layerwise 2 of 40 layers x 1048576 tokens, Hq 16 / Hkv 2, D 256, q8_0 K /
               fp16 V, resident summaries, top-48, layer l+1 scored while
               layer l's pages stream in
"""
import numpy as np
import pytest
import torch

import kvmem_amd as K
import oracle as O
from gpu_util import host, zeros
from kvmem_amd.hip import runtime

pytestmark = pytest.mark.gpu
SEED = 42
REL = 1e-9


def _rel_err(a, b):
    return float(np.max(np.abs(np.asarray(a) - b) / np.maximum(np.abs(b), 1e-300)))


class Synth:
    """Device-generated input plus its pinned host copy."""

    def __init__(self, ctx, nbytes, fill):
        self.dev = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        torch.cuda.synchronize()
        fill(self.dev)
        ctx.check()
        self.pin = K.PinnedBuffer(nbytes)
        runtime().d2h(self.pin.ptr, self.dev.data_ptr(), nbytes)

    def np(self, dtype=np.uint8):
        return self.pin.numpy(dtype)

    def free(self):
        self.pin.free()
        self.dev = None


def _f16(ctx, sid, count):
    return lambda t: ctx.synth_normal_f16(SEED, sid, count, t)


def test_128k_layer_fp16(ctx):
    T, HQ, HKV, D, PT, KSEL = 131072, 32, 8, 128, 256, 32
    W, P = HKV * D, T // PT
    kh = Synth(ctx, T * W * 2, _f16(ctx, 1000, T * W))
    vh = Synth(ctx, T * W * 2, _f16(ctx, 2000, T * W))
    qh = Synth(ctx, HQ * D * 2, _f16(ctx, 3000, HQ * D))
    try:
        keys = kh.np(np.uint16)
        m32_expect = O.page_summaries(keys, O.FMT_F16, T, W, PT)[1]
        qf = qh.np(np.uint16).view(np.float16).astype(np.float32).reshape(1, 1, HQ, D)
        expect = O.page_softmax_scores(m32_expect[None], qf, [1], HQ, HKV, D, O.AGG_MEAN)
        for tie in (K.TIE_LOWER_FIRST, K.TIE_HIGHER_FIRST):
            s16, m32 = zeros(P * W, np.uint16), zeros(P * W, np.float32)
            scores, sel, cnt = zeros(P, np.float64), zeros(KSEL, np.uint32), zeros(1, np.uint32)
            ks, vs = zeros(KSEL * PT * W, np.uint16), zeros(KSEL * PT * W, np.uint16)
            planes = [K.make_plane(kh.pin, K.FMT_F16, W, T, K.GATHER_COPY, ks),
                      K.make_plane(vh.pin, K.FMT_F16, W, T, K.GATHER_COPY, vs)]
            ctx.recall_layer(keys=K.make_keys(kh.dev, K.FMT_F16, T, HKV, D, PT), summaries=s16, means=m32,
                             query=K.make_query(qh.dev, K.FMT_F16, 1, HQ, HKV, D), scores=scores, selected=sel,
                             count=cnt, k=KSEL, tie_rule=tie, planes=planes)
            ctx.check()
            assert np.array_equal(host(m32, np.uint32), m32_expect.ravel().view(np.uint32))
            assert _rel_err(host(scores, np.float64), expect) <= REL
            got = host(sel, np.uint32)
            assert np.array_equal(got, O.pick_scored_blocks(expect, KSEL, (), tie))
            assert np.array_equal(host(ks, np.uint8), O.gather(kh.np(), O.FMT_F16, W, T, PT, got, O.GATHER_COPY))
            assert np.array_equal(host(vs, np.uint8), O.gather(vh.np(), O.FMT_F16, W, T, PT, got, O.GATHER_COPY))
    finally:
        for s in (kh, vh, qh):
            s.free()


def test_128k_k8v4_dequant_on_gather(ctx):
    T, HQ, HKV, D, PT, KSEL = 131072, 32, 8, 128, 256, 32
    W, P = HKV * D, T // PT
    blocks = T * W // 32
    kh = Synth(ctx, blocks * 34, lambda t: ctx.synth_q8_0(SEED, 1100, blocks, 0.01, 0.05, t))
    vh = Synth(ctx, blocks * 20, lambda t: ctx.synth_q4_1(SEED, 1101, blocks, 0.01, 0.05, -0.4, 0.0, t))
    qh = Synth(ctx, HQ * D * 2, _f16(ctx, 1102, HQ * D))
    try:
        _, means = O.page_summaries(kh.np(), O.FMT_Q8_0, T, W, PT)
        qf = qh.np(np.uint16).view(np.float16).astype(np.float32).reshape(1, 1, HQ, D)
        expect = O.page_softmax_scores(means[None], qf, [1], HQ, HKV, D, O.AGG_MEAN)
        s16, scores = zeros(P * W, np.uint16), zeros(P, np.float64)
        sel, cnt = zeros(KSEL, np.uint32), zeros(1, np.uint32)
        ks, vs = zeros(KSEL * PT * W, np.uint16), zeros(KSEL * PT * W, np.uint16)
        planes = [K.make_plane(kh.pin, K.FMT_Q8_0, W, T, K.GATHER_DEQUANT_F16, ks),
                  K.make_plane(vh.pin, K.FMT_Q4_1, W, T, K.GATHER_DEQUANT_F16, vs)]
        ctx.recall_layer(keys=K.make_keys(kh.dev, K.FMT_Q8_0, T, HKV, D, PT), summaries=s16,
                         query=K.make_query(qh.dev, K.FMT_F16, 1, HQ, HKV, D), scores=scores, selected=sel,
                         count=cnt, k=KSEL, planes=planes)
        ctx.check()
        assert _rel_err(host(scores, np.float64), expect) <= REL
        got = host(sel, np.uint32)
        for tie in (O.TIE_LOWER_FIRST, O.TIE_HIGHER_FIRST):  # no exact ties at this shape
            assert np.array_equal(got, O.pick_scored_blocks(expect, KSEL, (), tie))
        assert np.array_equal(host(ks, np.uint8), O.gather(kh.np(), O.FMT_Q8_0, W, T, PT, got, O.GATHER_DEQUANT_F16))
        assert np.array_equal(host(vs, np.uint8), O.gather(vh.np(), O.FMT_Q4_1, W, T, PT, got, O.GATHER_DEQUANT_F16))
    finally:
        for s in (kh, vh, qh):
            s.free()


def test_8_lanes_262k_matrix_cores(ctx):
    L, T, HQ, HKV, D, PT, R, KSEL = 8, 262144, 40, 8, 128, 256, 4, 64
    W, P = HKV * D, T // PT
    kh = Synth(ctx, L * T * W * 2, _f16(ctx, 1200, L * T * W))
    vh = Synth(ctx, L * T * W * 2, _f16(ctx, 1201, L * T * W))
    qh = Synth(ctx, L * R * HQ * D * 2, _f16(ctx, 1202, L * R * HQ * D))
    try:
        keys = kh.np(np.uint16).reshape(L, T * W)
        qf = qh.np(np.uint16).view(np.float16).astype(np.float32).reshape(L, R, HQ, D)
        s16, scores = zeros(L * P * W, np.uint16), zeros(L * P, np.float64)
        sel, cnt = zeros(L * KSEL, np.uint32), zeros(L, np.uint32)
        ks, vs = zeros(L * KSEL * PT * W, np.uint16), zeros(L * KSEL * PT * W, np.uint16)
        planes = [K.make_plane(kh.pin, K.FMT_F16, W, T, K.GATHER_COPY, ks),
                  K.make_plane(vh.pin, K.FMT_F16, W, T, K.GATHER_COPY, vs)]
        ctx.recall_layer(keys=K.make_keys(kh.dev, K.FMT_F16, T, HKV, D, PT, lanes=L), summaries=s16,
                         query=K.make_query(qh.dev, K.FMT_F16, R, HQ, HKV, D, lanes=L), scores=scores,
                         selected=sel, count=cnt, k=KSEL, planes=planes)
        ctx.check()
        got_s = host(scores, np.float64).reshape(L, P)
        got = host(sel, np.uint32).reshape(L, KSEL)
        assert (host(cnt, np.uint32) == KSEL).all()
        kslots = host(ks, np.uint8).reshape(L, -1)
        vslots = host(vs, np.uint8).reshape(L, -1)
        vals = vh.np(np.uint16).reshape(L, T * W)
        for l in range(L):
            _, means = O.page_summaries(keys[l], O.FMT_F16, T, W, PT)
            expect = O.page_softmax_scores(means[None], qf[l][None], [R], HQ, HKV, D, O.AGG_MEAN)
            assert _rel_err(got_s[l], expect) <= REL
            assert np.array_equal(got[l], O.pick_scored_blocks(expect, KSEL))
            assert np.array_equal(kslots[l], O.gather(keys[l].view(np.uint8), O.FMT_F16, W, T, PT, got[l],
                                                      O.GATHER_COPY))
            assert np.array_equal(vslots[l], O.gather(vals[l].view(np.uint8), O.FMT_F16, W, T, PT, got[l],
                                                      O.GATHER_COPY))
    finally:
        for s in (kh, vh, qh):
            s.free()


def test_1m_layerwise_q8_resident_summaries(ctx):
    LAYERS, T, HQ, HKV, D, PT, KSEL = 2, 1048576, 16, 2, 256, 256, 48
    W, P = HKV * D, T // PT
    blocks = T * W // 32
    layers = []
    try:
        for l in range(LAYERS):
            kh = Synth(ctx, blocks * 34, lambda t, l=l: ctx.synth_normal_q8_0(SEED, 1300 + l, blocks, t))
            vh = Synth(ctx, T * W * 2, _f16(ctx, 1310 + l, T * W))
            qh = Synth(ctx, HQ * D * 4, lambda t, l=l: ctx.synth_normal_f32(SEED, 1320 + l, HQ * D, t))
            s16 = zeros(P * W, np.uint16)
            # summaries built once in setup and kept resident
            ctx.summary_build(K.make_keys(kh.dev, K.FMT_Q8_0, T, HKV, D, PT), None, s16)
            layers.append(dict(kh=kh, vh=vh, qh=qh, s16=s16, scores=zeros(P, np.float64),
                               sel=zeros(KSEL, np.uint32), cnt=zeros(1, np.uint32),
                               ks=zeros(KSEL * PT * W, np.uint16), vs=zeros(KSEL * PT * W, np.uint16)))
        ctx.check()
        for b in layers:  # layer l+1's select runs while layer l's pages stream in
            planes = [K.make_plane(b["kh"].pin, K.FMT_Q8_0, W, T, K.GATHER_DEQUANT_F16, b["ks"]),
                      K.make_plane(b["vh"].pin, K.FMT_F16, W, T, K.GATHER_COPY, b["vs"])]
            ctx.recall_layer(query=K.make_query(b["qh"].dev, K.FMT_F32, 1, HQ, HKV, D), summaries=b["s16"],
                             pages=P, page_tokens=PT, scores=b["scores"], selected=b["sel"], count=b["cnt"],
                             k=KSEL, planes=planes)
        ctx.check()
        for b in layers:
            kq = b["kh"].np()
            _, means = O.page_summaries(kq, O.FMT_Q8_0, T, W, PT)
            assert np.array_equal(host(b["s16"], np.uint16),
                                  means.ravel().astype(np.float16).view(np.uint16))
            q = b["qh"].np(np.float32).reshape(1, 1, HQ, D)
            expect = O.page_softmax_scores(means[None], q, [1], HQ, HKV, D, O.AGG_MEAN)
            assert _rel_err(host(b["scores"], np.float64), expect) <= REL
            got = host(b["sel"], np.uint32)
            assert np.array_equal(got, O.pick_scored_blocks(expect, KSEL))
            assert np.array_equal(host(b["ks"], np.uint8),
                                  O.gather(kq, O.FMT_Q8_0, W, T, PT, got, O.GATHER_DEQUANT_F16))
            assert np.array_equal(host(b["vs"], np.uint8),
                                  O.gather(b["vh"].np(), O.FMT_F16, W, T, PT, got, O.GATHER_COPY))
    finally:
        for b in layers:
            for s in ("kh", "vh", "qh"):
                b[s].free()
