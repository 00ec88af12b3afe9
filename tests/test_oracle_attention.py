"""Pins the oracle's sampled-attention page masses (the attention-feedback
observer, src/adapter/llama-kvmem-attention-cuda.cu:59-193 and its dense
check at src/adapter/llama-kvmem-attention.cpp:44-96) without the GPU:

* q4_0 / q5_0 decoding on hand-built blocks whose values are written out
  by hand from the block layouts (cu:31-56);
* closed forms: zero keys give every unmasked token the same weight (page
  mass = its share of unmasked tokens), two tokens give the logistic of
  their logit difference, softcap applies tanh, the mask adds log-weights,
  masked pages get nothing and a fully masked row is NaN;
* an independent restatement through per-page log-sum-exps (the route the
  reference's GPU kernels take), which the oracle's dense softmax has to
  match on random inputs of every key format.
"""
import math

import numpy as np
import pytest

import oracle as O


def f16(x):
    return np.asarray(x, np.float32).astype(np.float16)


def mass(q, k, mask, *, dim, heads, kv, tokens, page, rows, q_fmt=O.FMT_F32, k_fmt=O.FMT_F32,
         m_fmt=O.FMT_F32, scale=1.0, softcap=0.0, k_row=None, k_head=None):
    qel = 4 if q_fmt == O.FMT_F32 else 2
    mel = 4 if m_fmt == O.FMT_F32 else 2
    k_head = k_head if k_head is not None else key_row_bytes(k_fmt, dim)
    k_row = k_row if k_row is not None else kv * k_head
    return O.attention_page_mass(q, q_fmt, heads * dim * qel, dim * qel, k, k_fmt, k_row, k_head,
                                 mask, m_fmt, tokens * mel, dim, heads, kv, tokens, page, scale, softcap, rows)


def key_row_bytes(fmt, dim):
    return {O.FMT_F32: 4 * dim, O.FMT_F16: 2 * dim, O.FMT_BF16: 2 * dim, O.FMT_Q8_0: dim // 32 * 34,
            O.FMT_Q4_0: dim // 32 * 18, O.FMT_Q5_0: dim // 32 * 22}[fmt]


# ---------------------------------------------------------------------------
# block decoding
# ---------------------------------------------------------------------------
def test_q4_0_hand_block():
    d = 0.5  # exact in fp16
    nib = np.arange(32) % 16  # element j has code (j % 16)
    qs = np.zeros(16, np.uint8)
    for j in range(16):
        qs[j] = nib[j] | (nib[j + 16] << 4)
    block = np.concatenate([f16([d]).view(np.uint8), qs])
    expect = np.array([(nib[j] - 8) * d for j in range(32)], np.float32)
    np.testing.assert_array_equal(O.dequant_q4_0(block), expect)


def test_q5_0_hand_block():
    d = 0.25
    codes = (np.arange(32) * 7) % 32  # 5-bit codes 0..31
    qs = np.zeros(16, np.uint8)
    for j in range(16):
        qs[j] = (codes[j] & 15) | ((codes[j + 16] & 15) << 4)
    qh = 0
    for j in range(32):
        qh |= ((int(codes[j]) >> 4) & 1) << j
    block = np.concatenate([f16([d]).view(np.uint8), np.array([qh], "<u4").view(np.uint8), qs])
    assert block.size == O.Q5_0_BYTES
    expect = np.array([(c - 16) * d for c in codes], np.float32)
    np.testing.assert_array_equal(O.dequant_q5_0(block), expect)


def test_q8_0_hand_block():
    d = 0.125
    codes = np.arange(-16, 16, dtype=np.int8)
    block = np.concatenate([f16([d]).view(np.uint8), codes.view(np.uint8)])
    np.testing.assert_array_equal(O.dequant_q8_0(block), codes.astype(np.float32) * d)


# ---------------------------------------------------------------------------
# closed forms
# ---------------------------------------------------------------------------
def test_zero_keys_give_token_shares():
    dim, heads, kv, tokens, page = 32, 4, 2, 10, 4
    rng = np.random.default_rng(1)
    q = rng.standard_normal((2, heads, dim)).astype(np.float32)
    k = np.zeros((tokens, kv, dim), np.float32)
    mask = np.zeros((2, tokens), np.float32)
    mask[1, 7:] = -np.inf  # row 1 sees tokens 0..6
    out = mass(q, k, mask, dim=dim, heads=heads, kv=kv, tokens=tokens, page=page, rows=[0, 1])
    np.testing.assert_allclose(out[0], [0.4, 0.4, 0.2], rtol=1e-15)
    np.testing.assert_allclose(out[1], [4 / 7, 3 / 7, 0.0], rtol=1e-15)
    assert out[1, 2] == 0.0


def test_two_tokens_logistic_and_softcap():
    dim, heads, kv, tokens = 32, 2, 1, 2
    q = np.zeros((1, heads, dim), np.float32)
    q[0, :, 0] = 1.0
    k = np.zeros((tokens, kv, dim), np.float32)
    k[0, 0, 0], k[1, 0, 0] = 3.0, -1.0
    mask = np.zeros((1, tokens), np.float32)
    scale = 0.5
    out = mass(q, k, mask, dim=dim, heads=heads, kv=kv, tokens=tokens, page=1, rows=[0], scale=scale)
    p0 = 1.0 / (1.0 + math.exp(scale * (-1.0 - 3.0)))
    np.testing.assert_allclose(out[0], [p0, 1 - p0], rtol=1e-14)
    cap = 0.75
    out = mass(q, k, mask, dim=dim, heads=heads, kv=kv, tokens=tokens, page=1, rows=[0], scale=scale,
               softcap=cap)
    l0, l1 = cap * math.tanh(1.5 / cap), cap * math.tanh(-0.5 / cap)
    p0 = 1.0 / (1.0 + math.exp(l1 - l0))
    np.testing.assert_allclose(out[0], [p0, 1 - p0], rtol=1e-14)


def test_mask_adds_log_weights():
    dim, heads, kv, tokens, page = 32, 1, 1, 6, 2
    q = np.ones((1, heads, dim), np.float32)
    k = np.zeros((tokens, kv, dim), np.float32)
    w = np.array([1, 2, 3, 4, 5, 6], np.float64)
    mask = np.log(w).astype(np.float32)[None, :]
    out = mass(q, k, mask, dim=dim, heads=heads, kv=kv, tokens=tokens, page=page, rows=[0])
    wf = np.exp(mask[0].astype(np.float64))
    np.testing.assert_allclose(out[0], [wf[0:2].sum(), wf[2:4].sum(), wf[4:6].sum()] / wf.sum(), rtol=1e-14)


def test_fully_masked_row_is_nan():
    dim, heads, kv, tokens = 32, 2, 1, 5
    q = np.ones((1, heads, dim), np.float32)
    k = np.ones((tokens, kv, dim), np.float32)
    mask = np.full((1, tokens), -np.inf, np.float32)
    out = mass(q, k, mask, dim=dim, heads=heads, kv=kv, tokens=tokens, page=2, rows=[0])
    assert np.isnan(out).all()


# ---------------------------------------------------------------------------
# independent per-page log-sum-exp restatement on random inputs
# ---------------------------------------------------------------------------
def random_keys(rng, fmt, tokens, kv, dim):
    """Raw key bytes [tokens][kv][row] and their decoded binary32 values."""
    nb = dim // 32
    if fmt in (O.FMT_F32, O.FMT_F16, O.FMT_BF16):
        x = rng.standard_normal((tokens, kv, dim)).astype(np.float32)
        if fmt == O.FMT_F32:
            return x.view(np.uint8).reshape(tokens, -1), x
        if fmt == O.FMT_F16:
            h = x.astype(np.float16)
            return h.view(np.uint8).reshape(tokens, -1), h.astype(np.float32)
        b = (x.view(np.uint32) >> 16).astype(np.uint16)
        return b.view(np.uint8).reshape(tokens, -1), (b.astype(np.uint32) << 16).view(np.float32)
    size = {O.FMT_Q8_0: 34, O.FMT_Q4_0: 18, O.FMT_Q5_0: 22}[fmt]
    dec = {O.FMT_Q8_0: O.dequant_q8_0, O.FMT_Q4_0: O.dequant_q4_0, O.FMT_Q5_0: O.dequant_q5_0}[fmt]
    raw = rng.integers(0, 256, (tokens, kv, nb, size), dtype=np.uint8)
    d = f16(rng.uniform(0.01, 0.05, (tokens, kv, nb))).view(np.uint8).reshape(tokens, kv, nb, 2)
    raw[..., :2] = d
    vals = np.stack([dec(raw[t, h, b]) for t in range(tokens) for h in range(kv) for b in range(nb)])
    return raw.reshape(tokens, -1), vals.reshape(tokens, kv, dim)


def lse_restatement(qv, kv_vals, bias, heads, kv, page, scale, softcap):
    tokens = kv_vals.shape[0]
    pages = -(-tokens // page)
    group = heads // kv
    out = np.zeros(pages)
    for h in range(heads):
        logit = kv_vals[:, h // group, :].astype(np.float64) @ qv[h].astype(np.float64) * scale
        if softcap > 0:
            logit = softcap * np.tanh(logit / softcap)
        logit = np.where(np.isfinite(bias), logit + bias, -np.inf)
        lse = np.array([np.logaddexp.reduce(logit[p * page:(p + 1) * page]) for p in range(pages)])
        out += np.exp(lse - np.logaddexp.reduce(lse))
    return out / heads


@pytest.mark.parametrize("fmt", [O.FMT_F32, O.FMT_F16, O.FMT_BF16, O.FMT_Q8_0, O.FMT_Q4_0, O.FMT_Q5_0])
def test_dense_softmax_matches_page_lse(fmt):
    rng = np.random.default_rng(100 + fmt)
    dim, heads, kv, tokens, page = 64, 6, 2, 150, 16
    raw, vals = random_keys(rng, fmt, tokens, kv, dim)
    q = rng.standard_normal((3, heads, dim)).astype(np.float32)
    mask = np.zeros((3, tokens), np.float32)
    for r in range(3):
        mask[r, 40 * (r + 1):] = -np.inf  # causal prefix
        mask[r, :5] = rng.standard_normal(5)
    softcap = 2.0 if fmt == O.FMT_Q8_0 else 0.0
    scale = 1 / math.sqrt(dim)
    out = mass(q, raw, mask, dim=dim, heads=heads, kv=kv, tokens=tokens, page=page, rows=[2, 0],
               k_fmt=fmt, scale=scale, softcap=softcap)
    for i, r in enumerate([2, 0]):
        ref = lse_restatement(q[r], vals, mask[r].astype(np.float64), heads, kv, page, np.float32(scale),
                              softcap)
        np.testing.assert_allclose(out[i], ref, rtol=1e-9, atol=1e-15)
        assert abs(out[i].sum() - 1.0) < 1e-12
