"""GPU parity of kvr_attention_page_mass (the attention-feedback observer)
against the oracle's dense FP64 statement, through the C ABI.

Bar: binary32 on the device against binary64 in the oracle, so masses agree
to |gpu - oracle| <= 1e-6 + 2e-4 * oracle (the reference's own check allows
2e-3 absolute, src/adapter/llama-kvmem-attention.cpp:44-96).  Covered: every
key format (f16, bf16, f32, q8_0, q4_0, q5_0), query and mask scalars, head
dims 32..256, causal and fully masked pages, a fully masked row (NaN, as in
the reference), softcap, pages of 1 to 16 tiles and longer than a workgroup, more rows than one
launch holds, padded and 2-byte-offset key layouts, and the argument checks.
"""
import math

import numpy as np
import pytest

import kvmem_amd as K
import oracle as O
from gpu_util import dev, host, sync, zeros

pytestmark = pytest.mark.gpu

SCALAR_BYTES = {O.FMT_F32: 4, O.FMT_F16: 2, O.FMT_BF16: 2}
BLOCK_BYTES = {O.FMT_F32: 128, O.FMT_F16: 64, O.FMT_BF16: 64, O.FMT_Q8_0: 34, O.FMT_Q4_0: 18, O.FMT_Q5_0: 22}


def scalars(x: np.ndarray, fmt: int) -> np.ndarray:
    x = np.asarray(x, np.float32)
    if fmt == O.FMT_F32:
        return x
    if fmt == O.FMT_F16:
        return x.astype(np.float16).view(np.uint16)
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def key_rows(rng, fmt, tokens, kv, dim, head_stride, row_stride):
    """Raw key bytes [tokens * row_stride] with head h of token t at
    t*row_stride + h*head_stride (padding bytes random)."""
    hb = dim // 32 * BLOCK_BYTES[fmt]
    buf = rng.integers(0, 256, tokens * row_stride, dtype=np.uint8)
    for t in range(tokens):
        for h in range(kv):
            off = t * row_stride + h * head_stride
            if fmt in SCALAR_BYTES:
                buf[off:off + hb] = scalars(rng.standard_normal(dim), fmt).view(np.uint8)
            else:
                nb = dim // 32
                blk = rng.integers(0, 256, (nb, BLOCK_BYTES[fmt]), dtype=np.uint8)
                d = rng.uniform(0.01, 0.05, nb).astype(np.float16).view(np.uint8).reshape(nb, 2)
                blk[:, :2] = d
                buf[off:off + hb] = blk.reshape(-1)
    return buf


def run_case(ctx, rng, *, dim=128, heads=8, kv=2, tokens=1000, page=64, rows=(3, 0, 5), n_q_rows=6,
             k_fmt=O.FMT_F16, q_fmt=O.FMT_F32, m_fmt=O.FMT_F32, softcap=0.0, head_pad=0, row_pad=0,
             q_row_pad=0, mask_fn=None, scale=None, q_fn=None):
    scale = 1 / math.sqrt(dim) if scale is None else scale
    hb = dim // 32 * BLOCK_BYTES[k_fmt]
    head_stride = hb + head_pad
    row_stride = kv * head_stride + row_pad
    kbytes = key_rows(rng, k_fmt, tokens, kv, dim, head_stride, row_stride)
    qel, mel = SCALAR_BYTES[q_fmt], SCALAR_BYTES[m_fmt]
    q_row_stride = heads * dim * qel + q_row_pad
    qf = rng.standard_normal((n_q_rows, q_row_stride // qel)).astype(np.float32)
    if q_fn is not None:
        qf = q_fn(qf).astype(np.float32)
    qraw = scalars(qf, q_fmt).view(np.uint8).reshape(-1)
    mask = np.zeros((n_q_rows, tokens), np.float32)
    for r in range(n_q_rows):
        # causal prefix that grows with the row, some finite biases
        mask[r, min(tokens, tokens // 2 + r * 37):] = -np.inf
        mask[r, :3] = rng.standard_normal(3)
    if mask_fn is not None:
        mask_fn(mask)
    mraw = scalars(mask, m_fmt).view(np.uint8).reshape(-1)
    pages = -(-tokens // page)
    want = O.attention_page_mass(qraw, q_fmt, q_row_stride, dim * qel, kbytes, k_fmt, row_stride, head_stride,
                                 mraw, m_fmt, tokens * mel, dim, heads, kv, tokens, page, scale, softcap, rows)
    qd, kd, md = dev(qraw), dev(kbytes), dev(mraw)
    out = zeros(len(rows) * pages, np.float32)
    ctx.attention_page_mass(q=qd, q_format=q_fmt, q_row_stride=q_row_stride, q_head_stride=dim * qel, k=kd,
                            k_format=k_fmt, k_row_stride=row_stride, k_head_stride=head_stride, mask=md,
                            mask_format=m_fmt, mask_row_stride=tokens * mel, head_dim=dim, query_heads=heads,
                            kv_heads=kv, tokens=tokens, page_tokens=page, scale=scale, softcap=softcap,
                            rows=list(rows), mass=out)
    ctx.check()
    sync()
    got = host(out, np.float32).reshape(len(rows), pages).astype(np.float64)
    return got, want


def assert_close(got, want):
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan), "NaN positions differ"
    g, w = got[~nan], want[~nan]
    bad = np.abs(g - w) > 1e-6 + 2e-4 * np.abs(w)
    assert not bad.any(), f"max abs err {np.max(np.abs(g - w)):.3e} at {np.argmax(np.abs(g - w))}"


@pytest.mark.parametrize("k_fmt", [O.FMT_F16, O.FMT_BF16, O.FMT_F32, O.FMT_Q8_0, O.FMT_Q4_0, O.FMT_Q5_0])
def test_key_formats(ctx, k_fmt):
    rng = np.random.default_rng(10 + k_fmt)
    got, want = run_case(ctx, rng, k_fmt=k_fmt)
    assert_close(got, want)
    np.testing.assert_allclose(got.sum(axis=1), 1.0, rtol=1e-5)


@pytest.mark.parametrize("q_fmt,m_fmt", [(O.FMT_F16, O.FMT_F16), (O.FMT_BF16, O.FMT_BF16), (O.FMT_F32, O.FMT_F16)])
def test_query_and_mask_scalars(ctx, q_fmt, m_fmt):
    rng = np.random.default_rng(20 + q_fmt + 7 * m_fmt)
    assert_close(*run_case(ctx, rng, q_fmt=q_fmt, m_fmt=m_fmt, k_fmt=O.FMT_Q8_0))


@pytest.mark.parametrize("dim,heads,kv", [(32, 4, 4), (64, 16, 2), (96, 6, 3), (256, 8, 1)])
def test_head_dims_and_groups(ctx, dim, heads, kv):
    rng = np.random.default_rng(dim + heads)
    for k_fmt in (O.FMT_F16, O.FMT_Q8_0, O.FMT_Q5_0):
        assert_close(*run_case(ctx, rng, dim=dim, heads=heads, kv=kv, tokens=700, page=32, k_fmt=k_fmt))


@pytest.mark.parametrize("page", [16, 32, 64, 128, 256])
def test_page_runs(ctx, page):
    # pages of 1, 2, 4, 8 and 16 tiles: a wave's tiles of a page form runs of
    # 1, 1, 1, 2 and 4 tiles (one exponential per token); a partial last page
    rng = np.random.default_rng(70 + page)
    for k_fmt in (O.FMT_F16, O.FMT_Q8_0):
        assert_close(*run_case(ctx, rng, tokens=5 * page + 37, page=page, k_fmt=k_fmt, heads=8, kv=2))


def test_query_magnitudes(ctx):
    # f32 queries from 1e-6 to 1e6: each (row, head) pair at its own
    # magnitude and elements spread over three decades inside a pair (the
    # fp16 matrix-core forms scale each pair by a power of two either way)
    rng = np.random.default_rng(81)
    heads, dim = 8, 128

    def spread(q):
        rows = q.shape[0]
        mag = 10.0 ** rng.uniform(-6, 6, (rows, heads, 1))
        inner = 10.0 ** rng.uniform(-1.5, 1.5, (rows, heads, dim))
        return (q.reshape(rows, heads, dim) * mag * inner).reshape(rows, -1)
    for k_fmt in (O.FMT_F16, O.FMT_Q8_0):
        assert_close(*run_case(ctx, rng, heads=heads, kv=2, dim=dim, tokens=800, page=64, k_fmt=k_fmt,
                               q_fn=spread, scale=0.05))


def test_softcap_and_long_pages(ctx):
    rng = np.random.default_rng(31)
    # 600-token pages: lanes fold several tokens each (online rescaling)
    assert_close(*run_case(ctx, rng, tokens=1900, page=600, softcap=1.5, k_fmt=O.FMT_Q4_0))
    assert_close(*run_case(ctx, rng, tokens=513, page=256, softcap=30.0, k_fmt=O.FMT_F16, scale=0.3))


def test_many_rows_split_over_launches(ctx):
    rng = np.random.default_rng(41)
    rows = [(7 * i) % 90 for i in range(70)]  # > 64 rows per launch, repeats allowed
    assert_close(*run_case(ctx, rng, rows=rows, n_q_rows=90, heads=16, kv=2, tokens=400, page=16, dim=64,
                           k_fmt=O.FMT_Q8_0))


def test_padded_and_offset_key_layouts(ctx):
    rng = np.random.default_rng(51)
    # quantized heads at 2-byte (not 4-byte) offsets; padded rows and query rows
    for k_fmt in (O.FMT_Q8_0, O.FMT_Q4_0, O.FMT_Q5_0):
        assert_close(*run_case(ctx, rng, k_fmt=k_fmt, head_pad=2, row_pad=6, q_row_pad=8, tokens=300, page=50))
    assert_close(*run_case(ctx, rng, k_fmt=O.FMT_F16, head_pad=16, row_pad=32, tokens=300, page=50))


def test_masked_pages_and_rows(ctx):
    rng = np.random.default_rng(61)

    def masks(m):
        m[:, 64:128] = -np.inf      # a fully masked page for every row
        m[1, :] = -np.inf           # row 1 sees nothing: NaN, as in the reference
        m[2, ::3] = np.inf          # +inf is non-finite: left out
    got, want = run_case(ctx, rng, rows=(0, 1, 2), mask_fn=masks, tokens=500, page=64)
    assert_close(got, want)
    assert (got[0, 1] == 0.0) and (got[2, 1] == 0.0)
    assert np.isnan(got[1]).all()


def test_rejects(ctx):
    q = zeros(1024, np.float32)
    k = zeros(65536, np.uint8)
    out = zeros(64, np.float32)

    def call(**over):
        kw = dict(q=q, q_format=O.FMT_F32, q_row_stride=512, q_head_stride=256, k=k, k_format=O.FMT_F16,
                  k_row_stride=256, k_head_stride=128, mask=q, mask_format=O.FMT_F32, mask_row_stride=256,
                  head_dim=64, query_heads=2, kv_heads=2, tokens=64, page_tokens=16, scale=0.125, softcap=0.0,
                  rows=[0], mass=out)
        kw.update(over)
        with pytest.raises(K.KvrError) as e:
            ctx.attention_page_mass(**kw)
        return e.value.status

    assert call(k_format=O.FMT_Q4_1) == K._capi.ERR_UNSUPPORTED
    assert call(q_format=O.FMT_Q8_0) == K._capi.ERR_UNSUPPORTED
    assert call(head_dim=48) == K._capi.ERR_UNSUPPORTED
    assert call(head_dim=288) == K._capi.ERR_UNSUPPORTED
    assert call(kv_heads=3) == K._capi.ERR_INVALID
    assert call(rows=[]) == K._capi.ERR_INVALID
    assert call(k_head_stride=136) == K._capi.ERR_INVALID      # f16 heads must be 16-byte aligned
    assert call(k_row_stride=192) == K._capi.ERR_INVALID       # rows overlap
    assert call(softcap=-1.0) == K._capi.ERR_INVALID
    assert call(k_format=O.FMT_Q8_0, k_head_stride=69, k_row_stride=138) == K._capi.ERR_INVALID
