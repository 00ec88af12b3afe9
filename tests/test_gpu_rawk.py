"""GPU parity of the raw-K stage-in transform (KVR_GATHER_ROPE_FWHT: decode
q8_0/q4_0, NeoX RoPE at each token's position, Walsh-Hadamard, requantize;
kvmem_stagein_enqueue_k + flush, src/adapter/llama-kvmem-stagein.cu:105-234,
746-783) against the oracle, through the C ABI.

Bar: bit-exact slot bytes.  Both sides compute sin/cos by the same binary64
operations and round once, the rotation and the quantizers with the same
explicit fused multiply-adds, and the Walsh-Hadamard butterflies in the
reference's order.  Covered: both formats, partial rotation, Walsh-Hadamard
runs spanning heads, no transform, large positions, a partial last page,
several lanes with counts, both copy engines, and the argument checks.
"""
import numpy as np
import pytest

import kvmem_amd as K
import oracle as O
from gpu_util import dev, host, sync, zeros

pytestmark = pytest.mark.gpu


def history(rng, fmt, tokens, width):
    nb = width // 32
    bb = 34 if fmt == K.FMT_Q8_0 else 18
    raw = rng.integers(0, 256, (tokens, nb, bb), dtype=np.uint8)
    raw[:, :, :2] = rng.uniform(0.01, 0.05, (tokens, nb)).astype(np.float16).view(np.uint8).reshape(tokens, nb, 2)
    return raw.reshape(-1)


def thetas(n_rot, base=10000.0):
    return (base ** (-np.arange(max(n_rot // 2, 1)) * 2 / max(n_rot, 1))).astype(np.float32)


def run(ctx, rng, *, fmt, width, head_dim, n_rot, fwht, tokens=1100, pt=256, sel=(0, 2, 4), pos_base=0,
        lanes=1, counts=None, engine=K.ENGINE_KERNEL):
    hist = np.concatenate([history(rng, fmt, tokens, width) for _ in range(lanes)])
    pin = K.PinnedBuffer(hist.size)
    pin.numpy()[:] = hist
    k = len(sel)
    row = K.row_bytes(fmt, width)
    theta = thetas(n_rot)
    th = dev(theta)
    fill = np.full(lanes * k * pt * row, 0x3C, np.uint8)
    counts = counts if counts is not None else [k] * lanes
    expect = fill.copy().reshape(lanes, -1)
    for l in range(lanes):
        lane = hist[l * tokens * row:(l + 1) * tokens * row]
        expect[l] = O.gather_rope(lane, fmt, width, tokens, pt, list(sel)[:counts[l]], head_dim, n_rot, theta, fwht,
                                  pos_base, slots=expect[l])
    slots = dev(fill)
    plane = K.make_plane(pin, fmt, width, tokens, K.GATHER_ROPE_FWHT, slots,
                         rope=dict(head_dim=head_dim, n_rot=n_rot, theta=th, fwht=fwht, pos_base=pos_base))
    seld = dev(np.tile(np.asarray(sel, np.uint32), lanes))
    ctx.stage_in([plane], pt, seld, dev(np.asarray(counts, np.uint32)), k, lanes=lanes, engine=engine)
    ctx.check()
    sync()
    got = host(slots, np.uint8)
    pin.free()
    return got, expect.ravel()


@pytest.mark.parametrize("engine", [K.ENGINE_KERNEL, K.ENGINE_SDMA])
@pytest.mark.parametrize("fmt", [K.FMT_Q8_0, K.FMT_Q4_0])
def test_rope_fwht_bit_exact(ctx, fmt, engine):
    rng = np.random.default_rng(3 + fmt)
    # 8 heads x 128, full rotation, Walsh-Hadamard per head; last page short
    got, want = run(ctx, rng, fmt=fmt, width=1024, head_dim=128, n_rot=128, fwht=128, engine=engine)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("n_rot,fwht", [(64, 256), (0, 512), (96, 0), (0, 0)])
def test_partial_rotation_and_runs_across_heads(ctx, n_rot, fwht):
    rng = np.random.default_rng(10 + n_rot + fwht)
    for fmt in (K.FMT_Q8_0, K.FMT_Q4_0):
        got, want = run(ctx, rng, fmt=fmt, width=512, head_dim=128, n_rot=n_rot, fwht=fwht, tokens=700, pt=128,
                        sel=(5, 1, 3))
        assert np.array_equal(got, want), (fmt, n_rot, fwht)


def test_large_positions_and_lanes(ctx):
    rng = np.random.default_rng(21)
    # positions around a million (range reduction), three lanes with counts
    got, want = run(ctx, rng, fmt=K.FMT_Q8_0, width=256, head_dim=64, n_rot=64, fwht=64, tokens=600, pt=64,
                    sel=(0, 7, 9, 3), pos_base=1_000_000, lanes=3, counts=[4, 1, 0])
    assert np.array_equal(got, want)


def test_rejects(ctx):
    pin = K.PinnedBuffer(4096 * 34)
    slots = zeros(4096 * 34, np.uint8)
    th = dev(thetas(64))

    def call(fmt=K.FMT_Q8_0, **rope):
        r = dict(head_dim=128, n_rot=64, theta=th, fwht=128, pos_base=0)
        r.update(rope)
        plane = K.make_plane(pin, fmt, 256, 64, K.GATHER_ROPE_FWHT, slots, rope=r)
        with pytest.raises(K.KvrError) as e:
            ctx.stage_in([plane], 64, dev(np.zeros(1, np.uint32)), dev(np.ones(1, np.uint32)), 1)
        return e.value.status

    assert call(fmt=K.FMT_F16) == K._capi.ERR_UNSUPPORTED
    assert call(fmt=K.FMT_Q4_1) == K._capi.ERR_UNSUPPORTED
    assert call(head_dim=96) == K._capi.ERR_INVALID       # does not divide the width
    assert call(n_rot=63) == K._capi.ERR_INVALID          # odd
    assert call(n_rot=192) == K._capi.ERR_INVALID         # past the head
    assert call(fwht=32) == K._capi.ERR_INVALID           # not a Walsh-Hadamard size
    assert call(fwht=512) == K._capi.ERR_INVALID          # does not divide the width
    assert call(theta=None) == K._capi.ERR_INVALID
    pin.free()


# ---- requantization at exact ties -------------------------------------------
# The rows of tests/test_oracle_requant_ties.py: products x*id that are exact
# half-integers after the Walsh-Hadamard transform, with the expected codes
# stated in exact rationals (ties away from zero for q8_0, truncation after
# +8.5 for q4_0).  A device or oracle switched to ties-to-even fails here.
import test_oracle_requant_ties as T  # noqa: E402


def _tie_gather(ctx, fmt, vectors, row_fn, expect_fn):
    per_row = 4  # four 64-value runs per 256-wide row
    rows, want = [], []
    for i in range(0, len(vectors) - len(vectors) % per_row, per_row):
        rows.append(b"".join(row_fn(c) for c in vectors[i:i + per_row]))
        want.append(b"".join(expect_fn(c)[0] for c in vectors[i:i + per_row]))
    tokens, pt, width = len(rows), 16, 256
    hist = np.frombuffer(b"".join(rows), np.uint8)
    pages = (tokens + pt - 1) // pt
    sel = np.arange(pages, dtype=np.uint32)
    row = K.row_bytes(fmt, width)
    pin = K.PinnedBuffer(hist.size)
    pin.numpy()[:] = hist
    slots = zeros(pages * pt * row, np.uint8)
    th = dev(np.zeros(1, np.float32))
    plane = K.make_plane(pin, fmt, width, tokens, K.GATHER_ROPE_FWHT, slots,
                         rope=dict(head_dim=64, n_rot=0, theta=th, fwht=64, pos_base=0))
    ctx.stage_in([plane], pt, dev(sel), dev(np.array([pages], np.uint32)), pages)
    ctx.check()
    sync()
    got = host(slots, np.uint8)[:tokens * row]
    pin.free()
    oracle = O.gather_rope(hist, fmt, width, tokens, pt, sel, 64, 0, None, 64)[:tokens * row]
    return got, np.frombuffer(b"".join(want), np.uint8), oracle


def test_q8_0_ties_on_device(ctx):
    got, exact, oracle = _tie_gather(ctx, K.FMT_Q8_0, T.Q8_CODES, T.q8_row, T.expected_q8)
    assert np.array_equal(oracle, exact)
    assert np.array_equal(got, exact)


def test_q4_0_ties_on_device(ctx):
    got, exact, oracle = _tie_gather(ctx, K.FMT_Q4_0, T.Q4_CODES, T.q4_row, T.expected_q4)
    assert np.array_equal(oracle, exact)
    assert np.array_equal(got, exact)


def test_requant_q8_0_half_ratio_blocks(ctx):
    """GATHER_REQUANT_Q8_0 on blocks whose codes include +-m/2 of the block's
    largest |code| m (x*id = +-63.5 there, the only half-integer this mode can
    produce), over many block scales: bit-exact against the oracle."""
    rng = np.random.default_rng(31)
    tokens, width, pt = 512, 256, 64
    nb = width // 32
    blocks = np.zeros((tokens, nb, 34), np.uint8)
    for t in range(tokens):
        for b in range(nb):
            m = int(rng.integers(1, 64)) * 2
            codes = rng.integers(-m, m + 1, 32)
            codes[0] = m if rng.integers(2) else -m
            codes[1:9] = rng.choice([m // 2, -(m // 2)], 8)
            blocks[t, b, :2] = np.frombuffer(np.float16(rng.uniform(0.001, 4.0)).tobytes(), np.uint8)
            blocks[t, b, 2:] = codes.astype(np.int8).view(np.uint8)
    hist = blocks.reshape(-1)
    sel = np.array([0, 3, 5, 7], np.uint32)
    row = K.row_bytes(K.FMT_Q8_0, width)
    pin = K.PinnedBuffer(hist.size)
    pin.numpy()[:] = hist
    slots = zeros(len(sel) * pt * row, np.uint8)
    plane = K.make_plane(pin, K.FMT_Q8_0, width, tokens, K.GATHER_REQUANT_Q8_0, slots)
    ctx.stage_in([plane], pt, dev(sel), dev(np.array([len(sel)], np.uint32)), len(sel))
    ctx.check()
    sync()
    want = O.gather(hist, K.FMT_Q8_0, width, tokens, pt, sel, O.GATHER_REQUANT_Q8_0)
    got = host(slots, np.uint8)
    pin.free()
    assert np.array_equal(got, want)
    codes = want.reshape(-1, 34)[:, 2:].view(np.int8)
    assert np.count_nonzero(np.abs(codes.astype(np.int32)) == 64) > 1000  # the +-63.5 products
