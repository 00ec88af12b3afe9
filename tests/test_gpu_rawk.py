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
