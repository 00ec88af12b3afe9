"""GPU stage-in straight from native payload records (one record per page
holding every layer's planes at fixed offsets: PayloadLayout,
kvmem/include/kvmem/memory_contract.hpp:39-68) through kvr_plane.page_stride,
against the oracle's gather of the same rows laid out token-major.

Bar: bit-exact slot bytes, for copies, q8_0 -> fp16 decode and the raw-K
transform, both copy engines, a partial last page and two lanes.
"""
import numpy as np
import pytest

import kvmem_amd as K
import oracle as O
from gpu_util import dev, host, sync

pytestmark = pytest.mark.gpu

PT, W, PAGES = 64, 256, 20
TOKENS = PAGES * PT - 10
KROW = W // 32 * 34      # q8_0
VROW = W * 2             # fp16


def layout():
    """Two layers, each [K q8_0][scale pad][V f16], planes 16-byte aligned;
    returns (record_bytes, {(layer, 'k'|'v'): offset})."""
    off, at = {}, 0
    for layer in range(2):
        off[(layer, "k")] = at
        at += PT * KROW + 48           # a 48-byte scale plane follows K
        at = (at + 15) // 16 * 16
        off[(layer, "v")] = at
        at += PT * VROW
    return (at + 255) // 256 * 256, off


def archive(rng, lanes, rec, off):
    """Records [lanes][PAGES][rec] and the token-major planes they hold."""
    arc = rng.integers(0, 256, (lanes, PAGES, rec), dtype=np.uint8)
    k = {}
    for lane in range(lanes):
        for layer in range(2):
            kb = arc[lane, :, off[(layer, "k")]:off[(layer, "k")] + PT * KROW].reshape(PAGES, PT, W // 32, 34)
            kb[..., :2] = rng.uniform(0.01, 0.05, kb.shape[:3]).astype(np.float16).view(np.uint8).reshape(
                *kb.shape[:3], 2)
            arc[lane, :, off[(layer, "k")]:off[(layer, "k")] + PT * KROW] = kb.reshape(PAGES, -1)
            v = rng.standard_normal((PAGES, PT * W)).astype(np.float16).view(np.uint8)
            arc[lane, :, off[(layer, "v")]:off[(layer, "v")] + PT * VROW] = v
    for lane in range(lanes):
        for layer in range(2):
            for name, row in (("k", KROW), ("v", VROW)):
                o = off[(layer, name)]
                k[(lane, layer, name)] = arc[lane, :, o:o + PT * row].reshape(-1)[:TOKENS * row].copy()
    return arc, k


@pytest.mark.parametrize("engine", [K.ENGINE_KERNEL, K.ENGINE_SDMA])
def test_records_copy_decode_and_raw_k(ctx, engine):
    rng = np.random.default_rng(5 + engine)
    lanes = 2
    rec, off = layout()
    arc, tm = archive(rng, lanes, rec, off)
    pin = K.PinnedBuffer(arc.size)
    pin.numpy()[:] = arc.reshape(-1)
    sel = [[0, 3, 7, 19], [2, 5, 11, 19]]  # ascending, as selections are
    k = 4
    theta = (10000.0 ** (-np.arange(32) * 2 / 64)).astype(np.float32)
    th = dev(theta)
    layer = 1
    cases = [("k", K.FMT_Q8_0, K.GATHER_COPY, KROW, None), ("v", K.FMT_F16, K.GATHER_COPY, VROW, None),
             ("k", K.FMT_Q8_0, K.GATHER_DEQUANT_F16, W * 2, None),
             ("k", K.FMT_Q8_0, K.GATHER_ROPE_FWHT, KROW,
              dict(head_dim=128, n_rot=64, theta=th, fwht=128, pos_base=1000))]
    slots, planes = [], []
    for name, fmt, mode, drow, rope in cases:
        s = dev(np.full(lanes * k * PT * drow, 0x5A, np.uint8))
        slots.append(s)
        planes.append(K.make_plane(pin, fmt, W, TOKENS, mode, s, host_lane_stride=PAGES * rec, rope=rope,
                                   history_offset=off[(layer, name)], page_stride=rec))
    ctx.stage_in(planes, PT, dev(np.array(sel, np.uint32).ravel()), dev(np.full(lanes, k, np.uint32)), k,
                 lanes=lanes, engine=engine)
    ctx.check()
    sync()
    for (name, fmt, mode, drow, rope), s in zip(cases, slots):
        got = host(s, np.uint8).reshape(lanes, -1)
        for lane in range(lanes):
            hist = tm[(lane, layer, name)]
            fill = np.full(k * PT * drow, 0x5A, np.uint8)
            if mode == K.GATHER_ROPE_FWHT:
                want = O.gather_rope(hist, fmt, W, TOKENS, PT, sel[lane], 128, 64, theta, 128, 1000, slots=fill)
            else:
                want = O.gather(hist, fmt, W, TOKENS, PT, sel[lane], mode, slots=fill)
            assert np.array_equal(got[lane], want), (name, mode, lane)
    pin.free()


def test_record_stride_checks(ctx):
    rec, off = layout()
    pin = K.PinnedBuffer(PAGES * rec)
    s = dev(np.zeros(PT * KROW, np.uint8))
    plane = K.make_plane(pin, K.FMT_Q8_0, W, TOKENS, K.GATHER_COPY, s, page_stride=PT * KROW - 1)
    with pytest.raises(K.KvrError) as e:
        ctx.stage_in([plane], PT, dev(np.zeros(1, np.uint32)), dev(np.ones(1, np.uint32)), 1)
    assert e.value.status == K._capi.ERR_INVALID
    pin.free()
