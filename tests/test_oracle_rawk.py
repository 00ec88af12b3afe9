"""Pins the oracle's raw-K stage-in transform (kvmem_stagein_enqueue_k and
flush, src/adapter/llama-kvmem-stagein.cu:105-234, 746-783) without the GPU:
the binary32 sin/cos against numpy's binary64 values, the NeoX rotation by
its closed forms, the Walsh-Hadamard transform as an involution with
Sylvester-ordered rows, the q4_0 quantizer on hand-built blocks, and the
whole transform as the identity on blocks it must return unchanged.
"""
import math

import numpy as np
import pytest

import oracle as O


def ulp32(x):
    return np.spacing(np.float32(abs(x)))


def test_sincos_within_one_ulp_of_binary64():
    rng = np.random.default_rng(3)
    angles = np.concatenate([rng.uniform(-10, 10, 2000), rng.uniform(0, 2e6, 2000),
                             np.array([0.0, 1e-30, math.pi / 4, math.pi / 2, 1e6])]).astype(np.float32)
    exact = 0
    for a in angles:
        s, c = O.rope_sincos(float(a))
        ts, tc = math.sin(float(a)), math.cos(float(a))
        assert abs(s - ts) <= ulp32(ts) and abs(c - tc) <= ulp32(tc), a
        exact += (np.float32(ts) == np.float32(s)) and (np.float32(tc) == np.float32(c))
    assert exact >= len(angles) - 2  # rounded once from ~1e-16 accurate values


def test_rope_closed_forms():
    rng = np.random.default_rng(4)
    hd, n_rot, heads = 64, 48, 3
    row = rng.standard_normal(hd * heads).astype(np.float32)
    theta = (10000.0 ** (-np.arange(n_rot // 2) * 2 / n_rot)).astype(np.float32)
    # position 0 (angle 0): the identity, bit for bit
    np.testing.assert_array_equal(O.rope_neox_row(row, hd, n_rot, theta, 0.0), row)
    # zero angles: the identity
    np.testing.assert_array_equal(O.rope_neox_row(row, hd, n_rot, np.zeros_like(theta), 37.0), row)
    out = O.rope_neox_row(row, hd, n_rot, theta, 1234.0)
    half = n_rot // 2
    for h in range(heads):
        x, y = row[h * hd:(h + 1) * hd].astype(np.float64), out[h * hd:(h + 1) * hd].astype(np.float64)
        # dims past n_rot are untouched; each rotated pair keeps its norm and
        # turns by pos*theta[i]
        np.testing.assert_array_equal(y[n_rot:], x[n_rot:])
        a = (np.float32(1234.0) * theta).astype(np.float64)  # the angle is a binary32 product
        np.testing.assert_allclose(y[:half], x[:half] * np.cos(a) - x[half:n_rot] * np.sin(a), atol=2e-6)
        np.testing.assert_allclose(y[half:n_rot], x[:half] * np.sin(a) + x[half:n_rot] * np.cos(a), atol=2e-6)
    # a rotation undone by the opposite position
    back = O.rope_neox_row(out, hd, n_rot, theta, -1234.0)
    np.testing.assert_allclose(back, row, atol=3e-6)


@pytest.mark.parametrize("n", [64, 128, 256, 512])
def test_fwht_rows_and_involution(n):
    width = 2 * n
    # a unit vector gives row j of the Sylvester Hadamard matrix, scaled
    for j in (0, 1, 5, n - 1):
        e = np.zeros(width, np.float32)
        e[n + j] = 1.0
        out = O.fwht_row(e, n)
        sign = np.array([(-1) ** bin(i & j).count("1") for i in range(n)], np.float64)
        np.testing.assert_allclose(out[n:], sign / math.sqrt(n), rtol=1e-6)
        assert not out[:n].any()
    rng = np.random.default_rng(n)
    x = rng.integers(-50, 50, width).astype(np.float32)
    twice = O.fwht_row(O.fwht_row(x, n), n)
    if n in (64, 256):  # 1/sqrt(n) exact: integers come back bit for bit
        np.testing.assert_array_equal(twice, x)
    else:
        np.testing.assert_allclose(twice, x, atol=1e-4)


def test_q4_0_quantizer_hand_block():
    d = 0.25
    codes = np.arange(32) % 16  # includes code 0 (value -8d): d is recovered
    x = ((codes - 8) * d).astype(np.float32)
    blk = O.quant_q4_0(x)
    assert np.float16(blk[:2].view(np.float16)[0]) == np.float16(d)
    np.testing.assert_array_equal(O.dequant_q4_0(blk), x)
    # equal magnitudes: the first sets the sign of d
    y = np.zeros(32, np.float32)
    y[3], y[9] = -4.0, 4.0
    b2 = O.quant_q4_0(y)
    assert b2[:2].view(np.float16)[0] == np.float16(0.5)
    z = np.zeros(32, np.float32)
    z[3], z[9] = 4.0, -4.0
    assert O.quant_q4_0(z)[:2].view(np.float16)[0] == np.float16(-0.5)


def _blocks(rng, fmt, rows, width):
    nb = width // 32
    if fmt == O.FMT_Q8_0:
        raw = rng.integers(-126, 127, (rows, nb, 34)).astype(np.int16).astype(np.uint8)
        raw[:, :, 2 + 5] = np.uint8(127)  # full-scale code: requant returns the block
        raw[:, :, :2] = rng.uniform(0.01, 0.05, (rows, nb)).astype(np.float16).view(np.uint8).reshape(rows, nb, 2)
    else:
        raw = rng.integers(0, 256, (rows, nb, 18)).astype(np.uint8)
        raw[:, :, 2] = (raw[:, :, 2] & 0xF0)  # code 0 (-8d) present
        raw[:, :, :2] = rng.uniform(0.01, 0.05, (rows, nb)).astype(np.float16).view(np.uint8).reshape(rows, nb, 2)
    return raw.reshape(rows, -1)


@pytest.mark.parametrize("fmt", [O.FMT_Q8_0, O.FMT_Q4_0])
def test_transform_without_rotation_is_identity(fmt):
    rng = np.random.default_rng(7 + fmt)
    rows, width = 9, 256
    raw = _blocks(rng, fmt, rows, width)
    out = O.rope_fwht_rows(raw, fmt, width, rows, 100, 128, 0, None, 0)
    np.testing.assert_array_equal(out, raw)


def test_transform_matches_its_steps():
    """rope_fwht_rows = dequant -> rotation -> Walsh-Hadamard -> quant, step
    by step through the pinned pieces."""
    rng = np.random.default_rng(11)
    width, hd, n_rot, n = 256, 128, 96, 128
    raw = _blocks(rng, O.FMT_Q8_0, 3, width)
    theta = (500000.0 ** (-np.arange(n_rot // 2) * 2 / n_rot)).astype(np.float32)
    out = O.rope_fwht_rows(raw, O.FMT_Q8_0, width, 3, 70000, hd, n_rot, theta, n)
    for t in range(3):
        x = np.concatenate([O.dequant_q8_0(raw[t, b * 34:(b + 1) * 34]) for b in range(width // 32)])
        x = O.rope_neox_row(x, hd, n_rot, theta, float(70000 + t))
        x = O.fwht_row(x, n)
        want = np.concatenate([O.quant_q8_0(x[b * 32:(b + 1) * 32]) for b in range(width // 32)])
        np.testing.assert_array_equal(out[t], want)
