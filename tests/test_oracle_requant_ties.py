"""Requantization rounding at exact ties, and how sensitive the raw-K
transform's output codes are to its floating-point choices.

The reference requantizes with q = roundf(x*id) for q8_0 (ties away from
zero) and (int)(x*id + 8.5) for q4_0 (truncation after the offset), both in
src/adapter/llama-kvmem-stagein.cu:181-234.  These tests build inputs whose
products x*id are exact half-integers, state the expected codes with exact
rationals (no call into the oracle), and check that the oracle gives exactly
them -- and that a ties-to-even requantizer would not, so a switch of either
side to round-to-nearest-even fails.

Construction (raw-K transform, head_dim = fwht = 64, no rotation): source
codes c at input positions {0,1,2,4,8,16} with block scale 1.0.  The
Walsh-Hadamard transform scales by 1/8 and adds, so every output is
(H c)_i / 8 exactly.  With q8_0 codes (127, 127, 127, 126, 1) the largest
|(H c)_i| is 508, so d = 63.5/127 = 0.5 and x*id = (H c)_i / 4: every
output with (H c)_i = 2 mod 4 is a tie.  With q4_0 codes (-8, -8, -8, -7,
-1) the first extreme value is -32/8 = -4, so d = -4/-8 = 0.5 and again
x*id = (H c)_i / 4.
"""
from fractions import Fraction
import itertools

import numpy as np
import pytest

import oracle as O

SUPPORT = (0, 1, 2, 4, 8, 16)


def sylvester(n):
    h = np.array([[1]], np.int64)
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


H64 = sylvester(64)


def round_half_away(x: Fraction) -> int:
    n = abs(x.numerator) * 2 + x.denominator
    q = n // (2 * x.denominator)  # floor(|x| + 1/2)
    return q if x >= 0 else -q


def f16_bytes(v: float) -> bytes:
    return np.array([v], np.float16).tobytes()


def code_vectors(values):
    """Distinct 64-value code vectors: `values` placed on five of SUPPORT's
    positions in every order (and negated, for q8_0)."""
    out = []
    for pos in itertools.combinations(SUPPORT, len(values)):
        for perm in set(itertools.permutations(values)):
            c = np.zeros(64, np.int64)
            c[list(pos)] = perm
            out.append(c)
    return out


def q8_row(c):
    return b"".join(f16_bytes(1.0) + c[b * 32:(b + 1) * 32].astype(np.int8).tobytes() for b in range(2))


def q4_row(c):
    blocks = []
    for b in range(2):
        nib = (c[b * 32:(b + 1) * 32] + 8).astype(np.uint8)
        blocks.append(f16_bytes(1.0) + bytes((nib[:16] | (nib[16:] << 4)).tolist()))
    return b"".join(blocks)


def expected_q8(c):
    """q8_0 of (H c)/8, block by block, ties away from zero (exact)."""
    y = [Fraction(int(v), 8) for v in H64 @ c]
    out = b""
    ties = 0
    for b in range(2):
        blk = y[b * 32:(b + 1) * 32]
        amax = max(abs(v) for v in blk)
        d = amax / 127
        assert d == Fraction(1, 2)
        q = []
        for v in blk:
            p = v / d
            ties += p.denominator == 2 and round_half_away(p) % 2 != 0
            q.append(round_half_away(p))
        out += f16_bytes(0.5) + np.array(q, np.int8).tobytes()
    return out, ties


def expected_q4(c):
    """q4_0 of (H c)/8: d = (first extreme value)/-8, codes min(trunc(x*id + 8.5), 15)."""
    y = [Fraction(int(v), 8) for v in H64 @ c]
    out = b""
    ties = 0
    for b in range(2):
        blk = y[b * 32:(b + 1) * 32]
        vmax = Fraction(0)
        for v in blk:
            if abs(v) > abs(vmax):
                vmax = v
        d = vmax / -8
        assert d == Fraction(1, 2)
        q = []
        for v in blk:
            p = v / d + Fraction(17, 2)
            assert p >= 0
            q.append(min(p.numerator // p.denominator, 15))
            # a tie: x*id is a half-integer where rint(x*id) + 8 disagrees
            x = v / d
            ties += x.denominator == 2 and q[-1] != min(int(np.rint(float(x))) + 8, 15)
        nib = np.array(q, np.uint8)
        out += f16_bytes(0.5) + bytes((nib[:16] | (nib[16:] << 4)).tolist())
    return out, ties


def transform(rows, fmt, variant=0):
    n = len(rows)
    buf = np.frombuffer(b"".join(rows), np.uint8)
    if variant:
        return O.rope_fwht_rows_variant(buf, fmt, 64, n, 0, 64, 0, None, 64, variant)
    return O.rope_fwht_rows(buf, fmt, 64, n, 0, 64, 0, None, 64)


Q8_CODES = code_vectors((127, 127, 127, 126, 1))
Q8_CODES += [-c for c in Q8_CODES]
Q4_CODES = code_vectors((-8, -8, -8, -7, -1))


def tie_rows_q8():
    rows, want, ties = [], [], 0
    for c in Q8_CODES:
        rows.append(q8_row(c))
        e, t = expected_q8(c)
        want.append(e)
        ties += t
    return rows, b"".join(want), ties


def tie_rows_q4():
    rows, want, ties = [], [], 0
    for c in Q4_CODES:
        rows.append(q4_row(c))
        e, t = expected_q4(c)
        want.append(e)
        ties += t
    return rows, b"".join(want), ties


def test_q8_0_ties_round_away_from_zero():
    rows, want, ties = tie_rows_q8()
    assert ties > 1000  # half-integer products whose even neighbour differs
    got = transform(rows, O.FMT_Q8_0)
    assert got.tobytes() == want
    # ties to even would change those codes: the comparison above catches it
    rne = transform(rows, O.FMT_Q8_0, O.VAR_RNE)
    assert int(np.count_nonzero(rne != got)) == ties


def test_q4_0_ties_truncate_after_offset():
    rows, want, ties = tie_rows_q4()
    assert ties > 500
    got = transform(rows, O.FMT_Q4_0)
    assert got.tobytes() == want
    rne = transform(rows, O.FMT_Q4_0, O.VAR_RNE)
    assert np.count_nonzero(rne != got) > 0
    # the unfused x*id + 8.5 gives the same codes here: x*id is exact
    assert np.array_equal(transform(rows, O.FMT_Q4_0, O.VAR_UNFUSED_Q4), got)


def test_q8_0_requant_of_q8_0_input_has_no_other_ties():
    """GATHER_REQUANT_Q8_0 decodes q8_0 (c*ds) and requantizes: x*id is
    about 127*c/m (m the block's largest |code|), which is a half-integer
    only at c/m = +-1/2 (x*id = +-63.5, where away-from-zero and even both
    give +-64).  In binary32 arithmetic the computed products stay at least
    1/254 minus a few ulp away from every other half-integer: checked for
    every (c, m) and 400 block scales."""
    rng = np.random.default_rng(5)
    scales = np.concatenate([
        2.0 ** np.arange(-14, 16, dtype=np.float64),
        rng.uniform(0.001, 1000.0, 370)]).astype(np.float16).astype(np.float32)
    m = np.arange(1, 128, dtype=np.float32)[:, None]
    c = np.arange(-127, 128, dtype=np.float32)[None, :]
    valid = np.abs(c) <= m
    for ds in scales:
        x = (c * ds).astype(np.float32)
        amax = (m * ds).astype(np.float32)
        d = (amax / np.float32(127)).astype(np.float32)
        idv = (np.float32(1) / d).astype(np.float32)
        p = (x * idv).astype(np.float32)
        half = (p * 2 == np.floor(p * 2)) & (p != np.floor(p)) & valid
        assert np.all(np.abs(p[half]) == np.float32(63.5)), ds
        assert np.array_equal(np.round(np.abs(p[half])), np.full(np.count_nonzero(half), 64.0, np.float32))


def sensitivity(fmt, tokens=2048, width=1024, head_dim=128, seed=11):
    """Codes (and blocks) of the raw-K transform that change under each
    variant, on random q8_0/q4_0 history at the rawk shape (8 heads x 128,
    full rotation at positions up to 131072, Walsh-Hadamard 128)."""
    rng = np.random.default_rng(seed)
    nb = width // 32
    bb = 34 if fmt == O.FMT_Q8_0 else 18
    raw = rng.integers(0, 256, (tokens, nb, bb), dtype=np.uint8)
    raw[:, :, :2] = rng.uniform(0.01, 0.05, (tokens, nb)).astype(np.float16).view(np.uint8).reshape(tokens, nb, 2)
    raw = raw.reshape(-1)
    theta = (10000.0 ** (-np.arange(64) * 2 / 128)).astype(np.float32)
    pos0 = 131072 - tokens
    base = O.rope_fwht_rows(raw, fmt, width, tokens, pos0, head_dim, 128, theta, 128).reshape(tokens * nb, bb)
    out = {}
    for name, v in [("unfused rotation", O.VAR_UNFUSED_ROT), ("unfused q4_0 multiply-add", O.VAR_UNFUSED_Q4),
                    ("sin +1 ulp", O.VAR_SIN_UP), ("sin -1 ulp", O.VAR_SIN_DOWN), ("cos +1 ulp", O.VAR_COS_UP),
                    ("cos -1 ulp", O.VAR_COS_DOWN), ("ties to even", O.VAR_RNE)]:
        if v == O.VAR_UNFUSED_Q4 and fmt != O.FMT_Q4_0:
            continue
        var = O.rope_fwht_rows_variant(raw, fmt, width, tokens, pos0, head_dim, 128, theta, 128, v)
        var = var.reshape(tokens * nb, bb)
        if fmt == O.FMT_Q8_0:
            codes_changed = int(np.count_nonzero(var[:, 2:] != base[:, 2:]))
            total = tokens * width
        else:
            lo = lambda a: a[:, 2:] & 15  # noqa: E731
            hi = lambda a: a[:, 2:] >> 4  # noqa: E731
            codes_changed = int(np.count_nonzero(lo(var) != lo(base)) + np.count_nonzero(hi(var) != hi(base)))
            total = tokens * width
        scales_changed = int(np.count_nonzero(np.any(var[:, :2] != base[:, :2], axis=1)))
        out[name] = (codes_changed, total, scales_changed, tokens * nb)
    return out


@pytest.mark.parametrize("fmt", [O.FMT_Q8_0, O.FMT_Q4_0])
def test_transform_sensitivity_report(fmt, capsys):
    res = sensitivity(fmt)
    with capsys.disabled():
        print(f"\nraw-K transform sensitivity ({'q8_0' if fmt == O.FMT_Q8_0 else 'q4_0'}, 2048 rows x 1024):")
        for name, (codes, total, scales, blocks) in res.items():
            print(f"  {name:26s} {codes:6d} of {total} codes ({codes / total:.2e}), "
                  f"{scales} of {blocks} block scales")
    # one ulp in sin/cos or an unfused rounding moves a code only where a
    # product sits within an ulp of a rounding boundary: rare, never absent
    for name, (codes, total, _, _) in res.items():
        assert codes / total < 1e-4, name
    assert sum(codes + scales for codes, _, scales, _ in res.values()) > 0
