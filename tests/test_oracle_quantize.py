"""The oracle's quantizer, pinned by the reference's invariant tests
(test/quantize.test.js:22-223) and by hand-computed tie cases that separate
round-half-away-from-zero (quantize.js:25-27) from banker's rounding."""
import numpy as np
import pytest

import oracle_lib as O
from conftest import lcg


def frobenius(orig, approx):
    o, a = orig.astype(np.float64), approx.astype(np.float64)
    den = np.sum(o * o)
    return 0.0 if den == 0 else float(np.sqrt(np.sum((a - o) ** 2) / den))


# -------------------------------------------------------------------- int8

def test_int8_codes_stay_in_symmetric_grid():
    q, _ = O.quantize_int8(lcg(4 * 64, 1).reshape(4, 64))
    assert q.min() >= -127 and q.max() <= 127


def test_int8_peak_lands_on_127():
    W = np.array([[1, -2, 0.5, 0], [0.1, 0.05, -0.1, 0]], np.float32)
    q, s = O.quantize_int8(W)
    assert q[0, 1] == -127
    assert s[0] == np.float32(2 / 127)
    assert np.abs(q[1]).max() == 127


def test_int8_scales_per_row():
    cols = 32
    c = np.arange(cols)
    W = np.stack([100 * np.sin(c), 0.001 * np.cos(c)]).astype(np.float32)
    back = O.round_trip(W, "int8")
    assert frobenius(W[1], back[1]) < 0.01


def test_int8_zero_exact():
    back = O.round_trip(np.array([[0, 1, -1], [0, 0.5, 0]], np.float32), "int8")
    assert back[0, 0] == 0 and back[1, 0] == 0 and back[1, 2] == 0


def test_int8_all_zero_row():
    q, s = O.quantize_int8(np.array([[0, 0, 0, 0], [1, 2, 3, 4]], np.float32))
    assert s[0] == 0
    back = O.dequantize_int8(q, s)
    assert np.all(back[0] == 0) and np.isfinite(back[1, 3])


def test_int8_error_within_half_step():
    W = lcg(6 * 128, 7).reshape(6, 128)
    q, s = O.quantize_int8(W)
    back = O.dequantize_int8(q, s)
    for r in range(6):
        assert np.all(np.abs(back[r] - W[r]) <= s[r] / 2 * 1.0001)


def test_int8_negation_negates_codes():
    W = lcg(3 * 16, 11).reshape(3, 16)
    a, _ = O.quantize_int8(W)
    b, _ = O.quantize_int8(-W)
    np.testing.assert_array_equal(b, -a)


def test_int8_rounds_half_away_from_zero():
    # peak 127 -> scale 1 -> the codes are round(w): 0.5 -> 1, 2.5 -> 3, -2.5 -> -3, 63.5 -> 64.
    # Banker's rounding would give 0, 2, -2, 64; truncation 0, 2, -2, 63.
    W = np.array([[127, 0.5, 2.5, -2.5, 63.5, -0.5, 1.49999, -126.5]], np.float32)
    q, s = O.quantize_int8(W)
    assert s[0] == np.float32(1.0)
    assert list(q[0]) == [127, 1, 3, -3, 64, -1, 1, -127]


def test_int8_inverse_comes_from_the_f64_scale():
    # peak = 3 -> scale = 3/127 in f64. These f32 weights sit just inside a half level
    # with the f64 inverse (-106.4999997, -74.4999998) and just past it with the inverse
    # of the f32-stored scale (-106.50000008, -74.50000008): codes -106, -74 vs -107, -75.
    W = np.array([[3, -2.5157480239868164, -1.7598425149917603]], np.float32)
    q, s = O.quantize_int8(W)
    assert list(q[0]) == [127, -106, -74]
    assert s[0] == np.float32(3 / 127)


def test_int8_dequant_is_one_rounding_of_the_exact_product():
    W = lcg(8 * 256, 3).reshape(8, 256)
    q, s = O.quantize_int8(W)
    back = O.dequantize_int8(q, s)
    exact = (q.astype(np.float64) * s.astype(np.float64)[:, None]).astype(np.float32)
    np.testing.assert_array_equal(back, exact)
    # which equals the f32 product (an f32 multiply rounds once too)
    np.testing.assert_array_equal(back, q.astype(np.float32) * s[:, None])


# -------------------------------------------------------------------- int4

def levels(packed, cols):
    flat = packed.reshape(-1)
    out = np.empty(flat.size * 2, np.int32)
    out[0::2] = flat & 0x0F
    out[1::2] = flat >> 4
    return out.reshape(-1, cols)


def test_int4_packs_low_nibble_first_and_monotone():
    W = (np.arange(16) - 8).astype(np.float32)[None, :]
    q, s, z = O.quantize_int4(W, 16)
    assert q.size == 8
    lv = levels(q, 16)[0]
    assert lv.min() >= 0 and lv.max() <= 15
    assert np.all(np.diff(lv) >= 0)


def test_int4_zero_exact_in_positive_group():
    W = np.array([[0] + [1 + i * 0.1 for i in range(1, 32)]], np.float32)
    assert O.round_trip(W, "int4", 32)[0, 0] == 0


def test_int4_groups_independent():
    W = np.concatenate([50 * np.sin(np.arange(16)), 0.01 * np.cos(np.arange(16))]).astype(np.float32)[None]
    back = O.round_trip(W, "int4", 16)
    assert frobenius(W[0, 16:], back[0, 16:]) < 0.1


def test_int4_rejects_bad_groups():
    with pytest.raises(O.QuantizeError, match="does not divide"):
        O.quantize_int4(np.zeros((1, 100), np.float32), 32)
    with pytest.raises(O.QuantizeError, match="at least 2"):
        O.quantize_int4(np.zeros((1, 8), np.float32), 1)


def test_int4_constant_group():
    q, s, z = O.quantize_int4(np.zeros((1, 16), np.float32), 16)
    assert s[0, 0] == 0
    assert np.all(O.dequantize_int4(q, s, z, 16, 16) == 0)


def test_int4_error_within_half_step():
    W = lcg(128, 21)[None]
    q, s, z = O.quantize_int4(W, 32)
    back = O.dequantize_int4(q, s, z, 128, 32)
    for g in range(4):
        sl = slice(32 * g, 32 * g + 32)
        assert np.all(np.abs(back[0, sl] - W[0, sl]) <= s[0, g] / 2 * 1.0001)


def test_int4_hand_computed_levels_and_ties():
    # lo = -1, hi = 14 -> scale = 1, zero = round(1) = 1, level = round(w) + 1, clamped.
    W = np.array([[-1, 14, 0.5, 2.5, -0.5, 3.5, 0, 7.25, 12.5, -1, 5, 6, 9.5, 1.5, 13.49, 11]],
                 np.float32)
    q, s, z = O.quantize_int4(W, 16)
    assert s[0, 0] == 1 and z[0, 0] == 1
    assert list(levels(q, 16)[0]) == [0, 15, 2, 4, 0, 5, 1, 8, 14, 0, 6, 7, 11, 3, 14, 12]


def test_int4_zero_point_rounds_half_away():
    # lo = -2.5, hi = 12.5 -> scale = 1, zero = round(2.5) = 3 (banker's would give 2).
    W = np.array([[-2.5, 12.5] + [0] * 14], np.float32)
    q, s, z = O.quantize_int4(W, 16)
    assert s[0, 0] == 1 and z[0, 0] == 3
    lv = levels(q, 16)[0]
    assert lv[0] == 0 and lv[1] == 15 and lv[2] == 3   # round(-2.5) + 3 = 0; 12.5 -> 13 + 3 -> 15


def test_int4_dequant_formula():
    W = lcg(4 * 256, 5).reshape(4, 256)
    q, s, z = O.quantize_int4(W, 128)
    back = O.dequantize_int4(q, s, z, 256, 128)
    lv = levels(q, 256).astype(np.float64)
    exact = ((lv - np.repeat(z, 128, axis=1)) * np.repeat(s, 128, axis=1)).astype(np.float32)
    np.testing.assert_array_equal(back, exact)


# ------------------------------------------------------------- comparisons

def test_smaller_groups_more_accurate():
    W = lcg(512, 31)[None]
    prev = np.inf
    for g in [256, 128, 64, 32]:
        e = frobenius(W, O.round_trip(W, "int4", g))
        assert e < prev
        prev = e


def test_int8_beats_int4_by_a_wide_margin():
    W = lcg(4 * 256, 41).reshape(4, 256)
    e8 = frobenius(W, O.round_trip(W, "int8"))
    e4 = frobenius(W, O.round_trip(W, "int4", 128))
    assert e8 < e4 and e4 / e8 > 4


def test_bits_per_weight():
    L = O.lib()
    assert L.or_bits_per_weight(4, 896, 128) == 4 + 64 / 128
    assert L.or_bits_per_weight(4, 896, 64) == 4 + 64 / 64
    assert 8 < L.or_bits_per_weight(8, 896, 0) < 8.1
    assert L.or_bits_per_weight(16, 0, 0) == 16


# ------------------------------------------------------------ special values
# What the reference's arithmetic gives non-finite inputs, worked by hand from its
# JavaScript semantics: `m > peak` and `v < lo` skip NaN; Math.round(NaN) is NaN;
# Math.min/Math.max propagate NaN; a typed-array store turns NaN into 0; Infinity * 0
# and Infinity / Infinity are NaN; Math.max(0, -0) is +0.

def test_int8_nan_is_skipped_by_the_peak_and_stored_as_zero():
    q, s = O.quantize_int8(np.array([[np.nan, 0.5, -1.0, 0.0]], np.float32))
    assert s[0] == np.float32(1 / 127)
    np.testing.assert_array_equal(q[0], [0, 64, -127, 0])      # 63.5 rounds away to 64


def test_int8_infinite_peak_gives_infinite_scale_and_zero_codes():
    q, s = O.quantize_int8(np.array([[np.inf, 1.0, -3.0, 0.0], [np.nan] * 4], np.float32))
    assert np.isposinf(s[0]) and s[1] == 0
    np.testing.assert_array_equal(q, 0)


def test_int4_nan_in_a_group():
    # lo -15, hi 15: scale 2, zero round(7.5) = 8; 15 -> 7.5 -> 8 + 8 clamps to 15;
    # -15 -> -7.5 -> -8 + 8 = 0; 0 -> 8; NaN -> 0.
    q, s, z = O.quantize_int4(np.array([[np.nan, 15.0, -15.0, 0.0]], np.float32), 4)
    assert s[0, 0] == 2 and z[0, 0] == 8
    np.testing.assert_array_equal(q[0], [0xF0, 0x80])


def test_int4_infinite_range():
    # +inf: scale inf, zero round(-0/inf) = -0 -> Math.max(0, -0) = +0, inverse 0, levels 0.
    # -inf: -lo/scale = inf/inf = NaN, so the zero point is NaN and every level NaN -> 0.
    q, s, z = O.quantize_int4(np.array([[np.inf, 1.0, 0.0, 0.0, -np.inf, 1.0, 0.0, 0.0]], np.float32), 4)
    assert np.isposinf(s[0, 0]) and z[0, 0] == 0 and not np.signbit(z[0, 0])
    assert np.isposinf(s[0, 1]) and np.isnan(z[0, 1])
    np.testing.assert_array_equal(q, 0)


def test_int4_signed_zero_groups_have_zero_scale():
    q, s, z = O.quantize_int4(np.array([[-0.0, 0.0, 0.0, -0.0, np.nan, np.nan, np.nan, np.nan]], np.float32), 4)
    np.testing.assert_array_equal(s, 0)
    np.testing.assert_array_equal(z, 0)
    np.testing.assert_array_equal(q, 0)
