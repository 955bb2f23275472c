"""The oracle's float conversions (src/core/dtype.js), checked exhaustively
against independent implementations: numpy's float16 and torch's bfloat16
(test/dtype.test.js uses V8's Float16Array for the same purpose)."""
import numpy as np
import torch

import oracle_lib as O

ALL = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)


def is_nan16(b):
    return ((b & 0x7C00) == 0x7C00) & ((b & 0x03FF) != 0)


def test_f16_widening_exhaustive_vs_numpy():
    got = O.f16_to_f32(ALL)
    ref = ALL.view(np.float16).astype(np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_f16_round_trip_every_value():
    back = O.f32_to_f16(O.f16_to_f32(ALL))
    keep = ~is_nan16(ALL)
    np.testing.assert_array_equal(back[keep], ALL[keep])
    assert np.all(is_nan16(back[~keep]))


def test_f16_narrowing_vs_numpy_on_every_f32_exponent():
    # Every f32 exponent with a spread of mantissas, plus all halfway cases around f16 values.
    rng = np.random.default_rng(0)
    exps = np.repeat(np.arange(256, dtype=np.uint32), 4096)
    mant = rng.integers(0, 1 << 23, exps.size, dtype=np.uint32)
    sign = rng.integers(0, 2, exps.size, dtype=np.uint32)
    bits = (sign << 31) | (exps << 23) | mant
    halves = O.f16_to_f32(ALL[~is_nan16(ALL)]).view(np.uint32)
    ties = np.concatenate([halves + (1 << 12), halves - (1 << 12), halves + 1, halves - 1])
    bits = np.concatenate([bits, ties.astype(np.uint32)])
    x = bits.view(np.float32)
    got = O.f32_to_f16(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    np.testing.assert_array_equal(got[~nan], ref[~nan])
    assert np.all(is_nan16(got[nan]))


def test_f16_overflow_and_underflow():
    assert O.f32_to_f16(np.array([65520.0], np.float32))[0] == 0x7C00   # rounds up to inf
    assert O.f32_to_f16(np.array([65519.0], np.float32))[0] == 0x7BFF
    assert O.f32_to_f16(np.array([2.0 ** -25], np.float32))[0] == 0      # tie to even: 0
    assert O.f32_to_f16(np.array([2.0 ** -24], np.float32))[0] == 1      # smallest subnormal
    assert O.f32_to_f16(np.array([-0.0], np.float32))[0] == 0x8000


def test_bf16_widening_is_a_shift_for_all_values():
    got = O.bf16_to_f32(ALL).view(np.uint32)
    np.testing.assert_array_equal(got, ALL.astype(np.uint32) << 16)


def test_bf16_narrowing_vs_torch():
    L = O.lib()
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 1 << 32, 200000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    got = np.array([L.or_f32_to_bf16(float(v)) for v in x[:20000]], np.uint16)
    ref = torch.from_numpy(x[:20000].copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, ref)


def test_bf16_ties_to_even_and_nan():
    L = O.lib()
    assert L.or_f32_to_bf16(float(np.uint32(0x3F808000).view(np.float32))) == 0x3F80
    assert L.or_f32_to_bf16(float(np.uint32(0x3F818000).view(np.float32))) == 0x3F82
    nan = np.uint32(0x7F800001).view(np.float32)
    b = L.or_f32_to_bf16(float(nan))
    assert (b & 0x7F80) == 0x7F80 and (b & 0x7F) != 0
