"""The CPU oracle's numeric ops, pinned by the reference's known-answer tests
(test/ops.test.js) and by closed forms that a plausible mistake breaks."""
import math

import numpy as np
import pytest

import oracle_lib as O
from conftest import lcg, lcg_fast


def close(a, b, tol):
    assert abs(a - b) <= tol, f"{a} vs {b} (tolerance {tol})"


# ---------------------------------------------------------------- rmsNorm (ops.test.js:15-57)

def test_rmsnorm_unit_rms_with_unit_gain():
    out = O.rmsnorm([1, -2, 3, -4, 5], np.ones(5), 0)
    close(math.sqrt(float(np.mean(out.astype(np.float64) ** 2))), 1, 1e-6)


def test_rmsnorm_applies_gain_per_channel():
    out = O.rmsnorm([3, 4], [2, 10], 0)
    rms = math.sqrt(25 / 2)
    close(out[0], 3 / rms * 2, 1e-6)
    close(out[1], 4 / rms * 10, 1e-6)


def test_rmsnorm_eps_inside_the_root():
    out = O.rmsnorm([1e-4, 1e-4], [1, 1], 1e-6)
    expected = 1e-4 / math.sqrt(1e-8 + 1e-6)
    close(out[0], expected, 1e-9)
    assert abs(out[0] - 1e-4 / (math.sqrt(1e-8) + 1e-6)) > 0.5


def test_rmsnorm_scale_equivariant():
    a = O.rmsnorm([1, 2, 3, 4], np.ones(4), 0)
    b = O.rmsnorm([2, 4, 6, 8], np.ones(4), 0)
    np.testing.assert_allclose(a, b, atol=1e-6)


def test_rmsnorm_is_f64_statistic_stored_f32():
    # 896 values: the f64 sum over f32 squares differs from an f32 sum; the result
    # must equal the f64 evaluation rounded once.
    x = lcg(896, 5) * 7
    g = lcg(896, 6)
    x64, g64 = x.astype(np.float64), g.astype(np.float64)
    scale = 1 / math.sqrt(math.fsum(x64 * x64) / 896 + 1e-6)
    expected = ((x64 * scale) * g64).astype(np.float32)
    out = O.rmsnorm(x, g, 1e-6)
    assert np.max(np.abs(out.view(np.int32) - expected.view(np.int32))) <= 1


# ---------------------------------------------------------------- matVec (ops.test.js:61-100)

def test_matvec_rows_of_w_times_x():
    assert list(O.matvec([1, 2, 3, 4, 5, 6], [1, 0, -1], 2, 3)) == [-2, -2]


def test_matvec_adds_bias():
    assert list(O.matvec([1, 2, 3, 4, 5, 6], [1, 0, -1], 2, 3, bias=[10, 100])) == [8, 98]


def test_matvec_is_row_major_out_by_in():
    assert list(O.matvec([1, 2, 3, 4, 5, 6, 7, 8], [1, 10], 4, 2)) == [21, 43, 65, 87]


def test_matvec_bf16_agrees_with_widened():
    rows, cols = 7, 5
    vals = np.array([((i % 9) - 4) * 0.25 for i in range(rows * cols)], np.float32)
    bits = (vals.view(np.uint32) >> 16).astype(np.uint16)
    x = np.array([1, -2, 0.5, 3, -0.25], np.float32)
    np.testing.assert_allclose(O.matvec_bf16(bits, x, rows, cols), O.matvec(vals, x, rows, cols), atol=1e-6)


def test_matvec_accumulates_in_f64_from_the_bias():
    # A sum whose f32 evaluation loses the small terms: 2^24 + 1 + 1 + ... In f64 from the
    # bias every unit survives; in f32 none does.
    cols = 64
    W = np.ones((1, cols), np.float32)
    x = np.ones(cols, np.float32)
    got = O.matvec(W, x, 1, cols, bias=[2.0 ** 24])
    assert got[0] == np.float32(2.0 ** 24 + cols)


def test_matvec_matches_exact_rational_sum_at_layer_shapes():
    rng = np.random.default_rng(3)
    for rows, cols in [(128, 896), (64, 4864)]:
        W = rng.standard_normal((rows, cols)).astype(np.float32)
        x = rng.standard_normal(cols).astype(np.float32)
        b = rng.standard_normal(rows).astype(np.float32)
        got = O.matvec(W, x, rows, cols, b)
        exact = np.array([math.fsum([float(b[r])] + list((W[r].astype(np.float64) * x).tolist()))
                          for r in range(rows)])
        # f64 sequential error is ~1e-16 relative: after the f32 store it is within 1 ulp.
        np.testing.assert_allclose(got, exact.astype(np.float32), rtol=2 ** -23, atol=1e-30)


# ---------------------------------------------------------------- softmax (ops.test.js:104-151)

def test_softmax_is_a_distribution():
    x = O.softmax([1, 2, 3, 4])
    assert np.all((x > 0) & (x < 1))
    close(float(np.sum(x, dtype=np.float64)), 1, 1e-6)
    assert x[3] > x[2] > x[1]


def test_softmax_shift_invariant():
    np.testing.assert_allclose(O.softmax([1, 2, 3]), O.softmax([101, 102, 103]), atol=1e-6)


def test_softmax_survives_overflow_range():
    x = O.softmax([800, 801, 802])
    assert np.all(np.isfinite(x))
    close(float(np.sum(x, dtype=np.float64)), 1, 1e-6)


def test_softmax_prefix_leaves_rest():
    x = O.softmax([1, 1, 999, 999], 2)
    close(x[0], 0.5, 1e-6)
    close(x[1], 0.5, 1e-6)
    assert x[2] == 999


def test_one_element_softmax_is_exactly_one():
    assert O.softmax([-12345], 1)[0] == 1


# ---------------------------------------------------------------- silu (ops.test.js:155-171)

def test_silu_known_points():
    close(O.silu(0), 0, 1e-12)
    close(O.silu(1), 1 / (1 + math.exp(-1)), 1e-12)
    close(O.silu(-1), -1 / (1 + math.exp(1)), 1e-12)
    assert -0.279 < O.silu(-1.2784) < -0.278


def test_swiglu_multiplies_gated_branch():
    g = O.swiglu([1, -1, 0], [2, 3, 5])
    close(g[0], O.silu(1) * 2, 1e-6)
    close(g[1], O.silu(-1) * 3, 1e-6)
    close(g[2], 0, 1e-12)


# ---------------------------------------------------------------- rope (ops.test.js:175-316)

def test_rope_frequencies_decay_from_one():
    inv = O.rope_freqs(8, 10000)
    assert inv.size == 4
    close(inv[0], 1, 1e-12)
    assert np.all(np.diff(inv) < 0)
    close(inv[1], 10000 ** (-2 / 8), 1e-12)


def test_rope_preserves_pair_lengths():
    inv = O.rope_freqs(8, 10000)
    v = np.arange(1, 9, dtype=np.float32)
    before = v.copy()
    O.rope_inplace(v, 0, 8, 37, inv)
    for j in range(4):
        close(math.hypot(v[j], v[j + 4]), math.hypot(before[j], before[j + 4]), 1e-5)


def test_rope_is_half_split_not_interleaved():
    inv = O.rope_freqs(8, 10000)
    v = np.zeros(8, np.float32)
    v[0] = 1
    O.rope_inplace(v, 0, 8, 1, inv)
    close(v[0], math.cos(1), 1e-6)
    close(v[4], math.sin(1), 1e-6)
    close(v[1], 0, 1e-12)


def test_rope_position_zero_is_identity():
    inv = O.rope_freqs(8, 10000)
    v = np.arange(1, 9, dtype=np.float32)
    before = v.copy()
    O.rope_inplace(v, 0, 8, 0, inv)
    np.testing.assert_array_equal(v, before)


def test_rope_dot_depends_on_relative_position():
    hd, inv = 16, O.rope_freqs(16, 1e6)
    q0 = np.array([math.sin(i * 1.7) for i in range(hd)], np.float32)
    k0 = np.array([math.cos(i * 0.9) for i in range(hd)], np.float32)

    def dot_at(m, n):
        q, k = q0.copy(), k0.copy()
        O.rope_inplace(q, 0, hd, m, inv)
        O.rope_inplace(k, 0, hd, n, inv)
        return float(np.dot(q.astype(np.float64), k.astype(np.float64)))

    for m, n in [(0, 0), (5, 2), (100, 97), (1000, 997)]:
        close(dot_at(m, n), dot_at(m - n, 0), 1e-4)
    assert abs(dot_at(5, 2) - dot_at(5, 1)) > 1e-3


def test_rope_applies_at_offset_only():
    inv = O.rope_freqs(4, 10000)
    buf = np.array([9, 9, 9, 9, 1, 0, 0, 0, 7, 7, 7, 7], np.float32)
    O.rope_inplace(buf, 4, 4, 1, inv)
    assert list(buf[:4]) == [9, 9, 9, 9]
    assert list(buf[8:]) == [7, 7, 7, 7]
    close(buf[4], math.cos(1), 1e-6)


def test_rope_table_reproduces_direct_rotation():
    hd, theta, positions, heads = 64, 1e6, 40, 3
    cos, sin = O.rope_tables(hd, theta, positions)
    inv = O.rope_freqs(hd, theta)
    half = hd // 2
    assert cos.shape == (positions, half)
    for position in [0, 1, 7, 39]:
        direct = np.array([math.sin(i * 0.3) + 0.1 for i in range(heads * hd)], np.float32)
        via = direct.copy()
        for h in range(heads):
            O.rope_inplace(direct, h * hd, hd, position, inv)
        for h in range(heads):
            b = h * hd
            c, s = cos[position], sin[position]
            lo, hi = via[b:b + half].copy(), via[b + half:b + hd].copy()
            via[b:b + half] = lo * c - hi * s
            via[b + half:b + hd] = hi * c + lo * s
        np.testing.assert_allclose(via, direct, atol=1e-6)


def test_rope_table_identity_at_zero_and_bounded():
    cos, sin = O.rope_tables(64, 1e6, 2048)
    assert np.all(cos[0] == 1) and np.all(sin[0] == 0)
    assert np.all(np.abs(cos) <= 1.0000001) and np.all(np.abs(sin) <= 1.0000001)


def test_rope_table_matches_numpy_libm_within_one_ulp():
    # numpy's own cos/sin on the f64 angles: an independent evaluation.
    hd, theta, positions = 64, 1e6, 4096
    cos, sin = O.rope_tables(hd, theta, positions)
    j = np.arange(hd // 2)
    inv = np.power(theta, (-2.0 * j) / hd)
    ang = np.arange(positions, dtype=np.float64)[:, None] * inv[None, :]
    for got, ref in [(cos, np.cos(ang).astype(np.float32)), (sin, np.sin(ang).astype(np.float32))]:
        ulps = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
        assert ulps.max() <= 1


def test_argmax_strict_greater_semantics():
    assert O.argmax([1, 3, 3, 2]) == 1           # lowest index wins ties
    assert O.argmax([np.nan, 5, 6]) == 0         # NaN at 0 is never beaten by '>'
    assert O.argmax([1, np.nan, 2]) == 2         # NaN elsewhere never wins
    assert O.argmax([-0.0, 0.0]) == 0            # -0 == +0
    assert O.argmax([-np.inf, -np.inf]) == 0
    assert O.argmax([1, np.inf, np.inf]) == 1


@pytest.mark.parametrize("n", [2, 1000, 151936])
def test_nll_matches_log_softmax(n):
    """The oracle's perplexity term (web/perplexity.html:158-166) against scipy's log_softmax of
    the same f32 logits in f64, at several targets including the largest and smallest logit."""
    from scipy.special import log_softmax
    logits = lcg_fast(n, 7) * 12
    ref = log_softmax(logits.astype(np.float64))
    for t in sorted({0, n - 1, int(np.argmax(logits)), int(np.argmin(logits)), n // 3}):
        assert O.nll(logits, t) == pytest.approx(-ref[t], rel=1e-13, abs=1e-13)


def test_nll_closed_forms():
    # equal logits: the uniform distribution, -log(1/n) = log(n)
    assert O.nll(np.full(151936, 3.25, np.float32), 17) == pytest.approx(np.log(151936), rel=1e-15)
    # two logits a, b: -log softmax = log(1 + exp(b - a)) for the target a
    a, b = np.float32(1.5), np.float32(-2.0)
    assert O.nll([a, b], 0) == pytest.approx(np.log1p(np.exp(np.float64(b) - np.float64(a))), rel=1e-15)
    assert O.nll([a, b], 1) == pytest.approx(np.log1p(np.exp(np.float64(a) - np.float64(b))), rel=1e-15)
    # the max shift keeps large logits finite
    assert np.isfinite(O.nll([1e30, 0.0, -1e30], 1))
    assert O.nll([1e30, 0.0], 0) == 0.0
    # a NaN logit is skipped by the max but enters the sum (as the reference's loops do)
    assert np.isnan(O.nll([1.0, np.nan, 2.0], 2))


@pytest.mark.parametrize("n", [1, 17, 4864])
def test_swiglu_matches_f64_definition(n):
    g = lcg(n, 11) * 6
    u = lcg(n, 12) * 3
    g64 = g.astype(np.float64)
    expected = (g64 / (1 + np.exp(-g64)) * u.astype(np.float64)).astype(np.float32)
    got = O.swiglu(g, u)
    assert np.max(np.abs(got.view(np.int32) - expected.view(np.int32))) <= 1
