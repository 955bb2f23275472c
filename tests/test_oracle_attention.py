"""The oracle's grouped attention, pinned as the reference pins it
(test/attention.test.js): an expanded-heads brute force that must agree
exactly, causality, the single-position closed form, the convex hull, plus an
f64 brute force at long contexts."""
import math

import numpy as np
import pytest

import oracle_lib as O
from conftest import lcg

QWEN = dict(num_heads=14, num_kv_heads=2, head_dim=64)


def f32(v):
    return float(np.float32(v))


def expanded_attention(q, keys, values, seq, past, num_heads, num_kv_heads, head_dim):
    """test/attention.test.js:15-58: repeat each kv head `group` times, then plain
    multi-head attention with the same f64-accumulate / f32-store steps."""
    group = num_heads // num_kv_heads
    q_dim, kv_dim, total = num_heads * head_dim, num_kv_heads * head_dim, past + seq
    wide_k = np.empty((total, q_dim), np.float32)
    wide_v = np.empty((total, q_dim), np.float32)
    for s in range(total):
        for h in range(num_heads):
            src = s * kv_dim + (h // group) * head_dim
            wide_k[s, h * head_dim:(h + 1) * head_dim] = keys[src:src + head_dim]
            wide_v[s, h * head_dim:(h + 1) * head_dim] = values[src:src + head_dim]
    out = [0.0] * (seq * q_dim)
    scale = 1 / math.sqrt(head_dim)
    for h in range(num_heads):
        for t in range(seq):
            up_to = past + t
            qb = t * q_dim + h * head_dim
            qv = [float(v) for v in q[qb:qb + head_dim]]
            scores = []
            for s in range(up_to + 1):
                kv = wide_k[s, h * head_dim:(h + 1) * head_dim]
                dot = 0.0
                for i in range(head_dim):
                    dot += qv[i] * float(kv[i])
                scores.append(f32(dot * scale))
            mx = max(scores)
            es, ssum = [], 0.0
            for sc in scores:
                e = math.exp(sc - mx)
                es.append(f32(e))
                ssum += e
            inv = 1 / ssum
            probs = [f32(e * inv) for e in es]
            ob = t * q_dim + h * head_dim
            for s in range(up_to + 1):
                vv = wide_v[s, h * head_dim:(h + 1) * head_dim]
                for i in range(head_dim):
                    out[ob + i] = f32(out[ob + i] + probs[s] * float(vv[i]))
    return np.array(out, np.float32)


def run(seq, past, num_heads, num_kv_heads, head_dim, seed=1):
    total = past + seq
    q = lcg(seq * num_heads * head_dim, seed)
    k = lcg(total * num_kv_heads * head_dim, seed + 1)
    v = lcg(total * num_kv_heads * head_dim, seed + 2)
    mine = O.grouped_attention(q, k, v, seq, past, num_heads, num_kv_heads, head_dim)
    ref = expanded_attention(q, k, v, seq, past, num_heads, num_kv_heads, head_dim)
    return mine, ref


def test_head_map_is_blocked():
    mapping = [O.kv_head_for(h, 14, 2) for h in range(14)]
    assert mapping == [0] * 7 + [1] * 7
    assert mapping != [h % 2 for h in range(14)]
    assert [mapping.count(0), mapping.count(1)] == [7, 7]


@pytest.mark.parametrize("shape,seed", [
    (dict(seq=5, past=0, **QWEN), 1),
    (dict(seq=1, past=11, **QWEN), 99),
    (dict(seq=3, past=7, **QWEN), 4242),
    (dict(seq=4, past=2, num_heads=4, num_kv_heads=4, head_dim=8), 1),
    (dict(seq=4, past=3, num_heads=6, num_kv_heads=1, head_dim=8), 1),
])
def test_grouped_equals_expanded_exactly(shape, seed):
    mine, ref = run(**shape, seed=seed)
    np.testing.assert_array_equal(mine, ref)


def test_causal():
    seq, nh, nkv, hd = 4, 4, 2, 8
    q_dim, kv_dim = nh * hd, nkv * hd
    q, k, v = lcg(seq * q_dim, 7), lcg(seq * kv_dim, 8), lcg(seq * kv_dim, 9)
    before = O.grouped_attention(q, k, v, seq, 0, nh, nkv, hd)
    k2, v2 = k.copy(), v.copy()
    k2[(seq - 1) * kv_dim:] += 3.5
    v2[(seq - 1) * kv_dim:] -= 2.25
    after = O.grouped_attention(q, k2, v2, seq, 0, nh, nkv, hd)
    np.testing.assert_array_equal(after[:(seq - 1) * q_dim], before[:(seq - 1) * q_dim])
    assert np.any(after[(seq - 1) * q_dim:] != before[(seq - 1) * q_dim:])


def test_first_position_returns_its_value():
    nh, nkv, hd = 4, 2, 8
    q, k, v = lcg(nh * hd, 21), lcg(nkv * hd, 22), lcg(nkv * hd, 23)
    out = O.grouped_attention(q, k, v, 1, 0, nh, nkv, hd)
    for h in range(nh):
        kb = O.kv_head_for(h, nh, nkv) * hd
        np.testing.assert_array_equal(out[h * hd:(h + 1) * hd], v[kb:kb + hd])


def test_convex_combination():
    seq, nh, nkv, hd = 6, 4, 2, 8
    q_dim, kv_dim = nh * hd, nkv * hd
    q, k, v = lcg(seq * q_dim, 31), lcg(seq * kv_dim, 32), lcg(seq * kv_dim, 33)
    out = O.grouped_attention(q, k, v, seq, 0, nh, nkv, hd).reshape(seq, nh, hd)
    vv = v.reshape(seq, nkv, hd)
    for h in range(nh):
        g = O.kv_head_for(h, nh, nkv)
        for t in range(seq):
            lo, hi = vv[:t + 1, g].min(axis=0), vv[:t + 1, g].max(axis=0)
            assert np.all(out[t, h] >= lo - 1e-6) and np.all(out[t, h] <= hi + 1e-6)


@pytest.mark.parametrize("ctx", [128, 1024, 4096])
def test_long_context_against_f64_brute_force(ctx):
    # Config 3's shape: one query, 14 heads over 2 kv heads, f16-valued K/V ~ N(0,1).
    rng = np.random.default_rng(ctx)
    nh, nkv, hd = 14, 2, 64
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = O.through_f16(rng.standard_normal(ctx * nkv * hd).astype(np.float32))
    v = O.through_f16(rng.standard_normal(ctx * nkv * hd).astype(np.float32))
    got = O.grouped_attention(q, k, v, 1, ctx - 1, nh, nkv, hd).reshape(nh, hd)
    K = k.reshape(ctx, nkv, hd).astype(np.float64)
    V = v.reshape(ctx, nkv, hd).astype(np.float64)
    for h in range(nh):
        g = h // 7
        s = K[:, g] @ q[h * hd:(h + 1) * hd].astype(np.float64) / 8
        p = np.exp(s - s.max())
        p /= p.sum()
        ref = p @ V[:, g]
        # The reference's PV sum is sequential f32, so it is not exact: ~ctx * 2^-24.
        assert np.max(np.abs(got[h] - ref)) <= 1e-7 * ctx + 1e-6
