"""The C ABI on the CPU: the library loads, exports every symbol the header
declares, and its host-side logic (the quantizer the load path uses, the rope
tables, the seeded generator) agrees with the oracle and with independent
restatements. No kernel runs here."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle_lib as O
from conftest import ROOT, lcg

HEADER = os.path.join(ROOT, "include", "qwen_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|void\*|const char\*|int32_t)\s+(qh_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol(hip):
    lib = hip.load_library()
    names = declared_symbols()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert lib.qh_abi_version() == 1


# (context, caches) -> (slots, waves) of the list launch: the four config-3 shapes the bench
# times, the list lengths the GPU parity test uses for them, and short lists.
LIST_PLANS = [((128, 8192), (1, 1)), ((1024, 1024), (1, 4)), ((4096, 256), (1, 8)), ((32768, 32), (4, 8)),
              ((128, 128), (1, 1)), ((1024, 128), (1, 4)), ((4096, 128), (1, 8)), ((1000, 128), (1, 4)),
              ((4000, 128), (1, 8)), ((1, 5), (4, 1)), ((100, 5), (4, 1)), ((1000, 5), (64, 1)),
              ((5000, 5), (64, 1))]


@pytest.mark.parametrize("shape,plan", LIST_PLANS)
def test_attention_list_plan(hip, shape, plan):
    assert hip.attention_list_plan(shape[0], shape[1], 2) == plan
    with pytest.raises(hip.QwenHipError):
        hip.attention_list_plan(0, shape[1], 2)


def test_no_device_is_an_error_not_a_fallback(hip):
    if hip.device_count() > 0:
        pytest.skip("a device is present")
    with pytest.raises(hip.QwenHipError, match="no HIP device"):
        hip.GpuContext.create(0)


@pytest.mark.parametrize("rows,cols", [(896, 896), (128, 896), (64, 4864)])
def test_product_int8_quantizer_matches_oracle(hip, rows, cols):
    w = (np.random.default_rng(rows + cols).standard_normal((rows, cols)) * 0.02).astype(np.float32)
    w[3, :] = 0          # an all-zero row
    w[5, 7] = 1.0        # an outlier
    q, s = hip.quantize_int8(w)
    oq, os_ = O.quantize_int8(w)
    np.testing.assert_array_equal(q, oq)
    np.testing.assert_array_equal(s.view(np.uint32), os_.view(np.uint32))


@pytest.mark.parametrize("rows,cols,group", [(896, 896, 128), (128, 896, 128), (64, 4864, 128),
                                             (16, 256, 32), (8, 96, 2)])
def test_product_int4_quantizer_matches_oracle(hip, rows, cols, group):
    w = (np.random.default_rng(rows * cols).standard_normal((rows, cols)) * 0.02).astype(np.float32)
    w[2, :group] = 0.0                 # constant group
    w[4, :group] = np.abs(w[4, :group])  # all-positive group
    q, s, z = hip.quantize_int4(w, group)
    oq, os_, oz = O.quantize_int4(w, group)
    np.testing.assert_array_equal(q, oq)
    np.testing.assert_array_equal(s.view(np.uint32), os_.view(np.uint32))
    np.testing.assert_array_equal(z.view(np.uint32), oz.view(np.uint32))


def test_product_quantizers_match_oracle_on_special_values(hip):
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((8, 256)) * 0.02).astype(np.float32)
    w[0, ::5] = np.nan
    w[1, 3], w[2, 200] = np.inf, -np.inf
    w[3, :] = np.nan
    w[4, :] = -0.0
    w[5, :] = np.float32(1e-44) * np.sign(w[5, :])   # the f32 scale underflows, the f64 one does not
    w[6, :8] = [0.0, -0.0, 1e-40, 3.4e38, -3.4e38, 65520.0, 2.0 ** -25, np.nan]
    q, s = hip.quantize_int8(w)
    oq, os_ = O.quantize_int8(w)
    np.testing.assert_array_equal(q, oq)
    np.testing.assert_array_equal(s.view(np.uint32), os_.view(np.uint32))
    for group in (4, 32, 256):
        q, s, z = hip.quantize_int4(w, group)
        oq, os_, oz = O.quantize_int4(w, group)
        np.testing.assert_array_equal(q, oq)
        np.testing.assert_array_equal(s.view(np.uint32), os_.view(np.uint32))
        np.testing.assert_array_equal(z.view(np.uint32), oz.view(np.uint32))


def test_product_quantizer_tie_cases(hip):
    W = np.array([[127, 0.5, 2.5, -2.5, 63.5, -0.5, 1.49999, -126.5]], np.float32)
    q, _ = hip.quantize_int8(W)
    assert list(q[0]) == [127, 1, 3, -3, 64, -1, 1, -127]
    W = np.array([[-2.5, 12.5] + [0] * 14], np.float32)
    q, s, z = hip.quantize_int4(W, 16)
    assert z[0, 0] == 3 and (q[0, 0] & 0xF) == 0 and (q[0, 0] >> 4) == 15


def test_product_int4_rejects_bad_groups(hip):
    with pytest.raises(hip.RangeError, match="does not divide"):
        hip.quantize_int4(np.zeros((1, 100), np.float32), 32)
    with pytest.raises(hip.RangeError, match="at least 2"):
        hip.quantize_int4(np.zeros((1, 8), np.float32), 1)


def test_rope_tables_match_oracle(hip):
    cos, sin = hip.rope_tables(64, 1e6, 2048)
    ocos, osin = O.rope_tables(64, 1e6, 2048)
    np.testing.assert_array_equal(cos, ocos)
    np.testing.assert_array_equal(sin, osin)


# ---- the generator, restated independently in numpy uint64 arithmetic ----

M64 = (1 << 64) - 1
GOLDEN = 0x9E3779B97F4A7C15


def mix64(z):
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9 & M64
    z = (z ^ (z >> 27)) * 0x94D049BB133111EB & M64
    return z ^ (z >> 31)


def fnv1a(s):
    h = 0xCBF29CE484222325
    for ch in s.encode():
        h = ((h ^ ch) * 0x100000001B3) & M64
    return h


def ref_normal(seed, name, std, n, offset=0):
    key = mix64((fnv1a(name) + GOLDEN * (seed + 1)) & M64)
    out = []
    for i in range(offset, offset + n):
        total = 0
        for j in range(6):
            r = mix64((key + GOLDEN * (6 * i + j + 1)) & M64)
            total += (r & 0xFFFFFFFF) + (r >> 32)
        out.append(np.float32(std * ((total - 6 * (1 << 32)) / 2 ** 32)))
    return np.array(out, np.float32)


def test_synth_matches_restatement(hip):
    got = hip.synth_f32(1234, "model.layers.3.mlp.up_proj.weight", 0.02, 300, offset=1000)
    ref = ref_normal(1234, "model.layers.3.mlp.up_proj.weight", 0.02, 300, offset=1000)
    np.testing.assert_array_equal(got, ref)


def test_synth_is_counter_based_and_seeded(hip):
    a = hip.synth_f32(7, "x", 1.0, 100)
    b = hip.synth_f32(7, "x", 1.0, 60, offset=40)
    np.testing.assert_array_equal(a[40:], b)
    assert not np.array_equal(a, hip.synth_f32(8, "x", 1.0, 100))
    assert not np.array_equal(a, hip.synth_f32(7, "y", 1.0, 100))


def test_synth_moments(hip):
    v = hip.synth_f32(3, "moments", 0.02, 1 << 20).astype(np.float64)
    assert abs(v.mean()) < 1e-4
    assert abs(v.std() / 0.02 - 1) < 5e-3
    assert np.abs(v).max() <= 6 * 0.02


def test_synth_bf16_is_rne_of_f32(hip):
    f = hip.synth_f32(5, "w", 0.02, 4096)
    b = hip.synth_bf16(5, "w", 0.02, 4096)
    expect = np.array([O.lib().or_f32_to_bf16(float(v)) for v in f], np.uint16)
    np.testing.assert_array_equal(b, expect)


def test_synth_tokens_in_range(hip):
    t = hip.synth_tokens(11, "prompt", 151936, 4096)
    assert t.min() >= 0 and t.max() < 151936
    assert len(np.unique(t)) > 4000
