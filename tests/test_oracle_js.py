"""oracle/cpu_model.js -- the reference CPU path restated in JavaScript for Node 12, the
CPU baseline bench.py times under Node -- against the C oracle (oracle.c) on the same
quantized weights: greedy tokens identical and logits equal to f32 rounding (the two
evaluate the same f64 expressions; only V8's and libm's exp/cos/sin/pow may differ in a
last f64 bit)."""
import json
import shutil
import subprocess
import tempfile

import numpy as np
import pytest

import oracle_lib as O
from test_oracle_model import tiny_cfg, tiny_ckpt

pytestmark = pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


@pytest.mark.parametrize("scheme", ["int4", "int8"])
def test_js_decode_from_empty_cache_matches_c_oracle(scheme):
    cfg = tiny_cfg()
    ckpt = tiny_ckpt(cfg, seed=4)
    oracle = O.OracleModel(cfg, ckpt, scheme=scheme, group=128, lm_head="int8", kv_f16=True)
    want, _ = oracle.generate([7], 6)
    logits = oracle.forward([7], oracle.new_cache(4))
    with tempfile.TemporaryDirectory() as d:
        res = O.run_js_model(O.write_js_manifest(d, cfg, ckpt, scheme=scheme, first=7, steps=6))
    assert res["tokens"] == [int(t) for t in want]
    assert rel(res["logitsFirst"], logits[:8]) <= 1e-6


def test_js_continues_a_loaded_context_like_the_c_oracle():
    cfg = tiny_cfg(layers=3)
    ckpt = tiny_ckpt(cfg, seed=9)
    oracle = O.OracleModel(cfg, ckpt, scheme="int4", group=128, lm_head="int8", kv_f16=True)
    prompt = [3, 14, 15, 92, 65, 35]
    cache = oracle.new_cache(len(prompt) + 8)
    first = O.argmax(oracle.forward(prompt, cache))
    bits = O.js_cache_bits([cache.present(L) for L in range(cfg.layers)], len(prompt))
    want = []
    tok = first
    for _ in range(5):
        tok = O.argmax(oracle.forward([tok], cache))
        want.append(int(tok))
    with tempfile.TemporaryDirectory() as d:
        m = O.write_js_manifest(d, cfg, ckpt, scheme="int4", cache_bits=bits, context=len(prompt),
                                first=first, steps=5)
        res = O.run_js_model(m)
    assert res["tokens"] == want


def test_js_f16_narrowing_matches_numpy():
    # the cache's f16 rounding (src/core/dtype.js:81-113) over specials, subnormals and ties
    x = np.concatenate([np.array([0.0, -0.0, 1.0, 65504.0, 65520.0, 1e-8, 6.0e-8, 2.98e-8, np.inf, -np.inf,
                                  1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], np.float32),
                        np.random.default_rng(0).standard_normal(4000).astype(np.float32) * 3])
    code = ("const m = require(%r); const bits = JSON.parse(require('fs').readFileSync(0, 'utf8'));"
            "const f = new Float32Array(1), u = new Uint32Array(f.buffer);"
            "process.stdout.write(JSON.stringify(bits.map(function (b) { u[0] = b; return m.f32ToF16(f[0]); })));"
            ) % O.JS_MODEL
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    out = subprocess.run(["node", "-e", code], input=json.dumps([int(b) for b in x.view(np.uint32)]),
                         capture_output=True, text=True, check=True)
    np.testing.assert_array_equal(np.array(json.loads(out.stdout), np.uint16), want)
