"""The Node-API binding (js/addon/qwen_napi.node) and the GpuModel-shaped JS driver
(js/gpu_model.js) over the same C ABI: exports, host-side helpers equal to the Python
binding's, and on the GPU the same logits (bit for bit) and greedy tokens as the Python
binding for the same seeded model."""
import base64
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
JS = os.path.join(ROOT, "llm-inference-webgpu_amd", "js")
ADDON = os.path.join(JS, "addon", "qwen_napi.node")

pytestmark = pytest.mark.skipif(not shutil.which("node"), reason="node is not installed")


def node(script, *args, timeout=120):
    r = subprocess.run(["node", "-e", script, *args], capture_output=True, text=True, timeout=timeout, cwd=JS)
    assert r.returncode == 0, r.stderr
    return r.stdout


@pytest.fixture(scope="module")
def addon_built():
    if not os.path.exists(ADDON):
        pytest.fail("qwen_napi.node is not built: run __graft_entry__.build()")
    return ADDON


def test_addon_exports_the_driver_surface(addon_built):
    keys = json.loads(node("const a=require('./addon/qwen_napi.node'); console.log(JSON.stringify(Object.keys(a)))"))
    assert set(keys) == {"abiVersion", "open", "close", "describe", "synthBf16", "synthTokens", "quantizeInt8",
                         "quantizeInt4", "modelCreate", "modelSetMode", "modelSetTensor", "modelLoadTensor", "modelFinalize",
                         "modelFree", "cacheCreate", "cacheFree", "cacheLength", "cachePresent", "forward", "decode", "score"}
    assert node("console.log(require('./addon/qwen_napi.node').abiVersion())").strip() == "1"


def test_host_helpers_equal_the_python_binding(addon_built, hip):
    out = json.loads(node(
        "const q=require('./gpu_model.js'); const a=q.addon;"
        "const w=q.bf16ToF32Array(a.synthBf16(5,'w',0.02,64*256));"
        "const r8=a.quantizeInt8(w,64,256), r4=a.quantizeInt4(w,64,256,128);"
        "console.log(JSON.stringify({t:Array.from(a.synthTokens(9,'ids',1000,32)),"
        "q8:Array.from(r8.q), s8:Array.from(r8.scales), q4:Array.from(r4.q), z4:Array.from(r4.zeros),"
        "s4:Array.from(r4.scales)}))"))
    w = hip.bf16_to_f32(hip.synth_bf16(5, "w", 0.02, 64 * 256)).reshape(64, 256)
    q8, s8 = hip.quantize_int8(w)
    q4, s4, z4 = hip.quantize_int4(w, 128)
    assert out["t"] == list(hip.synth_tokens(9, "ids", 1000, 32))
    assert out["q8"] == list(q8.ravel()) and np.array_equal(np.float32(out["s8"]), s8)
    assert out["q4"] == list(q4.ravel()) and np.array_equal(np.float32(out["s4"]), s4.ravel())
    assert np.array_equal(np.float32(out["z4"]), z4.ravel())


def test_js_f16_narrowing_matches_numpy(addon_built):
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(2000) * 10.0 ** rng.integers(-9, 6, 2000),
                        [0.0, -0.0, 65504.0, 65520.0, 1e5, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, np.inf, -np.inf]])
    x = x.astype(np.float32)
    got = json.loads(node("const q=require('./gpu_model.js'); const b=Buffer.from(process.argv[1],'base64');"
                          "const x=new Float32Array(b.buffer, b.byteOffset, b.length / 4);"
                          "console.log(JSON.stringify(Array.from(q.f32ToF16Array(x))))",
                          base64.b64encode(x.tobytes()).decode()))
    with np.errstate(over="ignore"):   # values past 65504 narrow to infinity, as intended
        want = x.astype(np.float16)
    assert got == list(want.view(np.uint16).astype(int))


def test_typed_arrays_are_checked_before_any_c_call(addon_built):
    """Arrays of the wrong element type, or shorter than rows * cols (or the groups, rows or seq
    they must cover), are refused in the binding with TypeError / RangeError, so no entry point
    reads past a caller's array."""
    out = json.loads(node(
        "const a=require('./addon/qwen_napi.node'); const r=[];"
        "const t=(f)=>{ try { f(); r.push(null); } catch (e) { r.push(e.constructor.name + ': ' + e.message); } };"
        "t(()=>a.quantizeInt8(new Float32Array(11), 3, 4));"
        "t(()=>a.quantizeInt8(new Float64Array(12), 3, 4));"
        "t(()=>a.quantizeInt4(new Float32Array(255), 1, 256, 128));"
        "t(()=>a.quantizeInt8(new Float32Array(12), 0, 4));"
        "t(()=>a.quantizeInt8([1, 2, 3], 1, 3));"
        "console.log(JSON.stringify(r));"))
    assert out[0].startswith("RangeError") and "holds 11 values where 12" in out[0]
    assert out[1].startswith("TypeError") and "Float32Array" in out[1]
    assert out[2].startswith("RangeError") and out[3].startswith("RangeError")
    assert out[4].startswith("TypeError")


def test_range_error_surfaces_as_js_range_error(addon_built):
    msg = node("const a=require('./addon/qwen_napi.node');"
               "try { a.quantizeInt4(new Float32Array(12), 1, 12, 5); } catch (e) { console.log(e.constructor.name) }")
    assert msg.strip() in ("Error", "RangeError")


@pytest.mark.gpu
@pytest.mark.parametrize("scheme,numerics,matmul,convert", [
    ("int4", "fast", "batched", "device"), ("int4", "fast", "batched", "host"), ("int8", "exact", "mfma", "device"),
    ("int8", "fast", "batched", "host"), ("f16", "fast", "matvec", "device"), ("f16", "exact", "batched", "host")])
def test_js_driver_matches_python_binding(addon_built, ctx, hip, scheme, numerics, matmul, convert):
    # The JS loader converts on the device or on the host; the Python side loads host-quantized
    # tensors, so equal logits also show the two conversions store the same bits.
    r = subprocess.run(["node", os.path.join(ROOT, "tests", "js", "tiny_decode.js"), scheme, numerics, matmul,
                        convert],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    js = json.loads(r.stdout)
    cfg = hip.ModelConfig(hidden=128, intermediate=256, layers=2, heads=2, kv_heads=1, vocab=1000)
    ckpt = hip.synthesize_checkpoint(cfg, seed=3)
    model = hip.GpuModel.load(ctx, hip.device_tensors(ckpt, cfg, scheme, 128, "f16" if scheme == "f16" else "int8"),
                              cfg, maxPositions=256, numerics=numerics, matmul=matmul)
    prompt = hip.synth_tokens(3, "prompt", cfg.vocab, 12)
    cache = model.newCache(64)
    out = model.forward_tokens(prompt, cache)
    gen = model.decode(cache, out["argmax"], 8)
    js_logits = np.frombuffer(base64.b64decode(js["logits"]), np.float32)
    np.testing.assert_array_equal(js_logits.view(np.uint32), out["logits"].view(np.uint32))
    assert js["argmax"] == out["argmax"] and js["tokens"] == list(gen)
    assert js["hiddenArgmax"] == out["argmax"]
    np.testing.assert_array_equal(np.frombuffer(base64.b64decode(js["hiddenLogits"]), np.float32), js_logits)
    assert js["cacheLength"] == 20 and js["rangeError"] is not None
    scored = model.newCache(64)
    np.testing.assert_array_equal(np.frombuffer(base64.b64decode(js["score"]), np.float64),
                                  model.score(prompt, scored))
    assert js["scoredLength"] == scored.length == 11
    scored.destroy()
    cache.destroy()
    model.destroy()


@pytest.mark.gpu
def test_reference_shaped_caller_drives_the_backend(addon_built, ctx, hip):
    """web/bench.html's loop over objects shaped exactly like the reference's ModelConfig and
    Safetensors (async readRaw, one tensor at an odd offset), f16 weights (quantize = null),
    two kv heads: the logits equal the Python binding's bit for bit, the greedy tokens too;
    `present` comes back position-major [length, kv_dim] as the reference GPU forward returns
    it (src/gpu/model.js:388-395), and web/model.html's reshape of it (toPresentLayout) gives
    the head-major present rows; cache.keys / values destroy the cache once all are
    destroyed; a second forward while one is pending is refused; batchTileFor and matmul
    'tiled' are the reference's."""
    r = subprocess.run(["node", os.path.join(ROOT, "tests", "js", "reference_caller.js")],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    js = json.loads(r.stdout)
    cfg = hip.ModelConfig(hidden=256, intermediate=256, layers=2, heads=4, kv_heads=2, vocab=1000)
    ckpt = hip.synthesize_checkpoint(cfg, seed=3)
    model = hip.GpuModel.load(ctx, hip.device_tensors(ckpt, cfg, "f16", 128, "f16"), cfg, maxPositions=64)
    prompt = hip.synth_tokens(3, "prompt", cfg.vocab, 12)
    cache = model.newCache(28)
    out = model.forward_tokens(prompt, cache)
    np.testing.assert_array_equal(np.frombuffer(base64.b64decode(js["firstLogits"]), np.uint32),
                                  out["logits"].view(np.uint32))
    gen = model.decode(cache, out["argmax"], 6)
    assert js["tokens"] == [out["argmax"]] + list(gen)
    assert cache.length == js["presentLength"] == 18
    for L in range(cfg.layers):
        pres = cache.present(L)   # [kv_heads, length, head_dim]
        for kind in ("key", "value"):
            rows = np.frombuffer(base64.b64decode(js["present"][L][kind]), np.float32)
            onnx = np.frombuffer(base64.b64decode(js["present"][L][kind + "Onnx"]), np.float32)
            np.testing.assert_array_equal(rows.reshape(18, 128), pres[kind].transpose(1, 0, 2).reshape(18, 128))
            np.testing.assert_array_equal(onnx, pres[kind].ravel())
            assert not np.array_equal(rows, onnx)
    assert js["rowsOk"] is True
    assert js["ticks"] == 26 and js["layers"] == 2 and js["warmBytes"] > 0 and js["freed"] is True
    assert js["hiddenBuffer"] is None and "already running" in js["busy"] and js["cacheLength"] == 19
    assert js["tiles"] == [1, 2, 2, 4, 4, 8, 8] and js["tiled"] is True and "matmul must be" in js["badMatmul"]
    cache.destroy()
    model.destroy()
