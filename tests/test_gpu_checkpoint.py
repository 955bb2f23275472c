"""A model loaded from a safetensors checkpoint (GpuModel.load_safetensors; the Node
driver's GpuModel.load over a Safetensors) against the same weights loaded from memory:
the stored codes are the device quantizer's, so the logits and greedy tokens must be
bit-identical -- for a tied bf16 checkpoint, an untied one (its own lm_head.weight), one
with f32 and f16 tensors, and through the Node driver."""
import base64
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from conftest import ROOT

import checkpoint as C

pytestmark = pytest.mark.gpu

HAS_NODE = shutil.which("node") is not None


def tiny(hip, tied=True):
    return hip.ModelConfig(hidden=128, intermediate=256, layers=2, heads=2, kv_heads=1, vocab=1000,
                           tie_word_embeddings=tied)


def hf_config(cfg):
    return {"model_type": "qwen2", "hidden_act": "silu", "hidden_size": cfg.hidden,
            "intermediate_size": cfg.intermediate, "num_hidden_layers": cfg.layers,
            "num_attention_heads": cfg.heads, "num_key_value_heads": cfg.kv_heads, "vocab_size": cfg.vocab,
            "max_position_embeddings": 32768, "rope_theta": cfg.rope_theta, "rms_norm_eps": cfg.eps,
            "tie_word_embeddings": cfg.tie_word_embeddings, "use_sliding_window": False}


def write_dir(tmp_path, cfg, tensors):
    with open(tmp_path / "config.json", "w") as f:
        json.dump(hf_config(cfg), f)
    C.write(str(tmp_path / "model.safetensors"), tensors, metadata={"format": "pt"})
    return str(tmp_path)


def run(hip, model, cfg):
    prompt = hip.synth_tokens(9, "prompt", cfg.vocab, 7)
    cache = model.newCache(32)
    out = model.forward_tokens(prompt, cache)
    gen = model.decode(cache, out["argmax"], 8)
    cache.destroy()
    return out["logits"], out["argmax"], list(gen)


def assert_same(a, b):
    np.testing.assert_array_equal(a[0].view(np.uint32), b[0].view(np.uint32))
    assert a[1:] == b[1:]


@pytest.mark.parametrize("scheme,head", [("int4", "int8"), ("int8", "int8"), ("f16", "f16")])
def test_tied_bf16_checkpoint_equals_memory_load(ctx, hip, tmp_path, scheme, head):
    cfg = tiny(hip)
    ckpt = hip.synthesize_checkpoint(cfg, seed=9)
    d = write_dir(tmp_path, cfg, {k: ("BF16", v) for k, v in ckpt.items()})
    a = hip.GpuModel.load_safetensors(ctx, d, None, scheme, 128, head, maxPositions=64)
    b = hip.GpuModel.load(ctx, hip.device_tensors(ckpt, cfg, scheme, 128, head), cfg, maxPositions=64)
    assert a.config == cfg and a.device_bytes == b.device_bytes
    assert_same(run(hip, a, cfg), run(hip, b, cfg))
    a.destroy()
    b.destroy()


def test_untied_checkpoint_uses_its_own_output_projection(ctx, hip, tmp_path):
    cfg = tiny(hip, tied=False)
    ckpt = hip.synthesize_checkpoint(cfg, seed=4)
    lm = hip.synth_bf16(4, "lm_head.weight", 0.02, cfg.vocab * cfg.hidden).reshape(cfg.vocab, cfg.hidden)
    d = write_dir(tmp_path, cfg, {k: ("BF16", v) for k, v in ckpt.items()} | {"lm_head.weight": ("BF16", lm)})
    a = hip.GpuModel.load_safetensors(ctx, d, None, "int4", 128, "int8", maxPositions=64)
    tensors = hip.device_tensors(ckpt, cfg, "int4", 128, "int8")
    q, s = hip.quantize_int8(hip.bf16_to_f32(lm))
    tensors["lm_head.weight"] = (hip.FMT_INT8, cfg.vocab, cfg.hidden, 0, q, s, None)
    b = hip.GpuModel.load(ctx, tensors, cfg, maxPositions=64)
    tied = hip.GpuModel.load(ctx, hip.device_tensors(ckpt, cfg, "int4", 128, "int8"), cfg, maxPositions=64)
    ra, rb, rt = run(hip, a, cfg), run(hip, b, cfg), run(hip, tied, cfg)
    assert_same(ra, rb)
    assert not np.array_equal(ra[0], rt[0])   # the separate head is the one in use
    for m in (a, b, tied):
        m.destroy()


def test_f32_and_f16_tensors_are_widened_exactly(ctx, hip, tmp_path):
    cfg = tiny(hip)
    ckpt = hip.synthesize_checkpoint(cfg, seed=5)
    wide = {k: hip.bf16_to_f32(v) for k, v in ckpt.items()}
    # Norms and biases as F32, the MLP matrices as F16; the memory load gets the same values widened.
    tensors, ref = {}, {}
    for k, v in ckpt.items():
        if k == "model.embed_tokens.weight":
            tensors[k], ref[k] = ("BF16", v), v
        elif v.ndim == 1:
            tensors[k], ref[k] = ("F32", wide[k]), wide[k]
        elif "mlp" in k:
            h = wide[k].astype(np.float16)
            tensors[k], ref[k] = ("F16", h.view(np.uint16)), h.astype(np.float32)
        else:
            tensors[k], ref[k] = ("BF16", v), v
    d = write_dir(tmp_path, cfg, tensors)
    a = hip.GpuModel.load_safetensors(ctx, d, None, "int8", 128, "int8", maxPositions=64)
    b = hip.GpuModel.load_checkpoint(ctx, ref, cfg, "int8", 128, "int8", maxPositions=64)
    assert_same(run(hip, a, cfg), run(hip, b, cfg))
    a.destroy()
    b.destroy()


def test_file_that_disagrees_with_its_config_is_refused_before_upload(ctx, hip, tmp_path):
    cfg = tiny(hip)
    ckpt = hip.synthesize_checkpoint(cfg, seed=6)
    d = write_dir(tmp_path, hip.ModelConfig(hidden=128, intermediate=384, layers=2, heads=2, kv_heads=1, vocab=1000),
                  {k: ("BF16", v) for k, v in ckpt.items()})
    with pytest.raises(hip.QwenHipError, match="the checkpoint does not match the config: 6 misshapen"):
        hip.GpuModel.load_safetensors(ctx, d)


@pytest.mark.skipif(not HAS_NODE, reason="node is not installed")
@pytest.mark.parametrize("convert", ["device", "host"])
def test_node_driver_loads_the_file_like_the_python_binding(ctx, hip, tmp_path, convert):
    cfg = tiny(hip)
    ckpt = hip.synthesize_checkpoint(cfg, seed=9)
    d = write_dir(tmp_path, cfg, {k: ("BF16", v) for k, v in ckpt.items()})
    r = subprocess.run(["node", os.path.join(ROOT, "tests", "js", "file_decode.js"), d, "int4", "int8", convert],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    js = json.loads(r.stdout)
    a = hip.GpuModel.load_safetensors(ctx, d, None, "int4", 128, "int8", maxPositions=64)
    logits, argmax, gen = run(hip, a, cfg)
    np.testing.assert_array_equal(np.frombuffer(base64.b64decode(js["logits"]), np.float32).view(np.uint32),
                                  logits.view(np.uint32))
    assert js["argmax"] == argmax and js["tokens"] == gen
    a.destroy()
