"""The load path's checkpoint handling on the CPU: the safetensors readers (Python and the
Node driver's) against the independent `safetensors` library and against malformed files
(every defect the format allows a header to have, reported together), and config.json
parsing / the checkpoint-vs-config check (src/core/config.js's ModelConfig surface). No
device is touched."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from conftest import ROOT

import checkpoint as C

JS_DIR = os.path.join(ROOT, "llm-inference-webgpu_amd", "js")
HAS_NODE = shutil.which("node") is not None

QWEN_CONFIG = {   # the public config.json of Qwen2.5-0.5B
    "architectures": ["Qwen2ForCausalLM"], "model_type": "qwen2", "hidden_act": "silu",
    "hidden_size": 896, "intermediate_size": 4864, "num_hidden_layers": 24,
    "num_attention_heads": 14, "num_key_value_heads": 2, "vocab_size": 151936,
    "max_position_embeddings": 32768, "rope_theta": 1000000.0, "rms_norm_eps": 1e-06,
    "tie_word_embeddings": True, "use_sliding_window": False, "sliding_window": 32768,
}


def tiny_cfg(hip, **kw):
    base = dict(hidden=128, intermediate=256, layers=2, heads=2, kv_heads=1, vocab=1000)
    base.update(kw)
    return hip.ModelConfig(**base)


def test_reader_agrees_with_the_safetensors_library(tmp_path):
    from safetensors.numpy import save_file
    rng = np.random.default_rng(0)
    tensors = {"a": rng.standard_normal((3, 5)).astype(np.float32), "b": rng.standard_normal(7).astype(np.float16),
               "c": np.arange(6, dtype=np.int32).reshape(2, 3), "empty": np.zeros((0, 4), np.float32)}
    path = str(tmp_path / "x.safetensors")
    save_file(tensors, path, metadata={"format": "pt"})
    st = C.Safetensors.open(path)
    assert sorted(st.names()) == sorted(tensors) and st.metadata == {"format": "pt"}
    for name, a in tensors.items():
        info = st.info(name)
        assert info.shape == a.shape and info.byte_length == a.nbytes
        assert st.read_raw(name).tobytes() == a.tobytes()
    np.testing.assert_array_equal(st.array("a"), tensors["a"])
    np.testing.assert_array_equal(st.array("b"), tensors["b"].view(np.uint16))


def test_writer_output_reads_back_in_the_safetensors_library(tmp_path):
    from safetensors.numpy import load_file
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    bits = np.array([0x3F80, 0xBF80, 0x7FC0], np.uint16)
    path = str(tmp_path / "w.safetensors")
    C.write(path, {"a": ("F32", a), "h": ("F16", bits)})
    got = load_file(path)
    np.testing.assert_array_equal(got["a"], a)
    np.testing.assert_array_equal(got["h"].view(np.uint16), bits)
    C.write(path, {"w": ("BF16", bits)})
    np.testing.assert_array_equal(C.Safetensors.open(path).array("w"), bits)


def raw_file(path, header, data=b"", header_len=None):
    text = json.dumps(header).encode() if not isinstance(header, bytes) else header
    with open(path, "wb") as f:
        f.write((len(text) if header_len is None else header_len).to_bytes(8, "little"))
        f.write(text)
        f.write(data)
    return str(path)


@pytest.mark.parametrize("header,data,header_len,match", [
    ({}, b"", 10 ** 6, "length prefix declares a 1000000-byte header"),
    (b"\xff\xfe{}", b"", None, "not UTF-8 JSON"),
    (b"[1, 2]", b"", None, "not an object of tensor records"),
    ({"t": {"dtype": "Q7", "shape": [1], "data_offsets": [0, 1]}}, b"\0", None, "not a safetensors element type"),
    ({"t": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 4]}}, b"\0" * 4, None,
     "not a list of non-negative integers"),
    ({"t": {"dtype": "F32", "shape": [1], "data_offsets": [0]}}, b"\0" * 4, None, r"is not \[start, stop\]"),
    ({"t": {"dtype": "F32", "shape": [1], "data_offsets": [4, 0]}}, b"\0" * 4, None, r"is not \[start, stop\]"),
    ({"t": {"dtype": "F32", "shape": [1], "data_offsets": [0, True]}}, b"\0" * 4, None, r"is not \[start, stop\]"),
    ({"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}, b"\0" * 4, None, "extend past the 4-byte buffer"),
    ({"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 4]}}, b"\0" * 8, None,
     "2 x F32 is 8 bytes, the record spans 4"),
    ({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
      "b": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}, b"\0" * 8, None,
     r"'b' \[4, 8\) overlaps 'a' \[0, 8\)"),
    # a shape whose element count wraps to 0 in 64-bit arithmetic is still 2**64 elements
    ({"t": {"dtype": "F32", "shape": [2 ** 32, 2 ** 32], "data_offsets": [0, 0]}}, b"", None,
     "18446744073709551616 x F32 is 73786976294838206464 bytes, the record spans 0"),
    ({"t": 7}, b"", None, "the record is a JSON int"),
    ({"__metadata__": {"k": 1}}, b"", None, "__metadata__ is not an object of strings"),
])
def test_reader_rejects_malformed_files(tmp_path, header, data, header_len, match):
    path = raw_file(tmp_path / "bad.safetensors", header, data, header_len)
    with pytest.raises(C.SafetensorsError, match=match):
        C.Safetensors.open(path)


def test_reader_reports_every_defect_at_once(tmp_path):
    header = {"a": {"dtype": "Q7", "shape": [1], "data_offsets": [0, 1]},
              "b": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]},
              "c": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
              "d": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}
    path = raw_file(tmp_path / "bad.safetensors", header, b"\0" * 8)
    with pytest.raises(C.SafetensorsError) as e:
        C.Safetensors.open(path)
    msg = str(e.value)
    assert "3 defects" in msg and "'a'" in msg and "3 x F32 is 12 bytes" in msg and "'d' [4, 8) overlaps 'c'" in msg


def test_reader_rejects_a_short_file(tmp_path):
    p = tmp_path / "short"
    p.write_bytes(b"1234")
    with pytest.raises(C.SafetensorsError, match="too short for a safetensors length prefix"):
        C.Safetensors.open(str(p))


def test_config_parse_gives_the_model_dimensions(hip):
    cfg = hip.ModelConfig.from_hf(QWEN_CONFIG)
    assert cfg == hip.QWEN25_05B
    assert (cfg.head_dim, cfg.kv_dim) == (64, 128)
    assert len(cfg.expected_tensors()) == 2 + 24 * 12
    untied = hip.ModelConfig.from_hf(json.dumps({**QWEN_CONFIG, "tie_word_embeddings": False}))
    assert untied.expected_tensors()["lm_head.weight"] == (151936, 896)


@pytest.mark.parametrize("change,match", [
    ({"model_type": "llama"}, "only the qwen2 architecture"), ({"hidden_act": "gelu"}, "SiLU-gated"),
    ({"use_sliding_window": True}, "whole context"), ({"num_attention_heads": 13}, "does not split into 13"),
    ({"num_key_value_heads": 3}, "do not group evenly over 3"), ({"rope_theta": None}, "positive finite number"),
    ({"vocab_size": "151936"}, "positive integer"), ({"num_hidden_layers": 24.0}, "positive integer"),
    ({"rms_norm_eps": float("nan")}, "positive finite number"),
])
def test_config_parse_refuses_what_the_engine_does_not_implement(hip, change, match):
    with pytest.raises(hip.QwenHipError, match=match):
        hip.ModelConfig.from_hf({**QWEN_CONFIG, **change})


def test_config_parse_reports_every_problem_at_once(hip):
    with pytest.raises(hip.QwenHipError) as e:
        hip.ModelConfig.from_hf({**QWEN_CONFIG, "model_type": "llama", "vocab_size": -1, "hidden_act": "relu"})
    msg = str(e.value)
    assert "vocab_size = -1" in msg and "llama" in msg and "relu" in msg


def test_check_against_reports_missing_extra_and_misshapen(hip, tmp_path):
    cfg = tiny_cfg(hip)
    ckpt = hip.synthesize_checkpoint(cfg, seed=1)
    path = str(tmp_path / "m.safetensors")
    C.write(path, {k: ("BF16", v) for k, v in ckpt.items()})
    assert cfg.check_against(C.Safetensors.open(path)) == 26
    bad = {k: ("BF16", v) for k, v in ckpt.items() if k != "model.norm.weight"}
    bad["model.layers.0.mlp.down_proj.weight"] = ("BF16", ckpt["model.layers.0.mlp.down_proj.weight"].T.copy())
    bad["extra.weight"] = ("BF16", np.zeros(2, np.uint16))
    C.write(path, bad)
    with pytest.raises(hip.QwenHipError) as e:
        cfg.check_against(C.Safetensors.open(path))
    msg = str(e.value)
    assert "1 missing (model.norm.weight)" in msg and "1 not part of the model (extra.weight)" in msg
    assert "model.layers.0.mlp.down_proj.weight is [256, 128] where the config implies [128, 256]" in msg


@pytest.mark.skipif(not HAS_NODE, reason="node is not installed")
def test_js_reader_reads_what_the_python_reader_reads(hip, tmp_path):
    cfg = tiny_cfg(hip)
    ckpt = hip.synthesize_checkpoint(cfg, seed=2)
    path = str(tmp_path / "model.safetensors")
    C.write(path, {k: ("BF16", v) for k, v in ckpt.items()} | {"x": ("F16", np.array([0x3C00, 0xC000], np.uint16))},
            metadata={"format": "pt"})
    code = ("const s=require('./safetensors.js'); const st=s.Safetensors.open(process.argv[1]);"
            "const out={meta:st.metadata, names:st.names()};"
            "out.sum=st.names().filter(n=>n!=='x').map(n=>Array.from(st.tensor(n).data).reduce((a,b)=>(a*31+b)%1000003,0));"
            "out.x=Array.from(st.tensor('x').data); st.close(); console.log(JSON.stringify(out));")
    r = subprocess.run(["node", "-e", code, path], cwd=JS_DIR, capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout)
    st = C.Safetensors.open(path)
    assert out["meta"] == {"format": "pt"} and out["names"] == st.names()

    def digest(a):
        h = 0
        for v in a.ravel().tolist():
            h = (h * 31 + v) % 1000003
        return h
    assert out["sum"] == [digest(st.array(n)) for n in st.names() if n != "x"]
    assert out["x"] == [1.0, -2.0]


@pytest.mark.skipif(not HAS_NODE, reason="node is not installed")
def test_js_reader_and_config_errors(tmp_path):
    path = raw_file(tmp_path / "bad.safetensors", {"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
                                                   "b": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}},
                    b"\0" * 8)
    code = ("const s=require('./safetensors.js'); const k=require('./config.js'); const r=[];"
            "try { s.Safetensors.open(process.argv[1]); } catch (e) { r.push(e.message); }"
            "try { k.parseConfig(Object.assign(JSON.parse(process.argv[2]), {model_type:'llama'})); } catch (e) { r.push(e.message); }"
            "const c=k.ModelConfig.parse(process.argv[2]); r.push([c.hiddenSize,c.numKVHeads,c.vocabSize,c.tieWordEmbeddings,c.headDim,c.kvDim]);"
            "r.push(c.expectedTensors().size);"
            "try { k.parseConfig(Object.assign(JSON.parse(process.argv[2]), {vocab_size:'x', num_attention_heads:13})); } catch (e) { r.push(e.message); }"
            "console.log(JSON.stringify(r));")
    r = subprocess.run(["node", "-e", code, path, json.dumps(QWEN_CONFIG)], cwd=JS_DIR, capture_output=True,
                       text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout)
    assert "'b' [4, 8) overlaps 'a' [0, 8)" in out[0] and "only the qwen2" in out[1]
    assert out[2] == [896, 2, 151936, True, 64, 128] and out[3] == 2 + 24 * 12
    assert 'vocab_size = "x"' in out[4] and "does not split into 13" in out[4]
