"""ctypes binding of libqwen_hip.so for Python callers (tests, bench.py).

Mirrors the reference's GPU layer interface (abho7/llm-inference-webgpu):
``GpuContext`` (src/gpu/device.js:21-392) and ``GpuModel`` / ``GpuKVCache``
(src/gpu/model.js:69-403), with the same method names and argument meaning:
``GpuModel.load(ctx, tensors, config, maxPositions=..., quantize=...)``,
``model.newCache(capacity)``, ``model.forward(hidden, seq, cache=..., wantLogits=...)``.
Misuse raises ``RangeError`` / ``QwenHipError`` synchronously, as the reference
throws ``RangeError`` / ``Error``.

Everything here only marshals arguments: the arithmetic runs in the HIP
kernels behind the C ABI (include/qwen_hip.h). There is no CPU fallback; if the
library is missing or no device is present, calls raise.
"""
from __future__ import annotations

import ctypes
import json
import math
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqwen_hip.so")

QH_OK, QH_ERR_INVALID, QH_ERR_RANGE, QH_ERR_BUSY, QH_ERR_DEVICE, QH_ERR_NOMEM, QH_ERR_STATE = range(7)
FMT_F32, FMT_F16, FMT_INT8, FMT_INT4, FMT_BF16 = range(5)
NUMERICS = {"fast": 0, "exact": 1}
MATMUL = {"batched": 0, "matvec": 1, "mfma": 2}
FORMAT_OF = {"f32": FMT_F32, "f16": FMT_F16, "int8": FMT_INT8, "int4": FMT_INT4, "bf16": FMT_BF16}
# Kernel roles of a decode step, in QH_ROLE_* order.
ROLES = ("embed", "qkv", "attention", "oproj", "gateup", "down", "head")
# Decode-state vectors of a cache, in QH_VEC_* order.
VECTORS = ("x", "q", "h", "logits", "key", "value")


class QwenHipError(RuntimeError):
    """A failing libqwen_hip call; ``code`` is the C status."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class RangeError(QwenHipError):
    """Capacity, rope-table or vocabulary overflow (the reference's RangeError)."""


class BusyError(QwenHipError):
    """forward() while another is running (src/gpu/model.js:231)."""


class Weight(ctypes.Structure):
    _fields_ = [("format", ctypes.c_int32), ("rows", ctypes.c_int32), ("cols", ctypes.c_int32),
                ("group", ctypes.c_int32), ("d_data", ctypes.c_void_p),
                ("d_scales", ctypes.c_void_p), ("d_zeros", ctypes.c_void_p)]


class Config(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int32), ("intermediate", ctypes.c_int32),
                ("layers", ctypes.c_int32), ("heads", ctypes.c_int32),
                ("kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("vocab", ctypes.c_int32), ("rope_theta", ctypes.c_double),
                ("eps", ctypes.c_double), ("max_positions", ctypes.c_int32)]


# The config.json fields a model is built from: (attribute, key, kind), where a "count" is a
# positive integer and a "real" a positive finite number. max_position_embeddings is checked
# but not kept (the rope table is sized by the caller's maxPositions).
_HF_FIELDS = (
    ("hidden", "hidden_size", "count"), ("intermediate", "intermediate_size", "count"),
    ("layers", "num_hidden_layers", "count"), ("heads", "num_attention_heads", "count"),
    ("kv_heads", "num_key_value_heads", "count"), ("vocab", "vocab_size", "count"),
    (None, "max_position_embeddings", "count"), ("rope_theta", "rope_theta", "real"),
    ("eps", "rms_norm_eps", "real"),
)

# The tensors of one decoder layer (checkpoint names, src/core/config.js:88-119) and their
# shapes in terms of d = hidden, k = kv_dim, f = intermediate.
_LAYER_TENSORS = (
    ("input_layernorm.weight", "d"), ("post_attention_layernorm.weight", "d"),
    ("self_attn.q_proj.weight", "dd"), ("self_attn.q_proj.bias", "d"),
    ("self_attn.k_proj.weight", "kd"), ("self_attn.k_proj.bias", "k"),
    ("self_attn.v_proj.weight", "kd"), ("self_attn.v_proj.bias", "k"),
    ("self_attn.o_proj.weight", "dd"),
    ("mlp.gate_proj.weight", "fd"), ("mlp.up_proj.weight", "fd"), ("mlp.down_proj.weight", "df"),
)


def _field_ok(v, kind) -> bool:
    if isinstance(v, bool) or not isinstance(v, (int, float)):
        return False
    if kind == "count":
        return isinstance(v, int) and v > 0
    return math.isfinite(v) and v > 0


def _few(names, n=4) -> str:
    return ", ".join(names[:n]) + (f", ... ({len(names) - n} more)" if len(names) > n else "")


@dataclass(frozen=True)
class ModelConfig:
    """The model's dimensions, from config.json (the fields of src/core/config.js's ModelConfig;
    headDim, kvDim and the GQA group follow from them)."""

    hidden: int = 896
    intermediate: int = 4864
    layers: int = 24
    heads: int = 14
    kv_heads: int = 2
    vocab: int = 151936
    rope_theta: float = 1e6
    eps: float = 1e-6
    tie_word_embeddings: bool = True

    @staticmethod
    def from_hf(raw) -> "ModelConfig":
        """From a config.json given as a path, JSON text or a dict. Every field is checked and all
        problems are reported together; architectures other than the one the kernels implement
        (qwen2: SiLU-gated MLP, full-context GQA attention) are refused."""
        if isinstance(raw, str):
            raw = json.loads(open(raw).read() if os.path.exists(raw) else raw)
        if not isinstance(raw, dict):
            raise QwenHipError(QH_ERR_INVALID, f"config.json holds a JSON {type(raw).__name__}, not an object")
        problems, got = [], {}
        for attr, key, kind in _HF_FIELDS:
            v = raw.get(key)
            if not _field_ok(v, kind):
                what = "positive integer" if kind == "count" else "positive finite number"
                problems.append(f"{key} = {json.dumps(v)} is not a {what}")
            elif attr is not None:
                got[attr] = v
        if raw.get("model_type") != "qwen2":
            problems.append(f"model_type {json.dumps(raw.get('model_type'))}: only the qwen2 architecture is built here")
        if raw.get("hidden_act", "silu") != "silu":
            problems.append(f"hidden_act {json.dumps(raw.get('hidden_act'))}: the MLP here is SiLU-gated")
        if raw.get("use_sliding_window") is True:
            problems.append("use_sliding_window: attention here always spans the whole context")
        if "hidden" in got and "heads" in got and got["hidden"] % got["heads"]:
            problems.append(f"hidden_size {got['hidden']} does not split into {got['heads']} equal heads")
        if "heads" in got and "kv_heads" in got and got["heads"] % got["kv_heads"]:
            problems.append(f"{got['heads']} query heads do not group evenly over {got['kv_heads']} key/value heads")
        if problems:
            raise QwenHipError(QH_ERR_INVALID, "config.json describes no model this engine runs: "
                               + "; ".join(problems))
        return ModelConfig(hidden=got["hidden"], intermediate=got["intermediate"], layers=got["layers"],
                           heads=got["heads"], kv_heads=got["kv_heads"], vocab=got["vocab"],
                           rope_theta=float(got["rope_theta"]), eps=float(got["eps"]),
                           tie_word_embeddings=raw.get("tie_word_embeddings") is True)

    def expected_tensors(self) -> dict:
        """Every tensor the architecture needs, by checkpoint name, with its shape (a tied model
        has no lm_head.weight: the embedding is the output projection)."""
        dims = {"d": self.hidden, "k": self.kv_dim, "f": self.intermediate}
        shapes = {"model.embed_tokens.weight": (self.vocab, self.hidden), "model.norm.weight": (self.hidden,)}
        for i in range(self.layers):
            for suffix, form in _LAYER_TENSORS:
                shapes[f"model.layers.{i}.{suffix}"] = tuple(dims[c] for c in form)
        if not self.tie_word_embeddings:
            shapes["lm_head.weight"] = (self.vocab, self.hidden)
        return shapes

    def check_against(self, st) -> int:
        """Checks that a checkpoint (anything with names / has / info) holds exactly the tensors
        the config implies, each with its shape; reports what is missing, misshapen and surplus
        together. Returns the number of tensors."""
        expected = self.expected_tensors()
        missing = [n for n in expected if not st.has(n)]
        misshapen = [f"{n} is {list(st.info(n).shape)} where the config implies {list(s)}"
                     for n, s in expected.items() if st.has(n) and tuple(st.info(n).shape) != tuple(s)]
        surplus = [n for n in st.names() if n not in expected]
        parts = []
        if missing:
            parts.append(f"{len(missing)} missing ({_few(missing)})")
        if misshapen:
            parts.append(f"{len(misshapen)} misshapen ({_few(misshapen)})")
        if surplus:
            parts.append(f"{len(surplus)} not part of the model ({_few(surplus)})")
        if parts:
            raise QwenHipError(QH_ERR_INVALID, "the checkpoint does not match the config: " + "; ".join(parts))
        return len(expected)

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim

    def c_config(self, max_positions: int) -> Config:
        return Config(self.hidden, self.intermediate, self.layers, self.heads, self.kv_heads,
                      self.head_dim, self.vocab, self.rope_theta, self.eps, max_positions)


QWEN25_05B = ModelConfig()

LAYER_TENSORS = {
    "inputNorm": "input_layernorm.weight",
    "wq": "self_attn.q_proj.weight", "bq": "self_attn.q_proj.bias",
    "wk": "self_attn.k_proj.weight", "bk": "self_attn.k_proj.bias",
    "wv": "self_attn.v_proj.weight", "bv": "self_attn.v_proj.bias",
    "wo": "self_attn.o_proj.weight",
    "postAttnNorm": "post_attention_layernorm.weight",
    "wGate": "mlp.gate_proj.weight", "wUp": "mlp.up_proj.weight",
    "wDown": "mlp.down_proj.weight",
}
MATRIX_KEYS = ("wq", "wk", "wv", "wo", "wGate", "wUp", "wDown")

_lib = None


def load_library(path: str | None = None) -> ctypes.CDLL:
    """Load libqwen_hip.so (built in-tree by __graft_entry__.build())."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise QwenHipError(QH_ERR_STATE, f"{p} is not built; run __graft_entry__.build() first")
    lib = ctypes.CDLL(p)
    _declare(lib)
    if path is None:
        _lib = lib
    return lib


def _declare(lib: ctypes.CDLL) -> None:
    vp, i32, sz, f64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_size_t, ctypes.c_double
    u64 = ctypes.c_uint64
    lib.qh_last_error.restype = ctypes.c_char_p
    sigs = {
        "qh_abi_version": [], "qh_device_count": [vp], "qh_open": [ctypes.c_int, vp],
        "qh_close": [vp], "qh_describe": [vp, ctypes.c_char_p, sz], "qh_sync": [vp],
        "qh_alloc": [vp, sz, vp], "qh_free": [vp, vp], "qh_upload": [vp, vp, vp, sz],
        "qh_download": [vp, vp, vp, sz], "qh_memset": [vp, vp, ctypes.c_int, sz],
        "qh_copy": [vp, vp, vp, sz],
        "qh_event_create": [vp, vp], "qh_event_record": [vp, vp],
        "qh_event_elapsed_ms": [vp, vp, vp], "qh_event_destroy": [vp],
        "qh_matvec": [vp, vp, vp, vp, vp, i32], "qh_matvec_xh": [vp, vp, vp, vp],
        "qh_matvec_xh_list": [vp, vp, i32, sz, sz, vp, sz, vp],
        "qh_rmsnorm": [vp, vp, vp, vp, i32, i32, f64],
        "qh_rope": [vp, vp, vp, vp, i32, i32, i32, i32, i32],
        "qh_rope_tables": [i32, f64, i32, vp, vp],
        "qh_kv_append": [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32],
        "qh_attention": [vp, vp, vp, vp, i32, vp, i32, i32, i32, i32, i32],
        "qh_attention_splitk": [vp, vp, vp, vp, i32, vp, i32, i32, i32, i32, i32],
        "qh_attention_mfma": [vp, vp, vp, vp, i32, vp, i32, i32, i32, i32, i32],
        "qh_swiglu": [vp, vp, vp, i32], "qh_add": [vp, vp, vp, i32],
        "qh_matmul_prefill": [vp, vp, vp, vp, vp, i32], "qh_matmul_prefill_noalloc": [vp, vp, vp, vp, vp, i32],
        "qh_attention_splitk_list": [vp, vp, vp, vp, sz, sz, i32, i32, vp, i32, i32, i32, i32],
        "qh_attention_list_plan": [i32, i32, i32, vp, vp],
        "qh_argmax": [vp, vp, i32, vp],
        "qh_quantize_int8": [vp, i32, i32, vp, vp],
        "qh_quantize_int4": [vp, i32, i32, i32, vp, vp, vp],
        "qh_quantize": [vp, i32, vp, i32, i32, i32, i32, vp, vp, vp],
        "qh_synth_f32": [u64, ctypes.c_char_p, f64, sz, sz, vp],
        "qh_synth_bf16": [u64, ctypes.c_char_p, f64, sz, sz, vp],
        "qh_synth_tokens": [u64, ctypes.c_char_p, i32, sz, vp],
        "qh_model_create": [vp, vp, vp],
        "qh_model_set_tensor": [vp, ctypes.c_char_p, i32, i32, i32, i32, vp, vp, vp],
        "qh_model_load_tensor": [vp, ctypes.c_char_p, i32, i32, i32, vp, i32, i32],
        "qh_model_finalize": [vp], "qh_model_free": [vp], "qh_model_bytes": [vp, vp],
        "qh_score": [vp, vp, vp, i32, vp],
        "qh_model_config": [vp, vp],
        "qh_decode_kernel_time_cold": [vp, vp, i32, sz, i32, vp, vp],
        "qh_decode_kernel_time_stream": [vp, vp, i32, sz, i32, i32, vp, vp],
        "qh_probe_launch_floor": [vp, i32, i32, i32, vp], "qh_read_ceiling": [vp, sz, i32, vp],
        "qh_model_set_numerics": [vp, i32], "qh_model_set_matmul": [vp, i32],
        "qh_cache_create": [vp, i32, vp], "qh_cache_free": [vp], "qh_cache_length": [vp, vp],
        "qh_cache_set_length": [vp, i32], "qh_cache_present": [vp, i32, vp, vp],
        "qh_forward": [vp, vp, vp, i32, vp, vp], "qh_forward_tokens": [vp, vp, vp, i32, vp, vp],
        "qh_decode": [vp, vp, i32, i32, vp], "qh_decode_launch": [vp, vp, i32, i32],
        "qh_decode_collect": [vp, vp, i32, vp], "qh_decode_use_graph": [vp, i32],
        "qh_decode_profile": [vp, vp, i32, i32, vp, vp, vp],
        "qh_decode_kernel_time": [vp, vp, i32, i32, vp],
        "qh_decode_prepare": [vp, vp], "qh_decode_role": [vp, vp, i32, i32, vp],
        "qh_cache_vector": [vp, i32, i32, vp, vp],
    }
    for name, args in sigs.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = ctypes.c_int
    lib.qh_stream.argtypes = [vp]
    lib.qh_stream.restype = vp
    lib.qh_value_cache_bytes.argtypes = [i32, i32, i32]
    lib.qh_value_cache_bytes.restype = ctypes.c_size_t


def value_cache_bytes(capacity: int, kv_heads: int, head_dim: int = 64) -> int:
    """Bytes of a dimension-major value cache (rows of capacity rounded up to 64)."""
    return int(load_library().qh_value_cache_bytes(capacity, kv_heads, head_dim))


def _check(rc: int) -> None:
    if rc == QH_OK:
        return
    msg = load_library().qh_last_error().decode()
    if rc == QH_ERR_RANGE:
        raise RangeError(rc, msg)
    if rc == QH_ERR_BUSY:
        raise BusyError(rc, msg)
    raise QwenHipError(rc, msg)


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("arrays must be C-contiguous")
    return a.ctypes.data


# ------------------------------------------------------------- host helpers --

def device_count() -> int:
    n = ctypes.c_int(0)
    _check(load_library().qh_device_count(ctypes.byref(n)))
    return n.value


def attention_list_plan(context: int, count: int, kv_heads: int) -> tuple:
    """(slots, waves) of the launch qh_attention_splitk_list makes for a query at position
    context-1 over `count` caches (host-only)."""
    slots, waves = ctypes.c_int32(), ctypes.c_int32()
    _check(load_library().qh_attention_list_plan(context, count, kv_heads, ctypes.byref(slots),
                                                 ctypes.byref(waves)))
    return slots.value, waves.value


def quantize_int8(w: np.ndarray):
    """quantizeInt8PerChannel (src/core/quantize.js:36-58): (codes int8, scales f32)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    _check(load_library().qh_quantize_int8(_ptr(w), rows, cols, _ptr(q), _ptr(s)))
    return q, s


def quantize_int4(w: np.ndarray, group: int = 128):
    """quantizeInt4Group (src/core/quantize.js:80-132): (packed u8, scales f32, zeros f32)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols // 2), np.uint8)
    s = np.empty((rows, max(cols // max(group, 1), 1)), np.float32)
    z = np.empty_like(s)
    _check(load_library().qh_quantize_int4(_ptr(w), rows, cols, group, _ptr(q), _ptr(s), _ptr(z)))
    return q, s, z


def rope_tables(head_dim: int, theta: float, positions: int):
    cos = np.empty((positions, head_dim // 2), np.float32)
    sin = np.empty_like(cos)
    _check(load_library().qh_rope_tables(head_dim, theta, positions, _ptr(cos), _ptr(sin)))
    return cos, sin


def synth_f32(seed: int, name: str, std: float, n: int, offset: int = 0) -> np.ndarray:
    out = np.empty(n, np.float32)
    _check(load_library().qh_synth_f32(seed, name.encode(), std, offset, n, _ptr(out)))
    return out


def synth_bf16(seed: int, name: str, std: float, n: int, offset: int = 0) -> np.ndarray:
    out = np.empty(n, np.uint16)
    _check(load_library().qh_synth_bf16(seed, name.encode(), std, offset, n, _ptr(out)))
    return out


def synth_tokens(seed: int, name: str, vocab: int, n: int) -> np.ndarray:
    out = np.empty(n, np.int32)
    _check(load_library().qh_synth_tokens(seed, name.encode(), vocab, n, _ptr(out)))
    return out


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact widening (src/core/dtype.js:43-48)."""
    return (bits.astype(np.uint32) << 16).view(np.float32)


def synthesize_checkpoint(cfg: ModelConfig, seed: int, std: float = 0.02) -> dict:
    """Seeded random-init weights of the architecture, as bf16 checkpoint tensors.

    Linear, embedding and bias tensors ~ N(0, std) (Irwin-Hall approximation, see
    qh_synth_f32), norm gains 1.0, named as src/core/config.js:88-119 expects.
    Returns {name: uint16 array of bf16 bits, shaped}.
    """
    d, kv, ffn = cfg.hidden, cfg.kv_dim, cfg.intermediate
    shapes = {"model.embed_tokens.weight": (cfg.vocab, d), "model.norm.weight": (d,)}
    for i in range(cfg.layers):
        p = f"model.layers.{i}."
        shapes.update({
            p + "input_layernorm.weight": (d,), p + "post_attention_layernorm.weight": (d,),
            p + "self_attn.q_proj.weight": (d, d), p + "self_attn.q_proj.bias": (d,),
            p + "self_attn.k_proj.weight": (kv, d), p + "self_attn.k_proj.bias": (kv,),
            p + "self_attn.v_proj.weight": (kv, d), p + "self_attn.v_proj.bias": (kv,),
            p + "self_attn.o_proj.weight": (d, d),
            p + "mlp.gate_proj.weight": (ffn, d), p + "mlp.up_proj.weight": (ffn, d),
            p + "mlp.down_proj.weight": (d, ffn),
        })
    out = {}
    one = np.uint16(0x3F80)  # bf16 1.0
    for name, shape in shapes.items():
        n = int(np.prod(shape))
        if name.endswith("norm.weight"):
            out[name] = np.full(shape, one, np.uint16)
        else:
            out[name] = synth_bf16(seed, name, std, n).reshape(shape)
    return out


def device_tensors(ckpt: dict, cfg: ModelConfig, scheme: str = "int4", group: int = 128,
                   lm_head: str = "int8") -> dict:
    """Quantize a bf16 checkpoint into the device formats (the loader's job,
    src/gpu/model.js:147-207): layer matrices per `scheme` ('f16' | 'int8' |
    'int4'), the tied embedding per `lm_head` as the output projection, the bf16
    embedding as the gather table, norms and biases f32.

    Returns {name: (format, rows, cols, group, data, scales, zeros)}.
    """
    def mat(w32: np.ndarray, sch: str):
        rows, cols = w32.shape
        if sch == "f16":
            return (FMT_F16, rows, cols, 0, w32.astype(np.float16).view(np.uint16), None, None)
        if sch == "int8":
            q, s = quantize_int8(w32)
            return (FMT_INT8, rows, cols, 0, q, s, None)
        if sch == "int4":
            q, s, z = quantize_int4(w32, group)
            return (FMT_INT4, rows, cols, group, q, s, z)
        raise ValueError(f"unknown scheme {sch}")

    out = {}
    for name, bits in ckpt.items():
        if name == "model.embed_tokens.weight":
            out[name] = (FMT_BF16, bits.shape[0], bits.shape[1], 0, bits, None, None)
            out["lm_head.weight"] = mat(bf16_to_f32(bits), lm_head)
        elif bits.ndim == 1:
            out[name] = (FMT_F32, bits.shape[0], 1, 0, bf16_to_f32(bits), None, None)
        else:
            out[name] = mat(bf16_to_f32(bits), scheme)
    return out


# ---------------------------------------------------------------- context --

class DeviceBuffer:
    def __init__(self, ctx: "GpuContext", ptr: int, nbytes: int, dtype=np.float32, shape=None):
        self.ctx, self.ptr, self.nbytes = ctx, ptr, nbytes
        self.dtype = np.dtype(dtype)
        self.shape = shape if shape is not None else (nbytes // self.dtype.itemsize,)

    def read(self, dtype=None, count=None) -> np.ndarray:
        dt = np.dtype(dtype or self.dtype)
        n = count if count is not None else self.nbytes // dt.itemsize
        out = np.empty(n, dt)
        self.ctx.download_into(out, self)
        return out

    def free(self) -> None:
        if self.ptr:
            _check(self.ctx.lib.qh_free(self.ctx.handle, self.ptr))
            self.ptr = 0


class GpuContext:
    """GpuContext.create / upload / empty / readF32 / done (src/gpu/device.js)."""

    def __init__(self, handle: int, lib: ctypes.CDLL):
        self.handle, self.lib = handle, lib

    @staticmethod
    def create(device: int = 0) -> "GpuContext":
        lib = load_library()
        h = ctypes.c_void_p()
        _check(lib.qh_open(device, ctypes.byref(h)))
        return GpuContext(h.value, lib)

    def close(self) -> None:
        if self.handle:
            _check(self.lib.qh_close(self.handle))
            self.handle = None

    def launch_floor(self, kind: int, blocks: int = 224, launches: int = 200) -> float:
        """Microseconds per launch of `launches` graph-replayed probe launches (qh_probe_launch_floor:
        kind 0 empty, 1 reading the previous launch's output, 2 reading nothing)."""
        us = ctypes.c_float()
        _check(self.lib.qh_probe_launch_floor(self.handle, kind, blocks, launches, ctypes.byref(us)))
        return us.value

    def read_ceiling(self, nbytes: int = 1 << 30, reps: int = 10) -> float:
        """GB/s of a pure streaming read of nbytes (qh_read_ceiling)."""
        g = ctypes.c_float()
        _check(self.lib.qh_read_ceiling(self.handle, nbytes, reps, ctypes.byref(g)))
        return g.value

    def describe(self) -> str:
        buf = ctypes.create_string_buffer(512)
        _check(self.lib.qh_describe(self.handle, buf, 512))
        return buf.value.decode()

    @property
    def stream(self) -> int:
        return self.lib.qh_stream(self.handle)

    def empty(self, nbytes: int, dtype=np.float32) -> DeviceBuffer:
        p = ctypes.c_void_p()
        _check(self.lib.qh_alloc(self.handle, nbytes, ctypes.byref(p)))
        return DeviceBuffer(self, p.value, nbytes, dtype)

    def upload(self, a: np.ndarray) -> DeviceBuffer:
        a = np.ascontiguousarray(a)
        b = self.empty(max(a.nbytes, 4), a.dtype)
        b.shape = a.shape
        _check(self.lib.qh_upload(self.handle, b.ptr, _ptr(a), a.nbytes))
        return b

    def download_into(self, out: np.ndarray, buf: DeviceBuffer, offset: int = 0) -> None:
        _check(self.lib.qh_download(self.handle, _ptr(out), buf.ptr + offset, out.nbytes))

    def copy(self, src, src_offset: int, dst, dst_offset: int, nbytes: int) -> None:
        """GpuContext.copy (device.js:168-175): a device copy kernel on the context stream."""
        _check(self.lib.qh_copy(self.handle, dst.ptr + dst_offset, src.ptr + src_offset, nbytes))

    def quantize(self, src: DeviceBuffer, src_format: int, rows: int, cols: int, fmt: int,
                 group: int = 0, data=None, scales=None, zeros=None):
        """qh_quantize: [rows, cols] bf16 or f32 values on the device converted to `fmt`
        (the loader's per-tensor conversion, src/gpu/model.js:165-173). Allocates the outputs
        that are not given; returns (data, scales, zeros), absent ones None."""
        n = rows * cols
        nbytes = {FMT_F32: 4 * n, FMT_F16: 2 * n, FMT_INT8: n, FMT_INT4: n // 2}.get(fmt, 4)   # else rejected
        per = rows if fmt == FMT_INT8 else rows * (cols // group) if fmt == FMT_INT4 and group > 0 else 0
        if data is None:
            data = self.empty(max(nbytes, 4), np.uint8)
        if scales is None and per:
            scales = self.empty(4 * per)
        if zeros is None and fmt == FMT_INT4 and per:
            zeros = self.empty(4 * per)
        _check(self.lib.qh_quantize(self.handle, src_format, src.ptr, rows, cols, fmt, group, data.ptr,
                                    scales.ptr if scales else None, zeros.ptr if zeros else None))
        return data, scales, zeros

    def done(self) -> None:
        _check(self.lib.qh_sync(self.handle))

    # Device-side timing on the context stream (GpuContext.timed, device.js:301-338).
    def event(self):
        e = ctypes.c_void_p()
        _check(self.lib.qh_event_create(self.handle, ctypes.byref(e)))
        return e.value

    def record(self, ev) -> None:
        _check(self.lib.qh_event_record(self.handle, ev))

    def elapsed_ms(self, start, stop) -> float:
        ms = ctypes.c_float()
        _check(self.lib.qh_event_elapsed_ms(start, stop, ctypes.byref(ms)))
        return ms.value

    def destroy_event(self, ev) -> None:
        self.lib.qh_event_destroy(ev)

    # ------------------------------------------------------------ operators --
    def weight(self, fmt: int, rows: int, cols: int, data: DeviceBuffer, scales=None, zeros=None,
               group: int = 0) -> Weight:
        return Weight(fmt, rows, cols, group, data.ptr, scales.ptr if scales else None,
                      zeros.ptr if zeros else None)

    def matvec(self, w: Weight, x: DeviceBuffer, bias, y: DeviceBuffer, seq: int = 1) -> None:
        _check(self.lib.qh_matvec(self.handle, ctypes.byref(w), x.ptr, bias.ptr if bias else None,
                                  y.ptr, seq))

    def matmul_prefill(self, w: Weight, x: DeviceBuffer, bias, y: DeviceBuffer, M: int) -> None:
        """y [M, rows] = x [M, cols] . W^T (+ bias) on the int8 matrix cores (int8 / int4 weights)."""
        _check(self.lib.qh_matmul_prefill(self.handle, ctypes.byref(w), x.ptr,
                                          bias.ptr if bias else None, y.ptr, M))

    def matmul_prefill_noalloc(self, w: Weight, x: DeviceBuffer, bias, y: DeviceBuffer, M: int) -> None:
        """matmul_prefill with its scratch in the library's per-device static array (no allocation)."""
        _check(self.lib.qh_matmul_prefill_noalloc(self.handle, ctypes.byref(w), x.ptr,
                                                  bias.ptr if bias else None, y.ptr, M))

    def matvec_xh_list(self, w: Weight, count: int, data_stride: int, scale_stride: int,
                       x: DeviceBuffer, x_stride: int, y: DeviceBuffer) -> None:
        _check(self.lib.qh_matvec_xh_list(self.handle, ctypes.byref(w), count, data_stride,
                                          scale_stride, x.ptr, x_stride, y.ptr))

    def rmsnorm(self, x, gain, y, rows, cols, eps) -> None:
        _check(self.lib.qh_rmsnorm(self.handle, x.ptr, gain.ptr, y.ptr, rows, cols, eps))

    def rope(self, v, cos, sin, table_positions, rows, heads, head_dim, base_pos) -> None:
        _check(self.lib.qh_rope(self.handle, v.ptr, cos.ptr, sin.ptr, table_positions, rows, heads,
                                head_dim, base_pos))

    def kv_append(self, k, v, kc, vc, capacity, kv_heads, head_dim, past, seq) -> None:
        _check(self.lib.qh_kv_append(self.handle, k.ptr, v.ptr, kc.ptr, vc.ptr, capacity, kv_heads,
                                     head_dim, past, seq))

    def attention(self, q, kc, vc, capacity, out, seq, past, heads, kv_heads, head_dim=64,
                  splitk=False, kind=None) -> None:
        """kind: "exact" (qh_attention), "splitk" or "mfma"; `splitk` picks between the first two."""
        kind = kind or ("splitk" if splitk else "exact")
        fn = {"exact": self.lib.qh_attention, "splitk": self.lib.qh_attention_splitk,
              "mfma": self.lib.qh_attention_mfma}[kind]
        _check(fn(self.handle, q.ptr, kc.ptr, vc.ptr, capacity, out.ptr, seq, past, heads, kv_heads,
                  head_dim))

    def attention_list(self, q, kc, vc, key_stride, value_stride, count, capacity, out, past, heads,
                       kv_heads, head_dim=64) -> None:
        """Split-K attention of one query against `count` caches (strides in f16 elements)."""
        _check(self.lib.qh_attention_splitk_list(self.handle, q.ptr, kc.ptr, vc.ptr, key_stride, value_stride,
                                                 count, capacity, out.ptr, past, heads, kv_heads, head_dim))

    def swiglu(self, gate, up, n) -> None:
        _check(self.lib.qh_swiglu(self.handle, gate.ptr, up.ptr, n))

    def add(self, x, delta, n) -> None:
        _check(self.lib.qh_add(self.handle, x.ptr, delta.ptr, n))

    def argmax(self, v, n) -> int:
        out = ctypes.c_int32()
        _check(self.lib.qh_argmax(self.handle, v.ptr, n, ctypes.byref(out)))
        return out.value


# ------------------------------------------------------------------ model --

class GpuKVCache:
    """GpuKVCache (src/gpu/model.js:69-84): f16 keys/values on the device."""

    def __init__(self, model: "GpuModel", handle: int, capacity: int):
        self.model, self.handle, self.capacity = model, handle, capacity

    @property
    def length(self) -> int:
        n = ctypes.c_int32()
        _check(self.model.lib.qh_cache_length(self.handle, ctypes.byref(n)))
        return n.value

    @length.setter
    def length(self, value: int) -> None:
        _check(self.model.lib.qh_cache_set_length(self.handle, value))

    def reset(self) -> None:
        self.length = 0

    @property
    def byteLength(self) -> int:
        c = self.model.config
        return c.layers * self.capacity * c.kv_dim * 2 * 2

    def vector(self, which: str, value=None, layer: int = 0) -> np.ndarray:
        """One decode-state vector of the cache ("x", "q", "h", "logits"; or, read-only, the
        "key" / "value" row of `layer` at the current position): writes `value` first when
        given, then returns the vector's contents."""
        c = self.model.config
        n = {"x": c.hidden, "q": c.hidden, "h": c.intermediate, "logits": c.vocab,
             "key": c.kv_dim, "value": c.kv_dim}[which]
        src = None if value is None else np.ascontiguousarray(value, np.float32)
        if src is not None and src.size != n:
            raise ValueError(f"{which} has {n} values, got {src.size}")
        out = np.empty(n, np.float32)
        _check(self.model.lib.qh_cache_vector(self.handle, VECTORS.index(which), layer, _ptr(src), _ptr(out)))
        return out

    def present(self, layer: int):
        """{key, value} as [kvHeads, length, headDim] f32 (src/cpu/cache.js:97-115)."""
        c, n = self.model.config, self.length
        k = np.empty((c.kv_heads, n, c.head_dim), np.float32)
        v = np.empty_like(k)
        _check(self.model.lib.qh_cache_present(self.handle, layer, _ptr(k), _ptr(v)))
        return {"key": k, "value": v}

    def destroy(self) -> None:
        if self.handle:
            _check(self.model.lib.qh_cache_free(self.handle))
            self.handle = None


class GpuModel:
    """GpuModel (src/gpu/model.js:86-403) over libqwen_hip.so."""

    def __init__(self, ctx: GpuContext, handle: int, config: ModelConfig, max_positions: int):
        self.ctx, self.lib, self.handle = ctx, ctx.lib, handle
        self.config, self.maxPositions = config, max_positions

    @staticmethod
    def load(ctx: GpuContext, tensors: dict, config: ModelConfig, maxPositions: int = 2048,
             onProgress=None, numerics: str = "fast", matmul: str = "batched") -> "GpuModel":
        """Upload device tensors (see device_tensors) and finalize. numerics: "fast"
        (f32 sums, split-K attention on the f16 matrix cores) or "exact" (the CPU path's
        arithmetic, bit for bit). matmul: how forward() runs several positions --
        "batched" (8-position weight tiles, bitwise equal to decoding them one by one),
        "matvec" (one decode step per position) or "mfma" (int8 matrix cores over exact
        activation digits, for int8/int4 weights)."""
        def upload(lib, handle):
            total = len(tensors)
            for i, (name, (fmt, rows, cols, group, data, scales, zeros)) in enumerate(tensors.items()):
                data = np.ascontiguousarray(data)
                scales = None if scales is None else np.ascontiguousarray(scales, np.float32)
                zeros = None if zeros is None else np.ascontiguousarray(zeros, np.float32)
                _check(lib.qh_model_set_tensor(handle, name.encode(), fmt, rows, cols, group,
                                               _ptr(data), _ptr(scales), _ptr(zeros)))
                if onProgress:
                    onProgress(i + 1, total, name)

        return GpuModel._build(ctx, config, maxPositions, numerics, matmul, upload)

    @staticmethod
    def load_checkpoint(ctx: GpuContext, ckpt: dict, config: ModelConfig, scheme: str = "int4",
                        group: int = 128, lm_head: str = "int8", maxPositions: int = 2048,
                        onProgress=None, numerics: str = "fast",
                        matmul: str = "batched") -> "GpuModel":
        """GpuModel.load (src/gpu/model.js:147-207) from the checkpoint's own tensors
        ({name: uint16 bf16 bits or float32 values}), each uploaded in its checkpoint width
        and converted on the device (qh_model_load_tensor): layer matrices per `scheme`, the
        tied embedding per `lm_head` as the output projection, the bf16 embedding as the
        gather table, norms and biases f32. Stores the same bits as
        load(ctx, device_tensors(ckpt, config, scheme, group, lm_head), config)."""
        def src_of(a: np.ndarray):
            if a.dtype == np.uint16:
                return FMT_BF16, np.ascontiguousarray(a)
            if a.dtype == np.float32:
                return FMT_F32, np.ascontiguousarray(a)
            raise ValueError(f"checkpoint tensors are bf16 bits (uint16) or float32, got {a.dtype}")

        def upload(lib, handle):
            jobs = []
            for name, a in ckpt.items():
                if name == "model.embed_tokens.weight":
                    jobs.append((name, a, FMT_BF16))
                    jobs.append(("lm_head.weight", a, FORMAT_OF[lm_head]))
                elif a.ndim == 1:
                    jobs.append((name, a, FMT_F32))
                else:
                    jobs.append((name, a, FORMAT_OF[scheme]))
            for i, (name, a, fmt) in enumerate(jobs):
                sf, src = src_of(a)
                rows, cols = (a.shape[0], 1) if a.ndim == 1 else a.shape
                _check(lib.qh_model_load_tensor(handle, name.encode(), sf, rows, cols, _ptr(src), fmt,
                                                group if fmt == FMT_INT4 else 0))
                if onProgress:
                    onProgress(i + 1, len(jobs), name)

        return GpuModel._build(ctx, config, maxPositions, numerics, matmul, upload)

    @staticmethod
    def load_safetensors(ctx: GpuContext, path: str, config: ModelConfig | None = None, scheme: str = "int4",
                         group: int = 128, lm_head: str = "int8", maxPositions: int = 2048, onProgress=None,
                         numerics: str = "fast", matmul: str = "batched") -> "GpuModel":
        """GpuModel.load (src/gpu/model.js:147-207) from a safetensors checkpoint. `path` is the
        model file, or a directory holding model.safetensors and config.json (which then gives
        `config`). The file is checked against the config first (checkAgainst,
        src/core/config.js:128-153). Each tensor goes to the device from the read-only file
        mapping as stored -- bf16 bits or f32 -- one at a time, and is converted there
        (qh_model_load_tensor); an f16 tensor is widened exactly on the host first. The
        embedding is the bf16 gather table and, for a tied model, also the output projection
        in `lm_head` format; an untied checkpoint's lm_head.weight is used instead."""
        import checkpoint

        if os.path.isdir(path):
            if config is None:
                config = ModelConfig.from_hf(os.path.join(path, "config.json"))
            path = os.path.join(path, "model.safetensors")
        if config is None:
            raise QwenHipError(QH_ERR_INVALID, "load_safetensors needs a config (or a directory with config.json)")
        st = checkpoint.Safetensors.open(path)
        config.check_against(st)

        def upload(lib, handle):
            jobs = []
            for name, shape in config.expected_tensors().items():
                if name == "model.embed_tokens.weight":
                    jobs.append((name, name, FMT_BF16))
                    if config.tie_word_embeddings:
                        jobs.append(("lm_head.weight", name, FORMAT_OF[lm_head]))
                elif name == "lm_head.weight":
                    jobs.append((name, name, FORMAT_OF[lm_head]))
                else:
                    jobs.append((name, name, FMT_F32 if len(shape) == 1 else FORMAT_OF[scheme]))
            for i, (as_name, name, fmt) in enumerate(jobs):
                dtype = st.info(name).dtype
                a = st.array(name)
                if dtype == "BF16":
                    sf, src = FMT_BF16, a
                elif dtype == "F32":
                    sf, src = FMT_F32, a
                elif dtype == "F16":
                    sf, src = FMT_F32, a.view(np.float16).astype(np.float32)
                else:
                    raise QwenHipError(QH_ERR_INVALID, f"{name}: dtype {dtype} is not a weight format")
                if fmt == FMT_BF16 and sf != FMT_BF16:
                    raise QwenHipError(QH_ERR_INVALID, f"{name}: the gather table is bf16 and the file holds "
                                                       f"{dtype}")
                rows, cols = (a.shape[0], 1) if a.ndim == 1 else a.shape
                _check(lib.qh_model_load_tensor(handle, as_name.encode(), sf, rows, cols,
                                                _ptr(np.ascontiguousarray(src)), fmt,
                                                group if fmt == FMT_INT4 else 0))
                if onProgress:
                    onProgress(i + 1, len(jobs), as_name)

        try:
            return GpuModel._build(ctx, config, maxPositions, numerics, matmul, upload)
        finally:
            st.close()

    @staticmethod
    def _build(ctx: GpuContext, config: ModelConfig, maxPositions: int, numerics: str, matmul: str,
               upload) -> "GpuModel":
        lib = ctx.lib
        h = ctypes.c_void_p()
        cc = config.c_config(maxPositions)
        _check(lib.qh_model_create(ctx.handle, ctypes.byref(cc), ctypes.byref(h)))
        model = GpuModel(ctx, h.value, config, maxPositions)
        try:
            _check(lib.qh_model_set_numerics(h.value, NUMERICS[numerics]))
            _check(lib.qh_model_set_matmul(h.value, MATMUL[matmul]))
            upload(lib, h.value)
            _check(lib.qh_model_finalize(h.value))
        except Exception:
            lib.qh_model_free(h.value)
            raise
        return model

    def set_matmul(self, matmul: str) -> None:
        """Switch forward()'s multi-position mode ("batched" | "matvec" | "mfma")."""
        _check(self.lib.qh_model_set_matmul(self.handle, MATMUL[matmul]))

    @property
    def device_bytes(self) -> int:
        n = ctypes.c_size_t()
        _check(self.lib.qh_model_bytes(self.handle, ctypes.byref(n)))
        return n.value

    def newCache(self, capacity: int) -> GpuKVCache:
        h = ctypes.c_void_p()
        _check(self.lib.qh_cache_create(self.handle, capacity, ctypes.byref(h)))
        return GpuKVCache(self, h.value, capacity)

    def forward(self, hidden: np.ndarray, seq: int, cache: GpuKVCache, wantLogits: bool = True,
                wantPresent: bool = False):
        """forward(hidden [seq*hidden] f32, seq, {cache, wantLogits, wantPresent})."""
        hidden = np.ascontiguousarray(hidden, dtype=np.float32)
        if hidden.size != seq * self.config.hidden:
            raise ValueError(f"hidden has {hidden.size} values, expected {seq * self.config.hidden}")
        logits = np.empty(self.config.vocab, np.float32) if wantLogits else None
        am = ctypes.c_int32(-1)
        _check(self.lib.qh_forward(self.handle, cache.handle, _ptr(hidden), seq, _ptr(logits),
                                   ctypes.byref(am) if wantLogits else None))
        present = [cache.present(i) for i in range(self.config.layers)] if wantPresent else None
        return {"logits": logits, "argmax": am.value if wantLogits else None, "present": present}

    def forward_tokens(self, ids, cache: GpuKVCache, wantLogits: bool = True):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        logits = np.empty(self.config.vocab, np.float32) if wantLogits else None
        am = ctypes.c_int32(-1)
        _check(self.lib.qh_forward_tokens(self.handle, cache.handle, _ptr(ids), ids.size,
                                          _ptr(logits), ctypes.byref(am) if wantLogits else None))
        return {"logits": logits, "argmax": am.value if wantLogits else None}

    def decode(self, cache: GpuKVCache, first_token: int, steps: int) -> np.ndarray:
        """Greedy decode of `steps` tokens by hipGraph replay; returns the generated ids."""
        out = np.empty(steps, np.int32)
        _check(self.lib.qh_decode(self.handle, cache.handle, first_token, steps, _ptr(out)))
        return out

    def decode_use_graph(self, cache: GpuKVCache, use_graph: bool) -> None:
        """False: later decodes on `cache` launch each kernel directly (same kernels and
        tokens) instead of replaying the captured graph."""
        _check(self.lib.qh_decode_use_graph(cache.handle, int(bool(use_graph))))

    def decode_launch(self, cache: GpuKVCache, first_token: int, steps: int) -> None:
        _check(self.lib.qh_decode_launch(self.handle, cache.handle, first_token, steps))

    def decode_collect(self, cache: GpuKVCache, steps: int) -> np.ndarray:
        out = np.empty(steps, np.int32)
        _check(self.lib.qh_decode_collect(self.handle, cache.handle, steps, _ptr(out)))
        return out

    def decode_profile(self, cache: GpuKVCache, first_token: int, steps: int):
        """Greedy decode with a device event around every launch; returns
        (tokens, {role: (total ms, launches)}) over the steps."""
        out = np.empty(steps, np.int32)
        ms = np.zeros(len(ROLES), np.float32)
        n = np.zeros(len(ROLES), np.int32)
        _check(self.lib.qh_decode_profile(self.handle, cache.handle, first_token, steps, _ptr(out),
                                          _ptr(ms), _ptr(n)))
        return out, {r: (float(ms[i]), int(n[i])) for i, r in enumerate(ROLES)}

    def decode_prepare(self, cache: GpuKVCache) -> None:
        """Capture and upload the cache's decode graphs now (before a timed decode)."""
        _check(self.lib.qh_decode_prepare(self.handle, cache.handle))

    def decode_role(self, cache: GpuKVCache, role: str, layer: int = 0):
        """Run one decode launch of `role` for `layer` at the cache's position (which does not
        advance); for "head", returns the argmax token."""
        tok = ctypes.c_int32(-1)
        _check(self.lib.qh_decode_role(self.handle, cache.handle, ROLES.index(role), layer, ctypes.byref(tok)))
        return tok.value if role == "head" else None

    def score(self, ids, cache: GpuKVCache) -> np.ndarray:
        """Negative log-likelihood of ids[1:] given their left context (qh_score: one position at
        a time through `cache`, web/perplexity.html:146-170); perplexity = exp(mean)."""
        a = np.ascontiguousarray(np.asarray(ids, dtype=np.int32))
        out = np.empty(max(len(a) - 1, 0), np.float64)
        _check(self.lib.qh_score(self.handle, cache.handle, _ptr(a), len(a), _ptr(out)))
        return out

    def kernel_time(self, cache: GpuKVCache, role: str, reps: int = 240) -> float:
        """Microseconds per back-to-back launch of one decode role's kernel (see the C ABI)."""
        us = ctypes.c_float()
        _check(self.lib.qh_decode_kernel_time(self.handle, cache.handle, ROLES.index(role), reps,
                                              ctypes.byref(us)))
        return us.value

    def kernel_time_cold(self, cache: GpuKVCache, role: str, min_bytes: int = 512 << 20, reps: int = 5):
        """(microseconds per launch, copies): one launch of `role` over copies of its operands
        exceeding min_bytes (see qh_decode_kernel_time_cold)."""
        us, n = ctypes.c_float(), ctypes.c_int32()
        _check(self.lib.qh_decode_kernel_time_cold(self.handle, cache.handle, ROLES.index(role), min_bytes, reps,
                                                   ctypes.byref(us), ctypes.byref(n)))
        return us.value, n.value

    def kernel_time_stream(self, cache: GpuKVCache, role: str, blocks_per_copy: int, min_bytes: int = 512 << 20,
                           reps: int = 5):
        """kernel_time_cold with blocks_per_copy blocks per copy: the same kernel on a grid sized for
        streaming (see qh_decode_kernel_time_stream)."""
        us, n = ctypes.c_float(), ctypes.c_int32()
        _check(self.lib.qh_decode_kernel_time_stream(self.handle, cache.handle, ROLES.index(role), min_bytes, reps,
                                                     blocks_per_copy, ctypes.byref(us), ctypes.byref(n)))
        return us.value, n.value

    def destroy(self) -> None:
        if self.handle:
            _check(self.lib.qh_model_free(self.handle))
            self.handle = None
