"""ctypes wrapper of the CPU oracle (oracle/liboracle.so) for the tests.

Test infrastructure: the oracle is the checker the HIP path is compared with;
nothing in the product imports this module.
"""
from __future__ import annotations

import ctypes
import json
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "liboracle.so")

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    src = os.path.join(ORACLE_DIR, "oracle.c")
    if not os.path.exists(ORACLE_SO) or os.path.getmtime(ORACLE_SO) < os.path.getmtime(src):
        subprocess.run(["make", "-C", ORACLE_DIR], check=True, capture_output=True)
    L = ctypes.CDLL(ORACLE_SO)
    vp, i32, f64, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_double, ctypes.c_size_t
    sigs = {
        "or_bf16_to_f32": ([ctypes.c_uint16], ctypes.c_float),
        "or_f32_to_bf16": ([ctypes.c_float], ctypes.c_uint16),
        "or_f16_to_f32": ([ctypes.c_uint16], ctypes.c_float),
        "or_f32_to_f16": ([ctypes.c_float], ctypes.c_uint16),
        "or_f32_to_f16_array": ([vp, vp, sz], None),
        "or_f16_to_f32_array": ([vp, vp, sz], None),
        "or_bf16_to_f32_array": ([vp, vp, sz], None),
        "or_quantize_int8": ([vp, i32, i32, vp, vp], None),
        "or_dequantize_int8": ([vp, vp, i32, i32, vp], None),
        "or_quantize_int4": ([vp, i32, i32, i32, vp, vp, vp], i32),
        "or_dequantize_int4": ([vp, vp, vp, i32, i32, i32, vp], None),
        "or_bits_per_weight": ([i32, i32, i32], f64),
        "or_rmsnorm": ([vp, vp, f64, i32, vp], None),
        "or_matvec": ([vp, vp, i32, i32, vp, vp], None),
        "or_matvec_bf16": ([vp, vp, i32, i32, vp], None),
        "or_softmax": ([vp, i32], None),
        "or_silu": ([f64], f64),
        "or_swiglu": ([vp, vp, i32], None),
        "or_rope_freqs": ([i32, f64, vp], None),
        "or_rope_tables": ([i32, f64, i32, vp, vp], None),
        "or_rope_inplace": ([vp, i32, i32, i32, vp], None),
        "or_grouped_attention": ([vp, vp, vp, vp, vp, i32, i32, i32, i32, i32], None),
        "or_kv_head_for": ([i32, i32, i32], i32),
        "or_cache_new": ([vp, i32], vp),
        "or_cache_free": ([vp], None),
        "or_cache_length": ([vp], i32),
        "or_cache_set_length": ([vp, i32], None),
        "or_cache_present": ([vp, i32, vp, vp], None),
        "or_cache_write": ([vp, i32, i32, vp, vp, i32, i32], i32),
        "or_cache_pin": ([vp, i32], None),
        "or_cache_shadow": ([vp, i32, i32, vp, vp], i32),
        "or_forward": ([vp, vp, vp, i32, vp], i32),
        "or_forward_hidden": ([vp, vp, vp, i32, vp], i32),
        "or_argmax": ([vp, i32], ctypes.c_int32),
        "or_nll": ([vp, i32, i32], ctypes.c_double),
        "or_generate": ([vp, vp, vp, i32, i32, vp], i32),
        "or_set_threads": ([i32], None),
    }
    for name, (args, res) in sigs.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    _lib = L
    return L


def P(a):
    return None if a is None else a.ctypes.data


def c32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ------------------------------------------------------------------ formats --

def f32_to_f16(a) -> np.ndarray:
    a = c32(a)
    out = np.empty(a.shape, np.uint16)
    lib().or_f32_to_f16_array(P(a), P(out), a.size)
    return out


def f16_to_f32(bits) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().or_f16_to_f32_array(P(bits), P(out), bits.size)
    return out


def through_f16(a) -> np.ndarray:
    """throughF16 of web/kernels.html:51-54."""
    return f16_to_f32(f32_to_f16(a))


def bf16_to_f32(bits) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().or_bf16_to_f32_array(P(bits), P(out), bits.size)
    return out


# ---------------------------------------------------------------- quantizer --

def quantize_int8(w):
    w = c32(w)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    lib().or_quantize_int8(P(w), rows, cols, P(q), P(s))
    return q, s


def dequantize_int8(q, s):
    rows, cols = q.shape
    out = np.empty((rows, cols), np.float32)
    lib().or_dequantize_int8(P(np.ascontiguousarray(q)), P(c32(s)), rows, cols, P(out))
    return out


class QuantizeError(ValueError):
    pass


def quantize_int4(w, group=128):
    w = c32(w)
    rows, cols = w.shape
    q = np.empty((rows, cols // 2), np.uint8)
    g = max(group, 1)
    s = np.empty((rows, max(cols // g, 1)), np.float32)
    z = np.empty_like(s)
    rc = lib().or_quantize_int4(P(w), rows, cols, group, P(q), P(s), P(z))
    if rc == -1:
        raise QuantizeError(f"groupSize must be an integer of at least 2, got {group}")
    if rc == -2:
        raise QuantizeError(f"groupSize {group} does not divide {cols} columns")
    return q, s, z


def dequantize_int4(q, s, z, cols, group=128):
    rows = q.shape[0]
    out = np.empty((rows, cols), np.float32)
    lib().or_dequantize_int4(P(np.ascontiguousarray(q)), P(c32(s)), P(c32(z)), rows, cols, group, P(out))
    return out


def round_trip(w, scheme, group=128):
    """roundTrip (src/core/quantize.js:155-163)."""
    w = c32(w)
    if scheme == "int8":
        return dequantize_int8(*quantize_int8(w))
    if scheme == "int4":
        q, s, z = quantize_int4(w, group)
        return dequantize_int4(q, s, z, w.shape[1], group)
    raise ValueError(scheme)


# ---------------------------------------------------------------------- ops --

def rmsnorm(x, w, eps):
    x, w = c32(x), c32(w)
    out = np.empty_like(x)
    lib().or_rmsnorm(P(x), P(w), eps, x.size, P(out))
    return out


def matvec(W, x, rows, cols, bias=None):
    W, x = c32(W), c32(x)
    b = None if bias is None else c32(bias)
    out = np.empty(rows, np.float32)
    lib().or_matvec(P(W), P(x), rows, cols, P(b), P(out))
    return out


def matvec_bf16(bits, x, rows, cols):
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(rows, np.float32)
    lib().or_matvec_bf16(P(bits), P(c32(x)), rows, cols, P(out))
    return out


def softmax(x, n=None):
    x = c32(x).copy()
    lib().or_softmax(P(x), x.size if n is None else n)
    return x


def silu(v):
    return lib().or_silu(v)


def swiglu(gate, up):
    g = c32(gate).copy()
    lib().or_swiglu(P(g), P(c32(up)), g.size)
    return g


def rope_freqs(head_dim, theta):
    out = np.empty(head_dim // 2, np.float64)
    lib().or_rope_freqs(head_dim, theta, P(out))
    return out


def rope_tables(head_dim, theta, positions):
    cos = np.empty((positions, head_dim // 2), np.float32)
    sin = np.empty_like(cos)
    lib().or_rope_tables(head_dim, theta, positions, P(cos), P(sin))
    return cos, sin


def rope_inplace(v, offset, head_dim, position, inv):
    """Rotates v (f32, modified in place) like ropeInPlace."""
    lib().or_rope_inplace(P(v), offset, head_dim, position, P(np.ascontiguousarray(inv, np.float64)))
    return v


def grouped_attention(q, keys, values, seq, past, num_heads, num_kv_heads, head_dim):
    q, keys, values = c32(q), c32(keys), c32(values)
    out = np.empty(seq * num_heads * head_dim, np.float32)
    scores = np.empty(past + seq, np.float32)
    lib().or_grouped_attention(P(q), P(keys), P(values), P(out), P(scores), seq, past, num_heads,
                               num_kv_heads, head_dim)
    return out


def kv_head_for(h, nh, nkv):
    return lib().or_kv_head_for(h, nh, nkv)


def argmax(v):
    return int(lib().or_argmax(P(c32(v)), np.asarray(v).size))


def nll(logits, target):
    """-log softmax(logits)[target] (web/perplexity.html:158-166), the oracle's f64 expression."""
    v = c32(logits)
    return float(lib().or_nll(P(v), v.size, int(target)))


# -------------------------------------------------------------------- model --

class Config(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("intermediate", ctypes.c_int), ("layers", ctypes.c_int),
                ("heads", ctypes.c_int), ("kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int),
                ("vocab", ctypes.c_int), ("rope_theta", ctypes.c_double), ("eps", ctypes.c_double)]


class Layer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "input_norm", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "post_norm", "w_gate", "w_up", "w_down")]


class Model(ctypes.Structure):
    _fields_ = [("cfg", Config), ("layers", ctypes.c_void_p), ("final_norm", ctypes.c_void_p),
                ("embed_bf16", ctypes.c_void_p), ("lm_head_f32", ctypes.c_void_p),
                ("kv_f16", ctypes.c_int)]


class OracleModel:
    """ReferenceModel (src/cpu/model.js) over f32 weights.

    `ckpt` maps checkpoint names to bf16 bit arrays. `scheme` is the layer
    matrices' storage as the loader would round-trip them ('f32' = none,
    'f16' = through f16, 'int8' / 'int4' = the quantizer's round trip);
    `lm_head` likewise for the tied output projection ('bf16' streams the
    unquantized embedding, as ReferenceModel#logits does). `kv_f16` rounds the
    cache through f16 (the same-f16 comparison).
    """

    KEYS = [("input_norm", "input_layernorm.weight"), ("wq", "self_attn.q_proj.weight"),
            ("bq", "self_attn.q_proj.bias"), ("wk", "self_attn.k_proj.weight"),
            ("bk", "self_attn.k_proj.bias"), ("wv", "self_attn.v_proj.weight"),
            ("bv", "self_attn.v_proj.bias"), ("wo", "self_attn.o_proj.weight"),
            ("post_norm", "post_attention_layernorm.weight"), ("w_gate", "mlp.gate_proj.weight"),
            ("w_up", "mlp.up_proj.weight"), ("w_down", "mlp.down_proj.weight")]

    def __init__(self, cfg, ckpt, scheme="f32", group=128, lm_head="bf16", kv_f16=True):
        self.cfg = cfg
        self._keep = []
        layers = (Layer * cfg.layers)()
        for i in range(cfg.layers):
            for field, suffix in self.KEYS:
                bits = ckpt[f"model.layers.{i}.{suffix}"]
                w = bf16_to_f32(bits)
                if w.ndim == 2:
                    w = self._store(w, scheme, group)
                w = np.ascontiguousarray(w)
                self._keep.append(w)
                setattr(layers[i], field, w.ctypes.data)
        self.layers = layers
        self.final_norm = bf16_to_f32(ckpt["model.norm.weight"])
        self.embed = np.ascontiguousarray(ckpt["model.embed_tokens.weight"])
        self.lm = None if lm_head == "bf16" else self._store(bf16_to_f32(self.embed), lm_head, group)
        c = Config(cfg.hidden, cfg.intermediate, cfg.layers, cfg.heads, cfg.kv_heads, cfg.head_dim,
                   cfg.vocab, cfg.rope_theta, cfg.eps)
        self.model = Model(c, ctypes.cast(layers, ctypes.c_void_p), self.final_norm.ctypes.data,
                           self.embed.ctypes.data, None if self.lm is None else self.lm.ctypes.data,
                           1 if kv_f16 else 0)
        self.cconfig = c

    @staticmethod
    def _store(w, scheme, group):
        if scheme == "f32":
            return w
        if scheme == "f16":
            return through_f16(w)
        return round_trip(w, scheme, group)

    def new_cache(self, capacity):
        return OracleCache(self, capacity)

    def forward(self, ids, cache, want_logits=True):
        ids = np.ascontiguousarray(ids, np.int32)
        logits = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        rc = lib().or_forward(ctypes.byref(self.model), cache.h, P(ids), ids.size, P(logits))
        if rc:
            raise ValueError(f"or_forward failed with {rc}")
        return logits

    def forward_hidden(self, hidden, seq, cache, want_logits=True):
        hidden = c32(hidden)
        logits = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        rc = lib().or_forward_hidden(ctypes.byref(self.model), cache.h, P(hidden), seq, P(logits))
        if rc:
            raise ValueError(f"or_forward_hidden failed with {rc}")
        return logits

    def generate(self, prompt, max_tokens, capacity=None):
        prompt = np.ascontiguousarray(prompt, np.int32)
        cache = self.new_cache(capacity or prompt.size + max_tokens)
        out = np.empty(max_tokens, np.int32)
        rc = lib().or_generate(ctypes.byref(self.model), cache.h, P(prompt), prompt.size, max_tokens, P(out))
        if rc:
            raise ValueError(f"or_generate failed with {rc}")
        return out, cache


class OracleCache:
    def __init__(self, model, capacity):
        self.model = model
        self.h = lib().or_cache_new(ctypes.byref(model.cconfig), capacity)
        if not self.h:
            raise ValueError("cache capacity must be a positive integer")

    @property
    def length(self):
        return lib().or_cache_length(self.h)

    @length.setter
    def length(self, n):
        lib().or_cache_set_length(self.h, n)

    def write(self, layer, at, k, v, count, kv_f16=False):
        rc = lib().or_cache_write(self.h, layer, at, P(c32(k)), P(c32(v)), count, 1 if kv_f16 else 0)
        if rc:
            raise ValueError("cache write outside the capacity")

    def pin(self, positions):
        """Positions below `positions` keep their loaded contents when a forward appends over
        them (or_cache_pin): the same-input comparison of web/kernels.html:51-54."""
        lib().or_cache_pin(self.h, positions)

    def shadow(self, layer, n):
        """{key, value} [kv_heads, n, head_dim]: what forward passes computed (unrounded f32)
        for pinned rows 0..n-1 of `layer`."""
        c = self.model.cfg
        k = np.empty((c.kv_heads, n, c.head_dim), np.float32)
        v = np.empty_like(k)
        if lib().or_cache_shadow(self.h, layer, n, P(k), P(v)):
            raise ValueError("no shadow rows: pin the cache and run a forward over them first")
        return {"key": k, "value": v}

    def load_device(self, device_cache, positions, pin=False):
        """Copy the first `positions` K/V rows of every layer from a device cache (its f16
        values, widened exactly) into this cache, and set the length to `positions`; with
        `pin`, a later forward over those positions attends to these rows, not its own."""
        c = self.model.cfg
        for L in range(c.layers):
            p = device_cache.present(L)
            k = np.ascontiguousarray(p["key"][:, :positions].transpose(1, 0, 2).reshape(positions, -1))
            v = np.ascontiguousarray(p["value"][:, :positions].transpose(1, 0, 2).reshape(positions, -1))
            self.write(L, 0, k, v, positions)
        self.length = positions
        if pin:
            self.pin(positions)

    def present(self, layer):
        c = self.model.cfg
        n = self.length
        k = np.empty((c.kv_heads, n, c.head_dim), np.float32)
        v = np.empty_like(k)
        lib().or_cache_present(self.h, layer, P(k), P(v))
        return {"key": k, "value": v}

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_cache_free(self.h)
            self.h = None


# ------------------------------------------- the CPU path under Node (cpu_model.js) --
JS_MODEL = os.path.join(ROOT, "oracle", "cpu_model.js")


def write_js_manifest(directory, cfg, ckpt, scheme="int4", group=128, kv_f16=True, cache_bits=None,
                      context=0, first=0, steps=1):
    """Files for oracle/cpu_model.js: the layer matrices as the quantizer's arrays (this
    module's quantize_int4/int8, the reference quantizer restated), norms and biases f32,
    the embedding's bf16 bits, the output head int8, and optionally a context of `context`
    cache positions as f16 bits [layers][2][context][kv_dim]. Returns the manifest path."""
    tensors = {}

    def put(name, arr, dtype):
        fn = name.replace("/", "_") + ".bin"
        np.ascontiguousarray(arr).tofile(os.path.join(directory, fn))
        tensors[name] = {"file": fn, "dtype": dtype, "length": int(np.asarray(arr).size)}

    for name, bits in ckpt.items():
        if name == "model.embed_tokens.weight":
            put(name, bits, "u16")
            q, s = quantize_int8(bf16_to_f32(bits))
            put("lm_head.weight.q", q, "i8")
            put("lm_head.weight.scales", s, "f32")
        elif bits.ndim == 1:
            put(name, bf16_to_f32(bits), "f32")
        elif scheme == "int4":
            q, s, z = quantize_int4(bf16_to_f32(bits), group)
            put(name + ".q", q, "u8")
            put(name + ".scales", s, "f32")
            put(name + ".zeros", z, "f32")
        else:
            q, s = quantize_int8(bf16_to_f32(bits))
            put(name + ".q", q, "i8")
            put(name + ".scales", s, "f32")
    cache = {"file": None, "length": 0}
    if context:
        fn = "cache.bin"
        np.ascontiguousarray(cache_bits, np.uint16).tofile(os.path.join(directory, fn))
        cache = {"file": fn, "length": int(context)}
    manifest = {
        "config": {"hidden": cfg.hidden, "intermediate": cfg.intermediate, "layers": cfg.layers,
                   "heads": cfg.heads, "kvHeads": cfg.kv_heads, "headDim": cfg.head_dim,
                   "vocab": cfg.vocab, "ropeTheta": cfg.rope_theta, "eps": cfg.eps},
        "tensors": tensors, "scheme": scheme, "group": group, "kvF16": bool(kv_f16),
        "cache": cache, "first": int(first), "steps": int(steps),
    }
    path = os.path.join(directory, "manifest.json")
    with open(path, "w") as f:
        json.dump(manifest, f)
    return path


def run_js_model(manifest, timeout=600):
    """Runs oracle/cpu_model.js under Node on one thread; returns its JSON result."""
    out = subprocess.run(["node", JS_MODEL, manifest], capture_output=True, text=True, timeout=timeout,
                         check=True)
    return json.loads(out.stdout.strip().splitlines()[-1])


def js_cache_bits(presents, context):
    """f16 bits [layers][2][context][kv_dim] from per-layer present() dicts ([kv_heads, n, 64]
    f32 values that are f16 numbers)."""
    out = []
    for p in presents:
        for kind in ("key", "value"):
            a = np.asarray(p[kind])[:, :context]
            out.append(np.ascontiguousarray(a.transpose(1, 0, 2).reshape(context, -1)).astype(np.float16)
                       .view(np.uint16))
    return np.stack(out)
