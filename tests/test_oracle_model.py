"""The oracle's KV cache and model forward (src/cpu/cache.js, src/cpu/model.js),
pinned by the reference's cache tests (test/cache.test.js), its strongest gate
-- incremental decode equals full recomputation bit for bit
(test/cache.test.js:172-208, validate/phase2.js:83-87) -- and an independent
float64 re-derivation of the architecture."""
import ctypes
import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle_lib as O
from conftest import lcg_fast


def tiny_cfg(**kw):
    base = dict(hidden=128, intermediate=256, layers=2, heads=2, kv_heads=1, vocab=512,
                rope_theta=1e6, eps=1e-6)
    base.update(kw)
    c = SimpleNamespace(**base)
    c.head_dim = c.hidden // c.heads
    c.kv_dim = c.kv_heads * c.head_dim
    return c


def to_bf16(a):
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def tiny_ckpt(cfg, seed=1, std=0.05):
    d, kv, ffn = cfg.hidden, cfg.kv_dim, cfg.intermediate
    shapes = {"model.embed_tokens.weight": (cfg.vocab, d), "model.norm.weight": (d,)}
    for i in range(cfg.layers):
        p = f"model.layers.{i}."
        shapes.update({p + "input_layernorm.weight": (d,), p + "post_attention_layernorm.weight": (d,),
                       p + "self_attn.q_proj.weight": (d, d), p + "self_attn.q_proj.bias": (d,),
                       p + "self_attn.k_proj.weight": (kv, d), p + "self_attn.k_proj.bias": (kv,),
                       p + "self_attn.v_proj.weight": (kv, d), p + "self_attn.v_proj.bias": (kv,),
                       p + "self_attn.o_proj.weight": (d, d), p + "mlp.gate_proj.weight": (ffn, d),
                       p + "mlp.up_proj.weight": (ffn, d), p + "mlp.down_proj.weight": (d, ffn)})
    out = {}
    for k, (name, shape) in enumerate(shapes.items()):
        n = int(np.prod(shape))
        if name.endswith("norm.weight"):
            vals = 1 + 0.1 * lcg_fast(n, seed * 1000 + k)
        else:
            vals = std * lcg_fast(n, seed * 1000 + k) * math.sqrt(3)
        out[name] = to_bf16(vals).reshape(shape)
    return out


# ------------------------------------------------------------------- cache

REF_TINY = tiny_cfg(hidden=8, intermediate=16, layers=2, heads=4, kv_heads=2, vocab=32, rope_theta=1e4)


def new_cache(cfg, capacity):
    m = SimpleNamespace(cconfig=O.Config(cfg.hidden, cfg.intermediate, cfg.layers, cfg.heads,
                                         cfg.kv_heads, cfg.head_dim, cfg.vocab, cfg.rope_theta,
                                         cfg.eps), cfg=cfg)
    return O.OracleCache(m, capacity)


def test_cache_rejects_nonpositive_capacity():
    with pytest.raises(ValueError, match="positive"):
        new_cache(REF_TINY, 0)


def test_present_transposes_to_heads_positions_dims():
    c = new_cache(REF_TINY, 2)
    keys = np.array([0, 1, 2, 3, 10, 11, 12, 13], np.float32)
    c.write(0, 0, keys, keys, 2)
    c.length = 2
    assert list(c.present(0)["key"].reshape(-1)) == [0, 1, 10, 11, 2, 3, 12, 13]


def test_multi_token_write_equals_single_writes():
    bulk, single = new_cache(REF_TINY, 4), new_cache(REF_TINY, 4)
    kv = REF_TINY.kv_dim
    keys = np.arange(3 * kv, dtype=np.float32) * 1.5
    vals = -np.arange(3 * kv, dtype=np.float32)
    for L in range(2):
        bulk.write(L, 0, keys, vals, 3)
    for t in range(3):
        for L in range(2):
            single.write(L, t, keys[t * kv:(t + 1) * kv], vals[t * kv:(t + 1) * kv], 1)
    bulk.length = single.length = 3
    for L in range(2):
        np.testing.assert_array_equal(bulk.present(L)["key"], single.present(L)["key"])
        np.testing.assert_array_equal(bulk.present(L)["value"], single.present(L)["value"])


def test_write_past_capacity_refused():
    c = new_cache(REF_TINY, 3)
    with pytest.raises(ValueError):
        c.write(0, 2, np.zeros(8, np.float32), np.zeros(8, np.float32), 2)


def test_f16_cache_rounds_on_write():
    c = new_cache(REF_TINY, 1)
    k = np.full(4, 1 + 2.0 ** -12, np.float32)   # not representable in f16: rounds to 1
    c.write(0, 0, k, k, 1, kv_f16=True)
    c.length = 1
    assert np.all(c.present(0)["key"] == 1.0)


# ------------------------------------------------------------------- model

CFG = tiny_cfg()


@pytest.fixture(scope="module")
def model():
    return O.OracleModel(CFG, tiny_ckpt(CFG), scheme="f32", lm_head="bf16", kv_f16=False)


IDS = [5, 77, 300, 12, 511, 0, 256, 42]


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.parametrize("chunks", [
    [[i] for i in IDS],
    [IDS[:5]] + [[i] for i in IDS[5:]],
    [IDS[:3], IDS[3:4], IDS[4:]],
])
def test_incremental_equals_full_recompute_bitwise(model, chunks):
    full_cache = model.new_cache(len(IDS))
    full = model.forward(IDS, full_cache)
    cache = model.new_cache(len(IDS))
    for ch in chunks:
        last = model.forward(ch, cache)
    np.testing.assert_array_equal(bits(last), bits(full))
    for L in range(CFG.layers):
        for kind in ("key", "value"):
            np.testing.assert_array_equal(bits(cache.present(L)[kind]), bits(full_cache.present(L)[kind]))


def test_cached_generation_equals_uncached(model):
    prompt = [7, 8, 9, 10, 11]
    cached, _ = model.generate(prompt, 4)
    uncached = []
    for _ in range(4):
        seq = prompt + uncached
        logits = model.forward(seq, model.new_cache(len(seq)))
        uncached.append(O.argmax(logits))
    assert list(cached) == uncached


def test_forward_refuses_overflow_and_bad_ids(model):
    c = model.new_cache(3)
    with pytest.raises(ValueError, match="-3"):
        model.forward([1, 2, 3, 4], c)
    assert c.length == 0
    with pytest.raises(ValueError, match="-2"):
        model.forward([CFG.vocab], c)
    with pytest.raises(ValueError, match="-1"):
        model.forward([], c)


def f64_forward(cfg, ckpt, ids):
    """The Qwen2 architecture written out in float64 numpy, from the definition:
    h = x + O(attn(RoPE(Q(rms(x))), RoPE(K(rms(x))), V(rms(x)))),
    y = h + Down(silu(Gate(rms(h))) * Up(rms(h))); logits = E rms(y)."""
    W = {k: (v.astype(np.uint32) << 16).view(np.float32).astype(np.float64) for k, v in ckpt.items()}
    d, hd, nh, nkv = cfg.hidden, cfg.head_dim, cfg.heads, cfg.kv_heads
    T = len(ids)
    x = W["model.embed_tokens.weight"][ids]
    inv = cfg.rope_theta ** (-2.0 * np.arange(hd // 2) / hd)
    ang = np.arange(T)[:, None] * inv[None, :]
    cos, sin = np.cos(ang), np.sin(ang)

    def rms(v, g):
        return v / np.sqrt(np.mean(v * v, axis=-1, keepdims=True) + cfg.eps) * g

    def rope(v):  # v [T, heads, hd]
        lo, hi = v[..., :hd // 2], v[..., hd // 2:]
        c, s = cos[:, None, :], sin[:, None, :]
        return np.concatenate([lo * c - hi * s, hi * c + lo * s], axis=-1)

    for i in range(cfg.layers):
        p = f"model.layers.{i}."
        h = rms(x, W[p + "input_layernorm.weight"])
        q = rope((h @ W[p + "self_attn.q_proj.weight"].T + W[p + "self_attn.q_proj.bias"]).reshape(T, nh, hd))
        k = rope((h @ W[p + "self_attn.k_proj.weight"].T + W[p + "self_attn.k_proj.bias"]).reshape(T, nkv, hd))
        v = (h @ W[p + "self_attn.v_proj.weight"].T + W[p + "self_attn.v_proj.bias"]).reshape(T, nkv, hd)
        att = np.empty((T, nh, hd))
        for head in range(nh):
            g = head // (nh // nkv)
            s = q[:, head] @ k[:, g].T / math.sqrt(hd)
            s = np.where(np.tril(np.ones((T, T), bool)), s, -np.inf)
            pr = np.exp(s - s.max(axis=1, keepdims=True))
            pr /= pr.sum(axis=1, keepdims=True)
            att[:, head] = pr @ v[:, g]
        x = x + att.reshape(T, d) @ W[p + "self_attn.o_proj.weight"].T
        h = rms(x, W[p + "post_attention_layernorm.weight"])
        gt = h @ W[p + "mlp.gate_proj.weight"].T
        up = h @ W[p + "mlp.up_proj.weight"].T
        x = x + (gt / (1 + np.exp(-gt)) * up) @ W[p + "mlp.down_proj.weight"].T
    y = rms(x[-1], W["model.norm.weight"])
    return W["model.embed_tokens.weight"] @ y


def test_forward_matches_float64_rederivation(model):
    logits = model.forward(IDS, model.new_cache(len(IDS)))
    ref = f64_forward(CFG, tiny_ckpt(CFG), IDS)
    rel = np.max(np.abs(logits - ref)) / np.max(np.abs(ref))
    assert rel < 2e-6, rel
    assert O.argmax(logits) == int(np.argmax(ref))


# ------------------------------------------------- same-input comparison (pinned rows)

class _DeviceLike:
    """A cache-shaped source of rows for OracleCache.load_device (present() per layer)."""

    def __init__(self, presents):
        self.presents = presents

    def present(self, layer):
        return self.presents[layer]


def test_pinned_rows_with_the_oracles_own_values_reproduce_its_forward_bitwise():
    """Pinning a cache loaded with exactly the rows the forward would write changes nothing:
    same logits bit for bit. The shadow rows are the unrounded values: their f16 rounding is the
    f16-cache run's present at every layer, and at layer 0 (whose input does not depend on the
    cache) they equal an f32-cache run's present."""
    cfg = tiny_cfg()
    ck = tiny_ckpt(cfg, seed=5)
    ids = np.arange(1, 20, dtype=np.int32) * 7 % cfg.vocab
    m16 = O.OracleModel(cfg, ck, kv_f16=True)
    m32 = O.OracleModel(cfg, ck, kv_f16=False)
    c16 = m16.new_cache(32)
    want = m16.forward(ids, c16)
    c32 = m32.new_cache(32)
    m32.forward(ids, c32)
    pinned = m16.new_cache(32)
    pinned.load_device(_DeviceLike([c16.present(L) for L in range(cfg.layers)]), ids.size, pin=True)
    pinned.length = 0
    got = m16.forward(ids, pinned)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    for L in range(cfg.layers):
        sh, p32, p16 = pinned.shadow(L, ids.size), c32.present(L), c16.present(L)
        for kind in ("key", "value"):
            if L == 0:
                np.testing.assert_array_equal(sh[kind].view(np.uint32), p32[kind].view(np.uint32))
            np.testing.assert_array_equal(O.through_f16(sh[kind]).view(np.uint32), p16[kind].view(np.uint32))
            assert not np.array_equal(sh[kind], p16[kind])     # unrounded, not the stored f16


def test_pinned_rows_are_attended_to_and_kept():
    """A forward over pinned positions attends to the loaded rows (a perturbed row changes the
    logits) and leaves them in place; unpinned positions are written as usual."""
    cfg = tiny_cfg()
    ck = tiny_ckpt(cfg, seed=6)
    ids = np.arange(3, 15, dtype=np.int32) * 5 % cfg.vocab
    m = O.OracleModel(cfg, ck, kv_f16=True)
    c = m.new_cache(16)
    base = m.forward(ids, c)
    presents = [c.present(L) for L in range(cfg.layers)]
    presents[0]["value"][:, 2] += 0.25            # position 2 of layer 0, every kv head
    pinned = m.new_cache(16)
    pinned.load_device(_DeviceLike(presents), 6, pin=True)   # rows 0..5 pinned
    pinned.length = 0
    got = m.forward(ids, pinned)
    assert not np.array_equal(got, base)
    np.testing.assert_array_equal(pinned.present(0)["value"][:, :6], presents[0]["value"][:, :6])
    # rows past the pin are the pass's own: layer 0's keys there do not depend on any cache row
    np.testing.assert_array_equal(pinned.present(0)["key"][:, 6:], c.present(0)["key"][:, 6:])
    with pytest.raises(ValueError):
        m.new_cache(4).shadow(0, 1)       # nothing pinned
