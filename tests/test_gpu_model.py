"""End-to-end parity of the decode step against the CPU oracle: logits within
the reference's model tolerance (test/model.test.js:39-40: logits 1e-4
relative), greedy tokens identical, and the bit-exact properties the reference
holds its GPU path to (prefill == incremental decode, web/model.html:169-198;
every replay of a step equal, web/decode-profile.html:162-167)."""
import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu

LOGIT_REL = 1e-4      # test/model.test.js:40


def rel_err(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / np.max(np.abs(ref)))


def tiny(hip, **kw):
    base = dict(hidden=128, intermediate=256, layers=2, heads=2, kv_heads=1, vocab=1000)
    base.update(kw)
    return hip.ModelConfig(**base)


@pytest.fixture(scope="module", params=[(s, n) for n in ("fast", "exact") for s in ("f16", "int8", "int4")],
                ids=lambda p: f"{p[0]}-{p[1]}")
def tiny_model(request, ctx, hip):
    scheme, numerics = request.param
    cfg = tiny(hip)
    ckpt = hip.synthesize_checkpoint(cfg, seed=3)
    lm = "int8" if scheme != "f16" else "f16"
    model = hip.GpuModel.load(ctx, hip.device_tensors(ckpt, cfg, scheme, 128, lm), cfg, maxPositions=256,
                              numerics=numerics)
    oracle = O.OracleModel(cfg, ckpt, scheme=scheme, group=128, lm_head=lm, kv_f16=True)
    yield cfg, model, oracle, scheme
    model.destroy()


def test_prompt_logits_and_greedy_tokens_match_oracle(hip, tiny_model):
    cfg, model, oracle, scheme = tiny_model
    prompt = hip.synth_tokens(3, "prompt", cfg.vocab, 12)
    cache = model.newCache(64)
    out = model.forward_tokens(prompt, cache)
    ologits = oracle.forward(prompt, oracle.new_cache(64))
    print(f"{scheme}: logits rel {rel_err(out['logits'], ologits):.2e}")
    assert rel_err(out["logits"], ologits) <= LOGIT_REL
    assert out["argmax"] == O.argmax(ologits) == int(np.argmax(out["logits"]))
    gen = model.decode(cache, out["argmax"], 20)
    want, _ = oracle.generate(prompt, 21)
    assert [out["argmax"]] + list(gen[:-1]) == list(want[:-1])
    assert gen[-1] == want[-1]
    assert cache.length == 12 + 20
    cache.destroy()


def test_prefill_equals_incremental_decode_bitwise(hip, tiny_model):
    cfg, model, _, _ = tiny_model
    ids = hip.synth_tokens(5, "ids", cfg.vocab, 9)
    full = model.newCache(16)
    a = model.forward_tokens(ids, full)
    inc = model.newCache(16)
    model.forward_tokens(ids[:4], inc, wantLogits=False)
    for t in ids[4:]:
        b = model.forward_tokens([t], inc)
    np.testing.assert_array_equal(a["logits"].view(np.uint32), b["logits"].view(np.uint32))
    for L in range(cfg.layers):
        pa, pb = full.present(L), inc.present(L)
        np.testing.assert_array_equal(pa["key"].view(np.uint32), pb["key"].view(np.uint32))
        np.testing.assert_array_equal(pa["value"].view(np.uint32), pb["value"].view(np.uint32))
    full.destroy()
    inc.destroy()


def test_graph_replay_equals_direct_steps(hip, tiny_model):
    cfg, model, _, _ = tiny_model
    prompt = hip.synth_tokens(6, "p", cfg.vocab, 5)
    c1, c2 = model.newCache(32), model.newCache(32)
    first = model.forward_tokens(prompt, c1)["argmax"]
    assert model.forward_tokens(prompt, c2)["argmax"] == first
    # runs of 8 steps replay as one graph launch, the rest step by step; the second call
    # reuses the captured graphs
    graph = list(model.decode(c1, first, 10))
    graph += list(model.decode(c1, graph[-1], 9))
    direct, tok = [], first
    for _ in range(19):
        tok = model.forward_tokens([tok], c2)["argmax"]
        direct.append(tok)
    assert list(graph) == direct
    for L in range(cfg.layers):
        np.testing.assert_array_equal(c1.present(L)["key"], c2.present(L)["key"])
    c1.destroy()
    c2.destroy()


def test_decode_calls_of_every_length_equal_one_token_forwards(hip, tiny_model):
    """A decode call is a gather, a first step, steps that each make their predecessor's pick
    in their own first launch (replayed in runs of 8, one at a time, or launched directly) and
    a pick launch for the last step. Calls of 1, 2, 8, 9 and 3 steps, replayed and launched
    directly, give the tokens, lengths and K/V of one-token forwards, each of which picks at the
    end of its own step. The last call fills the caches to their capacity."""
    cfg, model, _, _ = tiny_model
    prompt = hip.synth_tokens(9, "calls", cfg.vocab, 5)
    lengths = [1, 2, 8, 9, 3]
    capacity = len(prompt) + sum(lengths)
    graph, direct, single = (model.newCache(capacity) for _ in range(3))
    model.decode_use_graph(direct, False)
    first = model.forward_tokens(prompt, graph)["argmax"]
    for c in (direct, single):
        assert model.forward_tokens(prompt, c)["argmax"] == first
    got = {"graph": [], "direct": []}
    for name, c in (("graph", graph), ("direct", direct)):
        tok = first
        for n in lengths:
            out = list(model.decode(c, tok, n))
            assert len(out) == n
            got[name] += out
            tok = out[-1]
    want, tok = [], first
    for _ in range(sum(lengths)):
        tok = model.forward_tokens([tok], single)["argmax"]
        want.append(tok)
    assert got["graph"] == want and got["direct"] == want
    assert graph.length == direct.length == single.length == capacity
    for L in range(cfg.layers):
        ref = single.present(L)
        for c in (graph, direct):
            p = c.present(L)
            np.testing.assert_array_equal(p["key"].view(np.uint32), ref["key"].view(np.uint32))
            np.testing.assert_array_equal(p["value"].view(np.uint32), ref["value"].view(np.uint32))
    for c in (graph, direct, single):
        c.destroy()


def test_hidden_input_equals_token_gather(hip, tiny_model):
    cfg, model, _, _ = tiny_model
    ckpt_embed = hip.synthesize_checkpoint(cfg, seed=3)["model.embed_tokens.weight"]
    ids = hip.synth_tokens(8, "h", cfg.vocab, 4)
    hidden = hip.bf16_to_f32(ckpt_embed[ids]).reshape(-1)
    c1, c2 = model.newCache(8), model.newCache(8)
    a = model.forward(hidden, 4, cache=c1)
    b = model.forward_tokens(ids, c2)
    np.testing.assert_array_equal(a["logits"].view(np.uint32), b["logits"].view(np.uint32))
    c1.destroy()
    c2.destroy()


def test_rewind_replays_the_same_step(hip, tiny_model):
    # The profiler's replay (web/decode-profile.html:151): rewinding the length and
    # repeating a step reproduces its logits bit for bit.
    cfg, model, _, _ = tiny_model
    c = model.newCache(8)
    model.forward_tokens([1, 2, 3], c)
    a = model.forward_tokens([4], c)
    c.length = 3
    b = model.forward_tokens([4], c)
    np.testing.assert_array_equal(a["logits"].view(np.uint32), b["logits"].view(np.uint32))
    c.destroy()


def test_errors_are_raised_before_any_work(hip, tiny_model):
    cfg, model, _, _ = tiny_model
    c = model.newCache(4)
    with pytest.raises(hip.RangeError, match="cannot add"):
        model.forward_tokens([1, 2, 3, 4, 5], c)
    assert c.length == 0
    with pytest.raises(hip.RangeError, match="outside the vocabulary"):
        model.forward_tokens([cfg.vocab], c)
    with pytest.raises(hip.RangeError):
        model.decode(c, 1, 5)
    model.decode_launch(c, 1, 2)
    with pytest.raises(hip.BusyError):
        model.forward_tokens([1], c)
    model.decode_collect(c, 2)
    assert c.length == 2
    with pytest.raises(hip.RangeError):
        c.length = 3
    c.destroy()


def test_rope_table_bound(ctx, hip):
    cfg = tiny(hip, layers=1, vocab=256)
    ckpt = hip.synthesize_checkpoint(cfg, seed=1)
    model = hip.GpuModel.load(ctx, hip.device_tensors(ckpt, cfg, "int8", 128, "int8"), cfg, maxPositions=4)
    c = model.newCache(8)
    model.forward_tokens([1, 2, 3, 4], c)
    with pytest.raises(hip.RangeError, match="rope table"):
        model.forward_tokens([5], c)
    c.destroy()
    model.destroy()


def test_missing_tensor_is_reported(ctx, hip):
    cfg = tiny(hip, layers=1, vocab=256)
    t = hip.device_tensors(hip.synthesize_checkpoint(cfg, seed=1), cfg, "int4", 128, "int8")
    del t["model.layers.0.mlp.up_proj.weight"]
    with pytest.raises(hip.QwenHipError, match="missing 1 tensors: model.layers.0.mlp.up_proj"):
        hip.GpuModel.load(ctx, t, cfg, maxPositions=8)


# ---------------------------------------------------------------- full size

@pytest.fixture(scope="module")
def full_ckpt(hip):
    return hip.synthesize_checkpoint(hip.QWEN25_05B, seed=1)


@pytest.mark.parametrize("numerics", ["fast", "exact"])
def test_config1_full_shape_greedy_matches_oracle(ctx, hip, full_ckpt, numerics):
    """Config 1: 16 seeded prompt ids, 32 greedy tokens, Qwen2.5-0.5B shape. Weights are
    the reference GPU path's f16; the oracle sees the same f16 weights and f16 cache."""
    cfg = hip.QWEN25_05B
    model = hip.GpuModel.load(ctx, hip.device_tensors(full_ckpt, cfg, "f16", 128, "f16"), cfg,
                              maxPositions=64, numerics=numerics)
    prompt = hip.synth_tokens(1, "config1.prompt", cfg.vocab, 16)
    cache = model.newCache(48)
    out = model.forward_tokens(prompt, cache)
    gen = model.decode(cache, out["argmax"], 31)
    tokens = [out["argmax"]] + list(gen)
    oracle = O.OracleModel(cfg, full_ckpt, scheme="f16", lm_head="f16", kv_f16=True)
    ocache = oracle.new_cache(48)
    ologits = oracle.forward(prompt, ocache)
    print(f"config1 logits rel {rel_err(out['logits'], ologits):.2e}")
    assert rel_err(out["logits"], ologits) <= LOGIT_REL
    want, _ = oracle.generate(prompt, 32)
    assert tokens == list(want)
    cache.destroy()
    model.destroy()


@pytest.mark.parametrize("numerics", ["fast", "exact"])
def test_config4_full_shape_int4_matches_oracle(ctx, hip, full_ckpt, numerics):
    """Config 4's model (int4-g128 layers, int8 output head, f16 cache) on a shorter
    context: 64 prompt ids then 24 greedy tokens, plus the per-layer present K/V. Exact
    numerics: the cache equals the oracle's bit for bit but for f64-ordering ties. Both: every
    stored entry within half an f16 unit of the CPU's unrounded value on the same inputs (the
    same-f16 oracle's shadow rows), so the per-layer max-abs is within the reference's 5e-4."""
    cfg = hip.QWEN25_05B
    model = hip.GpuModel.load(ctx, hip.device_tensors(full_ckpt, cfg, "int4", 128, "int8"), cfg,
                              maxPositions=128, numerics=numerics)
    prompt = hip.synth_tokens(4, "config4.prompt", cfg.vocab, 64)
    cache = model.newCache(96)
    out = model.forward_tokens(prompt, cache)
    oracle = O.OracleModel(cfg, full_ckpt, scheme="int4", group=128, lm_head="int8", kv_f16=True)
    ocache = oracle.new_cache(96)
    ologits = oracle.forward(prompt, ocache)
    print(f"config4 logits rel {rel_err(out['logits'], ologits):.2e}")
    assert rel_err(out["logits"], ologits) <= LOGIT_REL
    same = oracle.new_cache(96)
    same.load_device(cache, 64, pin=True)
    same.length = 0
    slogits = oracle.forward(prompt, same)
    worst, worst_same, min_cos, equal, total = 0.0, 0.0, 1.0, 0, 0
    for L in range(cfg.layers):
        for kind in ("key", "value"):
            g, o, sh = cache.present(L)[kind], ocache.present(L)[kind], same.shadow(L, 64)[kind]
            worst = max(worst, rel_err(g, o))
            worst_same = max(worst_same, rel_err(g, sh))
            half = 0.5 * np.spacing(np.abs(sh).astype(np.float16)).astype(np.float64)
            assert np.all(np.abs(g.astype(np.float64) - sh) <= half + 1e-5 * np.max(np.abs(sh))), (L, kind)
            gd, od = g.astype(np.float64).ravel(), o.astype(np.float64).ravel()
            min_cos = min(min_cos, float(gd @ od / (np.linalg.norm(gd) * np.linalg.norm(od))))
            equal += int(np.sum(g.view(np.uint32) == o.view(np.uint32)))
            total += g.size
    print(f"config4 {numerics}: per-layer present max-abs rel {worst:.2e} vs the oracle, {worst_same:.2e} vs the "
          f"CPU's unrounded values; min cosine {min_cos:.9f}, bit-identical {equal}/{total}; same-f16 logits rel "
          f"{rel_err(out['logits'], slogits):.2e}")
    assert worst_same <= 5e-4      # PER_LAYER_REL, test/model.test.js:39
    assert rel_err(out["logits"], slogits) <= LOGIT_REL
    assert min_cos >= 0.99999
    if numerics == "exact":
        assert worst <= 5e-4
        assert equal / total >= 0.999
    gen = model.decode(cache, out["argmax"], 23)
    want, _ = oracle.generate(prompt, 24)
    assert [out["argmax"]] + list(gen) == list(want)
    cache.destroy()
    model.destroy()


@pytest.mark.parametrize("prompt_len", [1400, 3000, 9000])
def test_fast_numerics_long_context_matches_exact(ctx, hip, prompt_len):
    """Past 16 x 64 positions each split-K slot of the fast path spans several chunks, past
    2048 a slot has more 32-key steps than its block has waves (each wave then walks several),
    and past 8192 the cache takes the long form (128 slots, merged by a launch of its own); the
    fast step must stay within the logit tolerance of the exact one and choose the same greedy
    tokens."""
    cfg = tiny(hip)
    ckpt = hip.synthesize_checkpoint(cfg, seed=11)
    tensors = hip.device_tensors(ckpt, cfg, "int4", 128, "int8")
    fast = hip.GpuModel.load(ctx, tensors, cfg, maxPositions=prompt_len + 200, numerics="fast")
    exact = hip.GpuModel.load(ctx, tensors, cfg, maxPositions=prompt_len + 200, numerics="exact")
    prompt = hip.synth_tokens(11, "long", cfg.vocab, prompt_len)
    cf, ce = fast.newCache(prompt_len + 100), exact.newCache(prompt_len + 100)
    a = fast.forward_tokens(prompt, cf)
    b = exact.forward_tokens(prompt, ce)
    print(f"long context fast vs exact logits rel {rel_err(a['logits'], b['logits']):.2e}")
    assert rel_err(a["logits"], b["logits"]) <= LOGIT_REL
    assert a["argmax"] == b["argmax"]
    assert list(fast.decode(cf, a["argmax"], 16)) == list(exact.decode(ce, b["argmax"], 16))
    with pytest.raises(hip.QwenHipError, match="before the model's first cache"):
        hip._check(fast.lib.qh_model_set_numerics(fast.handle, 1))
    for c in (cf, ce):
        c.destroy()
    fast.destroy()
    exact.destroy()


@pytest.mark.parametrize("numerics", ["fast", "exact"])
@pytest.mark.parametrize("scheme", ["f16", "int8", "int4"])
def test_batched_prefill_equals_one_position_steps_bitwise(ctx, hip, numerics, scheme):
    """QH_MATMUL_BATCHED runs all positions per layer through 8-position weight tiles; every
    output is summed as the decode step sums it, so its logits and cache equal a prefill made
    of single decode steps (QH_MATMUL_MATVEC) bit for bit -- over two 512-position chunks."""
    cfg = tiny(hip)
    ckpt = hip.synthesize_checkpoint(cfg, seed=21)
    lm = "int8" if scheme != "f16" else "f16"
    model = hip.GpuModel.load(ctx, hip.device_tensors(ckpt, cfg, scheme, 128, lm), cfg, maxPositions=1100,
                              numerics=numerics)
    ids = hip.synth_tokens(21, "batched", cfg.vocab, 600)
    cb, cs = model.newCache(1024), model.newCache(1024)
    a = model.forward_tokens(ids, cb)
    model.set_matmul("matvec")
    b = model.forward_tokens(ids, cs)
    np.testing.assert_array_equal(a["logits"].view(np.uint32), b["logits"].view(np.uint32))
    assert a["argmax"] == b["argmax"]
    for L in range(cfg.layers):
        pa, pb = cb.present(L), cs.present(L)
        np.testing.assert_array_equal(pa["key"].view(np.uint32), pb["key"].view(np.uint32))
        np.testing.assert_array_equal(pa["value"].view(np.uint32), pb["value"].view(np.uint32))
    # and decoding on from either cache continues identically
    assert list(model.decode(cb, a["argmax"], 6)) == list(model.decode(cs, b["argmax"], 6))
    cb.destroy()
    cs.destroy()
    model.destroy()


def test_long_cache_batched_prefill_equals_one_position_steps_bitwise(ctx, hip):
    """A cache past 8192 positions takes the long attention form (128 slots per head, merged
    by their own launch before the o-projection); the batched prefill (the slots of a share
    of the rows at a time) still equals single decode steps bit for bit, and decoding on
    matches."""
    cfg = tiny(hip)
    ckpt = hip.synthesize_checkpoint(cfg, seed=23)
    model = hip.GpuModel.load(ctx, hip.device_tensors(ckpt, cfg, "int4", 128, "int8"), cfg, maxPositions=8400)
    ids = hip.synth_tokens(23, "long.batched", cfg.vocab, 700)
    cb, cs = model.newCache(8300), model.newCache(8300)
    a = model.forward_tokens(ids, cb)
    model.set_matmul("matvec")
    b = model.forward_tokens(ids, cs)
    np.testing.assert_array_equal(a["logits"].view(np.uint32), b["logits"].view(np.uint32))
    for L in range(cfg.layers):
        pa, pb = cb.present(L), cs.present(L)
        np.testing.assert_array_equal(pa["key"].view(np.uint32), pb["key"].view(np.uint32))
        np.testing.assert_array_equal(pa["value"].view(np.uint32), pb["value"].view(np.uint32))
    assert list(model.decode(cb, a["argmax"], 6)) == list(model.decode(cs, b["argmax"], 6))
    cb.destroy()
    cs.destroy()
    model.destroy()


@pytest.mark.parametrize("numerics", ["fast", "exact"])
def test_config5_prefill_batched_and_mfma_match_oracle(ctx, hip, full_ckpt, numerics):
    """Config 5's model (int8 layers and head, f16 cache) prefilling a seeded 96-token prompt.

    The batched tiles sum as the CPU does: logits within LOGIT_REL of the oracle's own prefill
    (exact numerics: equal). The MFMA contraction agrees with the CPU's f64 sums to ~4e-7 per
    output but not to the bit, so an entry of its f16 cache can round to the neighbouring f16
    value where the CPU's does not; it is held to LOGIT_REL against the same-f16 oracle (the
    oracle attending to the MFMA run's own cache rows, web/kernels.html:51-54), with the same
    argmax, and every stored K/V entry within half an f16 unit of the CPU's unrounded value."""
    cfg = hip.QWEN25_05B
    model = hip.GpuModel.load(ctx, hip.device_tensors(full_ckpt, cfg, "int8", 128, "int8"), cfg,
                              maxPositions=256, numerics=numerics)
    prompt = hip.synth_tokens(5, "config5.prompt", cfg.vocab, 96)
    oracle = O.OracleModel(cfg, full_ckpt, scheme="int8", lm_head="int8", kv_f16=True)
    ologits = oracle.forward(prompt, oracle.new_cache(128))
    for mode in ("batched", "mfma"):
        model.set_matmul(mode)
        cache = model.newCache(128)
        out = model.forward_tokens(prompt, cache)
        err = rel_err(out["logits"], ologits)
        same = oracle.new_cache(128)
        same.load_device(cache, prompt.size, pin=True)
        same.length = 0
        serr = rel_err(out["logits"], oracle.forward(prompt, same))
        print(f"config5 {numerics} {mode}: logits rel {err:.2e} (oracle), {serr:.2e} (same-f16 oracle)")
        assert serr <= LOGIT_REL
        assert out["argmax"] == O.argmax(ologits)
        if mode == "batched":
            assert err <= LOGIT_REL
            if numerics == "exact":
                assert err == 0.0
        for L in range(cfg.layers):
            g, o = cache.present(L), same.shadow(L, prompt.size)
            for kind in ("key", "value"):
                a, b = g[kind].astype(np.float64), o[kind].astype(np.float64)
                half = 0.5 * np.spacing(np.abs(b).astype(np.float16)).astype(np.float64)
                assert np.all(np.abs(a - b) <= half + 1e-5 * np.max(np.abs(b))), (mode, L, kind)
        cache.destroy()
    model.destroy()


@pytest.mark.parametrize("capacity,seq", [(66, 64), (130, 64), (600, 65)])
def test_mfma_prefill_shorter_than_its_workspace(ctx, hip, full_ckpt, capacity, seq):
    """A cache's prefill workspace serves every prompt of up to min(capacity, 512) positions.
    The MFMA contraction splits K more finely when a prompt has fewer 64-row tiles, so a
    prompt shorter than the workspace can need more split partials than the workspace's own
    length (capacity 66 or 130 with 64 positions, at the o-projection's 896 x 896); the
    workspace is sized for the largest need over every length."""
    cfg = hip.QWEN25_05B
    model = hip.GpuModel.load_checkpoint(ctx, full_ckpt, cfg, "int8", 128, "int8", maxPositions=capacity + 8)
    prompt = hip.synth_tokens(6, "short.prompt", cfg.vocab, seq)
    oracle = O.OracleModel(cfg, full_ckpt, scheme="int8", lm_head="int8", kv_f16=True)
    res = {}
    for mode in ("batched", "mfma"):
        model.set_matmul(mode)
        cache = model.newCache(capacity)
        res[mode] = model.forward_tokens(prompt, cache)
        if mode == "mfma":     # the same-f16 oracle: attending to this run's own cache rows
            same = oracle.new_cache(capacity)
            same.load_device(cache, seq, pin=True)
            same.length = 0
            ref = oracle.forward(prompt, same)
        cache.destroy()
    err = rel_err(res["mfma"]["logits"], ref)
    print(f"mfma prefill {seq} positions, capacity {capacity}: logits rel {err:.2e} vs the same-f16 oracle, "
          f"{rel_err(res['mfma']['logits'], res['batched']['logits']):.2e} vs batched")
    assert err <= LOGIT_REL
    assert res["mfma"]["argmax"] == res["batched"]["argmax"] == O.argmax(ref)
    model.destroy()


@pytest.mark.parametrize("path", ["batched", "mfma"])
def test_prefill_graph_replays_equal_direct_launches(ctx, hip, path):
    """A prompt shape run again is replayed from a graph captured on its second use: every run
    (direct, capturing, replayed) stores the same K/V and returns the same logits, bit for bit,
    as a cache that launches every kernel directly, with other work on the stream and host
    synchronizations between the replays."""
    cfg = tiny(hip)
    ckpt = hip.synthesize_checkpoint(cfg, seed=21)
    model = hip.GpuModel.load(ctx, hip.device_tensors(ckpt, cfg, "int8", 128, "int8"), cfg, maxPositions=128)
    model.set_matmul(path)
    prompt = hip.synth_tokens(21, "graph.prompt", cfg.vocab, 40)
    direct = model.newCache(64)
    model.decode_use_graph(direct, False)
    ref = model.forward_tokens(prompt, direct)
    other = model.newCache(64)
    replayed = model.newCache(64)
    for run in range(4):
        replayed.length = 0
        out = model.forward_tokens(prompt, replayed)
        np.testing.assert_array_equal(out["logits"].view(np.uint32), ref["logits"].view(np.uint32))
        assert out["argmax"] == ref["argmax"]
        for L in (0, cfg.layers - 1):
            a, b = replayed.present(L), direct.present(L)
            np.testing.assert_array_equal(a["key"].view(np.uint32), b["key"].view(np.uint32))
            np.testing.assert_array_equal(a["value"].view(np.uint32), b["value"].view(np.uint32))
        other.length = 0
        model.forward_tokens(prompt[: 7 + run], other)   # eager work between the replays
        ctx.done()
    for c in (direct, other, replayed):
        c.destroy()
    model.destroy()
