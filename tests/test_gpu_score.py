"""Perplexity scoring on the device kernels (qh_score): the reference's perplexity page scores a
passage one token at a time through the cache and takes -log softmax at the true next token
(web/perplexity.html:146-170). Here every step is the decode step itself (int8/int4 codes read by
the kernels, not an f16 round trip), and the log-softmax runs on the device in f64.

Checks, per weight format and numerics mode:
  - each NLL equals the oracle's expression (oracle/oracle.c `or_nll`) applied to the logits the
    same step returns through forward() (same kernels, so the same f32 logits): 1e-12;
  - against the CPU oracle's own logits for the same fed tokens: within what the logit tolerance
    allows (|dNLL| <= 2 x 1e-4 x max|logit|, test/model.test.js:40), exactly (1e-11) for the exact
    numerics, whose logits equal the oracle's;
  - the cache holds the same K/V rows as the forward() run."""
import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu

LOGIT_REL = 1e-4      # test/model.test.js:40


def tiny(hip):
    return hip.ModelConfig(hidden=128, intermediate=256, layers=2, heads=2, kv_heads=1, vocab=1000)


@pytest.mark.parametrize("numerics", ["fast", "exact"])
@pytest.mark.parametrize("scheme", ["f16", "int8", "int4"])
def test_score_matches_step_logits_and_the_oracle(ctx, hip, scheme, numerics):
    cfg = tiny(hip)
    ckpt = hip.synthesize_checkpoint(cfg, seed=31)
    lm = "f16" if scheme == "f16" else "int8"
    model = hip.GpuModel.load(ctx, hip.device_tensors(ckpt, cfg, scheme, 128, lm), cfg, maxPositions=128,
                              numerics=numerics)
    ids = hip.synth_tokens(31, "score.ids", cfg.vocab, 30)
    scored = model.newCache(64)
    nll = model.score(ids, scored)
    assert nll.shape == (29,) and scored.length == 29

    stepped = model.newCache(64)
    oracle = O.OracleModel(cfg, ckpt, scheme=scheme, group=128, lm_head=lm, kv_f16=True)
    oc = oracle.new_cache(64)
    worst = 0.0
    for t in range(29):
        out = model.forward_tokens([ids[t]], stepped)
        assert nll[t] == pytest.approx(O.nll(out["logits"], ids[t + 1]), rel=1e-12, abs=1e-12)
        ol = oracle.forward([ids[t]], oc)
        diff = abs(nll[t] - O.nll(ol, ids[t + 1]))
        bound = 1e-11 if numerics == "exact" else 2 * LOGIT_REL * float(np.max(np.abs(ol)))
        assert diff <= bound, (t, diff, bound)
        worst = max(worst, diff)
    ppl = float(np.exp(nll.mean()))
    print(f"{scheme}-{numerics}: perplexity {ppl:.4f} over 29 positions, worst |dNLL| vs the oracle {worst:.2e}")
    for L in range(cfg.layers):
        a, b = scored.present(L), stepped.present(L)
        np.testing.assert_array_equal(a["key"].view(np.uint32), b["key"].view(np.uint32))
        np.testing.assert_array_equal(a["value"].view(np.uint32), b["value"].view(np.uint32))
    scored.destroy()
    stepped.destroy()
    model.destroy()


def test_score_continues_from_a_prompt(ctx, hip):
    """Scoring after a batched prefill scores the later tokens with the full left context."""
    cfg = tiny(hip)
    ckpt = hip.synthesize_checkpoint(cfg, seed=32)
    model = hip.GpuModel.load(ctx, hip.device_tensors(ckpt, cfg, "int4", 128, "int8"), cfg, maxPositions=128)
    ids = hip.synth_tokens(32, "score.context", cfg.vocab, 40)
    a = model.newCache(64)
    whole = model.score(ids, a)
    b = model.newCache(64)
    model.forward_tokens(ids[:15], b, wantLogits=False)   # positions 0..14 through the 8-position tiles
    tail = model.score(ids[15:], b)                        # feeds ids[15..38], scores ids[16..39]
    assert tail.shape == (24,) and b.length == 15 + 24
    # the batched prefill equals one-position steps bit for bit, so the scores agree exactly
    np.testing.assert_array_equal(whole[15:], tail)
    a.destroy()
    b.destroy()
    model.destroy()


def test_score_errors(ctx, hip):
    cfg = tiny(hip)
    ckpt = hip.synthesize_checkpoint(cfg, seed=33)
    model = hip.GpuModel.load(ctx, hip.device_tensors(ckpt, cfg, "int8", 128, "int8"), cfg, maxPositions=64)
    c = model.newCache(8)
    with pytest.raises(hip.QwenHipError, match="at least two tokens"):
        model.score([1], c)
    with pytest.raises(hip.RangeError, match="outside the vocabulary"):
        model.score([1, cfg.vocab], c)
    with pytest.raises(hip.RangeError, match="cannot add"):
        model.score(list(range(12)), c)
    assert c.length == 0
    c.destroy()
    model.destroy()
