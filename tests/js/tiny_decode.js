'use strict';
// Drives a tiny Qwen2-shaped model through the Node-API driver: prompt logits, argmax and a
// greedy decode, printed as JSON for tests/test_js_addon.py to compare with the Python binding.
// Usage: node tiny_decode.js <scheme> <numerics> <matmul> <convert: device|host>
const path = require('path');
const qh = require(path.join(__dirname, '..', '..', 'llm-inference-webgpu_amd', 'js', 'gpu_model.js'));

async function main() {
  const scheme = process.argv[2] || 'int4';
  const numerics = process.argv[3] || 'fast';
  const matmul = process.argv[4] || 'batched';
  const convert = process.argv[5] || 'device';
  const cfg = { hidden: 128, intermediate: 256, layers: 2, heads: 2, kvHeads: 1, vocab: 1000, ropeTheta: 1e6, eps: 1e-6 };
  const ctx = qh.GpuContext.create(0);
  const ckpt = qh.synthesizeCheckpoint(cfg, 3);
  const model = await qh.GpuModel.load(ctx, ckpt, cfg, {
    maxPositions: 256, quantize: { scheme: scheme, groupSize: 128 }, headScheme: scheme === 'f16' ? 'f16' : 'int8',
    numerics: numerics, matmul: matmul, convert: convert,
  });
  const prompt = qh.synthTokens(3, 'prompt', cfg.vocab, 12);
  const cache = model.newCache(64);
  const out = model.forwardTokens(prompt, cache);
  const gen = model.decode(cache, out.argmax, 8);
  // the caller's loop of web/bench.html:121-134 with host-side embedding: forward(hidden) per token
  const c2 = model.newCache(64);
  const emb = ckpt['model.embed_tokens.weight'];
  const hidden = new Float32Array(prompt.length * cfg.hidden);
  for (let t = 0; t < prompt.length; t++) {
    hidden.set(qh.bf16ToF32Array(emb.data.subarray(prompt[t] * cfg.hidden, (prompt[t] + 1) * cfg.hidden)), t * cfg.hidden);
  }
  const viaHidden = await model.forward(hidden, prompt.length, { cache: c2 });
  const c3 = model.newCache(64);
  const nll = model.score(prompt, c3);   // web/perplexity.html's per-token NLLs
  let rangeError = null;
  try { model.forwardTokens([cfg.vocab], c2); } catch (e) { rangeError = e instanceof RangeError ? e.message : 'other'; }
  process.stdout.write(JSON.stringify({
    argmax: out.argmax, tokens: Array.from(gen), logits: Buffer.from(out.logits.buffer).toString('base64'),
    hiddenArgmax: viaHidden.argmax, hiddenLogits: Buffer.from(viaHidden.logits.buffer).toString('base64'),
    cacheLength: cache.length, rangeError: rangeError, bytes: model.byteLength,
    score: Buffer.from(nll.buffer).toString('base64'), scoredLength: c3.length,
  }) + '\n');
  cache.destroy();
  c2.destroy();
  c3.destroy();
  model.destroy();
  ctx.destroy();
}

main().catch(function (e) { console.error(e && e.stack ? e.stack : e); process.exit(1); });
