'use strict';
// Loads a checkpoint directory (config.json + model.safetensors) through the Node-API driver
// and prints the prompt logits and a greedy decode as JSON, for tests/test_gpu_checkpoint.py.
// Usage: node file_decode.js <dir> <scheme> <headScheme> <convert: device|host>
const fs = require('fs');
const path = require('path');
const qh = require(path.join(__dirname, '..', '..', 'llm-inference-webgpu_amd', 'js', 'gpu_model.js'));

async function main() {
  const dir = process.argv[2];
  const scheme = process.argv[3] || 'int4';
  const head = process.argv[4] || 'int8';
  const convert = process.argv[5] || 'device';
  const cfg = qh.ModelConfig.parse(fs.readFileSync(path.join(dir, 'config.json'), 'utf8'));
  const ctx = qh.GpuContext.create(0);
  const st = qh.Safetensors.open(path.join(dir, 'model.safetensors'));
  const model = await qh.GpuModel.load(ctx, st, cfg, {
    maxPositions: 64, quantize: { scheme: scheme, groupSize: 128 }, headScheme: head, convert: convert,
  });
  st.close();
  const prompt = qh.synthTokens(9, 'prompt', cfg.vocabSize, 7);
  const cache = model.newCache(32);
  const out = model.forwardTokens(prompt, cache);
  const gen = model.decode(cache, out.argmax, 8);
  process.stdout.write(JSON.stringify({
    argmax: out.argmax, tokens: Array.from(gen), logits: Buffer.from(out.logits.buffer).toString('base64'),
  }) + '\n');
  cache.destroy();
  model.destroy();
  ctx.destroy();
}

main().catch(function (e) { console.error(e && e.stack ? e.stack : e); process.exit(1); });
