'use strict';
// The reference's caller, web/bench.html:62-134, against this backend's JS driver: a config
// and a checkpoint reader shaped exactly like the reference's ModelConfig and Safetensors
// (src/core/config.js, src/core/safetensors.js: plain properties; async readRaw / readF32),
// GpuModel.load with quantize = null (f16 weights, the reference's format), host-side
// embedding, forward() per token with the host argmax scan, wantPresent, and the cache's
// per-layer keys / values buffers destroyed as the caller destroys them. Two kv heads, so the
// position-major `present` rows and web/model.html's reshape of them (toPresentLayout) differ
// from the head-major layout. Prints JSON for tests/test_js_addon.py. Usage: node reference_caller.js
const path = require('path');
const qh = require(path.join(__dirname, '..', '..', 'llm-inference-webgpu_amd', 'js', 'gpu_model.js'));
const { GpuContext, GpuModel } = qh;

// What the reference's ModelConfig constructor leaves on the object (config.js:16-70).
const config = {
  modelType: 'qwen2', architectures: ['Qwen2ForCausalLM'], hiddenSize: 256, intermediateSize: 256, numLayers: 2,
  numHeads: 4, numKVHeads: 2, vocabSize: 1000, maxPositionEmbeddings: 32768, ropeTheta: 1000000, rmsNormEps: 1e-6,
  hiddenAct: 'silu', tieWordEmbeddings: true, useSlidingWindow: false, slidingWindow: null, bosTokenId: null,
  eosTokenId: null, headDim: 64, kvGroupSize: 2, kvDim: 128,
};

// web/model.html's reshape of a present row block: [positions, kvHeads*headDim] into the ONNX
// [kvHeads, positions, headDim] (written here for this test, same index map).
function toPresentLayout(flat, positions, numKVHeads, headDim) {
  const kvDim = numKVHeads * headDim;
  const out = new Float32Array(numKVHeads * positions * headDim);
  for (let t = 0; t < positions; t++) {
    for (let h = 0; h < numKVHeads; h++) {
      for (let i = 0; i < headDim; i++) out[(h * positions + t) * headDim + i] = flat[t * kvDim + h * headDim + i];
    }
  }
  return out;
}

// A reader with the reference Safetensors' surface over an in-memory bf16 checkpoint; one
// tensor's bytes come back at an odd offset, as a byte source may return them.
function referenceReader(ckpt) {
  const infos = new Map();
  let at = 0;
  Object.keys(ckpt).forEach(function (name) {
    const t = ckpt[name];
    const numel = t.shape.reduce(function (a, b) { return a * b; }, 1);
    infos.set(name, Object.freeze({ name: name, dtype: 'BF16', shape: Object.freeze(t.shape.slice()), begin: at,
                                    end: at + 2 * numel, numel: numel, byteLength: 2 * numel }));
    at += 2 * numel;
  });
  return {
    metadata: null,
    get size() { return infos.size; },
    names: function () { return Array.from(infos.keys()); },
    has: function (n) { return infos.has(n); },
    info: function (n) {
      const t = infos.get(n);
      if (!t) throw new Error('no tensor named ' + JSON.stringify(n));
      return t;
    },
    readRaw: async function (n) {
      const bits = ckpt[n].data;
      const bytes = new Uint8Array(bits.buffer, bits.byteOffset, bits.byteLength);
      if (n !== 'model.layers.1.mlp.down_proj.weight') return bytes.slice();
      const odd = new Uint8Array(bytes.length + 1);
      odd.set(bytes, 1);
      return odd.subarray(1);
    },
    readF32: async function (n) { return qh.bf16ToF32Array(ckpt[n].data); },
  };
}

async function main() {
  const dims = { hidden: 256, intermediate: 256, layers: 2, heads: 4, kvHeads: 2, vocab: 1000 };
  const ckpt = qh.synthesizeCheckpoint(dims, 3);
  const st = referenceReader(ckpt);
  const ctx = GpuContext.create(0);
  let ticks = 0;
  const model = await GpuModel.load(ctx, st, config, {
    maxPositions: 64, onProgress: function (done, total) { ticks = total; },
  });
  const d = config.hiddenSize;
  const embedBits = ckpt['model.embed_tokens.weight'].data;
  function embed(ids) {
    const arr = new Float32Array(ids.length * d);
    for (let t = 0; t < ids.length; t++) {
      arr.set(qh.bf16ToF32Array(embedBits.subarray(ids[t] * d, (ids[t] + 1) * d)), t * d);
    }
    return arr;
  }
  function argmax(logits) {
    let best = 0;
    for (let j = 1; j < logits.length; j++) if (logits[j] > logits[best]) best = j;
    return best;
  }
  const ids = Array.from(qh.synthTokens(3, 'prompt', config.vocabSize, 12));
  // a warm pass, its cache's buffers destroyed one by one as web/bench.html:101-104 does
  const warm = model.newCache(ids.length + 4);
  await model.forward(embed(ids).subarray(0, 4 * d), 4, { cache: warm, wantLogits: true });
  const warmBytes = warm.byteLength, layers = warm.keys.length;
  for (const b of warm.keys.concat(warm.values)) b.destroy();
  const freed = warm.handle === null;

  const cache = model.newCache(ids.length + 16);
  const first = await model.forward(embed(ids), ids.length, { cache: cache, wantLogits: true });
  let token = argmax(first.logits);
  const generated = [token];
  let last = null;
  for (let i = 0; i < 6; i++) {
    last = await model.forward(embed([token]), 1, { cache: cache, wantLogits: true, wantPresent: i === 5 });
    token = argmax(last.logits);
    generated.push(token);
  }
  let busy = null;
  const p = model.forward(embed([token]), 1, { cache: cache, wantLogits: false });
  try { await model.forward(embed([token]), 1, { cache: cache }); } catch (e) { busy = e.message; }
  await p;
  const b64 = function (a) { return Buffer.from(a.buffer, a.byteOffset, a.byteLength).toString('base64'); };
  const positions = cache.length - 1;
  const present = last.present.map(function (l) {
    return {
      key: b64(l.key), value: b64(l.value),
      keyOnnx: b64(toPresentLayout(l.key, positions, config.numKVHeads, config.headDim)),
      valueOnnx: b64(toPresentLayout(l.value, positions, config.numKVHeads, config.headDim)),
    };
  });
  const rowsOk = cache.keys[1].read().length === (cache.length) * config.kvDim;
  let tiledOk = true;
  try { model.setMatmul('tiled'); model.setMatmul('batched'); } catch (e) { tiledOk = e.message; }
  let badMatmul = null;
  try { model.setMatmul('blocked'); } catch (e) { badMatmul = e.message; }
  process.stdout.write(JSON.stringify({
    ticks: ticks, layers: layers, warmBytes: warmBytes, freed: freed, tokens: generated,
    firstLogits: Buffer.from(first.logits.buffer).toString('base64'), hiddenBuffer: first.hiddenBuffer,
    present: present, presentLength: positions, cacheLength: cache.length, busy: busy, rowsOk: rowsOk,
    tiles: [1, 2, 3, 4, 7, 8, 512].map(GpuModel.batchTileFor), tiled: tiledOk, badMatmul: badMatmul,
  }) + '\n');
  cache.destroy();
  model.destroy();
  ctx.destroy();
}

main().catch(function (e) { console.error(e && e.stack ? e.stack : e); process.exit(1); });
