'use strict';
// The reference engine's CPU path, restated for Node 12 (CommonJS, no `??`, `?.` or
// private members): ReferenceModel.forward / generate (src/cpu/model.js:55-187) over
// the KV cache of src/cpu/cache.js, with the numeric ops of src/core/ops.js, the
// grouped attention of src/core/attention.js and the dequantizers of
// src/core/quantize.js:60-68,134-151. Storage is Float32Array, every reduction is a
// JavaScript number (f64), every store a Float32Array narrowing -- the reference's
// arithmetic in the reference's language and runtime (V8's Math.exp/cos/sin/pow).
//
// TEST INFRASTRUCTURE ONLY, like the rest of oracle/: bench.py's cpu_baseline leg runs
// it as the CPU baseline timed under Node, and tests/ check it against the C oracle
// (oracle.c). The product never loads it.
//
// Usage: node cpu_model.js <manifest.json>. The manifest names little-endian raw files:
//   config        {hidden, intermediate, layers, heads, kvHeads, headDim, vocab, ropeTheta, eps}
//   tensors       {name: {file, dtype: 'f32'|'u8'|'i8'|'u16', length}} -- layer matrices as the
//                 reference quantizer's arrays (int4: name.q/.scales/.zeros, int8: name.q/.scales),
//                 norms and biases f32, the embedding as bf16 bits (the input gather), the
//                 output head as int8 (the loader's round-tripped tied embedding)
//   scheme        'int4' | 'int8', group, kvF16 (cache entries rounded through f16)
//   cache         {file: u16 f16 bits [layers][2][context][kvDim], length: context}
//   first, steps  greedy decode of `steps` tokens from token `first` at position `context`
// Prints one JSON line: {tokens, seconds, steps, perStepSeconds, logitsFirst}.
const fs = require('fs');
const path = require('path');

// ------------------------------------------------------------- dtype.js ---
const f32buf = new Float32Array(1);
const u32buf = new Uint32Array(f32buf.buffer);

function bf16ToF32(bits) {  // src/core/dtype.js:17-20
  u32buf[0] = bits << 16;
  return f32buf[0];
}

function f16ToF32(h) {  // src/core/dtype.js:55-78
  const sign = h & 0x8000 ? -1 : 1;
  const exp = (h >> 10) & 0x1f;
  const mant = h & 0x3ff;
  if (exp === 0) return sign * mant * Math.pow(2, -24);
  if (exp === 0x1f) return mant ? NaN : sign * Infinity;
  return sign * (1 + mant / 1024) * Math.pow(2, exp - 15);
}

function f32ToF16(x) {  // src/core/dtype.js:81-113, round to nearest even
  f32buf[0] = x;
  const b = u32buf[0];
  const sign = (b >>> 16) & 0x8000;
  const exp = (b >>> 23) & 0xff;
  let mant = b & 0x7fffff;
  if (exp === 0xff) return sign | 0x7c00 | (mant ? (mant >>> 13) | 0x200 : 0);
  const e = exp - 127 + 15;
  if (e >= 0x1f) return sign | 0x7c00;
  if (e <= 0) {
    if (e < -10) return sign;
    mant |= 0x800000;
    const shift = 14 - e;
    let h = mant >>> shift;
    const rem = mant & ((1 << shift) - 1), half = 1 << (shift - 1);
    if (rem > half || (rem === half && (h & 1))) h++;
    return sign | h;
  }
  let h = (e << 10) | (mant >>> 13);
  const rem = mant & 0x1fff;
  if (rem > 0x1000 || (rem === 0x1000 && (h & 1))) h++;
  return sign | h;
}

// ---------------------------------------------------------- quantize.js ---
function dequantizeInt8(q, scales, rows, cols) {  // src/core/quantize.js:60-68
  const out = new Float32Array(rows * cols);
  for (let r = 0; r < rows; r++) {
    const s = scales[r], base = r * cols;
    for (let c = 0; c < cols; c++) out[base + c] = q[base + c] * s;
  }
  return out;
}

function dequantizeInt4(q, scales, zeros, rows, cols, group) {  // src/core/quantize.js:134-151
  const out = new Float32Array(rows * cols);
  const gpr = cols / group;
  for (let r = 0; r < rows; r++) {
    for (let g = 0; g < gpr; g++) {
      const s = scales[r * gpr + g], z = zeros[r * gpr + g];
      const base = r * cols + g * group;
      for (let i = 0; i < group; i++) {
        const at = base + i, byte = q[at >> 1];
        const level = (at & 1) === 0 ? byte & 0x0f : byte >> 4;
        out[at] = (level - z) * s;
      }
    }
  }
  return out;
}

// --------------------------------------------------------------- ops.js ---
function rmsNorm(x, xo, weight, eps, n, out) {  // src/core/ops.js:17-24
  let ss = 0;
  for (let i = 0; i < n; i++) ss += x[xo + i] * x[xo + i];
  const scale = 1 / Math.sqrt(ss / n + eps);
  for (let i = 0; i < n; i++) out[i] = x[xo + i] * scale * weight[i];
}

function matVec(W, x, xo, rows, cols, bias, out, oo) {  // src/core/ops.js:33-41
  for (let r = 0; r < rows; r++) {
    let acc = bias ? bias[r] : 0;
    const base = r * cols;
    for (let c = 0; c < cols; c++) acc += W[base + c] * x[xo + c];
    out[oo + r] = acc;
  }
}

function softmaxInPlace(x, n) {  // src/core/ops.js:66-78
  let max = -Infinity;
  for (let i = 0; i < n; i++) if (x[i] > max) max = x[i];
  let sum = 0;
  for (let i = 0; i < n; i++) {
    const e = Math.exp(x[i] - max);
    x[i] = e;
    sum += e;
  }
  const inv = 1 / sum;
  for (let i = 0; i < n; i++) x[i] = x[i] * inv;
}

function silu(x) { return x / (1 + Math.exp(-x)); }  // src/core/ops.js:81-83

function ropeFreqs(headDim, theta) {  // src/core/ops.js:99-104
  const half = headDim >> 1, inv = new Float64Array(half);
  for (let j = 0; j < half; j++) inv[j] = Math.pow(theta, (-2 * j) / headDim);
  return inv;
}

function ropeInPlace(v, offset, headDim, position, inv) {  // src/core/ops.js:147-159
  const half = headDim >> 1;
  for (let j = 0; j < half; j++) {
    const angle = position * inv[j], c = Math.cos(angle), s = Math.sin(angle);
    const lo = v[offset + j], hi = v[offset + j + half];
    v[offset + j] = lo * c - hi * s;
    v[offset + j + half] = hi * c + lo * s;
  }
}

// --------------------------------------------------------- attention.js ---
// src/core/attention.js:32-66: f64 dots stored f32, softmax, output accumulated in the
// f32 output array position by position; query head h reads kv head h / (heads/kvHeads).
function groupedAttention(q, keys, values, out, scores, seq, past, heads, kvHeads, headDim) {
  const group = heads / kvHeads, qDim = heads * headDim, kvDim = kvHeads * headDim;
  const scale = 1 / Math.sqrt(headDim);
  out.fill(0, 0, seq * qDim);
  for (let h = 0; h < heads; h++) {
    const kvBase = Math.floor(h / group) * headDim;
    for (let t = 0; t < seq; t++) {
      const qBase = t * qDim + h * headDim, upTo = past + t;
      for (let s = 0; s <= upTo; s++) {
        const kBase = s * kvDim + kvBase;
        let dot = 0;
        for (let i = 0; i < headDim; i++) dot += q[qBase + i] * keys[kBase + i];
        scores[s] = dot * scale;
      }
      softmaxInPlace(scores, upTo + 1);
      const oBase = t * qDim + h * headDim;
      for (let s = 0; s <= upTo; s++) {
        const w = scores[s], vBase = s * kvDim + kvBase;
        for (let i = 0; i < headDim; i++) out[oBase + i] = out[oBase + i] + w * values[vBase + i];
      }
    }
  }
}

// ------------------------------------------------------------ cache.js ---
class KVCache {  // src/cpu/cache.js:20-86
  constructor(layers, kvDim, capacity, kvF16) {
    this.kvDim = kvDim;
    this.capacity = capacity;
    this.length = 0;
    this.kvF16 = kvF16;
    this.keys = [];
    this.values = [];
    for (let l = 0; l < layers; l++) {
      this.keys.push(new Float32Array(capacity * kvDim));
      this.values.push(new Float32Array(capacity * kvDim));
    }
  }
  writeAt(layer, at, k, v, count) {  // cache.js:66-71 (entries through f16 when kvF16)
    const n = count * this.kvDim, kd = this.keys[layer], vd = this.values[layer], o = at * this.kvDim;
    for (let i = 0; i < n; i++) {
      kd[o + i] = this.kvF16 ? f16ToF32(f32ToF16(k[i])) : k[i];
      vd[o + i] = this.kvF16 ? f16ToF32(f32ToF16(v[i])) : v[i];
    }
  }
}

// ------------------------------------------------------------ model.js ---
class ReferenceModel {
  constructor(cfg, layers, finalNorm, embedBf16, lmHead) {
    this.cfg = cfg;
    this.layers = layers;
    this.finalNorm = finalNorm;
    this.embed = embedBf16;
    this.lmHead = lmHead;
    this.inv = ropeFreqs(cfg.headDim, cfg.ropeTheta);
  }

  // model.js:55-166 over token ids (the bf16 gather of model.js:190-209); returns the
  // last position's logits.
  forward(ids, cache) {
    const c = this.cfg, d = c.hidden, hd = c.headDim, kvDim = c.kvHeads * hd, ffn = c.intermediate;
    const seq = ids.length, past = cache.length;
    if (past + seq > cache.capacity) throw new RangeError('cache overflow');
    const x = new Float32Array(seq * d);
    for (let t = 0; t < seq; t++) {
      const id = ids[t];
      if (id < 0 || id >= c.vocab) throw new RangeError('token outside the vocabulary');
      for (let i = 0; i < d; i++) x[t * d + i] = bf16ToF32(this.embed[id * d + i]);
    }
    const normed = new Float32Array(d), q = new Float32Array(seq * d);
    const k = new Float32Array(seq * kvDim), v = new Float32Array(seq * kvDim);
    const attn = new Float32Array(seq * d), scores = new Float32Array(past + seq);
    const gate = new Float32Array(ffn), up = new Float32Array(ffn), proj = new Float32Array(d);
    for (let L = 0; L < c.layers; L++) {
      const w = this.layers[L];
      for (let t = 0; t < seq; t++) {
        rmsNorm(x, t * d, w.inputNorm, c.eps, d, normed);
        matVec(w.wq, normed, 0, d, d, w.bq, q, t * d);
        matVec(w.wk, normed, 0, kvDim, d, w.bk, k, t * kvDim);
        matVec(w.wv, normed, 0, kvDim, d, w.bv, v, t * kvDim);
        for (let h = 0; h < c.heads; h++) ropeInPlace(q, t * d + h * hd, hd, past + t, this.inv);
        for (let h = 0; h < c.kvHeads; h++) ropeInPlace(k, t * kvDim + h * hd, hd, past + t, this.inv);
      }
      cache.writeAt(L, past, k, v, seq);
      groupedAttention(q, cache.keys[L], cache.values[L], attn, scores, seq, past, c.heads, c.kvHeads, hd);
      for (let t = 0; t < seq; t++) {
        matVec(w.wo, attn, t * d, d, d, null, proj, 0);
        for (let i = 0; i < d; i++) x[t * d + i] = x[t * d + i] + proj[i];
      }
      for (let t = 0; t < seq; t++) {
        rmsNorm(x, t * d, w.postNorm, c.eps, d, normed);
        matVec(w.wGate, normed, 0, ffn, d, null, gate, 0);
        matVec(w.wUp, normed, 0, ffn, d, null, up, 0);
        for (let i = 0; i < ffn; i++) gate[i] = silu(gate[i]) * up[i];
        matVec(w.wDown, gate, 0, d, ffn, null, proj, 0);
        for (let i = 0; i < d; i++) x[t * d + i] = x[t * d + i] + proj[i];
      }
    }
    cache.length += seq;
    const logits = new Float32Array(c.vocab);
    rmsNorm(x, (seq - 1) * d, this.finalNorm, c.eps, d, normed);
    matVec(this.lmHead, normed, 0, c.vocab, d, null, logits, 0);
    return logits;
  }
}

function argmax(v) {  // model.js:181-182: strict '>', the lowest index wins ties
  let best = 0;
  for (let i = 1; i < v.length; i++) if (v[i] > v[best]) best = i;
  return best;
}

// ------------------------------------------------------------- loading ---
function readTyped(dir, t) {
  const buf = fs.readFileSync(path.join(dir, t.file));
  const ab = buf.buffer.slice(buf.byteOffset, buf.byteOffset + buf.length);
  switch (t.dtype) {
    case 'f32': return new Float32Array(ab);
    case 'u8': return new Uint8Array(ab);
    case 'i8': return new Int8Array(ab);
    case 'u16': return new Uint16Array(ab);
    default: throw new Error('unknown dtype ' + t.dtype);
  }
}

function loadModel(manifestPath) {
  const m = JSON.parse(fs.readFileSync(manifestPath, 'utf8'));
  const dir = path.dirname(manifestPath);
  const c = m.config, T = m.tensors;
  const get = function (name) { return readTyped(dir, T[name]); };
  const matrix = function (name, rows, cols) {
    if (m.scheme === 'int4') {
      return dequantizeInt4(get(name + '.q'), get(name + '.scales'), get(name + '.zeros'), rows, cols, m.group);
    }
    return dequantizeInt8(get(name + '.q'), get(name + '.scales'), rows, cols);
  };
  const d = c.hidden, kvDim = c.kvHeads * c.headDim, ffn = c.intermediate;
  const layers = [];
  for (let L = 0; L < c.layers; L++) {
    const p = 'model.layers.' + L + '.';
    layers.push({
      inputNorm: get(p + 'input_layernorm.weight'), postNorm: get(p + 'post_attention_layernorm.weight'),
      wq: matrix(p + 'self_attn.q_proj.weight', d, d), bq: get(p + 'self_attn.q_proj.bias'),
      wk: matrix(p + 'self_attn.k_proj.weight', kvDim, d), bk: get(p + 'self_attn.k_proj.bias'),
      wv: matrix(p + 'self_attn.v_proj.weight', kvDim, d), bv: get(p + 'self_attn.v_proj.bias'),
      wo: matrix(p + 'self_attn.o_proj.weight', d, d),
      wGate: matrix(p + 'mlp.gate_proj.weight', ffn, d), wUp: matrix(p + 'mlp.up_proj.weight', ffn, d),
      wDown: matrix(p + 'mlp.down_proj.weight', d, ffn),
    });
  }
  const lmHead = dequantizeInt8(get('lm_head.weight.q'), get('lm_head.weight.scales'), c.vocab, d);
  const model = new ReferenceModel(c, layers, get('model.norm.weight'), get('model.embed_tokens.weight'), lmHead);
  return { model: model, manifest: m, dir: dir };
}

function main() {
  const loaded = loadModel(process.argv[2]);
  const model = loaded.model, m = loaded.manifest, c = model.cfg;
  const kvDim = c.kvHeads * c.headDim;
  const cache = new KVCache(c.layers, kvDim, m.cache.length + m.steps + 1, m.kvF16);
  if (m.cache.length > 0) {  // the context, as f16 bits [layers][2][length][kvDim]
    const bits = readTyped(loaded.dir, { file: m.cache.file, dtype: 'u16' });
    const per = m.cache.length * kvDim;
    for (let L = 0; L < c.layers; L++) {
      for (let i = 0; i < per; i++) {
        cache.keys[L][i] = f16ToF32(bits[(2 * L) * per + i]);
        cache.values[L][i] = f16ToF32(bits[(2 * L + 1) * per + i]);
      }
    }
    cache.length = m.cache.length;
  }
  const tokens = [];
  let tok = m.first, logitsFirst = null;
  const t0 = process.hrtime.bigint();
  for (let s = 0; s < m.steps; s++) {
    const logits = model.forward([tok], cache);
    if (s === 0) logitsFirst = Array.prototype.slice.call(logits, 0, 8);
    tok = argmax(logits);
    tokens.push(tok);
  }
  const seconds = Number(process.hrtime.bigint() - t0) / 1e9;
  process.stdout.write(JSON.stringify({ tokens: tokens, seconds: seconds, steps: m.steps,
                                        perStepSeconds: seconds / m.steps, logitsFirst: logitsFirst }) + '\n');
}

if (require.main === module) main();

module.exports = { ReferenceModel, KVCache, loadModel, argmax, f32ToF16, f16ToF32, bf16ToF32,
                   dequantizeInt4, dequantizeInt8, groupedAttention, rmsNorm, matVec, softmaxInPlace };
