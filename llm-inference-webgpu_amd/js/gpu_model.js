'use strict';
// GpuContext / GpuModel / GpuKVCache over libqwen_hip.so, with the method names and
// argument shapes of the reference's src/gpu/device.js and src/gpu/model.js, so the
// callers' decode loop (web/bench.html:121-134) carries over. Written for Node 12
// (CommonJS, no optional chaining or private methods). The addon only marshals
// arguments; this file holds the loader logic of GpuModel.load (src/gpu/model.js:147-207):
// tensors by checkpoint name, bf16 widened exactly, 2-D layer weights quantized per
// the `quantize` option with the reference quantizer's layout, the tied embedding as
// the output projection.

const path = require('path');
const addon = require(path.join(__dirname, 'addon', 'qwen_napi.node'));
const { Safetensors, parseConfig, expectedTensors, checkAgainst } = require('./safetensors.js');

const FMT = { f32: 0, f16: 1, int8: 2, int4: 3, bf16: 4 };
const NUMERICS = { fast: 0, exact: 1 };
const MATMUL = { batched: 0, matvec: 1, mfma: 2 };

class GpuContext {
  constructor(handle) { this.handle = handle; }
  static create(device) { return new GpuContext(addon.open(device === undefined ? 0 : device)); }
  describe() { return JSON.parse(addon.describe(this.handle)); }
  destroy() {
    if (this.handle) addon.close(this.handle);
    this.handle = null;
  }
}

class GpuKVCache {
  constructor(model, handle, capacity) {
    this.model = model;
    this.handle = handle;
    this.capacity = capacity;
  }
  get length() { return addon.cacheLength(this.handle); }
  set length(n) { addon.cacheLength(this.handle, n); }
  reset() { this.length = 0; }
  destroy() {
    if (this.handle) addon.cacheFree(this.handle);
    this.handle = null;
  }
}

// bf16 bits -> f32, exactly (src/core/dtype.js:43-48).
function bf16ToF32Array(bits) {
  const u = new Uint32Array(bits.length);
  for (let i = 0; i < bits.length; i++) u[i] = bits[i] << 16;
  return new Float32Array(u.buffer);
}

// f32 -> f16 bits, round to nearest even (src/core/dtype.js:81-113).
function f32ToF16Array(x) {
  const f = new Float32Array(1);
  const u = new Uint32Array(f.buffer);
  const out = new Uint16Array(x.length);
  for (let i = 0; i < x.length; i++) {
    f[0] = x[i];
    const b = u[0];
    const sign = (b >>> 16) & 0x8000;
    const exp = (b >>> 23) & 0xff;
    let mant = b & 0x7fffff;
    if (exp === 0xff) { out[i] = sign | 0x7c00 | (mant ? (mant >>> 13) | 0x200 : 0); continue; }
    let e = exp - 127 + 15;
    if (e >= 0x1f) { out[i] = sign | 0x7c00; continue; }
    if (e <= 0) {
      if (e < -10) { out[i] = sign; continue; }
      mant |= 0x800000;
      const shift = 14 - e;
      let h = mant >>> shift;
      const rem = mant & ((1 << shift) - 1), half = 1 << (shift - 1);
      if (rem > half || (rem === half && (h & 1))) h++;
      out[i] = sign | h;
      continue;
    }
    let h = (e << 10) | (mant >>> 13);
    const rem = mant & 0x1fff;
    if (rem > 0x1000 || (rem === 0x1000 && (h & 1))) h++;
    out[i] = sign | h;
  }
  return out;
}

function deviceMatrix(w32, rows, cols, scheme, group) {
  if (scheme === 'f16') return { format: FMT.f16, rows, cols, group: 0, data: f32ToF16Array(w32) };
  if (scheme === 'int8') {
    const r = addon.quantizeInt8(w32, rows, cols);
    return { format: FMT.int8, rows, cols, group: 0, data: r.q, scales: r.scales };
  }
  if (scheme === 'int4') {
    const r = addon.quantizeInt4(w32, rows, cols, group);
    return { format: FMT.int4, rows, cols, group, data: r.q, scales: r.scales, zeros: r.zeros };
  }
  throw new Error('unknown quantization scheme ' + scheme);
}

class GpuModel {
  constructor(ctx, handle, config, maxPositions) {
    this.ctx = ctx;
    this.handle = handle;
    this.config = config;
    this.maxPositions = maxPositions;
  }

  // tensors: a Safetensors checkpoint (./safetensors.js, src/gpu/model.js:147's `safetensors`), or
  // {name: {dtype: 'bf16'|'f32', shape: [...], data: Uint16Array|Float32Array}}. config: the
  // dimensions (parseConfig of config.json gives them). opts: maxPositions (2048), quantize {scheme:
  // 'int8'|'int4'|'f16', groupSize}, headScheme (the output projection's format, default the
  // layers'), matmul ('batched'|'matvec'|'mfma'), numerics ('fast'|'exact'), convert ('device':
  // each tensor uploaded in its checkpoint width and widened, quantized or narrowed by the
  // library's kernels; 'host': converted here first, as the reference's loader does; both store
  // the same bits).
  static load(ctx, tensors, config, opts) {
    opts = opts || {};
    const maxPositions = opts.maxPositions || 2048;
    const q = opts.quantize || { scheme: 'f16', groupSize: 128 };
    const group = q.groupSize || 128;
    const cfg = Object.assign({ headDim: config.hidden / config.heads, maxPositions: maxPositions }, config);
    const handle = addon.modelCreate(ctx.handle, cfg);
    const model = new GpuModel(ctx, handle, cfg, maxPositions);
    try {
      addon.modelSetMode(handle, 'numerics', NUMERICS[opts.numerics || 'fast']);
      addon.modelSetMode(handle, 'matmul', MATMUL[opts.matmul || 'batched']);
      // A checkpoint file (Safetensors) is checked against the config and read one tensor at
      // a time; a dict of tensors is taken as given.
      const file = typeof tensors.tensor === 'function' ? tensors : null;
      if (file) checkAgainst(cfg, file);
      const names = file ? Object.keys(expectedTensors(cfg)) : Object.keys(tensors);
      const tied = names.indexOf('lm_head.weight') < 0;
      const head = opts.headScheme || q.scheme;
      const onDevice = (opts.convert || 'device') === 'device';
      if (!onDevice && opts.convert !== 'host') throw new Error('convert must be "device" or "host"');
      names.forEach(function (name, i) {
        const t = file ? file.tensor(name) : tensors[name];
        if (t.dtype !== 'bf16' && t.dtype !== 'f32') throw new Error(name + ': dtype must be bf16 or f32');
        const embed = name === 'model.embed_tokens.weight';
        if (embed && t.dtype !== 'bf16') throw new Error(name + ': the gather table is bf16, got ' + t.dtype);
        const scheme = name === 'lm_head.weight' ? head : q.scheme;
        if (onDevice) {
          const src = t.dtype === 'bf16' ? FMT.bf16 : FMT.f32;
          const rows = t.shape[0], cols = t.shape.length === 1 ? 1 : t.shape[1];
          const load = function (as, fmt) {
            addon.modelLoadTensor(handle, as, src, rows, cols, t.data, fmt, fmt === FMT.int4 ? group : 0);
          };
          if (embed) {
            load(name, FMT.bf16);
            if (tied) load('lm_head.weight', FMT[head]);
          } else {
            load(name, t.shape.length === 1 ? FMT.f32 : FMT[scheme]);
          }
          if (opts.onProgress) opts.onProgress(i + 1, names.length, name);
          return;
        }
        const w32 = t.dtype === 'bf16' ? bf16ToF32Array(t.data) : t.data;
        if (embed) {
          addon.modelSetTensor(handle, name, FMT.bf16, t.shape[0], t.shape[1], 0, t.data, null, null);
          if (tied) {
            const m = deviceMatrix(w32, t.shape[0], t.shape[1], head, group);
            addon.modelSetTensor(handle, 'lm_head.weight', m.format, m.rows, m.cols, m.group, m.data,
                                 m.scales || null, m.zeros || null);
          }
        } else if (t.shape.length === 1) {
          addon.modelSetTensor(handle, name, FMT.f32, t.shape[0], 1, 0, w32, null, null);
        } else {
          const m = deviceMatrix(w32, t.shape[0], t.shape[1], scheme, group);
          addon.modelSetTensor(handle, name, m.format, m.rows, m.cols, m.group, m.data,
                               m.scales || null, m.zeros || null);
        }
        if (opts.onProgress) opts.onProgress(i + 1, names.length, name);
      });
      model.byteLength = addon.modelFinalize(handle);
    } catch (e) {
      addon.modelFree(handle);
      throw e;
    }
    return model;
  }

  newCache(capacity) { return new GpuKVCache(this, addon.cacheCreate(this.handle, capacity), capacity); }

  // forward(hidden: Float32Array[seq*hidden], seq, {cache, wantLogits}) (src/gpu/model.js:227-238)
  forward(hidden, seq, opts) {
    const want = !opts || opts.wantLogits !== false;
    return addon.forward(this.handle, opts.cache.handle, hidden, seq, want, this.config.vocab);
  }

  // The same from token ids (embedding gather on the device).
  forwardTokens(ids, cache, wantLogits) {
    const a = ids instanceof Int32Array ? ids : Int32Array.from(ids);
    return addon.forward(this.handle, cache.handle, a, a.length, wantLogits !== false, this.config.vocab);
  }

  // Greedy decode of `steps` tokens, every step on the device (hipGraph replay).
  decode(cache, firstToken, steps) { return addon.decode(this.handle, cache.handle, firstToken, steps); }

  setMatmul(mode) { addon.modelSetMode(this.handle, 'matmul', MATMUL[mode]); }

  destroy() {
    if (this.handle) addon.modelFree(this.handle);
    this.handle = null;
  }
}

// Seeded random-init checkpoint of the architecture (the tensor names of
// src/core/config.js:88-119; linear/embedding/bias ~ N(0, std), norm gains 1.0), drawn
// from the library's counter-based generator, stream per tensor name.
function synthesizeCheckpoint(config, seed, std) {
  std = std === undefined ? 0.02 : std;
  const shapes = expectedTensors(Object.assign({}, config, { tieWordEmbeddings: true }));
  const out = {};
  Object.keys(shapes).forEach(function (name) {
    const shape = shapes[name];
    const n = shape.reduce(function (a, b) { return a * b; }, 1);
    const data = /norm\.weight$/.test(name) ? new Uint16Array(n).fill(0x3f80) : addon.synthBf16(seed, name, std, n);
    out[name] = { dtype: 'bf16', shape: shape, data: data };
  });
  return out;
}

function synthTokens(seed, name, vocab, n) { return addon.synthTokens(seed, name, vocab, n); }

const QWEN25_05B = {
  hidden: 896, intermediate: 4864, layers: 24, heads: 14, kvHeads: 2, vocab: 151936,
  ropeTheta: 1e6, eps: 1e-6,
};

module.exports = {
  GpuContext, GpuModel, GpuKVCache, synthesizeCheckpoint, synthTokens, bf16ToF32Array, f32ToF16Array,
  QWEN25_05B, addon, Safetensors, parseConfig,
};
