'use strict';
// GpuContext / GpuModel / GpuKVCache over libqwen_hip.so, with the method names, argument
// shapes and promises of the reference's src/gpu/device.js and src/gpu/model.js, so its
// callers (web/bench.html:62-134: ModelConfig.parse, Safetensors.open, GpuModel.load,
// newCache, forward, cache.keys / values) carry over. Written for Node 12 (CommonJS, no
// optional chaining or private fields). The addon only marshals arguments; this file holds
// the loader logic of GpuModel.load (src/gpu/model.js:147-207): tensors by checkpoint name,
// 2-D layer weights stored per the `quantize` option in the reference quantizer's layout,
// the tied embedding as the output projection.

const path = require('path');
const addon = require(path.join(__dirname, 'addon', 'qwen_napi.node'));
const { Safetensors } = require('./safetensors.js');
const { ModelConfig, parseConfig, modelDims, configOf } = require('./config.js');

const FMT = { f32: 0, f16: 1, int8: 2, int4: 3, bf16: 4 };
const NUMERICS = { fast: 0, exact: 1 };
// 'tiled' is the reference's non-bitwise prefill contraction (src/gpu/kernels.js:119-215);
// here that role is the MFMA contraction.
const MATMUL = { batched: 0, matvec: 1, mfma: 2, tiled: 2 };

function matmulMode(name) {
  if (!Object.prototype.hasOwnProperty.call(MATMUL, name)) {
    throw new Error("matmul must be 'batched', 'tiled', 'mfma' or 'matvec', got " + JSON.stringify(name));
  }
  return MATMUL[name];
}

class GpuContext {
  constructor(handle) { this.handle = handle; }
  static create(device) { return new GpuContext(addon.open(device === undefined ? 0 : device)); }
  describe() { return JSON.parse(addon.describe(this.handle)); }
  destroy() {
    if (this.handle) addon.close(this.handle);
    this.handle = null;
  }
}

// [kvHeads, length, headDim] rows -> position-major [length, kvHeads * headDim]: the layout of
// the reference's per-layer cache buffers (src/gpu/model.js:69-84, 336-338), which its forward()
// returns as `present` (src/gpu/model.js:388-395).
function positionMajor(headMajor, kvHeads, headDim) {
  const length = headMajor.length / (kvHeads * headDim);
  const kvDim = kvHeads * headDim;
  const out = new Float32Array(headMajor.length);
  for (let h = 0; h < kvHeads; h++) {
    for (let t = 0; t < length; t++) {
      const from = (h * length + t) * headDim;
      out.set(headMajor.subarray(from, from + headDim), t * kvDim + h * headDim);
    }
  }
  return out;
}

// One layer's keys or values of a cache, standing where the reference keeps a GPUBuffer per
// layer (src/gpu/model.js:69-84). The device memory belongs to the cache; read() returns the
// rows 0 .. length-1 as the reference's buffer holds them, f32 position-major
// [length, kvHeads * headDim], and once every layer view of the cache is destroyed, the cache's
// memory is freed.
class LayerBuffer {
  constructor(cache, layer, kind, byteLength) {
    this.cache = cache;
    this.layer = layer;
    this.kind = kind;
    this.size = byteLength;
    this.destroyed = false;
  }
  read() { return this.cache.layerRows(this.layer)[this.kind]; }
  destroy() {
    if (this.destroyed) return;
    this.destroyed = true;
    this.cache.release();
  }
}

class GpuKVCache {
  constructor(model, handle, capacity) {
    const c = model.dims;
    this.model = model;
    this.handle = handle;
    this.capacity = capacity;
    // f16 keys [kv_heads][capacity][head_dim] and values [kv_heads][head_dim][capacity rounded to 64]
    const headDim = c.hidden / c.heads;
    const perLayer = c.kvHeads * headDim * 2 * (capacity + Math.ceil(capacity / 64) * 64);
    this.byteLength = perLayer * c.layers;
    this.keys = [];
    this.values = [];
    for (let i = 0; i < c.layers; i++) {
      this.keys.push(new LayerBuffer(this, i, 'key', c.kvHeads * headDim * 2 * capacity));
      this.values.push(new LayerBuffer(this, i, 'value', perLayer - c.kvHeads * headDim * 2 * capacity));
    }
    this.live = 2 * c.layers;
  }
  get length() { return addon.cacheLength(this.handle); }
  set length(n) { addon.cacheLength(this.handle, n); }
  reset() { this.length = 0; }
  // {key, value} of one layer, f32 [kv_heads, length, head_dim]: what the CPU cache's present()
  // returns (src/cpu/cache.js:97-115), the ONNX `present` layout.
  present(layer) { return addon.cachePresent(this.model.handle, this.handle, layer); }
  // {key, value} of one layer, f32 position-major [length, kv_heads * head_dim]: the reference
  // GPU cache's rows (src/gpu/model.js:388-395).
  layerRows(layer) {
    const p = this.present(layer);
    const kvHeads = this.model.dims.kvHeads, headDim = this.model.dims.hidden / this.model.dims.heads;
    return { key: positionMajor(p.key, kvHeads, headDim), value: positionMajor(p.value, kvHeads, headDim) };
  }
  release() {
    if (--this.live === 0) this.destroy();
  }
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

// One tensor of a checkpoint as {dtype: 'bf16'|'f32', shape, data}. A checkpoint is a
// Safetensors-like object (info(name) -> {dtype, shape}; readRaw(name) -> the stored bytes or
// a promise of them, as the reference's reader returns them) or a plain map of such tensors.
async function readTensor(source, name) {
  if (typeof source.info !== 'function') return source[name];
  if (typeof source.tensor === 'function') return source.tensor(name);  // this package's reader
  const info = source.info(name);
  const raw = await source.readRaw(name);
  const bytes = raw.byteOffset % 4 === 0 ? raw : new Uint8Array(raw);   // copied when misaligned
  const n = info.shape.reduce(function (a, b) { return a * b; }, 1);
  if (info.dtype === 'BF16') return { dtype: 'bf16', shape: info.shape, data: new Uint16Array(bytes.buffer, bytes.byteOffset, n) };
  if (info.dtype === 'F32') return { dtype: 'f32', shape: info.shape, data: new Float32Array(bytes.buffer, bytes.byteOffset, n) };
  if (typeof source.readF32 === 'function') return { dtype: 'f32', shape: info.shape, data: await source.readF32(name) };
  throw new Error(name + ': the loader reads BF16 and F32 tensors, not ' + info.dtype);
}

class GpuModel {
  constructor(ctx, handle, config, dims, maxPositions) {
    this.ctx = ctx;
    this.handle = handle;
    this.config = config;
    this.dims = dims;
    this.maxPositions = maxPositions;
    this.running = false;
  }

  // Positions one weight tile of the batched matvec serves (src/gpu/model.js:133-138); every
  // choice sums each output in the same order, so results do not depend on it.
  static batchTileFor(seq) {
    if (seq >= 8) return 8;
    if (seq >= 4) return 4;
    if (seq >= 2) return 2;
    return 1;
  }

  // load(ctx, safetensors, config, opts) -> Promise<GpuModel> (src/gpu/model.js:147-207).
  //   safetensors: a checkpoint reader (this package's Safetensors or the reference's: info,
  //     readRaw[, readF32]) -- checked against the config first -- or a map of tensors.
  //   config: a ModelConfig (this package's or the reference's) or plain dimensions.
  //   opts: maxPositions (2048), onProgress(done, total, name), quantize (null: f16 weights,
  //     the reference's format; or {scheme: 'int8'|'int4'|'f16', groupSize}), matmul
  //     ('batched' | 'tiled' | 'matvec'; 'mfma' = 'tiled'), and this backend's numerics
  //     ('fast' | 'exact'), headScheme (the output projection's format, default the layers'),
  //     convert ('device': each tensor uploaded in its checkpoint width and converted by the
  //     library's kernels; 'host': converted here first; both store the same bits).
  static async load(ctx, safetensors, config, opts) {
    opts = opts || {};
    const maxPositions = opts.maxPositions || 2048;
    const q = opts.quantize || { scheme: 'f16', groupSize: 128 };
    const group = q.groupSize || 128;
    const dims = modelDims(config);
    const cfg = Object.assign({ headDim: dims.hidden / dims.heads, maxPositions: maxPositions }, dims);
    const matmul = matmulMode(opts.matmul || 'batched');
    const onDevice = (opts.convert || 'device') === 'device';
    if (!onDevice && opts.convert !== 'host') throw new Error('convert must be "device" or "host"');
    const file = typeof safetensors.info === 'function';
    const expected = configOf(dims).expectedTensors();
    if (file) configOf(dims).checkAgainst(safetensors);
    const names = file ? Array.from(expected.keys()) : Object.keys(safetensors);
    const tied = names.indexOf('lm_head.weight') < 0;
    const head = opts.headScheme || q.scheme;
    const handle = addon.modelCreate(ctx.handle, cfg);
    const model = new GpuModel(ctx, handle, config, dims, maxPositions);
    try {
      addon.modelSetMode(handle, 'numerics', NUMERICS[opts.numerics || 'fast']);
      addon.modelSetMode(handle, 'matmul', matmul);
      for (let i = 0; i < names.length; i++) {
        const name = names[i];
        const t = await readTensor(safetensors, name);
        if (t.dtype !== 'bf16' && t.dtype !== 'f32') throw new Error(name + ': dtype must be bf16 or f32');
        const embed = name === 'model.embed_tokens.weight';
        if (embed && t.dtype !== 'bf16') throw new Error(name + ': the gather table is bf16, got ' + t.dtype);
        const scheme = name === 'lm_head.weight' ? head : q.scheme;
        const rows = t.shape[0], cols = t.shape.length === 1 ? 1 : t.shape[1];
        if (onDevice) {
          const src = t.dtype === 'bf16' ? FMT.bf16 : FMT.f32;
          const load = function (as, fmt) {
            addon.modelLoadTensor(handle, as, src, rows, cols, t.data, fmt, fmt === FMT.int4 ? group : 0);
          };
          if (embed) {
            load(name, FMT.bf16);
            if (tied) load('lm_head.weight', FMT[head]);
          } else {
            load(name, t.shape.length === 1 ? FMT.f32 : FMT[scheme]);
          }
        } else {
          const w32 = t.dtype === 'bf16' ? bf16ToF32Array(t.data) : t.data;
          if (embed) {
            addon.modelSetTensor(handle, name, FMT.bf16, rows, cols, 0, t.data, null, null);
            if (tied) {
              const m = deviceMatrix(w32, rows, cols, head, group);
              addon.modelSetTensor(handle, 'lm_head.weight', m.format, m.rows, m.cols, m.group, m.data,
                                   m.scales || null, m.zeros || null);
            }
          } else if (t.shape.length === 1) {
            addon.modelSetTensor(handle, name, FMT.f32, rows, 1, 0, w32, null, null);
          } else {
            const m = deviceMatrix(w32, rows, cols, scheme, group);
            addon.modelSetTensor(handle, name, m.format, m.rows, m.cols, m.group, m.data,
                                 m.scales || null, m.zeros || null);
          }
        }
        if (opts.onProgress) opts.onProgress(i + 1, names.length, name);
      }
      model.byteLength = addon.modelFinalize(handle);
    } catch (e) {
      addon.modelFree(handle);
      throw e;
    }
    return model;
  }

  newCache(capacity) { return new GpuKVCache(this, addon.cacheCreate(this.handle, capacity), capacity); }

  // forward(hidden: Float32Array[seq*hidden], seq, {cache, wantLogits = true, wantPresent = false})
  //   -> Promise<{logits, present, hiddenBuffer}> (src/gpu/model.js:227-240, 401). present: per
  //   layer {key, value} f32 position-major [length, kv_heads * head_dim] after the pass, as the
  //   reference reads its cache buffers (src/gpu/model.js:388-395; its caller reshapes them,
  //   web/model.html:49-60); hiddenBuffer is null (the residual rows stay in the library's
  //   workspace). One pass at a time.
  async forward(hidden, seq, options) {
    if (this.running) throw new Error('forward() is already running; await it first');
    const o = options || {};
    this.running = true;
    try {
      await null;  // the pass runs after the caller's current turn, as a queued GPU pass does
      const want = o.wantLogits !== false;
      const r = addon.forward(this.handle, o.cache.handle, hidden, seq, want);
      let present = null;
      if (o.wantPresent) {
        present = [];
        for (let L = 0; L < this.dims.layers; L++) present.push(o.cache.layerRows(L));
      }
      return { logits: r.logits, present: present, hiddenBuffer: null, argmax: r.argmax };
    } finally {
      this.running = false;
    }
  }

  // The same from token ids, synchronously (embedding gather on the device): {logits, argmax}.
  forwardTokens(ids, cache, wantLogits) {
    const a = ids instanceof Int32Array ? ids : Int32Array.from(ids);
    return addon.forward(this.handle, cache.handle, a, a.length, wantLogits !== false);
  }

  // Greedy decode of `steps` tokens, every step on the device (hipGraph replay).
  decode(cache, firstToken, steps) { return addon.decode(this.handle, cache.handle, firstToken, steps); }

  // The negative log-likelihood of ids[t + 1] given ids[0..t], for every t, scored one token at
  // a time through `cache` as web/perplexity.html:146-170 does (the log-softmax on the device, in
  // f64): a Float64Array of ids.length - 1; perplexity is exp of its mean.
  score(ids, cache) {
    const a = ids instanceof Int32Array ? ids : Int32Array.from(ids);
    return addon.score(this.handle, cache.handle, a);
  }

  setMatmul(mode) { addon.modelSetMode(this.handle, 'matmul', matmulMode(mode)); }

  destroy() {
    if (this.handle) addon.modelFree(this.handle);
    this.handle = null;
  }
}

// Seeded random-init checkpoint of the architecture (the checkpoint tensor names;
// linear/embedding/bias ~ N(0, std), norm gains 1.0), drawn from the library's counter-based
// generator, stream per tensor name.
function synthesizeCheckpoint(config, seed, std) {
  std = std === undefined ? 0.02 : std;
  const dims = Object.assign({}, modelDims(config), { tieWordEmbeddings: true });
  const out = {};
  configOf(dims).expectedTensors().forEach(function (shape, name) {
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
  QWEN25_05B, addon, Safetensors, ModelConfig, parseConfig,
};
