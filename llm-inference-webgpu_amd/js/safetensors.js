'use strict';
// Checkpoint files for the loader, for Node 12 (CommonJS, synchronous reads): a safetensors
// reader with the validation of the reference's Safetensors.open (src/core/safetensors.js:56-125)
// and the config checks of src/core/config.js:16-153. Tensors are read one at a time, as the
// reference's loader reads them, and handed on as stored (bf16 bits, f16 bits or f32).

const fs = require('fs');
const util = require('util');

// Bytes per element of every dtype safetensors defines (safetensors.js:15-21).
const DTYPE_SIZE = {
  BOOL: 1, U8: 1, I8: 1, F8_E4M3: 1, F8_E5M2: 1,
  I16: 2, U16: 2, F16: 2, BF16: 2,
  I32: 4, U32: 4, F32: 4,
  I64: 8, U64: 8, F64: 8,
};

function isInt(v) { return Number.isSafeInteger(v); }

class Safetensors {
  constructor(fd, tensors, dataStart, metadata) {
    this.fd = fd;
    this.tensors = tensors;
    this.dataStart = dataStart;
    this.metadata = metadata;
  }

  static open(path) {
    const fd = fs.openSync(path, 'r');
    try {
      const size = fs.fstatSync(fd).size;
      if (size < 8) throw new Error('not a safetensors file: ' + size + ' bytes');
      const lenBuf = Buffer.alloc(8);
      fs.readSync(fd, lenBuf, 0, 8, 0);
      const headerLen = Number(lenBuf.readBigUInt64LE(0));
      if (!isInt(headerLen) || headerLen <= 0 || 8 + headerLen > size) {
        throw new Error('header length ' + headerLen + ' does not fit in a ' + size + '-byte file');
      }
      const headerBuf = Buffer.alloc(headerLen);
      fs.readSync(fd, headerBuf, 0, headerLen, 8);
      let header;
      try {
        header = JSON.parse(new util.TextDecoder('utf-8', { fatal: true }).decode(headerBuf));
      } catch (e) {
        throw new Error('header is not valid UTF-8 JSON: ' + e.message);
      }
      if (header === null || typeof header !== 'object' || Array.isArray(header)) {
        throw new Error('header must be a JSON object');
      }
      const metadata = header.__metadata__ === undefined ? null : header.__metadata__;
      delete header.__metadata__;
      const dataStart = 8 + headerLen;
      const dataSize = size - dataStart;
      const tensors = new Map();
      Object.keys(header).forEach(function (name) {
        const e = header[name] || {};
        const el = DTYPE_SIZE[e.dtype];
        if (el === undefined) throw new Error(name + ': unknown dtype ' + JSON.stringify(e.dtype));
        if (!Array.isArray(e.shape) || !e.shape.every(function (d) { return isInt(d) && d >= 0; })) {
          throw new Error(name + ': shape must be an array of non-negative integers');
        }
        if (!Array.isArray(e.data_offsets) || e.data_offsets.length !== 2) {
          throw new Error(name + ': data_offsets must be a pair');
        }
        const begin = e.data_offsets[0], end = e.data_offsets[1];
        if (!isInt(begin) || !isInt(end) || begin < 0 || end < begin) {
          throw new Error(name + ': bad data_offsets [' + begin + ', ' + end + ']');
        }
        if (end > dataSize) throw new Error(name + ': ends at ' + end + ' but the data section is only ' + dataSize + ' bytes');
        const numel = e.shape.reduce(function (a, b) { return a * b; }, 1);
        if (end - begin !== numel * el) {
          throw new Error(name + ': shape [' + e.shape + '] of ' + e.dtype + ' needs ' + numel * el +
                          ' bytes but the header reserves ' + (end - begin));
        }
        tensors.set(name, { name: name, dtype: e.dtype, shape: e.shape.slice(), begin: begin, end: end, numel: numel });
      });
      const ranges = Array.from(tensors.values()).sort(function (a, b) { return a.begin - b.begin; });
      for (let i = 1; i < ranges.length; i++) {
        if (ranges[i].begin < ranges[i - 1].end) throw new Error(ranges[i].name + ' overlaps ' + ranges[i - 1].name);
      }
      return new Safetensors(fd, tensors, dataStart, metadata);
    } catch (e) {
      fs.closeSync(fd);
      throw e;
    }
  }

  get size() { return this.tensors.size; }
  names() { return Array.from(this.tensors.keys()); }
  has(name) { return this.tensors.has(name); }
  info(name) {
    const t = this.tensors.get(name);
    if (!t) throw new Error('no tensor named ' + JSON.stringify(name));
    return t;
  }

  // The tensor's bytes exactly as stored, in a fresh (so aligned) buffer.
  readRaw(name) {
    const t = this.info(name);
    const buf = Buffer.alloc(t.end - t.begin);
    let done = 0;
    while (done < buf.length) {
      const n = fs.readSync(this.fd, buf, done, buf.length - done, this.dataStart + t.begin + done);
      if (n <= 0) throw new Error(name + ': short read');
      done += n;
    }
    return buf;
  }

  // {dtype: 'bf16'|'f32', shape, data}: bf16 as its bits, f32 as is, f16 widened exactly to f32.
  tensor(name) {
    const t = this.info(name);
    const raw = this.readRaw(name);
    const ab = raw.buffer.slice(raw.byteOffset, raw.byteOffset + raw.length);
    if (t.dtype === 'BF16') return { dtype: 'bf16', shape: t.shape, data: new Uint16Array(ab) };
    if (t.dtype === 'F32') return { dtype: 'f32', shape: t.shape, data: new Float32Array(ab) };
    if (t.dtype === 'F16') {
      const h = new Uint16Array(ab), out = new Float32Array(h.length);
      for (let i = 0; i < h.length; i++) out[i] = f16ToF32(h[i]);
      return { dtype: 'f32', shape: t.shape, data: out };
    }
    throw new Error(name + ': dtype ' + t.dtype + ' is not a weight format the loader reads');
  }

  close() {
    if (this.fd !== null) fs.closeSync(this.fd);
    this.fd = null;
  }
}

// f16 bits -> f32, exactly (src/core/dtype.js:58-77).
function f16ToF32(h) {
  const sign = h & 0x8000 ? -1 : 1;
  const exp = (h >>> 10) & 0x1f, mant = h & 0x3ff;
  if (exp === 0) return sign * mant * Math.pow(2, -24);
  if (exp === 0x1f) return mant ? NaN : sign * Infinity;
  return sign * (1 + mant / 1024) * Math.pow(2, exp - 15);
}

const REQUIRED = ['hidden_size', 'intermediate_size', 'num_hidden_layers', 'num_attention_heads',
  'num_key_value_heads', 'vocab_size', 'max_position_embeddings', 'rope_theta', 'rms_norm_eps'];

// config.json (text or object) -> the loader's config (src/core/config.js:16-80).
function parseConfig(raw) {
  if (typeof raw === 'string') raw = JSON.parse(raw);
  REQUIRED.forEach(function (key) {
    if (typeof raw[key] !== 'number' || !Number.isFinite(raw[key])) {
      throw new Error('config: ' + key + ' must be a finite number, got ' + JSON.stringify(raw[key]));
    }
  });
  if (raw.model_type !== 'qwen2') throw new Error('config: only qwen2 is implemented, got ' + JSON.stringify(raw.model_type));
  const act = raw.hidden_act === undefined ? 'silu' : raw.hidden_act;
  if (act !== 'silu') throw new Error('config: only the silu/SwiGLU MLP is implemented, got ' + act);
  if (raw.use_sliding_window === true) throw new Error('config: sliding-window attention is not implemented');
  if (raw.hidden_size % raw.num_attention_heads !== 0) {
    throw new Error('config: hidden_size ' + raw.hidden_size + ' is not divisible by num_attention_heads ' +
                    raw.num_attention_heads);
  }
  if (raw.num_attention_heads % raw.num_key_value_heads !== 0) {
    throw new Error('config: num_attention_heads ' + raw.num_attention_heads +
                    ' is not divisible by num_key_value_heads ' + raw.num_key_value_heads);
  }
  return {
    hidden: raw.hidden_size, intermediate: raw.intermediate_size, layers: raw.num_hidden_layers,
    heads: raw.num_attention_heads, kvHeads: raw.num_key_value_heads, vocab: raw.vocab_size,
    ropeTheta: raw.rope_theta, eps: raw.rms_norm_eps, tieWordEmbeddings: raw.tie_word_embeddings === true,
  };
}

// Every tensor the architecture requires, with its shape (config.js:89-121).
function expectedTensors(config) {
  const d = config.hidden, kv = config.kvHeads * (config.hidden / config.heads), f = config.intermediate;
  const shapes = { 'model.embed_tokens.weight': [config.vocab, d], 'model.norm.weight': [d] };
  for (let i = 0; i < config.layers; i++) {
    const p = 'model.layers.' + i + '.';
    shapes[p + 'input_layernorm.weight'] = [d];
    shapes[p + 'post_attention_layernorm.weight'] = [d];
    shapes[p + 'self_attn.q_proj.weight'] = [d, d];
    shapes[p + 'self_attn.q_proj.bias'] = [d];
    shapes[p + 'self_attn.k_proj.weight'] = [kv, d];
    shapes[p + 'self_attn.k_proj.bias'] = [kv];
    shapes[p + 'self_attn.v_proj.weight'] = [kv, d];
    shapes[p + 'self_attn.v_proj.bias'] = [kv];
    shapes[p + 'self_attn.o_proj.weight'] = [d, d];
    shapes[p + 'mlp.gate_proj.weight'] = [f, d];
    shapes[p + 'mlp.up_proj.weight'] = [f, d];
    shapes[p + 'mlp.down_proj.weight'] = [d, f];
  }
  if (config.tieWordEmbeddings === false) shapes['lm_head.weight'] = [config.vocab, d];
  return shapes;
}

// checkAgainst (config.js:128-153): exactly the implied tensors, each with its shape.
function checkAgainst(config, st) {
  const expected = expectedTensors(config);
  const problems = [];
  Object.keys(expected).forEach(function (name) {
    if (!st.has(name)) { problems.push('missing ' + name); return; }
    const got = st.info(name).shape, want = expected[name];
    if (got.length !== want.length || got.some(function (d, i) { return d !== want[i]; })) {
      problems.push(name + ': expected shape [' + want + '], file has [' + got + ']');
    }
  });
  st.names().forEach(function (name) { if (!(name in expected)) problems.push('unexpected tensor ' + name); });
  if (problems.length) {
    throw new Error('weights do not match config (' + problems.length + ' problem' + (problems.length === 1 ? '' : 's') +
                    '):\n  ' + problems.slice(0, 10).join('\n  ') +
                    (problems.length > 10 ? '\n  ... and ' + (problems.length - 10) + ' more' : ''));
  }
  return Object.keys(expected).length;
}

module.exports = { Safetensors, parseConfig, expectedTensors, checkAgainst, f16ToF32, DTYPE_SIZE };
