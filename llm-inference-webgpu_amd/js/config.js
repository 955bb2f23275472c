'use strict';
// The model's dimensions from config.json, for the Node driver (Node 12, CommonJS).
//
// ModelConfig carries the property and method names of the reference's ModelConfig that
// its callers read (hiddenSize, intermediateSize, numLayers, numHeads, numKVHeads, vocabSize,
// ropeTheta, rmsNormEps, tieWordEmbeddings, headDim, kvDim, kvGroupSize; parse,
// expectedTensors, checkAgainst -- src/core/config.js), so an object built by either one
// drives GpuModel.load. Every field is checked and all problems are reported together; the
// checks and messages are this file's own.

// config.json fields: [property, key, kind]; a 'count' is a positive integer, a 'real' a
// positive finite number.
const FIELDS = [
  ['hiddenSize', 'hidden_size', 'count'], ['intermediateSize', 'intermediate_size', 'count'],
  ['numLayers', 'num_hidden_layers', 'count'], ['numHeads', 'num_attention_heads', 'count'],
  ['numKVHeads', 'num_key_value_heads', 'count'], ['vocabSize', 'vocab_size', 'count'],
  ['maxPositionEmbeddings', 'max_position_embeddings', 'count'], ['ropeTheta', 'rope_theta', 'real'],
  ['rmsNormEps', 'rms_norm_eps', 'real'],
];

// One decoder layer's tensors (checkpoint names) and their shapes in d = hidden,
// k = kv dim, f = intermediate.
const LAYER_TENSORS = [
  ['input_layernorm.weight', 'd'], ['post_attention_layernorm.weight', 'd'],
  ['self_attn.q_proj.weight', 'dd'], ['self_attn.q_proj.bias', 'd'],
  ['self_attn.k_proj.weight', 'kd'], ['self_attn.k_proj.bias', 'k'],
  ['self_attn.v_proj.weight', 'kd'], ['self_attn.v_proj.bias', 'k'],
  ['self_attn.o_proj.weight', 'dd'],
  ['mlp.gate_proj.weight', 'fd'], ['mlp.up_proj.weight', 'fd'], ['mlp.down_proj.weight', 'df'],
];

function fieldOk(v, kind) {
  if (typeof v !== 'number') return false;
  return kind === 'count' ? Number.isSafeInteger(v) && v > 0 : Number.isFinite(v) && v > 0;
}

function few(list) {
  return list.slice(0, 4).join(', ') + (list.length > 4 ? ', ... (' + (list.length - 4) + ' more)' : '');
}

class ModelConfig {
  constructor(raw) {
    if (raw === null || typeof raw !== 'object' || Array.isArray(raw)) {
      throw new Error('config.json holds a JSON ' + (raw === null ? 'null' : typeof raw) + ', not an object');
    }
    const problems = [];
    const self = this;
    FIELDS.forEach(function (f) {
      const v = raw[f[1]];
      if (fieldOk(v, f[2])) self[f[0]] = v;
      else problems.push(f[1] + ' = ' + JSON.stringify(v) + ' is not a ' +
                         (f[2] === 'count' ? 'positive integer' : 'positive finite number'));
    });
    this.modelType = raw.model_type;
    this.hiddenAct = raw.hidden_act === undefined ? 'silu' : raw.hidden_act;
    this.tieWordEmbeddings = raw.tie_word_embeddings === true;
    if (this.modelType !== 'qwen2') {
      problems.push('model_type ' + JSON.stringify(this.modelType) + ': only the qwen2 architecture is built here');
    }
    if (this.hiddenAct !== 'silu') problems.push('hidden_act ' + JSON.stringify(this.hiddenAct) + ': the MLP here is SiLU-gated');
    if (raw.use_sliding_window === true) problems.push('use_sliding_window: attention here always spans the whole context');
    if (this.hiddenSize && this.numHeads && this.hiddenSize % this.numHeads) {
      problems.push('hidden_size ' + this.hiddenSize + ' does not split into ' + this.numHeads + ' equal heads');
    }
    if (this.numHeads && this.numKVHeads && this.numHeads % this.numKVHeads) {
      problems.push(this.numHeads + ' query heads do not group evenly over ' + this.numKVHeads + ' key/value heads');
    }
    if (problems.length) throw new Error('config.json describes no model this engine runs: ' + problems.join('; '));
    this.headDim = this.hiddenSize / this.numHeads;
    this.kvDim = this.numKVHeads * this.headDim;
    this.kvGroupSize = this.numHeads / this.numKVHeads;
    Object.freeze(this);
  }

  static parse(text) { return new ModelConfig(JSON.parse(text)); }

  // Map of checkpoint name -> shape for every tensor the architecture needs (a tied model
  // has no lm_head.weight: the embedding is the output projection).
  expectedTensors() {
    const dims = { d: this.hiddenSize, k: this.kvDim, f: this.intermediateSize };
    const out = new Map([['model.embed_tokens.weight', [this.vocabSize, this.hiddenSize]],
                         ['model.norm.weight', [this.hiddenSize]]]);
    for (let i = 0; i < this.numLayers; i++) {
      LAYER_TENSORS.forEach(function (t) {
        out.set('model.layers.' + i + '.' + t[0], t[1].split('').map(function (c) { return dims[c]; }));
      });
    }
    if (!this.tieWordEmbeddings) out.set('lm_head.weight', [this.vocabSize, this.hiddenSize]);
    return out;
  }

  // Checks that a checkpoint (anything with names / has / info) holds exactly the tensors the
  // config implies, each with its shape; returns their number.
  checkAgainst(st) {
    const expected = this.expectedTensors();
    const missing = [], misshapen = [], surplus = [];
    expected.forEach(function (shape, name) {
      if (!st.has(name)) { missing.push(name); return; }
      const got = Array.from(st.info(name).shape);
      if (got.length !== shape.length || got.some(function (d, i) { return d !== shape[i]; })) {
        misshapen.push(name + ' is [' + got + '] where the config implies [' + shape + ']');
      }
    });
    st.names().forEach(function (name) { if (!expected.has(name)) surplus.push(name); });
    const parts = [];
    if (missing.length) parts.push(missing.length + ' missing (' + few(missing) + ')');
    if (misshapen.length) parts.push(misshapen.length + ' misshapen (' + few(misshapen) + ')');
    if (surplus.length) parts.push(surplus.length + ' not part of the model (' + few(surplus) + ')');
    if (parts.length) throw new Error('the checkpoint does not match the config: ' + parts.join('; '));
    return expected.size;
  }
}

// config.json as text or an already parsed object -> ModelConfig.
function parseConfig(raw) { return new ModelConfig(typeof raw === 'string' ? JSON.parse(raw) : raw); }

// The dimensions GpuModel needs from a ModelConfig (this file's or the reference's) or from a
// plain {hidden, intermediate, layers, heads, kvHeads, vocab, ropeTheta, eps} object.
function modelDims(c) {
  if (c.hiddenSize !== undefined) {
    return { hidden: c.hiddenSize, intermediate: c.intermediateSize, layers: c.numLayers, heads: c.numHeads,
             kvHeads: c.numKVHeads, vocab: c.vocabSize, ropeTheta: c.ropeTheta, eps: c.rmsNormEps,
             tieWordEmbeddings: c.tieWordEmbeddings !== false };
  }
  return { hidden: c.hidden, intermediate: c.intermediate, layers: c.layers, heads: c.heads, kvHeads: c.kvHeads,
           vocab: c.vocab, ropeTheta: c.ropeTheta === undefined ? 1e6 : c.ropeTheta,
           eps: c.eps === undefined ? 1e-6 : c.eps, tieWordEmbeddings: c.tieWordEmbeddings !== false };
}

// A ModelConfig-shaped view of plain dimensions (for expectedTensors of a synthesized model).
function configOf(dims) {
  return Object.create(ModelConfig.prototype, {
    hiddenSize: { value: dims.hidden }, intermediateSize: { value: dims.intermediate },
    numLayers: { value: dims.layers }, numHeads: { value: dims.heads }, numKVHeads: { value: dims.kvHeads },
    vocabSize: { value: dims.vocab }, kvDim: { value: dims.kvHeads * (dims.hidden / dims.heads) },
    tieWordEmbeddings: { value: dims.tieWordEmbeddings !== false },
  });
}

module.exports = { ModelConfig, parseConfig, modelDims, configOf };
