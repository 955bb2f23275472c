'use strict';
// Safetensors checkpoints for the Node driver (Node 12: CommonJS, synchronous file reads).
//
// The container, as the safetensors format defines it: an unsigned 64-bit little-endian
// byte count N, N bytes of UTF-8 JSON, then one byte buffer. The JSON object maps each
// tensor name to {dtype, shape, data_offsets: [start, stop]} with the offsets counted from
// the start of the buffer, and may carry "__metadata__" (an object of strings).
//
// Safetensors.open checks the whole header before anything is read and reports every
// defect it finds in one error. The reader offers the methods the reference's callers use
// (names / has / info / readRaw / readRawRange / readF32, src/core/safetensors.js); they
// return their results directly, which `await` accepts as it accepts the reference's
// promises. The checks and messages are this file's own.

const fs = require('fs');
const util = require('util');

// Bytes per element of each element type of the format.
const ELEMENT_BYTES = {
  BOOL: 1, U8: 1, I8: 1, F8_E4M3: 1, F8_E5M2: 1,
  I16: 2, U16: 2, F16: 2, BF16: 2,
  I32: 4, U32: 4, F32: 4,
  I64: 8, U64: 8, F64: 8,
};
const HEADER_LIMIT = 100 * 1024 * 1024;  // headers beyond this are refused outright

function isCount(v) { return typeof v === 'number' && Number.isSafeInteger(v) && v >= 0; }
function typeName(v) { return v === null ? 'null' : Array.isArray(v) ? 'array' : typeof v; }

// {info, defects} for one header record; info is null when the record is unusable.
function checkRecord(name, rec, bufferBytes) {
  if (rec === null || typeof rec !== 'object' || Array.isArray(rec)) {
    return { info: null, defects: ["'" + name + "': the record is a JSON " + typeName(rec) + ', not an object'] };
  }
  const defects = [];
  const dtype = rec.dtype, shape = rec.shape, span = rec.data_offsets;
  if (!Object.prototype.hasOwnProperty.call(ELEMENT_BYTES, dtype)) {
    defects.push("'" + name + "': " + JSON.stringify(dtype) + ' is not a safetensors element type');
  }
  if (!Array.isArray(shape) || !shape.every(isCount)) {
    defects.push("'" + name + "': dimensions " + JSON.stringify(shape) + ' are not a list of non-negative integers');
  }
  if (!Array.isArray(span) || span.length !== 2 || !span.every(isCount) || span[0] > span[1]) {
    defects.push("'" + name + "': data_offsets " + JSON.stringify(span) + ' is not [start, stop] with 0 <= start <= stop');
  }
  if (defects.length) return { info: null, defects: defects };
  const numel = shape.reduce(function (a, b) { return a * b; }, 1);
  const info = { name: name, dtype: dtype, shape: shape.slice(), begin: span[0], end: span[1], numel: numel,
                 byteLength: span[1] - span[0] };
  if (info.end > bufferBytes) {
    return { info: null, defects: ["'" + name + "': bytes [" + info.begin + ', ' + info.end + ') extend past the ' +
                                   bufferBytes + '-byte buffer'] };
  }
  const need = numel * ELEMENT_BYTES[dtype];
  if (info.byteLength !== need) {
    return { info: null, defects: ["'" + name + "': " + numel + ' x ' + dtype + ' is ' + need +
                                   ' bytes, the record spans ' + info.byteLength] };
  }
  return { info: info, defects: [] };
}

// f16 bits -> the f32 value (exact).
function f16ToF32(h) {
  const sign = h & 0x8000 ? -1 : 1;
  const e = (h >>> 10) & 0x1f, m = h & 0x3ff;
  if (e === 0x1f) return m ? NaN : sign * Infinity;
  return e === 0 ? sign * m * Math.pow(2, -24) : sign * (1024 + m) * Math.pow(2, e - 25);
}

class Safetensors {
  constructor(path, fd, records, bufferStart, metadata) {
    this.path = path;
    this.fd = fd;
    this.records = records;        // Map name -> info
    this.bufferStart = bufferStart;
    this.metadata = metadata;
  }

  static open(path) {
    const where = require('path').basename(path);
    const fd = fs.openSync(path, 'r');
    try {
      const fileBytes = fs.fstatSync(fd).size;
      if (fileBytes < 8) throw new Error(where + ': ' + fileBytes + ' bytes is too short for a safetensors length prefix');
      const prefix = Buffer.alloc(8);
      fs.readSync(fd, prefix, 0, 8, 0);
      const n = Number(prefix.readBigUInt64LE(0));
      if (n === 0 || n > Math.min(fileBytes - 8, HEADER_LIMIT)) {
        throw new Error(where + ': the length prefix declares a ' + n + '-byte header, but ' + (fileBytes - 8) +
                        ' bytes follow it (and headers are limited to ' + HEADER_LIMIT + ' bytes)');
      }
      const text = Buffer.alloc(n);
      fs.readSync(fd, text, 0, n, 8);
      let header;
      try {
        header = JSON.parse(new util.TextDecoder('utf-8', { fatal: true }).decode(text));
      } catch (e) {
        throw new Error(where + ': the header is not UTF-8 JSON (' + e.message + ')');
      }
      if (header === null || typeof header !== 'object' || Array.isArray(header)) {
        throw new Error(where + ': the header is a JSON ' + typeName(header) + ', not an object of tensor records');
      }
      const bufferStart = 8 + n, bufferBytes = fileBytes - bufferStart;
      const defects = [];
      let metadata = null;
      if (Object.prototype.hasOwnProperty.call(header, '__metadata__')) {
        metadata = header.__metadata__;
        const ok = metadata !== null && typeof metadata === 'object' && !Array.isArray(metadata) &&
                   Object.keys(metadata).every(function (k) { return typeof metadata[k] === 'string'; });
        if (!ok) defects.push('__metadata__ is not an object of strings');
        delete header.__metadata__;
      }
      const records = new Map();
      Object.keys(header).forEach(function (name) {
        const r = checkRecord(name, header[name], bufferBytes);
        Array.prototype.push.apply(defects, r.defects);
        if (r.info) records.set(name, r.info);
      });
      // Two records must never claim the same byte.
      const byStart = Array.from(records.values()).filter(function (r) { return r.byteLength > 0; })
        .sort(function (a, b) { return a.begin - b.begin || a.end - b.end; });
      for (let i = 1; i < byStart.length; i++) {
        const a = byStart[i - 1], b = byStart[i];
        if (b.begin < a.end) {
          defects.push("'" + b.name + "' [" + b.begin + ', ' + b.end + ") overlaps '" + a.name + "' [" + a.begin + ', ' +
                       a.end + ')');
        }
      }
      if (defects.length) {
        throw new Error(where + ': ' + defects.length + ' defect' + (defects.length > 1 ? 's' : '') + ' in the header: ' +
                        defects.join('; '));
      }
      return new Safetensors(path, fd, records, bufferStart, metadata);
    } catch (e) {
      fs.closeSync(fd);
      throw e;
    }
  }

  get size() { return this.records.size; }
  names() { return Array.from(this.records.keys()); }
  has(name) { return this.records.has(name); }
  info(name) {
    const t = this.records.get(name);
    if (!t) throw new Error(require('path').basename(this.path) + ' holds no tensor ' + JSON.stringify(name));
    return t;
  }

  // `length` bytes of a tensor from `offset` within it, into a fresh (so aligned) buffer.
  readRawRange(name, offset, length) {
    const t = this.info(name);
    if (!isCount(offset) || !isCount(length) || offset + length > t.byteLength) {
      throw new RangeError(name + ': bytes ' + offset + '..' + (offset + length) + ' lie outside its ' + t.byteLength +
                           ' bytes');
    }
    const buf = Buffer.alloc(length);
    for (let done = 0; done < length;) {
      const got = fs.readSync(this.fd, buf, done, length - done, this.bufferStart + t.begin + offset + done);
      if (got <= 0) throw new Error(name + ': the file ended ' + (length - done) + ' bytes early');
      done += got;
    }
    return buf;
  }

  // The tensor's bytes as stored.
  readRaw(name) { return this.readRawRange(name, 0, this.info(name).byteLength); }

  // The tensor widened exactly to f32 (BF16, F16 or F32 storage); into `out` when given.
  readF32(name, out) {
    const t = this.info(name);
    const raw = this.readRaw(name);
    const ab = raw.buffer.slice(raw.byteOffset, raw.byteOffset + raw.length);
    const dst = out || new Float32Array(t.numel);
    if (dst.length < t.numel) throw new RangeError(name + ': ' + t.numel + ' values do not fit ' + dst.length);
    if (t.dtype === 'F32') {
      dst.set(new Float32Array(ab));
    } else if (t.dtype === 'BF16') {
      const h = new Uint16Array(ab), u = new Uint32Array(dst.buffer, dst.byteOffset, t.numel);
      for (let i = 0; i < h.length; i++) u[i] = h[i] << 16;
    } else if (t.dtype === 'F16') {
      const h = new Uint16Array(ab);
      for (let i = 0; i < h.length; i++) dst[i] = f16ToF32(h[i]);
    } else {
      throw new Error(name + ': the loader reads BF16, F16 and F32 tensors, not ' + t.dtype);
    }
    return dst;
  }

  // {dtype: 'bf16'|'f32', shape, data} as the loader uploads it: BF16 as its bits (the device
  // widens it), F32 as is, F16 widened here.
  tensor(name) {
    const t = this.info(name);
    if (t.dtype === 'BF16') {
      const raw = this.readRaw(name);
      return { dtype: 'bf16', shape: t.shape, data: new Uint16Array(raw.buffer.slice(raw.byteOffset, raw.byteOffset + raw.length)) };
    }
    return { dtype: 'f32', shape: t.shape, data: this.readF32(name) };
  }

  close() {
    if (this.fd !== null) fs.closeSync(this.fd);
    this.fd = null;
  }
}

module.exports = { Safetensors, ELEMENT_BYTES, f16ToF32 };
