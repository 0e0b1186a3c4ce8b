"use strict";
// GGUF model files for the Node.js host.
//
// A GGUF file is: magic "GGUF", version, tensor count, metadata count, the metadata (key, typed
// value), the tensor directory (name, dims, GGML type, offset into the data section) and the data
// section, aligned to general.alignment (32 by default).  parseGGUF returns the object the engine's
// backends consume (h2-own-inference-engine/engine/gguf.js:15-69): {version, meta, tensors, dataStart}
// with tensors[name] = {name, shape, type, offset, count, start, bytes}, shape[0] being the row
// length and start the absolute byte offset of the tensor's data.  qwen2Config reads the model's
// hyperparameters (gguf.js:72-88).  readModel(path) stands in for the browser download.
//
// The reader is a cursor over the file's bytes that checks every read against the end of the file,
// so a truncated or corrupt file fails with a message instead of reading garbage.

const fs = require("fs");

const TYPE = Object.freeze({ F32: 0, F16: 1, Q4_0: 2, Q8_0: 8 });

// GGML storage of the supported types: values per block, bytes per block.
const STORAGE = new Map([
  [TYPE.F32, { values: 1, bytes: 4 }],
  [TYPE.F16, { values: 1, bytes: 2 }],
  [TYPE.Q4_0, { values: 32, bytes: 18 }],
  [TYPE.Q8_0, { values: 32, bytes: 34 }],
]);

function tensorBytes(type, count) {
  const s = STORAGE.get(type);
  if (s === undefined) throw new Error(`unsupported tensor type ${type}`);
  if (count % s.values !== 0) throw new Error(`a tensor of type ${type} needs a multiple of ${s.values} values, not ${count}`);
  return (count / s.values) * s.bytes;
}

// Metadata value types of GGUF v2/v3.  Fixed-size ones: byte size and DataView read.
const V_STRING = 8, V_ARRAY = 9;
const FIXED = {
  0: [1, (d, o) => d.getUint8(o)],
  1: [1, (d, o) => d.getInt8(o)],
  2: [2, (d, o) => d.getUint16(o, true)],
  3: [2, (d, o) => d.getInt16(o, true)],
  4: [4, (d, o) => d.getUint32(o, true)],
  5: [4, (d, o) => d.getInt32(o, true)],
  6: [4, (d, o) => d.getFloat32(o, true)],
  7: [1, (d, o) => d.getUint8(o) !== 0],
  10: [8, (d, o) => Number(d.getBigUint64(o, true))],
  11: [8, (d, o) => Number(d.getBigInt64(o, true))],
  12: [8, (d, o) => d.getFloat64(o, true)],
};
// Arrays of these element types come back as typed arrays (token types, scores), others as Arrays.
const TYPED_ARRAY = { 5: Int32Array, 6: Float32Array };

const MAGIC = 0x46554747;   // "GGUF" read as a little-endian uint32

class Cursor {
  constructor(bytes) {
    this.bytes = bytes;
    this.view = new DataView(bytes.buffer, bytes.byteOffset, bytes.byteLength);
    this.at = 0;
    this.utf8 = new TextDecoder("utf-8");
  }

  take(n) {
    if (!(n >= 0) || this.at + n > this.bytes.byteLength)
      throw new Error(`GGUF file ends inside a field at byte ${this.at}`);
    const at = this.at;
    this.at += n;
    return at;
  }

  fixed(type) {
    const f = FIXED[type];
    if (f === undefined) throw new Error(`unknown GGUF value type ${type}`);
    return f[1](this.view, this.take(f[0]));
  }

  u32() { return this.fixed(4); }
  u64() { return this.fixed(10); }

  string() {
    const n = this.u64();
    const at = this.take(n);
    return this.utf8.decode(this.bytes.subarray(at, at + n));
  }

  array() {
    const type = this.u32(), n = this.u64();
    const Typed = TYPED_ARRAY[type];
    if (Typed) {
      const size = FIXED[type][0], at = this.take(n * size), out = new Typed(n), get = FIXED[type][1];
      for (let i = 0; i < n; i++) out[i] = get(this.view, at + i * size);
      return out;
    }
    const out = new Array(n);
    for (let i = 0; i < n; i++) out[i] = this.value(type);
    return out;
  }

  value(type) {
    if (type === V_STRING) return this.string();
    if (type === V_ARRAY) return this.array();
    return this.fixed(type);
  }
}

// `buffer`: an ArrayBuffer, or a Uint8Array / Buffer view of the whole file.
function parseGGUF(buffer) {
  const bytes = buffer instanceof Uint8Array ? buffer : new Uint8Array(buffer);
  if (bytes.byteLength < 24) throw new Error("not a GGUF file");
  const c = new Cursor(bytes);
  if (c.u32() !== MAGIC) throw new Error("not a GGUF file");
  const version = c.u32();
  const nTensors = c.u64();
  const nMeta = c.u64();

  const meta = {};
  for (let i = 0; i < nMeta; i++) {
    const key = c.string();
    meta[key] = c.value(c.u32());
  }

  const directory = [];
  for (let i = 0; i < nTensors; i++) {
    const name = c.string();
    const rank = c.u32();
    const shape = [];
    while (shape.length < rank) shape.push(c.u64());
    const type = c.u32();
    const offset = c.u64();
    directory.push({ name, shape, type, offset });
  }

  const align = meta["general.alignment"] || 32;
  const dataStart = Math.ceil(c.at / align) * align;
  const tensors = {};
  for (const d of directory) {
    const count = d.shape.reduce((n, x) => n * x, 1);
    const start = dataStart + d.offset;
    const size = tensorBytes(d.type, count);
    if (start + size > bytes.byteLength) throw new Error(`${d.name}: data past the end of the file`);
    tensors[d.name] = { name: d.name, shape: d.shape, type: d.type, offset: d.offset, count, start, bytes: size };
  }
  return { version, meta, tensors, dataStart };
}

// Hyperparameters of a Qwen2-family model: the fields and defaults the engine's backends expect.
function qwen2Config(meta) {
  const arch = meta["general.architecture"];
  const hp = (name) => meta[arch + "." + name];
  const vocabulary = meta["tokenizer.ggml.tokens"];
  return {
    arch,
    dim: hp("embedding_length"),
    layers: hp("block_count"),
    ffn: hp("feed_forward_length"),
    heads: hp("attention.head_count"),
    kvHeads: hp("attention.head_count_kv"),
    ropeTheta: hp("rope.freq_base") || 10000,
    eps: hp("attention.layer_norm_rms_epsilon"),
    vocab: vocabulary ? vocabulary.length : 0,
    eos: meta["tokenizer.ggml.eos_token_id"],
    contextMax: hp("context_length"),
  };
}

// The whole file in memory (the browser engine downloads it instead).
function readModel(path, onProgress) {
  const data = fs.readFileSync(path);
  if (onProgress) onProgress(data.length, data.length, true);
  return new Uint8Array(data.buffer, data.byteOffset, data.byteLength);
}

module.exports = { TYPE, tensorBytes, parseGGUF, qwen2Config, readModel };
