"use strict";
// GGUF reader for Node.js: the file format of the model weights.
//
//   "GGUF" | version | tensor count | metadata (key -> value) | tensor table (name, shape, type, offset) | data
//
// Same results as the reference's parseGGUF/qwen2Config (h2-own-inference-engine/engine/gguf.js:15-88):
// `tensors[name] = {name, shape, type, offset, count, start, bytes}` with shape[0] the row length and
// `start` the absolute byte offset of the tensor's data.  The reference's fetchModel (browser download +
// Cache Storage) has a Node counterpart here, readModel(path).

const fs = require("fs");

const TYPE = { F32: 0, F16: 1, Q4_0: 2, Q8_0: 8 };
const BLOCK = { 0: [1, 4], 1: [1, 2], 2: [32, 18], 8: [32, 34] };   // type -> [values per block, bytes per block]

function tensorBytes(type, count) {
  const b = BLOCK[type];
  if (!b) throw new Error(`unsupported tensor type ${type}`);
  return (count / b[0]) * b[1];
}

// `buffer`: an ArrayBuffer, or a Uint8Array / Buffer view of the file.
function parseGGUF(buffer) {
  const bytes = buffer instanceof Uint8Array ? buffer : new Uint8Array(buffer);
  const view = new DataView(bytes.buffer, bytes.byteOffset, bytes.byteLength);
  const dec = new TextDecoder();
  let p = 0;
  const u32 = () => { const v = view.getUint32(p, true); p += 4; return v; };
  const u64 = () => { const v = Number(view.getBigUint64(p, true)); p += 8; return v; };
  const str = () => { const n = u64(); const s = dec.decode(bytes.subarray(p, p + n)); p += n; return s; };
  const readValue = (type) => {
    switch (type) {
      case 0: return view.getUint8(p++);
      case 1: return view.getInt8(p++);
      case 2: { const v = view.getUint16(p, true); p += 2; return v; }
      case 3: { const v = view.getInt16(p, true); p += 2; return v; }
      case 4: return u32();
      case 5: { const v = view.getInt32(p, true); p += 4; return v; }
      case 6: { const v = view.getFloat32(p, true); p += 4; return v; }
      case 7: return view.getUint8(p++) !== 0;
      case 8: return str();
      case 9: {
        const t = u32(), n = u64();
        const a = new Array(n);
        for (let i = 0; i < n; i++) a[i] = readValue(t);
        return a;
      }
      case 10: return u64();
      case 11: { const v = Number(view.getBigInt64(p, true)); p += 8; return v; }
      case 12: { const v = view.getFloat64(p, true); p += 8; return v; }
      default: throw new Error(`unknown GGUF value type ${type}`);
    }
  };

  if (u32() !== 0x46554747) throw new Error("not a GGUF file");
  const version = u32();
  const nTensors = u64(), nKV = u64();
  const meta = {};
  for (let i = 0; i < nKV; i++) { const k = str(); meta[k] = readValue(u32()); }
  const tensors = {};
  for (let i = 0; i < nTensors; i++) {
    const name = str();
    const nd = u32();
    const shape = [];
    for (let d = 0; d < nd; d++) shape.push(u64());                   // shape[0] = row length
    const type = u32(), offset = u64();
    tensors[name] = { name, shape, type, offset, count: shape.reduce((a, b) => a * b, 1) };
  }
  const align = meta["general.alignment"] || 32;
  const dataStart = Math.ceil(p / align) * align;
  for (const t of Object.values(tensors)) {
    t.start = dataStart + t.offset;
    t.bytes = tensorBytes(t.type, t.count);
    if (t.start + t.bytes > bytes.byteLength) throw new Error(`${t.name}: data past the end of the file`);
  }
  return { version, meta, tensors, dataStart };
}

// Qwen2-family hyperparameters from the metadata (gguf.js:72-88).
function qwen2Config(meta) {
  const a = meta["general.architecture"];
  const g = (k) => meta[`${a}.${k}`];
  const tokens = meta["tokenizer.ggml.tokens"];
  return {
    arch: a,
    dim: g("embedding_length"),
    layers: g("block_count"),
    ffn: g("feed_forward_length"),
    heads: g("attention.head_count"),
    kvHeads: g("attention.head_count_kv"),
    ropeTheta: g("rope.freq_base") || 10000,
    eps: g("attention.layer_norm_rms_epsilon"),
    vocab: tokens ? tokens.length : 0,
    eos: meta["tokenizer.ggml.eos_token_id"],
    contextMax: g("context_length"),
  };
}

// Read a model file into memory (the Node counterpart of fetchModel, gguf.js:91-118).
function readModel(path, onProgress) {
  const buf = fs.readFileSync(path);
  if (onProgress) onProgress(buf.length, buf.length, true);
  return new Uint8Array(buf.buffer, buf.byteOffset, buf.byteLength);
}

module.exports = { TYPE, tensorBytes, parseGGUF, qwen2Config, readModel };
