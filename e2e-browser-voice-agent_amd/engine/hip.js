"use strict";
// HIP backend for Qwen2-style GGUF models (Q4_0 layers) on one AMD MI355X.
//
//   createHIP(gguf, bytes, cfg, opts) -> Promise<backend>
//
// The backend object has the surface the reference engine's LLM class drives
// (h2-own-inference-engine/engine/cpu.js:52-68, engine/webgpu.js:617-620):
//   name, ctx, info, forward(ids, pos, {temperature, seed, wantLogits}) -> next id,
//   readLogits() -> Float32Array(vocab), profile(), destroy()
// plus generate(first, pos, steps), the greedy loop run on the device; setKv(layer, kvHead, pos0,
// k, v), rows written straight into the K/V cache; setDecodeMode / decodeModeUsed, the choice
// between the persistent decode kernel and the captured graph; and createBatch(B), B sequences
// decoded together with this backend's weights (see makeBatch).
//
// Below it is the N-API addon lib/q4hip.node over the C ABI of include/q4hip.h.  The addon is
// required, not optional: without it (or without a GPU) createHIP throws.

const path = require("path");
const { TYPE } = require("./gguf.js");

let addon = null;
function loadAddon() {
  if (!addon) addon = require(path.join(__dirname, "..", "lib", "q4hip.node"));
  return addon;
}

// Tensor kinds of the C ABI (the reference's set_tensor numbering, engine/kernels.c:422).
const KIND = { QKV: 0, O: 1, GU: 2, DOWN: 3, ATTN_NORM: 4, FFN_NORM: 5, BQKV: 6, EMBD: 7, OUTPUT: 8, OUTPUT_NORM: 9 };
const PROFILE_NAMES = ["embed", "norm+quantize", "matvec qkv", "rope+kv", "attention", "quantize", "matvec o",
  "matvec gate+up", "swiglu+quantize", "matvec down", "matvec output", "sample"];

// cos/sin of pos * theta^(-2i/hd) for every position, computed in double and stored as fp32,
// exactly as engine/cpu-worker.js:130-135.
function ropeTable(ctx, hd, theta) {
  const rope = new Float32Array(ctx * hd);
  for (let pos = 0; pos < ctx; pos++) {
    for (let i = 0; i < hd / 2; i++) {
      const a = pos / Math.pow(theta, (2 * i) / hd);
      rope[pos * hd + 2 * i] = Math.cos(a);
      rope[pos * hd + 2 * i + 1] = Math.sin(a);
    }
  }
  return rope;
}

// Sampling on the logits as engine/cpu-worker.js:154-167: greedy (first maximum wins), or
// softmax(logits / temperature) with the same seeded generator.
function sample(lg, temperature, seed) {
  let best = 0;
  for (let i = 1; i < lg.length; i++) if (lg[i] > lg[best]) best = i;
  if (!(temperature > 0)) return best;
  let s = seed >>> 0;
  const rand = () => {
    s = (s + 0x6d2b79f5) >>> 0;
    let t = s;
    t = Math.imul(t ^ (t >>> 15), t | 1);
    t ^= t + Math.imul(t ^ (t >>> 7), t | 61);
    return ((t ^ (t >>> 14)) >>> 0) / 4294967296;
  };
  const mx = lg[best] / temperature;
  let sum = 0;
  for (let i = 0; i < lg.length; i++) sum += Math.exp(lg[i] / temperature - mx);
  let r = rand() * sum;
  for (let i = 0; i < lg.length; i++) { r -= Math.exp(lg[i] / temperature - mx); if (r <= 0) return i; }
  return best;
}

// The token forward() returns after a call at position pos: sample() seeded with (seed + pos) >>> 0,
// as engine/cpu-worker.js:180 seeds it.
function sampleAt(lg, temperature, seed, pos) {
  return sample(lg, temperature, (seed + pos) >>> 0);
}

const DECODE_MODES = { auto: 0, graph: 1, persistent: 2 };
const DECODE_NAMES = { 0: null, 1: "graph", 2: "persistent" };

// B independent sequences on the weights of context h, each with its own K/V cache (the reference
// runs one sequence per backend; a batch runs B such loops in one pass per step):
//   prefill(seq, ids, pos) -> next id of that sequence after ids at positions pos..
//   setKv(seq, layer, kvHead, pos0, k, v)   K/V rows of one sequence, as the backend's setKv
//   generate(first, pos, steps) -> B arrays of steps greedy tokens; sequence b starts with first[b]
//                                  at position pos[b]
//   readLogits() -> Float32Array(B * vocab), the last step's logits, sequence by sequence
//   destroy()
// Calls on a batch and on its backend share the backend's buffers and run one at a time.
function makeBatch(a, h, B, vocab, ctx) {
  const bt = a.batchCreate(h, B);
  const ints = (xs, what) => {
    if (xs.length !== B) throw new Error(`${what}: ${B} entries expected, got ${xs.length}`);
    return Int32Array.from(xs);
  };
  return {
    B,
    async prefill(seq, ids, pos = 0) {
      if (!ids.length) throw new Error("prefill: no token ids");
      if (pos + ids.length >= ctx) throw new Error("context full");
      return a.batchPrefill(bt, seq, Int32Array.from(ids), pos);
    },
    setKv(seq, layer, kvHead, pos0, k, v) { a.batchSetKv(bt, seq, layer, kvHead, pos0, k, v); },
    async generate(first, pos, steps) {
      const o = new Int32Array(steps * B);
      a.batchGenerate(bt, ints(first, "first"), ints(pos, "pos"), o);
      const per = [];
      for (let b = 0; b < B; b++) {
        const t = new Array(steps);
        for (let i = 0; i < steps; i++) t[i] = o[i * B + b];
        per.push(t);
      }
      return per;
    },
    async readLogits() {
      const lg = new Float32Array(B * vocab);
      a.batchReadLogits(bt, lg);
      return lg;
    },
    destroy() { a.batchDestroy(bt); },
  };
}

function check(T, name, types, label) {
  const t = T[name];
  if (!t) throw new Error(`${name}: missing`);
  if (types.indexOf(t.type) < 0) throw new Error(`${name}: expected ${label}`);
  return t;
}

async function createHIP(gguf, bytes, cfg, opts = {}) {
  const { dim: D, layers: NL, ffn: F, heads: H, kvHeads: KVH, vocab, ropeTheta, eps } = cfg;
  const HD = D / H, KV = KVH * HD;
  const ctx = opts.ctx || 2048;
  const device = opts.device || 0;
  const T = gguf.tensors;
  const src = bytes instanceof Uint8Array ? bytes : new Uint8Array(bytes);

  // Validate every tensor before touching the GPU (the reference throws the same way while
  // copying, engine/cpu-worker.js:105,112,126).
  const Q4 = [TYPE.Q4_0], F32 = [TYPE.F32];
  const layers = [];
  for (let l = 0; l < NL; l++) {
    const p = `blk.${l}.`;
    const q = (n) => check(T, p + n, Q4, "Q4_0");
    const f = (n) => check(T, p + n, F32, "F32");
    layers.push({
      qkv: [q("attn_q.weight"), q("attn_k.weight"), q("attn_v.weight")],
      o: q("attn_output.weight"), gu: [q("ffn_gate.weight"), q("ffn_up.weight")], down: q("ffn_down.weight"),
      attnNorm: f("attn_norm.weight"), ffnNorm: f("ffn_norm.weight"),
      bias: [f("attn_q.bias"), f("attn_k.bias"), f("attn_v.bias")],
    });
  }
  const embd = check(T, "token_embd.weight", Q4, "Q4_0");
  // the head: Q4_0 in the synthetic configurations, Q8_0 in real Qwen2.5 files (cpu-worker.js:126)
  const out = check(T, "output.weight", [TYPE.Q4_0, TYPE.Q8_0], "Q4_0 or Q8_0");
  const outNorm = check(T, "output_norm.weight", F32, "F32");

  const kvDtype = opts.kvDtype || "f32";
  if (kvDtype !== "f32" && kvDtype !== "f16") throw new Error(`kvDtype must be "f32" or "f16", not ${kvDtype}`);
  const a = loadAddon();
  const h = a.create(D, NL, F, H, KVH, vocab, ctx, opts.prefillChunk || 0, eps, device, kvDtype === "f16" ? 1 : 0);
  const rows = (t) => (t.type === TYPE.F32 ? t.count : t.count / t.shape[0]);
  const up = (kind, layer, row0, t) =>
    a.setTensor(h, kind, layer, row0, t.type, src.subarray(t.start, t.start + t.bytes), rows(t));
  try {
    for (let l = 0; l < NL; l++) {
      const y = layers[l];
      up(KIND.QKV, l, 0, y.qkv[0]); up(KIND.QKV, l, D, y.qkv[1]); up(KIND.QKV, l, D + KV, y.qkv[2]);
      up(KIND.O, l, 0, y.o);
      up(KIND.GU, l, 0, y.gu[0]); up(KIND.GU, l, F, y.gu[1]);
      up(KIND.DOWN, l, 0, y.down);
      up(KIND.ATTN_NORM, l, 0, y.attnNorm); up(KIND.FFN_NORM, l, 0, y.ffnNorm);
      up(KIND.BQKV, l, 0, y.bias[0]); up(KIND.BQKV, l, D, y.bias[1]); up(KIND.BQKV, l, D + KV, y.bias[2]);
      if (opts.onProgress) opts.onProgress(l + 1, NL);
    }
    up(KIND.EMBD, 0, 0, embd);
    up(KIND.OUTPUT, 0, 0, out);
    up(KIND.OUTPUT_NORM, 0, 0, outNorm);
    a.setRope(h, ropeTable(ctx, HD, ropeTheta));
  } catch (e) {
    a.destroy(h);
    throw e;
  }

  const logits = new Float32Array(vocab);
  return {
    name: "hip",
    ctx,
    device,
    kvDtype,
    info: `HIP device ${device}, Q4_0 x int8 kernels, ${out.type === TYPE.Q8_0 ? "Q8_0" : "Q4_0"} head, ${kvDtype === "f16" ? "fp16" : "fp32"} KV cache, persistent decode kernel`,
    // Run ids at positions pos.. and return the next token (engine/cpu-worker.js:169-182).
    async forward(ids, pos, { temperature = 0, seed = 1, wantLogits = false } = {}) {
      if (pos + ids.length >= ctx) throw new Error("context full");
      const next = a.forward(h, Int32Array.from(ids), pos);
      if (!(temperature > 0)) return next;
      a.readLogits(h, logits);
      return sampleAt(logits, temperature, seed, pos);
    },
    async readLogits() {
      a.readLogits(h, logits);
      return logits.slice();
    },
    // Greedy continuation on the device: `steps` tokens after `first` at position pos.
    async generate(first, pos, steps) {
      const o = new Int32Array(steps);
      a.generate(h, first, pos, o);
      return Array.from(o);
    },
    // GPU time per operation of one decode step, in microseconds (engine/cpu-worker.js:31-37).
    async profile(token = 0, pos = 64) {
      const us = new Float32Array(PROFILE_NAMES.length);
      a.profile(h, token, pos, us);
      const by = {};
      PROFILE_NAMES.forEach((n, i) => { by[n] = us[i]; });
      return by;
    },
    // K and V rows [n][head_dim] (Float32Array each) of one layer and kv head at positions pos0..,
    // e.g. a cache prefilled from stored activations (rounded to fp16 in an fp16 cache).
    setKv(layer, kvHead, pos0, k, v) { a.setKv(h, layer, kvHead, pos0, k, v); },
    // "auto" (persistent kernel where the model and device admit it), "graph" or "persistent";
    // both paths give identical tokens.
    setDecodeMode(mode) {
      if (!(mode in DECODE_MODES)) throw new Error(`decode mode must be auto, graph or persistent, not ${mode}`);
      a.setDecodeMode(h, DECODE_MODES[mode]);
    },
    // The path of the last decode step: "persistent", "graph", or null before any.
    decodeModeUsed() { return DECODE_NAMES[a.decodeModeUsed(h)]; },
    createBatch(B) { return makeBatch(a, h, B, vocab, ctx); },
    destroy() { a.destroy(h); },
  };
}

module.exports = { createHIP, ropeTable, sample, sampleAt, KIND, DECODE_MODES };
