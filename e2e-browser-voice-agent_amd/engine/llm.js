"use strict";
// The engine's public face in Node.js: load a Qwen2 GGUF model onto the GPU and run token ids.
//
//   const llm = await LLM.load({ path: "model.gguf", backend: "hip", ctx: 2048 });
//   for await (const piece of llm.chat(messages, { maxTokens: 128 })) process.stdout.write(piece);
//   const ids = await llm.generateIds(promptIds, 64);
//
// Same cache discipline as the reference (h2-own-inference-engine/engine/llm.js:35-97): `seen`
// holds the ids whose K/V are in the cache, and feed() reruns only what differs from it, so a chat
// turn only runs the new messages.

const { parseGGUF, qwen2Config, readModel } = require("./gguf.js");
const { createHIP } = require("./hip.js");
const { Tokenizer, chatPrompt } = require("./tokenizer.js");
const { performance } = require("perf_hooks");

class LLM {
  static async load({ path, bytes, backend = "hip", ctx = 2048, onProgress = () => {}, ...opts }) {
    const t0 = performance.now();
    const data = bytes ? (bytes instanceof Uint8Array ? bytes : new Uint8Array(bytes))
      : readModel(path, (got, total, cached) => onProgress({ stage: cached ? "cache" : "read", got, total }));
    const tRead = performance.now() - t0;
    const gguf = parseGGUF(data);
    const cfg = qwen2Config(gguf.meta);
    if (cfg.arch !== "qwen2") throw new Error(`unsupported architecture ${cfg.arch}`);
    if (backend !== "hip") throw new Error(`unknown backend ${backend}`);
    // files without merges (token ids only) load; chat() then reports the missing tokenizer
    const tok = Array.isArray(gguf.meta["tokenizer.ggml.merges"]) ? new Tokenizer(gguf.meta) : null;
    const t1 = performance.now();
    const be = await createHIP(gguf, data, cfg,
      Object.assign({ ctx, onProgress: (l, n) => onProgress({ stage: "upload", got: l, total: n }) }, opts));
    const llm = new LLM(be, cfg, tok);
    llm.loadTimes = { read: tRead, prepare: performance.now() - t1 };
    return llm;
  }

  constructor(backend, cfg, tokenizer = null) {
    this.be = backend;
    this.cfg = cfg;
    this.tok = tokenizer;
    this.seen = [];                     // tokens whose K/V are in the cache, in order
    this.stats = null;
    this.stopIds = new Set([cfg.eos]);
    if (tokenizer && tokenizer.ids.has("<|endoftext|>")) this.stopIds.add(tokenizer.ids.get("<|endoftext|>"));
  }

  get backend() { return this.be.name; }

  // Process `ids` as a continuation of the cache, reusing the longest common prefix (llm.js:45-54).
  async feed(ids, sampling) {
    let common = 0;
    while (common < ids.length && common < this.seen.length && ids[common] === this.seen[common]) common++;
    if (common === ids.length) common--;            // always run at least one token to get fresh logits
    this.seen = ids.slice(0, common);
    const fresh = ids.slice(common);
    const next = await this.be.forward(fresh, common, sampling);
    this.seen.push(...fresh);
    return { next, prefilled: fresh.length, reused: common };
  }

  // Stream the assistant's reply to `messages` ({role, content}) as text pieces (llm.js:56-83): the
  // ChatML prompt, trimmed from the oldest exchange (never the system message) until prompt +
  // maxTokens fit the context; decoding stops at an end-of-text id, maxTokens or signal.aborted.  The
  // end-of-turn id stays in the cache so that the next turn's prompt continues it.
  async *chat(messages, { maxTokens = 256, temperature = 0, seed = (Math.random() * 2 ** 32) >>> 0, signal } = {}) {
    if (!this.tok) throw new Error("the model file has no tokenizer");
    let msgs = messages;
    let ids = this.tok.encode(chatPrompt(msgs));
    while (ids.length + maxTokens > this.be.ctx - 8 && msgs.length > 2) {
      msgs = msgs[0].role === "system" ? [msgs[0], ...msgs.slice(3)] : msgs.slice(2);
      ids = this.tok.encode(chatPrompt(msgs));
    }
    const piece = this.tok.streamDecoder();
    const t0 = performance.now();
    const first = await this.feed(ids, { temperature, seed });
    let next = first.next;
    const tFirst = performance.now() - t0;
    const out = [];
    while (!this.stopIds.has(next) && out.length < maxTokens && !(signal && signal.aborted)) {
      out.push(next);
      const text = piece(next);
      if (text) yield text;
      next = await this.be.forward([next], this.seen.length, { temperature, seed });
      this.seen.push(out[out.length - 1]);
    }
    if (this.stopIds.has(next)) {
      await this.be.forward([next], this.seen.length, { temperature, seed });
      this.seen.push(next);
    }
    const tTotal = performance.now() - t0;
    this.stats = { promptTokens: ids.length, prefilled: first.prefilled, reused: first.reused, firstTokenMs: tFirst,
      tokens: out.length, decodeTokPerS: out.length > 1 ? (out.length - 1) / ((tTotal - tFirst) / 1000) : 0,
      totalMs: tTotal, ids: out, stop: this.stopIds.has(next) ? next : null };
  }

  // Greedy continuation of raw token ids, one forward() per step (llm.js:86-97).  Resets the cache.
  async generateIds(ids, steps) {
    this.seen = [];
    const out = [];
    const t0 = performance.now();
    let { next } = await this.feed(ids, { temperature: 0 });
    const tFirst = performance.now() - t0;
    for (let i = 0; i < steps; i++) {
      out.push(next);
      if (i === steps - 1) break;
      next = await this.be.forward([next], this.seen.length, { temperature: 0 });
      this.seen.push(out[out.length - 1]);
    }
    const tTotal = performance.now() - t0;
    this.stats = { promptTokens: ids.length, firstTokenMs: tFirst, tokens: out.length, totalMs: tTotal,
      decodeTokPerS: out.length > 1 ? (out.length - 1) / ((tTotal - tFirst) / 1000) : 0 };
    return out;
  }

  // The same tokens as generateIds, with the decode loop on the device (no host round trip per token).
  async generateIdsDevice(ids, steps) {
    this.seen = [];
    const t0 = performance.now();
    const { next } = await this.feed(ids, { temperature: 0 });
    const tFirst = performance.now() - t0;
    const rest = steps > 1 ? await this.be.generate(next, this.seen.length, steps - 1) : [];
    const out = [next, ...rest];
    this.seen.push(...out.slice(0, -1));
    const tTotal = performance.now() - t0;
    this.stats = { promptTokens: ids.length, firstTokenMs: tFirst, tokens: out.length, totalMs: tTotal,
      decodeTokPerS: out.length > 1 ? (out.length - 1) / ((tTotal - tFirst) / 1000) : 0 };
    return out;
  }

  reset() { this.seen = []; }

  destroy() { this.be.destroy(); }
}

module.exports = { LLM };
