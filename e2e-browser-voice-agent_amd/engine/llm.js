"use strict";
// The engine's public face in Node.js: load a Qwen2 GGUF model onto the GPU and run token ids.
//
//   const llm = await LLM.load({ path: "model.gguf", ctx: 2048 });
//   for await (const piece of llm.chat(messages, { maxTokens: 128 })) process.stdout.write(piece);
//   const ids = await llm.generateIds(promptIds, 64);
//
// The surface is the reference engine's LLM (h2-own-inference-engine/engine/llm.js:12-100): load,
// feed, chat, generateIds, reset, backend, stats, seen.  Its cache discipline is kept: the backend's
// K/V cache is positional, `seen` lists the ids whose K/V it holds, and a call reruns only what
// differs from `seen` (a chat turn runs just the new messages).  Backends are chosen by name; this
// host has one, "hip" (the reference chooses between "webgpu" and "cpu", llm.js:23-29).

const { performance } = require("perf_hooks");
const { parseGGUF, qwen2Config, readModel } = require("./gguf.js");
const { createHIP } = require("./hip.js");
const { Tokenizer, chatPrompt } = require("./tokenizer.js");

const BACKENDS = { hip: createHIP };
const CONTEXT_MARGIN = 8;   // positions kept free when a chat prompt is fitted to the context

// Length of the common prefix of two id lists.
function commonPrefix(a, b) {
  const n = Math.min(a.length, b.length);
  let i = 0;
  while (i < n && a[i] === b[i]) i++;
  return i;
}

// Drop the oldest exchange (the first user/assistant pair after the system message, if any) until
// the encoded prompt leaves room for `room` tokens in `ctx` positions, or only the last exchange is
// left.  Returns the prompt's ids.
function fitPrompt(tok, messages, room, ctx) {
  let msgs = messages;
  let ids = tok.encode(chatPrompt(msgs));
  while (ids.length + room > ctx - CONTEXT_MARGIN && msgs.length > 2) {
    const keep = msgs[0].role === "system" ? 1 : 0;
    msgs = msgs.slice(0, keep).concat(msgs.slice(keep + 2));
    ids = tok.encode(chatPrompt(msgs));
  }
  return ids;
}

function rate(tokens, totalMs, firstMs) {
  return tokens > 1 ? (tokens - 1) / ((totalMs - firstMs) / 1000) : 0;
}

class LLM {
  static async load({ path, bytes, backend = "hip", ctx = 2048, onProgress = () => {}, ...opts }) {
    const make = BACKENDS[backend];
    if (!make) throw new Error(`unknown backend ${backend}`);
    const t0 = performance.now();
    const data = bytes !== undefined ? (bytes instanceof Uint8Array ? bytes : new Uint8Array(bytes))
      : readModel(path, (got, total, cached) => onProgress({ stage: cached ? "cache" : "read", got, total }));
    const tRead = performance.now() - t0;
    const gguf = parseGGUF(data);
    const cfg = qwen2Config(gguf.meta);
    if (cfg.arch !== "qwen2") throw new Error(`unsupported architecture ${cfg.arch}`);
    // a file without merges (token ids only) loads; chat() then reports the missing tokenizer
    const tok = Array.isArray(gguf.meta["tokenizer.ggml.merges"]) ? new Tokenizer(gguf.meta) : null;
    const t1 = performance.now();
    const be = await make(gguf, data, cfg,
      Object.assign({ ctx, onProgress: (l, n) => onProgress({ stage: "upload", got: l, total: n }) }, opts));
    const llm = new LLM(be, cfg, tok);
    llm.loadTimes = { read: tRead, prepare: performance.now() - t1 };
    return llm;
  }

  constructor(backend, cfg, tokenizer = null) {
    this.be = backend;
    this.cfg = cfg;
    this.tok = tokenizer;
    this.seen = [];          // ids whose K/V the backend's cache holds, position by position
    this.stats = null;
    this.stopIds = new Set([cfg.eos]);
    if (tokenizer && tokenizer.ids.has("<|endoftext|>")) this.stopIds.add(tokenizer.ids.get("<|endoftext|>"));
  }

  get backend() { return this.be.name; }

  // Run `ids` as the cache's new contents: positions that already hold the same ids are kept, the
  // rest (at least the last id, whose logits give the next token) run from the first difference on.
  async feed(ids, sampling) {
    if (!ids.length) throw new Error("feed: no token ids");
    const reused = Math.min(commonPrefix(ids, this.seen), ids.length - 1);
    const fresh = ids.slice(reused);
    this.seen.length = reused;
    const next = await this.be.forward(fresh, reused, sampling);
    for (const id of fresh) this.seen.push(id);
    return { next, prefilled: fresh.length, reused };
  }

  // One decode step: `id` goes into the cache at the next position; returns the token after it.
  async step(id, sampling) {
    const next = await this.be.forward([id], this.seen.length, sampling);
    this.seen.push(id);
    return next;
  }

  // Stream the assistant's reply to `messages` ({role, content}) as text pieces.  The ChatML prompt is
  // fitted to the context by dropping old exchanges (never the system message); decoding stops at an
  // end-of-text id, after maxTokens tokens, or when signal.aborted.  A stop id is run into the cache
  // too, so the next turn's prompt continues it.
  async *chat(messages, { maxTokens = 256, temperature = 0, seed = (Math.random() * 2 ** 32) >>> 0, signal } = {}) {
    if (!this.tok) throw new Error("the model file has no tokenizer");
    const sampling = { temperature, seed };
    const ids = fitPrompt(this.tok, messages, maxTokens, this.be.ctx);
    const text = this.tok.streamDecoder();
    const t0 = performance.now();
    const fed = await this.feed(ids, sampling);
    const tFirst = performance.now() - t0;
    const reply = [];
    let next = fed.next;
    for (;;) {
      if (this.stopIds.has(next) || reply.length >= maxTokens || (signal && signal.aborted)) break;
      reply.push(next);
      const piece = text(next);
      if (piece) yield piece;
      next = await this.step(next, sampling);
    }
    const stop = this.stopIds.has(next) ? next : null;
    if (stop !== null) await this.step(stop, sampling);
    const tTotal = performance.now() - t0;
    this.stats = { promptTokens: ids.length, prefilled: fed.prefilled, reused: fed.reused, firstTokenMs: tFirst,
      tokens: reply.length, decodeTokPerS: rate(reply.length, tTotal, tFirst), totalMs: tTotal, ids: reply, stop };
  }

  // Greedy continuation of raw token ids, one backend call per token.  Starts from an empty cache.
  // Also records the host-side time of each decode call (stats.stepMs).
  async generateIds(ids, steps) {
    this.seen = [];
    const t0 = performance.now();
    const fed = await this.feed(ids, { temperature: 0 });
    const tFirst = performance.now() - t0;
    const out = steps > 0 ? [fed.next] : [];
    const stepMs = [];
    while (out.length < steps) {
      const s0 = performance.now();
      out.push(await this.step(out[out.length - 1], { temperature: 0 }));
      stepMs.push(performance.now() - s0);
    }
    const tTotal = performance.now() - t0;
    this.stats = { promptTokens: ids.length, firstTokenMs: tFirst, tokens: out.length, totalMs: tTotal,
      decodeTokPerS: rate(out.length, tTotal, tFirst), stepMs };
    return out;
  }

  // The tokens of generateIds with the decode loop on the device (no host round trip per token).
  async generateIdsDevice(ids, steps) {
    this.seen = [];
    const t0 = performance.now();
    const fed = await this.feed(ids, { temperature: 0 });
    const tFirst = performance.now() - t0;
    const rest = steps > 1 ? await this.be.generate(fed.next, this.seen.length, steps - 1) : [];
    const out = steps > 0 ? [fed.next].concat(rest) : [];
    for (const id of out.slice(0, -1)) this.seen.push(id);
    const tTotal = performance.now() - t0;
    this.stats = { promptTokens: ids.length, firstTokenMs: tFirst, tokens: out.length, totalMs: tTotal,
      decodeTokPerS: rate(out.length, tTotal, tFirst) };
    return out;
  }

  reset() { this.seen = []; }

  destroy() { this.be.destroy(); }
}

module.exports = { LLM, commonPrefix, fitPrompt };
