"use strict";
// Text <-> token ids for Qwen2 GGUF files: byte-level BPE over the vocabulary and merge list the
// file stores (tokenizer.ggml.tokens / token_type / merges), and the ChatML prompt of Qwen2.5 chat
// models.  Mirrors the reference's Tokenizer and chatPrompt (h2-own-inference-engine/engine/
// tokenizer.js:1-110): same inputs, same ids, same text.
//
// Fixed by the model, so necessarily identical to any other implementation: the GPT-2 byte -> char
// table, Qwen2's pre-tokenization pattern, merge-by-lowest-rank, and the ChatML template text.

// Printable stand-ins for the 256 byte values: printable Latin-1 bytes stand for themselves, the
// other 68 take code points 256, 257, ... in byte order.
function byteChars() {
  const printable = (b) => (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255);
  const out = new Array(256);
  let extra = 0;
  for (let b = 0; b < 256; b++) out[b] = String.fromCodePoint(printable(b) ? b : 256 + extra++);
  return out;
}

// Qwen2's pre-tokenizer split (its tokenizer.json "Split" pattern): contractions, letter runs with one
// optional leading non-letter, single digits, punctuation runs with trailing newlines, newline runs,
// trailing whitespace, whitespace.
const SPLIT = /(?:'[sS]|'[tT]|'[rR][eE]|'[vV][eE]|'[mM]|'[lL][lL]|'[dD])|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+/gu;

const CONTROL = 3, USER_DEFINED = 4;   // GGUF token types matched literally

class Tokenizer {
  constructor(meta) {
    const tokens = meta["tokenizer.ggml.tokens"], merges = meta["tokenizer.ggml.merges"];
    if (!Array.isArray(tokens) || !Array.isArray(merges)) throw new Error("the file has no BPE tokenizer");
    const types = meta["tokenizer.ggml.token_type"] || [];
    this.tokens = tokens;
    this.ids = new Map();
    tokens.forEach((t, i) => { if (!this.ids.has(t)) this.ids.set(t, i); });
    this.rank = new Map();
    merges.forEach((m, i) => { if (!this.rank.has(m)) this.rank.set(m, i); });
    this.chars = byteChars();
    this.byteOf = new Map(this.chars.map((c, b) => [c, b]));
    this.specialIds = new Set();
    const specials = [];
    types.forEach((ty, i) => {
      if (ty === CONTROL || ty === USER_DEFINED) { this.specialIds.add(i); specials.push(tokens[i]); }
    });
    // longest first, so that a special token that prefixes another never wins
    specials.sort((a, b) => b.length - a.length);
    const esc = (s) => s.replace(/[.*+?^${}()|[\]\\]/g, "\\$&");
    this.specialSplit = specials.length ? new RegExp(`(${specials.map(esc).join("|")})`) : null;
    this.memo = new Map();
    this.utf8 = new TextEncoder();
  }

  // One pre-tokenized piece -> ids: start from one symbol per byte, merge the adjacent pair of lowest
  // rank (every occurrence, left to right) until no pair has a rank.
  pieceIds(piece) {
    const known = this.memo.get(piece);
    if (known) return known;
    let sym = Array.from(this.utf8.encode(piece), (b) => this.chars[b]);
    for (;;) {
      let best = Infinity, at = -1;
      for (let i = 0; i + 1 < sym.length; i++) {
        const r = this.rank.get(`${sym[i]} ${sym[i + 1]}`);
        if (r !== undefined && r < best) { best = r; at = i; }
      }
      if (at < 0) break;
      const left = sym[at], right = sym[at + 1], next = [];
      for (let i = 0; i < sym.length;) {
        if (i + 1 < sym.length && sym[i] === left && sym[i + 1] === right) { next.push(left + right); i += 2; }
        else next.push(sym[i++]);
      }
      sym = next;
    }
    const ids = sym.map((s) => {
      const id = this.ids.get(s);
      if (id === undefined) throw new Error(`no token for ${JSON.stringify(s)}`);
      return id;
    });
    if (this.memo.size < 50000) this.memo.set(piece, ids);
    return ids;
  }

  encode(text) {
    const out = [];
    const norm = text.normalize("NFC");
    const parts = this.specialSplit ? norm.split(this.specialSplit) : [norm];
    for (let k = 0; k < parts.length; k++) {
      const part = parts[k];
      if (!part) continue;
      if (k % 2 === 1 && this.specialSplit) { out.push(this.ids.get(part)); continue; }   // a captured special
      for (const m of part.matchAll(SPLIT)) for (const id of this.pieceIds(m[0])) out.push(id);
    }
    return out;
  }

  // The bytes a token stands for (a special token: its literal text).
  tokenBytes(id) {
    const t = this.tokens[id];
    if (this.specialIds.has(id)) return this.utf8.encode(t);
    const out = new Uint8Array(t.length);
    let n = 0;
    for (const c of t) out[n++] = this.byteOf.get(c);
    return out.subarray(0, n);
  }

  decode(ids) {
    const parts = ids.map((id) => this.tokenBytes(id));
    const all = new Uint8Array(parts.reduce((s, p) => s + p.length, 0));
    let o = 0;
    for (const p of parts) { all.set(p, o); o += p.length; }
    return new TextDecoder().decode(all);
  }

  // Incremental decoding: bytes of a character split over tokens are held until it is complete.
  streamDecoder() {
    const td = new TextDecoder();
    return (id) => td.decode(this.tokenBytes(id), { stream: true });
  }
}

// ChatML as Qwen2.5's chat template renders plain-text messages (with its default system message
// when the conversation has none).
const DEFAULT_SYSTEM = "You are Qwen, created by Alibaba Cloud. You are a helpful assistant.";

function chatPrompt(messages, addGenerationPrompt = true) {
  const turn = (role, content) => `<|im_start|>${role}\n${content}<|im_end|>\n`;
  let s = messages.length && messages[0].role === "system" ? "" : turn("system", DEFAULT_SYSTEM);
  for (const m of messages) s += turn(m.role, m.content);
  return addGenerationPrompt ? s + "<|im_start|>assistant\n" : s;
}

module.exports = { Tokenizer, chatPrompt, byteChars };
