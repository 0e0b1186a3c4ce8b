"use strict";
// Text <-> token ids for Qwen2 GGUF files, and the ChatML prompt of Qwen2.5 chat models.
//
// Byte-level BPE over the vocabulary and merge list the file stores (tokenizer.ggml.tokens,
// token_type, merges), with the interface of the reference engine's Tokenizer and chatPrompt
// (h2-own-inference-engine/engine/tokenizer.js): encode(text) -> ids, decode(ids) -> text,
// streamDecoder() -> (id -> text piece), ids (token text -> first id).
//
// Fixed by the model, so the same in every implementation that yields its ids: the GPT-2 byte ->
// character table, Qwen2's pre-tokenization pattern, lowest-rank-first merging (all occurrences of
// the chosen pair, left to right, before the next choice) and the ChatML template text.
//
// Here the merges run on token ids, not strings: each merge "A B" of rank r becomes an entry
// (id(A), id(B)) -> (r, id(AB)) in a table keyed by the id pair, and a piece starts as the ids of
// its UTF-8 bytes' tokens.  A merge whose result is not in the vocabulary (a malformed file) stays
// in the table and throws when it would apply.

// Printable stand-ins for the 256 byte values: printable Latin-1 bytes stand for themselves, the
// other 68 take code points 256, 257, ... in byte order.
function byteChars() {
  const shown = (b) => (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255);
  const out = [];
  let next = 256;
  for (let b = 0; b < 256; b++) out.push(String.fromCodePoint(shown(b) ? b : next++));
  return out;
}

// Qwen2's pre-tokenizer split (its tokenizer.json "Split" pattern): contractions, letter runs with one
// optional leading non-letter, single digits, punctuation runs with trailing newlines, newline runs,
// trailing whitespace, whitespace.
const SPLIT = /(?:'[sS]|'[tT]|'[rR][eE]|'[vV][eE]|'[mM]|'[lL][lL]|'[dD])|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+/gu;

const TOKEN_CONTROL = 3, TOKEN_USER_DEFINED = 4;   // GGUF token types that match their text literally
const PAIR = 262144;                               // pair key = left * PAIR + right (vocabularies < 2^18)
const MEMO_LIMIT = 1 << 16;

class Tokenizer {
  constructor(meta) {
    const tokens = meta["tokenizer.ggml.tokens"], merges = meta["tokenizer.ggml.merges"];
    if (!Array.isArray(tokens) || !Array.isArray(merges)) throw new Error("the file has no BPE tokenizer");
    if (tokens.length > PAIR) throw new Error(`vocabulary of ${tokens.length} tokens is too large`);
    this.tokens = tokens;
    this.ids = new Map();
    for (let i = 0; i < tokens.length; i++) if (!this.ids.has(tokens[i])) this.ids.set(tokens[i], i);

    const chars = byteChars();
    this.charByte = new Map(chars.map((ch, b) => [ch, b]));
    this.byteId = Int32Array.from(chars, (ch) => (this.ids.has(ch) ? this.ids.get(ch) : -1));

    // (left id, right id) -> [rank, merged id or -1]; the first rank of a pair counts
    this.pairs = new Map();
    this.mergedText = [];
    for (let r = 0; r < merges.length; r++) {
      const sp = merges[r].indexOf(" ");
      const a = this.ids.get(merges[r].slice(0, sp)), b = this.ids.get(merges[r].slice(sp + 1));
      if (a === undefined || b === undefined) continue;     // can never apply: its operands are no tokens
      const key = a * PAIR + b;
      if (this.pairs.has(key)) continue;
      const text = tokens[a] + tokens[b];
      this.pairs.set(key, [r, this.ids.has(text) ? this.ids.get(text) : -1]);
      this.mergedText[r] = text;
    }

    // literal tokens, grouped by first character, longest first
    const types = meta["tokenizer.ggml.token_type"] || [];
    this.literal = new Set();
    this.literalByFirst = new Map();
    for (let i = 0; i < types.length; i++) {
      if (types[i] !== TOKEN_CONTROL && types[i] !== TOKEN_USER_DEFINED) continue;
      this.literal.add(i);
      const t = tokens[i];
      if (!t) continue;
      if (!this.literalByFirst.has(t[0])) this.literalByFirst.set(t[0], []);
      this.literalByFirst.get(t[0]).push(t);
    }
    for (const list of this.literalByFirst.values()) list.sort((x, y) => y.length - x.length);

    this.memo = new Map();
    this.utf8 = new TextEncoder();
    this.byteCache = [];
  }

  // Ids of one pre-tokenized piece.
  pieceIds(piece) {
    const hit = this.memo.get(piece);
    if (hit !== undefined) return hit;
    const bytes = this.utf8.encode(piece);
    let seq = new Int32Array(bytes.length);
    for (let i = 0; i < bytes.length; i++) {
      seq[i] = this.byteId[bytes[i]];
      if (seq[i] < 0) throw new Error(`no token for byte ${bytes[i]}`);
    }
    let n = seq.length;
    while (n > 1) {
      let best = -1, rank = Infinity;
      for (let i = 0; i + 1 < n; i++) {
        const e = this.pairs.get(seq[i] * PAIR + seq[i + 1]);
        if (e !== undefined && e[0] < rank) { rank = e[0]; best = i; }
      }
      if (best < 0) break;
      const left = seq[best], right = seq[best + 1], merged = this.pairs.get(left * PAIR + right)[1];
      if (merged < 0) throw new Error(`no token for ${JSON.stringify(this.mergedText[rank])}`);
      let w = best;
      for (let i = best; i < n; i++, w++) {
        if (i + 1 < n && seq[i] === left && seq[i + 1] === right) { seq[w] = merged; i++; }
        else seq[w] = seq[i];
      }
      n = w;
    }
    const ids = Array.from(seq.subarray(0, n));
    if (this.memo.size >= MEMO_LIMIT) this.memo.clear();
    this.memo.set(piece, ids);
    return ids;
  }

  // Literal (special) tokens are matched first, longest at each position; the text between them is
  // pre-tokenized and merged.
  encode(text) {
    const s = text.normalize("NFC");
    const out = [];
    let plain = 0;
    const flush = (end) => {
      if (end > plain) for (const m of s.slice(plain, end).matchAll(SPLIT)) out.push(...this.pieceIds(m[0]));
    };
    for (let i = 0; i < s.length;) {
      const cands = this.literalByFirst.get(s[i]);
      const hit = cands ? cands.find((t) => s.startsWith(t, i)) : undefined;
      if (hit === undefined) { i++; continue; }
      flush(i);
      out.push(this.ids.get(hit));
      i += hit.length;
      plain = i;
    }
    flush(s.length);
    return out;
  }

  // The bytes a token stands for (a literal token: its text in UTF-8).
  tokenBytes(id) {
    let b = this.byteCache[id];
    if (b === undefined) {
      const t = this.tokens[id];
      if (this.literal.has(id)) b = this.utf8.encode(t);
      else b = Uint8Array.from(Array.from(t, (ch) => this.charByte.get(ch)));
      this.byteCache[id] = b;
    }
    return b;
  }

  decode(ids) {
    let total = 0;
    for (const id of ids) total += this.tokenBytes(id).length;
    const all = new Uint8Array(total);
    let at = 0;
    for (const id of ids) { const b = this.tokenBytes(id); all.set(b, at); at += b.length; }
    return new TextDecoder().decode(all);
  }

  // Incremental decoding: the bytes of a character split over tokens are held until it is whole.
  streamDecoder() {
    const td = new TextDecoder();
    return (id) => td.decode(this.tokenBytes(id), { stream: true });
  }
}

// ChatML as Qwen2.5's chat template renders plain-text messages, with its default system message
// when the conversation has none.
const DEFAULT_SYSTEM = "You are Qwen, created by Alibaba Cloud. You are a helpful assistant.";

function chatPrompt(messages, addGenerationPrompt = true) {
  const turns = messages.length && messages[0].role === "system" ? messages
    : [{ role: "system", content: DEFAULT_SYSTEM }].concat(messages);
  const parts = turns.map((m) => "<|im_start|>" + m.role + "\n" + m.content + "<|im_end|>\n");
  if (addGenerationPrompt) parts.push("<|im_start|>assistant\n");
  return parts.join("");
}

module.exports = { Tokenizer, chatPrompt, byteChars };
