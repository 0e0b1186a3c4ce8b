"use strict";
// Test driver for the Node.js host (engine/*.js): one command per run, JSON on stdout.
//   parse <gguf>                                   -> {cfg, tensors}
//   load <gguf> <ctx>                              -> {ok} or {error, code}
//   generate <gguf> <ctx> <ids.json> <steps> <logits.f32>
//        -> {tokens (per-step forward loop), device (device loop), stats}; last logits written raw
//   sample <logits.f32> <temperature> <seed>      -> {id}
//   samples <cases.json>                           -> [id] for [{logits (path to raw f32), temperature, seed, pos}]
//   tokenize <meta.json> <texts.json>              -> {ids, text, pieces} per text (tokenizer alone)
//   chat <gguf> <ctx> <turns.json> <maxTokens>     -> per turn {pieces, ids, prompt, stats}
//   batch <gguf> <ctx> <prompts.json> <steps> <logits.f32> <kvDtype>
//        -> {first, tokens (per sequence), afterDestroy}; the batch's last logits written raw
//   setkv <gguf> <ctx> <kv.f32> <positions> <first> <steps> <kvDtype>
//        -> {modes: {graph|persistent: {tokens, used}}} after the cache [K|V][layer][kvHead][pos][hd]
//           is written through setKv
const fs = require("fs");
const path = require("path");
const engine = path.join(__dirname, "..", "..", "e2e-browser-voice-agent_amd", "engine");
const { parseGGUF, qwen2Config, readModel } = require(path.join(engine, "gguf.js"));
const { LLM } = require(path.join(engine, "llm.js"));
const { sample, sampleAt } = require(path.join(engine, "hip.js"));
const { Tokenizer, chatPrompt } = require(path.join(engine, "tokenizer.js"));

async function main() {
  const [cmd, ...args] = process.argv.slice(2);
  if (cmd === "parse") {
    const g = parseGGUF(readModel(args[0]));
    const tensors = {};
    for (const [n, t] of Object.entries(g.tensors)) tensors[n] = [t.type, t.shape, t.start, t.bytes];
    return { cfg: qwen2Config(g.meta), version: g.version, dataStart: g.dataStart, tensors };
  }
  if (cmd === "load") {
    try {
      const llm = await LLM.load({ path: args[0], ctx: Number(args[1]) });
      llm.destroy();
      return { ok: true };
    } catch (e) {
      return { error: String(e.message), code: e.code === undefined ? null : e.code };
    }
  }
  if (cmd === "generate") {
    const ids = JSON.parse(fs.readFileSync(args[2], "utf8"));
    const steps = Number(args[3]);
    const llm = await LLM.load({ path: args[0], ctx: Number(args[1]) });
    const tokens = await llm.generateIds(ids, steps);
    const stats = llm.stats;
    const lg = await llm.be.readLogits();
    fs.writeFileSync(args[4], Buffer.from(lg.buffer));
    const device = await llm.generateIdsDevice(ids, steps);
    let ctxError = null;
    try { await llm.be.forward([1], llm.be.ctx - 1); } catch (e) { ctxError = e.message; }
    llm.destroy();
    return { tokens, device, stats, deviceStats: llm.stats, ctxError };
  }
  if (cmd === "sample") {
    const b = fs.readFileSync(args[0]);
    const lg = new Float32Array(b.buffer, b.byteOffset, b.length / 4);
    return { id: sample(lg, Number(args[1]), Number(args[2]) >>> 0) };
  }
  if (cmd === "samples") {
    const cases = JSON.parse(fs.readFileSync(args[0], "utf8"));
    return cases.map((c) => {
      const b = fs.readFileSync(c.logits);
      const lg = new Float32Array(b.buffer, b.byteOffset, b.length / 4);
      return sampleAt(lg, c.temperature, c.seed, c.pos);
    });
  }
  if (cmd === "tokenize") {
    const tok = new Tokenizer(JSON.parse(fs.readFileSync(args[0], "utf8")));
    const texts = JSON.parse(fs.readFileSync(args[1], "utf8"));
    return texts.map((t) => {
      const ids = tok.encode(t);
      const dec = tok.streamDecoder();
      return { ids, text: tok.decode(ids), pieces: ids.map((id) => dec(id)) };
    });
  }
  if (cmd === "chat") {
    const turns = JSON.parse(fs.readFileSync(args[2], "utf8"));
    const maxTokens = Number(args[3]);
    const llm = await LLM.load({ path: args[0], ctx: Number(args[1]) });
    const out = [];
    const history = [];
    for (const user of turns) {
      history.push({ role: "user", content: user });
      const prompt = llm.tok.encode(chatPrompt(history));
      const pieces = [];
      for await (const p of llm.chat(history, { maxTokens, temperature: 0 })) pieces.push(p);
      out.push({ pieces, ids: llm.stats.ids, text: llm.tok.decode(llm.stats.ids), prompt, stats: llm.stats });
      history.push({ role: "assistant", content: pieces.join("") });
    }
    llm.destroy();
    return out;
  }
  if (cmd === "batch") {
    const prompts = JSON.parse(fs.readFileSync(args[2], "utf8"));
    const steps = Number(args[3]);
    const llm = await LLM.load({ path: args[0], ctx: Number(args[1]), kvDtype: args[5] });
    const bt = llm.be.createBatch(prompts.length);
    const first = [];
    for (let b = 0; b < prompts.length; b++) first.push(await bt.prefill(b, prompts[b], 0));
    const tokens = await bt.generate(first, prompts.map((p) => p.length), steps);
    const lg = await bt.readLogits();
    fs.writeFileSync(args[4], Buffer.from(lg.buffer));
    llm.destroy();                     // releases the batch too
    let afterDestroy = null;
    try { await bt.generate(first, prompts.map((p) => p.length), 1); } catch (e) { afterDestroy = e.message; }
    return { first, tokens, afterDestroy };
  }
  if (cmd === "setkv") {
    const b = fs.readFileSync(args[2]);
    const kv = new Float32Array(b.buffer, b.byteOffset, b.length / 4);
    const P = Number(args[3]), first = Number(args[4]), steps = Number(args[5]);
    const llm = await LLM.load({ path: args[0], ctx: Number(args[1]), kvDtype: args[6] });
    const { layers, kvHeads, dim, heads } = llm.cfg;
    const hd = dim / heads, block = P * hd, half = layers * kvHeads * block;
    for (let l = 0; l < layers; l++) {
      for (let kh = 0; kh < kvHeads; kh++) {
        const at = (l * kvHeads + kh) * block;
        llm.be.setKv(l, kh, 0, kv.subarray(at, at + block), kv.subarray(half + at, half + at + block));
      }
    }
    const modes = {};
    for (const mode of ["graph", "persistent"]) {
      llm.be.setDecodeMode(mode);
      const tokens = await llm.be.generate(first, P, steps);
      modes[mode] = { tokens, used: llm.be.decodeModeUsed() };
    }
    llm.destroy();
    return { modes };
  }
  throw new Error(`unknown command ${cmd}`);
}

main().then((r) => { process.stdout.write(JSON.stringify(r) + "\n"); },
  (e) => { process.stderr.write(String(e && e.stack || e) + "\n"); process.exit(1); });
