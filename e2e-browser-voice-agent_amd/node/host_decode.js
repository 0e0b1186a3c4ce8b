"use strict";
// Decode through the Node.js host as an application drives it: LLM.load of a GGUF file, then
// generateIds, one backend forward() call (one N-API call, one decode step) per token.
//
//   node host_decode.js <model.gguf> <ctx> <ids.json> <steps>
//
// Prints one JSON line: the tokens, the host-side milliseconds of every decode call (stats.stepMs)
// and their median, the time to the first token, and the decode path the steps took.
const fs = require("fs");
const path = require("path");
const { LLM } = require(path.join(__dirname, "..", "engine", "llm.js"));

async function main() {
  const [file, ctx, idsPath, steps] = process.argv.slice(2);
  const ids = JSON.parse(fs.readFileSync(idsPath, "utf8"));
  const llm = await LLM.load({ path: file, ctx: Number(ctx) });
  const tokens = await llm.generateIds(ids, Number(steps));
  const ms = llm.stats.stepMs.slice().sort((a, b) => a - b);
  const median = ms.length ? (ms[(ms.length - 1) >> 1] + ms[ms.length >> 1]) / 2 : null;
  const out = { tokens, stepMs: llm.stats.stepMs, medianStepMs: median, firstTokenMs: llm.stats.firstTokenMs,
    decodePath: llm.be.decodeModeUsed(), loadMs: llm.loadTimes };
  llm.destroy();
  return out;
}

main().then((r) => { process.stdout.write(JSON.stringify(r) + "\n"); },
  (e) => { process.stderr.write(String(e && e.stack || e) + "\n"); process.exit(1); });
