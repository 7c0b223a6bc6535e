'use strict';
// Runs a Node restatement of Gemma4WebGPU on a small checkpoint: greedy on a
// prompt, then `steps` one-token greedy calls.  Driver "ops" is Gemma4Hip
// (one GPUOps call per op); "engine" is Gemma4HipEngine (the native engine),
// which also replays the prompt and decodes `steps` tokens on its recorded
// decode step.
// argv: checkpoint.safetensors config.json [ops|engine]
// Prints one JSON line: {tokens, logits0, cache, appendError[, decoded]}.
const fs = require('fs');
const rt = require('../../gemma4-js_amd/node/hip-runtime.js');
const { Gemma4Hip, Gemma4HipEngine } = require('../../gemma4-js_amd/node/gemma4-hip.js');

(async () => {
  const cfg = JSON.parse(fs.readFileSync(process.argv[3], 'utf8'));
  const device = await rt.requestDevice();
  const reader = await new rt.SafeFileReader(process.argv[2]).init();
  const engine = process.argv[4] === 'engine';
  const Driver = engine ? Gemma4HipEngine : Gemma4Hip;
  const model = new Driver(device, reader, {
    maxSeq: cfg.maxSeq, hidden: cfg.hidden, pleDim: cfg.pleDim, layers: cfg.specs.length,
    heads: cfg.heads, window: cfg.window, lmChunkRows: cfg.lmChunkRows,
    spec: (i) => cfg.specs[i],
  });
  await model.load();
  const first = await model.greedy(cfg.prompt, 0);
  const tokens = [first.nextTokenId];
  let pos = cfg.prompt.length;
  for (let s = 0; s < cfg.steps; s++) {
    const r = await model.greedy([tokens[tokens.length - 1]], pos);
    tokens.push(r.nextTokenId);
    pos += 1;
  }
  const cache = model.cacheSummary();
  let err = null;
  try { await model.forward([1], pos + 5); } catch (e) { err = e.message; }
  let decoded;
  if (engine) {
    model.resetCache();
    await model.greedy(cfg.prompt, 0);
    decoded = Array.from(model.decode(cfg.steps));
  }
  model.dispose();
  reader.close();
  console.log(JSON.stringify({ tokens, logits0: Array.from(first.logits), cache, appendError: err, decoded }));
})().catch((e) => { console.error(e.stack || String(e)); process.exit(1); });
