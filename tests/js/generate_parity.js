'use strict';
// generate() on the small checkpoint with a toy tokenizer.
// argv: checkpoint.safetensors config.json tokenizer-dir [ops|engine]
// Runs, each from a reset cache:
//   step:      one greedy call per token (as main.js);
//   chunk:     (engine) the device decode loop in chunks of 5;
//   stop:      step, with the token at index k (the first token from index 2
//              on that did not occur before it) added to the stop ids;
//   stopChunk: (engine) the same in chunks of 4;
//   cap:       step with a KV capacity of prompt + 4.
// Prints one JSON line {k, runs: {name: result}}.
const fs = require('fs');
const rt = require('../../gemma4-js_amd/node/hip-runtime.js');
const { Gemma4Hip, Gemma4HipEngine } = require('../../gemma4-js_amd/node/gemma4-hip.js');
const { Gemma4Tokenizer } = require('../../gemma4-js_amd/node/tokenizer.js');
const { generate } = require('../../gemma4-js_amd/node/generate.js');

(async () => {
  const cfg = JSON.parse(fs.readFileSync(process.argv[3], 'utf8'));
  const engine = process.argv[5] === 'engine';
  const device = await rt.requestDevice();
  const reader = await new rt.SafeFileReader(process.argv[2]).init();
  const Driver = engine ? Gemma4HipEngine : Gemma4Hip;
  const model = new Driver(device, reader, {
    maxSeq: cfg.maxSeq, hidden: cfg.hidden, pleDim: cfg.pleDim, layers: cfg.specs.length,
    heads: cfg.heads, window: cfg.window, lmChunkRows: cfg.lmChunkRows,
    spec: (i) => cfg.specs[i],
  });
  await model.load();
  const tk = Gemma4Tokenizer.fromDirectorySync(process.argv[4]);
  const keep = (r) => ({
    rendered: r.rendered, inputIds: r.inputIds, generated: r.generated, text: r.text, rawText: r.rawText,
    stopReason: r.stopReason, stopTokenId: r.stopTokenId,
  });
  const opts = { maxNewTokens: cfg.genMax, maxSeq: cfg.maxSeq };
  const runs = {};
  runs.step = keep(await generate(model, tk, cfg.genPrompt, opts));
  if (engine) runs.chunk = keep(await generate(model, tk, cfg.genPrompt, Object.assign({ chunk: 5 }, opts)));
  const g = runs.step.generated;
  let k = -1;
  for (let i = 2; i < g.length; i++) if (g.indexOf(g[i]) === i) { k = i; break; }
  if (k >= 0) {
    const tk2 = new Gemma4Tokenizer(tk.json, tk.config, { eos_token_id: [g[k]] });
    runs.stop = keep(await generate(model, tk2, cfg.genPrompt, opts));
    if (engine) runs.stopChunk = keep(await generate(model, tk2, cfg.genPrompt, Object.assign({ chunk: 4 }, opts)));
  }
  const cap = runs.step.inputIds.length + 4;
  runs.cap = keep(await generate(model, tk, cfg.genPrompt, { maxNewTokens: cfg.genMax, maxSeq: cap }));
  model.dispose();
  reader.close();
  console.log(JSON.stringify({ k, runs }));
})().catch((e) => { console.error(e.stack || String(e)); process.exit(1); });
