'use strict';
// forward(prompt, 0, {diagnostic: true}) and logits(h, {diagnostic: true}) of
// a Node restatement of Gemma4WebGPU on a small checkpoint, collecting the
// logged lines.  With a fourth argument naming a BF16 tensor, that tensor
// reads back as NaN, and the first non-finite stage must be reported by a
// throw.
// argv: checkpoint.safetensors config.json [ops|engine] [nanTensor]
// Prints one JSON line: {lines, error}.
const fs = require('fs');
const rt = require('../../gemma4-js_amd/node/hip-runtime.js');
const { Gemma4Hip, Gemma4HipEngine } = require('../../gemma4-js_amd/node/gemma4-hip.js');

(async () => {
  const cfg = JSON.parse(fs.readFileSync(process.argv[3], 'utf8'));
  const device = await rt.requestDevice();
  const reader = await new rt.SafeFileReader(process.argv[2]).init();
  const nanName = process.argv[5];
  if (nanName) {
    const bf16 = reader.bf16.bind(reader);
    reader.bf16 = async (name) => {
      const v = await bf16(name);
      if (name === nanName) v[0] = NaN;
      return v;
    };
  }
  const Driver = process.argv[4] === 'engine' ? Gemma4HipEngine : Gemma4Hip;
  const lines = [];
  const model = new Driver(device, reader, {
    maxSeq: cfg.maxSeq, hidden: cfg.hidden, pleDim: cfg.pleDim, layers: cfg.specs.length,
    heads: cfg.heads, window: cfg.window, lmChunkRows: cfg.lmChunkRows,
    spec: (i) => cfg.specs[i], log: (s) => { if (s.startsWith('[diag') || s.startsWith('  ')) lines.push(s); },
  });
  await model.load();
  let error = null;
  try {
    const h = await model.forward(cfg.prompt, 0, { diagnostic: true });
    await model.logits(h, { diagnostic: true });
    h.destroy();
  } catch (e) { error = e.message; }
  model.dispose();
  reader.close();
  console.log(JSON.stringify({ lines, error }));
})().catch((e) => { console.error(e.stack || String(e)); process.exit(1); });
