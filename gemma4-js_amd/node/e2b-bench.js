'use strict';
// Random-init Gemma-4-E2B decode driven from Node through the N-API bridge.
//
// Same shapes and synthetic distributions as the Python benchmark: W4 q
// uniform in [-7, 7] with bf16 scales |N(0,1)| * 0.02, PLE table scales
// |N(0,1)| * 0.05, a bf16 N(0,1) * 0.03 tied embedding, norm weights uniform
// in [0.9, 1.1] and layer scalars 1.  Every large tensor is generated on the
// device.  A prompt of random ids is prefilled with engine.greedy, then
// engine.decode(steps) continues on the recorded one-token step (one graph
// replay per token, tokens kept on the device).
//
// usage: node e2b-bench.js [prompt=512] [steps=256] [maxSeq=1024] [seed=4]
// Prints one JSON line.

const rt = require('./hip-runtime.js');

const native = rt.native;
const U = rt.GPUBufferUsage;

// xorshift32: reproducible host-side draws (norm weights, prompt ids)
function rng(seed) {
  let s = (seed ^ 0x2545f491) >>> 0 || 1;
  return () => {
    s ^= s << 13; s >>>= 0;
    s ^= s >>> 17;
    s ^= s << 5; s >>>= 0;
    return s / 4294967296;
  };
}

function build(device, cfg, seed) {
  const H = cfg.hidden, P = cfg.pleDim, NL = cfg.layers.length, V = cfg.vocab;
  const engine = new native.GemmaEngine(cfg);
  const keep = [];
  const rand = rng(seed);
  let counter = seed * 1000;
  const nxt = () => ++counter;
  const buf = (bytes, label) => rt.createBuffer(device, bytes, U.STORAGE, label);

  const E = buf(V * H * 2, 'embed');
  native.fillRandom(E, V * H, native.RAND_BF16_NORMAL, nxt(), 0.03);
  engine.setEmbedding(E);
  keep.push(E);

  const width = NL * P, packedRow = width / 2, scaleRow = (width / 32) * 2;
  const ple = new native.PleTable(V, width, 32, 4096);
  let stage = null;
  for (let s = 0; ; s++) {
    let nbytes;
    try { nbytes = ple.shardBytes(s); } catch (e) { break; }
    const rows = nbytes / (packedRow + scaleRow);
    if (!stage || stage.size < nbytes) {
      if (stage) stage.destroy();
      stage = buf(nbytes, 'ple-stage');
    }
    native.fillRandom(stage, rows * packedRow, native.RAND_PLE_PACKED, nxt());
    native.fillRandom(stage, rows * (width / 32), native.RAND_BF16_ABS_NORMAL, nxt(), 0.05, rows * packedRow);
    ple.uploadShard(s, stage);
  }
  if (stage) stage.destroy();
  engine.setPle(ple);
  keep.push(ple);

  const lin = (layer, which, n, k) => {
    const pk = buf(n * k / 2, 'packed'), sc = buf(n * (k / 32) * 2, 'scales');
    native.fillRandom(pk, n * k / 8, native.RAND_W4_PACKED, nxt());
    native.fillRandom(sc, n * (k / 32), native.RAND_BF16_ABS_NORMAL, nxt(), 0.02);
    const w = new native.W4Weight(pk, sc, n, k, 32);
    pk.destroy();
    sc.destroy();
    engine.setLinear(layer, which, w);
    keep.push(w);
  };
  const norm = (layer, which, n) => {
    const v = new Float32Array(n);
    for (let i = 0; i < n; i++) v[i] = 0.9 + 0.2 * rand();
    engine.setNorm(layer, which, v);
  };
  // engine indices (include/g4hip.h G4_PROJ_* / G4_NORM_*)
  lin(-1, 9, NL * P, H);
  norm(-1, 7, P);
  norm(-1, 8, H);
  for (let i = 0; i < NL; i++) {
    const L = cfg.layers[i], hd = L.headDim, shared = L.kvSource >= 0;
    lin(i, 0, cfg.heads * hd, H);
    if (!shared) {
      lin(i, 1, hd, H);
      lin(i, 2, hd, H);
    }
    lin(i, 3, H, cfg.heads * hd);
    lin(i, 4, L.intermediate, H);
    lin(i, 5, L.intermediate, H);
    lin(i, 6, H, L.intermediate);
    lin(i, 7, P, H);
    lin(i, 8, H, P);
    for (let n = 0; n < 5; n++) norm(i, n, H);
    norm(i, 5, hd);
    if (!shared) norm(i, 6, hd);
    engine.setLayerScalar(i, 1.0);
  }
  return { engine, keep, rand };
}

function main() {
  const [prompt, steps, maxSeq, seed] = [512, 256, 1024, 4].map((d, i) => {
    const v = process.argv[2 + i];
    return v === undefined ? d : Number(v);
  });
  const device = rt.requestDevice(0);
  const cfg = native.e2bConfig(maxSeq);
  const { engine, keep, rand } = build(device, cfg, seed);
  const ids = new Int32Array(prompt);
  for (let i = 0; i < prompt; i++) ids[i] = Math.floor(rand() * cfg.vocab);

  engine.greedy(ids, 0);
  engine.decode(4);  // records the decode step
  engine.reset();
  const t0 = process.hrtime.bigint();
  const first = engine.greedy(ids, 0);  // prefill + head + argmax (synchronises)
  const t1 = process.hrtime.bigint();
  const toks = engine.decode(steps);    // returns after the last token is read back
  const t2 = process.hrtime.bigint();
  const prefillMs = Number(t1 - t0) / 1e6, decodeMs = Number(t2 - t1) / 1e6;
  engine.dispose();
  for (const k of keep) (k.dispose ? k.dispose() : k.destroy());
  console.log(JSON.stringify({
    driver: 'node', prompt, steps, max_seq: maxSeq,
    prefill_ms: prefillMs, prefill_tok_s: prompt / (prefillMs / 1e3),
    decode_ms: decodeMs, ms_per_token: decodeMs / steps, decode_tok_s: steps / (decodeMs / 1e3),
    first_token: first, last_token: toks[toks.length - 1],
  }));
}

main();
