'use strict';
// Gemma4WebGPU (custom-webgpu/gemma4-webgpu.js:139-502) for Node 12 on the HIP
// path: the same load / forward / logits / greedy surface and the same op
// sequence per layer (encodeLayer, gemma4-webgpu.js:215-301), driven through
// hip-runtime.js's GPUOps instead of WebGPU.  The reference module cannot be
// loaded by Node 12 (ES modules, optional chaining), so the driver is
// restated here; the checkpoint reader, PLE bundle and ops keep the
// reference's interfaces.
//
// Geometry: the reference fixes HIDDEN 1536, PLE 256, LAYERS 35, HEADS 8 and
// the E2B layer schedule spec(i) (gemma4-webgpu.js:12, 65-77).  They are the
// defaults here; options override them (used to run small checkpoints of the
// same layout).

const rt = require('./hip-runtime.js');

const U = rt.GPUBufferUsage;

// encodeLayer's probe names (gemma4-webgpu.js:224-309), the order of the
// engine's diagnostic stage buffers (G4_STAGE_*)
const STAGE_NAMES = ['preAttention', 'qRaw', 'qNormRoPE', 'kRaw', 'vRaw', 'kNormRoPE', 'vNorm',
  'attentionContext', 'attentionOutput', 'postAttentionNorm', 'attentionResidual', 'preFfw',
  'mlpGate', 'mlpUp', 'mlpActivated', 'ffwOutput', 'postFfwNorm', 'ffwResidual', 'pleGate',
  'pleModulated', 'pleProjected', 'pleNormalized', 'output'];

// spec(i) of gemma4-webgpu.js:65-77: every 5th layer global (head_dim 512,
// RoPE base 1e6 on a quarter of the pairs), intermediate 12288 from layer 15,
// layers >= 15 reuse the KV caches of layers 13 (sliding) and 14 (global).
function e2bSpec(i) {
  const full = (i + 1) % 5 === 0;
  return {
    full,
    headDim: full ? 512 : 256,
    intermediate: i < 15 ? 6144 : 12288,
    shared: i >= 15,
    storeShared: i === 13 || i === 14,
    attentionType: full ? 'full' : 'sliding',
    ropeBase: full ? 1000000 : 10000,
    ropeProp: full ? 0.25 : 1.0,
  };
}

function layerNames(i, s) {
  const root = `model.language_model.layers.${i}`;
  const names = {
    q: `${root}.self_attn.q_proj`, o: `${root}.self_attn.o_proj`,
    gate: `${root}.mlp.gate_proj`, up: `${root}.mlp.up_proj`, down: `${root}.mlp.down_proj`,
    pleGate: `${root}.per_layer_input_gate`, pleProj: `${root}.per_layer_projection`,
  };
  if (!s.shared) {
    names.k = `${root}.self_attn.k_proj`;
    names.v = `${root}.self_attn.v_proj`;
  }
  return names;
}

// The diagnostic statistics of gemma4-webgpu.js:15-63: counts of finite, NaN
// and infinite values, and min / max / mean / std of the finite ones.
function finiteStats(a) {
  let finite = 0, nan = 0, inf = 0, min = Infinity, max = -Infinity, sum = 0, sumSq = 0;
  for (let i = 0; i < a.length; i++) {
    const v = a[i];
    if (Number.isNaN(v)) { nan++; continue; }
    if (!Number.isFinite(v)) { inf++; continue; }
    finite++;
    if (v < min) min = v;
    if (v > max) max = v;
    sum += v;
    sumSq += v * v;
  }
  const mean = finite > 0 ? sum / finite : NaN;
  const variance = finite > 0 ? Math.max(0, sumSq / finite - mean * mean) : NaN;
  return {
    count: a.length, finite, nan, inf,
    min: finite > 0 ? min : NaN, max: finite > 0 ? max : NaN,
    mean, std: Number.isFinite(variance) ? Math.sqrt(variance) : NaN,
  };
}

function formatStats(s) {
  const e = (x) => Number(x).toExponential(3);
  return `finite=${s.finite}/${s.count} nan=${s.nan} inf=${s.inf} ` +
    `min=${e(s.min)} max=${e(s.max)} mean=${e(s.mean)} std=${e(s.std)}`;
}

// forward's diagnostic lines for the layer-1 stages and a layer's hidden
// state (gemma4-webgpu.js:342-372, 376-389); both throw at the first
// non-finite value, as the reference does.
function logStages(log, probes) {
  log('[diag layer 01 stages]');
  for (const p of probes) {
    const stats = finiteStats(p.values);
    log(`  ${p.name.padEnd(20)} ${formatStats(stats)}`);
    if (stats.nan > 0 || stats.inf > 0) throw new Error(`First non-finite Layer 1 stage: ${p.name}.`);
  }
}

function logLayer(log, i, values) {
  const stats = finiteStats(values);
  log(`[diag layer ${String(i).padStart(2, '0')}] ` + formatStats(stats));
  if (stats.nan > 0 || stats.inf > 0) {
    throw new Error(`First non-finite hidden state detected at layer ${i}.`);
  }
}

// logits' diagnostic lines (gemma4-webgpu.js:419-428)
function logLogits(log, out) {
  log(`[diag logits] ${formatStats(finiteStats(out))}`);
  log('[diag logits first 16] ' + Array.from(out.slice(0, 16)).map((x) => Number(x).toExponential(4)).join(' '));
}

async function scaleBuffer(device, reader, name) {
  return rt.uploadF32(device, await reader.bf16(name), U.STORAGE, name);
}

// KVCache (gemma4-webgpu.js:117-137): appends with copyBufferToBuffer.
class KVCache {
  constructor(device, headDim, maxSeq, label) {
    this.headDim = headDim;
    this.maxSeq = maxSeq;
    this.length = 0;
    this.k = rt.createBuffer(device, maxSeq * headDim * 4, U.STORAGE | U.COPY_DST | U.COPY_SRC, `${label}:k`);
    this.v = rt.createBuffer(device, maxSeq * headDim * 4, U.STORAGE | U.COPY_DST | U.COPY_SRC, `${label}:v`);
  }
  append(encoder, kNew, vNew, rows, startPos) {
    if (startPos !== this.length) throw new Error(`KV append position ${startPos} != cache length ${this.length}`);
    if (startPos + rows > this.maxSeq) throw new Error(`KV cache capacity ${this.maxSeq} exceeded`);
    const off = startPos * this.headDim * 4, bytes = rows * this.headDim * 4;
    encoder.copyBufferToBuffer(kNew, 0, this.k, off, bytes);
    encoder.copyBufferToBuffer(vNew, 0, this.v, off, bytes);
    this.length += rows;
  }
  dispose() { this.k.destroy(); this.v.destroy(); }
}

class Gemma4Hip {
  // reader: SafeFileReader over the CORE checkpoint (plus pleRowsToGpu when a
  // W4 PLE bundle is attached, as the distribution reader has).
  constructor(device, reader, opts = {}) {
    this.device = device;
    this.reader = reader;
    this.maxSeq = opts.maxSeq || 512;
    this.lmChunkRows = opts.lmChunkRows || 4096;
    this.log = opts.log || (() => {});
    this.hidden = opts.hidden || 1536;
    this.pleDim = opts.pleDim || 256;
    this.numLayers = opts.layers || 35;
    this.heads = opts.heads || 8;
    this.window = opts.window || 512;
    this.spec = opts.spec || e2bSpec;
    this.ops = new rt.GPUOps(device, { pleWidth: this.pleDim, pleLayers: this.numLayers });
    this.layers = [];
    this.caches = [];
    this.shared = {};
    this.lmChunks = [];
    this.loaded = false;
  }

  async loadLayer(i) {
    const root = `model.language_model.layers.${i}`, s = this.spec(i), reader = this.reader;
    const linear = {};
    const names = layerNames(i, s);
    for (const key of Object.keys(names)) {
      linear[key] = await rt.GPUW4Linear.load(this.device, reader, names[key]);
    }
    const norm = {
      input: await scaleBuffer(this.device, reader, `${root}.input_layernorm.weight`),
      postAttn: await scaleBuffer(this.device, reader, `${root}.post_attention_layernorm.weight`),
      preFfw: await scaleBuffer(this.device, reader, `${root}.pre_feedforward_layernorm.weight`),
      postFfw: await scaleBuffer(this.device, reader, `${root}.post_feedforward_layernorm.weight`),
      postPle: await scaleBuffer(this.device, reader, `${root}.post_per_layer_input_norm.weight`),
      q: await scaleBuffer(this.device, reader, `${root}.self_attn.q_norm.weight`),
      k: s.shared ? null : await scaleBuffer(this.device, reader, `${root}.self_attn.k_norm.weight`),
    };
    const skipScale = await reader.scalarBF16(`${root}.layer_scalar`);
    return { i, s, linear, norm, skipScale };
  }

  // load() (gemma4-webgpu.js:150-189)
  async load() {
    this.log('Loading top-level W4A16 projection...');
    this.topProj = await rt.GPUW4Linear.load(this.device, this.reader, 'model.language_model.per_layer_model_projection');
    this.pleNorm = await scaleBuffer(this.device, this.reader, 'model.language_model.per_layer_projection_norm.weight');
    this.finalNorm = await scaleBuffer(this.device, this.reader, 'model.language_model.norm.weight');
    this.log(`Loading ${this.numLayers} quantized transformer layers...`);
    for (let i = 0; i < this.numLayers; i++) {
      const layer = await this.loadLayer(i);
      this.layers.push(layer);
      this.caches[i] = layer.s.shared ? null : new KVCache(this.device, layer.s.headDim, this.maxSeq, `layer${i}`);
    }
    this.log('Loading tied BF16 LM-head embedding in device chunks...');
    const info = this.reader.info('model.language_model.embed_tokens.weight');
    this.vocab = info.shape[0];
    const width = info.shape[1], rowBytes = width * 2;
    if (width !== this.hidden) throw new Error(`embedding width ${width} != hidden ${this.hidden}`);
    for (let start = 0; start < this.vocab; start += this.lmChunkRows) {
      const rows = Math.min(this.lmChunkRows, this.vocab - start);
      const ab = await this.reader.rangeInTensor('model.language_model.embed_tokens.weight', start * rowBytes, rows * rowBytes);
      this.lmChunks.push({ start, rows, buffer: rt.uploadBytes(this.device, new Uint8Array(ab), U.STORAGE | U.COPY_DST, `lm-head:${start}`) });
    }
    this.loaded = true;
    this.log('Device model preload complete.');
  }

  resetCache() {
    for (const c of this.caches) if (c) c.length = 0;
    this.shared = {};
  }

  // inputBuffers (gemma4-webgpu.js:198-215)
  async inputBuffers(tokenIds) {
    const embed = await this.reader.bf16Rows('model.language_model.embed_tokens.weight', tokenIds);
    let ple;
    if (typeof this.reader.pleRowsToGpu === 'function') {
      ple = await this.reader.pleRowsToGpu(this.device, tokenIds);
    } else {
      ple = rt.uploadF32(this.device, await this.reader.bf16Rows('model.language_model.embed_tokens_per_layer.weight', tokenIds), U.STORAGE, 'token-ple');
    }
    return { embed: rt.uploadF32(this.device, embed, U.STORAGE, 'token-embed'), ple };
  }

  // encodeLayer (gemma4-webgpu.js:215-301): one decoder layer, every op output
  // a fresh buffer that goes on `garbage` once consumed.  With `probes` (an
  // array) each stage's buffer is listed under the reference's probe name.
  encodeLayer(encoder, layer, hidden, perLayer, rows, startPos, garbage, probes = null) {
    const ops = this.ops, s = layer.s, L = layer.linear, N = layer.norm, H = this.hidden;
    const nHidden = rows * H, QD = rows * this.heads * s.headDim;
    const trash = (x) => { if (x) garbage.push(x); return x; };
    const probe = (name, buffer, count) => {
      if (probes) probes.push({ name, buffer, count });
      return buffer;
    };
    const pre = probe('preAttention', ops.rms(encoder, hidden, rows, H, N.input, garbage), nHidden);
    const [qRaw, kRaw, vRaw] = ops.w4Multi(encoder, s.shared ? [L.q] : [L.q, L.k, L.v], pre, rows, garbage);
    probe('qRaw', qRaw, QD);
    const q = probe('qNormRoPE', ops.normRope(encoder, trash(qRaw), rows, this.heads, s.headDim, startPos, N.q, s.ropeProp, s.ropeBase, garbage), QD);
    let cache;
    if (s.shared) {
      cache = this.shared[s.attentionType];
      if (!cache) throw new Error(`Missing shared ${s.attentionType} KV cache at layer ${layer.i}`);
    } else {
      probe('kRaw', kRaw, rows * s.headDim);
      probe('vRaw', vRaw, rows * s.headDim);
      const k = probe('kNormRoPE', ops.normRope(encoder, trash(kRaw), rows, 1, s.headDim, startPos, N.k, s.ropeProp, s.ropeBase, garbage), rows * s.headDim);
      const v = probe('vNorm', ops.rms(encoder, trash(vRaw), rows, s.headDim, null, garbage), rows * s.headDim);
      cache = this.caches[layer.i];
      cache.append(encoder, k, v, rows, startPos);
      trash(k);
      trash(v);
      if (s.storeShared) this.shared[s.attentionType] = cache;
    }
    trash(pre);
    const context = probe('attentionContext', trash(ops.attention(encoder, q, cache.k, cache.v, rows, this.heads, s.headDim, startPos + rows, startPos, !s.full, this.window, garbage)), QD);
    trash(q);
    const attnProj = probe('attentionOutput', trash(ops.w4(encoder, L.o, context, rows, garbage)), nHidden);
    const attnNorm = probe('postAttentionNorm', trash(ops.rms(encoder, attnProj, rows, H, N.postAttn, garbage)), nHidden);
    const attnResidual = probe('attentionResidual', ops.addScale(encoder, hidden, attnNorm, nHidden, 1, garbage), nHidden);
    trash(hidden);
    const preFfw = probe('preFfw', trash(ops.rms(encoder, attnResidual, rows, H, N.preFfw, garbage)), nHidden);
    const [gate, up] = ops.w4Multi(encoder, [L.gate, L.up], preFfw, rows, garbage).map(trash);
    probe('mlpGate', gate, rows * s.intermediate);
    probe('mlpUp', up, rows * s.intermediate);
    const act = probe('mlpActivated', trash(ops.geluMul(encoder, gate, up, rows * s.intermediate, garbage)), rows * s.intermediate);
    const down = probe('ffwOutput', trash(ops.w4(encoder, L.down, act, rows, garbage)), nHidden);
    const ffwNorm = probe('postFfwNorm', trash(ops.rms(encoder, down, rows, H, N.postFfw, garbage)), nHidden);
    const ffwResidual = probe('ffwResidual', trash(ops.addScale(encoder, attnResidual, ffwNorm, nHidden, 1, garbage)), nHidden);
    trash(attnResidual);
    const pg = probe('pleGate', trash(ops.w4(encoder, L.pleGate, ffwResidual, rows, garbage)), rows * this.pleDim);
    const pm = probe('pleModulated', trash(ops.geluPle(encoder, pg, perLayer, rows, layer.i, garbage)), rows * this.pleDim);
    const pp = probe('pleProjected', trash(ops.w4(encoder, L.pleProj, pm, rows, garbage)), nHidden);
    const pn = probe('pleNormalized', trash(ops.rms(encoder, pp, rows, H, N.postPle, garbage)), nHidden);
    return probe('output', ops.addScale(encoder, ffwResidual, pn, nHidden, layer.skipScale, garbage), nHidden);
  }

  // forward (gemma4-webgpu.js:303-402); returns the final-norm last row [hidden].
  // With {diagnostic: true} it logs the statistics of the top-level hidden
  // and PLE rows, of every layer-1 stage and of every layer's hidden state,
  // and throws at the first non-finite one.
  async forward(tokenIds, startPos, { diagnostic = false } = {}) {
    if (!this.loaded) throw new Error('Model not loaded.');
    const rows = tokenIds.length, H = this.hidden, P = this.pleDim, NL = this.numLayers;
    const inp = await this.inputBuffers(tokenIds);
    let encoder = this.device.createCommandEncoder();
    let garbage = [];
    let hidden = this.ops.scale(encoder, inp.embed, rows * H, Math.sqrt(H), garbage);
    const projected = this.ops.w4(encoder, this.topProj, hidden, rows, garbage);
    const projectedScaled = this.ops.scale(encoder, projected, rows * NL * P, 1 / Math.sqrt(H), garbage);
    const perLayer = this.ops.pleMix(encoder, projectedScaled, this.pleNorm, inp.ple, rows, garbage);
    garbage.push(inp.embed, inp.ple, projected, projectedScaled);
    this.device.queue.submit([encoder.finish()]);
    for (const b of garbage) b.destroy();
    if (diagnostic) {
      this.log(`[diag top hidden] ${formatStats(finiteStats(await rt.readF32(this.device, hidden, rows * H)))}`);
      this.log(`[diag top PLE]    ${formatStats(finiteStats(await rt.readF32(this.device, perLayer, rows * NL * P)))}`);
    }
    try {
      for (const layer of this.layers) {
        encoder = this.device.createCommandEncoder();
        garbage = [];
        const stageProbes = diagnostic && layer.i === 1 ? [] : null;
        hidden = this.encodeLayer(encoder, layer, hidden, perLayer, rows, startPos, garbage, stageProbes);
        this.device.queue.submit([encoder.finish()]);
        try {
          if (stageProbes) {
            for (const p of stageProbes) p.values = await rt.readF32(this.device, p.buffer, p.count);
            logStages(this.log, stageProbes);
          }
        } finally {
          for (const b of garbage) b.destroy();
        }
        if (diagnostic) logLayer(this.log, layer.i, await rt.readF32(this.device, hidden, rows * H));
      }
    } catch (e) {
      // a diagnostic stop: the live hidden state and PLE rows go too
      hidden.destroy();
      perLayer.destroy();
      throw e;
    }
    perLayer.destroy();
    encoder = this.device.createCommandEncoder();
    garbage = [];
    const final = this.ops.rms(encoder, hidden, rows, H, this.finalNorm, garbage);
    const last = this.ops.emptyF32(H, 'last-hidden');
    encoder.copyBufferToBuffer(final, (rows - 1) * H * 4, last, 0, H * 4);
    garbage.push(hidden, final);
    this.device.queue.submit([encoder.finish()]);
    for (const b of garbage) b.destroy();
    return last;
  }

  // logits (gemma4-webgpu.js:404-431); {diagnostic: true} logs their statistics
  // and the first 16 values
  async logits(lastHidden, { diagnostic = false } = {}) {
    const logits = this.ops.emptyF32(this.vocab, 'logits');
    const encoder = this.device.createCommandEncoder();
    for (const c of this.lmChunks) this.ops.headChunk(encoder, lastHidden, c.buffer, logits, c.start, c.rows, null, this.hidden);
    this.device.queue.submit([encoder.finish()]);
    const out = await rt.readF32(this.device, logits, this.vocab);
    logits.destroy();
    if (diagnostic) logLogits(this.log, out);
    return out;
  }

  // greedy (gemma4-webgpu.js:441-481)
  async greedy(tokenIds, startPos) {
    const h = await this.forward(tokenIds, startPos);
    const l = await this.logits(h);
    h.destroy();
    let finite = 0;
    for (let i = 0; i < l.length; i++) if (Number.isFinite(l[i])) finite++;
    if (finite !== l.length) throw new Error(`Non-finite logits: ${l.length - finite}/${l.length}`);
    const top10 = rt.topK(l, 10);
    return { logits: l, top10, nextTokenId: top10[0].tokenId };
  }

  cacheSummary() {
    let bytes = 0, caches = 0;
    for (const c of this.caches) if (c) { caches++; bytes += c.length * c.headDim * 4 * 2; }
    return { caches, bytes };
  }

  dispose() {
    if (this.topProj) this.topProj.dispose();
    if (this.pleNorm) this.pleNorm.destroy();
    if (this.finalNorm) this.finalNorm.destroy();
    for (const l of this.layers) {
      for (const x of Object.values(l.linear)) x.dispose();
      for (const x of Object.values(l.norm)) if (x) x.destroy();
    }
    for (const c of this.caches) if (c) c.dispose();
    for (const c of this.lmChunks) c.buffer.destroy();
    this.ops.dispose();
  }
}

// Engine indices of the projections and norms (include/g4hip.h G4_PROJ_* /
// G4_NORM_*).
const PROJ = { q: 0, k: 1, v: 2, o: 3, gate: 4, up: 5, down: 6, pleGate: 7, pleProj: 8, top: 9 };
const NORM = {
  input: 0, postAttn: 1, preFfw: 2, postFfw: 3, postPle: 4, q: 5, k: 6, pleProjection: 7, final: 8,
};

// Gemma4WebGPU's surface (gemma4-webgpu.js:139-481) on the native decoder
// engine (g4_gemma_*): load / resetCache / forward / logits / greedy keep the
// reference's meaning and return values, and each runs as one C-ABI call
// instead of one GPUOps dispatch per op.  decode(steps) continues a greedy
// generation on the engine's recorded decode step (one HIP graph replay per
// token, no host round trip), returning the chosen token ids.
class Gemma4HipEngine {
  constructor(device, reader, opts = {}) {
    this.device = device;
    this.reader = reader;
    this.maxSeq = opts.maxSeq || 512;
    this.lmChunkRows = opts.lmChunkRows || 4096;
    this.log = opts.log || (() => {});
    this.hidden = opts.hidden || 1536;
    this.pleDim = opts.pleDim || 256;
    this.numLayers = opts.layers || 35;
    this.heads = opts.heads || 8;
    this.window = opts.window || 512;
    this.spec = opts.spec || e2bSpec;
    this.engine = null;
    this.owned = [];   // W4 weights and device buffers the engine borrows
    this.vocab = 0;
    this.loaded = false;
  }

  // Layer specs as the engine takes them: a shared-KV layer reads the cache of
  // the last earlier layer that stores its attention type (encodeLayer's
  // this.shared[attentionType], gemma4-webgpu.js:228-240).
  engineLayers() {
    const out = [], store = {};
    for (let i = 0; i < this.numLayers; i++) {
      const s = this.spec(i);
      let kvSource = -1;
      if (s.shared) {
        if (store[s.attentionType] === undefined) {
          throw new Error(`Missing shared ${s.attentionType} KV cache at layer ${i}`);
        }
        kvSource = store[s.attentionType];
      } else if (s.storeShared) {
        store[s.attentionType] = i;
      }
      out.push({
        headDim: s.headDim, intermediate: s.intermediate, full: s.full ? 1 : 0, kvSource,
        ropeBase: s.ropeBase, ropeProp: s.ropeProp,
      });
    }
    return out;
  }

  async uploadTensor(name, label) {
    const info = this.reader.info(name);
    const [s, e] = info.data_offsets;
    const bytes = e - s;
    const buf = rt.createBuffer(this.device, bytes, U.STORAGE | U.COPY_DST, label);
    this.owned.push(buf);
    const chunk = 64 << 20;
    for (let off = 0; off < bytes; off += chunk) {
      const n = Math.min(chunk, bytes - off);
      this.device.queue.writeBuffer(buf, off, await this.reader.rangeInTensor(name, off, n));
    }
    return { buf, info };
  }

  async linear(layer, which, base) {
    const w = await rt.GPUW4Linear.load(this.device, this.reader, base);
    this.owned.push(w);
    this.engine.setLinear(layer, PROJ[which], w.weight);
  }

  // load() (gemma4-webgpu.js:150-189)
  async load() {
    const embedName = 'model.language_model.embed_tokens.weight';
    const info = this.reader.info(embedName);
    this.vocab = info.shape[0];
    if (info.shape[1] !== this.hidden) throw new Error(`embedding width ${info.shape[1]} != hidden ${this.hidden}`);
    this.engine = new rt.native.GemmaEngine({
      hidden: this.hidden, heads: this.heads, pleDim: this.pleDim, vocab: this.vocab,
      maxSeq: this.maxSeq, window: this.window, eps: 1e-6, softcap: 30,
      layers: this.engineLayers(),
    });
    const E = this.engine, r = this.reader;
    this.log('Loading top-level W4A16 projection...');
    await this.linear(-1, 'top', 'model.language_model.per_layer_model_projection');
    E.setNorm(-1, NORM.pleProjection, await r.bf16('model.language_model.per_layer_projection_norm.weight'));
    E.setNorm(-1, NORM.final, await r.bf16('model.language_model.norm.weight'));
    this.log(`Loading ${this.numLayers} quantized transformer layers...`);
    for (let i = 0; i < this.numLayers; i++) {
      const root = `model.language_model.layers.${i}`, s = this.spec(i);
      const names = layerNames(i, s);
      for (const key of Object.keys(names)) await this.linear(i, key, names[key]);
      E.setNorm(i, NORM.input, await r.bf16(`${root}.input_layernorm.weight`));
      E.setNorm(i, NORM.postAttn, await r.bf16(`${root}.post_attention_layernorm.weight`));
      E.setNorm(i, NORM.preFfw, await r.bf16(`${root}.pre_feedforward_layernorm.weight`));
      E.setNorm(i, NORM.postFfw, await r.bf16(`${root}.post_feedforward_layernorm.weight`));
      E.setNorm(i, NORM.postPle, await r.bf16(`${root}.post_per_layer_input_norm.weight`));
      E.setNorm(i, NORM.q, await r.bf16(`${root}.self_attn.q_norm.weight`));
      if (!s.shared) E.setNorm(i, NORM.k, await r.bf16(`${root}.self_attn.k_norm.weight`));
      E.setLayerScalar(i, await r.scalarBF16(`${root}.layer_scalar`));
    }
    this.log('Loading tied BF16 embedding / LM head...');
    E.setEmbedding((await this.uploadTensor(embedName, 'embed-tokens')).buf);
    if (r.pleBundle) {
      await r.pleBundle.loadToDevice(this.device);
      E.setPle(r.pleBundle.table);
    } else {
      const { buf } = await this.uploadTensor('model.language_model.embed_tokens_per_layer.weight', 'embed-tokens-per-layer');
      E.setPleDense(buf);
    }
    this.loaded = true;
    this.log('Device model preload complete.');
  }

  resetCache() { this.engine.reset(); }

  check() { if (!this.loaded) throw new Error('Model not loaded.'); }

  // forward (gemma4-webgpu.js:303-402): the final-norm last row [hidden] in a
  // new device buffer the caller destroys.  {diagnostic: true} runs the
  // engine's diagnostic forward (the op-by-op path, every stage kept) and logs
  // the reference's lines: the top-level hidden and PLE rows, the layer-1
  // stages, every layer's hidden state; it throws at the first non-finite one.
  async forward(tokenIds, startPos, { diagnostic = false } = {}) {
    this.check();
    const last = rt.createBuffer(this.device, this.hidden * 4, U.STORAGE | U.COPY_SRC, 'last-hidden');
    if (!diagnostic) {
      try {
        this.engine.forward(Int32Array.from(tokenIds), startPos, last);
      } catch (e) { last.destroy(); throw e; }
      return last;
    }
    const rows = tokenIds.length, H = this.hidden, NL = this.numLayers, P = this.pleDim;
    const mk = (n, label) => rt.createBuffer(this.device, n * 4, U.STORAGE | U.COPY_SRC, label);
    const stageLayer = NL > 1 ? 1 : -1;
    const off = stageLayer >= 0 ? this.engine.diagStages(stageLayer, rows) : null;
    const top = mk(rows * H, 'diag-top-hidden'), ple = mk(rows * NL * P, 'diag-top-ple');
    const layers = mk(NL * rows * H, 'diag-layers');
    const stages = off ? mk(off[off.length - 1], 'diag-stages') : null;
    try {
      this.engine.forwardDiag(Int32Array.from(tokenIds), startPos, last, top, ple, layers, stageLayer, stages);
      this.log(`[diag top hidden] ${formatStats(finiteStats(await rt.readF32(this.device, top, rows * H)))}`);
      this.log(`[diag top PLE]    ${formatStats(finiteStats(await rt.readF32(this.device, ple, rows * NL * P)))}`);
      const all = await rt.readF32(this.device, layers, NL * rows * H);
      const st = stages ? await rt.readF32(this.device, stages, off[off.length - 1]) : null;
      for (let i = 0; i < NL; i++) {
        if (i === stageLayer) {
          const probes = [];
          for (let k = 0; k < STAGE_NAMES.length; k++) {
            if (off[k + 1] > off[k]) probes.push({ name: STAGE_NAMES[k], values: st.subarray(off[k], off[k + 1]) });
          }
          logStages(this.log, probes);
        }
        logLayer(this.log, i, all.subarray(i * rows * H, (i + 1) * rows * H));
      }
    } catch (e) {
      last.destroy();
      throw e;
    } finally {
      for (const b of [top, ple, layers, stages]) if (b) b.destroy();
    }
    return last;
  }

  // logits (gemma4-webgpu.js:404-431); {diagnostic: true} logs their statistics
  // and the first 16 values
  async logits(lastHidden, { diagnostic = false } = {}) {
    this.check();
    const buf = rt.createBuffer(this.device, this.vocab * 4, U.STORAGE | U.COPY_SRC, 'logits');
    try {
      this.engine.logits(lastHidden, buf);
      const out = await rt.readF32(this.device, buf, this.vocab);
      if (diagnostic) logLogits(this.log, out);
      return out;
    } finally { buf.destroy(); }
  }

  // greedy (gemma4-webgpu.js:441-481)
  async greedy(tokenIds, startPos) {
    this.check();
    const buf = rt.createBuffer(this.device, this.vocab * 4, U.STORAGE | U.COPY_SRC, 'logits');
    let l;
    try {
      this.engine.greedy(Int32Array.from(tokenIds), startPos, buf);
      l = await rt.readF32(this.device, buf, this.vocab);
    } finally { buf.destroy(); }
    let finite = 0;
    for (let i = 0; i < l.length; i++) if (Number.isFinite(l[i])) finite++;
    if (finite !== l.length) throw new Error(`Non-finite logits: ${l.length - finite}/${l.length}`);
    const top10 = rt.topK(l, 10);
    return { logits: l, top10, nextTokenId: top10[0].tokenId };
  }

  // The next `steps` greedy tokens after the last greedy()/decode() call, on
  // the recorded decode step; an Int32Array.
  decode(steps) {
    this.check();
    return this.engine.decode(steps);
  }

  cacheLength() { return this.engine.cacheLength(); }

  cacheSummary() {
    const len = this.engine.cacheLength();
    let bytes = 0, caches = 0;
    for (const L of this.engineLayers()) {
      if (L.kvSource < 0) { caches++; bytes += len * L.headDim * 4 * 2; }
    }
    return { caches, bytes };
  }

  dispose() {
    if (this.engine) { this.engine.dispose(); this.engine = null; }
    for (const x of this.owned) (x.dispose ? x.dispose() : x.destroy());
    this.owned = [];
    this.loaded = false;
  }
}

// The distribution reader: the CORE safetensors reader plus pleRowsToGpu from
// a device-resident W4 PLE bundle (gpu-runtime.js:905-907, 993-995).
function withPleBundle(reader, bundle) {
  const r = Object.create(reader);
  r.pleRowsToGpu = (device, ids) => bundle.rowsToGpu(device, ids);
  r.pleBundle = bundle;
  return r;
}

module.exports = {
  Gemma4Hip, Gemma4HipEngine, KVCache, e2bSpec, withPleBundle, finiteStats, formatStats, STAGE_NAMES,
};
