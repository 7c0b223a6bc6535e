'use strict';
// Drives the HIP path through the reference-shaped JS surface:
// SafeFileReader -> GPUW4Linear.load -> GPUOps.w4, W4PleShardBundle.rowsToGpu
// and GPUOps.headChunk over a chunked tied head, like gemma4-webgpu.js does.
// Inputs come from tests/test_gpu_node.py; outputs are written back as raw
// FP32 files for the oracle comparison.
// Usage: node tests/js/gpu_parity.js <dir>
const fs = require('fs');
const path = require('path');
const rt = require('../../gemma4-js_amd/node/hip-runtime.js');

async function main() {
  const dir = process.argv[2];
  const meta = JSON.parse(fs.readFileSync(path.join(dir, 'meta.json'), 'utf8'));
  const readF32File = f => {
    const b = fs.readFileSync(path.join(dir, f));
    return new Float32Array(b.buffer.slice(b.byteOffset, b.byteOffset + b.byteLength));
  };
  const writeF32File = (f, a) => fs.writeFileSync(path.join(dir, f), Buffer.from(a.buffer, a.byteOffset, a.byteLength));
  const out = {};

  const device = rt.requestDevice(0);
  out.device = device.info.name;
  const ops = new rt.GPUOps(device);
  const reader = await new rt.SafeFileReader(path.join(dir, 'model.safetensors')).init();

  // W4A16 linear through the GPUW4Linear.load path
  const lin = await rt.GPUW4Linear.load(device, reader, 'model.layers.0.mlp.gate_proj');
  out.linear = { inDim: lin.inDim, outDim: lin.outDim, groupSize: lin.groupSize, groups: lin.groups };
  const rows = meta.rows;
  const x = rt.uploadF32(device, readF32File('x.f32'), rt.GPUBufferUsage.STORAGE, 'x');
  const enc = device.createCommandEncoder();
  const garbage = [];
  const y = ops.w4(enc, lin, x, rows, garbage);
  device.queue.submit([enc.finish()]);
  writeF32File('y.f32', await rt.readF32(device, y, rows * lin.outDim));

  // a one-row launch run eagerly, then recorded once and replayed twice
  const y1 = ops.w4(device.createCommandEncoder(), lin, x, 1, garbage);
  writeF32File('y_one.f32', await rt.readF32(device, y1, lin.outDim));
  const y2 = rt.createBuffer(device, rows * lin.outDim * 4, rt.GPUBufferUsage.STORAGE, 'y2');
  const rec = rt.HipCommandRecorder.record(() => lin.weight.linear(x, rt.F32, 1, y2, rt.F32));
  device.queue.submit([rec, rec]);
  await device.queue.onSubmittedWorkDone();
  writeF32File('y_replay.f32', await rt.readF32(device, y2, lin.outDim));
  rec.recorded.destroy();

  // PLE rows through the shard bundle, table resident on the device
  const bundle = await rt.W4PleShardBundle.fromFiles(path.join(dir, 'ple', 'manifest.json'));
  const ple = await bundle.rowsToGpu(device, meta.ple_ids);
  writeF32File('ple.f32', await rt.readF32(device, ple, meta.ple_ids.length * bundle.width));
  try {
    await bundle.rowsToGpu(device, [1, meta.vocab]);
    out.ple_range_error = null;
  } catch (e) {
    out.ple_range_error = e.message;
  }

  // tied head in lmChunkRows chunks (gemma4-webgpu.js:170-188, 413-423)
  const info = reader.info('model.embed_tokens.weight');
  const vocab = info.shape[0], width = info.shape[1], chunkRows = meta.chunk_rows;
  const h = rt.uploadF32(device, readF32File('h.f32'));
  const logitsBuf = ops.emptyF32(vocab, 'logits');
  const chunks = [];
  for (let start = 0; start < vocab; start += chunkRows) {
    const n = Math.min(chunkRows, vocab - start);
    const ab = await reader.rangeInTensor('model.embed_tokens.weight', start * width * 2, n * width * 2);
    const buf = rt.createBuffer(device, ab.byteLength, rt.GPUBufferUsage.STORAGE, `lm-head:${start}`);
    device.queue.writeBuffer(buf, 0, ab);
    chunks.push({ start, rows: n, buffer: buf });
  }
  const enc2 = device.createCommandEncoder();
  for (const c of chunks) ops.headChunk(enc2, h, c.buffer, logitsBuf, c.start, c.rows, garbage, width);
  device.queue.submit([enc2.finish()]);
  const logits = await rt.readF32(device, logitsBuf, vocab);
  writeF32File('logits.f32', logits);
  out.top10 = rt.topK(logits, 10).map(e => e.tokenId);

  for (const b of [x, y, y1, y2, h, logitsBuf, ple, ...chunks.map(c => c.buffer)]) b.destroy();
  lin.dispose();
  bundle.dispose();
  reader.close();
  out.ok = true;
  process.stdout.write(JSON.stringify(out) + '\n');
}

main().catch(e => { console.error(e && e.stack || e); process.exit(1); });
