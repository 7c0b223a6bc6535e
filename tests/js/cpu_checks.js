'use strict';
// CPU-only checks of the Node side of the HIP bridge (no GPU needed):
// the addon loads, the runtime's host logic matches the reference semantics.
// Usage: node tests/js/cpu_checks.js <tmpdir> <ple_layout_fixture.json>
const assert = require('assert');
const fs = require('fs');
const path = require('path');
const rt = require('../../gemma4-js_amd/node/hip-runtime.js');

const tmp = process.argv[2];
const fixture = process.argv[3];
const results = [];
const pending = [];
function check(name, fn) {
  const r = fn();
  if (r && typeof r.then === 'function') pending.push(r.then(() => results.push(name)));
  else results.push(name);
}

check('addon exports the C ABI surface', () => {
  for (const f of ['init', 'deviceInfo', 'sync', 'copy', 'bf16Head', 'encoderBegin', 'encoderFinish', 'timeMs']) {
    assert.strictEqual(typeof rt.native[f], 'function', f);
  }
  for (const c of ['DeviceBuffer', 'W4Weight', 'PleTable', 'CommandBuffer']) {
    assert.strictEqual(typeof rt.native[c], 'function', c);
  }
  assert.strictEqual(rt.F32, 0);
  assert.strictEqual(rt.BF16, 1);
});

check('buffers before init throw the C ABI error', () => {
  assert.throws(() => new rt.native.DeviceBuffer(16), e => e.code === 'G4_STATUS_3' && /g4_init/.test(e.message));
});

check('int arguments outside the int32 range throw instead of wrapping', () => {
  // checked in the addon before the C ABI call, so no device is needed
  assert.throws(() => rt.native.init(2 ** 32), e => e instanceof RangeError && /device is out of the int range/.test(e.message));
  assert.throws(() => rt.native.init(-(2 ** 31) - 1), e => e instanceof RangeError);
});

check('topK: largest first, finite only, ties keep the lower index', () => {
  const brute = (a, k) => Array.from(a.keys()).filter(i => Number.isFinite(a[i]))
    .sort((x, y) => (a[y] - a[x]) || (x - y)).slice(0, k);
  let seed = 12345;
  const rnd = () => { seed = (seed * 1103515245 + 12345) % 2147483648; return seed / 2147483648; };
  for (let t = 0; t < 200; t++) {
    const n = 1 + Math.floor(rnd() * 300);
    const a = new Float32Array(n);
    for (let i = 0; i < n; i++) {
      const r = rnd();
      a[i] = r < 0.04 ? NaN : r < 0.07 ? Infinity : Math.floor(rnd() * 11) - 5;
    }
    const k = 1 + Math.floor(rnd() * 12);
    if (!Array.from(a).some(Number.isFinite)) continue;
    assert.deepStrictEqual(rt.topK(a, k).map(e => e.tokenId), brute(a, k));
  }
  assert.throws(() => rt.topK(new Float32Array([NaN, Infinity]), 3), /no finite logits/);
});

check('bf16ToF32 widens by a 16-bit shift', () => {
  const bits = new Uint16Array([0x3f80, 0xbf80, 0x4049, 0x7f80, 0x0001, 0x8000]);
  const f = rt.bf16ToF32(bits.buffer);
  const back = new Uint32Array(f.buffer);
  for (let i = 0; i < bits.length; i++) assert.strictEqual(back[i], (bits[i] << 16) >>> 0);
});

check('SafeFileReader reads tensors, ranges and BF16 rows', () => {
  // a hand-made safetensors file: 8-byte header length, JSON header, data
  const a = new Int32Array([1, -2, 3, 0x7fffffff]);
  const b = new Uint16Array([0x3f80, 0x4000, 0x4040, 0x4080, 0x40a0, 0x40c0]);  // 1..6 as bf16
  const header = {
    __metadata__: { gemma4_webgpu_role: 'core' },
    a: { dtype: 'I32', shape: [4], data_offsets: [0, 16] },
    b: { dtype: 'BF16', shape: [3, 2], data_offsets: [16, 28] },
  };
  let hj = Buffer.from(JSON.stringify(header), 'utf8');
  const pad = (8 - (hj.length % 8)) % 8;
  hj = Buffer.concat([hj, Buffer.alloc(pad, 0x20)]);
  const len = Buffer.alloc(8);
  len.writeBigUInt64LE(BigInt(hj.length));
  const file = path.join(tmp, 'tiny.safetensors');
  fs.writeFileSync(file, Buffer.concat([len, hj, Buffer.from(a.buffer), Buffer.from(b.buffer)]));
  const r = new rt.SafeFileReader(file);
  return r.init().then(async () => {
    assert.strictEqual(r.metadata.gemma4_webgpu_role, 'core');
    assert.deepStrictEqual(Array.from(new Int32Array(await r.bytes('a'))), Array.from(a));
    assert.deepStrictEqual(Array.from(await r.bf16('b')), [1, 2, 3, 4, 5, 6]);
    assert.deepStrictEqual(Array.from(await r.bf16Rows('b', [2, 0])), [5, 6, 1, 2]);
    assert.strictEqual(await r.scalarBF16('b'), 1);
    await assert.rejects(r.rangeInTensor('b', 10, 4), /Range outside b/);
    assert.throws(() => r.info('missing'), /Tensor not found: missing/);
    r.close();
  });
});

check('PLE manifest validation follows the reference', () => {
  const m = JSON.parse(fs.readFileSync(fixture, 'utf8'));
  rt.W4PleShardBundle.checkManifest(m);
  assert.throws(() => rt.W4PleShardBundle.checkManifest(Object.assign({}, m, { complete: false })),
    /Unexpected\/incomplete PLE shard manifest/);
  assert.throws(() => rt.W4PleShardBundle.checkManifest(Object.assign({}, m, { width: 8192 })),
    /unexpected geometry\/layout/);
  assert.throws(() => new rt.W4PleShardBundle(m, []), /PLE shard directory is incomplete: missing 64 file\(s\)/);
});

Promise.all(pending).then(() => {
  process.stdout.write(JSON.stringify({ ok: true, checks: results }) + '\n');
}).catch(e => { console.error(e); process.exit(1); });

process.on('unhandledRejection', e => { console.error(e); process.exit(1); });
