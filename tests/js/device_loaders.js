'use strict';
// The addon's device-side loaders against their host-bytes counterparts:
// W4Weight from DeviceBuffers (g4_w4_load_dev) vs from host bytes, and
// PleTable.uploadShard from a DeviceBuffer (g4_ple_upload_shard_dev) vs host
// bytes, on data made by fillRandom.  Prints one JSON line.
const rt = require('../../gemma4-js_amd/node/hip-runtime.js');

const native = rt.native;
const device = rt.requestDevice(0);
const U = rt.GPUBufferUsage;
const buf = (n) => rt.createBuffer(device, n, U.STORAGE);

function same(a, b) {
  if (a.length !== b.length) return false;
  for (let i = 0; i < a.length; i++) if (a[i] !== b[i] && !(a[i] !== a[i] && b[i] !== b[i])) return false;
  return true;
}

const out = {};
{
  const n = 96, k = 512;
  const pk = buf(n * k / 2), sc = buf(n * (k / 32) * 2), x = buf(3 * k * 4);
  native.fillRandom(pk, n * k / 8, native.RAND_W4_PACKED, 11);
  native.fillRandom(sc, n * (k / 32), native.RAND_BF16_ABS_NORMAL, 12, 0.02);
  native.fillRandom(x, 3 * k, native.RAND_F32_NORMAL, 13, 1.0);
  const wd = new native.W4Weight(pk, sc, n, k, 32);
  const wh = new native.W4Weight(pk.read(0, n * k / 2), sc.read(0, n * (k / 32) * 2), n, k, 32);
  const yd = buf(3 * n * 4), yh = buf(3 * n * 4);
  wd.linear(x, rt.F32, 3, yd, rt.F32);
  wh.linear(x, rt.F32, 3, yh, rt.F32);
  out.w4 = same(new Float32Array(yd.read(0, 3 * n * 4)), new Float32Array(yh.read(0, 3 * n * 4)));
  const scales = new Uint16Array(sc.read(0, n * (k / 32) * 2));
  out.scalesNonzero = scales.some((v) => v !== 0);
  wd.dispose(); wh.dispose();
  for (const b of [pk, sc, x, yd, yh]) b.destroy();
}
{
  const vocab = 100, width = 64, rps = 32;  // 4 shards, the last one short
  const td = new native.PleTable(vocab, width, 32, rps), th = new native.PleTable(vocab, width, 32, rps);
  const packedRow = width / 2, scaleRow = (width / 32) * 2;
  for (let s = 0; s < 4; s++) {
    const nbytes = td.shardBytes(s), rows = nbytes / (packedRow + scaleRow);
    const st = buf(nbytes);
    native.fillRandom(st, rows * packedRow, native.RAND_PLE_PACKED, 100 + s);
    native.fillRandom(st, rows * (width / 32), native.RAND_BF16_ABS_NORMAL, 200 + s, 0.05, rows * packedRow);
    td.uploadShard(s, st);
    th.uploadShard(s, st.read(0, nbytes));
    st.destroy();
  }
  const ids = Int32Array.from([0, 31, 32, 99, 64, 5, 99]);
  const gd = buf(ids.length * width * 4), gh = buf(ids.length * width * 4);
  td.gather(ids, gd, rt.F32);
  th.gather(ids, gh, rt.F32);
  const a = new Float32Array(gd.read(0, ids.length * width * 4));
  out.ple = same(a, new Float32Array(gh.read(0, ids.length * width * 4)));
  out.pleNonzero = a.some((v) => v !== 0);
  td.dispose(); th.dispose(); gd.destroy(); gh.destroy();
}
console.log(JSON.stringify(out));
