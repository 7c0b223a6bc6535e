'use strict';
/*
 * ple_rows_cpu.js - the PLE row dequant of the reference's CPU path, in
 * single-threaded JavaScript.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE: run only by the benchmark's CPU
 * baseline leg and by the tests, as a timed and checked restatement.
 *
 * It restates the per-row loop of LocalPleW4ShardReader.readRows
 * (browser-tfjs-webgl-distribution/runtime/ple-w4-shard-reader.js:89-96):
 * byte = packed[i >> 1], the low nibble for even i and the high one for odd
 * i, two's-complement q (nibble >= 8 ? nibble - 16 : nibble), times the
 * group's BF16 scale widened to FP32 (bits << 16).  The reader's file slices
 * (File.slice per id, lines 71-87) are not restated: the caller hands over
 * each id's packed row and scale row already read.
 *
 * Usage: node ple_rows_cpu.js R W rows.bin out.bin SECONDS
 *   rows.bin  R records of W/2 packed bytes followed by W/32 BF16 scale bits;
 *   dequantizes all R rows repeatedly for about SECONDS, writes the last
 *   output (float32 [R, W]) to out.bin and prints one JSON line
 *   {"calls", "seconds", "ms_per_call"}.
 */
const fs = require('fs');

function bf16BitsToFloat32(bits) {
  // ple-w4-shard-reader.js:1-6: a 4-byte view per call, as the reader does
  const buffer = new ArrayBuffer(4);
  const view = new DataView(buffer);
  view.setUint32(0, (bits << 16) >>> 0, true);
  return view.getFloat32(0, true);
}

function readRows(rows, R, W, output) {
  const packedRowBytes = W / 2;
  const scaleRowBytes = W / 16;
  const record = packedRowBytes + scaleRowBytes;
  for (let outputRow = 0; outputRow < R; ++outputRow) {
    const off = outputRow * record;
    const packed = new Uint8Array(rows.buffer, rows.byteOffset + off, packedRowBytes);
    const scaleBits = new Uint16Array(rows.buffer.slice(rows.byteOffset + off + packedRowBytes,
                                                        rows.byteOffset + off + record));
    const base = outputRow * W;
    for (let i = 0; i < W; ++i) {
      const byte = packed[i >> 1];
      const nibble = (i & 1) === 0 ? byte & 0x0f : byte >> 4;
      const q = nibble >= 8 ? nibble - 16 : nibble;
      const scale = bf16BitsToFloat32(scaleBits[Math.floor(i / 32)]);
      output[base + i] = q * scale;
    }
  }
}

function main() {
  const a = process.argv.slice(2);
  if (a.length !== 5) {
    console.error('usage: node ple_rows_cpu.js R W rows.bin out.bin SECONDS');
    process.exit(2);
  }
  const R = Number(a[0]), W = Number(a[1]), seconds = Number(a[4]);
  const rows = fs.readFileSync(a[2]);
  if (rows.length !== R * (W / 2 + W / 16)) throw new Error('rows.bin has the wrong size');
  const output = new Float32Array(R * W);
  let calls = 0;
  const t0 = process.hrtime.bigint();
  let el = 0;
  do {
    readRows(rows, R, W, output);
    ++calls;
    el = Number(process.hrtime.bigint() - t0) / 1e9;
  } while (el < seconds);
  fs.writeFileSync(a[3], Buffer.from(output.buffer));
  console.log(JSON.stringify({calls, seconds: el, ms_per_call: el / calls * 1e3}));
}

main();
