'use strict';
/*
 * w4_linear_cpu.js - the W4A16 linear of the reference's CPU path, in
 * single-threaded JavaScript.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE: run only by the benchmark's CPU
 * baseline leg and by the tests, as a timed and checked restatement.
 *
 * It restates OfficialW4A16Linear.apply
 * (browser-tfjs-webgl-distribution/runtime/official-quantized-linear.js:82-128):
 * for each chunk of outputChunkSize = 256 output rows (line 13),
 * dequantizeOfficialW4A16Rows (official-w4a16.js:50-101) writes the FP32
 * weights of the chunk, then tf.matMul(x, w, false, true) (line 116) runs on
 * tfjs-backend-cpu 4.22.0 (package-lock.json:36; not vendored in the
 * reference): 48x48x48 blocks, each block's partial dot product a JS number
 * (binary64) added into the Float32Array result once per k block.  The
 * chunks are concatenated along the output axis (tf.concat, line 121).
 * The scales arrive as BF16 bits and are widened (bits << 16,
 * checkpoint/browser-w4a16-reader.js:1-6) once, as the loader does.
 *
 * Usage: node w4_linear_cpu.js M K N packed.bin scales.bin x.bin y.bin SECONDS
 *   packed.bin  int32 [N, K/8]; scales.bin  uint16 BF16 [N, K/32];
 *   x.bin float32 [M, K].  Runs the linear repeatedly for about SECONDS,
 *   writes the last y (float32 [M, N]) to y.bin and prints one JSON line
 *   {"calls", "seconds", "ms_per_call"}.
 */
const fs = require('fs');

function signedInt4FromNibble(nibble) {
  // official-w4a16.js:15-19
  return (nibble & 0x0f) - 8;
}

function bf16ToFloat32Array(bits) {
  const u32 = new Uint32Array(bits.length);
  for (let i = 0; i < bits.length; i++) u32[i] = bits[i] << 16;
  return new Float32Array(u32.buffer);
}

function dequantizeRows(packed, scales, outDim, inDim, rowStart, rowCount, groupSize, out) {
  // official-w4a16.js:50-101 (validation at 56-74 is done once by the caller)
  const packedInDim = inDim / 8;
  const groupsPerRow = inDim / groupSize;
  for (let localRow = 0; localRow < rowCount; localRow++) {
    const row = rowStart + localRow;
    const packedRowOffset = row * packedInDim;
    const scaleRowOffset = row * groupsPerRow;
    const outputRowOffset = localRow * inDim;
    for (let packedCol = 0; packedCol < packedInDim; packedCol++) {
      const word = packed[packedRowOffset + packedCol] >>> 0;
      const baseInput = packedCol * 8;
      for (let k = 0; k < 8; k++) {
        const inputIndex = baseInput + k;
        const q = signedInt4FromNibble((word >>> (k * 4)) & 0x0f);
        const scale = scales[scaleRowOffset + Math.floor(inputIndex / groupSize)];
        out[outputRowOffset + inputIndex] = q * scale;
      }
    }
  }
}

function matMulXWt(x, M, w, N, K, y) {
  // tfjs-backend-cpu BatchMatMul with transposeB, blockSize 48
  const bs = 48;
  y.fill(0);
  for (let i0 = 0; i0 < M; i0 += bs) {
    const iB = Math.min(i0 + bs, M);
    for (let j0 = 0; j0 < N; j0 += bs) {
      const jB = Math.min(j0 + bs, N);
      for (let k0 = 0; k0 < K; k0 += bs) {
        const kB = Math.min(k0 + bs, K);
        for (let i = i0; i < iB; i++) {
          for (let j = j0; j < jB; j++) {
            let sum = 0.0;
            const xo = i * K;
            const wo = j * K;
            for (let k = k0; k < kB; k++) sum += x[xo + k] * w[wo + k];
            y[i * N + j] += sum;
          }
        }
      }
    }
  }
}

function w4Linear(x, M, packed, scalesF32, N, K, groupSize, chunk, y, wChunk, yChunk) {
  for (let rowStart = 0; rowStart < N; rowStart += chunk) {
    const rowCount = Math.min(chunk, N - rowStart);
    dequantizeRows(packed, scalesF32, N, K, rowStart, rowCount, groupSize, wChunk);
    const yc = yChunk.subarray(0, M * rowCount);
    matMulXWt(x, M, wChunk, rowCount, K, yc);
    for (let i = 0; i < M; i++) {
      y.set(yc.subarray(i * rowCount, (i + 1) * rowCount), i * N + rowStart);
    }
  }
}

function readTyped(path, Ctor) {
  const b = fs.readFileSync(path);
  const copy = new Uint8Array(b.length);
  copy.set(b);
  return new Ctor(copy.buffer, 0, b.length / Ctor.BYTES_PER_ELEMENT);
}

function main() {
  const a = process.argv.slice(2);
  if (a.length !== 8) {
    throw new Error('usage: node w4_linear_cpu.js M K N packed scales x y seconds');
  }
  const M = parseInt(a[0], 10);
  const K = parseInt(a[1], 10);
  const N = parseInt(a[2], 10);
  const groupSize = 32;
  if (K % 8 !== 0) throw new Error('inDim must be divisible by 8.');
  if (K % groupSize !== 0) throw new Error('inDim must be divisible by groupSize.');
  const packed = readTyped(a[3], Int32Array);
  const scales = bf16ToFloat32Array(readTyped(a[4], Uint16Array));
  const x = readTyped(a[5], Float32Array);
  if (packed.length !== N * K / 8) throw new Error('packedWeight length mismatch.');
  if (scales.length !== N * K / groupSize) throw new Error('scales length mismatch.');
  if (x.length !== M * K) throw new Error('x length mismatch.');
  const seconds = parseFloat(a[7]);
  const chunk = 256;
  const y = new Float32Array(M * N);
  const wChunk = new Float32Array(chunk * K);
  const yChunk = new Float32Array(M * chunk);
  w4Linear(x, M, packed, scales, N, K, groupSize, chunk, y, wChunk, yChunk); // warm
  let calls = 0;
  const t0 = process.hrtime();
  let el = 0;
  do {
    w4Linear(x, M, packed, scales, N, K, groupSize, chunk, y, wChunk, yChunk);
    calls++;
    const d = process.hrtime(t0);
    el = d[0] + d[1] * 1e-9;
  } while (el < seconds);
  fs.writeFileSync(a[6], Buffer.from(y.buffer));
  process.stdout.write(JSON.stringify({ calls: calls, seconds: el, ms_per_call: el * 1e3 / calls }) + '\n');
}

main();
