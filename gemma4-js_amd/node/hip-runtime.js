'use strict';
// HIP (MI355X, gfx950) replacement of the WebGPU buffer + dispatch layer and
// the hot-path ops of custom-webgpu/gpu-runtime.js, for Node (CommonJS; runs
// on Node 12).  The exported names, argument meaning and error behaviour
// follow gpu-runtime.js so that a model driver written against it (e.g.
// gemma4-webgpu.js:2-10 imports GPUOps, GPUW4Linear, SafeFileReader,
// uploadF32, createBuffer, readF32, topK) can run on the HIP path.
//
// Queue semantics.  The reference records ops into a command encoder and
// runs them at queue.submit() in submission order (gpu-runtime.js:328-332,
// gemma4-webgpu.js:339-358).  Here every op is enqueued on the library's one
// HIP stream as it is encoded, so device order equals encode order, which is
// the order the reference submits in; submit() is therefore a no-op.
// buffer.destroy() returns the memory to the library's stream-ordered cache:
// only work enqueued after the destroy can reuse it, so nothing waits, as
// WebGPU defers the release until submitted work is done.  Recording for
// replay is available separately through HipCommandRecorder (HIP graphs).

const fs = require('fs');
const path = require('path');
const native = require('./g4hip.node');

// GPUBufferUsage flag values; accepted for signature compatibility.
const GPUBufferUsage = Object.freeze({
  MAP_READ: 0x0001, MAP_WRITE: 0x0002, COPY_SRC: 0x0004, COPY_DST: 0x0008, INDEX: 0x0010,
  VERTEX: 0x0020, UNIFORM: 0x0040, STORAGE: 0x0080, INDIRECT: 0x0100, QUERY_RESOLVE: 0x0200,
});
const U = GPUBufferUsage;
const F32 = native.F32;
const BF16 = native.BF16;

function align4(n) { return Math.max(4, (n + 3) & ~3); }

// ---- device / queue / encoder ------------------------------------------------

class HipQueue {
  constructor(device) { this.device = device; }
  // queue.writeBuffer(buffer, bufferOffset, data, dataOffset?, size?) (bytes)
  writeBuffer(buffer, bufferOffset, data, dataOffset, size) {
    const u8 = toU8(data, dataOffset || 0, size);
    buffer.write(u8, bufferOffset || 0);
  }
  submit(commandBuffers) {
    if (!Array.isArray(commandBuffers)) throw new TypeError('submit() expects an array');
    for (const cb of commandBuffers) {
      if (cb && cb.recorded) cb.recorded.submit();
    }
  }
  onSubmittedWorkDone() { native.sync(); return Promise.resolve(); }
}

class HipCommandEncoder {
  constructor(device) { this.device = device; this.finished = false; }
  copyBufferToBuffer(src, srcOffset, dst, dstOffset, size) {
    native.copy(dst, dstOffset, src, srcOffset, size);
  }
  finish() {
    if (this.finished) throw new Error('command encoder already finished');
    this.finished = true;
    return { label: 'hip-command-buffer', recorded: null };
  }
}

// Records the launches made by fn() into a replayable command buffer.
class HipCommandRecorder {
  static record(fn) {
    native.encoderBegin();
    let ok = false;
    try { fn(); ok = true; } finally {
      const cb = native.encoderFinish();
      if (!ok) cb.destroy();
      else return { label: 'hip-recorded', recorded: cb };
    }
    return null;
  }
}

class HipDevice {
  constructor(index) {
    native.init(index);
    this.index = index;
    this.info = native.deviceInfo();
    this.queue = new HipQueue(this);
    this.label = this.info.name;
  }
  createCommandEncoder() { return new HipCommandEncoder(this); }
  createBuffer({ size, label = '' }) {
    const b = new native.DeviceBuffer(align4(size));
    b.label = label;
    return b;
  }
}

const devices = new Map();
// Stands in for navigator.gpu.requestAdapter() + adapter.requestDevice().
function requestDevice(index = 0) {
  if (!devices.has(index)) devices.set(index, new HipDevice(index));
  return devices.get(index);
}

function toU8(data, offset, size) {
  let u8;
  if (data instanceof ArrayBuffer) u8 = new Uint8Array(data);
  else if (ArrayBuffer.isView(data)) u8 = new Uint8Array(data.buffer, data.byteOffset, data.byteLength);
  else throw new TypeError('expected an ArrayBuffer or a typed array');
  const end = size === undefined ? u8.length : offset + size;
  return u8.subarray(offset, end);
}

// ---- buffers (gpu-runtime.js:6-38) -------------------------------------------------

function createBuffer(device, size, usage, label = '') {
  return device.createBuffer({ size: align4(size), usage, label });
}

function uploadBytes(device, bytes, usage = U.STORAGE, label = '') {
  const b = createBuffer(device, bytes.byteLength, usage | U.COPY_DST, label);
  if (bytes.byteLength) b.write(toU8(bytes, 0));
  return b;
}

function uploadF32(device, data, usage = U.STORAGE, label = '') {
  return uploadBytes(device, new Uint8Array(data.buffer, data.byteOffset, data.byteLength), usage, label);
}

function uploadU32(device, data, usage = U.UNIFORM, label = '') {
  return uploadBytes(device, new Uint8Array(data.buffer, data.byteOffset, data.byteLength), usage, label);
}

async function readF32(device, buffer, count) {
  return new Float32Array(buffer.read(0, count * 4));
}

function bf16ToF32(buffer) {
  const src = buffer instanceof ArrayBuffer ? new Uint8Array(buffer)
    : new Uint8Array(buffer.buffer, buffer.byteOffset, buffer.byteLength);
  const n = src.length >> 1;
  const out = new Float32Array(n);
  const bits = new Uint32Array(out.buffer);
  for (let i = 0; i < n; i++) bits[i] = (src[2 * i] | (src[2 * i + 1] << 8)) << 16 >>> 0;
  return out;
}

// ---- safetensors reader over a local file (gpu-runtime.js:40-87) --------------------

class SafeFileReader {
  constructor(file) {
    this.file = file;  // a path
    this.header = null;
    this.metadata = {};
    this.dataStart = null;
    this.fd = null;
  }
  async init() {
    this.fd = fs.openSync(this.file, 'r');
    const lenBuf = Buffer.alloc(8);
    fs.readSync(this.fd, lenBuf, 0, 8, 0);
    const headerLength = Number(lenBuf.readBigUInt64LE(0));
    const hb = Buffer.alloc(headerLength);
    fs.readSync(this.fd, hb, 0, headerLength, 8);
    this.header = JSON.parse(hb.toString('utf8'));
    this.metadata = this.header.__metadata__ || {};
    this.dataStart = 8 + headerLength;
    return this;
  }
  info(name) {
    const x = this.header[name];
    if (!x) throw new Error(`Tensor not found: ${name}`);
    return x;
  }
  _read(start, length) {
    const b = Buffer.alloc(length);
    let got = 0;
    while (got < length) {
      const n = fs.readSync(this.fd, b, got, length - got, start + got);
      if (n <= 0) throw new Error(`${this.file}: short read at ${start + got}`);
      got += n;
    }
    return b.buffer.slice(b.byteOffset, b.byteOffset + length);
  }
  async bytes(name) {
    const [s, e] = this.info(name).data_offsets;
    return this._read(this.dataStart + s, e - s);
  }
  async rangeInTensor(name, byteOffset, byteLength) {
    const [s, e] = this.info(name).data_offsets;
    if (byteOffset < 0 || byteOffset + byteLength > e - s) throw new Error(`Range outside ${name}`);
    return this._read(this.dataStart + s + byteOffset, byteLength);
  }
  async bf16(name) { return bf16ToF32(await this.bytes(name)); }
  async scalarBF16(name) { return (await this.bf16(name))[0]; }
  async bf16Rows(name, ids) {
    const x = this.info(name);
    if (x.dtype !== 'BF16' || x.shape.length !== 2) throw new Error(`${name}: BF16 rank2 expected`);
    const width = x.shape[1], rowBytes = width * 2;
    const out = new Float32Array(ids.length * width);
    for (let j = 0; j < ids.length; j++) {
      out.set(bf16ToF32(await this.rangeInTensor(name, ids[j] * rowBytes, rowBytes)), j * width);
    }
    return out;
  }
  close() { if (this.fd !== null) { fs.closeSync(this.fd); this.fd = null; } }
}

// ---- W4A16 linear (gpu-runtime.js:1380-1394) ----------------------------------------

class GPUW4Linear {
  constructor(device, name, inDim, outDim, groupSize, weight) {
    Object.assign(this, { device, name, inDim, outDim, groupSize, weight });
    this.groups = inDim / groupSize;
  }
  static async load(device, reader, base) {
    const pi = reader.info(`${base}.weight_packed`), si = reader.info(`${base}.weight_scale`);
    const outDim = pi.shape[0], inDim = pi.shape[1] * 8, groups = si.shape[1], groupSize = inDim / groups;
    const [pb, sb] = await Promise.all([reader.bytes(`${base}.weight_packed`), reader.bytes(`${base}.weight_scale`)]);
    return GPUW4Linear.fromBytes(device, base, pb, sb, outDim, inDim, groupSize);
  }
  static fromBytes(device, name, packedBytes, scaleBytes, outDim, inDim, groupSize = 32) {
    const w = new native.W4Weight(packedBytes, scaleBytes, outDim, inDim, groupSize);
    return new GPUW4Linear(device, name, inDim, outDim, groupSize, w);
  }
  dispose() { this.weight.dispose(); }
}

// ---- ops (gpu-runtime.js:1295-1378) ---------------------------------------------------

// The reference's PLE geometry (gpu-runtime.js:1344-1347, 1366-1369: 256-wide
// rows for 35 layers); a GPUOps built for another model passes its own.
const PLE_WIDTH = 256, PLE_LAYERS = 35, RMS_EPS = 1e-6;

class GPUOps {
  constructor(device, { pleWidth = PLE_WIDTH, pleLayers = PLE_LAYERS } = {}) {
    this.device = device;
    this.pleWidth = pleWidth;
    this.pleLayers = pleLayers;
  }
  track(garbage, buffer) { if (garbage) garbage.push(buffer); return buffer; }
  emptyF32(n, label = '') { return createBuffer(this.device, n * 4, U.STORAGE | U.COPY_SRC | U.COPY_DST, label); }
  // y[rows, outDim] = x[rows, inDim] . W^T, FP32 in and out (gpu-runtime.js:1316-1324)
  w4(encoder, linear, x, rows, garbage = null) {
    const y = this.emptyF32(rows * linear.outDim, `${linear.name}:out`);
    linear.weight.linear(x, F32, rows, y, F32);
    return y;
  }
  // Consecutive w4 dispatches over one input (q/k/v at gemma4-webgpu.js:225,
  // 237-238; gate/up at 280-281) as one call, one launch for a single row;
  // returns one output buffer per linear.
  w4Multi(encoder, linears, x, rows, garbage = null) {
    const ys = linears.map((l) => this.emptyF32(rows * l.outDim, `${l.name}:out`));
    native.linearMulti(linears.map((l) => l.weight), x, F32, rows, ys, F32);
    return ys;
  }
  // RMS_SHADER (gpu-runtime.js:1325-1332): y = x / rms(x) * (scale or 1), eps 1e-6
  rms(encoder, x, rows, width, scale = null, garbage = null) {
    const y = this.emptyF32(rows * width, 'rms-out');
    native.rms(x, rows, width, scale, RMS_EPS, y);
    return y;
  }
  // ADD_SCALE_SHADER (gpu-runtime.js:1333-1336): y = (a + b) * scale
  addScale(encoder, a, b, n, scale = 1, garbage = null) {
    const y = this.emptyF32(n, 'add-out');
    native.addScale(a, b, n, scale, y);
    return y;
  }
  // SCALE_SHADER (gpu-runtime.js:1337-1340): y = a * s
  scale(encoder, a, n, s, garbage = null) {
    const y = this.emptyF32(n, 'scale-out');
    native.scale(a, n, s, y);
    return y;
  }
  // GELU_MUL_SHADER (gpu-runtime.js:1341-1344): y = gelu(gate) * up
  geluMul(encoder, gate, up, n, garbage = null) {
    const y = this.emptyF32(n, 'gelu-mul');
    native.geluMul(gate, up, n, y);
    return y;
  }
  // GELU_PLE_SHADER (gpu-runtime.js:1345-1348): y = gelu(gate) * ple[row, layer]
  geluPle(encoder, gate, ple, rows, layer, garbage = null) {
    const y = this.emptyF32(rows * this.pleWidth, 'gelu-ple');
    native.geluPle(gate, ple, rows, layer, this.pleWidth, this.pleLayers, y);
    return y;
  }
  // NORM_ROPE_SHADER (gpu-runtime.js:1349-1356): per-head RMS norm, rotate-half
  // RoPE of floor(ropeProp * hd / 2) pairs at positions pos0 + row
  normRope(encoder, x, rows, heads, hd, pos0, scale, ropeProp, base, garbage = null) {
    const y = this.emptyF32(rows * heads * hd, 'rope-out');
    native.normRope(x, rows, heads, hd, pos0, scale, Math.floor(ropeProp * hd / 2), base, RMS_EPS, y);
    return y;
  }
  // QK_SHADER + SOFTMAX_SHADER + ATTN_OUT_SHADER (gpu-runtime.js:1357-1365)
  attention(encoder, q, kcache, vcache, qrows, heads, hd, keylen, qpos0, sliding, window, garbage = null) {
    const out = this.emptyF32(qrows * heads * hd, 'attn-out');
    native.attention(q, kcache, vcache, qrows, heads, hd, keylen, qpos0, sliding ? 1 : 0, window, out);
    return out;
  }
  // PLE_MIX_SHADER (gpu-runtime.js:1366-1369)
  pleMix(encoder, proj, normScale, tokenPle, rows, garbage = null) {
    const y = this.emptyF32(rows * this.pleLayers * this.pleWidth, 'ple-mix');
    native.pleMix(proj, normScale, tokenPle, rows, this.pleWidth, this.pleLayers, y);
    return y;
  }
  // out[outOffset + r] = 30 * tanh((x . E[r]) / 30) over a chunk of rows
  // (gpu-runtime.js:1370-1376; in_dim fixed to 1536 there, derived here)
  headChunk(encoder, x, weightChunk, out, outOffset, rows, garbage = null, inDim = 1536) {
    if (weightChunk.size < rows * inDim * 2) throw new Error('headChunk: weight chunk too small');
    native.bf16Head(x, weightChunk, rows, inDim, out, 1.0, 30.0, 0, outOffset * 4);
  }
  dispose() {}
}

// ---- PLE W4 shard bundle, resident on the device (gpu-runtime.js:413-527) ---------------

class W4PleShardBundle {
  constructor(manifest, shardPaths) {
    this.manifest = manifest;
    this.vocabSize = Number(manifest.vocab_size);
    this.width = Number(manifest.width);
    this.groupSize = Number(manifest.quantization.group_size);
    this.rowsPerShard = Number(manifest.layout.rows_per_shard);
    this.packedRowBytes = Number(manifest.layout.packed_row_bytes);
    this.scaleRowBytes = Number(manifest.layout.scale_row_bytes);
    this.shards = manifest.shards;
    this.fileByName = new Map(shardPaths.map(p => [path.basename(p), p]));
    const missing = this.shards.map(s => s.file).filter(name => !this.fileByName.has(name));
    if (missing.length) {
      throw new Error(`PLE shard directory is incomplete: missing ${missing.length} file(s), first: ${missing[0]}`);
    }
    this.table = null;
  }
  static checkManifest(manifest) {
    const q = manifest.quantization || {}, layout = manifest.layout || {};
    if (manifest.format !== 'gemma4-ple-w4-sharded-v1' || manifest.complete !== true) {
      throw new Error(`Unexpected/incomplete PLE shard manifest: ${manifest.format}`);
    }
    if (Number(manifest.width) !== 8960 || Number(q.group_size) !== 32 ||
        layout.kind !== 'row_sharded_packed_then_scales') {
      throw new Error('PLE shard manifest has unexpected geometry/layout.');
    }
  }
  // manifestPath: manifest.json; shardDir: directory holding the shard files
  static async fromFiles(manifestPath, shardDir) {
    const manifest = JSON.parse(fs.readFileSync(manifestPath, 'utf8'));
    W4PleShardBundle.checkManifest(manifest);
    const dir = shardDir || path.dirname(manifestPath);
    const paths = fs.readdirSync(dir).map(f => path.join(dir, f));
    return new W4PleShardBundle(manifest, paths);
  }
  // Uploads every shard file into the device table (once).
  async loadToDevice(device) {
    if (this.table) return this;
    const t = new native.PleTable(this.vocabSize, this.width, this.groupSize, this.rowsPerShard);
    try {
      this.shards.forEach((s, i) => {
        const bytes = fs.readFileSync(this.fileByName.get(s.file));
        t.uploadShard(i, bytes);
      });
    } catch (e) { t.dispose(); throw e; }
    this.table = t;
    return this;
  }
  _check(tokenId) {
    const id = Number(tokenId);
    if (!Number.isInteger(id) || id < 0 || id >= this.vocabSize) {
      throw new Error(`PLE token id out of range: ${tokenId}`);
    }
    return id;
  }
  // FP32 [ids.length, width] device buffer of dequantized rows.
  async rowsToGpu(device, ids) {
    if (!this.table) await this.loadToDevice(device);
    const i32 = Int32Array.from(ids, id => this._check(id));
    const out = createBuffer(device, i32.length * this.width * 4, U.STORAGE | U.COPY_SRC, 'token-ple-w4-dequant');
    if (i32.length) this.table.gather(i32, out, F32);
    return out;
  }
  dispose() { if (this.table) { this.table.dispose(); this.table = null; } }
}

// ---- top-k over host logits (gpu-runtime.js:1396-1425 semantics) --------------------

// The k largest finite values, largest first; an equal value never displaces
// one already kept, and among equal values the earlier index comes first.
function topK(logits, k = 10) {
  const kept = [];
  for (let i = 0; i < logits.length; i++) {
    const value = logits[i];
    if (!Number.isFinite(value)) continue;
    if (kept.length < k || value > kept[kept.length - 1].value) {
      let pos = kept.length;
      while (pos > 0 && kept[pos - 1].value < value) pos--;
      kept.splice(pos, 0, { tokenId: i, value });
      if (kept.length > k) kept.pop();
    }
  }
  if (kept.length === 0) throw new Error('topK(): no finite logits.');
  return kept;
}

module.exports = {
  GPUBufferUsage, F32, BF16, native, requestDevice, HipCommandRecorder,
  createBuffer, uploadBytes, uploadF32, uploadU32, readF32, bf16ToF32,
  SafeFileReader, GPUW4Linear, GPUOps, W4PleShardBundle, topK,
};
