/*
 * g4_oracle.c - CPU restatement of the gemma4-js W4A16 / PLE hot path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE: loaded only by the tests, the smoke
 * check and the benchmark's CPU-baseline leg, to check results against.
 *
 * Third-party algorithm restated here: the FP32 matMul of TF.js
 * (@tensorflow/tfjs-backend-cpu 4.22.0, pinned by package-lock.json:36 of the
 * reference; not vendored in the reference).  Its BatchMatMul kernel walks
 * 48x48x48 blocks; inside a block the partial dot product is a JavaScript
 * number (binary64) and is added into the Float32Array result once per
 * k-block, i.e. y = f32(y + f64_block_sum) for k-blocks 0, 48, 96, ...
 * No reference test pins that rounding sequence; g4o_w4_linear follows it and
 * the tests bound it against the binary64 product.
 */
#include "g4_oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

float g4o_bf16_to_f32(uint16_t bits) {
  /* gpu-runtime.js:1058-1066: setUint32(bits << 16) then getFloat32 */
  uint32_t u = (uint32_t)bits << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t g4o_f32_to_bf16(float v) {
  /* official-w4a16.js:39-47 */
  uint32_t bits;
  memcpy(&bits, &v, 4);
  uint32_t lsb = (bits >> 16) & 1u;
  bits = bits + 0x7fffu + lsb; /* (bits + 0x7fff + lsb) >>> 0 : mod 2^32 */
  return (uint16_t)(bits >> 16);
}

void g4o_bf16_to_f32_array(const uint16_t *bits, size_t n, float *out) {
  for (size_t i = 0; i < n; ++i) out[i] = g4o_bf16_to_f32(bits[i]);
}

void g4o_f32_to_bf16_array(const float *v, size_t n, uint16_t *out) {
  for (size_t i = 0; i < n; ++i) out[i] = g4o_f32_to_bf16(v[i]);
}

int g4o_w4_nibble(uint32_t nibble) {
  /* official-w4a16.js:15-19 */
  return (int)(nibble & 0x0fu) - 8;
}

int g4o_ple_nibble(uint32_t nibble) {
  /* ple-w4-shard-reader.js:92 */
  int n = (int)(nibble & 0x0fu);
  return n >= 8 ? n - 16 : n;
}

int g4o_w4_dequant_rows(const int32_t *packed, size_t packed_len,
                        const float *scales, size_t scales_len, int outDim,
                        int inDim, int rowStart, int rowCount, int groupSize,
                        float *out) {
  /* official-w4a16.js:50-101 */
  if (inDim % 8 != 0) return 1;
  if (groupSize <= 0 || inDim % groupSize != 0) return 2;
  const int packedInDim = inDim / 8;
  const int groupsPerRow = inDim / groupSize;
  if (packed_len != (size_t)outDim * packedInDim) return 3;
  if (scales_len != (size_t)outDim * groupsPerRow) return 4;
  for (int localRow = 0; localRow < rowCount; ++localRow) {
    const int row = rowStart + localRow;
    const size_t packedRowOffset = (size_t)row * packedInDim;
    const size_t scaleRowOffset = (size_t)row * groupsPerRow;
    const size_t outputRowOffset = (size_t)localRow * inDim;
    for (int packedCol = 0; packedCol < packedInDim; ++packedCol) {
      const uint32_t word = (uint32_t)packed[packedRowOffset + packedCol];
      const int baseInput = packedCol * 8;
      for (int k = 0; k < 8; ++k) {
        const int inputIndex = baseInput + k;
        const uint32_t nibble = (word >> (k * 4)) & 0x0fu;
        const int q = g4o_w4_nibble(nibble);
        const int group = inputIndex / groupSize;
        const float scale = scales[scaleRowOffset + group];
        /* JS: q * scale in binary64, stored to Float32Array.  q has <= 4
         * significant bits and scale (a widened bf16) <= 8, so the product is
         * exact in binary32 and both roundings agree. */
        out[outputRowOffset + inputIndex] = (float)((double)q * (double)scale);
      }
    }
  }
  return 0;
}

/* tfjs-backend-cpu BatchMatMul for y[M, N] = x[M, K] . w[N, K]^T with
 * blockSize 48 (third-party semantics, see the file header). */
static void tfjs_matmul_xwT(const float *x, int M, const float *w, int N, int K,
                            float *y, int y_stride) {
  const int bs = 48;
  for (int i = 0; i < M; ++i)
    for (int j = 0; j < N; ++j) y[(size_t)i * y_stride + j] = 0.0f;
  for (int i0 = 0; i0 < M; i0 += bs) {
    const int iB = i0 + bs < M ? i0 + bs : M;
    for (int j0 = 0; j0 < N; j0 += bs) {
      const int jB = j0 + bs < N ? j0 + bs : N;
      for (int k0 = 0; k0 < K; k0 += bs) {
        const int kB = k0 + bs < K ? k0 + bs : K;
        for (int i = i0; i < iB; ++i) {
          for (int j = j0; j < jB; ++j) {
            double sum = 0.0;
            for (int k = k0; k < kB; ++k)
              sum += (double)x[(size_t)i * K + k] * (double)w[(size_t)j * K + k];
            float *r = &y[(size_t)i * y_stride + j];
            *r = (float)((double)*r + sum);
          }
        }
      }
    }
  }
}

int g4o_w4_linear(const float *x, int M, const int32_t *packed,
                  const uint16_t *scales_bf16, int N, int K, int groupSize,
                  int chunk, float *y) {
  /* official-quantized-linear.js:82-128 */
  if (chunk <= 0) chunk = 256; /* outputChunkSize default, line 13 */
  if (K % 8 != 0) return 1;
  if (groupSize <= 0 || K % groupSize != 0) return 2;
  const int groups = K / groupSize;
  const size_t nscales = (size_t)N * groups;
  float *scales = (float *)malloc(nscales * sizeof(float));
  float *wchunk = (float *)malloc((size_t)chunk * K * sizeof(float));
  float *ychunk = (float *)malloc((size_t)M * chunk * sizeof(float));
  if (!scales || !wchunk || !ychunk) {
    free(scales);
    free(wchunk);
    free(ychunk);
    return -1;
  }
  for (size_t i = 0; i < nscales; ++i) scales[i] = g4o_bf16_to_f32(scales_bf16[i]);
  int rc = 0;
  for (int rowStart = 0; rowStart < N && rc == 0; rowStart += chunk) {
    const int rowCount = chunk < N - rowStart ? chunk : N - rowStart;
    rc = g4o_w4_dequant_rows(packed, (size_t)N * (K / 8), scales, nscales, N, K,
                             rowStart, rowCount, groupSize, wchunk);
    if (rc) break;
    tfjs_matmul_xwT(x, M, wchunk, rowCount, K, ychunk, rowCount);
    /* tf.concat(outputs, -1) */
    for (int i = 0; i < M; ++i)
      memcpy(&y[(size_t)i * N + rowStart], &ychunk[(size_t)i * rowCount],
             (size_t)rowCount * sizeof(float));
  }
  free(scales);
  free(wchunk);
  free(ychunk);
  return rc;
}

int g4o_w4_linear_mt(const float *x, int M, const int32_t *packed,
                     const uint16_t *scales_bf16, int N, int K, int groupSize,
                     int chunk, float *y, int threads) {
  /* official-quantized-linear.js:82-128, chunks in parallel */
  if (chunk <= 0) chunk = 256;
  if (K % 8 != 0) return 1;
  if (groupSize <= 0 || K % groupSize != 0) return 2;
  const int groups = K / groupSize;
  const size_t nscales = (size_t)N * groups;
  float *scales = (float *)malloc(nscales * sizeof(float));
  if (!scales) return -1;
  for (size_t i = 0; i < nscales; ++i) scales[i] = g4o_bf16_to_f32(scales_bf16[i]);
  const int nchunks = (N + chunk - 1) / chunk;
  int rc = 0;
  const int nt = g4o_omp_threads(threads);
#pragma omp parallel num_threads(nt) reduction(| : rc)
  {
    float *wchunk = (float *)malloc((size_t)chunk * K * sizeof(float));
    float *ychunk = (float *)malloc((size_t)M * chunk * sizeof(float));
    const int have = wchunk && ychunk;
    if (!have) rc |= 1 << 8;
    /* every thread of the team reaches the worksharing loop (its implicit
     * barrier); a thread without buffers only skips the loop bodies */
#pragma omp for schedule(dynamic, 1)
    for (int c = 0; c < nchunks; ++c) {
      if (!have) continue;
      const int rowStart = c * chunk;
      const int rowCount = chunk < N - rowStart ? chunk : N - rowStart;
      int r = g4o_w4_dequant_rows(packed, (size_t)N * (K / 8), scales, nscales, N, K,
                                  rowStart, rowCount, groupSize, wchunk);
      if (r) {
        rc |= r;
        continue;
      }
      tfjs_matmul_xwT(x, M, wchunk, rowCount, K, ychunk, rowCount);
      for (int i = 0; i < M; ++i)
        memcpy(&y[(size_t)i * N + rowStart], &ychunk[(size_t)i * rowCount],
               (size_t)rowCount * sizeof(float));
    }
    free(wchunk);
    free(ychunk);
  }
  free(scales);
  return rc ? (rc & 0xff ? rc & 0xff : -1) : 0;
}

int g4o_omp_threads(int threads) {
  return threads > 0 ? threads : omp_get_max_threads();
}

int g4o_w4_linear_f64(const float *x, int M, const int32_t *packed,
                      const uint16_t *scales_bf16, int N, int K, int groupSize,
                      double *y) {
  if (K % 8 != 0) return 1;
  if (groupSize <= 0 || K % groupSize != 0) return 2;
  const int groups = K / groupSize;
  double *w = (double *)malloc((size_t)K * sizeof(double));
  if (!w) return -1;
  for (int o = 0; o < N; ++o) {
    for (int k = 0; k < K; ++k) {
      const uint32_t word = (uint32_t)packed[(size_t)o * (K / 8) + k / 8];
      const int q = g4o_w4_nibble(word >> ((k % 8) * 4));
      w[k] = (double)q * (double)g4o_bf16_to_f32(scales_bf16[(size_t)o * groups + k / groupSize]);
    }
    for (int i = 0; i < M; ++i) {
      double s = 0.0;
      for (int k = 0; k < K; ++k) s += (double)x[(size_t)i * K + k] * w[k];
      y[(size_t)i * N + o] = s;
    }
  }
  free(w);
  return 0;
}

void g4o_ple_dequant_row(const uint8_t *packed_row, const uint16_t *scale_bits,
                         int width, float *out) {
  /* ple-w4-shard-reader.js:89-96 */
  for (int i = 0; i < width; ++i) {
    const uint32_t byte = packed_row[i >> 1];
    const uint32_t nibble = (i & 1) == 0 ? (byte & 0x0fu) : (byte >> 4);
    const int q = g4o_ple_nibble(nibble);
    const float scale = g4o_bf16_to_f32(scale_bits[i / 32]);
    out[i] = (float)((double)q * (double)scale);
  }
}

int g4o_ple_locate(long long id, int vocab, int rows_per_shard, int *shard,
                   int *local_row) {
  /* ple-w4-shard-reader.js:47-63 (Number.isInteger / range check, floor) */
  if (id < 0 || id >= vocab) return -1;
  const int s = (int)(id / rows_per_shard);
  if (shard) *shard = s;
  if (local_row) *local_row = (int)(id - (long long)s * rows_per_shard);
  return 0;
}

void g4o_ple_row_offsets(int vocab, int width, int rows_per_shard, int shard,
                         int local_row, size_t *packed_off, size_t *scale_off) {
  /* tools/build_ple_w4_full.py:99-100 (row sizes), 131-136 (shard rows),
   * 151-154 (packed block then scales block) */
  const size_t packed_row = (size_t)width / 2;
  const size_t scale_row = (size_t)(width / 32) * 2;
  const long long r0 = (long long)shard * rows_per_shard;
  const long long left = vocab - r0;
  const size_t rows = (size_t)(left < rows_per_shard ? left : rows_per_shard);
  const size_t shard_base = (size_t)r0 * (packed_row + scale_row);
  if (packed_off) *packed_off = shard_base + (size_t)local_row * packed_row;
  if (scale_off)
    *scale_off = shard_base + rows * packed_row + (size_t)local_row * scale_row;
}

int g4o_ple_gather(const uint8_t *table, int vocab, int width,
                   int rows_per_shard, const int32_t *ids, int n, float *out) {
  /* ple-w4-shard-reader.js:65-103 */
  for (int j = 0; j < n; ++j) {
    int shard, local;
    if (g4o_ple_locate(ids[j], vocab, rows_per_shard, &shard, &local)) return -1 - j;
    size_t po, so;
    g4o_ple_row_offsets(vocab, width, rows_per_shard, shard, local, &po, &so);
    /* new Uint16Array(scaleBuffer): little-endian bf16 bits */
    uint16_t *sb = (uint16_t *)malloc((size_t)(width / 32) * 2);
    if (!sb) return -1 - n;
    memcpy(sb, table + so, (size_t)(width / 32) * 2);
    g4o_ple_dequant_row(table + po, sb, width, out + (size_t)j * width);
    free(sb);
  }
  return 0;
}

int g4o_ple_gather_mt(const uint8_t *table, int vocab, int width, int rows_per_shard,
                      const int32_t *ids, int n, float *out, int threads) {
  /* g4o_ple_gather with the ids over OpenMP threads (the all-core CPU
   * baseline): every row is the same computation, so the result is too */
  for (int j = 0; j < n; ++j)
    if (g4o_ple_locate(ids[j], vocab, rows_per_shard, NULL, NULL)) return -1 - j;
  int rc = 0;
#pragma omp parallel num_threads(g4o_omp_threads(threads)) reduction(| : rc)
  {
    uint16_t *sb = (uint16_t *)malloc((size_t)(width / 32) * 2);
    if (!sb) rc |= 1;
#pragma omp for schedule(static)
    for (int j = 0; j < n; ++j) {
      if (!sb) continue;
      int shard, local;
      g4o_ple_locate(ids[j], vocab, rows_per_shard, &shard, &local);
      size_t po, so;
      g4o_ple_row_offsets(vocab, width, rows_per_shard, shard, local, &po, &so);
      memcpy(sb, table + so, (size_t)(width / 32) * 2);
      g4o_ple_dequant_row(table + po, sb, width, out + (size_t)j * width);
    }
    free(sb);
  }
  return rc ? -1 - n : 0;
}

void g4o_ple_quantize_rows(const float *rows, int nrows, int width,
                           uint8_t *packed, uint16_t *scale_bits) {
  /* tools/build_ple_w4_full.py:48-60 */
  const int G = 32, QMAX = 7;
  const int groups = width / G;
  for (int b = 0; b < nrows; ++b) {
    int8_t *q = (int8_t *)malloc((size_t)width);
    for (int g = 0; g < groups; ++g) {
      const float *x = rows + (size_t)b * width + (size_t)g * G;
      float maxabs = 0.0f;
      for (int i = 0; i < G; ++i) {
        const float a = fabsf(x[i]);
        if (a > maxabs) maxabs = a;
      }
      /* float32 maxabs / 7 (numpy keeps float32), 1.0 for an all-zero group */
      const float s = maxabs == 0.0f ? 1.0f : maxabs / (float)QMAX;
      const uint16_t sbits = g4o_f32_to_bf16(s);
      scale_bits[(size_t)b * groups + g] = sbits;
      const float stored = g4o_bf16_to_f32(sbits);
      for (int i = 0; i < G; ++i) {
        float t = nearbyintf(x[i] / stored); /* np.rint: half to even */
        if (t < -QMAX) t = -QMAX;
        if (t > QMAX) t = QMAX;
        q[g * G + i] = (int8_t)t;
      }
    }
    for (int i = 0; i < width / 2; ++i) {
      const uint8_t lo = (uint8_t)(q[2 * i] & 0x0f);
      const uint8_t hi = (uint8_t)(q[2 * i + 1] & 0x0f);
      packed[(size_t)b * (width / 2) + i] = (uint8_t)(lo | (hi << 4));
    }
    free(q);
  }
}

void g4o_bf16_head(const float *x, const uint16_t *E, int rows, int K,
                   float scale, float softcap, float *out) {
  /* gpu-runtime.js:1273-1276: acc += x[k] * bf(w); raw = acc * scale;
   * out = tanh(raw / softcap) * softcap (tfjs-reference-engine.js:354-359:
   * matMul, div(30), tanh, mul(30) - each an FP32 tensor op) */
  for (int r = 0; r < rows; ++r) {
    float acc = 0.0f;
    for (int k = 0; k < K; ++k) {
      const float p = x[k] * g4o_bf16_to_f32(E[(size_t)r * K + k]);
      acc = acc + p;
    }
    const float raw = acc * scale;
    if (softcap > 0.0f) {
      const float t = raw / softcap;
      const float th = (float)tanh((double)t);
      out[r] = th * softcap;
    } else {
      out[r] = raw;
    }
  }
}

int g4o_topk(const float *logits, int n, int k, int32_t *ids, float *vals) {
  /* gpu-runtime.js:1396-1425: push, stable sort descending, pop. */
  if (k <= 0) return 0;
  int len = 0;
  for (int i = 0; i < n; ++i) {
    const float v = logits[i];
    if (!isfinite(v)) continue;
    if (len < k || v > vals[len - 1]) {
      /* stable insertion: after every kept value >= v */
      int pos = len;
      while (pos > 0 && vals[pos - 1] < v) --pos;
      const int keep = len < k ? len + 1 : k;
      for (int t = keep - 1; t > pos; --t) {
        vals[t] = vals[t - 1];
        ids[t] = ids[t - 1];
      }
      if (pos < keep) {
        vals[pos] = v;
        ids[pos] = i;
      }
      len = keep;
    }
  }
  return len;
}
