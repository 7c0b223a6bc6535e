/*
 * g4_oracle.h - CPU restatement of the gemma4-js W4A16 / PLE hot path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE.  Only the tests, the smoke check
 * and the benchmark's CPU-baseline leg load this library, and only to check
 * results against: the product path (libg4hip) never calls it and never
 * falls back to it.
 *
 * Every function restates one piece of the reference, cited by file:line
 * (paths relative to the gemma4-js repository root).  Plain C99, scalar,
 * single-threaded (the reference's own CPU path, TF.js on tfjs-backend-cpu,
 * is single-threaded JavaScript), except g4o_w4_linear_mt, which shares the
 * output chunks of the same computation out over OpenMP threads.
 */
#ifndef G4_ORACLE_H
#define G4_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* bf16 bits -> float: bits << 16 (gpu-runtime.js:1058-1066 bf16ToF32;
 * ple-w4-shard-reader.js:2-7 bf16BitsToFloat32). */
float g4o_bf16_to_f32(uint16_t bits);

/* roundFloat32ToBF16 (official-w4a16.js:34-48) returning the bf16 bits:
 * bits + 0x7fff + lsb, keep the upper half.  Also the builder's
 * f32_to_bf16_bits_rne (tools/build_ple_w4_full.py:42-45). */
uint16_t g4o_f32_to_bf16(float v);

/* Array forms of the two conversions above (no float->double round trip,
 * so NaN payloads survive). */
void g4o_bf16_to_f32_array(const uint16_t *bits, size_t n, float *out);
void g4o_f32_to_bf16_array(const float *v, size_t n, uint16_t *out);

/* signedInt4FromNibble (official-w4a16.js:15-19): (n & 15) - 8. */
int g4o_w4_nibble(uint32_t nibble);

/* PLE two's-complement nibble (ple-w4-shard-reader.js:92;
 * gpu-runtime.js:225-227 signed4): n >= 8 ? n - 16 : n. */
int g4o_ple_nibble(uint32_t nibble);

/* dequantizeOfficialW4A16Rows (official-w4a16.js:50-101), including its
 * validation (returns 1..4 for the four errors it throws, 0 on success):
 *   1 "inDim must be divisible by 8."       2 "... divisible by groupSize."
 *   3 "packedValues length mismatch."       4 "scale length mismatch."
 * packed: I32 [outDim, inDim/8]; scales: FP32 [outDim, inDim/groupSize];
 * out: FP32 [rowCount, inDim]. */
int g4o_w4_dequant_rows(const int32_t *packed, size_t packed_len,
                        const float *scales, size_t scales_len, int outDim,
                        int inDim, int rowStart, int rowCount, int groupSize,
                        float *out);

/* OfficialW4A16Linear.apply (official-quantized-linear.js:82-128):
 * per output chunk of `chunk` rows (256 by default, line 13) dequantize to
 * FP32, then y[:, chunk] = x . W_chunk^T in FP32 (tf.matMul(x, w, false,
 * true), line 116; accumulation in k order), concatenated along the last
 * axis.  Scales arrive as bf16 bits and are widened first, as the TF.js
 * loader does before setOfficialWeights (which requires a Float32Array).
 * x: FP32 [M, K]; y: FP32 [M, N].  Returns the dequant error code. */
int g4o_w4_linear(const float *x, int M, const int32_t *packed,
                  const uint16_t *scales_bf16, int N, int K, int groupSize,
                  int chunk, float *y);

/* g4o_w4_linear with the output chunks shared out over `threads` OpenMP
 * threads (threads <= 0: the OpenMP default).  Each output element goes
 * through exactly the same dequant and k-block sequence as in
 * g4o_w4_linear, so the result is bit-identical; only the chunks run
 * concurrently.  The benchmark's all-core CPU leg. */
int g4o_w4_linear_mt(const float *x, int M, const int32_t *packed,
                     const uint16_t *scales_bf16, int N, int K, int groupSize,
                     int chunk, float *y, int threads);

/* Threads an OpenMP parallel region of g4o_w4_linear_mt gets for `threads`. */
int g4o_omp_threads(int threads);

/* The same product in double precision (the error yardstick). */
int g4o_w4_linear_f64(const float *x, int M, const int32_t *packed,
                      const uint16_t *scales_bf16, int N, int K, int groupSize,
                      double *y);

/* PLE row dequant (ple-w4-shard-reader.js:85-96; the WGSL twin is
 * gpu-runtime.js:218-256): out[i] = q(nibble i) * bf16(scale[i / 32]),
 * element i = nibble (i & 1) of byte i >> 1, low nibble first. */
void g4o_ple_dequant_row(const uint8_t *packed_row, const uint16_t *scale_bits,
                         int width, float *out);

/* _location (ple-w4-shard-reader.js:47-63; gpu-runtime.js:463-485):
 * returns 0 and the shard/local row, or -1 for an id outside [0, vocab). */
int g4o_ple_locate(long long id, int vocab, int rows_per_shard, int *shard,
                   int *local_row);

/* Byte offsets of a row inside its shard file (ple-w4-shard-reader.js:72-73
 * with the builder's packed_offset = 0, scales_offset = rows * packed_row,
 * tools/build_ple_w4_full.py:99-100, 151-154, 165-169). */
void g4o_ple_row_offsets(int vocab, int width, int rows_per_shard, int shard,
                         int local_row, size_t *packed_off, size_t *scale_off);

/* readRows (ple-w4-shard-reader.js:65-103) over a table held as the
 * concatenation of its shard files.  Returns 0, or -1 - j for the first
 * out-of-range id at position j (the reference throws there). */
int g4o_ple_gather(const uint8_t *table, int vocab, int width,
                   int rows_per_shard, const int32_t *ids, int n, float *out);
/* g4o_ple_gather with the ids spread over OpenMP threads (0: all); the same
 * output.  Every id is range-checked first. */
int g4o_ple_gather_mt(const uint8_t *table, int vocab, int width, int rows_per_shard,
                      const int32_t *ids, int n, float *out, int threads);

/* quantize_batch (tools/build_ple_w4_full.py:48-60): per 32-column group
 * s = maxabs/7 (1.0 when maxabs == 0), stored as bf16 (RNE), then
 * q = clip(rint(x / s_bf16), -7, 7) (rint = round half to even), packed as
 * two's-complement nibbles, low nibble first. */
void g4o_ple_quantize_rows(const float *rows, int nrows, int width,
                           uint8_t *packed, uint16_t *scale_bits);

/* BF16_HEAD_SHADER (gpu-runtime.js:1265-1277) / computeTiedHeadLogits
 * (tfjs-reference-engine.js:348-376): out[r] = softcap *
 * tanh((scale * sum_k x[k] * E[r,k]) / softcap), FP32 accumulate in k
 * order; softcap <= 0 returns the raw product. */
void g4o_bf16_head(const float *x, const uint16_t *E, int rows, int K,
                   float scale, float softcap, float *out);

/* topK (gpu-runtime.js:1396-1425): the k largest finite logits, largest
 * first; on equal values the lower index comes first (insertion order kept
 * by a stable sort, and an equal value never displaces a kept one).
 * Returns the number found (0 means "no finite logits", which throws). */
int g4o_topk(const float *logits, int n, int k, int32_t *ids, float *vals);

#ifdef __cplusplus
}
#endif

#endif /* G4_ORACLE_H */
