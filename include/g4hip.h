/*
 * g4hip.h - C ABI of the MI355X (gfx950) W4A16 / PLE hot path of gemma4-js.
 *
 * This library replaces the WebGPU buffer + dispatch layer of
 * custom-webgpu/gpu-runtime.js and the hot-path kernels behind GPUOps.w4,
 * the PLE W4 gather-dequant and the tied BF16 LM head.  Every entry point
 * takes plain pointers and sizes, returns an int status (G4_OK == 0) and,
 * on failure, leaves a message for g4_last_error().  The Node binding turns
 * a non-zero status into `throw new Error(g4_last_error())`, which is the
 * reference's own error convention (synchronous JS throws for shape, range
 * and capacity errors, e.g. gpu-runtime.js:58, 466-470).
 *
 * Ordering: all device work is enqueued on ONE HIP stream owned by the
 * library, so the reference's WebGPU queue-order guarantees carry over
 * (gpu-runtime.js:328-332, 393).  Calls that read results back to the host
 * (g4_download) wait for that stream.
 *
 * Device pointers: "device pointer" arguments must point into memory from
 * g4_alloc (or any other HIP device allocation).  Before a launch the library
 * checks that every operand range lies inside its allocation, so a wrong
 * size is reported as G4_E_RANGE instead of faulting the GPU.
 *
 * Not thread-safe: like the reference (one JS thread), callers serialise.
 */
#ifndef G4HIP_H
#define G4HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define G4_OK 0
#define G4_E_ARG 1    /* bad shape / geometry / dtype argument               */
#define G4_E_RANGE 2  /* index or byte range outside its buffer or table     */
#define G4_E_STATE 3  /* library not initialised, or object already freed    */
#define G4_E_HIP 4    /* a HIP runtime call failed (message has the details)  */
#define G4_E_NOMEM 5  /* device allocation failed                            */

/* ---- element types of activations and outputs -------------------------- */
#define G4_F32 0  /* IEEE binary32, as every reference activation buffer   */
#define G4_BF16 1 /* bfloat16 bits (upper half of binary32)                 */

/* ---- device and queue --------------------------------------------------- */

/* Select the HIP device and create the library's stream.  Stands in for
 * navigator.gpu.requestAdapter()/requestDevice() (custom-webgpu/main.js:96-114).
 * Calling it again with the same device is a no-op. */
int g4_init(int device);

/* Message of the last failing call on this thread ("" if none). */
const char *g4_last_error(void);

/* Device name, compute-unit count, HBM bytes and peak engine clock (kHz). */
int g4_device_info(char *name, size_t name_len, int *cu_count,
                   size_t *hbm_bytes, int *clock_khz);

/* createBuffer(device, size, usage, label) (gpu-runtime.js:8-12): the size is
 * rounded up to 4 bytes like align4(), and the buffer starts zero-filled as
 * a WebGPU buffer does. */
int g4_alloc(size_t bytes, void **dptr);

/* GPUBuffer.destroy().  Stream-ordered: work already enqueued that uses the
 * buffer completes first. */
int g4_free(void *dptr);

/* queue.writeBuffer via uploadBytes/uploadF32/uploadU32 (gpu-runtime.js:14-26):
 * copy n host bytes into the device buffer at byte offset dst_off.  The host
 * memory may be reused as soon as the call returns. */
int g4_upload(void *dst, size_t dst_off, const void *src, size_t n);

/* readF32 (gpu-runtime.js:28-38): wait for the queue, then copy n bytes from
 * the device buffer at src_off into host memory. */
int g4_download(const void *src, size_t src_off, void *dst, size_t n);

/* encoder.copyBufferToBuffer (gemma4-webgpu.js:131-133, 406), stream-ordered. */
int g4_copy(void *dst, size_t dst_off, const void *src, size_t src_off,
            size_t n);

/* device.queue.onSubmittedWorkDone(): block until the queue is drained. */
int g4_sync(void);

/* The library's hipStream_t (as void*), for callers that time or order their
 * own work against it. */
void *g4_stream(void);

/* ---- command encoders ------------------------------------------------------
 * device.createCommandEncoder() / encoder.finish() / device.queue.submit()
 * (gemma4-webgpu.js:316-323, 339-358): between g4_encoder_begin and
 * g4_encoder_finish, kernel-launching calls (g4_w4_linear, g4_w4_linear_multi,
 * g4_w4_dequant, g4_ple_gather_dev, g4_bf16_head, g4_copy) are recorded instead
 * of run; g4_submit replays the recording on the queue (a HIP graph).  Calls that
 * must wait for the device or move host memory (g4_alloc, g4_free,
 * g4_upload, g4_download, g4_sync, g4_ple_gather with host ids, loads) fail
 * with G4_E_STATE while an encoder is open.  Unlike a WebGPU command buffer,
 * a finished recording may be submitted any number of times, also after
 * later calls made the library's internal scratch grow: scratch outgrown
 * while a recording exists is kept until the last recording is freed. */
typedef struct g4_cmdbuf g4_cmdbuf;
int g4_encoder_begin(void);
int g4_encoder_finish(g4_cmdbuf **out);
int g4_submit(const g4_cmdbuf *cb);
int g4_cmdbuf_free(g4_cmdbuf *cb);

/* hipEvent helpers on the library's stream (timing only). */
int g4_event_create(void **ev);
int g4_event_record(void *ev);
int g4_event_elapsed_ms(void *start, void *stop, float *ms);
int g4_event_destroy(void *ev);

/* ---- W4A16 group-32 linear --------------------------------------------- */

typedef struct g4_w4 g4_w4;

/* GPUW4Linear.load (gpu-runtime.js:1385-1392).  `packed` and `scales` are the
 * host bytes of a compressed-tensors pair exactly as stored in the checkpoint
 * (official-w4a16.js:4-13):
 *   weight_packed  I32  [out_dim, in_dim/8]   nibble k of word j is input 8j+k,
 *                                             low nibble first, value = nibble-8
 *   weight_scale   BF16 [out_dim, in_dim/group]
 * in_dim must be a multiple of 8 and of `group`; group must be 32 (the only
 * group size of the checkpoint; official-w4a16.js:56-61 validation).  The
 * weights are uploaded once and re-laid out on the device for the kernels;
 * the handle owns that memory until g4_w4_free. */
int g4_w4_load(const void *packed, const void *scales, int out_dim, int in_dim,
               int group, g4_w4 **out);

/* g4_w4_load from DEVICE memory (same layouts): for weights produced on the
 * device, e.g. by g4_fill_random, or already staged there.  Synchronises. */
int g4_w4_load_dev(const void *packed_dev, const void *scales_dev, int out_dim,
                   int in_dim, int group, g4_w4 **out);

/* g4_w4_load / g4_w4_load_dev with options (no reference counterpart; the
 * reference keeps one buffer per tensor, gpu-runtime.js:1385-1392):
 *   G4_W4_SRC_DEVICE     packed and scales are device pointers
 *   G4_W4_NO_GEMM_TILES  do not build the prefill GEMM's stage-major tile copy
 *                        of the words and scales (about half the handle's
 *                        device bytes).  For weights that only ever run the
 *                        decode GEMV; a prefill call on such a weight takes the
 *                        row-major MFMA kernel instead (same results to FP32
 *                        rounding, slower at large row counts). */
#define G4_W4_SRC_DEVICE 1
#define G4_W4_NO_GEMM_TILES 2
int g4_w4_load_opts(const void *packed, const void *scales, int out_dim, int in_dim,
                    int group, int flags, g4_w4 **out);

/* GPUW4Linear.dispose(). */
int g4_w4_free(g4_w4 *w);

/* out_dim, in_dim, group and the device bytes the handle holds. */
int g4_w4_info(const g4_w4 *w, int *out_dim, int *in_dim, int *group,
               size_t *device_bytes);

/* GPUOps.w4 (gpu-runtime.js:1316-1324, W4_SHADER 1068-1102) and the oracle
 * OfficialW4A16Linear.apply (official-quantized-linear.js:82-128):
 *   y[r, o] = sum_k x[r, k] * (nibble(o, k) - 8) * scale[o, k/32]
 * x: device [rows, in_dim] of x_dtype; y: device [rows, out_dim] of y_dtype.
 * Accumulation is FP32.  rows >= 1; small row counts take the streaming
 * GEMV kernel, large ones the MFMA GEMM kernel. */
int g4_w4_linear(const g4_w4 *w, const void *x, int x_dtype, int rows,
                 void *y, int y_dtype);

/* No counterpart in the reference.  g4_w4_linear for callers that cannot
 * allocate device memory: code under HIP graph capture (a g4 encoder), tight
 * serving loops, harnesses that forbid hipMalloc.  Same arguments, kernels
 * and results; the prefill GEMM path (rows > 4, or an in_dim beyond the GEMV
 * staging) takes its x' staging, row exponents and K-slice partial sums from
 * a static 64 MiB device array instead of the library's growing scratch, so
 * the call never allocates or frees.  A call whose scratch would exceed
 * 64 MiB (e.g. 4096 FP32 rows of in_dim 4096) fails with G4_E_ARG and a
 * message giving the bytes it needs.  Every call on one GPU shares that
 * GPU's array: calls whose device work overlaps (replays of recordings made
 * from it on other streams) race; calls enqueued on the library's one stream
 * run in order and are safe. */
int g4_w4_linear_noalloc(const g4_w4 *w, const void *x, int x_dtype, int rows,
                         void *y, int y_dtype);

/* Consecutive GPUOps.w4 dispatches over one input (gemma4-webgpu.js:225,
 * 237-238 for q/k/v and 280-281 for gate/up): y[i] = x * W[i]^T for i < n,
 * 1 <= n <= 3, every W[i] of the same in_dim, outputs as g4_w4_linear's.
 * One activation row runs the n GEMVs as one launch; more than 4 rows share
 * one activation pre-pass and, when the weights' tiles fill the GPU, one GEMM
 * launch; 2-4 rows take g4_w4_linear per weight.  The outputs must not
 * overlap x or each other. */
int g4_w4_linear_multi(const g4_w4 *const *w, int n, const void *x, int x_dtype,
                       int rows, void *const *y, int y_dtype);

/* No counterpart in the reference: a diagnostic of the decode GEMV.  One
 * activation row through the row-split kernel that g4_w4_linear(rows = 1)
 * runs for in_dim 1536 and 2048, with the same output, plus clock stamps:
 * lane 0 of every wave writes 5 values of the 100 MHz real-time clock to
 * stamps[wave * 5 + 0..4]: the wave's start, its x chunks staged in LDS, the
 * staging barrier passed, all of its weight loads landed (the stamp waits
 * for them, so group j's arithmetic no longer overlaps the later groups'
 * loads), and its output store issued.  *waves receives the launch's wave
 * count; with stamps null nothing is launched (a size query).  Other in_dims
 * fail with G4_E_ARG. */
int g4_w4_gemv_stamps(const g4_w4 *w, const void *x, int x_dtype, void *y, int y_dtype,
                      uint64_t *stamps, int *waves);

/* dequantizeOfficialW4A16Rows (official-w4a16.js:50-101) on the device:
 * out[r, k] = (nibble - 8) * scale for rows row_start..row_start+row_count-1,
 * as FP32 (exact) or as BF16 rounded to nearest even, which is
 * roundFloat32ToBF16 (official-w4a16.js:34-48). */
int g4_w4_dequant(const g4_w4 *w, int row_start, int row_count, void *out,
                  int out_dtype);

/* ---- PLE W4 gather-dequant ---------------------------------------------- */

typedef struct g4_ple g4_ple;

/* W4PleShardBundle geometry (gpu-runtime.js:413-461): a device-resident table
 * of `vocab` rows of `width` signed W4 values, group 32, stored as the
 * builder's shards (tools/build_ple_w4_full.py:130-170): shard s holds rows
 * [s*rows_per_shard, ...), its packed block (rows x width/2 bytes, low nibble
 * first, two's-complement nibbles) followed by its scales block
 * (rows x width/32 BF16). */
int g4_ple_create(int vocab, int width, int group, int rows_per_shard,
                  g4_ple **out);

/* Copy the bytes of one shard file (exact builder layout) into the table. */
int g4_ple_upload_shard(g4_ple *t, int shard, const void *bytes, size_t n);

/* g4_ple_upload_shard from DEVICE memory (stream-ordered, no wait). */
int g4_ple_upload_shard_dev(g4_ple *t, int shard, const void *bytes_dev,
                            size_t n);

/* Number of shards and the byte size of shard `shard`. */
int g4_ple_shard_bytes(const g4_ple *t, int shard, int *num_shards,
                       size_t *bytes);

int g4_ple_free(g4_ple *t);

/* quantize_batch and the shard layout of the PLE builder
 * (tools/build_ple_w4_full.py:48-60, 130-170) on the device.  `rows` BF16
 * rows [rows, width] (device, 16-byte aligned, width a multiple of 32)
 * become the bytes of one shard file at shard_dev (device, 16-byte aligned,
 * rows * (width/2 + width/16) bytes): the packed block, q = clip(rint(x / s),
 * -7, 7) as two's-complement nibbles, low nibble first (rint rounds half to
 * even), then the scales block, s = bf16_rne(max |x| / 7) per 32-column group
 * (1.0 for an all-zero group), q computed against that stored BF16 scale.
 * Finite inputs; stream-ordered, no wait. */
int g4_ple_quantize_rows(const void *rows_bf16, int rows, int width, void *shard_dev);

/* The whole table from a dense BF16 embed_tokens_per_layer [vocab, width] in
 * device memory (the builder's source tensor): every shard quantized in
 * place, the bytes the builder's shard files would hold, so a model that has
 * only the dense rows (the inputBuffers fallback, gemma4-webgpu.js:198-213)
 * can gather from a W4 table instead.  Stream-ordered, no wait. */
int g4_ple_quantize_table(g4_ple *t, const void *dense_bf16);

/* W4PleShardBundle.rowsToGpu (gpu-runtime.js:487-527) with the dequant shader
 * (gpu-runtime.js:218-256) and the oracle LocalPleW4ShardReader.readRows
 * (ple-w4-shard-reader.js:65-103): out[j, i] = q(ids[j], i) * scale, with
 * q the two's-complement nibble.  `ids` is HOST memory; every id is checked
 * against [0, vocab) first, as _location does (gpu-runtime.js:463-485), and
 * an out-of-range id fails with G4_E_RANGE before anything is launched.
 * out: device [n, width] FP32 or BF16 (round to nearest even). */
int g4_ple_gather(const g4_ple *t, const int32_t *ids, int n, void *out,
                  int out_dtype);

/* Same gather with `ids` already in DEVICE memory (e.g. a token chosen on the
 * device).  Ids cannot be checked on the host here: a row whose id is outside
 * [0, vocab) is filled with quiet NaN and no table memory is touched. */
int g4_ple_gather_dev(const g4_ple *t, const int32_t *ids_dev, int n,
                      void *out, int out_dtype);

/* ---- BF16 tied LM head ---------------------------------------------------- */

/* GPUOps.headChunk (gpu-runtime.js:1370-1376) with BF16_HEAD_SHADER
 * (gpu-runtime.js:1265-1277); oracle computeTiedHeadLogits
 * (tfjs-reference-engine.js:348-376):
 *   out[r] = softcap * tanh((scale * sum_k x[k] * E[r, k]) / softcap)
 * x: device FP32 [in_dim]; E: device BF16 [rows, in_dim]; out: device FP32
 * [rows] (pass the chunk's offset into the logits buffer as the pointer).
 * softcap <= 0 disables the cap. */
int g4_bf16_head(const float *x, const void *E, int rows, int in_dim,
                 float *out, float scale, float softcap);

/* ---- remaining GPUOps of a decoder layer ---------------------------------
 * FP32 device buffers throughout, as every activation of the reference.  The
 * caller allocates the output (the reference's ops allocate it and hand it
 * back; the Node binding does that part).  Reductions are tree-shaped, so
 * results match the shaders to FP32 rounding rather than bit for bit. */

/* GPUOps.rms / RMS_SHADER (gpu-runtime.js:1104-1118, 1325-1332):
 *   y[r, i] = x[r, i] / sqrt(mean_k x[r, k]^2 + eps) * (scale ? scale[i] : 1)
 * scale may be NULL (the shader's has_scale = 0).  The reference uses eps 1e-6. */
int g4_rms(const float *x, int rows, int width, const float *scale, float eps,
           float *y);

/* GPUOps.addScale / ADD_SCALE_SHADER (gpu-runtime.js:1120-1128, 1333-1336):
 * y[i] = (a[i] + b[i]) * scale. */
int g4_add_scale(const float *a, const float *b, size_t n, float scale, float *y);

/* GPUOps.scale / SCALE_SHADER (gpu-runtime.js:1130-1137, 1337-1340):
 * y[i] = a[i] * scale. */
int g4_scale(const float *a, size_t n, float scale, float *y);

/* GPUOps.geluMul / GELU_MUL_SHADER (gpu-runtime.js:1139-1157, 1341-1344):
 * y[i] = gelu_tanh(gate[i]) * up[i], the tanh argument clamped to [-10, 10]. */
int g4_gelu_mul(const float *gate, const float *up, size_t n, float *y);

/* GPUOps.geluPle / GELU_PLE_SHADER (gpu-runtime.js:1159-1173, 1345-1348):
 * y[r, d] = gelu_tanh(gate[r, d]) * ple[r, layer, d]; ple is [rows, layers,
 * width] (the reference: width 256, layers 35). */
int g4_gelu_ple(const float *gate, const float *ple, int rows, int layer,
                int width, int layers, float *y);

/* GPUOps.normRope / NORM_ROPE_SHADER (gpu-runtime.js:1175-1202, 1349-1356):
 * per (row, head) RMS norm with scale[head_dim], then rotate-half RoPE of the
 * first rope_angles pairs (d, d + head_dim/2) at position pos0 + row with
 * theta = pos / base^(2 pair / head_dim).  The reference passes
 * rope_angles = floor(ropeProp * head_dim / 2) and eps 1e-6.
 * head_dim even and <= 512. */
int g4_norm_rope(const float *x, int rows, int heads, int head_dim, int pos0,
                 const float *scale, int rope_angles, float base, float eps,
                 float *y);

/* GPUOps.attention (gpu-runtime.js:1357-1365): QK_SHADER, SOFTMAX_SHADER and
 * ATTN_OUT_SHADER (1204-1248) as one split-key pass plus a merge.
 *   q [qrows, heads, head_dim]; k, v [keylen, head_dim] (one KV head shared
 *   by all query heads); y [qrows, heads, head_dim].
 * Query row r sits at position qpos0 + r and sees keys key <= qpos0 + r, and
 * with `sliding` only those with key + window > qpos0 + r.  No 1/sqrt(d)
 * factor (the shader has none).  heads <= 8; head_dim 64, 128, 256 or 512. */
int g4_attention(const float *q, const float *k, const float *v, int qrows,
                 int heads, int head_dim, int keylen, int qpos0, int sliding,
                 int window, float *y);

/* GPUOps.pleMix / PLE_MIX_SHADER (gpu-runtime.js:1250-1263, 1366-1369):
 * for each [width] chunk c of proj ([rows, layers, width]):
 *   y = (rms(proj_c) * norm_scale + token_ple_c * 16) / sqrt(2). */
int g4_ple_mix(const float *proj, const float *norm_scale,
               const float *token_ple, int rows, int width, int layers,
               float *y);

/* Embedding rows (Gemma4WebGPU.inputBuffers + ops.scale,
 * gemma4-webgpu.js:198-215, 318): y[r, i] = float(E[ids[r], i]) * scale.
 * E: device BF16 [vocab, width]; ids: DEVICE int32 [n].  An id outside
 * [0, vocab) yields a NaN row (no table memory is read). */
int g4_embed(const void *E, int vocab, int width, const int32_t *ids_dev,
             int n, float scale, float *y);

/* Greedy pick of Gemma4WebGPU.greedy (gemma4-webgpu.js:441-481) with topK
 * (gpu-runtime.js:1396-1425) done on the device: out_dev[0] = the first
 * index of the largest finite x[i], or -1 if none is finite (topK throws). */
int g4_argmax(const float *x, int n, int32_t *out_dev);

/* ---- synthetic data (random-init models) ----------------------------------
 * No reference counterpart: the benchmarks run random-init weights of the
 * checkpoint's shapes, generated on the device.  Fills `count` elements of
 * `kind` at dst with a counter-based generator (reproducible per seed):
 *   G4_RAND_W4_PACKED        uint32 words, 8 nibbles uniform in [1, 15]
 *                            (q = nibble - 8 in [-7, 7]); sigma unused
 *   G4_RAND_PLE_PACKED       bytes, 2 two's-complement nibbles in [-7, 7]
 *   G4_RAND_BF16_ABS_NORMAL  bf16 |N(0,1)| * sigma (group scales)
 *   G4_RAND_BF16_NORMAL      bf16 N(0,1) * sigma (embeddings)
 *   G4_RAND_F32_NORMAL       float N(0,1) * sigma
 *   G4_RAND_W4_PACKED_FULL   uint32 words, 8 nibbles uniform in [0, 15]: the
 *                            format's whole q range [-8, 7] (nibble 0 = -8)
 *   G4_RAND_PLE_PACKED_FULL  bytes, 2 nibbles uniform in [0, 15]: q in
 *                            [-8, 7] (two's-complement nibble 8 = -8) */
#define G4_RAND_W4_PACKED 0
#define G4_RAND_PLE_PACKED 1
#define G4_RAND_BF16_ABS_NORMAL 2
#define G4_RAND_BF16_NORMAL 3
#define G4_RAND_F32_NORMAL 4
#define G4_RAND_W4_PACKED_FULL 5
#define G4_RAND_PLE_PACKED_FULL 6
int g4_fill_random(void *dst, size_t count, int kind, uint64_t seed,
                   float sigma);

/* ---- decoder engine ----------------------------------------------------------
 * Gemma4WebGPU (custom-webgpu/gemma4-webgpu.js:139-502) on the kernels above:
 * load/forward/logits/greedy with the reference's op sequence (encodeLayer
 * 215-301), KV caches per non-shared layer (KVCache, 117-137) and the same
 * append/capacity errors.  Token position and the chosen token stay in device
 * memory; g4_gemma_decode replays one recorded decode step (a HIP graph) per
 * token.  Weights are borrowed: the g4_w4 / g4_ple handles and the BF16
 * embedding must outlive the model.  Norm vectors are copied in. */
#define G4_GEMMA_MAX_LAYERS 64

typedef struct {
  int hidden;                          /* 1536 (HIDDEN); multiple of 32, <= 2048 */
  int heads;                           /* query heads, <= 8; one KV head      */
  int ple_dim;                         /* 256 (PLE)                           */
  int vocab;                           /* 262144                              */
  int layers;                          /* 35 (LAYERS)                         */
  int max_seq;                         /* KV capacity in positions (maxSeq)   */
  int window;                          /* sliding window, 512                 */
  float eps;                           /* RMS epsilon, 1e-6                   */
  float softcap;                       /* final logit softcap, 30             */
  int head_dim[G4_GEMMA_MAX_LAYERS];   /* spec(i).headDim: 256 or 512         */
  int intermediate[G4_GEMMA_MAX_LAYERS];
  int full[G4_GEMMA_MAX_LAYERS];       /* 1: global attention, 0: sliding     */
  int kv_source[G4_GEMMA_MAX_LAYERS];  /* -1: own k/v; else the earlier layer
                                          whose cache is reused (spec.shared) */
  float rope_base[G4_GEMMA_MAX_LAYERS];
  float rope_prop[G4_GEMMA_MAX_LAYERS];
} g4_gemma_config;

/* Fills the Gemma-4-E2B schedule of spec(i) (gemma4-webgpu.js:12, 65-77):
 * every 5th layer global with head_dim 512 and RoPE (1e6, 0.25), the rest
 * sliding with head_dim 256 and RoPE (1e4, 1.0); intermediate 6144 for
 * layers 0-14 and 12288 after; layers 15-34 reuse the caches of layer 13
 * (sliding) and 14 (global). */
int g4_gemma_e2b_config(int max_seq, g4_gemma_config *cfg);

typedef struct g4_gemma g4_gemma;
int g4_gemma_create(const g4_gemma_config *cfg, g4_gemma **out);
int g4_gemma_free(g4_gemma *m);

/* Projections of linearsForLayer (gemma4-webgpu.js:79-96); layer -1 with
 * G4_PROJ_TOP is per_layer_model_projection.  Shapes are checked. */
#define G4_PROJ_Q 0
#define G4_PROJ_K 1
#define G4_PROJ_V 2
#define G4_PROJ_O 3
#define G4_PROJ_GATE 4
#define G4_PROJ_UP 5
#define G4_PROJ_DOWN 6
#define G4_PROJ_PLE_GATE 7
#define G4_PROJ_PLE_PROJ 8
#define G4_PROJ_TOP 9
int g4_gemma_set_linear(g4_gemma *m, int layer, int which, const g4_w4 *w);

/* Norm weights of loadLayer (gemma4-webgpu.js:104-113) as FP32 host arrays;
 * layer -1 takes per_layer_projection_norm and the final norm (151-156). */
#define G4_NORM_INPUT 0
#define G4_NORM_POST_ATTN 1
#define G4_NORM_PRE_FFW 2
#define G4_NORM_POST_FFW 3
#define G4_NORM_POST_PLE 4
#define G4_NORM_Q 5
#define G4_NORM_K 6
#define G4_NORM_PLE_PROJECTION 7
#define G4_NORM_FINAL 8
int g4_gemma_set_norm(g4_gemma *m, int layer, int which, const float *v, int n);
/* layer_scalar (skipScale, gemma4-webgpu.js:114). */
int g4_gemma_set_layer_scalar(g4_gemma *m, int layer, float s);
/* The tied BF16 embedding [vocab, hidden] in device memory (embed_tokens and
 * the LM head, gemma4-webgpu.js:170-188). */
int g4_gemma_set_embedding(g4_gemma *m, const void *E_dev);
/* The W4 PLE table of pleRowsToGpu (width layers * ple_dim). */
int g4_gemma_set_ple(g4_gemma *m, const g4_ple *t);
/* Or a dense BF16 embed_tokens_per_layer [vocab, layers * ple_dim] in device
 * memory, whose rows are widened to FP32 per token (inputBuffers without
 * pleRowsToGpu, gemma4-webgpu.js:198-215).  The last of the two calls wins. */
int g4_gemma_set_ple_dense(g4_gemma *m, const void *rows_dev);

/* resetCache (gemma4-webgpu.js:190-194) and the current KV length. */
int g4_gemma_reset(g4_gemma *m);
int g4_gemma_cache_length(const g4_gemma *m, int *len);

/* forward(tokenIds, startPos) (gemma4-webgpu.js:303-402): runs n host token
 * ids at positions start_pos.. and, if last_hidden (device [hidden]) is not
 * NULL, stores the final-norm hidden state of the last token there.
 * start_pos must equal the cache length ("KV append position ... != cache
 * length ...") and start_pos + n <= max_seq ("KV cache capacity ...
 * exceeded"). */
int g4_gemma_forward(g4_gemma *m, const int32_t *ids, int n, int start_pos,
                     float *last_hidden);

/* forward(tokenIds, startPos, {diagnostic: true}) (gemma4-webgpu.js:311-397):
 * g4_gemma_forward, taking the op-by-op path whatever the row count, and in
 * addition, into device buffers (each optional, NULL to skip):
 *   top_hidden   [n, hidden]               the scaled embedding rows
 *   top_ple      [n, layers * ple_dim]     the per-layer inputs (pleMix)
 *   layer_hidden [layers, n, hidden]       each layer's output rows
 *   stages       the G4_STAGE_* buffers of encodeLayer (224-309) for layer
 *                stage_layer, at the float offsets g4_gemma_diag_stages gives
 * The reference probes layer 1's stages (its diagnostic loop, 342-372). */
#define G4_STAGE_PRE_ATTENTION 0
#define G4_STAGE_Q_RAW 1
#define G4_STAGE_Q_NORM_ROPE 2
#define G4_STAGE_K_RAW 3
#define G4_STAGE_V_RAW 4
#define G4_STAGE_K_NORM_ROPE 5
#define G4_STAGE_V_NORM 6
#define G4_STAGE_ATTENTION_CONTEXT 7
#define G4_STAGE_ATTENTION_OUTPUT 8
#define G4_STAGE_POST_ATTENTION_NORM 9
#define G4_STAGE_ATTENTION_RESIDUAL 10
#define G4_STAGE_PRE_FFW 11
#define G4_STAGE_MLP_GATE 12
#define G4_STAGE_MLP_UP 13
#define G4_STAGE_MLP_ACTIVATED 14
#define G4_STAGE_FFW_OUTPUT 15
#define G4_STAGE_POST_FFW_NORM 16
#define G4_STAGE_FFW_RESIDUAL 17
#define G4_STAGE_PLE_GATE 18
#define G4_STAGE_PLE_MODULATED 19
#define G4_STAGE_PLE_PROJECTED 20
#define G4_STAGE_PLE_NORMALIZED 21
#define G4_STAGE_OUTPUT 22
#define G4_STAGES 23
int g4_gemma_forward_diag(g4_gemma *m, const int32_t *ids, int n, int start_pos,
                          float *last_hidden, float *top_hidden, float *top_ple,
                          float *layer_hidden, int stage_layer, float *stages);

/* Float offsets of layer `layer`'s G4_STAGE_* buffers at n rows in a stage
 * buffer: offsets[s] .. offsets[s + 1] (G4_STAGES + 1 entries; the reference's
 * probe counts, gemma4-webgpu.js:224-309; the k/v stages of a layer without
 * its own KV are empty). */
int g4_gemma_diag_stages(const g4_gemma *m, int layer, int n, size_t *offsets);

/* logits(lastHidden) (gemma4-webgpu.js:404-431) into device [vocab]. */
int g4_gemma_logits(g4_gemma *m, const float *last_hidden, float *logits);

/* greedy(tokenIds, startPos) (gemma4-webgpu.js:441-481): forward, logits and
 * the first index of the largest finite logit (topK's top-1).  logits
 * (device [vocab]) may be NULL. */
int g4_gemma_greedy(g4_gemma *m, const int32_t *ids, int n, int start_pos,
                    int32_t *next_token, float *logits);

/* The final-norm hidden state of the last token the model ran (by
 * g4_gemma_forward, g4_gemma_greedy or a g4_gemma_decode step) into device
 * [hidden]: forward's lastHidden (gemma4-webgpu.js:394-400) for the decode
 * loop, whose steps return only the token. */
int g4_gemma_last_hidden(g4_gemma *m, float *last_hidden);

/* `steps` further greedy tokens, each fed back as the next input (the
 * generation loop of custom-webgpu/main.js), from the state a g4_gemma_greedy
 * call left.  tokens (host [steps]) may be NULL.  The first call records the
 * decode step; later calls replay it. */
int g4_gemma_decode(g4_gemma *m, int steps, int32_t *tokens);

#ifdef __cplusplus
}
#endif

#endif /* G4HIP_H */
