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
 * g4_encoder_finish, kernel-launching calls (g4_w4_linear, g4_w4_dequant,
 * g4_ple_gather_dev, g4_bf16_head, g4_copy) are recorded instead of run;
 * g4_submit replays the recording on the queue (a HIP graph).  Calls that
 * must wait for the device or move host memory (g4_alloc, g4_free,
 * g4_upload, g4_download, g4_sync, g4_ple_gather with host ids, loads) fail
 * with G4_E_STATE while an encoder is open.  Unlike a WebGPU command buffer,
 * a finished recording may be submitted any number of times. */
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

/* Number of shards and the byte size of shard `shard`. */
int g4_ple_shard_bytes(const g4_ple *t, int shard, int *num_shards,
                       size_t *bytes);

int g4_ple_free(g4_ple *t);

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

#ifdef __cplusplus
}
#endif

#endif /* G4HIP_H */
