// Internal helpers shared by the gfx950 translation units of libg4hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "g4hip.h"

#define G4_API extern "C" __attribute__((visibility("default")))

namespace g4 {

// Records `code` and a printf-style message for g4_last_error(); returns code.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the last error and returns G4_OK.
int ok();

// The library stream; nullptr until g4_init succeeded.
hipStream_t stream();
bool initialised();
// True between g4_encoder_begin and g4_encoder_finish (stream capture).
bool encoding();

// Checks that [p, p + bytes) lies inside one live device allocation.  `what`
// names the operand in the error message.  Returns G4_OK or G4_E_RANGE.
int check_device_range(const void *p, size_t bytes, const char *what);

// Stream-ordered device allocation used by the object handles (zero-filled).
int device_alloc(size_t bytes, void **p);
int device_free(void *p);

// Device attribute cache.
int cu_count();
// The device g4_init selected.
int current_device();

// Scratch memory that grows on demand.  Growing allocates, which a command
// encoder cannot record: inside an encoder a request beyond the current size
// fails with G4_E_STATE and `who` in the message (make one call of that size
// outside the encoder first).  Contents are not preserved across growth.
// A block outgrown while a finished recording exists stays allocated until
// the last recording is freed, so replaying an older recording never writes
// through a stale scratch address into memory handed out since.
struct Workspace {
  void *mem = nullptr;
  size_t bytes = 0;
  bool captured = false;  // handed out while an encoder was recording
  int get(size_t need, void **p, const char *who);
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Streaming (non-temporal) 16-byte loads and stores for data touched once.
__device__ __forceinline__ uint4 ld_nt(const uint4 *p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
// A weight scale: streamed like the packed words it belongs to (3.01 -> 2.92 us
// for the M1 K1536 N6144 GEMV, cold weights, against plain loads).
__device__ __forceinline__ uint32_t ld_nt_u16(const uint16_t *p) {
  return __builtin_nontemporal_load(p);
}
__device__ __forceinline__ void st_nt(uint4 *p, uint4 v) {
  const u32x4 u = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(u, reinterpret_cast<u32x4 *>(p));
}
__device__ __forceinline__ void st_nt(float4 *p, float4 v) {
  const f32x4 u = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(u, reinterpret_cast<f32x4 *>(p));
}

}  // namespace g4

#define G4_CHECK_INIT()                                                     \
  do {                                                                      \
    if (!::g4::initialised())                                               \
      return ::g4::fail(G4_E_STATE, "%s: g4_init() has not been called",    \
                        __func__);                                          \
  } while (0)

// Entry points that synchronise or move host memory cannot be recorded.
#define G4_CHECK_NOT_ENCODING()                                              \
  do {                                                                      \
    if (::g4::encoding())                                                   \
      return ::g4::fail(G4_E_STATE, "%s: not allowed while a command "      \
                        "encoder is open", __func__);                       \
  } while (0)

#define G4_HIP_TRY(call)                                                    \
  do {                                                                      \
    hipError_t e_ = (call);                                                 \
    if (e_ != hipSuccess)                                                   \
      return ::g4::fail(G4_E_HIP, "%s failed: %s (%s:%d)", #call,           \
                        hipGetErrorString(e_), __FILE__, __LINE__);         \
  } while (0)

// After a kernel launch: report a launch-configuration error, if any.
#define G4_LAUNCH_CHECK(name)                                               \
  do {                                                                      \
    hipError_t e_ = hipGetLastError();                                      \
    if (e_ != hipSuccess)                                                   \
      return ::g4::fail(G4_E_HIP, "launch of %s failed: %s", name,          \
                        hipGetErrorString(e_));                             \
  } while (0)

// ---- device-side helpers ---------------------------------------------------

namespace g4 {

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even of the upper 16 bits, the exact arithmetic of
// roundFloat32ToBF16 (official-w4a16.js:34-48): bits + 0x7fff + lsb, then
// truncate.  Like the reference it has no special case for NaN payloads.
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float v) {
  uint32_t b = __float_as_uint(v);
  b += 0x7fffu + ((b >> 16) & 1u);
  return b >> 16;
}

}  // namespace g4

// A W4A16 weight resident on the device (GPUW4Linear).
struct g4_w4 {
  int N, K, group, G;
  uint8_t *mem;      // the one device allocation holding both arrays
  uint4 *packed;     // [N][G] 16-byte groups, compressed-tensors order
  uint16_t *scales;  // [N][G] bf16 bits
  int16_t *rshift;   // [N]: 2^rshift[o] * 8 * max_g |scale[o, g]| <= 2^15 (FP16 GEMM)
  // The same words and scales by GEMM stage (two groups) and 16-row tile, for
  // the packed-weight GEMM (even G only, else null).  Stage st of tile t
  // (T = ceil(N / 16) tiles; rows past N repeat row N - 1) is a 576-byte
  // block at tiles + (st * T + t) * 36 (in 16-byte units): 64 word pairs of
  // 8 bytes, pair c + 16 q holding words 2 q and 2 q + 1 of the stage's 8 words
  // of row c (group 2 st + q / 2), then the bf16 scale pairs of the 16 rows as
  // 16 u32 (units 32..35).  A stage of consecutive tiles is contiguous.
  uint4 *tiles;
  int shift;         // min_o rshift[o]: one shift for the whole tensor ...
  bool row_shift;    // ... unless the rows' maxima spread beyond 2^12: then per row
  size_t bytes;
};

namespace g4 {
// Activation rows up to which g4_w4_linear streams the weights (GEMV); more
// rows take the MFMA GEMM.
constexpr int kMaxGemvRows = 4;
// Prefill GEMM (more than kMaxGemvRows rows): y[rows, N] = x[rows, K] . W^T on
// the matrix cores (g4_gemm.hip).
int w4_gemm(const g4_w4 *w, const void *x, bool f32x, int rows, void *y, bool y_bf16);
// Caller-provided scratch for the GEMM (x', row exponents, K-slice planes)
// instead of the library's growing workspace: nothing is allocated, and a
// call whose scratch would exceed `bytes` fails with G4_E_ARG naming `who`.
struct ExtScratch {
  void *mem;
  size_t bytes;
  const char *who;
};
int w4_gemm_ext(const g4_w4 *w, const void *x, bool f32x, int rows, void *y, bool y_bf16,
                const ExtScratch &ext);
// g4_w4_linear's argument checks and dispatch; with ext set, the GEMM path
// uses that scratch (the GEMV paths use none).
int w4_linear_impl(const g4_w4 *w, const void *x, int x_dtype, int rows, void *y, int y_dtype,
                   const ExtScratch *ext, const char *who);
// Per-device address of the static GEMM scratch of g4_w4_linear_noalloc,
// looked up once when the library is initialised on a device.
int static_scratch_init(int device);
// nw (1..3) weights of one input dimension over the same x, y[i] receiving
// weight i's output: one x pre-pass and, when their joint grid fills the CUs,
// one GEMM launch.
int w4_gemm_multi(const g4_w4 *const *w, int nw, const void *x, bool f32x, int rows,
                  void *const *y, bool y_bf16);
// FP32 rows >= 2 (more than the GEMV's row count) whose consumer adds the K
// slices itself: y = x . W^T as out->n partial planes out->parts + s *
// out->stride (s < n, added in order), or in y itself (n = 1).  The planes
// live in the GEMM scratch until the next GEMM call on the stream.
struct GemmParts {
  const float *parts;
  int n;
  size_t stride;
};
int w4_gemm_parts(const g4_w4 *w, const float *x, int rows, float *y, GemmParts *out);
// The same for up to 3 weights of one in_dim in one launch, out[i] for
// weight i: its planes sit side by side with the others' in each slice plane
// (the same n and stride for all), or y[i] itself when K is not split.
int w4_gemm_multi_parts(const g4_w4 *const *w, int nw, const float *x, int rows,
                        float *const *y, GemmParts *out);
// FP32 rows (more than kMaxGemvRows): act = gelu(x . Wg^T) * (x . Wu^T) in one
// launch, each tile holding the same columns of gate and up (the GEMM outputs
// and the product as GELU_MUL computes them).
int w4_gemm_glu(const g4_w4 *gate, const g4_w4 *up, const float *x, int rows, float *act);
// The x pre-pass done by the producer of x instead: w4_gemm_prepare sizes the
// GEMM scratch for the call that follows (the same weights, FP32 rows) and
// returns where x' goes: hi plane xt[c * Mp + m] and lo plane
// xt[(K / 8 + c) * Mp + m] for chunk c (8 values, FP16 pairs (0,4) (1,5)
// (2,6) (3,7) of x * 2^-xe[m]), rows M..Mp-1 zero, xe[m] with max |x * 2^-xe|
// in [2^13, 2^14) (0 for all-zero or non-finite rows).  The GEMM entry points
// then take x = nullptr; no other GEMM call may come in between.
struct GemmXPrep {
  uint4 *xt;
  int *xe;
  int Mp;
};
int w4_gemm_prepare(const g4_w4 *const *w, int nw, int rows, GemmXPrep *out);
// Split-K decode GEMV of one FP32 row into per-slice partial sums
// parts[K / 1536][N] (g4_w4.hip); returns the slice count, 0 if K does not
// split (nothing launched), or minus a status.
int launch_gemv1_split(const g4_w4 *w, const float *x, float *parts);
}  // namespace g4

struct g4_ple;
namespace g4 {
// Rows and columns of a PLE table (g4_ple.hip).
void ple_geometry(const g4_ple *t, int *vocab, int *width);
}  // namespace g4
