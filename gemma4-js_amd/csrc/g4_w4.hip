// W4A16 group-32 linear: the gfx950 replacement of GPUOps.w4 / W4_SHADER
// (custom-webgpu/gpu-runtime.js:1068-1102, 1316-1324) and GPUW4Linear
// (gpu-runtime.js:1380-1394).
//
// Weight format (compressed-tensors, official-w4a16.js:1-19):
//   packed  u32  [N][K/8]   nibble k (bits 4k..4k+3) of word j = input 8j+k,
//                           logical value nibble - 8
//   scales  bf16 [N][K/32]  one scale per group of 32 inputs
// One group is exactly 16 packed bytes, so group g of row o is the 128-bit
// word packed[o*G + g] (G = K/32): a lane that owns a group reads it with one
// coalesced dwordx4 load.
//
// Arithmetic: per group the kernel forms d = sum_i x_i * n_i with the
// unsigned nibble n_i = q_i + 8, then adds s * (d - 8 * sum_i x_i).  The sum
// of x over a group is shared by every output row, so the -8 offset costs
// one FMA per group instead of one per element.  Accumulation is FP32.
#include "g4_internal.h"

struct g4_w4 {
  int N, K, group, G;
  uint4 *packed;     // [N][G] 16-byte groups
  uint16_t *scales;  // [N][G] bf16 bits
  size_t bytes;
};

namespace {

using namespace g4;

// ---------------------------------------------------------------------------
// Streaming GEMV (rows of x <= 4).
//
// A "team" of L lanes owns one output row at a time; lane t of a team handles
// groups t, t+L, t+2L, ... of that row, holding the x values of those groups
// in registers while it walks R rows.  L divides G, so no lane idles.  The
// team's partial sums are combined with cross-lane shuffles at the end.
// ---------------------------------------------------------------------------

template <typename XT>
__device__ __forceinline__ void load_x_group(const XT *__restrict__ x, float (&v)[32]);

template <>
__device__ __forceinline__ void load_x_group<float>(const float *__restrict__ x,
                                                    float (&v)[32]) {
  const float4 *p = reinterpret_cast<const float4 *>(x);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float4 f = p[i];
    v[4 * i + 0] = f.x;
    v[4 * i + 1] = f.y;
    v[4 * i + 2] = f.z;
    v[4 * i + 3] = f.w;
  }
}

template <>
__device__ __forceinline__ void load_x_group<uint16_t>(const uint16_t *__restrict__ x,
                                                       float (&v)[32]) {
  const uint4 *p = reinterpret_cast<const uint4 *>(x);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint4 u = p[i];
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[8 * i + 2 * j + 0] = __uint_as_float(w[j] << 16);
      v[8 * i + 2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  }
}

// sum_i x_i * n_i over one 16-byte group, n_i the unsigned nibble.
__device__ __forceinline__ float group_dot(const uint4 q, const float (&x)[32]) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  float d0 = 0.f, d1 = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t lo = w[j] & 0x0f0f0f0fu;         // nibbles 0,2,4,6
    const uint32_t hi = (w[j] >> 4) & 0x0f0f0f0fu;  // nibbles 1,3,5,7
    const float *xj = x + 8 * j;
    d0 = fmaf(xj[0], (float)(lo & 0xffu), d0);
    d1 = fmaf(xj[1], (float)(hi & 0xffu), d1);
    d0 = fmaf(xj[2], (float)((lo >> 8) & 0xffu), d0);
    d1 = fmaf(xj[3], (float)((hi >> 8) & 0xffu), d1);
    d0 = fmaf(xj[4], (float)((lo >> 16) & 0xffu), d0);
    d1 = fmaf(xj[5], (float)((hi >> 16) & 0xffu), d1);
    d0 = fmaf(xj[6], (float)(lo >> 24), d0);
    d1 = fmaf(xj[7], (float)(hi >> 24), d1);
  }
  return d0 + d1;
}

template <int L, int C, int M, int R, typename XT>
__global__ __launch_bounds__(256) void w4_gemv_kernel(
    const XT *__restrict__ x, const uint4 *__restrict__ wq,
    const uint16_t *__restrict__ ws, void *__restrict__ y, int y_bf16, int K,
    int N) {
  constexpr int TPW = 64 / L;  // teams per wave
  const int G = K >> 5;
  const int GL = G / L;  // groups per lane per row
  const int lane = threadIdx.x & 63;
  const int tl = lane & (L - 1);
  const int team = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * TPW + lane / L;
  const int row0 = team * R;

  float acc[M][R];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.f;

  for (int j0 = 0; j0 < GL; j0 += C) {
    // Weight loads first: they come from HBM and take the longest.
    uint4 q[R][C];
    uint32_t s[R][C];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = row0 + r;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        if (row < N) {
          const size_t idx = (size_t)row * G + tl + L * (j0 + c);
          q[r][c] = ld_nt(&wq[idx]);
          s[r][c] = ws[idx];
        } else {
          q[r][c] = make_uint4(0, 0, 0, 0);
          s[r][c] = 0;
        }
      }
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int g = tl + L * (j0 + c);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float xv[32];
        load_x_group<XT>(x + (size_t)m * K + (size_t)g * 32, xv);
        float sx = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) sx += xv[i];
        const float off = -8.f * sx;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float d = group_dot(q[r][c], xv) + off;
          acc[m][r] = fmaf(bf16_to_f32(s[r][c]), d, acc[m][r]);
        }
      }
    }
  }

#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float v = acc[m][r];
#pragma unroll
      for (int o = L / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
      acc[m][r] = v;
    }

  if (tl == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = row0 + r;
      if (row >= N) continue;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const size_t o = (size_t)m * N + row;
        if (y_bf16)
          static_cast<uint16_t *>(y)[o] = (uint16_t)f32_to_bf16_rne(acc[m][r]);
        else
          static_cast<float *>(y)[o] = acc[m][r];
      }
    }
  }
}

template <int L, int C, int M, int R, typename XT>
int launch_gemv_lcmr(const g4_w4 *w, const XT *x, void *y, int y_bf16) {
  constexpr int TPW = 64 / L;
  const int teams = (w->N + R - 1) / R;
  const int waves = (teams + TPW - 1) / TPW;
  const int blocks = (waves + 3) / 4;
  hipLaunchKernelGGL((w4_gemv_kernel<L, C, M, R, XT>), dim3(blocks), dim3(256), 0,
                     stream(), x, w->packed, w->scales, y, y_bf16, w->K, w->N);
  G4_LAUNCH_CHECK("w4_gemv_kernel");
  return G4_OK;
}

template <int L, int M, typename XT>
int launch_gemv_lm(const g4_w4 *w, const XT *x, void *y, int y_bf16) {
  const int GL = w->G / L;
  if (M > 1) return launch_gemv_lcmr<L, 1, M, 1, XT>(w, x, y, y_bf16);
  // Rows per team: keep >= ~1500 waves in flight on the 256 CUs.
  constexpr int TPW = 64 / L;
  const int waves1 = (w->N + TPW - 1) / TPW;
  const int R = waves1 >= 8192 ? 4 : waves1 >= 4096 ? 2 : 1;
  const int C = (GL % 3 == 0) ? 3 : (GL % 2 == 0) ? 2 : 1;
#define G4_GEMV_CASE(CC, RR) \
  if (C == CC && R == RR) return launch_gemv_lcmr<L, CC, 1, RR, XT>(w, x, y, y_bf16);
  G4_GEMV_CASE(1, 1) G4_GEMV_CASE(1, 2) G4_GEMV_CASE(1, 4)
  G4_GEMV_CASE(2, 1) G4_GEMV_CASE(2, 2) G4_GEMV_CASE(2, 4)
  G4_GEMV_CASE(3, 1) G4_GEMV_CASE(3, 2) G4_GEMV_CASE(3, 4)
#undef G4_GEMV_CASE
  return fail(G4_E_ARG, "no GEMV variant for C=%d R=%d", C, R);
}

template <int M, typename XT>
int launch_gemv_m(const g4_w4 *w, const XT *x, void *y, int y_bf16) {
  const int G = w->G;
  if (G % 64 == 0) return launch_gemv_lm<64, M, XT>(w, x, y, y_bf16);
  if (G % 16 == 0) return launch_gemv_lm<16, M, XT>(w, x, y, y_bf16);
  if (G % 8 == 0) return launch_gemv_lm<8, M, XT>(w, x, y, y_bf16);
  return launch_gemv_lm<1, M, XT>(w, x, y, y_bf16);
}

template <typename XT>
int launch_gemv(const g4_w4 *w, const XT *x, int rows, void *y, int y_bf16) {
  switch (rows) {
    case 1: return launch_gemv_m<1, XT>(w, x, y, y_bf16);
    case 2: return launch_gemv_m<2, XT>(w, x, y, y_bf16);
    case 3: return launch_gemv_m<3, XT>(w, x, y, y_bf16);
    case 4: return launch_gemv_m<4, XT>(w, x, y, y_bf16);
  }
  return fail(G4_E_ARG, "GEMV supports 1..4 rows, got %d", rows);
}

// ---------------------------------------------------------------------------
// Dequant: out[r, k] = (nibble - 8) * scale, exact in FP32
// (dequantizeOfficialW4A16Rows, official-w4a16.js:50-101).  One thread per
// 16-byte group writes its 32 outputs.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void w4_dequant_kernel(
    const uint4 *__restrict__ wq, const uint16_t *__restrict__ ws,
    void *__restrict__ out, int out_bf16, int G, int row_start, int row_count) {
  const size_t item = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= (size_t)row_count * G) return;
  const size_t src = (size_t)row_start * G + item;
  const uint4 q = wq[src];
  const float s = bf16_to_f32(ws[src]);
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  float v[32];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int k = 0; k < 8; ++k)
      v[8 * j + k] = (float)((int)((w[j] >> (4 * k)) & 15u) - 8) * s;
  if (out_bf16) {
    uint4 *o = reinterpret_cast<uint4 *>(static_cast<uint16_t *>(out) + item * 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t p[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        p[j] = f32_to_bf16_rne(v[8 * i + 2 * j]) | (f32_to_bf16_rne(v[8 * i + 2 * j + 1]) << 16);
      o[i] = make_uint4(p[0], p[1], p[2], p[3]);
    }
  } else {
    float4 *o = reinterpret_cast<float4 *>(static_cast<float *>(out) + item * 32);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      o[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
  }
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

G4_API int g4_w4_load(const void *packed, const void *scales, int out_dim,
                      int in_dim, int group, g4_w4 **out) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (!out) return fail(G4_E_ARG, "g4_w4_load: null output handle");
  *out = nullptr;
  if (!packed || !scales) return fail(G4_E_ARG, "g4_w4_load: null weight pointer");
  if (out_dim <= 0 || in_dim <= 0)
    return fail(G4_E_ARG, "g4_w4_load: bad shape [%d, %d]", out_dim, in_dim);
  // official-w4a16.js:56-61
  if (in_dim % 8 != 0) return fail(G4_E_ARG, "inDim must be divisible by 8.");
  if (group <= 0 || in_dim % group != 0)
    return fail(G4_E_ARG, "inDim must be divisible by groupSize.");
  if (group != 32)
    return fail(G4_E_ARG, "g4_w4_load: group size %d unsupported (the checkpoint uses 32)",
                group);
  g4_w4 *w = new g4_w4();
  w->N = out_dim;
  w->K = in_dim;
  w->group = group;
  w->G = in_dim / 32;
  const size_t qbytes = (size_t)out_dim * in_dim / 2;
  const size_t sbytes = (size_t)out_dim * w->G * 2;
  int rc = device_alloc(qbytes, reinterpret_cast<void **>(&w->packed));
  if (!rc) rc = device_alloc(sbytes, reinterpret_cast<void **>(&w->scales));
  if (rc) {
    device_free(w->packed);
    delete w;
    return rc;
  }
  w->bytes = qbytes + sbytes;
  hipError_t e = hipMemcpyAsync(w->packed, packed, qbytes, hipMemcpyHostToDevice, stream());
  if (e == hipSuccess)
    e = hipMemcpyAsync(w->scales, scales, sbytes, hipMemcpyHostToDevice, stream());
  if (e == hipSuccess) e = hipStreamSynchronize(stream());
  if (e != hipSuccess) {
    device_free(w->packed);
    device_free(w->scales);
    delete w;
    return fail(G4_E_HIP, "g4_w4_load: upload failed: %s", hipGetErrorString(e));
  }
  *out = w;
  return ok();
}

G4_API int g4_w4_free(g4_w4 *w) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (!w) return ok();
  int rc = device_free(w->packed);
  int rc2 = device_free(w->scales);
  delete w;
  return rc ? rc : rc2 ? rc2 : ok();
}

G4_API int g4_w4_info(const g4_w4 *w, int *out_dim, int *in_dim, int *group,
                      size_t *device_bytes) {
  if (!w) return fail(G4_E_ARG, "g4_w4_info: null handle");
  if (out_dim) *out_dim = w->N;
  if (in_dim) *in_dim = w->K;
  if (group) *group = w->group;
  if (device_bytes) *device_bytes = w->bytes;
  return ok();
}

G4_API int g4_w4_linear(const g4_w4 *w, const void *x, int x_dtype, int rows,
                        void *y, int y_dtype) {
  G4_CHECK_INIT();
  if (!w) return fail(G4_E_ARG, "g4_w4_linear: null weight handle");
  if (rows <= 0) return fail(G4_E_ARG, "g4_w4_linear: rows must be positive, got %d", rows);
  if (x_dtype != G4_F32 && x_dtype != G4_BF16)
    return fail(G4_E_ARG, "g4_w4_linear: bad x dtype %d", x_dtype);
  if (y_dtype != G4_F32 && y_dtype != G4_BF16)
    return fail(G4_E_ARG, "g4_w4_linear: bad y dtype %d", y_dtype);
  if (!aligned16(x)) return fail(G4_E_ARG, "g4_w4_linear: x must be 16-byte aligned");
  const size_t xe = x_dtype == G4_F32 ? 4 : 2, ye = y_dtype == G4_F32 ? 4 : 2;
  int rc = check_device_range(x, (size_t)rows * w->K * xe, "g4_w4_linear x");
  if (rc) return rc;
  rc = check_device_range(y, (size_t)rows * w->N * ye, "g4_w4_linear y");
  if (rc) return rc;
  // Rows are processed 4 at a time by the streaming kernel.
  for (int r0 = 0; r0 < rows; r0 += 4) {
    const int m = rows - r0 < 4 ? rows - r0 : 4;
    void *yr = static_cast<char *>(y) + (size_t)r0 * w->N * ye;
    if (x_dtype == G4_F32)
      rc = launch_gemv<float>(w, static_cast<const float *>(x) + (size_t)r0 * w->K, m, yr,
                              y_dtype == G4_BF16);
    else
      rc = launch_gemv<uint16_t>(w, static_cast<const uint16_t *>(x) + (size_t)r0 * w->K, m,
                                 yr, y_dtype == G4_BF16);
    if (rc) return rc;
  }
  return ok();
}

G4_API int g4_w4_dequant(const g4_w4 *w, int row_start, int row_count, void *out,
                         int out_dtype) {
  G4_CHECK_INIT();
  if (!w) return fail(G4_E_ARG, "g4_w4_dequant: null weight handle");
  if (row_start < 0 || row_count < 0 || row_start > w->N || row_count > w->N - row_start)
    return fail(G4_E_RANGE, "g4_w4_dequant: rows [%d, %d) outside [0, %d)", row_start,
                row_start + row_count, w->N);
  if (out_dtype != G4_F32 && out_dtype != G4_BF16)
    return fail(G4_E_ARG, "g4_w4_dequant: bad out dtype %d", out_dtype);
  if (row_count == 0) return ok();
  if (!aligned16(out)) return fail(G4_E_ARG, "g4_w4_dequant: out must be 16-byte aligned");
  const size_t oe = out_dtype == G4_F32 ? 4 : 2;
  int rc = check_device_range(out, (size_t)row_count * w->K * oe, "g4_w4_dequant out");
  if (rc) return rc;
  const size_t items = (size_t)row_count * w->G;
  const unsigned blocks = (unsigned)((items + 255) / 256);
  hipLaunchKernelGGL(w4_dequant_kernel, dim3(blocks), dim3(256), 0, stream(), w->packed,
                     w->scales, out, out_dtype == G4_BF16, w->G, row_start, row_count);
  G4_LAUNCH_CHECK("w4_dequant_kernel");
  return ok();
}
