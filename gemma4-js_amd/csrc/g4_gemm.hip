// Prefill W4A16 GEMM on the matrix cores (rows of x >= 2): the multi-row
// case of GPUOps.w4 (gpu-runtime.js:1316-1324, whose W4_SHADER re-reads every
// weight row for every token row) and of OfficialW4A16Linear.apply
// (official-quantized-linear.js:82-128).
//
// Numerics.  MFMA needs both operands in one 16-bit type.  A dequantized
// weight q*s has at most 11 significant bits (|q| <= 8, s a bf16 with 8), so
// it is exact in FP16 but not in BF16 (rounding it to BF16 alone would cost
// ~1.6e-3 relative L2 at the E2B shapes).  The GEMM therefore runs
// v_mfma_f32_16x16x32_f16 with FP32 accumulation on
//   W' = q * s * 2^shift      (exact FP16; shift per tensor, set at load)
//   x' = x * 2^-e[m]          (per row; max |x'| in [2^13, 2^14))
// and writes y = acc * 2^(e[m] - shift), an exact power-of-two rescale.
// BF16 activations are exact in FP16 after the rescale (8 significant bits;
// only values 2^28 below the row maximum lose bits).  FP32 activations are
// split as x' = hi + lo (two FP16 values, ~22 bits) and take two MFMAs.
//
// Structure.  A pre-pass (one block per row) finds e[m] and writes x' as
// FP16 in "pair order": each 8-element chunk (x0..x7) is stored as
// (x0,x4)(x1,x5)(x2,x6)(x3,x7), the order in which ((w >> 4t) & 0x000F000F)
// | 0x64006400 unpacks a packed word into FP16 pairs (1024 + n_t,
// 1024 + n_t+4).  The MFMA only needs A and B to share one k order inside
// each group, so no lane shuffles are needed.
//
// Main kernel: 128x128 output tile per 256-thread block, 4 waves of 64x64
// (4x4 MFMA tiles of 16x16), one 32-deep K step per group, double-buffered
// LDS.  Per step each thread fetches two 16-byte chunks of x' and half a
// packed group (8 bytes) plus its scale for the next step, runs its 16 MFMAs
// on the current buffers, then dequantizes into the other buffer:
//   pair = ((w >> 4t) & 0x000F000F) | 0x64006400     (1024 + n, exact)
//   pair = (pair - 1032) * s'                        (v_pk_add/mul_f16, exact)
// LDS layout [chunk c][row] (16 B each) so the 16 lanes that read one MFMA
// operand touch consecutive addresses.
#include <math.h>

#include "g4_internal.h"

namespace {

using namespace g4;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int BM = 128, BN = 128;
constexpr int kThreads = 256;

// ---- pre-pass: per-row exponent and FP16 x' in pair order ----------------

template <bool F32X>
__device__ __forceinline__ void load8(const void *x, size_t i8, float (&v)[8]) {
  if (F32X) {
    const float4 *p = reinterpret_cast<const float4 *>(x) + 2 * i8;
    const float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 u = reinterpret_cast<const uint4 *>(x)[i8];
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = bf16_to_f32(w[e] & 0xffffu);
      v[2 * e + 1] = bf16_to_f32(w[e] >> 16);
    }
  }
}

__device__ __forceinline__ uint32_t h2bits(_Float16 a, _Float16 b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

template <bool F32X>
__global__ __launch_bounds__(kThreads) void gemm_xprep_kernel(const void *__restrict__ x, int K,
                                                              uint4 *__restrict__ xh,
                                                              uint4 *__restrict__ xl,
                                                              int *__restrict__ xe) {
  __shared__ float red[kThreads / 64];
  const int m = blockIdx.x;
  const int nch = K >> 3;
  const size_t rowc = (size_t)m * nch;
  float mx = 0.f;
  for (int c = threadIdx.x; c < nch; c += kThreads) {
    float v[8];
    load8<F32X>(x, rowc + c, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[e]));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int i = 1; i < kThreads / 64; ++i) mx = fmaxf(mx, red[i]);
  // e: max * 2^-e in [2^13, 2^14); all-zero or non-finite rows keep e = 0
  int e = 0;
  if (mx > 0.f && mx <= 3.4e38f) e = ilogbf(mx) - 13;
  if (threadIdx.x == 0) xe[m] = e;
  for (int c = threadIdx.x; c < nch; c += kThreads) {
    float v[8];
    load8<F32X>(x, rowc + c, v);
    _Float16 h[8], l[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float s = ldexpf(v[i], -e);
      h[i] = (_Float16)s;
      if (F32X) l[i] = (_Float16)(s - (float)h[i]);
    }
    xh[rowc + c] = make_uint4(h2bits(h[0], h[4]), h2bits(h[1], h[5]), h2bits(h[2], h[6]),
                              h2bits(h[3], h[7]));
    if (F32X)
      xl[rowc + c] = make_uint4(h2bits(l[0], l[4]), h2bits(l[1], l[5]), h2bits(l[2], l[6]),
                                h2bits(l[3], l[7]));
  }
}

// ---- main kernel -------------------------------------------------------------

__device__ __forceinline__ f16x8 as_f16x8(uint4 u) { return __builtin_bit_cast(f16x8, u); }

__device__ __forceinline__ uint32_t deq_pair(uint32_t w, int t, f16x2 s2) {
  const uint32_t u = ((w >> (4 * t)) & 0x000F000Fu) | 0x64006400u;
  f16x2 h = __builtin_bit_cast(f16x2, u);
  const f16x2 off = {(_Float16)1032.f, (_Float16)1032.f};
  h = (h - off) * s2;
  return __builtin_bit_cast(uint32_t, h);
}

template <int NX>
__global__ __launch_bounds__(kThreads) void w4_gemm_kernel(
    const uint4 *__restrict__ xh, const uint4 *__restrict__ xl, const int *__restrict__ xe,
    const uint4 *__restrict__ wq, const uint16_t *__restrict__ ws, int shift,
    void *__restrict__ y, int y_bf16, int M, int N, int K) {
  // [buf][chunk][row] 16-byte entries
  __shared__ uint4 As[2][NX][4][BM];
  __shared__ uint4 Bs[2][4][BN];

  const int G = K >> 5;
  const int nch = K >> 3;
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

  // A fetch: entries idx = t, t + 256 of the 512 (row, chunk) pairs
  int a_row[2], a_c[2];
  size_t a_src[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int idx = t + i * kThreads;
    a_row[i] = idx >> 2;
    a_c[i] = idx & 3;
    const int gm = m0 + a_row[i] < M ? m0 + a_row[i] : M - 1;
    a_src[i] = (size_t)gm * nch + a_c[i];
  }
  // B fetch: row n = t >> 1 of the tile, words 2h, 2h+1 of the group
  const int b_row = t >> 1, b_h = t & 1;
  const int gn = n0 + b_row < N ? n0 + b_row : N - 1;
  const uint2 *bsrc = reinterpret_cast<const uint2 *>(wq + (size_t)gn * G) + b_h;
  const uint16_t *ssrc = ws + (size_t)gn * G;

  uint4 ra[NX][2];
  uint2 rb;
  uint32_t rs;
  auto fetch = [&](int g) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      ra[0][i] = xh[a_src[i] + (size_t)g * 4];
      if (NX == 2) ra[NX - 1][i] = xl[a_src[i] + (size_t)g * 4];
    }
    rb = bsrc[(size_t)g * 2];
    rs = ssrc[g];
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int x = 0; x < NX; ++x)
#pragma unroll
      for (int i = 0; i < 2; ++i) As[buf][x][a_c[i]][a_row[i]] = ra[x][i];
    const _Float16 sh = (_Float16)ldexpf(bf16_to_f32(rs), shift);
    const f16x2 s2 = {sh, sh};
    const uint32_t w2[2] = {rb.x, rb.y};
#pragma unroll
    for (int j = 0; j < 2; ++j)
      Bs[buf][2 * b_h + j][b_row] =
          make_uint4(deq_pair(w2[j], 0, s2), deq_pair(w2[j], 1, s2), deq_pair(w2[j], 2, s2),
                     deq_pair(w2[j], 3, s2));
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  fetch(0);
  stage(0);
  __syncthreads();

  const int lr = lane & 15, lc = lane >> 4;  // operand row/col within a 16-tile, k chunk
  for (int g = 0; g < G; ++g) {
    const int buf = g & 1;
    if (g + 1 < G) fetch(g + 1);
    f16x8 bop[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) bop[j] = as_f16x8(Bs[buf][lc][wn * 64 + j * 16 + lr]);
#pragma unroll
    for (int x = 0; x < NX; ++x)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f16x8 aop = as_f16x8(As[buf][x][lc][wm * 64 + i * 16 + lr]);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop[j], acc[i][j], 0, 0, 0);
      }
    if (g + 1 < G) stage(buf ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds rows 4*lc + r (r = 0..3) of column lr of each tile
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + wm * 64 + i * 16 + 4 * lc + r;
      if (m >= M) continue;
      const int sc = xe[m] - shift;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = n0 + wn * 64 + j * 16 + lr;
        if (n >= N) continue;
        const float v = ldexpf(acc[i][j][r], sc);
        const size_t o = (size_t)m * N + n;
        if (y_bf16)
          static_cast<uint16_t *>(y)[o] = (uint16_t)f32_to_bf16_rne(v);
        else
          static_cast<float *>(y)[o] = v;
      }
    }
  }
}

// Workspace for x' (and its low half) and the row exponents; grows on demand
// outside command encoders, reused by every later call.
struct Workspace {
  void *mem = nullptr;
  size_t bytes = 0;
};
Workspace g_ws;

int workspace(size_t need, void **p) {
  if (need <= g_ws.bytes) {
    *p = g_ws.mem;
    return G4_OK;
  }
  if (encoding())
    return fail(G4_E_STATE,
                "g4_w4_linear: the prefill workspace must grow (%zu bytes); make one call with "
                "this row count outside a command encoder first", need);
  if (g_ws.mem) {
    int rc = device_free(g_ws.mem);
    if (rc) return rc;
    g_ws.mem = nullptr;
    g_ws.bytes = 0;
  }
  int rc = device_alloc(need, &g_ws.mem);
  if (rc) return rc;
  g_ws.bytes = need;
  *p = g_ws.mem;
  return G4_OK;
}

}  // namespace

namespace g4 {

int w4_gemm(const g4_w4 *w, const void *x, bool f32x, int rows, void *y, bool y_bf16) {
  const size_t xbytes = (size_t)rows * w->K * 2;  // FP16 x' per half
  const size_t xoff_l = (xbytes + 255) & ~size_t(255);
  const size_t eoff = xoff_l + (f32x ? xoff_l : 0);
  void *ws = nullptr;
  int rc = workspace(eoff + (size_t)rows * 4, &ws);
  if (rc) return rc;
  uint4 *xh = static_cast<uint4 *>(ws);
  uint4 *xl = reinterpret_cast<uint4 *>(static_cast<char *>(ws) + xoff_l);
  int *xe = reinterpret_cast<int *>(static_cast<char *>(ws) + eoff);
  if (f32x)
    hipLaunchKernelGGL(gemm_xprep_kernel<true>, dim3(rows), dim3(kThreads), 0, stream(), x, w->K,
                       xh, xl, xe);
  else
    hipLaunchKernelGGL(gemm_xprep_kernel<false>, dim3(rows), dim3(kThreads), 0, stream(), x,
                       w->K, xh, xl, xe);
  G4_LAUNCH_CHECK("gemm_xprep_kernel");
  const dim3 grid((w->N + BN - 1) / BN, (rows + BM - 1) / BM);
  if (f32x)
    hipLaunchKernelGGL(w4_gemm_kernel<2>, grid, dim3(kThreads), 0, stream(), xh, xl, xe,
                       w->packed, w->scales, w->shift, y, (int)y_bf16, rows, w->N, w->K);
  else
    hipLaunchKernelGGL(w4_gemm_kernel<1>, grid, dim3(kThreads), 0, stream(), xh, xl, xe,
                       w->packed, w->scales, w->shift, y, (int)y_bf16, rows, w->N, w->K);
  G4_LAUNCH_CHECK("w4_gemm_kernel");
  return G4_OK;
}

}  // namespace g4
