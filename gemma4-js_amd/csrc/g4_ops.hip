// The element-wise, normalisation and attention ops of GPUOps
// (custom-webgpu/gpu-runtime.js:1104-1263 shaders, 1325-1369 methods) and the
// embedding lookup of Gemma4WebGPU.inputBuffers/forward
// (gemma4-webgpu.js:198-215, 318-320), as gfx950 kernels.
//
// All activations are FP32 as in the reference.  Reductions (RMS sums,
// softmax) are tree-shaped here instead of the shaders' serial loops, so
// results agree with the reference to FP32 rounding, not bit for bit.
//
// Kernels that a captured decode step replays read the token position from
// device memory when `pos_dev` is non-null (the host value is then ignored),
// so one recorded step serves every position.
#include <math.h>

#include "g4_gemv.h"
#include "g4_internal.h"
#include "g4_ops.h"

namespace g4 {

namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Sum over a block of NW waves (256 threads by default); every thread gets the
// total.  The wave sums are added in wave order, so a block of fewer waves
// gives the bits of a 256-thread block whose other waves hold zeros.
template <int NW = 4>
__device__ __forceinline__ float block_sum(float v, float *red) {
  v = wave_sum(v);
  __syncthreads();  // red may still be read by a previous call
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = red[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) s += red[w];
  return s;
}

// GELU, tanh form with the shader's clamp (gpu-runtime.js:1148-1155).
__device__ __forceinline__ float gelu_tanh(float x) {
  const float c = 0.7978845608028654f;
  const float z = c * (x + 0.044715f * x * x * x);
  const float t = tanhf(fminf(fmaxf(z, -10.f), 10.f));
  return 0.5f * x * (1.f + t);
}

__device__ __forceinline__ float inv_rms(float ss, int width, float eps) {
  return 1.f / sqrtf(ss / (float)width + eps);
}

// ---- RMS_SHADER (gpu-runtime.js:1104-1118) ----------------------------------
// One block per row.  y row index = row (+ *pos_dev when given: the row goes
// to that position of a cache).
__device__ __forceinline__ void rms_row(const float *__restrict__ x, int width,
                                        const float *__restrict__ scale, float eps,
                                        float *__restrict__ y, const int *__restrict__ pos_dev,
                                        int row, float *red) {
  const float *xr = x + (size_t)row * width;
  float ss = 0.f;
  for (int i = threadIdx.x; i < width; i += kBlock) ss += xr[i] * xr[i];
  const float inv = inv_rms(block_sum(ss, red), width, eps);
  const int orow = row + (pos_dev ? *pos_dev : 0);
  float *yr = y + (size_t)orow * width;
  for (int i = threadIdx.x; i < width; i += kBlock)
    yr[i] = xr[i] * inv * (scale ? scale[i] : 1.f);
}

__global__ __launch_bounds__(kBlock) void rms_kernel(const float *__restrict__ x, int width,
                                                     const float *__restrict__ scale, float eps,
                                                     float *__restrict__ y,
                                                     const int *__restrict__ pos_dev) {
  __shared__ float red[4];
  rms_row(x, width, scale, eps, y, pos_dev, blockIdx.x, red);
}

// ---- ADD_SCALE_SHADER / SCALE_SHADER / GELU_MUL_SHADER ----------------------
__global__ __launch_bounds__(kBlock) void add_scale_kernel(const float *__restrict__ a,
                                                           const float *__restrict__ b,
                                                           size_t n, float s,
                                                           float *__restrict__ y) {
  const size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (i < n) y[i] = (a[i] + b[i]) * s;
}

__global__ __launch_bounds__(kBlock) void scale_kernel(const float *__restrict__ a, size_t n,
                                                       float s, float *__restrict__ y) {
  const size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (i < n) y[i] = a[i] * s;
}

__global__ __launch_bounds__(kBlock) void gelu_mul_kernel(const float *__restrict__ gate,
                                                          const float *__restrict__ up, size_t n,
                                                          float *__restrict__ y) {
  const size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (i < n) y[i] = gelu_tanh(gate[i]) * up[i];
}

// ---- GELU_PLE_SHADER (gpu-runtime.js:1159-1173) -----------------------------
// y[r, d] = gelu(gate[r, d]) * ple[r, layer, d], ple laid out [rows][layers][width].
__global__ __launch_bounds__(kBlock) void gelu_ple_kernel(const float *__restrict__ gate,
                                                          const float *__restrict__ ple,
                                                          int rows, int layer, int width,
                                                          int layers, float *__restrict__ y) {
  const int i = blockIdx.x * kBlock + threadIdx.x;
  if (i >= rows * width) return;
  const int r = i / width, d = i - r * width;
  y[i] = gelu_tanh(gate[i]) * ple[((size_t)r * layers + layer) * width + d];
}

// ---- NORM_ROPE_SHADER (gpu-runtime.js:1175-1202) ----------------------------
// One block per (row, head); thread t < hd/2 owns the rotate-half pair
// (t, t + hd/2).  Output row index is row, or *pos_dev + row when pos_dev is
// given and `at_pos` is set (appending k straight into a cache).  x may be
// the sum of `parts` planes pstride floats apart (a GEMM's K slices), added
// in plane order.  NP: the planes loaded, parts itself up to 4, else 8 (the
// planes past `parts` re-read plane 0 and are left out).
constexpr int kNormRopeMaxParts = 8;
constexpr int norm_rope_np(int parts) { return parts <= 4 ? parts : kNormRopeMaxParts; }
template <int NP, int NW = 4>
__device__ __forceinline__ void norm_rope_row(
    const float *__restrict__ x, int parts, size_t pstride, int heads, int hd, int pos0,
    const int *__restrict__ pos_dev, const float *__restrict__ scale, int rope_angles,
    float base, float eps, float *__restrict__ y, int at_pos, int rh, float *red) {
  const int row = rh / heads, h = rh - row * heads;
  const float *xv = x + (size_t)rh * hd;
  const int half = hd >> 1, t = threadIdx.x;
  float a = 0.f, b = 0.f;
  if (t < half) {
    // every plane's load first, then the adds
    float pa[NP], pb[NP];
#pragma unroll
    for (int sp = 0; sp < NP; ++sp) {
      const size_t o = (size_t)(sp < parts ? sp : 0) * pstride;
      pa[sp] = xv[o + t];
      pb[sp] = xv[o + t + half];
    }
    a = pa[0];
    b = pb[0];
#pragma unroll
    for (int sp = 1; sp < NP; ++sp)
      if (sp < parts) {
        a += pa[sp];
        b += pb[sp];
      }
  }
  // the products that are fused are spelled out, so the rounding does not
  // depend on which one the compiler would contract
  const float inv = inv_rms(block_sum<NW>(fmaf(b, b, a * a), red), hd, eps);
  const int pos = (pos_dev ? *pos_dev : pos0) + row;
  if (t < half) {
    const float an = a * inv * scale[t], bn = b * inv * scale[t + half];
    float sn = 0.f, cs = 1.f;
    if (t < rope_angles) {
      const float ex = 2.f * (float)t / (float)hd;
      const float theta = (float)pos / powf(base, ex);
      sn = sinf(theta);
      cs = cosf(theta);
    }
    const size_t orow = at_pos ? (size_t)pos : (size_t)row;
    float *yv = y + (orow * heads + h) * hd;
    yv[t] = fmaf(an, cs, -(bn * sn));
    yv[t + half] = fmaf(bn, cs, an * sn);
  }
}

// NW waves: at least hd / 2 threads.
template <int NP, int NW>
__global__ __launch_bounds__(64 * NW) void norm_rope_kernel(
    const float *__restrict__ x, int parts, size_t pstride, int heads, int hd, int pos0,
    const int *__restrict__ pos_dev, const float *__restrict__ scale, int rope_angles,
    float base, float eps, float *__restrict__ y, int at_pos) {
  __shared__ float red[4];
  norm_rope_row<NP, NW>(x, parts, pstride, heads, hd, pos0, pos_dev, scale, rope_angles, base,
                        eps, y, at_pos, blockIdx.x, red);
}

// v's RMS norm without weights (rms_row) when v is the sum of `parts` planes
// pstride floats apart, added in plane order: thread t holds values t and
// t + 256 (width <= 512).
template <int NP>
__device__ __forceinline__ void rms_parts_row(const float *__restrict__ x, int parts,
                                              size_t pstride, int width, float eps,
                                              float *__restrict__ y,
                                              const int *__restrict__ pos_dev, int row,
                                              float *red) {
  const float *xr = x + (size_t)row * width;
  float v[2] = {0.f, 0.f}, ss = 0.f;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int i = threadIdx.x + u * kBlock;
    if (i < width) {
      float pa[NP];
#pragma unroll
      for (int sp = 0; sp < NP; ++sp) pa[sp] = xr[(size_t)(sp < parts ? sp : 0) * pstride + i];
      v[u] = pa[0];
#pragma unroll
      for (int sp = 1; sp < NP; ++sp)
        if (sp < parts) v[u] += pa[sp];
      ss = fmaf(v[u], v[u], ss);
    }
  }
  const float inv = inv_rms(block_sum(ss, red), width, eps);
  float *yr = y + (size_t)(row + (pos_dev ? *pos_dev : 0)) * width;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int i = threadIdx.x + u * kBlock;
    if (i < width) yr[i] = v[u] * inv;
  }
}

// The q, k and v steps of a prefill layer that owns its KV cache, in one
// launch: blocks [0, rows * heads) the q norm + RoPE (norm_rope_row), the next
// rows blocks the k norm + RoPE into the cache at *pos_dev + row, the last
// rows blocks v's RMS norm without weights into the cache (rms_row).  q, k
// and v are each the sum of `qparts` planes qpstride floats apart (the K
// slices of their one GEMM launch).
template <int NP>
__global__ __launch_bounds__(kBlock) void norm_rope_qkv_kernel(
    const float *__restrict__ q, int qparts, size_t qpstride, const float *__restrict__ k,
    const float *__restrict__ v, int rows, int heads, int hd, const int *__restrict__ pos_dev,
    const float *__restrict__ qscale, const float *__restrict__ kscale, int rope_angles,
    float base, float eps, float *__restrict__ qy, float *__restrict__ kc,
    float *__restrict__ vc) {
  __shared__ float red[4];
  const int nq = rows * heads, b = blockIdx.x;
  if (b < nq)
    norm_rope_row<NP>(q, qparts, qpstride, heads, hd, 0, pos_dev, qscale, rope_angles, base,
                      eps, qy, 0, b, red);
  else if (b < nq + rows)
    norm_rope_row<NP>(k, qparts, qpstride, 1, hd, 0, pos_dev, kscale, rope_angles, base, eps, kc,
                      1, b - nq, red);
  else if (NP > 1)
    rms_parts_row<NP>(v, qparts, qpstride, hd, eps, vc, pos_dev, b - nq - rows, red);
  else
    rms_row(v, hd, nullptr, eps, vc, pos_dev, b - nq - rows, red);
}

// ---- attention: QK_SHADER + SOFTMAX_SHADER + ATTN_OUT_SHADER ----------------
// (gpu-runtime.js:1204-1248), split over keys (flash decoding).
//
// Block = one wave; it owns `kpw` consecutive keys of one query row for all
// heads (the k/v rows are shared by every head).  Lane l holds dims
// [DPL*l, DPL*l + DPL) of q and of the output for each head.  Per key: the
// H partial dots are reduced across the wave, an online softmax updates the
// running max / sum per head, and p * v[key] accumulates.  The block writes
// (max, sum, unnormalised output) per head; attn_combine_kernel merges the
// splits.  Masked keys (key > qpos, or outside the sliding window) are
// skipped: the shader gives them logit -1e30, i.e. weight exactly 0.
constexpr int kMaxHeads = 8;

struct AttnArgs {
  const float *q;       // [qrows, H, hd]
  const float *k, *v;   // [keylen, hd] cache rows
  float *part;          // [qrows, nsplit, H, hd + 2]
  int H, hd, keylen, qpos0, sliding, window, kpw, nsplit;
  const int *pos_dev;   // if set: qpos0 = *pos_dev and keylen = *pos_dev + qrows
  int qrows;
  float *out;           // [qrows, H, hd] (attn_rows_mfma_kernel)
  // attn_rows_mfma_kernel, when xt is set: the output leaves as the prefill
  // GEMM's x' of [qrows, H * hd] rows (xt, xe, Mp of w4_gemm_prepare)
  // instead of through `out`
  uint4 *xt;
  int *xe;
  int Mp;
};

template <int DPL>
__global__ __launch_bounds__(64) void attn_split_kernel(AttnArgs a) {
  const int lane = threadIdx.x;
  const int split = blockIdx.x, qr = blockIdx.y;
  const int H = a.H, hd = a.hd;
  const int qpos0 = a.pos_dev ? *a.pos_dev : a.qpos0;
  const int keylen = a.pos_dev ? *a.pos_dev + a.qrows : a.keylen;
  const int qpos = qpos0 + qr;
  if (split * a.kpw >= keylen) return;  // past the keys of this call: not combined
  int k0 = split * a.kpw, k1 = k0 + a.kpw;
  if (k1 > keylen) k1 = keylen;
  if (k1 > qpos + 1) k1 = qpos + 1;                       // key <= qpos
  if (a.sliding && k0 < qpos - a.window + 1) k0 = qpos - a.window + 1;  // key + window > qpos
  if (k0 < 0) k0 = 0;

  float q[kMaxHeads][DPL], o[kMaxHeads][DPL], m[kMaxHeads], l[kMaxHeads];
  const int d0 = lane * DPL;
  const bool live = d0 < hd;
#pragma unroll
  for (int h = 0; h < kMaxHeads; ++h) {
    m[h] = -1e30f;
    l[h] = 0.f;
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      q[h][j] = (h < H && live) ? a.q[((size_t)qr * H + h) * hd + d0 + j] : 0.f;
      o[h][j] = 0.f;
    }
  }
  for (int key = k0; key < k1; ++key) {
    float kv[DPL], vv[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      kv[j] = live ? a.k[(size_t)key * hd + d0 + j] : 0.f;
      vv[j] = live ? a.v[(size_t)key * hd + d0 + j] : 0.f;
    }
#pragma unroll
    for (int h = 0; h < kMaxHeads; ++h) {
      if (h >= H) break;
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < DPL; ++j) s = fmaf(q[h][j], kv[j], s);
      s = wave_sum(s);
      const float mn = fmaxf(m[h], s);
      const float c = expf(m[h] - mn), p = expf(s - mn);
      l[h] = l[h] * c + p;
#pragma unroll
      for (int j = 0; j < DPL; ++j) o[h][j] = fmaf(p, vv[j], o[h][j] * c);
      m[h] = mn;
    }
  }
  const size_t stride = (size_t)hd + 2;
  float *pp = a.part + ((size_t)qr * a.nsplit + split) * H * stride;
#pragma unroll
  for (int h = 0; h < kMaxHeads; ++h) {
    if (h >= H) break;
    float *ph = pp + h * stride;
    if (live)
#pragma unroll
      for (int j = 0; j < DPL; ++j) ph[2 + d0 + j] = o[h][j];
    if (lane == 0) {
      ph[0] = m[h];
      ph[1] = l[h];
    }
  }
}

// ---- multi-row attention on the FP32 matrix cores ------------------------------
// q [qrows, H, hd] is read as nrows = qrows * H rows; row R sits at position
// qpos0 + R / H and sees the keys (pos - window, pos] (sliding) or [0, pos],
// all from the one k/v head.  A block (4 waves) owns 16 consecutive rows,
// staged in LDS; its waves take turns over the 16-key tiles of the rows' key
// range.  Per tile, with v_mfma_f32_16x16x4f32 (FP32 products, FP32 sums):
//   S = Q . K^T (16 x 16)        hd/4 MFMAs; lane (c, g) feeds Q row c / key
//                                c, dims 16j + 4g + i at step (j, i)
//   online softmax per row       rows 4g + v live in the 16 lanes of group g
//                                (one DPP row): max and sum by DPP
//   O += P . V (16 x hd)         P goes through LDS into the A layout; output
//                                tile n, column c holds dim 64(n/4) + 4c + n%4,
//                                so V and O move as 16-byte vectors
// Masked keys (the shader's -1e30 logits) get weight exactly 0, and key rows
// are clamped into the visible range, so rows past keylen are never read.
// The 4 waves' (max, sum, O) merge in LDS in wave order; the block writes the
// normalised rows.  The arithmetic is the reference's softmax(q.k) . v; only
// the summation order differs (MFMA dot chunks, online rescaling).  Head dims
// up to 256; head dim 512 runs attn_rows_dsplit_kernel.
template <typename F>
__device__ __forceinline__ float row16_reduce(float v, F op) {
  v = op(v, dpp_f32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = op(v, dpp_f32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = op(v, dpp_f32<0x141>(v));  // row_half_mirror
  v = op(v, dpp_f32<0x140>(v));  // row_mirror
  return v;
}

constexpr int kFaRows = 16, kFaWaves = 4, kFaPStride = 20;

// The rows of a 16-row attention block: qs holds each row's unnormalised O
// (padded stride HD + 4) and wm / wl the per-wave (max, sum) to merge with
// weights e^(m_w - M).  Writes the normalised rows to a.out, or with a.xt set
// the x' of the GEMM that takes them.
template <int HD, int NTH = 256>
__device__ __forceinline__ void attn_rows_store(const AttnArgs &a, const float *qs,
                                                const float (*wm)[kFaRows],
                                                const float (*wl)[kFaRows], int R0, int nrows,
                                                int t) {
  constexpr int QS = HD + 4;
  const int H = a.H;
  if (!a.xt) {
    for (int i = t; i < kFaRows * HD / 4; i += NTH) {
      const int r = i / (HD / 4), d4 = i - r * (HD / 4);
      if (R0 + r >= nrows) continue;
      const float M = fmaxf(fmaxf(wm[0][r], wm[1][r]), fmaxf(wm[2][r], wm[3][r]));
      const float L = wl[0][r] * expf(wm[0][r] - M) + wl[1][r] * expf(wm[1][r] - M) +
                      wl[2][r] * expf(wm[2][r] - M) + wl[3][r] * expf(wm[3][r] - M);
      const float4 x = *reinterpret_cast<const float4 *>(&qs[r * QS + 4 * d4]);
      reinterpret_cast<float4 *>(a.out + (size_t)(R0 + r) * HD)[d4] =
          make_float4(x.x / L, x.y / L, x.z / L, x.w / L);
    }
    return;
  }
  // x' of the GEMM that takes these rows ([qrows, H * HD]; H divides 16, so
  // the block holds whole query rows): the exponent of each query row from
  // the maximum over its H heads, then the chunks of 8 values as FP16 hi/lo
  // pairs (0,4) (1,5) (2,6) (3,7) of x * 2^-e, as gemm_xprep_fused_kernel
  // writes them.  The values are the ones the rows above would hold.
  __shared__ float rl[kFaRows];
  __shared__ int qmax[kFaRows];
  if (t < kFaRows) {
    const float M = fmaxf(fmaxf(wm[0][t], wm[1][t]), fmaxf(wm[2][t], wm[3][t]));
    rl[t] = wl[0][t] * expf(wm[0][t] - M) + wl[1][t] * expf(wm[1][t] - M) +
            wl[2][t] * expf(wm[2][t] - M) + wl[3][t] * expf(wm[3][t] - M);
    qmax[t] = 0;
  }
  __syncthreads();
  constexpr int C8 = HD / 8;  // chunks per head
  auto row_values = [&](int r, int c8, float (&v)[8]) {
    const float L = rl[r];
    const float4 x0 = *reinterpret_cast<const float4 *>(&qs[r * QS + 8 * c8]);
    const float4 x1 = *reinterpret_cast<const float4 *>(&qs[r * QS + 8 * c8 + 4]);
    v[0] = x0.x / L, v[1] = x0.y / L, v[2] = x0.z / L, v[3] = x0.w / L;
    v[4] = x1.x / L, v[5] = x1.y / L, v[6] = x1.z / L, v[7] = x1.w / L;
  };
  for (int i = t; i < kFaRows * C8; i += NTH) {
    const int r = i / C8, c8 = i - r * C8;
    if (R0 + r >= nrows) continue;
    float v[8], mx = 0.f;
    row_values(r, c8, v);
#pragma unroll
    for (int q = 0; q < 8; ++q) mx = fmaxf(mx, fabsf(v[q]));
    atomicMax(&qmax[r / H], __float_as_int(mx));  // non-negative: ordered as ints
  }
  __syncthreads();
  const int nch = H * C8;
  const size_t lo_plane = (size_t)nch * a.Mp;
  for (int i = t; i < kFaRows * C8; i += NTH) {
    const int r = i / C8, c8 = i - r * C8;
    const int qr = (R0 + r) / H, ch = (r % H) * C8 + c8;  // R0 is a multiple of H
    uint4 hi = make_uint4(0u, 0u, 0u, 0u), lo = hi;
    if (R0 + r < nrows) {
      const float mx = __int_as_float(qmax[r / H]);
      const int e = mx > 0.f && mx <= 3.4e38f ? ilogbf(mx) - 13 : 0;
      if (ch == 0) a.xe[qr] = e;
      float v[8];
      row_values(r, c8, v);
      _Float16 hh[8], ll[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const float sv = ldexpf(v[q], -e);
        hh[q] = (_Float16)sv;
        ll[q] = (_Float16)(sv - (float)hh[q]);
      }
      hi = make_uint4(half2_bits(hh[0], hh[4]), half2_bits(hh[1], hh[5]), half2_bits(hh[2], hh[6]),
                      half2_bits(hh[3], hh[7]));
      lo = make_uint4(half2_bits(ll[0], ll[4]), half2_bits(ll[1], ll[5]), half2_bits(ll[2], ll[6]),
                      half2_bits(ll[3], ll[7]));
    }
    if (qr < a.Mp) {
      a.xt[(size_t)ch * a.Mp + qr] = hi;
      a.xt[lo_plane + (size_t)ch * a.Mp + qr] = lo;
    }
  }
}

template <int HD>
__global__ __launch_bounds__(256) void attn_rows_mfma_kernel(AttnArgs a) {
  constexpr int QS = HD + 4;  // padded LDS row (floats): conflict-free 16-byte reads
  constexpr int NT = HD / 16;
  __shared__ float qs[kFaRows * QS];                 // the Q tile, later the merged O
  __shared__ float ps[kFaWaves][kFaRows * kFaPStride];  // per wave: P[row][g * 4 + s]
  __shared__ float wm[kFaWaves][kFaRows], wl[kFaWaves][kFaRows];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int H = a.H;
  const int qpos0 = a.pos_dev ? *a.pos_dev : a.qpos0;
  const int keylen = a.pos_dev ? *a.pos_dev + a.qrows : a.keylen;
  const int nrows = a.qrows * H;
  const int R0 = blockIdx.x * kFaRows;
  if (R0 >= nrows) {  // x' only: the GEMM's padding rows qrows .. Mp - 1 as zero chunks
    if (!a.xt) return;
    const int nch = H * (HD / 8), nq = kFaRows / H;
    const size_t lo_plane = (size_t)nch * a.Mp;
    for (int i = t; i < nq * nch; i += 256) {
      const int qr = R0 / H + i / nch, ch = i % nch;
      if (qr >= a.Mp) continue;
      a.xt[(size_t)ch * a.Mp + qr] = make_uint4(0u, 0u, 0u, 0u);
      a.xt[lo_plane + (size_t)ch * a.Mp + qr] = make_uint4(0u, 0u, 0u, 0u);
    }
    return;
  }
  const int Rl = (R0 + kFaRows < nrows ? R0 + kFaRows : nrows) - 1;  // last live row

  for (int i = t; i < kFaRows * HD / 4; i += 256) {
    const int r = i / (HD / 4), d4 = i - r * (HD / 4);
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (R0 + r < nrows) v = reinterpret_cast<const float4 *>(a.q + (size_t)(R0 + r) * HD)[d4];
    *reinterpret_cast<float4 *>(&qs[r * QS + 4 * d4]) = v;
  }
  // keys of the block's rows: [kmin, kmax]
  const int pos_first = qpos0 + R0 / H, pos_last = qpos0 + Rl / H;
  int kmin = a.sliding ? pos_first - a.window + 1 : 0;
  kmin = kmin > 0 ? kmin : 0;
  const int kmax = pos_last < keylen - 1 ? pos_last : keylen - 1;
  int rpos[4];
  bool rlive[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int R = R0 + 4 * g + v;
    rlive[v] = R < nrows;
    rpos[v] = qpos0 + (rlive[v] ? R : Rl) / H;
  }
  float m[4] = {-1e30f, -1e30f, -1e30f, -1e30f}, l[4] = {0.f, 0.f, 0.f, 0.f};
  f32x4 o[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) o[n] = (f32x4){0.f, 0.f, 0.f, 0.f};
  __syncthreads();

  float *pw = ps[w];
  static_assert(HD <= 256, "head dim 512 runs attn_rows_dsplit_kernel");
  {
    // The next key tile's K is loaded once this tile's scores are formed, its V
    // once this tile's P.V is done: each load has a phase of work to land in
    // (tile indices past the last re-read the last tile).
    constexpr int NV = HD / 64;
    const int kt_last = kmax / 16;
    float4 kr[NT], vr[4][NV];
    auto load_k = [&](int kt) {
      kt = kt < kt_last ? kt : kt_last;
      const int kc = kt * 16 + c < kmax ? kt * 16 + c : kmax;
      const float *kp = a.k + (size_t)kc * HD + 4 * g;
#pragma unroll
      for (int j = 0; j < NT; ++j) kr[j] = *reinterpret_cast<const float4 *>(kp + 16 * j);
    };
    auto load_v = [&](int kt) {
      kt = kt < kt_last ? kt : kt_last;
#pragma unroll
      for (int sp = 0; sp < 4; ++sp) {
        const int kr2 = kt * 16 + 4 * sp + g < kmax ? kt * 16 + 4 * sp + g : kmax;
        const float *vp = a.v + (size_t)kr2 * HD + 4 * c;
#pragma unroll
        for (int q = 0; q < NV; ++q) vr[sp][q] = *reinterpret_cast<const float4 *>(vp + 64 * q);
      }
    };
    int kt = kmin / 16 + w;
    load_k(kt);
    load_v(kt);
    for (; kt <= kt_last; kt += kFaWaves) {
      const int key0 = kt * 16;
      const float *qp = &qs[c * QS + 4 * g];
      f32x4 sa[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) sa[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const float4 kv = kr[j];
        const float4 qv = *reinterpret_cast<const float4 *>(qp + 16 * j);
        sa[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(qv.x, kv.x, sa[0], 0, 0, 0);
        sa[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(qv.y, kv.y, sa[1], 0, 0, 0);
        sa[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(qv.z, kv.z, sa[2], 0, 0, 0);
        sa[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(qv.w, kv.w, sa[3], 0, 0, 0);
      }
      load_k(kt + kFaWaves);
      const f32x4 s = (sa[0] + sa[1]) + (sa[2] + sa[3]);
      const int key = key0 + c;
      float corr[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const bool ok = rlive[v] && key <= rpos[v] && key < keylen &&
                        (!a.sliding || key > rpos[v] - a.window);
        const float tm = row16_reduce(ok ? s[v] : -1e30f, [](float x, float y) { return fmaxf(x, y); });
        const float mn = fmaxf(m[v], tm);
        corr[v] = expf(m[v] - mn);
        const float p = ok ? expf(s[v] - mn) : 0.f;
        l[v] = l[v] * corr[v] + row16_reduce(p, [](float x, float y) { return x + y; });
        m[v] = mn;
        pw[(4 * g + v) * kFaPStride + (c & 3) * 4 + (c >> 2)] = p;
      }
#pragma unroll
      for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int v = 0; v < 4; ++v) o[n][v] *= corr[v];
      const float4 pa = *reinterpret_cast<const float4 *>(&pw[c * kFaPStride + 4 * g]);
      const float pv[4] = {pa.x, pa.y, pa.z, pa.w};
#pragma unroll
      for (int sp = 0; sp < 4; ++sp)
#pragma unroll
        for (int q = 0; q < NV; ++q) {
          const float4 vv = vr[sp][q];
          o[4 * q + 0] = __builtin_amdgcn_mfma_f32_16x16x4f32(pv[sp], vv.x, o[4 * q + 0], 0, 0, 0);
          o[4 * q + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(pv[sp], vv.y, o[4 * q + 1], 0, 0, 0);
          o[4 * q + 2] = __builtin_amdgcn_mfma_f32_16x16x4f32(pv[sp], vv.z, o[4 * q + 2], 0, 0, 0);
          o[4 * q + 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(pv[sp], vv.w, o[4 * q + 3], 0, 0, 0);
        }
      load_v(kt + kFaWaves);
    }
  }

  // merge the waves: weights e^(m_w - M), O summed into qs in wave order
  if (c == 0)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      wm[w][4 * g + v] = m[v];
      wl[w][4 * g + v] = l[v];
    }
  __syncthreads();
  float f[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int r = 4 * g + v;
    const float M = fmaxf(fmaxf(wm[0][r], wm[1][r]), fmaxf(wm[2][r], wm[3][r]));
    f[v] = expf(m[v] - M);
  }
  for (int ww = 0; ww < kFaWaves; ++ww) {
    if (w == ww) {
#pragma unroll
      for (int q = 0; q < HD / 64; ++q)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          float4 *dst = reinterpret_cast<float4 *>(&qs[(4 * g + v) * QS + 64 * q + 4 * c]);
          const float4 add = make_float4(o[4 * q][v] * f[v], o[4 * q + 1][v] * f[v],
                                         o[4 * q + 2][v] * f[v], o[4 * q + 3][v] * f[v]);
          if (ww == 0) {
            *dst = add;
          } else {
            const float4 cur = *dst;
            *dst = make_float4(cur.x + add.x, cur.y + add.y, cur.z + add.z, cur.w + add.w);
          }
        }
    }
    __syncthreads();
  }
  attn_rows_store<HD>(a, qs, wm, wl, R0, nrows, t);
}

// Single-query attention (a decode step): the visible keys [lo, keylen) are
// split evenly over the grid (at most kDecMaxKeys per block).  Block = 4
// waves.  Phase 1: each wave takes every 4th key of the block; lane l holds
// dims [DPL*l, DPL*l + DPL) of q for all heads, and the 8 per-head partial
// dots of a key are reduced across the wave by a reduce-scatter (10 shuffles
// instead of 8 full reductions), leaving head (l >> 3) & 7 in lane group
// l >> 3.  Phase 2: per head (32 threads) the block's max, exp and sum.
// Phase 3: per head, 32 threads each accumulate hd/32 output dims over the
// block's keys.  Every block writes (max, sum, output) per head, an empty
// block (max -1e30, sum 0): attn_combine_kernel merges them.
// The same rows with the head dimension split over the block's waves, for
// large head dims: every wave walks every key tile of the block's rows and
// owns dims [w DW, (w + 1) DW) of q, k, v and O (DW = HD / 4):
//   S_w = Q[:, dims_w] . K[:, dims_w]^T   DW/4 MFMAs; the four partial S
//        meet in LDS and every wave adds them in wave order, so all hold
//        the same S and the same softmax (max, sum, P)
//   O[:, dims_w] += P . V[:, dims_w]      DW/4 MFMAs
// A wave's registers hold a quarter of the row's O and its k/v slices, so
// the next tile's K and V are loaded during the current one.  No merge of
// the waves is needed: O goes to LDS by dims and leaves through
// attn_rows_store.
template <int HD, int DQ, int KG>
__global__ __launch_bounds__(64 * DQ * KG) void attn_rows_dsplit_kernel(AttnArgs a) {
  static_assert(KG >= 1 && KG <= kFaWaves && DQ >= 1 && HD % (64 * DQ) == 0,
                "up to 4 key groups of DQ waves with whole 64-dim column groups");
  constexpr int NTH = 64 * DQ * KG;
  constexpr int QS = HD + 4;
  constexpr int DW = HD / DQ;  // dims per wave
  constexpr int NJ = DW / 16;  // S steps of 16 dims (4 MFMAs each)
  constexpr int NQ = DW / 64;  // 64-dim column groups of O per wave
  __shared__ float qs[kFaRows * QS];  // the Q tile, later O
  __shared__ f32x4 sx[2][KG][DQ][64];  // partial S per wave (two buffers)
  __shared__ float ps[KG * DQ][kFaRows * kFaPStride];
  __shared__ float wm[kFaWaves][kFaRows], wl[kFaWaves][kFaRows];
  const int t = threadIdx.x, lane = t & 63, w = (t >> 6) % DQ, kg = (t >> 6) / DQ;
  const int c = lane & 15, g = lane >> 4;
  const int H = a.H;
  const int qpos0 = a.pos_dev ? *a.pos_dev : a.qpos0;
  const int keylen = a.pos_dev ? *a.pos_dev + a.qrows : a.keylen;
  const int nrows = a.qrows * H;
  const int R0 = blockIdx.x * kFaRows;
  if (R0 >= nrows) {  // x' only: the GEMM's padding rows qrows .. Mp - 1 as zero chunks
    if (!a.xt) return;
    const int nch = H * (HD / 8), nq = kFaRows / H;
    const size_t lo_plane = (size_t)nch * a.Mp;
    for (int i = t; i < nq * nch; i += NTH) {
      const int qr = R0 / H + i / nch, ch = i % nch;
      if (qr >= a.Mp) continue;
      a.xt[(size_t)ch * a.Mp + qr] = make_uint4(0u, 0u, 0u, 0u);
      a.xt[lo_plane + (size_t)ch * a.Mp + qr] = make_uint4(0u, 0u, 0u, 0u);
    }
    return;
  }
  const int Rl = (R0 + kFaRows < nrows ? R0 + kFaRows : nrows) - 1;  // last live row
  for (int i = t; i < kFaRows * HD / 4; i += NTH) {
    const int r = i / (HD / 4), d4 = i - r * (HD / 4);
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (R0 + r < nrows) v = reinterpret_cast<const float4 *>(a.q + (size_t)(R0 + r) * HD)[d4];
    *reinterpret_cast<float4 *>(&qs[r * QS + 4 * d4]) = v;
  }
  const int pos_first = qpos0 + R0 / H, pos_last = qpos0 + Rl / H;
  int kmin = a.sliding ? pos_first - a.window + 1 : 0;
  kmin = kmin > 0 ? kmin : 0;
  const int kmax = pos_last < keylen - 1 ? pos_last : keylen - 1;
  int rpos[4];
  bool rlive[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int R = R0 + 4 * g + v;
    rlive[v] = R < nrows;
    rpos[v] = qpos0 + (rlive[v] ? R : Rl) / H;
  }
  __syncthreads();
  const int d0 = w * DW;
  float4 qr[NJ];  // lane (c, g): Q row c, dims d0 + 16 j + 4 g .. + 3
#pragma unroll
  for (int j = 0; j < NJ; ++j) qr[j] = *reinterpret_cast<const float4 *>(&qs[c * QS + d0 + 16 * j + 4 * g]);
  float m[4] = {-1e30f, -1e30f, -1e30f, -1e30f}, l[4] = {0.f, 0.f, 0.f, 0.f};
  f32x4 o[4 * NQ];  // output tile 4q + e, column c: dim d0 + 64 q + 4 c + e
#pragma unroll
  for (int n = 0; n < 4 * NQ; ++n) o[n] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const int kt0 = kmin / 16, kt1 = kmax / 16;
  float4 kr[NJ], vr[4][NQ];
  // the next tile's K once this tile's partial S is formed, its V once this
  // tile's P.V is done (past the last tile, the last one again)
  auto load_k = [&](int kt) {
    kt = kt < kt1 ? kt : kt1;
    const int kc = kt * 16 + c < kmax ? kt * 16 + c : kmax;
    const float *kp = a.k + (size_t)kc * HD + d0 + 4 * g;
#pragma unroll
    for (int j = 0; j < NJ; ++j) kr[j] = *reinterpret_cast<const float4 *>(kp + 16 * j);
  };
  auto load_v = [&](int kt) {
    kt = kt < kt1 ? kt : kt1;
#pragma unroll
    for (int sp = 0; sp < 4; ++sp) {
      const int kv = kt * 16 + 4 * sp + g < kmax ? kt * 16 + 4 * sp + g : kmax;
      const float *vp = a.v + (size_t)kv * HD + d0 + 4 * c;
#pragma unroll
      for (int q = 0; q < NQ; ++q) vr[sp][q] = *reinterpret_cast<const float4 *>(vp + 64 * q);
    }
  };
  // key group kg takes tiles kt0 + kg, kt0 + kg + KG, ...; every wave runs
  // the same number of steps (a step past kt1 re-reads tile kt1 with all of
  // its keys masked), so the barriers match
  const int steps = (kt1 - kt0) / KG + 1;
  load_k(kt0 + kg);
  load_v(kt0 + kg);
  float *pw = ps[kg * DQ + w];
  for (int it = 0; it < steps; ++it) {
    const int kt = kt0 + kg + it * KG;
    const int b = it & 1;
    f32x4 sa[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sa[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const float4 kv = kr[j], qv = qr[j];
      sa[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(qv.x, kv.x, sa[0], 0, 0, 0);
      sa[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(qv.y, kv.y, sa[1], 0, 0, 0);
      sa[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(qv.z, kv.z, sa[2], 0, 0, 0);
      sa[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(qv.w, kv.w, sa[3], 0, 0, 0);
    }
    load_k(kt + KG);
    sx[b][kg][w][lane] = (sa[0] + sa[1]) + (sa[2] + sa[3]);
    __syncthreads();
    f32x4 s = sx[b][kg][0][lane];
#pragma unroll
    for (int d = 1; d < DQ; ++d) s += sx[b][kg][d][lane];
    const int key = kt * 16 + c;
    float corr[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const bool ok = rlive[v] && key <= rpos[v] && key < keylen &&
                      (!a.sliding || key > rpos[v] - a.window);
      const float tm = row16_reduce(ok ? s[v] : -1e30f, [](float x, float y) { return fmaxf(x, y); });
      const float mn = fmaxf(m[v], tm);
      corr[v] = expf(m[v] - mn);
      const float p = ok ? expf(s[v] - mn) : 0.f;
      l[v] = l[v] * corr[v] + row16_reduce(p, [](float x, float y) { return x + y; });
      m[v] = mn;
      pw[(4 * g + v) * kFaPStride + (c & 3) * 4 + (c >> 2)] = p;
    }
#pragma unroll
    for (int n = 0; n < 4 * NQ; ++n)
#pragma unroll
      for (int v = 0; v < 4; ++v) o[n][v] *= corr[v];
    const float4 pa = *reinterpret_cast<const float4 *>(&pw[c * kFaPStride + 4 * g]);
    const float pv[4] = {pa.x, pa.y, pa.z, pa.w};
#pragma unroll
    for (int sp = 0; sp < 4; ++sp)
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const float4 vv = vr[sp][q];
        o[4 * q + 0] = __builtin_amdgcn_mfma_f32_16x16x4f32(pv[sp], vv.x, o[4 * q + 0], 0, 0, 0);
        o[4 * q + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(pv[sp], vv.y, o[4 * q + 1], 0, 0, 0);
        o[4 * q + 2] = __builtin_amdgcn_mfma_f32_16x16x4f32(pv[sp], vv.z, o[4 * q + 2], 0, 0, 0);
        o[4 * q + 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(pv[sp], vv.w, o[4 * q + 3], 0, 0, 0);
      }
    load_v(kt + KG);
  }
  // O by dims into qs: each key group's (max, sum) in slot kg (the other
  // slots weight 0), its O weighted by e^(m_kg - M) and added in key-group
  // order, as attn_rows_store merges them
  __syncthreads();
  if (w == 0 && c == 0)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      wm[kg][4 * g + v] = m[v];
      wl[kg][4 * g + v] = l[v];
    }
  if (KG < kFaWaves && t < kFaRows * (kFaWaves - KG)) {
    wm[KG + t / kFaRows][t % kFaRows] = -1e30f;
    wl[KG + t / kFaRows][t % kFaRows] = 0.f;
  }
  __syncthreads();
  float f[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int r = 4 * g + v;
    float M = wm[0][r];
#pragma unroll
    for (int k = 1; k < KG; ++k) M = fmaxf(M, wm[k][r]);
    f[v] = KG > 1 ? expf(m[v] - M) : 1.f;
  }
  for (int k = 0; k < KG; ++k) {
    if (kg == k)
#pragma unroll
      for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          float4 *dst = reinterpret_cast<float4 *>(&qs[(4 * g + v) * QS + d0 + 64 * q + 4 * c]);
          const float4 add = make_float4(o[4 * q][v] * f[v], o[4 * q + 1][v] * f[v],
                                         o[4 * q + 2][v] * f[v], o[4 * q + 3][v] * f[v]);
          if (k == 0) {
            *dst = add;
          } else {
            const float4 cur = *dst;
            *dst = make_float4(cur.x + add.x, cur.y + add.y, cur.z + add.z, cur.w + add.w);
          }
        }
    __syncthreads();
  }
  attn_rows_store<HD, NTH>(a, qs, wm, wl, R0, nrows, t);
}

constexpr int kDecMaxKeys = 16;
constexpr int kMaxSplits = 1024;


template <int DPL>
__global__ __launch_bounds__(kBlock) void attn_dec_kernel(const float *__restrict__ q,
                                                          const float *__restrict__ k,
                                                          const float *__restrict__ v,
                                                          float *__restrict__ part, int H,
                                                          int keylen_host,
                                                          const int *__restrict__ pos_dev,
                                                          int sliding, int window) {
  constexpr int HD = 64 * DPL;
  constexpr int D32 = HD / 32;                            // q dims per lane (32 lanes / head)
  constexpr int DPT = HD / kBlock > 0 ? HD / kBlock : 1;  // output dims per thread
  __shared__ float4 ks[kDecMaxKeys * HD / 4];
  __shared__ __align__(16) float ps[kDecMaxKeys][kMaxHeads];
  __shared__ float mh[kMaxHeads], lh[kMaxHeads];
  const int t = threadIdx.x;
  const int keylen = pos_dev ? *pos_dev + 1 : keylen_host;
  const int qpos = keylen - 1;
  int lo = 0;
  if (sliding && qpos - window + 1 > 0) lo = qpos - window + 1;
  const int per = (keylen - lo + (int)gridDim.x - 1) / (int)gridDim.x;
  const int k0 = lo + blockIdx.x * per;
  const int n = k0 < keylen ? (keylen - k0 < per ? keylen - k0 : per) : 0;
  const int h = t >> 5, ds = t & 31;
  const bool dlive = t < HD;

  // all global loads first: q slice of head h, the block's K rows (to LDS),
  // the V elements of this thread's output dims
  // (loads are unconditional from clamped in-bounds addresses, so no branch
  // separates them; keys >= n and dims >= HD are loaded but never used)
  const float hq = h < H ? 1.f : 0.f;
  const float *qh = q + (h < H ? h : 0) * HD + ds * D32;
  float qv[D32];
#pragma unroll
  for (int j = 0; j < D32; ++j) qv[j] = qh[j] * hq;
  auto row = [&](int kl) { return (size_t)(k0 + kl < keylen ? k0 + kl : keylen - 1) * HD; };
  float4 kr[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    const int idx = t + i * kBlock;  // float4 index in the 16 x HD tile
    const int kl = idx / (HD / 4);
    kr[i] = reinterpret_cast<const float4 *>(k + row(kl))[idx % (HD / 4)];  // rows >= n unused
  }
  const int td = dlive ? t : 0;
  float vv[kDecMaxKeys][DPT];
#pragma unroll
  for (int kl = 0; kl < kDecMaxKeys; ++kl)
#pragma unroll
    for (int i = 0; i < DPT; ++i) vv[kl][i] = v[row(kl) + td + i * kBlock];  // kl >= n unused
#pragma unroll
  for (int i = 0; i < DPL; ++i) ks[t + i * kBlock] = kr[i];
  __syncthreads();

  // QK of head h (32 lanes, lane ds holds dims [ds*D32, ds*D32 + D32)): the
  // 16 partial dots first, then one reduce-scatter over the 32 lanes (xor 16,
  // then the DPP row mirror, half-row mirror and quad swaps) leaves the logit
  // of key 8 b4 + 4 b3 + 2 b2 + b1 in lanes ds and ds ^ 1 (b = bits of ds).
  const float *ksf = reinterpret_cast<const float *>(ks);
  float dv[kDecMaxKeys];
#pragma unroll
  for (int kl = 0; kl < kDecMaxKeys; ++kl) {
    float a = 0.f;
#pragma unroll
    for (int j = 0; j < D32; ++j) a = fmaf(qv[j], ksf[kl * HD + ds * D32 + j], a);
    dv[kl] = a;  // rows >= n hold finite data of a clamped row: discarded below
  }
  const bool b4 = ds & 16, b3 = ds & 8, b2 = ds & 4, b1 = ds & 2;
  float a8[8], a4[4], a2[2];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float keep = b4 ? dv[8 + i] : dv[i], send = b4 ? dv[i] : dv[8 + i];
    a8[i] = keep + __shfl_xor(send, 16, 64);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float keep = b3 ? a8[4 + i] : a8[i], send = b3 ? a8[i] : a8[4 + i];
    a4[i] = keep + dpp_f32<0x140>(send);  // row_mirror: lane i <-> 15 - i
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float keep = b2 ? a4[2 + i] : a4[i], send = b2 ? a4[i] : a4[2 + i];
    a2[i] = keep + dpp_f32<0x141>(send);  // row_half_mirror: lane i <-> 7 - i
  }
  float sk = (b1 ? a2[1] : a2[0]) + dpp_f32<0x4E>(b1 ? a2[0] : a2[1]);  // quad swap pairs
  sk += dpp_f32<0xB1>(sk);
  const int key = (b4 ? 8 : 0) + (b3 ? 4 : 0) + (b2 ? 2 : 0) + (b1 ? 1 : 0);
  const bool kvalid = key < n;
  // softmax over the block's keys (each key sits in two lanes)
  float m = kvalid ? sk : -1e30f;
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  const float p = kvalid ? expf(sk - m) : 0.f;
  const float l = team_sum<32>((ds & 1) ? 0.f : p);
  if (!(ds & 1) && h < H && key < kDecMaxKeys) ps[key][h] = p;
  if (ds == 0 && h < H) {
    mh[h] = m;
    lh[h] = l;
  }
  __syncthreads();

  // PV: thread t owns dims t, t + 256, ... of every head
  float acc[kMaxHeads][DPT];
#pragma unroll
  for (int hh = 0; hh < kMaxHeads; ++hh)
#pragma unroll
    for (int i = 0; i < DPT; ++i) acc[hh][i] = 0.f;
#pragma unroll
  for (int kl = 0; kl < kDecMaxKeys; ++kl) {
    if (kl >= n) break;
    const float4 p0 = reinterpret_cast<const float4 *>(ps[kl])[0];
    const float4 p1 = reinterpret_cast<const float4 *>(ps[kl])[1];
    const float pk[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
    for (int hh = 0; hh < kMaxHeads; ++hh)
#pragma unroll
      for (int i = 0; i < DPT; ++i) acc[hh][i] = fmaf(pk[hh], vv[kl][i], acc[hh][i]);
  }
  if (dlive) {
#pragma unroll
    for (int hh = 0; hh < kMaxHeads; ++hh) {
      if (hh >= H) break;
      float *pp = part + ((size_t)blockIdx.x * H + hh) * (HD + 2);
#pragma unroll
      for (int i = 0; i < DPT; ++i) pp[2 + t + i * kBlock] = acc[hh][i];
      if (t == 0) {
        pp[0] = mh[hh];
        pp[1] = lh[hh];
      }
    }
  }
}

// Merges split partials:
//   out = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s.
// Block (query row, head, 64-dim slice).  Each thread issues the loads of the
// first 16 of its splits (s = wave + 4 i) before anything else; the 4 waves'
// sums meet in LDS.  Splits beyond the keys of this call (kpw > 0:
// ceil(keylen / kpw) splits) were not written.
__global__ __launch_bounds__(kBlock) void attn_combine_kernel(const float *__restrict__ part,
                                                              int H, int hd, int kpw,
                                                              int nsplit, int keylen,
                                                              const int *__restrict__ pos_dev,
                                                              int qrows, float *__restrict__ out) {
  constexpr int U = 16;
  __shared__ float red[4];
  __shared__ float accs[4][64];
  __shared__ float ls4[4];
  const int dslices = hd >> 6;
  const int b = blockIdx.x;
  const int dsl = b % dslices, qh = b / dslices;
  const int qr = qh / H, h = qh - qr * H;
  const int kl = pos_dev ? *pos_dev + qrows : keylen;
  int ns = nsplit;
  if (kpw > 0 && (kl + kpw - 1) / kpw < ns) ns = (kl + kpw - 1) / kpw;
  const size_t stride = (size_t)hd + 2, sstep = (size_t)H * stride;
  const float *pb = part + ((size_t)qr * nsplit * H + h) * stride;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int d = dsl * 64 + lane;
  float mv[U], lv[U], ov[U];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const int sp = wave + 4 * i;
    const float *ps = pb + (size_t)(sp < ns ? sp : 0) * sstep;  // clamped: no branch
    const float m0 = ps[0], l0 = ps[1], o0 = ps[2 + d];
    mv[i] = sp < ns ? m0 : -3.4e38f;
    lv[i] = sp < ns ? l0 : 0.f;
    ov[i] = sp < ns ? o0 : 0.f;
  }
  // block max of all split maxima (splits past 4U are read again below)
  float mx = -3.4e38f;
#pragma unroll
  for (int i = 0; i < U; ++i) mx = fmaxf(mx, mv[i]);
  for (int sp = wave + 4 * U; sp < ns; sp += 4) mx = fmaxf(mx, pb[(size_t)sp * sstep]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float acc = 0.f, lsum = 0.f;
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const float w = expf(mv[i] - M);
    acc = fmaf(w, ov[i], acc);
    lsum = fmaf(w, lv[i], lsum);
  }
  for (int sp = wave + 4 * U; sp < ns; sp += 4) {
    const float *ps = pb + (size_t)sp * sstep;
    const float w = expf(ps[0] - M);
    acc = fmaf(w, ps[2 + d], acc);
    lsum = fmaf(w, ps[1], lsum);
  }
  accs[wave][lane] = acc;
  if (lane == 0) ls4[wave] = lsum;
  __syncthreads();
  if (wave == 0) {
    const float L = ls4[0] + ls4[1] + ls4[2] + ls4[3];
    out[((size_t)qr * H + h) * hd + d] =
        (accs[0][lane] + accs[1][lane] + accs[2][lane] + accs[3][lane]) / L;
  }
}

// ---- PLE_MIX_SHADER (gpu-runtime.js:1250-1263) ------------------------------
// One block per (row, layer) chunk of `width` values.  p = proj * pre_scale
// is the input of the norm: the model's ops.scale of the projection
// (gemma4-webgpu.js, 1/sqrt(hidden)) travels here as the same FP32 product,
// and GPUOps.pleMix passes 1.  The products that are fused are spelled out,
// so both forms below round alike.
__global__ __launch_bounds__(kBlock) void ple_mix_kernel(const float *__restrict__ proj,
                                                         float pre_scale,
                                                         const float *__restrict__ norm_scale,
                                                         const float *__restrict__ token_ple,
                                                         int width, float eps, float ple_scale,
                                                         float out_scale,
                                                         float *__restrict__ y) {
  __shared__ float red[4];
  const size_t base = (size_t)blockIdx.x * width;
  float ss = 0.f;
  for (int d = threadIdx.x; d < width; d += kBlock) {
    const float p = proj[base + d] * pre_scale;
    ss = fmaf(p, p, ss);
  }
  const float inv = inv_rms(block_sum(ss, red), width, eps);
  for (int d = threadIdx.x; d < width; d += kBlock) {
    const float pn = proj[base + d] * pre_scale * inv;
    y[base + d] = fmaf(pn, norm_scale[d], token_ple[base + d] * ple_scale) * out_scale;
  }
}

// The same with one wave per chunk, four chunks per block, for many chunks
// (the prefill's rows x layers).  The sum of squares is the block's: lane l
// plays threads l, 64 + l, 128 + l and 192 + l, each adding its values
// d = thread (mod 256) in d order, then each set of 64 threads is summed as
// one wave and the four sums are added in order.  (512-token prefill, 17920
// chunks of 256: 18.6 against 21.1 us; one-token decode, 35 chunks: the
// block form, 3.5 against 5.7 us.)
__global__ __launch_bounds__(kBlock) void ple_mix_rows_kernel(
    const float *__restrict__ proj, float pre_scale, const float *__restrict__ norm_scale,
    const float *__restrict__ token_ple, int width, int chunks, float eps, float ple_scale,
    float out_scale, float *__restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int ck = blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  if (ck >= chunks) return;  // whole waves
  const size_t base = (size_t)ck * width;
  float ss[4] = {0.f, 0.f, 0.f, 0.f};
  for (int d0 = 0; d0 < width; d0 += kBlock)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = d0 + 64 * j + lane;
      if (d < width) {
        const float p = proj[base + d] * pre_scale;
        ss[j] = fmaf(p, p, ss[j]);
      }
    }
  const float tot = ((wave_sum(ss[0]) + wave_sum(ss[1])) + wave_sum(ss[2])) + wave_sum(ss[3]);
  const float inv = inv_rms(tot, width, eps);
  for (int d = lane; d < width; d += 64) {
    const float pn = proj[base + d] * pre_scale * inv;
    y[base + d] = fmaf(pn, norm_scale[d], token_ple[base + d] * ple_scale) * out_scale;
  }
}

// ---- embedding rows: bf16Rows(embed_tokens, ids) then ops.scale -------------
// y[r, i] = float(E[ids[r], i]) * scale.  An id outside [0, vocab) gives a
// NaN row and touches no table memory.
__global__ __launch_bounds__(kBlock) void embed_kernel(const uint16_t *__restrict__ E, int vocab,
                                                       int width, const int *__restrict__ ids,
                                                       float scale, float *__restrict__ y) {
  const int r = blockIdx.x;
  const int id = ids[r];
  const bool ok = id >= 0 && id < vocab;
  for (int i = threadIdx.x; i < width; i += kBlock)
    y[(size_t)r * width + i] =
        ok ? bf16_to_f32(E[(size_t)id * width + i]) * scale : __int_as_float(0x7fc00000);
}

int grid1(size_t n, dim3 *g) {
  const size_t b = (n + kBlock - 1) / kBlock;
  if (b > 0x7fffffffu) return fail(G4_E_ARG, "element count %zu too large", n);
  *g = dim3((unsigned)b);
  return G4_OK;
}

}  // namespace

// ---- launchers shared with the engine ---------------------------------------

int launch_norm_rope_qkv(const float *q, int qparts, size_t qpstride, const float *k,
                         const float *v, int rows, int heads, int hd, const int *pos_dev,
                         const float *qscale, const float *kscale, int rope_angles, float base,
                         float eps, float *qy, float *kc, float *vc) {
  if (rows == 0) return G4_OK;
  if (qparts < 1 || qparts > kNormRopeMaxParts || hd > 2 * kBlock)
    return fail(G4_E_ARG, "norm_rope q/k/v: %d planes (1..%d), head_dim %d", qparts,
                kNormRopeMaxParts, hd);
  const int np = norm_rope_np(qparts);
  auto kernel = np == 1   ? norm_rope_qkv_kernel<1>
                : np == 2 ? norm_rope_qkv_kernel<2>
                : np == 3 ? norm_rope_qkv_kernel<3>
                : np == 4 ? norm_rope_qkv_kernel<4>
                          : norm_rope_qkv_kernel<kNormRopeMaxParts>;
  hipLaunchKernelGGL(kernel, dim3(rows * (heads + 2)), dim3(kBlock), 0, stream(), q, qparts,
                     qpstride, k, v, rows, heads, hd, pos_dev, qscale, kscale, rope_angles, base,
                     eps, qy, kc, vc);
  G4_LAUNCH_CHECK("norm_rope_qkv_kernel");
  return G4_OK;
}

int launch_rms(const float *x, int rows, int width, const float *scale, float eps, float *y,
               const int *pos_dev) {
  if (rows == 0) return G4_OK;
  hipLaunchKernelGGL(rms_kernel, dim3(rows), dim3(kBlock), 0, stream(), x, width, scale, eps, y,
                     pos_dev);
  G4_LAUNCH_CHECK("rms_kernel");
  return G4_OK;
}

int launch_add_scale(const float *a, const float *b, size_t n, float s, float *y) {
  if (n == 0) return G4_OK;
  dim3 g;
  if (int rc = grid1(n, &g)) return rc;
  hipLaunchKernelGGL(add_scale_kernel, g, dim3(kBlock), 0, stream(), a, b, n, s, y);
  G4_LAUNCH_CHECK("add_scale_kernel");
  return G4_OK;
}

int launch_scale(const float *a, size_t n, float s, float *y) {
  if (n == 0) return G4_OK;
  dim3 g;
  if (int rc = grid1(n, &g)) return rc;
  hipLaunchKernelGGL(scale_kernel, g, dim3(kBlock), 0, stream(), a, n, s, y);
  G4_LAUNCH_CHECK("scale_kernel");
  return G4_OK;
}

int launch_gelu_mul(const float *gate, const float *up, size_t n, float *y) {
  if (n == 0) return G4_OK;
  dim3 g;
  if (int rc = grid1(n, &g)) return rc;
  hipLaunchKernelGGL(gelu_mul_kernel, g, dim3(kBlock), 0, stream(), gate, up, n, y);
  G4_LAUNCH_CHECK("gelu_mul_kernel");
  return G4_OK;
}

int launch_gelu_ple(const float *gate, const float *ple, int rows, int layer, int width,
                    int layers, float *y) {
  if (rows == 0) return G4_OK;
  dim3 g;
  if (int rc = grid1((size_t)rows * width, &g)) return rc;
  hipLaunchKernelGGL(gelu_ple_kernel, g, dim3(kBlock), 0, stream(), gate, ple, rows, layer,
                     width, layers, y);
  G4_LAUNCH_CHECK("gelu_ple_kernel");
  return G4_OK;
}

int launch_norm_rope(const float *x, int rows, int heads, int hd, int pos0, const int *pos_dev,
                     const float *scale, int rope_angles, float base, float eps, float *y,
                     bool at_pos, int parts, size_t pstride) {
  if (rows == 0) return G4_OK;
  if (parts < 1 || parts > kNormRopeMaxParts)
    return fail(G4_E_ARG, "norm_rope: %d planes (1..%d)", parts, kNormRopeMaxParts);
  if (hd > 2 * kBlock)
    return fail(G4_E_ARG, "norm_rope: head_dim %d (at most %d)", hd, 2 * kBlock);
  // waves for the hd / 2 pairs: 1, 2 or 4
  const int nw = hd <= 128 ? 1 : hd <= 256 ? 2 : 4;
  const int np = norm_rope_np(parts);
  void (*kernel)(const float *, int, size_t, int, int, int, const int *, const float *, int,
                 float, float, float *, int) = nullptr;
#define G4_NR(NP)                                                                 \
  kernel = nw == 1 ? norm_rope_kernel<NP, 1> : nw == 2 ? norm_rope_kernel<NP, 2> \
                                             : norm_rope_kernel<NP, 4>
  switch (np) {
    case 1: G4_NR(1); break;
    case 2: G4_NR(2); break;
    case 3: G4_NR(3); break;
    case 4: G4_NR(4); break;
    default: G4_NR(kNormRopeMaxParts); break;
  }
#undef G4_NR
  hipLaunchKernelGGL(kernel, dim3(rows * heads), dim3(64 * nw), 0, stream(), x, parts, pstride,
                     heads, hd, pos0, pos_dev, scale, rope_angles, base, eps, y, (int)at_pos);
  G4_LAUNCH_CHECK("norm_rope_kernel");
  return G4_OK;
}

// Splits of the single-query kernel for up to max_keylen keys.
int dec_splits(int max_keylen) {
  const int need = (max_keylen + kDecMaxKeys - 1) / kDecMaxKeys;
  return need > 64 ? need : 64;
}

// Keys per split for the multi-query kernel such that the split count stays
// within the combine's limit.
int split_kpw(int kpw, int max_keylen) {
  const int min_kpw = (max_keylen + kMaxSplits - 1) / kMaxSplits;
  return kpw > min_kpw ? kpw : min_kpw;
}

size_t attention_part_floats(int qrows, int heads, int hd, int max_keylen, int kpw) {
  const size_t multi = (size_t)qrows * ((max_keylen + split_kpw(kpw, max_keylen) - 1) /
                                        split_kpw(kpw, max_keylen));
  const size_t single = (size_t)dec_splits(max_keylen);
  return (multi > single ? multi : single) * heads * ((size_t)hd + 2);
}

int launch_attention(const float *q, const float *k, const float *v, int qrows, int heads,
                     int hd, int keylen, int qpos0, const int *pos_dev, int max_keylen,
                     bool sliding, int window, int kpw, float *part, float *out, void *xt,
                     int *xe, int Mp, bool *x_done) {
  if (x_done) *x_done = false;
  if (qrows == 0) return G4_OK;
  if (max_keylen > kDecMaxKeys * kMaxSplits)
    return fail(G4_E_ARG, "attention: %d keys exceed the supported %d", max_keylen,
                kDecMaxKeys * kMaxSplits);
  if (qrows == 1) {
    // one query row: position keylen - 1 (or *pos_dev), keys split over the grid
    const int ns = dec_splits(max_keylen);
    const dim3 grid(ns);
    const int sl = sliding ? 1 : 0;
    switch (hd / 64) {
      case 1: hipLaunchKernelGGL(attn_dec_kernel<1>, grid, dim3(kBlock), 0, stream(), q, k, v, part, heads, keylen, pos_dev, sl, window); break;
      case 2: hipLaunchKernelGGL(attn_dec_kernel<2>, grid, dim3(kBlock), 0, stream(), q, k, v, part, heads, keylen, pos_dev, sl, window); break;
      case 4: hipLaunchKernelGGL(attn_dec_kernel<4>, grid, dim3(kBlock), 0, stream(), q, k, v, part, heads, keylen, pos_dev, sl, window); break;
      case 8: hipLaunchKernelGGL(attn_dec_kernel<8>, grid, dim3(kBlock), 0, stream(), q, k, v, part, heads, keylen, pos_dev, sl, window); break;
      default: return fail(G4_E_ARG, "attention: head_dim %d must be 64, 128, 256 or 512", hd);
    }
    G4_LAUNCH_CHECK("attn_dec_kernel");
    hipLaunchKernelGGL(attn_combine_kernel, dim3(heads * (hd / 64)), dim3(kBlock), 0, stream(),
                       part, heads, hd, 0, ns, keylen, pos_dev, qrows, out);
    G4_LAUNCH_CHECK("attn_combine_kernel");
    return G4_OK;
  }
  kpw = split_kpw(kpw, max_keylen);
  AttnArgs a;
  a.out = out;
  a.q = q;
  a.k = k;
  a.v = v;
  a.part = part;
  a.H = heads;
  a.hd = hd;
  a.keylen = keylen;
  a.qpos0 = qpos0;
  a.sliding = sliding ? 1 : 0;
  a.window = window;
  a.kpw = kpw;
  a.nsplit = (max_keylen + kpw - 1) / kpw;
  a.pos_dev = pos_dev;
  a.qrows = qrows;
  a.xt = nullptr;
  a.xe = nullptr;
  a.Mp = 0;
  // Many rows, or few keys: the matrix-core kernel (16 rows per block, no
  // merge pass).  A handful of rows over a long cache keeps the key split.
  if ((size_t)qrows * heads >= 64 || max_keylen <= 512) {
    // x' for the next GEMM when asked for and the block's 16 rows hold whole
    // query rows; the grid then also covers the GEMM's padding rows
    const bool xprep = xt && x_done && kFaRows % heads == 0 && Mp >= qrows && Mp % 16 == 0;
    if (xprep) {
      a.xt = static_cast<uint4 *>(xt);
      a.xe = xe;
      a.Mp = Mp;
    }
    const dim3 fgrid(((xprep ? Mp : qrows) * heads + kFaRows - 1) / kFaRows);
    switch (hd) {
      case 64: hipLaunchKernelGGL(attn_rows_mfma_kernel<64>, fgrid, dim3(256), 0, stream(), a); break;
      case 128: hipLaunchKernelGGL(attn_rows_mfma_kernel<128>, fgrid, dim3(256), 0, stream(), a); break;
      case 256: hipLaunchKernelGGL(attn_rows_mfma_kernel<256>, fgrid, dim3(256), 0, stream(), a); break;
      case 512: hipLaunchKernelGGL((attn_rows_dsplit_kernel<512, 4, 2>), fgrid, dim3(512), 0, stream(), a); break;
      default: return fail(G4_E_ARG, "attention: head_dim %d must be 64, 128, 256 or 512", hd);
    }
    G4_LAUNCH_CHECK("attn_rows_mfma_kernel");
    if (xprep) *x_done = true;
    return G4_OK;
  }
  const dim3 grid(a.nsplit, qrows);
  switch (hd / 64) {
    case 1: hipLaunchKernelGGL(attn_split_kernel<1>, grid, dim3(64), 0, stream(), a); break;
    case 2: hipLaunchKernelGGL(attn_split_kernel<2>, grid, dim3(64), 0, stream(), a); break;
    case 4: hipLaunchKernelGGL(attn_split_kernel<4>, grid, dim3(64), 0, stream(), a); break;
    case 8: hipLaunchKernelGGL(attn_split_kernel<8>, grid, dim3(64), 0, stream(), a); break;
    default: return fail(G4_E_ARG, "attention: head_dim %d must be 64, 128, 256 or 512", hd);
  }
  G4_LAUNCH_CHECK("attn_split_kernel");
  hipLaunchKernelGGL(attn_combine_kernel, dim3(qrows * heads * (hd / 64)), dim3(kBlock), 0,
                     stream(), part, heads, hd, kpw, a.nsplit, keylen, pos_dev, qrows, out);
  G4_LAUNCH_CHECK("attn_combine_kernel");
  return G4_OK;
}

int launch_ple_mix(const float *proj, float pre_scale, const float *norm_scale,
                   const float *token_ple, int rows, int width, int layers, float eps,
                   float ple_scale, float out_scale, float *y) {
  if (rows == 0) return G4_OK;
  const int chunks = rows * layers;
  if (chunks < 1024) {
    hipLaunchKernelGGL(ple_mix_kernel, dim3(chunks), dim3(kBlock), 0, stream(), proj, pre_scale,
                       norm_scale, token_ple, width, eps, ple_scale, out_scale, y);
    G4_LAUNCH_CHECK("ple_mix_kernel");
    return G4_OK;
  }
  hipLaunchKernelGGL(ple_mix_rows_kernel, dim3((chunks + kBlock / 64 - 1) / (kBlock / 64)),
                     dim3(kBlock), 0, stream(), proj, pre_scale, norm_scale, token_ple, width,
                     chunks, eps, ple_scale, out_scale, y);
  G4_LAUNCH_CHECK("ple_mix_rows_kernel");
  return G4_OK;
}

int launch_embed(const uint16_t *E, int vocab, int width, const int *ids_dev, int n, float scale,
                 float *y) {
  if (n == 0) return G4_OK;
  hipLaunchKernelGGL(embed_kernel, dim3(n), dim3(kBlock), 0, stream(), E, vocab, width, ids_dev,
                     scale, y);
  G4_LAUNCH_CHECK("embed_kernel");
  return G4_OK;
}

}  // namespace g4

// ---- C ABI ---------------------------------------------------------------------

namespace {
using namespace g4;

Workspace g_attn_ws, g_argmax_ws;

int check_f32(const float *p, size_t n, const char *what) {
  return check_device_range(p, n * 4, what);
}

// Keys per split of the attention kernel: a few for decode (many small
// blocks), more when many query rows already fill the GPU.
int attn_kpw(int qrows) { return qrows <= 4 ? 4 : 32; }

}  // namespace

G4_API int g4_rms(const float *x, int rows, int width, const float *scale, float eps, float *y) {
  G4_CHECK_INIT();
  if (rows < 0 || width <= 0) return fail(G4_E_ARG, "g4_rms: rows %d, width %d", rows, width);
  if (rows == 0) return ok();
  const size_t n = (size_t)rows * width;
  int rc = check_f32(x, n, "g4_rms x");
  if (!rc && scale) rc = check_f32(scale, width, "g4_rms scale");
  if (!rc) rc = check_f32(y, n, "g4_rms y");
  if (!rc) rc = launch_rms(x, rows, width, scale, eps, y, nullptr);
  return rc ? rc : ok();
}

G4_API int g4_add_scale(const float *a, const float *b, size_t n, float scale, float *y) {
  G4_CHECK_INIT();
  if (n == 0) return ok();
  int rc = check_f32(a, n, "g4_add_scale a");
  if (!rc) rc = check_f32(b, n, "g4_add_scale b");
  if (!rc) rc = check_f32(y, n, "g4_add_scale y");
  if (!rc) rc = launch_add_scale(a, b, n, scale, y);
  return rc ? rc : ok();
}

G4_API int g4_scale(const float *a, size_t n, float scale, float *y) {
  G4_CHECK_INIT();
  if (n == 0) return ok();
  int rc = check_f32(a, n, "g4_scale a");
  if (!rc) rc = check_f32(y, n, "g4_scale y");
  if (!rc) rc = launch_scale(a, n, scale, y);
  return rc ? rc : ok();
}

G4_API int g4_gelu_mul(const float *gate, const float *up, size_t n, float *y) {
  G4_CHECK_INIT();
  if (n == 0) return ok();
  int rc = check_f32(gate, n, "g4_gelu_mul gate");
  if (!rc) rc = check_f32(up, n, "g4_gelu_mul up");
  if (!rc) rc = check_f32(y, n, "g4_gelu_mul y");
  if (!rc) rc = launch_gelu_mul(gate, up, n, y);
  return rc ? rc : ok();
}

G4_API int g4_gelu_ple(const float *gate, const float *ple, int rows, int layer, int width,
                       int layers, float *y) {
  G4_CHECK_INIT();
  if (rows < 0 || width <= 0 || layers <= 0 || layer < 0 || layer >= layers)
    return fail(G4_E_ARG, "g4_gelu_ple: rows %d, layer %d of %d, width %d", rows, layer, layers,
                width);
  if (rows == 0) return ok();
  const size_t n = (size_t)rows * width;
  int rc = check_f32(gate, n, "g4_gelu_ple gate");
  if (!rc) rc = check_f32(ple, n * layers, "g4_gelu_ple ple");
  if (!rc) rc = check_f32(y, n, "g4_gelu_ple y");
  if (!rc) rc = launch_gelu_ple(gate, ple, rows, layer, width, layers, y);
  return rc ? rc : ok();
}

G4_API int g4_norm_rope(const float *x, int rows, int heads, int head_dim, int pos0,
                        const float *scale, int rope_angles, float base, float eps, float *y) {
  G4_CHECK_INIT();
  if (rows < 0 || heads <= 0 || head_dim <= 0 || head_dim % 2 != 0 || head_dim > 512 ||
      pos0 < 0 || rope_angles < 0 || rope_angles > head_dim / 2)
    return fail(G4_E_ARG,
                "g4_norm_rope: rows %d, heads %d, head_dim %d (even, <= 512), pos0 %d, "
                "rope_angles %d",
                rows, heads, head_dim, pos0, rope_angles);
  if (rows == 0) return ok();
  const size_t n = (size_t)rows * heads * head_dim;
  int rc = check_f32(x, n, "g4_norm_rope x");
  if (!rc) rc = check_f32(scale, head_dim, "g4_norm_rope scale");
  if (!rc) rc = check_f32(y, n, "g4_norm_rope y");
  if (!rc)
    rc = launch_norm_rope(x, rows, heads, head_dim, pos0, nullptr, scale, rope_angles, base, eps,
                          y, false);
  return rc ? rc : ok();
}

G4_API int g4_attention(const float *q, const float *k, const float *v, int qrows, int heads,
                        int head_dim, int keylen, int qpos0, int sliding, int window, float *y) {
  G4_CHECK_INIT();
  if (qrows < 0 || heads <= 0 || heads > 8 ||
      (head_dim != 64 && head_dim != 128 && head_dim != 256 && head_dim != 512))
    return fail(G4_E_ARG, "g4_attention: qrows %d, heads %d (<= 8), head_dim %d (64..512)",
                qrows, heads, head_dim);
  if (qrows == 0) return ok();
  if (qpos0 < 0 || keylen < qpos0 + qrows || (sliding && window <= 0))
    return fail(G4_E_ARG,
                "g4_attention: keylen %d must cover query positions %d..%d (window %d)", keylen,
                qpos0, qpos0 + qrows - 1, window);
  const size_t qn = (size_t)qrows * heads * head_dim;
  int rc = check_f32(q, qn, "g4_attention q");
  if (!rc) rc = check_f32(k, (size_t)keylen * head_dim, "g4_attention k");
  if (!rc) rc = check_f32(v, (size_t)keylen * head_dim, "g4_attention v");
  if (!rc) rc = check_f32(y, qn, "g4_attention y");
  if (rc) return rc;
  const int kpw = attn_kpw(qrows);
  void *part = nullptr;
  rc = g_attn_ws.get(attention_part_floats(qrows, heads, head_dim, keylen, kpw) * 4, &part,
                     "g4_attention");
  if (!rc)
    rc = launch_attention(q, k, v, qrows, heads, head_dim, keylen, qpos0, nullptr, keylen,
                          sliding != 0, window, kpw, static_cast<float *>(part), y);
  return rc ? rc : ok();
}

G4_API int g4_ple_mix(const float *proj, const float *norm_scale, const float *token_ple,
                      int rows, int width, int layers, float *y) {
  G4_CHECK_INIT();
  if (rows < 0 || width <= 0 || layers <= 0)
    return fail(G4_E_ARG, "g4_ple_mix: rows %d, width %d, layers %d", rows, width, layers);
  if (rows == 0) return ok();
  const size_t n = (size_t)rows * layers * width;
  int rc = check_f32(proj, n, "g4_ple_mix proj");
  if (!rc) rc = check_f32(norm_scale, width, "g4_ple_mix norm_scale");
  if (!rc) rc = check_f32(token_ple, n, "g4_ple_mix token_ple");
  if (!rc) rc = check_f32(y, n, "g4_ple_mix y");
  // PLE_MIX_SHADER constants: eps 1e-6, token rows * 16 (= sqrt(256)), * 1/sqrt(2)
  if (!rc)
    rc = launch_ple_mix(proj, 1.f, norm_scale, token_ple, rows, width, layers, 1e-6f, 16.f,
                        0.7071067811865476f, y);
  return rc ? rc : ok();
}

G4_API int g4_embed(const void *E, int vocab, int width, const int32_t *ids_dev, int n,
                    float scale, float *y) {
  G4_CHECK_INIT();
  if (vocab <= 0 || width <= 0 || n < 0)
    return fail(G4_E_ARG, "g4_embed: vocab %d, width %d, n %d", vocab, width, n);
  if (n == 0) return ok();
  int rc = check_device_range(E, (size_t)vocab * width * 2, "g4_embed E");
  if (!rc) rc = check_device_range(ids_dev, (size_t)n * 4, "g4_embed ids");
  if (!rc) rc = check_f32(y, (size_t)n * width, "g4_embed y");
  if (!rc)
    rc = launch_embed(static_cast<const uint16_t *>(E), vocab, width, ids_dev, n, scale, y);
  return rc ? rc : ok();
}

G4_API int g4_argmax(const float *x, int n, int32_t *out_dev) {
  G4_CHECK_INIT();
  if (n <= 0) return fail(G4_E_ARG, "g4_argmax: n %d", n);
  int rc = check_f32(x, n, "g4_argmax x");
  if (!rc) rc = check_device_range(out_dev, 4, "g4_argmax out");
  void *part = nullptr;
  if (!rc) rc = g_argmax_ws.get(argmax_blocks(n) * sizeof(float2), &part, "g4_argmax");
  if (!rc) rc = launch_argmax(x, n, static_cast<float2 *>(part), out_dev);
  return rc ? rc : ok();
}
