// Tied BF16 LM head: the gfx950 replacement of GPUOps.headChunk and
// BF16_HEAD_SHADER (custom-webgpu/gpu-runtime.js:1265-1277, 1370-1376):
//   out[r] = softcap * tanh((scale * sum_k x[k] * E[r, k]) / softcap)
// The reference runs one thread per vocabulary row with a serial K loop and
// 64 dispatches of 4096 rows; here a wave owns a few rows at a time and the
// whole [rows, K] slab streams through with 16-byte loads.
#include "g4_gemv.h"
#include "g4_internal.h"
#include "g4_ops.h"

namespace g4 {
namespace {

constexpr int kRowsPerWave = 8;
constexpr int kNoIndex = 0x7fffffff;

// Greedy selection keeps the first index of the largest finite logit: topK
// (gpu-runtime.js:1396-1425) skips non-finite values and, with a stable sort,
// ranks equal values by index.
__device__ __forceinline__ void arg_better(float v, int i, float &bv, int &bi) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

__device__ __forceinline__ void wave_argmax(float &bv, int &bi) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    arg_better(ov, oi, bv, bi);
  }
}

// Block-wide (max, first index); thread 0 writes it to partials[blockIdx.x].
__device__ __forceinline__ void block_argmax_store(float bv, int bi, float2 *partials) {
  __shared__ float sv[4];
  __shared__ int si[4];
  wave_argmax(bv, bi);
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = bv;
    si[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) arg_better(sv[w], si[w], bv, bi);
    partials[blockIdx.x] = make_float2(bv, __int_as_float(bi));
  }
}

// Lane l holds x for the 8-element chunks l, l+64, ... (CPL chunks) and
// reads the same chunks of each of the wave's 8 rows. Every load is issued
// before any arithmetic: rows past the end are clamped to the last row and
// chunks past K are read in range and zeroed, so no load sits in a branch.
// The 8 row sums are reduced transposed: each exchange step halves the rows
// a lane carries (8 -> 4 -> 2 -> 1 over lane distances 32, 16, 8), and the
// last 8-lane sum runs on DPP, so lane 8*r' + j ends with row
// r' = 4*bit5 + 2*bit4 + bit3 of its lane index.
template <int CPL>
__global__ __launch_bounds__(256) void bf16_head_kernel(
    const float *__restrict__ x, const uint16_t *__restrict__ E, int rows, int K,
    float *__restrict__ out, float scale, float softcap, float2 *__restrict__ partials) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int row0 = wave * kRowsPerWave;
  // waves past the end still take part in the block's argmax
  if (row0 >= rows && !partials) return;
  const int chunks = K >> 3;

  uint4 w[kRowsPerWave][CPL];
#pragma unroll
  for (int r = 0; r < kRowsPerWave; ++r) {
    const int row = min(row0 + r, rows - 1);
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = min(lane + 64 * i, chunks - 1);
      w[r][i] = ld_nt(reinterpret_cast<const uint4 *>(E + (size_t)row * K) + c);
    }
  }
  float xv[CPL][8];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
#pragma unroll
    for (int e = 0; e < 8; ++e) xv[i][e] = x[min(c, chunks - 1) * 8 + e];
    if (c >= chunks) {
#pragma unroll
      for (int r = 0; r < kRowsPerWave; ++r) w[r][i] = make_uint4(0, 0, 0, 0);
    }
  }

  float acc[kRowsPerWave];
#pragma unroll
  for (int r = 0; r < kRowsPerWave; ++r) {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const uint32_t u[4] = {w[r][i].x, w[r][i].y, w[r][i].z, w[r][i].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        a0 = fmaf(xv[i][2 * k], __uint_as_float(u[k] << 16), a0);
        a1 = fmaf(xv[i][2 * k + 1], __uint_as_float(u[k] & 0xffff0000u), a1);
      }
    }
    acc[r] = a0 + a1;
  }

  const bool b5 = lane & 32, b4 = lane & 16, b3 = lane & 8;
  float a4[4], a2[2];
#pragma unroll
  for (int r = 0; r < 4; ++r)
    a4[r] = (b5 ? acc[r + 4] : acc[r]) + __shfl_xor(b5 ? acc[r] : acc[r + 4], 32, 64);
#pragma unroll
  for (int r = 0; r < 2; ++r)
    a2[r] = (b4 ? a4[r + 2] : a4[r]) + __shfl_xor(b4 ? a4[r] : a4[r + 2], 16, 64);
  float sum = (b3 ? a2[1] : a2[0]) + __shfl_xor(b3 ? a2[0] : a2[1], 8, 64);
  sum = team_sum<8>(sum);

  const int row = row0 + (b5 ? 4 : 0) + (b4 ? 2 : 0) + (b3 ? 1 : 0);
  float bv = -INFINITY;
  int bi = kNoIndex;
  if ((lane & 7) == 0 && row < rows) {
    const float raw = sum * scale;
    const float v = softcap > 0.f ? tanhf(raw / softcap) * softcap : raw;
    out[row] = v;
    if (isfinite(v)) {
      bv = v;
      bi = row;
    }
  }
  if (partials) block_argmax_store(bv, bi, partials);
}

// Plain argmax over x[0, n): per-block partials, then argmax_final_kernel.
__global__ __launch_bounds__(256) void argmax_blocks_kernel(const float *__restrict__ x, int n,
                                                            float2 *__restrict__ partials) {
  float bv = -INFINITY;
  int bi = kNoIndex;
  const int per = (n + gridDim.x - 1) / gridDim.x;
  const int i0 = blockIdx.x * per, i1 = i0 + per < n ? i0 + per : n;
  for (int i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
    const float v = x[i];
    if (isfinite(v)) arg_better(v, i, bv, bi);
  }
  block_argmax_store(bv, bi, partials);
}

// One block reduces the partials; out_idx gets -1 when no value was finite
// (topK throws "no finite logits" in that case).
__global__ __launch_bounds__(256) void argmax_final_kernel(const float2 *__restrict__ partials,
                                                           int nparts, int *__restrict__ out_idx) {
  __shared__ float sv[4];
  __shared__ int si[4];
  float bv = -INFINITY;
  int bi = kNoIndex;
  for (int i = threadIdx.x; i < nparts; i += blockDim.x) {
    const float2 p = partials[i];
    arg_better(p.x, __float_as_int(p.y), bv, bi);
  }
  wave_argmax(bv, bi);
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = bv;
    si[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) arg_better(sv[w], si[w], bv, bi);
    *out_idx = bi == kNoIndex ? -1 : bi;
  }
}

template <int CPL>
int launch_head(const float *x, const uint16_t *E, int rows, int K, float *out, float scale,
                float softcap, float2 *partials) {
  hipLaunchKernelGGL(bf16_head_kernel<CPL>, dim3(head_argmax_blocks(rows)), dim3(256), 0,
                     stream(), x, E, rows, K, out, scale, softcap, partials);
  G4_LAUNCH_CHECK("bf16_head_kernel");
  return G4_OK;
}

}  // namespace

size_t head_argmax_blocks(int rows) {
  const int waves = (rows + kRowsPerWave - 1) / kRowsPerWave;
  return (size_t)(waves + 3) / 4;
}

int launch_bf16_head(const float *x, const uint16_t *E, int rows, int K, float *out, float scale,
                     float softcap, float2 *partials) {
  if (rows == 0) return G4_OK;
  switch ((K / 8 + 63) / 64) {
    case 1: return launch_head<1>(x, E, rows, K, out, scale, softcap, partials);
    case 2: return launch_head<2>(x, E, rows, K, out, scale, softcap, partials);
    case 3: return launch_head<3>(x, E, rows, K, out, scale, softcap, partials);
    case 4: return launch_head<4>(x, E, rows, K, out, scale, softcap, partials);
    case 5: return launch_head<5>(x, E, rows, K, out, scale, softcap, partials);
    case 6: return launch_head<6>(x, E, rows, K, out, scale, softcap, partials);
    case 7: return launch_head<7>(x, E, rows, K, out, scale, softcap, partials);
    default: return launch_head<8>(x, E, rows, K, out, scale, softcap, partials);
  }
}

int launch_argmax_partials(const float2 *partials, int nparts, int *out_idx) {
  hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, stream(), partials, nparts,
                     out_idx);
  G4_LAUNCH_CHECK("argmax_final_kernel");
  return G4_OK;
}

size_t argmax_blocks(int n) {
  const int b = (n + 4095) / 4096;
  return (size_t)(b < 1 ? 1 : b > 1024 ? 1024 : b);
}

int launch_argmax(const float *x, int n, float2 *partials, int *out_idx) {
  const int blocks = (int)argmax_blocks(n);
  hipLaunchKernelGGL(argmax_blocks_kernel, dim3(blocks), dim3(256), 0, stream(), x, n,
                     partials);
  G4_LAUNCH_CHECK("argmax_blocks_kernel");
  return launch_argmax_partials(partials, blocks, out_idx);
}

}  // namespace g4

using namespace g4;

G4_API int g4_bf16_head(const float *x, const void *E, int rows, int in_dim, float *out,
                        float scale, float softcap) {
  G4_CHECK_INIT();
  if (rows < 0) return fail(G4_E_ARG, "g4_bf16_head: negative rows");
  if (rows == 0) return ok();
  if (in_dim <= 0 || in_dim % 8 != 0 || in_dim > 8 * 64 * 8)
    return fail(G4_E_ARG, "g4_bf16_head: in_dim %d must be a positive multiple of 8 <= 4096",
                in_dim);
  if ((reinterpret_cast<uintptr_t>(E) & 15u) != 0)
    return fail(G4_E_ARG, "g4_bf16_head: E must be 16-byte aligned");
  int rc = check_device_range(x, (size_t)in_dim * 4, "g4_bf16_head x");
  if (!rc) rc = check_device_range(E, (size_t)rows * in_dim * 2, "g4_bf16_head E");
  if (!rc) rc = check_device_range(out, (size_t)rows * 4, "g4_bf16_head out");
  if (rc) return rc;
  rc = launch_bf16_head(x, static_cast<const uint16_t *>(E), rows, in_dim, out, scale, softcap,
                        nullptr);
  return rc ? rc : ok();
}
