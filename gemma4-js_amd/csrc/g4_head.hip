// Tied BF16 LM head: the gfx950 replacement of GPUOps.headChunk and
// BF16_HEAD_SHADER (custom-webgpu/gpu-runtime.js:1265-1277, 1370-1376):
//   out[r] = softcap * tanh((scale * sum_k x[k] * E[r, k]) / softcap)
// The reference runs one thread per vocabulary row with a serial K loop and
// 64 dispatches of 4096 rows; here a wave owns a few rows at a time and the
// whole [rows, K] slab streams through with 16-byte loads.
#include "g4_internal.h"

namespace {

using namespace g4;

constexpr int kRowsPerWave = 8;

// Lane l holds x for the 8-element chunks l, l+64, ... (CPL chunks) and
// reads the same chunks of every row it visits.
template <int CPL>
__global__ __launch_bounds__(256) void bf16_head_kernel(
    const float *__restrict__ x, const uint16_t *__restrict__ E, int rows, int K,
    float *__restrict__ out, float scale, float softcap) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int row0 = wave * kRowsPerWave;
  if (row0 >= rows) return;
  const int chunks = K >> 3;

  float xv[CPL][8];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
#pragma unroll
    for (int e = 0; e < 8; ++e) xv[i][e] = c < chunks ? x[c * 8 + e] : 0.f;
  }

  uint4 w[kRowsPerWave][CPL];
#pragma unroll
  for (int r = 0; r < kRowsPerWave; ++r)
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = lane + 64 * i;
      const int row = row0 + r;
      if (row < rows && c < chunks)
        w[r][i] = ld_nt(reinterpret_cast<const uint4 *>(E + (size_t)row * K) + c);
      else
        w[r][i] = make_uint4(0, 0, 0, 0);
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
    float v = a0 + a1;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    acc[r] = v;
  }

  // Lane r finishes row r: every lane holds every sum after the butterfly.
  float mine = 0.f;
#pragma unroll
  for (int r = 0; r < kRowsPerWave; ++r)
    if (lane == r) mine = acc[r];
  const int row = row0 + lane;
  if (lane < kRowsPerWave && row < rows) {
    const float raw = mine * scale;
    out[row] = softcap > 0.f ? tanhf(raw / softcap) * softcap : raw;
  }
}

template <int CPL>
int launch_head(const float *x, const uint16_t *E, int rows, int K, float *out, float scale,
                float softcap) {
  const int waves = (rows + kRowsPerWave - 1) / kRowsPerWave;
  const int blocks = (waves + 3) / 4;
  hipLaunchKernelGGL(bf16_head_kernel<CPL>, dim3(blocks), dim3(256), 0, stream(), x, E, rows,
                     K, out, scale, softcap);
  G4_LAUNCH_CHECK("bf16_head_kernel");
  return G4_OK;
}

}  // namespace

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
  const uint16_t *e = static_cast<const uint16_t *>(E);
  const int cpl = (in_dim / 8 + 63) / 64;
  switch (cpl) {
    case 1: rc = launch_head<1>(x, e, rows, in_dim, out, scale, softcap); break;
    case 2: rc = launch_head<2>(x, e, rows, in_dim, out, scale, softcap); break;
    case 3: rc = launch_head<3>(x, e, rows, in_dim, out, scale, softcap); break;
    case 4: rc = launch_head<4>(x, e, rows, in_dim, out, scale, softcap); break;
    case 5: rc = launch_head<5>(x, e, rows, in_dim, out, scale, softcap); break;
    case 6: rc = launch_head<6>(x, e, rows, in_dim, out, scale, softcap); break;
    case 7: rc = launch_head<7>(x, e, rows, in_dim, out, scale, softcap); break;
    default: rc = launch_head<8>(x, e, rows, in_dim, out, scale, softcap); break;
  }
  return rc ? rc : ok();
}
