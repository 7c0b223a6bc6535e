// Device-side synthetic data for random-init models of the checkpoint's
// shapes: a counter-based generator (SplitMix64 of seed and element index),
// so a fill is reproducible for a given seed and independent of the launch
// shape, and gigabytes of weights never cross PCIe.
//
// Distributions match the synthetic configurations of the benchmarks:
//   W4 packed words: 8 nibbles, each uniform in [1, 15] (q = nibble - 8 in
//     [-7, 7], compressed-tensors offset binary);
//   PLE packed bytes: 2 two's-complement nibbles, each q uniform in [-7, 7];
//   the _FULL kinds: every nibble uniform over all 16 values (q in [-8, 7],
//     the format's whole range: W4 nibble 0 and PLE nibble 8 are q = -8);
//   BF16 |N(0,1)| * sigma (scales) and N(0,1) * sigma (embeddings), rounded
//   to nearest even; FP32 N(0,1) * sigma.
#include <math.h>

#include "g4_internal.h"

namespace {

using namespace g4;

__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// Uniform in (0, 1] from 24 bits.
__device__ __forceinline__ float unit24(uint32_t b) {
  return ((float)(b >> 8) + 1.f) * (1.f / 16777216.f);
}

// Box-Muller, one normal per element.
__device__ __forceinline__ float normal(uint64_t r) {
  const float u1 = unit24((uint32_t)r), u2 = unit24((uint32_t)(r >> 32));
  return sqrtf(-2.f * logf(u1)) * cosf(6.283185307179586f * u2);
}

// 15 values from 4 random bits is not uniform; take 32 bits per nibble.
__device__ __forceinline__ uint32_t uniform15(uint64_t r, int i) {
  const uint32_t b = (uint32_t)(r >> (i & 1 ? 32 : 0));
  return (uint32_t)(((uint64_t)b * 15u) >> 32);  // 0..14
}

__global__ __launch_bounds__(256) void fill_kernel(void *__restrict__ dst, size_t count,
                                                   int kind, uint64_t seed, float sigma) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const uint64_t base = seed * 0xd1342543de82ef95ull;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
    switch (kind) {
      case G4_RAND_W4_PACKED: {
        uint32_t w = 0;
#pragma unroll
        for (int k = 0; k < 8; k += 2) {
          const uint64_t r = splitmix64(base + i * 4 + (k >> 1));
          w |= (uniform15(r, 0) + 1u) << (4 * k);
          w |= (uniform15(r, 1) + 1u) << (4 * (k + 1));
        }
        static_cast<uint32_t *>(dst)[i] = w;
        break;
      }
      case G4_RAND_W4_PACKED_FULL: {  // 8 uniform nibbles = 32 uniform bits
        static_cast<uint32_t *>(dst)[i] = (uint32_t)splitmix64(base + i);
        break;
      }
      case G4_RAND_PLE_PACKED_FULL: {  // 2 uniform nibbles = a uniform byte
        static_cast<uint8_t *>(dst)[i] = (uint8_t)splitmix64(base + i);
        break;
      }
      case G4_RAND_PLE_PACKED: {
        const uint64_t r = splitmix64(base + i);
        const uint32_t lo = (uniform15(r, 0) + 9u) & 15u;  // q + 16 mod 16, q in [-7, 7]
        const uint32_t hi = (uniform15(r, 1) + 9u) & 15u;
        static_cast<uint8_t *>(dst)[i] = (uint8_t)(lo | (hi << 4));
        break;
      }
      case G4_RAND_BF16_ABS_NORMAL:
      case G4_RAND_BF16_NORMAL: {
        float v = normal(splitmix64(base + i)) * sigma;
        if (kind == G4_RAND_BF16_ABS_NORMAL) v = fabsf(v);
        static_cast<uint16_t *>(dst)[i] = (uint16_t)f32_to_bf16_rne(v);
        break;
      }
      default: {  // G4_RAND_F32_NORMAL
        static_cast<float *>(dst)[i] = normal(splitmix64(base + i)) * sigma;
        break;
      }
    }
  }
}

size_t elem_bytes(int kind) {
  switch (kind) {
    case G4_RAND_W4_PACKED:
    case G4_RAND_W4_PACKED_FULL: return 4;
    case G4_RAND_PLE_PACKED:
    case G4_RAND_PLE_PACKED_FULL: return 1;
    case G4_RAND_BF16_ABS_NORMAL:
    case G4_RAND_BF16_NORMAL: return 2;
    case G4_RAND_F32_NORMAL: return 4;
    default: return 0;
  }
}

}  // namespace

G4_API int g4_fill_random(void *dst, size_t count, int kind, uint64_t seed, float sigma) {
  G4_CHECK_INIT();
  const size_t eb = elem_bytes(kind);
  if (!eb) return fail(G4_E_ARG, "g4_fill_random: unknown kind %d", kind);
  if (count == 0) return ok();
  int rc = check_device_range(dst, count * eb, "g4_fill_random dst");
  if (rc) return rc;
  size_t blocks = (count + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)blocks), dim3(256), 0, stream(), dst, count,
                     kind, seed, sigma);
  G4_LAUNCH_CHECK("fill_kernel");
  return ok();
}
