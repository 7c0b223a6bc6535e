// Device helpers of the bf16-pair dot-product GEMVs (g4_w4.hip, g4_fused.hip)
// and the launch planner of the one-row decode GEMV.
#pragma once

#include "g4_internal.h"

namespace g4 {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

constexpr uint32_t kPairMagic = 0x43004300u;  // bf16 pair (128, 128)
constexpr float kPairBias = 136.f;            // (128 + n) - 136 = n - 8 = q

// The bf16 pairs of one 16-byte group (4 words of 8 nibbles): pair t of word
// c is ((w_c >> 4t) & 0x000F000F) | 0x43004300, the exact bf16 values
// (128 + n_{8c+t}, 128 + n_{8c+t+4}).  The shifts by 4, 8 and 12 take two
// words at a time (v_lshrrev_b64 on words 2h and 2h + 1; the low word's top
// bits then come from its neighbour and fall outside the mask), 1.5 shifts per
// word instead of 3: the headline GEMV measured 3.00 against 3.05 us.  mask is
// 0x000F000F held in a VGPR by the caller (so v_and_or_b32 can take the magic).
__device__ __forceinline__ void group_pairs(const uint4 q, uint32_t mask, uint32_t (&p)[4][4]) {
  const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint64_t u = ((uint64_t)wd[2 * h + 1] << 32) | wd[2 * h];
    uint64_t s4, s8, s12;
    asm("v_lshrrev_b64 %0, 4, %1" : "=v"(s4) : "v"(u));
    asm("v_lshrrev_b64 %0, 8, %1" : "=v"(s8) : "v"(u));
    asm("v_lshrrev_b64 %0, 12, %1" : "=v"(s12) : "v"(u));
    const uint32_t sh[3][2] = {{(uint32_t)s4, (uint32_t)(s4 >> 32)},
                               {(uint32_t)s8, (uint32_t)(s8 >> 32)},
                               {(uint32_t)s12, (uint32_t)(s12 >> 32)}};
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      p[2 * h + e][0] = (wd[2 * h + e] & mask) | kPairMagic;
#pragma unroll
      for (int t = 1; t < 4; ++t) p[2 * h + e][t] = (sh[t - 1][e] & mask) | kPairMagic;
    }
  }
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}

// Sum over aligned teams of L lanes; every lane of the team gets the sum.
template <int L>
__device__ __forceinline__ float team_sum(float v) {
  if (L >= 2) v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  if (L >= 4) v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  if (L >= 8) v += dpp_f32<0x141>(v);  // row_half_mirror
  if (L >= 16) v += dpp_f32<0x140>(v); // row_mirror
  if (L >= 32) v += __shfl_xor(v, 16, 64);
  if (L >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

// Sum over the 64 lanes of a wave; every lane gets it (DPP within rows of 16
// lanes, then the four row sums read from lanes 0, 16, 32 and 48).
__device__ __forceinline__ float wave_sum(float v) {
  v = team_sum<16>(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ uint32_t bf16_pair(uint32_t lo16, uint32_t hi16) {
  return (lo16 & 0xffffu) | (hi16 << 16);
}

// Two FP16 values as one 32-bit word, a in the low half (the pairs of the
// prefill GEMM's x' chunks).
__device__ __forceinline__ uint32_t half2_bits(_Float16 a, _Float16 b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) |
         ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// GELU, tanh form with the clamp of GELU_MUL_SHADER (gpu-runtime.js:1148-1155).
__device__ __forceinline__ float gelu_tanh(float x) {
  const float c = 0.7978845608028654f;
  const float z = c * (x + 0.044715f * x * x * x);
  const float t = tanhf(fminf(fmaxf(z, -10.f), 10.f));
  return 0.5f * x * (1.f + t);
}

struct Gemv1Plan {
  int T, IPL, RB;
  size_t lds;
};

// Rows per block RB >= min_rb (>= 4: x staging amortised over >= 4 rows),
// RB * G = T * IPL with T a multiple of 64 up to 1024 and IPL <= 4.  A larger
// min_rb trades blocks for less re-reading of x per weight byte.
inline bool plan_gemv1(int G, bool f32x, Gemv1Plan *p, int min_rb = 4) {
  for (int RB = min_rb; RB <= 256; RB *= 2) {
    const long items = (long)RB * G;
    if (items % 64) continue;
    for (int ipl = 1; ipl <= 4; ++ipl) {
      if (items % ipl) continue;
      const long T = items / ipl;
      if (T % 64 || T > 1024) continue;
      p->T = (int)T;
      p->IPL = ipl;
      p->RB = RB;
      p->lds = (size_t)G * 4 * 16 * (f32x ? 2 : 1) + (size_t)G * 4 + (size_t)RB * G * 4;
      return p->lds <= 64 * 1024;
    }
  }
  return false;
}

}  // namespace g4
