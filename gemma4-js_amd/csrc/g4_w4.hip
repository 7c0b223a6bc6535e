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
#include "g4_internal.h"
#include "g4_gemv.h"

namespace {

using namespace g4;

// ---------------------------------------------------------------------------
// Streaming GEMV (decode: rows of x <= 4 per launch).
//
// Work split: a "team" of L lanes owns one output row; lane t of the team
// handles groups t, t+L, t+2L, ... (L is the largest power of two <= 64 that
// divides G, so no lane idles).  Every lane issues the 128-bit loads of all
// its groups before anything else, so the whole weight slab is in flight
// while the block stages x.
//
// Arithmetic: v_dot2c_f32_bf16 on bf16 pairs.  A packed word w holds
// nibbles n_0..n_7 (bits 4t..4t+3).  ((w >> 4t) & 0x000F000F) | 0x43004300 is
// the bf16 pair (128 + n_t, 128 + n_{t+4}) - exact, one shift and one
// v_and_or_b32 - so the activation pairs are staged in the matching order
// (x[8c+t], x[8c+t+4]).  Per group d = sum x_i (128 + n_i) and
// sum x_i q_i = d - 136 * sum x_i; the block stages 136 * sum x per group
// once, shared by all rows.  FP32 activations are split into bf16 hi + lo
// (x = hi + lo to 2^-17 relative), two dot2 chains; BF16 activations need
// only hi.  Products are exact and accumulation is FP32.
//
// LDS image per activation row m (16-byte chunks, chunk c of group g at
// [c * G + g] so a team's lanes read consecutive chunks, conflict-free):
//   hi[4][G], lo[4][G] (FP32 input only), sx[G] = 136 * sum of the group.
// ---------------------------------------------------------------------------

// Stage group g of activation row m: 32 values -> hi/lo pair chunks + sum.
template <bool F32X>
__device__ __forceinline__ void stage_group(const void *__restrict__ xrow, int g, int G,
                                            uint4 *__restrict__ hi, uint4 *__restrict__ lo,
                                            float *__restrict__ sx) {
  uint32_t h[32], l[32];
  float sum = 0.f;
  if (F32X) {
    const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(xrow) + g * 32);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 f = p[i];
      const float v[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t hb = f32_to_bf16_rne(v[e]);
        const float r = v[e] - bf16_to_f32(hb);
        const uint32_t lb = f32_to_bf16_rne(r);
        h[4 * i + e] = hb;
        l[4 * i + e] = lb;
        sum += bf16_to_f32(hb) + bf16_to_f32(lb);
      }
    }
  } else {
    const uint4 *p = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(xrow) + g * 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 u = p[i];
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        h[8 * i + 2 * e] = w[e] & 0xffffu;
        h[8 * i + 2 * e + 1] = w[e] >> 16;
        sum += bf16_to_f32(w[e] & 0xffffu) + bf16_to_f32(w[e] >> 16);
      }
    }
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    hi[c * G + g] = make_uint4(bf16_pair(h[8 * c + 0], h[8 * c + 4]), bf16_pair(h[8 * c + 1], h[8 * c + 5]),
                               bf16_pair(h[8 * c + 2], h[8 * c + 6]), bf16_pair(h[8 * c + 3], h[8 * c + 7]));
    if (F32X)
      lo[c * G + g] = make_uint4(bf16_pair(l[8 * c + 0], l[8 * c + 4]), bf16_pair(l[8 * c + 1], l[8 * c + 5]),
                                 bf16_pair(l[8 * c + 2], l[8 * c + 6]), bf16_pair(l[8 * c + 3], l[8 * c + 7]));
  }
  sx[g] = kPairBias * sum;
}

// B: groups per lane whose loads are issued together (divides G / L).
// M: rows of x (1..4), uniform.
template <int L, int B, bool F32X>
__global__ __launch_bounds__(256) void w4_gemv_kernel(
    const void *__restrict__ x, const uint4 *__restrict__ wq, const uint16_t *__restrict__ ws,
    void *__restrict__ y, int y_bf16, int K, int N, int M) {
  extern __shared__ uint4 lds[];
  constexpr int TPW = 64 / L;
  const int G = K >> 5;
  const int GL = G / L;
  const int lane = threadIdx.x & 63;
  const int tl = lane & (L - 1);
  const int row = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * TPW + lane / L;
  // Lanes past the last row read the last row (no branch around the loads)
  // and do not store.
  const size_t rbase = (size_t)(row < N ? row : N - 1) * G + tl;

  // 1. weight loads of the first batch (HBM), all in flight together
  uint4 q[B];
  uint32_t s[B];
#pragma unroll
  for (int i = 0; i < B; ++i) {
    q[i] = ld_nt(&wq[rbase + (size_t)L * i]);
    s[i] = ld_nt_u16(&ws[rbase + (size_t)L * i]);
  }

  // 2. stage x (L2) into LDS
  constexpr int CH = F32X ? 2 : 1;
  uint4 *hi = lds;
  uint4 *lo = lds + (size_t)M * 4 * G;
  float *sx = reinterpret_cast<float *>(lds + (size_t)M * 4 * G * CH);
  for (int g = threadIdx.x; g < G; g += blockDim.x)
#pragma unroll
    for (int m = 0; m < kMaxGemvRows; ++m)
      if (m < M)
        stage_group<F32X>(F32X ? (const void *)(static_cast<const float *>(x) + (size_t)m * K)
                               : (const void *)(static_cast<const uint16_t *>(x) + (size_t)m * K),
                          g, G, hi + (size_t)m * 4 * G, lo + (size_t)m * 4 * G, sx + (size_t)m * G);
  __syncthreads();

  uint32_t mask = 0x000F000Fu;
  asm volatile("" : "+v"(mask));  // keep the mask in a VGPR: lets v_and_or_b32 take the magic

  float acc[kMaxGemvRows] = {0.f, 0.f, 0.f, 0.f};
  for (int b0 = 0; b0 < GL; b0 += B) {
    if (b0 > 0) {
#pragma unroll
      for (int i = 0; i < B; ++i) {
        q[i] = ld_nt(&wq[rbase + (size_t)L * (b0 + i)]);
        s[i] = ld_nt_u16(&ws[rbase + (size_t)L * (b0 + i)]);
      }
    }
#pragma unroll
    for (int i = 0; i < B; ++i) {
      const int g = tl + L * (b0 + i);
      uint32_t pr[4][4];
      group_pairs(q[i], mask, pr);
      uint32_t wp[16];
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int t = 0; t < 4; ++t) wp[4 * c + t] = pr[c][t];
      const float sc = bf16_to_f32(s[i]);
#pragma unroll
      for (int m = 0; m < kMaxGemvRows; ++m) {
        if (m >= M) break;
        const uint4 *hm = hi + (size_t)m * 4 * G;
        const uint4 *lm = lo + (size_t)m * 4 * G;
        float d = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint4 xp = hm[c * G + g];
          d = dot2_bf16(xp.x, wp[4 * c + 0], d);
          d = dot2_bf16(xp.y, wp[4 * c + 1], d);
          d = dot2_bf16(xp.z, wp[4 * c + 2], d);
          d = dot2_bf16(xp.w, wp[4 * c + 3], d);
          if (F32X) {
            const uint4 xl = lm[c * G + g];
            d = dot2_bf16(xl.x, wp[4 * c + 0], d);
            d = dot2_bf16(xl.y, wp[4 * c + 1], d);
            d = dot2_bf16(xl.z, wp[4 * c + 2], d);
            d = dot2_bf16(xl.w, wp[4 * c + 3], d);
          }
        }
        acc[m] = fmaf(sc, d - sx[(size_t)m * G + g], acc[m]);
      }
    }
  }

#pragma unroll
  for (int m = 0; m < kMaxGemvRows; ++m)
    if (m < M) acc[m] = team_sum<L>(acc[m]);

  if (tl == 0 && row < N) {
#pragma unroll
    for (int m = 0; m < kMaxGemvRows; ++m) {
      if (m >= M) break;
      const size_t o = (size_t)m * N + row;
      if (y_bf16)
        static_cast<uint16_t *>(y)[o] = (uint16_t)f32_to_bf16_rne(acc[m]);
      else
        static_cast<float *>(y)[o] = acc[m];
    }
  }
}

// LDS bytes the GEMV stages per activation row.
size_t gemv_lds_per_row(int K, bool f32x) {
  const size_t G = (size_t)K / 32;
  return G * 4 * 16 * (f32x ? 2 : 1) + G * 4;
}

constexpr size_t kGemvLdsBudget = 64 * 1024;

template <int L, int B, bool F32X>
int launch_gemv_lb(const g4_w4 *w, const void *x, int M, void *y, int y_bf16) {
  constexpr int TPW = 64 / L;
  const int waves = (w->N + TPW - 1) / TPW;
  const int blocks = (waves + 3) / 4;
  const size_t lds = gemv_lds_per_row(w->K, F32X) * M;
  hipLaunchKernelGGL((w4_gemv_kernel<L, B, F32X>), dim3(blocks), dim3(256), lds, stream(), x,
                     w->packed, w->scales, y, y_bf16, w->K, w->N, M);
  G4_LAUNCH_CHECK("w4_gemv_kernel");
  return G4_OK;
}

template <int L, bool F32X>
int launch_gemv_l(const g4_w4 *w, const void *x, int M, void *y, int y_bf16) {
  const int GL = w->G / L;
  if (GL % 8 == 0) return launch_gemv_lb<L, 8, F32X>(w, x, M, y, y_bf16);
  if (GL % 6 == 0) return launch_gemv_lb<L, 6, F32X>(w, x, M, y, y_bf16);
  if (GL % 4 == 0) return launch_gemv_lb<L, 4, F32X>(w, x, M, y, y_bf16);
  if (GL % 3 == 0) return launch_gemv_lb<L, 3, F32X>(w, x, M, y, y_bf16);
  if (GL % 2 == 0) return launch_gemv_lb<L, 2, F32X>(w, x, M, y, y_bf16);
  return launch_gemv_lb<L, 1, F32X>(w, x, M, y, y_bf16);
}

template <bool F32X>
int launch_gemv(const g4_w4 *w, const void *x, int M, void *y, int y_bf16) {
  if (M < 1 || M > kMaxGemvRows)
    return fail(G4_E_ARG, "GEMV takes 1..%d rows per launch, got %d", kMaxGemvRows, M);
  const int G = w->G;
  if (G % 64 == 0) return launch_gemv_l<64, F32X>(w, x, M, y, y_bf16);
  if (G % 32 == 0) return launch_gemv_l<32, F32X>(w, x, M, y, y_bf16);
  if (G % 16 == 0) return launch_gemv_l<16, F32X>(w, x, M, y, y_bf16);
  if (G % 8 == 0) return launch_gemv_l<8, F32X>(w, x, M, y, y_bf16);
  return launch_gemv_l<1, F32X>(w, x, M, y, y_bf16);
}

// Rows of x one GEMV launch takes: at most 4, and within the LDS budget.
int gemv_rows_per_launch(int K, bool f32x) {
  const size_t per = gemv_lds_per_row(K, f32x);
  int m = (int)(kGemvLdsBudget / per);
  return m < 1 ? 1 : m > kMaxGemvRows ? kMaxGemvRows : m;
}

// ---------------------------------------------------------------------------
// Decode GEMV, one row of x (the M = 1 hot path).
//
// Flat work split: the weights of RB consecutive output rows are RB * G
// 16-byte groups, contiguous in memory.  A block of T threads owns those RB
// rows and thread t takes groups t, t + T, ..., t + (IPL-1) T of that slab, so
// every load instruction of a wave reads 1 KB of consecutive bytes and every
// lane does the same work (one or a few groups: many short waves keep all
// four SIMDs of every CU busy when the data lands).  Each group's partial
// s * (d - 136 * sum x) goes to LDS and 16 lanes per row add them up.
//
// x staging: each thread first loads its 8-element chunks of x - before any
// weight load, because vmcnt retires loads in issue order and x must not wait
// behind the HBM stream - turns each chunk into the 4 pair dwords of one
// packed word and adds its 8 values into the group sum with a quad DPP
// reduction.  Needs RB >= 4, which makes chunks per thread <= IPL.
// ---------------------------------------------------------------------------
// GC, TC: the group count and block size when known at compile time (0 =
// taken from K and blockDim at run time); the E2B shapes use fixed ones.
//
// bx: the block's index among the blocks of this weight (blockIdx.x, or the
// index within its weight's blocks when one launch covers several weights).
template <int GC, int TC, int IPL, bool F32X>
__device__ __forceinline__ void gemv1_body(const void *__restrict__ x,
                                           const uint4 *__restrict__ wq,
                                           const uint16_t *__restrict__ ws, void *__restrict__ y,
                                           int y_bf16, int K, int N, int RB_, unsigned bx) {
  extern __shared__ uint4 lds[];
  const int T = TC ? TC : (int)blockDim.x;
  const int G = GC ? GC : K >> 5;
  const int RB = GC ? TC * IPL / GC : RB_;
  const int nch = 4 * G;
  const int t = threadIdx.x;

  // 1. x chunks (L2-resident), issued first
  uint4 xa[IPL], xb[IPL];
#pragma unroll
  for (int i = 0; i < IPL; ++i) {
    const int ct = t + i * T;
    const int cc = ct < nch ? ct : nch - 1;
    if (F32X) {
      xa[i] = reinterpret_cast<const uint4 *>(x)[2 * cc];
      xb[i] = reinterpret_cast<const uint4 *>(x)[2 * cc + 1];
    } else {
      xa[i] = reinterpret_cast<const uint4 *>(x)[cc];
    }
  }

  // 2. weight groups (HBM); rows past N re-read the last group and are not stored
  const size_t base = (size_t)bx * RB * G;
  const size_t last = (size_t)N * G - 1;
  uint4 q[IPL];
  uint32_t s[IPL];
#pragma unroll
  for (int i = 0; i < IPL; ++i) {
    size_t it = base + t + (size_t)i * T;
    it = it < last ? it : last;
    q[i] = ld_nt(&wq[it]);
    s[i] = ld_nt_u16(&ws[it]);
  }

  // 3. stage x into LDS: hi[4][G], lo[4][G] (FP32 x), sx[G], then partials
  constexpr int CH = F32X ? 2 : 1;
  uint4 *hi = lds;
  uint4 *lo = lds + 4 * G;
  float *sx = reinterpret_cast<float *>(lds + 4 * G * CH);
  float *part = sx + G;
#pragma unroll
  for (int i = 0; i < IPL; ++i) {
    const int ct = t + i * T;
    uint32_t h[8], l[8];
    float sum = 0.f;
    if (F32X) {
      const float v[8] = {__uint_as_float(xa[i].x), __uint_as_float(xa[i].y),
                          __uint_as_float(xa[i].z), __uint_as_float(xa[i].w),
                          __uint_as_float(xb[i].x), __uint_as_float(xb[i].y),
                          __uint_as_float(xb[i].z), __uint_as_float(xb[i].w)};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        h[e] = f32_to_bf16_rne(v[e]);
        l[e] = f32_to_bf16_rne(v[e] - bf16_to_f32(h[e]));
        sum += bf16_to_f32(h[e]) + bf16_to_f32(l[e]);
      }
    } else {
      const uint32_t w[4] = {xa[i].x, xa[i].y, xa[i].z, xa[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        h[2 * e] = w[e] & 0xffffu;
        h[2 * e + 1] = w[e] >> 16;
        sum += bf16_to_f32(h[2 * e]) + bf16_to_f32(h[2 * e + 1]);
      }
    }
    // chunks 4g..4g+3 of a group sit in one lane quad
    sum += dpp_f32<0xB1>(sum);
    sum += dpp_f32<0x4E>(sum);
    if (ct < nch) {
      const int g = ct >> 2, c = ct & 3;
      hi[c * G + g] = make_uint4(bf16_pair(h[0], h[4]), bf16_pair(h[1], h[5]),
                                 bf16_pair(h[2], h[6]), bf16_pair(h[3], h[7]));
      if (F32X)
        lo[c * G + g] = make_uint4(bf16_pair(l[0], l[4]), bf16_pair(l[1], l[5]),
                                   bf16_pair(l[2], l[6]), bf16_pair(l[3], l[7]));
      if (c == 0) sx[g] = kPairBias * sum;
    }
  }
  __syncthreads();

  // 4. one partial per group
  uint32_t mask = 0x000F000Fu;
  asm volatile("" : "+v"(mask));  // keep the mask in a VGPR: lets v_and_or_b32 take the magic
#pragma unroll
  for (int i = 0; i < IPL; ++i) {
    const int li = t + i * T;
    const int g = li % G;
    uint32_t pr[4][4];
    group_pairs(q[i], mask, pr);
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t p0 = pr[c][0], p1 = pr[c][1], p2 = pr[c][2], p3 = pr[c][3];
      const uint4 xp = hi[c * G + g];
      d0 = dot2_bf16(xp.x, p0, d0);
      d1 = dot2_bf16(xp.y, p1, d1);
      d0 = dot2_bf16(xp.z, p2, d0);
      d1 = dot2_bf16(xp.w, p3, d1);
      if (F32X) {
        const uint4 xl = lo[c * G + g];
        d0 = dot2_bf16(xl.x, p0, d0);
        d1 = dot2_bf16(xl.y, p1, d1);
        d0 = dot2_bf16(xl.z, p2, d0);
        d1 = dot2_bf16(xl.w, p3, d1);
      }
    }
    part[li] = bf16_to_f32(s[i]) * ((d0 + d1) - sx[g]);
  }
  __syncthreads();

  // 5. 16 lanes per row sum the row's G partials
  for (int b = 0; b < RB * 16; b += T) {
    const int idx = b + t;
    const int r = idx >> 4, j = idx & 15;
    float v = 0.f;
    if (r < RB) {
      if (GC) {
#pragma unroll
        for (int g = j; g < GC; g += 16) v += part[r * GC + g];
      } else {
        for (int g = j; g < G; g += 16) v += part[r * G + g];
      }
    }
    v = team_sum<16>(v);
    const size_t row = (size_t)bx * RB + r;
    if (j == 0 && r < RB && row < (size_t)N) {
      if (y_bf16)
        static_cast<uint16_t *>(y)[row] = (uint16_t)f32_to_bf16_rne(v);
      else
        static_cast<float *>(y)[row] = v;
    }
  }
}

template <int GC, int TC, int IPL, bool F32X>
__global__ __launch_bounds__(TC ? TC : 1024) void w4_gemv1_kernel(
    const void *__restrict__ x, const uint4 *__restrict__ wq, const uint16_t *__restrict__ ws,
    void *__restrict__ y, int y_bf16, int K, int N, int RB_) {
  gemv1_body<GC, TC, IPL, F32X>(x, wq, ws, y, y_bf16, K, N, RB_, blockIdx.x);
}

// Up to kMaxLinearSegs weights of one input dimension over the same x in one
// launch: the blocks of weight i are block0[i] .. block0[i + 1] - 1, each
// running the single-weight body on its own rows.
constexpr int kMaxLinearSegs = 3;
struct Gemv1Segs {
  const uint4 *wq[kMaxLinearSegs];
  const uint16_t *ws[kMaxLinearSegs];
  void *y[kMaxLinearSegs];
  int N[kMaxLinearSegs];
  int block0[kMaxLinearSegs];
  int n;
};

template <int GC, int TC, int IPL, bool F32X>
__global__ __launch_bounds__(TC ? TC : 1024) void w4_gemv1_multi_kernel(
    const void *__restrict__ x, Gemv1Segs S, int y_bf16, int K, int RB_) {
  const int b = blockIdx.x;
  const int i = S.n > 2 && b >= S.block0[2] ? 2 : S.n > 1 && b >= S.block0[1] ? 1 : 0;
  gemv1_body<GC, TC, IPL, F32X>(x, S.wq[i], S.ws[i], S.y[i], y_bf16, K, S.N[i], RB_,
                                (unsigned)(b - S.block0[i]));
}

// ---------------------------------------------------------------------------
// Decode GEMV, one row of x, for in_dim 1536 and 2048 (J = 3 or 4 groups of
// 16 per row): the row split.
//
// 16 lanes per output row (LPR); lane c of a row takes groups c, c + 16, ...,
// c + 16 (J - 1), so a block of W waves owns 4 W rows, and at instruction j
// the 16 lanes of a row read 256 consecutive bytes of it.  In_dim 6144 and
// 12288 take LPR = 64 (one row per wave, lane c taking groups c, c + 64, ...,
// J = 3 or 6): the same work per lane, a wave-wide row sum, and none of the
// flat split's LDS partials and second barrier.  x is staged in LDS
// as in the flat split, then every lane reads its J groups' pairs and group
// sums into registers right after the staging barrier, before its first
// weight use.  The row sum is a 16-lane DPP reduction: once the weights land,
// nothing goes back through LDS and no barrier sits between the last load and
// the store.  The arithmetic and its order are the flat split's (each group
// partial rounded, then added c, c + 16, ... before the 16-lane sum), so the
// two give bit-identical outputs.
//
// gstride: row length in memory, in groups (J * 16, or the full width when a
// split launch reads one slice of longer rows).  bx: the block's index among
// the blocks of this weight.
// ---------------------------------------------------------------------------
//
// STAMP (the clock-stamp diagnostic, g4_w4_gemv_stamps): lane 0 of every wave
// writes 5 real-time clock values (100 MHz) to stamps[wave][0..4]: the wave's
// start, x staged, the staging barrier passed, every weight load landed (a
// full wait inserted there, so group j's arithmetic no longer overlaps the
// later groups' loads), and the store issued.
template <int J, int W, bool F32X, bool STAMP = false, int LPR = 16>
__device__ __forceinline__ void gemv_r16_body(const void *__restrict__ x,
                                              const uint4 *__restrict__ wq,
                                              const uint16_t *__restrict__ ws,
                                              void *__restrict__ y, int y_bf16, int N,
                                              int gstride, unsigned bx,
                                              uint64_t *__restrict__ stamps = nullptr) {
  uint64_t st[5];
  if (STAMP) st[0] = __builtin_amdgcn_s_memrealtime();
  constexpr int G = LPR * J, T = 64 * W, nch = 4 * G;
  constexpr int RPW = 64 / LPR;  // rows per wave
  constexpr int XI = (nch + T - 1) / T;  // x chunks per thread
  constexpr int JL = F32X ? J : 1;
  __shared__ uint4 hi[4 * G];
  __shared__ uint4 lo[F32X ? 4 * G : 1];
  __shared__ float sx[G];
  const int t = threadIdx.x;
  const int c16 = t & (LPR - 1);  // the lane's place in its row's team
  const int row = (int)bx * (RPW * W) + t / LPR;
  const int rr = row < N ? row : N - 1;  // rows past N re-read the last row, store nothing
  const uint4 *x4 = static_cast<const uint4 *>(x);

  // 1. x chunks (L2-resident), issued before the weights
  uint4 xa[XI], xb[XI];
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int ct = t + i * T;
    const int cc = ct < nch ? ct : nch - 1;
    if (F32X) {
      xa[i] = x4[2 * cc];
      xb[i] = x4[2 * cc + 1];
    } else {
      xa[i] = x4[cc];
    }
  }

  // 2. the lane's J weight groups (HBM)
  uint4 q[J];
  uint32_t s[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const size_t it = (size_t)rr * gstride + c16 + LPR * j;
    q[j] = ld_nt(&wq[it]);
    s[j] = ld_nt_u16(&ws[it]);
  }

  // 3. stage x: bf16 pairs of each chunk (hi, and lo for FP32 x), 136 * group sum
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int ct = t + i * T;
    uint32_t h[8], l[8];
    float sum = 0.f;
    if (F32X) {
      const float v[8] = {__uint_as_float(xa[i].x), __uint_as_float(xa[i].y),
                          __uint_as_float(xa[i].z), __uint_as_float(xa[i].w),
                          __uint_as_float(xb[i].x), __uint_as_float(xb[i].y),
                          __uint_as_float(xb[i].z), __uint_as_float(xb[i].w)};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        h[e] = f32_to_bf16_rne(v[e]);
        l[e] = f32_to_bf16_rne(v[e] - bf16_to_f32(h[e]));
        sum += bf16_to_f32(h[e]) + bf16_to_f32(l[e]);
      }
    } else {
      const uint32_t w[4] = {xa[i].x, xa[i].y, xa[i].z, xa[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        h[2 * e] = w[e] & 0xffffu;
        h[2 * e + 1] = w[e] >> 16;
        sum += bf16_to_f32(h[2 * e]) + bf16_to_f32(h[2 * e + 1]);
      }
    }
    sum += dpp_f32<0xB1>(sum);  // chunks 4g..4g+3 of a group sit in one lane quad
    sum += dpp_f32<0x4E>(sum);
    if (ct < nch) {
      const int g = ct >> 2, c = ct & 3;
      hi[c * G + g] = make_uint4(bf16_pair(h[0], h[4]), bf16_pair(h[1], h[5]),
                                 bf16_pair(h[2], h[6]), bf16_pair(h[3], h[7]));
      if (F32X)
        lo[c * G + g] = make_uint4(bf16_pair(l[0], l[4]), bf16_pair(l[1], l[5]),
                                   bf16_pair(l[2], l[6]), bf16_pair(l[3], l[7]));
      if (c == 0) sx[g] = kPairBias * sum;
    }
  }
  // keep the weight arithmetic below the barrier: otherwise the compiler may
  // hoist the first group's unpacking above it, and the barrier waits for HBM
  __builtin_amdgcn_sched_barrier(0);
  if (STAMP) st[1] = __builtin_amdgcn_s_memrealtime();
  __syncthreads();
  if (STAMP) st[2] = __builtin_amdgcn_s_memrealtime();

  // 4. the lane's x groups into registers, all reads issued before any weight use
  uint4 xh[J][4], xl[JL][4];
  float sxr[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int g = c16 + LPR * j;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      xh[j][c] = hi[c * G + g];
      if (F32X) xl[j < JL ? j : 0][c] = lo[c * G + g];
    }
    sxr[j] = sx[g];
  }
  __builtin_amdgcn_sched_barrier(0);
  if (STAMP) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    st[3] = __builtin_amdgcn_s_memrealtime();
    __builtin_amdgcn_sched_barrier(0);
  }

  // 5. group partials, the row sum over 16 lanes, the store
  uint32_t mask = 0x000F000Fu;
  asm volatile("" : "+v"(mask));  // keep the mask in a VGPR: lets v_and_or_b32 take the magic
  float v = 0.f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    uint32_t pr[4][4];
    group_pairs(q[j], mask, pr);
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t p0 = pr[c][0], p1 = pr[c][1], p2 = pr[c][2], p3 = pr[c][3];
      const uint4 xp = xh[j][c];
      d0 = dot2_bf16(xp.x, p0, d0);
      d1 = dot2_bf16(xp.y, p1, d1);
      d0 = dot2_bf16(xp.z, p2, d0);
      d1 = dot2_bf16(xp.w, p3, d1);
      if (F32X) {
        const uint4 xq = xl[j < JL ? j : 0][c];
        d0 = dot2_bf16(xq.x, p0, d0);
        d1 = dot2_bf16(xq.y, p1, d1);
        d0 = dot2_bf16(xq.z, p2, d0);
        d1 = dot2_bf16(xq.w, p3, d1);
      }
    }
    float pj = bf16_to_f32(s[j]) * ((d0 + d1) - sxr[j]);
    asm volatile("" : "+v"(pj));  // rounded on its own (no FMA into the row sum)
    v += pj;
  }
  v = team_sum<LPR>(v);
  if (c16 == 0 && row < N) {
    if (y_bf16)
      static_cast<uint16_t *>(y)[row] = (uint16_t)f32_to_bf16_rne(v);
    else  // written through to memory (sc0 sc1): 3.06 against 3.09 us at N 6144
      __hip_atomic_store(static_cast<float *>(y) + row, v, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_SYSTEM);
  }
  if (STAMP) {
    st[4] = __builtin_amdgcn_s_memrealtime();
    if ((t & 63) == 0) {
      uint64_t *o = stamps + ((size_t)bx * W + (t >> 6)) * 5;
#pragma unroll
      for (int k = 0; k < 5; ++k) o[k] = st[k];
    }
  }
}

// The row split with clock stamps (BF16 or FP32 x, one weight); stamps:
// [blocks * W waves][5].
template <int J, int W, bool F32X>
__global__ __launch_bounds__(64 * W) void w4_gemv_r16_stamp_kernel(
    const void *__restrict__ x, const uint4 *__restrict__ wq, const uint16_t *__restrict__ ws,
    void *__restrict__ y, int y_bf16, int N, uint64_t *__restrict__ stamps) {
  gemv_r16_body<J, W, F32X, true>(x, wq, ws, y, y_bf16, N, 16 * J, blockIdx.x, stamps);
}

// SPLIT: slice blockIdx.y of the input dimension (16 J groups of rows
// gstride groups long), x from slice * 512 J, FP32 partial sums to
// y + slice * N.
template <int J, int W, bool F32X, bool SPLIT>
__global__ __launch_bounds__(64 * W) void w4_gemv_r16_kernel(
    const void *__restrict__ x, const uint4 *__restrict__ wq, const uint16_t *__restrict__ ws,
    void *__restrict__ y, int y_bf16, int N, int gstride) {
  if (SPLIT) {
    const int slice = blockIdx.y;
    x = static_cast<const char *>(x) + (size_t)slice * 512 * J * (F32X ? 4 : 2);
    wq += (size_t)slice * 16 * J;
    ws += (size_t)slice * 16 * J;
    y = static_cast<float *>(y) + (size_t)slice * N;
  }
  gemv_r16_body<J, W, F32X>(x, wq, ws, y, y_bf16, N, gstride, blockIdx.x);
}

template <int J, int W, bool F32X>
__global__ __launch_bounds__(64 * W) void w4_gemv_r16_multi_kernel(const void *__restrict__ x,
                                                                   Gemv1Segs S, int y_bf16) {
  const int b = blockIdx.x;
  const int i = S.n > 2 && b >= S.block0[2] ? 2 : S.n > 1 && b >= S.block0[1] ? 1 : 0;
  gemv_r16_body<J, W, F32X>(x, S.wq[i], S.ws[i], S.y[i], y_bf16, S.N[i], 16 * J,
                            (unsigned)(b - S.block0[i]));
}

// LPR = 64: W rows per block of W waves.
template <int J, int W, bool F32X>
__global__ __launch_bounds__(64 * W) void w4_gemv_r64_kernel(
    const void *__restrict__ x, const uint4 *__restrict__ wq, const uint16_t *__restrict__ ws,
    void *__restrict__ y, int y_bf16, int N) {
  gemv_r16_body<J, W, F32X, false, 64>(x, wq, ws, y, y_bf16, N, 64 * J, blockIdx.x);
}

template <int J, int W, bool F32X>
__global__ __launch_bounds__(64 * W) void w4_gemv_r64_multi_kernel(const void *__restrict__ x,
                                                                   Gemv1Segs S, int y_bf16) {
  const int b = blockIdx.x;
  const int i = S.n > 2 && b >= S.block0[2] ? 2 : S.n > 1 && b >= S.block0[1] ? 1 : 0;
  gemv_r16_body<J, W, F32X, false, 64>(x, S.wq[i], S.ws[i], S.y[i], y_bf16, S.N[i], 64 * J,
                                       (unsigned)(b - S.block0[i]));
}

// Waves per block of the row split: 4 (16 rows) from 4096 rows on, else 2
// (measured at in_dim 1536, cold weights: N 6144 3.09 us with 4 waves against
// 3.34 with 2; N 2048 2.46 us with 2 against 2.49 with 4).
inline int r16_waves(int rows) { return rows >= 4096 ? 4 : 2; }

inline bool has_r16(int G) { return G == 48 || G == 64; }

// The 64-lane row split: in_dim 4096 and 6144, and 12288 with BF16 x (FP32 x
// there would hold 192 registers of x pairs per lane).  8 rows (waves) per block:
// every block stages the whole x row (12 or 24 KB), so fewer, larger blocks
// re-read less of it.  Measured, one row of BF16 x, N 1536, cold weights:
// K 6144 3.40 us with 8 waves, 3.64 with 4, 3.89 with 2, 4.01 with 16 (the
// flat split: 3.56); K 12288 4.51 us with 8 waves, 4.87 with 4 (flat: 5.47);
// K 4096 2.71 us (flat: 2.85), with FP32 x 2.85 us (flat: 3.28).
inline bool has_r64(int G, bool f32x) { return G == 128 || G == 192 || (G == 384 && !f32x); }
constexpr int kR64Waves = 8;

template <int J, bool F32X>
int launch_r64_i(const g4_w4 *w, const void *x, void *y, int y_bf16) {
  constexpr int W = kR64Waves;
  hipLaunchKernelGGL((w4_gemv_r64_kernel<J, W, F32X>), dim3((w->N + W - 1) / W), dim3(64 * W), 0,
                     stream(), x, w->packed, w->scales, y, y_bf16, w->N);
  G4_LAUNCH_CHECK("w4_gemv_r64_kernel");
  return G4_OK;
}

template <bool F32X>
int launch_r64(const g4_w4 *w, const void *x, void *y, int y_bf16) {
  if (w->G == 128) return launch_r64_i<2, F32X>(w, x, y, y_bf16);
  if (w->G == 192) return launch_r64_i<3, F32X>(w, x, y, y_bf16);
  return launch_r64_i<6, false>(w, x, y, y_bf16);
}

template <int J, bool F32X>
int launch_r64_multi_i(const g4_w4 *const *w, int n, const void *x, void *const *y, int y_bf16) {
  constexpr int W = kR64Waves;
  Gemv1Segs S{};
  int blocks = 0;
  for (int i = 0; i < n; ++i) {
    S.wq[i] = w[i]->packed;
    S.ws[i] = w[i]->scales;
    S.y[i] = y[i];
    S.N[i] = w[i]->N;
    S.block0[i] = blocks;
    blocks += (w[i]->N + W - 1) / W;
  }
  S.n = n;
  hipLaunchKernelGGL((w4_gemv_r64_multi_kernel<J, W, F32X>), dim3(blocks), dim3(64 * W), 0,
                     stream(), x, S, y_bf16);
  G4_LAUNCH_CHECK("w4_gemv_r64_multi_kernel");
  return G4_OK;
}

template <bool F32X>
int launch_r64_multi(const g4_w4 *const *w, int n, const void *x, void *const *y, int y_bf16) {
  if (w[0]->G == 128) return launch_r64_multi_i<2, F32X>(w, n, x, y, y_bf16);
  if (w[0]->G == 192) return launch_r64_multi_i<3, F32X>(w, n, x, y, y_bf16);
  return launch_r64_multi_i<6, false>(w, n, x, y, y_bf16);
}

template <int J, int W, bool F32X>
int launch_r16_i(const g4_w4 *w, const void *x, void *y, int y_bf16) {
  hipLaunchKernelGGL((w4_gemv_r16_kernel<J, W, F32X, false>),
                     dim3((w->N + 4 * W - 1) / (4 * W)), dim3(64 * W), 0, stream(), x, w->packed,
                     w->scales, y, y_bf16, w->N, w->G);
  G4_LAUNCH_CHECK("w4_gemv_r16_kernel");
  return G4_OK;
}

template <bool F32X>
int launch_r16(const g4_w4 *w, const void *x, void *y, int y_bf16) {
  const bool w4 = r16_waves(w->N) == 4;
  if (w->G == 48)
    return w4 ? launch_r16_i<3, 4, F32X>(w, x, y, y_bf16) : launch_r16_i<3, 2, F32X>(w, x, y, y_bf16);
  return w4 ? launch_r16_i<4, 4, F32X>(w, x, y, y_bf16) : launch_r16_i<4, 2, F32X>(w, x, y, y_bf16);
}

template <int J, int W, bool F32X>
int launch_r16_multi_i(const g4_w4 *const *w, int n, const void *x, void *const *y,
                       int y_bf16) {
  Gemv1Segs S{};
  int blocks = 0;
  for (int i = 0; i < n; ++i) {
    S.wq[i] = w[i]->packed;
    S.ws[i] = w[i]->scales;
    S.y[i] = y[i];
    S.N[i] = w[i]->N;
    S.block0[i] = blocks;
    blocks += (w[i]->N + 4 * W - 1) / (4 * W);
  }
  S.n = n;
  hipLaunchKernelGGL((w4_gemv_r16_multi_kernel<J, W, F32X>), dim3(blocks), dim3(64 * W), 0,
                     stream(), x, S, y_bf16);
  G4_LAUNCH_CHECK("w4_gemv_r16_multi_kernel");
  return G4_OK;
}

template <bool F32X>
int launch_r16_multi(const g4_w4 *const *w, int n, const void *x, void *const *y, int y_bf16) {
  int rows = 0;
  for (int i = 0; i < n; ++i) rows += w[i]->N;
  const bool w4 = r16_waves(rows) == 4;
  if (w[0]->G == 48)
    return w4 ? launch_r16_multi_i<3, 4, F32X>(w, n, x, y, y_bf16)
              : launch_r16_multi_i<3, 2, F32X>(w, n, x, y, y_bf16);
  return w4 ? launch_r16_multi_i<4, 4, F32X>(w, n, x, y, y_bf16)
            : launch_r16_multi_i<4, 2, F32X>(w, n, x, y, y_bf16);
}

template <int GC, int TC, int IPL, bool F32X>
int launch_gemv1_i(const g4_w4 *w, const Gemv1Plan &p, const void *x, void *y, int y_bf16) {
  const int blocks = (w->N + p.RB - 1) / p.RB;
  hipLaunchKernelGGL((w4_gemv1_kernel<GC, TC, IPL, F32X>), dim3(blocks), dim3(p.T), p.lds,
                     stream(), x, w->packed, w->scales, y, y_bf16, w->K, w->N, p.RB);
  G4_LAUNCH_CHECK("w4_gemv1_kernel");
  return G4_OK;
}

// Whether the one-row GEMV has a launch shape for G groups per row (RB * G =
// T * IPL needs a block size of whole waves); other widths take the general
// GEMV with one row.
bool has_gemv1_plan(int G, bool f32x) {
  Gemv1Plan p;
  return plan_gemv1(G, f32x, &p);
}

// The M = 1 launch shape for w's input dimension.
template <bool F32X>
int gemv1_plan(const g4_w4 *w, Gemv1Plan *p) {
  // FP32 x of a long row is 4 K bytes per block against 4 rows * K / 2 bytes of
  // weights: from K = 4096 on, 8 rows per block halve that re-read.
  const int min_rb = F32X && w->K >= 4096 ? 8 : 4;
  if (!plan_gemv1(w->G, F32X, p, min_rb) && !plan_gemv1(w->G, F32X, p))
    return fail(G4_E_ARG, "g4_w4_linear: no decode GEMV plan for in_dim %d", w->K);
  return G4_OK;
}

template <bool F32X>
int launch_gemv1(const g4_w4 *w, const void *x, void *y, int y_bf16) {
  if (has_r16(w->G)) return launch_r16<F32X>(w, x, y, y_bf16);
  if (has_r64(w->G, F32X)) return launch_r64<F32X>(w, x, y, y_bf16);
  Gemv1Plan p;
  if (int rc = gemv1_plan<F32X>(w, &p)) return rc;
  // compile-time variants for the plans of the Gemma-4-E2B projections
#define G4_GEMV1_FIXED(GG, TT, II)                                      \
  if (w->G == GG && p.T == TT && p.IPL == II)                           \
    return launch_gemv1_i<GG, TT, II, F32X>(w, p, x, y, y_bf16);
  G4_GEMV1_FIXED(128, 512, 1)   // K = 4096
  G4_GEMV1_FIXED(192, 768, 1)   // K = 6144
  G4_GEMV1_FIXED(384, 768, 2)   // K = 12288
  G4_GEMV1_FIXED(8, 64, 1)      // K = 256
  G4_GEMV1_FIXED(128, 1024, 1)  // K = 4096, FP32 x: 8 rows
  G4_GEMV1_FIXED(192, 768, 2)   // K = 6144, FP32 x: 8 rows
  G4_GEMV1_FIXED(384, 1024, 3)  // K = 12288, FP32 x: 8 rows
#undef G4_GEMV1_FIXED
  switch (p.IPL) {
    case 1: return launch_gemv1_i<0, 0, 1, F32X>(w, p, x, y, y_bf16);
    case 2: return launch_gemv1_i<0, 0, 2, F32X>(w, p, x, y, y_bf16);
    case 3: return launch_gemv1_i<0, 0, 3, F32X>(w, p, x, y, y_bf16);
    default: return launch_gemv1_i<0, 0, 4, F32X>(w, p, x, y, y_bf16);
  }
}

template <int GC, int TC, int IPL, bool F32X>
int launch_gemv1_multi_i(const g4_w4 *const *w, int n, const Gemv1Plan &p, const void *x,
                         void *const *y, int y_bf16) {
  Gemv1Segs S{};
  int blocks = 0;
  for (int i = 0; i < n; ++i) {
    S.wq[i] = w[i]->packed;
    S.ws[i] = w[i]->scales;
    S.y[i] = y[i];
    S.N[i] = w[i]->N;
    S.block0[i] = blocks;
    blocks += (w[i]->N + p.RB - 1) / p.RB;
  }
  S.n = n;
  hipLaunchKernelGGL((w4_gemv1_multi_kernel<GC, TC, IPL, F32X>), dim3(blocks), dim3(p.T), p.lds,
                     stream(), x, S, y_bf16, w[0]->K, p.RB);
  G4_LAUNCH_CHECK("w4_gemv1_multi_kernel");
  return G4_OK;
}

// n (2..kMaxLinearSegs) weights of one input dimension over one x row.
template <bool F32X>
int launch_gemv1_multi(const g4_w4 *const *w, int n, const void *x, void *const *y,
                       int y_bf16) {
  if (has_r16(w[0]->G)) return launch_r16_multi<F32X>(w, n, x, y, y_bf16);
  if (has_r64(w[0]->G, F32X)) return launch_r64_multi<F32X>(w, n, x, y, y_bf16);
  Gemv1Plan p;
  if (int rc = gemv1_plan<F32X>(w[0], &p)) return rc;
  switch (p.IPL) {
    case 1: return launch_gemv1_multi_i<0, 0, 1, F32X>(w, n, p, x, y, y_bf16);
    case 2: return launch_gemv1_multi_i<0, 0, 2, F32X>(w, n, p, x, y, y_bf16);
    case 3: return launch_gemv1_multi_i<0, 0, 3, F32X>(w, n, p, x, y, y_bf16);
    default: return launch_gemv1_multi_i<0, 0, 4, F32X>(w, n, p, x, y, y_bf16);
  }
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

namespace g4 {

// Split-K decode GEMV for one FP32 row: parts[s][n] = sum over inputs
// [1536 s, 1536 s + 1536) of x[k] * W[n, k], each slice on the in_dim 1536
// row split with 16 rows per block (E2B decode step, down 1536 x 6144:
// 1.243 ms/token against 1.259 with 8 rows and 1.267 with 4).  A long input
// row then needs neither the whole row staged per block nor fewer blocks than
// CUs; the consumer adds the slices in order.
// Returns the slice count, 0 when K is not a multiple of 1536 of at least two
// slices (nothing launched), or a negative status.
int launch_gemv1_split(const g4_w4 *w, const float *x, float *parts) {
  constexpr int kSliceK = 1536, W = 4;
  if (w->K % kSliceK || w->K / kSliceK < 2) return 0;
  const int slices = w->K / kSliceK;
  hipLaunchKernelGGL((w4_gemv_r16_kernel<kSliceK / 512, W, true, true>),
                     dim3((w->N + 4 * W - 1) / (4 * W), slices), dim3(64 * W), 0, stream(), x,
                     w->packed, w->scales, parts, 0, w->N, w->G);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return -fail(G4_E_HIP, "w4_gemv_r16_kernel (split): %s", hipGetErrorString(e));
  return slices;
}

}  // namespace g4

namespace {

// Per output row, the power-of-two shift of the FP16 path of the prefill
// GEMM: with 2^shift[o] * 8 * max_g |s[o, g]| <= 2^15 every q * s * 2^shift[o]
// of the row (<= 11 significant bits) is an exact FP16 value, unless the
// group's scale is more than 2^26 below the row's largest (then its products
// may lose bits, each at most 2^-26 of the row's largest product).  Rows are
// independent, so their magnitudes may differ by any factor.  Rows whose
// scales are all zero (or not finite) have no constraint: they get kNoShift
// here and the tensor shift once the range is known (row_shift_range_kernel),
// so a pruned or padding row neither lowers the tensor shift nor forces the
// per-row path.
constexpr int16_t kNoShift = -32768;

__global__ __launch_bounds__(256) void row_shift_kernel(const uint16_t *__restrict__ s, int N,
                                                        int G, int16_t *__restrict__ shift) {
  const int o = blockIdx.x * 256 + threadIdx.x;
  if (o >= N) return;
  const uint16_t *row = s + (size_t)o * G;
  uint32_t mx = 0;
  for (int g = 0; g < G; ++g) {
    const uint32_t a = row[g] & 0x7fffu;
    if (a < 0x7f80u && a > mx) mx = a;  // finite magnitudes only
  }
  // floor(log2 max|s|) for a normal bf16; -127 for a subnormal one (its
  // true exponent is lower, so the shift only keeps it further from overflow)
  shift[o] = mx ? (int16_t)(11 - ((int)(mx >> 7) - 127)) : kNoShift;
}

constexpr int kRowShiftSpread = 12;

// One allocation per weight: packed groups, the scales, the row shifts and
// (even G) the stage-major tile copy of the words and scales for the GEMM.
int alloc_weight(g4_w4 *w, size_t qbytes, size_t sbytes, bool want_tiles) {
  const size_t soff = (qbytes + 255) & ~size_t(255);
  const size_t roff = (soff + sbytes + 255) & ~size_t(255);
  size_t total = roff + (((size_t)w->N * sizeof(int16_t) + 15) & ~size_t(15));
  const bool tiles = want_tiles && w->G % 2 == 0;
  const size_t Np = ((size_t)w->N + 15) / 16 * 16;
  const size_t toff = (total + 255) & ~size_t(255);
  if (tiles) total = toff + Np * w->G * 18;  // per row and stage: 32 B of words, 4 of scales
  // + 8 bytes past `bytes` for the row-shift range read back at load
  int rc = device_alloc(total + 8, reinterpret_cast<void **>(&w->mem));
  if (rc) return rc;
  w->packed = reinterpret_cast<uint4 *>(w->mem);
  w->scales = reinterpret_cast<uint16_t *>(w->mem + soff);
  w->rshift = reinterpret_cast<int16_t *>(w->mem + roff);
  w->tiles = tiles ? reinterpret_cast<uint4 *>(w->mem + toff) : nullptr;
  w->bytes = total;
  return G4_OK;
}

// The stage-major tile copy (g4_w4::tiles) from the row-major arrays: one
// thread per 16-byte unit.
__global__ __launch_bounds__(256) void tile_weight_kernel(const uint4 *__restrict__ packed,
                                                          const uint32_t *__restrict__ spairs,
                                                          int N, int G, uint4 *__restrict__ tw) {
  const int S2 = G / 2;
  const size_t T = ((size_t)N + 15) / 16;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)S2 * T * 36) return;
  const size_t blk = i / 36;  // st * T + t
  const int e = (int)(i - blk * 36);
  const int st = (int)(blk / T);
  const size_t t = blk - (size_t)st * T;
  auto row = [&](int r) {
    const size_t o = t * 16 + r;
    return o < (size_t)N ? o : (size_t)N - 1;
  };
  if (e < 32) {
    // unit e: the 8-byte word pairs (2 q, 2 q + 1) of rows c and c + 1, q = e / 8,
    // c = 2 (e % 8); both pairs come from group 2 st + q / 2
    const int q = e >> 3, c = 2 * (e & 7);
    const uint4 a = packed[row(c) * G + 2 * st + (q >> 1)];
    const uint4 b = packed[row(c + 1) * G + 2 * st + (q >> 1)];
    tw[i] = (q & 1) ? make_uint4(a.z, a.w, b.z, b.w) : make_uint4(a.x, a.y, b.x, b.y);
  } else {
    const int r0 = 4 * (e - 32);
    tw[i] = make_uint4(spairs[row(r0) * S2 + st], spairs[row(r0 + 1) * S2 + st],
                       spairs[row(r0 + 2) * S2 + st], spairs[row(r0 + 3) * S2 + st]);
  }
}

// Smallest and largest row shift over the rows that have one, one block
// (a uint32 pair, the shifts biased by 512 so they compare unsigned); then
// every kNoShift row takes the smallest (the tensor shift; 0 if no row has
// a non-zero scale).
__global__ __launch_bounds__(256) void row_shift_range_kernel(int16_t *__restrict__ shift,
                                                              int N, uint32_t *__restrict__ out) {
  uint32_t lo = 0xffffffffu, hi = 0u;
  for (int o = threadIdx.x; o < N; o += 256) {
    if (shift[o] == kNoShift) continue;
    const uint32_t v = (uint32_t)(shift[o] + 512);
    lo = v < lo ? v : lo;
    hi = v > hi ? v : hi;
  }
  __shared__ uint32_t slo[256], shi[256];
  slo[threadIdx.x] = lo;
  shi[threadIdx.x] = hi;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < 256; ++i) {
      lo = slo[i] < lo ? slo[i] : lo;
      hi = shi[i] > hi ? shi[i] : hi;
    }
    if (hi < lo) lo = hi = 512u;  // no row with a scale: shift 0
    slo[0] = lo;
    out[0] = lo;
    out[1] = hi;
  }
  __syncthreads();
  const int16_t fill = (int16_t)((int)slo[0] - 512);
  for (int o = threadIdx.x; o < N; o += 256)
    if (shift[o] == kNoShift) shift[o] = fill;
}

// The stage-major tile copy (even G), the row shifts into w->rshift, then the
// tensor shift (the smallest row shift, that of the row with the largest
// scale) and whether rows need their own:
// with one shift, a row whose largest scale is 2^d below the tensor's keeps
// 26 - d bits of headroom below its largest product before FP16 products
// lose bits; up to d = 12 that is far below what the 1e-3 contract can see,
// beyond it the GEMM rescales per row (a few percent slower).  Synchronises.
hipError_t finish_row_shift(g4_w4 *w) {
  if (w->tiles) {
    const size_t nu = (size_t)(w->G / 2) * ((w->N + 15) / 16) * 36;
    hipLaunchKernelGGL(tile_weight_kernel, dim3((unsigned)((nu + 255) / 256)), dim3(256), 0,
                       stream(), w->packed, reinterpret_cast<const uint32_t *>(w->scales), w->N,
                       w->G, w->tiles);
  }
  hipLaunchKernelGGL(row_shift_kernel, dim3((w->N + 255) / 256), dim3(256), 0, stream(),
                     w->scales, w->N, w->G, w->rshift);
  uint32_t *range_dev = reinterpret_cast<uint32_t *>(w->mem + w->bytes);
  hipLaunchKernelGGL(row_shift_range_kernel, dim3(1), dim3(256), 0, stream(), w->rshift, w->N,
                     range_dev);
  hipError_t e = hipGetLastError();
  uint32_t range[2] = {0, 0};
  if (e == hipSuccess)
    e = hipMemcpyAsync(range, range_dev, sizeof(range), hipMemcpyDeviceToHost, stream());
  if (e == hipSuccess) e = hipStreamSynchronize(stream());
  if (e == hipSuccess) {
    w->shift = (int)range[0] - 512;
    w->row_shift = (int)(range[1] - range[0]) > kRowShiftSpread;
  }
  return e;
}

}  // namespace

namespace {

// g4_w4_load / g4_w4_load_dev / g4_w4_load_opts: validation as
// official-w4a16.js:56-61, one allocation, the bytes copied in unchanged,
// then the GEMM's tile copy and row shifts.  Synchronises.
int load_weight(const void *packed, const void *scales, int out_dim, int in_dim, int group,
                bool from_device, bool tiles, const char *who, g4_w4 **out) {
  if (!out) return fail(G4_E_ARG, "%s: null output handle", who);
  *out = nullptr;
  if (!packed || !scales) return fail(G4_E_ARG, "%s: null weight pointer", who);
  if (out_dim <= 0 || in_dim <= 0)
    return fail(G4_E_ARG, "%s: bad shape [%d, %d]", who, out_dim, in_dim);
  if (in_dim % 8 != 0) return fail(G4_E_ARG, "inDim must be divisible by 8.");
  if (group <= 0 || in_dim % group != 0)
    return fail(G4_E_ARG, "inDim must be divisible by groupSize.");
  if (group != 32)
    return fail(G4_E_ARG, "%s: group size %d unsupported (the checkpoint uses 32)", who, group);
  const int G = in_dim / 32;
  const size_t qbytes = (size_t)out_dim * in_dim / 2;
  const size_t sbytes = (size_t)out_dim * G * 2;
  if (from_device) {
    int rc = check_device_range(packed, qbytes, "weight packed");
    if (!rc) rc = check_device_range(scales, sbytes, "weight scales");
    if (rc) return rc;
  }
  g4_w4 *w = new g4_w4();
  w->N = out_dim;
  w->K = in_dim;
  w->group = group;
  w->G = G;
  int rc = alloc_weight(w, qbytes, sbytes, tiles);
  if (rc) {
    delete w;
    return rc;
  }
  const hipMemcpyKind kind = from_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
  hipError_t e = hipMemcpyAsync(w->packed, packed, qbytes, kind, stream());
  if (e == hipSuccess) e = hipMemcpyAsync(w->scales, scales, sbytes, kind, stream());
  if (e == hipSuccess) e = finish_row_shift(w);
  if (e != hipSuccess) {
    device_free(w->mem);
    delete w;
    return fail(G4_E_HIP, "%s: copy failed: %s", who, hipGetErrorString(e));
  }
  *out = w;
  return ok();
}

}  // namespace

G4_API int g4_w4_load(const void *packed, const void *scales, int out_dim,
                      int in_dim, int group, g4_w4 **out) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  return load_weight(packed, scales, out_dim, in_dim, group, false, true, "g4_w4_load", out);
}

G4_API int g4_w4_load_dev(const void *packed_dev, const void *scales_dev, int out_dim,
                          int in_dim, int group, g4_w4 **out) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  return load_weight(packed_dev, scales_dev, out_dim, in_dim, group, true, true,
                     "g4_w4_load_dev", out);
}

G4_API int g4_w4_load_opts(const void *packed, const void *scales, int out_dim, int in_dim,
                           int group, int flags, g4_w4 **out) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (flags & ~(G4_W4_SRC_DEVICE | G4_W4_NO_GEMM_TILES))
    return fail(G4_E_ARG, "g4_w4_load_opts: unknown flags 0x%x", flags);
  return load_weight(packed, scales, out_dim, in_dim, group, (flags & G4_W4_SRC_DEVICE) != 0,
                     (flags & G4_W4_NO_GEMM_TILES) == 0, "g4_w4_load_opts", out);
}

G4_API int g4_w4_free(g4_w4 *w) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (!w) return ok();
  int rc = device_free(w->mem);
  delete w;
  return rc ? rc : ok();
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

namespace g4 {

int w4_linear_impl(const g4_w4 *w, const void *x, int x_dtype, int rows, void *y, int y_dtype,
                   const ExtScratch *ext, const char *who) {
  if (!w) return fail(G4_E_ARG, "%s: null weight handle", who);
  if (rows <= 0) return fail(G4_E_ARG, "%s: rows must be positive, got %d", who, rows);
  if (x_dtype != G4_F32 && x_dtype != G4_BF16) return fail(G4_E_ARG, "%s: bad x dtype %d", who, x_dtype);
  if (y_dtype != G4_F32 && y_dtype != G4_BF16) return fail(G4_E_ARG, "%s: bad y dtype %d", who, y_dtype);
  if (!aligned16(x)) return fail(G4_E_ARG, "%s: x must be 16-byte aligned", who);
  const size_t xe = x_dtype == G4_F32 ? 4 : 2, ye = y_dtype == G4_F32 ? 4 : 2;
  int rc = check_device_range(x, (size_t)rows * w->K * xe, "g4_w4_linear x");
  if (rc) return rc;
  rc = check_device_range(y, (size_t)rows * w->N * ye, "g4_w4_linear y");
  if (rc) return rc;
  const bool f32x = x_dtype == G4_F32;
  // The GEMVs stage a whole activation row in LDS; a longer in_dim (like any
  // row count above kMaxGemvRows) takes the GEMM, which streams x' tiles.
  const bool gemv_fits = gemv_lds_per_row(w->K, f32x) <= kGemvLdsBudget;
  if (rows == 1 && gemv_fits && has_gemv1_plan(w->G, f32x))
    return f32x ? launch_gemv1<true>(w, x, y, y_dtype == G4_BF16)
                : launch_gemv1<false>(w, x, y, y_dtype == G4_BF16);
  if (rows > kMaxGemvRows || !gemv_fits)
    return ext ? w4_gemm_ext(w, x, f32x, rows, y, y_dtype == G4_BF16, *ext)
               : w4_gemm(w, x, f32x, rows, y, y_dtype == G4_BF16);
  const int per = gemv_rows_per_launch(w->K, f32x);
  for (int r0 = 0; r0 < rows; r0 += per) {
    const int m = rows - r0 < per ? rows - r0 : per;
    const void *xr = static_cast<const char *>(x) + (size_t)r0 * w->K * xe;
    void *yr = static_cast<char *>(y) + (size_t)r0 * w->N * ye;
    rc = f32x ? launch_gemv<true>(w, xr, m, yr, y_dtype == G4_BF16)
              : launch_gemv<false>(w, xr, m, yr, y_dtype == G4_BF16);
    if (rc) return rc;
  }
  return G4_OK;
}

}  // namespace g4

G4_API int g4_w4_linear(const g4_w4 *w, const void *x, int x_dtype, int rows,
                        void *y, int y_dtype) {
  G4_CHECK_INIT();
  const int rc = w4_linear_impl(w, x, x_dtype, rows, y, y_dtype, nullptr, "g4_w4_linear");
  return rc ? rc : ok();
}

G4_API int g4_w4_linear_multi(const g4_w4 *const *w, int n, const void *x, int x_dtype,
                              int rows, void *const *y, int y_dtype) {
  G4_CHECK_INIT();
  if (!w || !y) return fail(G4_E_ARG, "g4_w4_linear_multi: null weight or output array");
  if (n < 1 || n > kMaxLinearSegs)
    return fail(G4_E_ARG, "g4_w4_linear_multi: takes 1..%d weights, got %d", kMaxLinearSegs, n);
  for (int i = 0; i < n; ++i) {
    if (!w[i]) return fail(G4_E_ARG, "g4_w4_linear_multi: null weight handle %d", i);
    if (w[i]->K != w[0]->K)
      return fail(G4_E_ARG, "g4_w4_linear_multi: weight %d has in_dim %d, weight 0 has %d", i,
                  w[i]->K, w[0]->K);
  }
  if (n == 1 || (rows > 1 && rows <= kMaxGemvRows) ||
      (rows == 1 && !has_gemv1_plan(w[0]->G, x_dtype == G4_F32))) {
    for (int i = 0; i < n; ++i)
      if (int rc = g4_w4_linear(w[i], x, x_dtype, rows, y[i], y_dtype)) return rc;
    return ok();
  }
  if (x_dtype != G4_F32 && x_dtype != G4_BF16)
    return fail(G4_E_ARG, "g4_w4_linear_multi: bad x dtype %d", x_dtype);
  if (y_dtype != G4_F32 && y_dtype != G4_BF16)
    return fail(G4_E_ARG, "g4_w4_linear_multi: bad y dtype %d", y_dtype);
  if (rows <= 0)
    return fail(G4_E_ARG, "g4_w4_linear_multi: rows must be positive, got %d", rows);
  if (!aligned16(x)) return fail(G4_E_ARG, "g4_w4_linear_multi: x must be 16-byte aligned");
  const bool f32x = x_dtype == G4_F32;
  const size_t xe = f32x ? 4 : 2, ye = y_dtype == G4_F32 ? 4 : 2;
  int rc = check_device_range(x, (size_t)rows * w[0]->K * xe, "g4_w4_linear_multi x");
  if (rc) return rc;
  for (int i = 0; i < n; ++i)
    if ((rc = check_device_range(y[i], (size_t)rows * w[i]->N * ye, "g4_w4_linear_multi y")))
      return rc;
  // more than kMaxGemvRows, or an in_dim beyond the GEMV's LDS staging: one
  // x pre-pass, one GEMM launch when it fills
  if (rows > 1 || gemv_lds_per_row(w[0]->K, f32x) > kGemvLdsBudget) {
    rc = w4_gemm_multi(w, n, x, f32x, rows, y, y_dtype == G4_BF16);
    return rc ? rc : ok();
  }
  rc = f32x ? launch_gemv1_multi<true>(w, n, x, y, y_dtype == G4_BF16)
            : launch_gemv1_multi<false>(w, n, x, y, y_dtype == G4_BF16);
  return rc ? rc : ok();
}

namespace g4 {
namespace {

template <int J, int W, bool F32X>
int launch_r16_stamps(const g4_w4 *w, const void *x, void *y, int y_bf16, uint64_t *stamps) {
  hipLaunchKernelGGL((w4_gemv_r16_stamp_kernel<J, W, F32X>), dim3((w->N + 4 * W - 1) / (4 * W)),
                     dim3(64 * W), 0, stream(), x, w->packed, w->scales, y, y_bf16, w->N, stamps);
  G4_LAUNCH_CHECK("w4_gemv_r16_stamp_kernel");
  return G4_OK;
}

}  // namespace
}  // namespace g4

G4_API int g4_w4_gemv_stamps(const g4_w4 *w, const void *x, int x_dtype, void *y, int y_dtype,
                             uint64_t *stamps, int *waves) {
  G4_CHECK_INIT();
  if (!w || !waves) return fail(G4_E_ARG, "g4_w4_gemv_stamps: null weight or wave count");
  if (!has_r16(w->G))
    return fail(G4_E_ARG, "g4_w4_gemv_stamps: in_dim %d does not take the row split "
                          "(1536 or 2048)", w->K);
  const int W = r16_waves(w->N);
  const int nw = (w->N + 4 * W - 1) / (4 * W) * W;
  *waves = nw;
  if (!stamps) return ok();
  if (x_dtype != G4_F32 && x_dtype != G4_BF16)
    return fail(G4_E_ARG, "g4_w4_gemv_stamps: bad x dtype %d", x_dtype);
  if (y_dtype != G4_F32 && y_dtype != G4_BF16)
    return fail(G4_E_ARG, "g4_w4_gemv_stamps: bad y dtype %d", y_dtype);
  if (!aligned16(x)) return fail(G4_E_ARG, "g4_w4_gemv_stamps: x must be 16-byte aligned");
  const bool f32x = x_dtype == G4_F32;
  int rc = check_device_range(x, (size_t)w->K * (f32x ? 4 : 2), "g4_w4_gemv_stamps x");
  if (!rc) rc = check_device_range(y, (size_t)w->N * (y_dtype == G4_F32 ? 4 : 2),
                                   "g4_w4_gemv_stamps y");
  if (!rc) rc = check_device_range(stamps, (size_t)nw * 5 * sizeof(uint64_t),
                                   "g4_w4_gemv_stamps stamps");
  if (rc) return rc;
  const int yb = y_dtype == G4_BF16;
  if (w->G == 48)
    rc = f32x ? (W == 4 ? launch_r16_stamps<3, 4, true>(w, x, y, yb, stamps)
                        : launch_r16_stamps<3, 2, true>(w, x, y, yb, stamps))
              : (W == 4 ? launch_r16_stamps<3, 4, false>(w, x, y, yb, stamps)
                        : launch_r16_stamps<3, 2, false>(w, x, y, yb, stamps));
  else
    rc = f32x ? (W == 4 ? launch_r16_stamps<4, 4, true>(w, x, y, yb, stamps)
                        : launch_r16_stamps<4, 2, true>(w, x, y, yb, stamps))
              : (W == 4 ? launch_r16_stamps<4, 4, false>(w, x, y, yb, stamps)
                        : launch_r16_stamps<4, 2, false>(w, x, y, yb, stamps));
  return rc ? rc : ok();
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
