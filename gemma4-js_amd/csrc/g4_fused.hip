// Fused one-token kernels of the decode step.  The reference runs every op of
// encodeLayer (custom-webgpu/gemma4-webgpu.js:215-301) as its own dispatch;
// at one token per step those dispatches are tiny and their launch cost, not
// HBM, bounds the step.  Here the element-wise ops travel with the GEMVs:
//
//  * prologue (x staging of the GEMV): the RMS norm, or the chain
//    r = (h + rms(a) * w1) * c; x = rms(r) * w2 that ends one sub-block and
//    starts the next (post-norm, residual add, skip scale, pre-norm).  Every
//    block recomputes the norms from the (L2-resident) vectors; block 0 also
//    writes r, the residual stream the later ops need.
//  * epilogue: gelu(gate) * up with the gate and up rows of one output index
//    in the same block, or gelu(y) * ple[layer] for the PLE gate.
//  * segments: q, k and v (same input) in one launch.
//
// The arithmetic per element is the reference's (rms = x * inv * scale,
// addScale = (a + b) * s, the tanh GELU); only the reductions are reordered.
// The GEMV core is the bf16-pair dot-product scheme of w4_gemv1_kernel
// (g4_w4.hip) with FP32 activations split into hi + lo.
#include <math.h>

#include "g4_gemv.h"
#include "g4_internal.h"
#include "g4_ops.h"

namespace g4 {
namespace {

enum { kProNone = 0, kProNorm = 1, kProResNorm = 2, kProRes = 3 };
enum { kEpiNone = 0, kEpiGeluUp = 1, kEpiGeluMul = 2 };
constexpr int kMaxParts = 8;  // partial input vectors a kProRes prologue adds

struct FusedSeg {
  const uint4 *wq;
  const uint16_t *ws;
  float *y;
  int N;
  int block0;  // first block of this segment
};

struct FusedArgs {
  FusedSeg seg[3];
  int nseg;
  const float *a, *h, *w1, *w2;  // prologue inputs
  int a_parts;                    // kProRes: a is the sum of a_parts vectors of K floats
  float c, eps;
  float *r_out;       // residual written by block 0 (kProRes, kProResNorm)
  const float *mul;   // kEpiGeluMul multiplier per output row
  int K;
};

// Sum over the block; all threads get it.  red: >= 16 floats.
__device__ __forceinline__ float fblock_sum(float v, float *red, int nwaves) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < nwaves; ++i) s += red[i];
  return s;
}

// Sum over the prologue waves 0..pw-1 (v of the other waves is ignored); all
// threads get it.  Every wave of the block must call it.  red: pw floats,
// not reused by the next call before a barrier.
__device__ __forceinline__ float pro_sum(float v, float *red, int pw, bool pro) {
  v = wave_sum(v);
  if (pro && (threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < pw; ++i) s += red[i];
  return s;
}

__device__ __forceinline__ void load8(const float *p, size_t c, float (&v)[8]) {
  const float4 a = reinterpret_cast<const float4 *>(p)[2 * c];
  const float4 b = reinterpret_cast<const float4 *>(p)[2 * c + 1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// Loads the weight groups of row group rg (RB rows; gate/up: RB/2 of each).
template <int IPL, int EPI>
__device__ __forceinline__ void load_rows(const FusedArgs &A, int rg, int G, int RB, int T,
                                          int t, uint4 (&q)[IPL], uint32_t (&s)[IPL]) {
  const int nseg = EPI == kEpiGeluUp ? 1 : A.nseg;
  int si = 0;
  if (nseg > 1 && rg >= A.seg[1].block0) si = 1;
  if (nseg > 2 && rg >= A.seg[2].block0) si = 2;
  const FusedSeg &S = si == 0 ? A.seg[0] : si == 1 ? A.seg[1] : A.seg[2];
  const int rows_here = EPI == kEpiGeluUp ? RB / 2 : RB;
  const int o0 = (rg - S.block0) * rows_here;
#pragma unroll
  for (int i = 0; i < IPL; ++i) {
    const int it = t + i * T;
    const uint4 *wq = S.wq;
    const uint16_t *ws = S.ws;
    size_t idx = (size_t)o0 * G + it;
    size_t last = (size_t)S.N * G - 1;
    if (EPI == kEpiGeluUp && it >= rows_here * G) {  // second half: the up rows
      wq = A.seg[1].wq;
      ws = A.seg[1].ws;
      idx -= (size_t)rows_here * G;
      last = (size_t)A.seg[1].N * G - 1;
    }
    idx = idx < last ? idx : last;
    q[i] = ld_nt(&wq[idx]);
    s[i] = ld_nt_u16(&ws[idx]);
  }
}

// The output segment that row group rg belongs to, and its first row.
template <int EPI>
__device__ __forceinline__ const FusedSeg &seg_for(const FusedArgs &A, int rg, int rows_here,
                                                   int *o0) {
  const int nseg = EPI == kEpiGeluUp ? 1 : A.nseg;
  int si = 0;
  if (nseg > 1 && rg >= A.seg[1].block0) si = 1;
  if (nseg > 2 && rg >= A.seg[2].block0) si = 2;
  const FusedSeg &S = si == 0 ? A.seg[0] : si == 1 ? A.seg[1] : A.seg[2];
  *o0 = (rg - S.block0) * rows_here;
  return S;
}

// The activation inputs of one prologue lane: XI chunks of 8 of each vector.
// With kProRes, a may come as up to kMaxParts partial vectors (split-K sums of
// the previous GEMV).
template <int XI, int PRO>
struct ProIn {
  static constexpr int NPART = PRO == kProRes ? kMaxParts : 1;
  float av[XI][8], hv[XI][8], w1v[XI][8], w2v[XI][8], apv[NPART > 1 ? NPART - 1 : 1][XI][8];
};

// Step 1 of a fused launch: the prologue lanes load their activation chunks
// (chunk t + i * cstride), before the weight stream.  All partial vectors are
// loaded here (past a_parts the last is re-read) and added in order later.
template <int XI, int PRO>
__device__ __forceinline__ void pro_load(const FusedArgs &A, int t, int cstride, int nch,
                                         bool pro, ProIn<XI, PRO> &in) {
  if (!pro) return;
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int ct = t + i * cstride;
    const int cc = ct < nch ? ct : nch - 1;
    load8(A.a, cc, in.av[i]);
#pragma unroll
    for (int pp = 1; pp < ProIn<XI, PRO>::NPART; ++pp) {
      const int pc = pp < A.a_parts ? pp : A.a_parts - 1;
      load8(A.a + (size_t)pc * A.K, cc, in.apv[pp - 1][i]);
    }
    if (PRO != kProNone) load8(A.w1, cc, in.w1v[i]);
    if (PRO == kProRes || PRO == kProResNorm) load8(A.h, cc, in.hv[i]);
    if (PRO == kProResNorm) load8(A.w2, cc, in.w2v[i]);
  }
}

// Steps 3 and 4: the prologue (norms, residual; block 0 writes r) and the x
// staging: hi/lo bf16 pairs per chunk in hi[c * G + g], lo[...], and
// 136 * group sum in sx[g].  Every wave of the block must call it (the
// reductions are block-wide); the element-wise work stays on the pw
// prologue waves.  red: 32 floats.  Ends with the block barrier after which
// the staged x may be read.
template <int XI, int PRO>
__device__ __forceinline__ void pro_stage(const FusedArgs &A, ProIn<XI, PRO> &in, int t,
                                          int cstride, int nch, int pw, bool pro, int G,
                                          uint4 *hi, uint4 *lo, float *sx, float *red) {
  float xv[XI][8];
  if (PRO == kProNone) {
    if (pro) {
#pragma unroll
      for (int i = 0; i < XI; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[i][e] = in.av[i][e];
    }
  } else {
    if (ProIn<XI, PRO>::NPART > 1 && pro) {
#pragma unroll
      for (int pp = 1; pp < ProIn<XI, PRO>::NPART; ++pp)
        if (pp < A.a_parts)
#pragma unroll
          for (int i = 0; i < XI; ++i)
#pragma unroll
            for (int e = 0; e < 8; ++e) in.av[i][e] += in.apv[pp - 1][i][e];
    }
    float ss = 0.f;
    if (pro) {
#pragma unroll
      for (int i = 0; i < XI; ++i)
        if (t + i * cstride < nch)
#pragma unroll
          for (int e = 0; e < 8; ++e) ss += in.av[i][e] * in.av[i][e];
    }
    const float tot1 = pro_sum(ss, red, pw, pro);
    float r[XI][8];
    float ss2 = 0.f;
    if (pro) {
      const float inv1 = 1.f / sqrtf(tot1 / (float)A.K + A.eps);
      if (PRO == kProNorm) {
#pragma unroll
        for (int i = 0; i < XI; ++i)
#pragma unroll
          for (int e = 0; e < 8; ++e) xv[i][e] = in.av[i][e] * inv1 * in.w1v[i][e];
      } else {
#pragma unroll
        for (int i = 0; i < XI; ++i)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            r[i][e] = (in.hv[i][e] + in.av[i][e] * inv1 * in.w1v[i][e]) * A.c;
            if (t + i * cstride < nch) ss2 += r[i][e] * r[i][e];
          }
        if (blockIdx.x == 0) {
#pragma unroll
          for (int i = 0; i < XI; ++i) {
            const int ct = t + i * cstride;
            if (ct < nch) {
              float4 *ro = reinterpret_cast<float4 *>(A.r_out) + 2 * ct;
              ro[0] = make_float4(r[i][0], r[i][1], r[i][2], r[i][3]);
              ro[1] = make_float4(r[i][4], r[i][5], r[i][6], r[i][7]);
            }
          }
        }
        if (PRO == kProRes) {
#pragma unroll
          for (int i = 0; i < XI; ++i)
#pragma unroll
            for (int e = 0; e < 8; ++e) xv[i][e] = r[i][e];
        }
      }
    }
    if (PRO == kProResNorm) {
      const float tot2 = pro_sum(ss2, red + 16, pw, pro);
      if (pro) {
        const float inv2 = 1.f / sqrtf(tot2 / (float)A.K + A.eps);
#pragma unroll
        for (int i = 0; i < XI; ++i)
#pragma unroll
          for (int e = 0; e < 8; ++e) xv[i][e] = r[i][e] * inv2 * in.w2v[i][e];
      }
    }
  }

  if (pro) {
#pragma unroll
    for (int i = 0; i < XI; ++i) {
      const int ct = t + i * cstride;
      uint32_t hb[8], lb[8];
      float sum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        hb[e] = f32_to_bf16_rne(xv[i][e]);
        lb[e] = f32_to_bf16_rne(xv[i][e] - bf16_to_f32(hb[e]));
        sum += bf16_to_f32(hb[e]) + bf16_to_f32(lb[e]);
      }
      sum += dpp_f32<0xB1>(sum);  // chunks 4g..4g+3 of a group sit in one lane quad
      sum += dpp_f32<0x4E>(sum);
      if (ct < nch) {
        const int g = ct >> 2, c = ct & 3;
        hi[c * G + g] = make_uint4(bf16_pair(hb[0], hb[4]), bf16_pair(hb[1], hb[5]),
                                   bf16_pair(hb[2], hb[6]), bf16_pair(hb[3], hb[7]));
        lo[c * G + g] = make_uint4(bf16_pair(lb[0], lb[4]), bf16_pair(lb[1], lb[5]),
                                   bf16_pair(lb[2], lb[6]), bf16_pair(lb[3], lb[7]));
        if (c == 0) sx[g] = kPairBias * sum;
      }
    }
  }
  __syncthreads();
}

// Block b owns row groups b, b + grid, ..., IT of them (ngroups in total).
// Every weight load of those groups is issued at the start, before the
// prologue: the prologue's chain of dependent steps (activation loads, two
// block reductions, staging) then overlaps one HBM round trip instead of
// delaying the later groups' loads.
template <int GC, int TC, int IPL, int IT, int PRO, int EPI>
__global__ __launch_bounds__(TC ? TC : 1024) void fused_gemv_kernel(FusedArgs A, int RB_,
                                                                    int ngroups) {
  extern __shared__ uint4 lds[];
  const int T = TC ? TC : (int)blockDim.x;
  const int G = GC ? GC : A.K >> 5;
  const int RB = GC ? TC * IPL / GC : RB_;
  const int nch = 4 * G;
  const int t = threadIdx.x;
  const int nwaves = (T + 63) >> 6;

  // The prologue runs on the first pw waves only (the 4G chunks of 8 inputs,
  // XI per lane): the other waves skip it and meet them at the barriers, so
  // the SIMDs are not busy with copies of the same element-wise work.
  const int wave = t >> 6;
  const int pw = ((nch + 63) >> 6) < nwaves ? ((nch + 63) >> 6) : nwaves;
  const bool pro = wave < pw;  // uniform per wave
  const int cstride = 64 * pw;
  constexpr int XI = (GC && TC) ? (4 * GC + 63) / 64 <= TC / 64 ? 1 : (4 * GC + TC - 1) / TC : IPL;

  // 1. activation chunks, issued before the weight stream
  ProIn<XI, PRO> in;
  pro_load<XI, PRO>(A, t, cstride, nch, pro, in);

  // 2. weights of all the block's row groups (groups past the last re-read it
  // and store nothing; rows past N re-read the last group)
  uint4 q[IT][IPL];
  uint32_t s[IT][IPL];
#pragma unroll
  for (int k = 0; k < IT; ++k) {
    const int rg = blockIdx.x + k * (int)gridDim.x;
    load_rows<IPL, EPI>(A, rg < ngroups ? rg : ngroups - 1, G, RB, T, t, q[k], s[k]);
  }

  // 3-4. prologue and x staging
  constexpr int CH = 2;  // FP32 activations: hi and lo
  uint4 *hi = lds;
  uint4 *lo = lds + 4 * G;
  float *sx = reinterpret_cast<float *>(lds + 4 * G * CH);
  float *part = sx + G;              // [IT * RB][G]
  float *rs = part + IT * RB * G;    // row sums [IT * RB] (kEpiGeluUp)
  float *red = rs + IT * RB;         // 2 x 16 wave sums
  pro_stage<XI, PRO>(A, in, t, cstride, nch, pw, pro, G, hi, lo, sx, red);

  // 5. one partial per group, for every row group of the block
  uint32_t mask = 0x000F000Fu;
  asm volatile("" : "+v"(mask));  // keep the mask in a VGPR: lets v_and_or_b32 take the magic
#pragma unroll
  for (int k = 0; k < IT; ++k)
#pragma unroll
    for (int i = 0; i < IPL; ++i) {
      const int li = t + i * T;
      const int g = li % G;
      uint32_t pr[4][4];
      group_pairs(q[k][i], mask, pr);
      float d0 = 0.f, d1 = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t p0 = pr[c][0], p1 = pr[c][1], p2 = pr[c][2], p3 = pr[c][3];
        const uint4 xp = hi[c * G + g];
        const uint4 xl = lo[c * G + g];
        d0 = dot2_bf16(xp.x, p0, d0);
        d1 = dot2_bf16(xp.y, p1, d1);
        d0 = dot2_bf16(xp.z, p2, d0);
        d1 = dot2_bf16(xp.w, p3, d1);
        d0 = dot2_bf16(xl.x, p0, d0);
        d1 = dot2_bf16(xl.y, p1, d1);
        d0 = dot2_bf16(xl.z, p2, d0);
        d1 = dot2_bf16(xl.w, p3, d1);
      }
      part[k * RB * G + li] = bf16_to_f32(s[k][i]) * ((d0 + d1) - sx[g]);
    }
  __syncthreads();

  // 6. 16 lanes per row sum the row's G partials, then the epilogue
  const int rows_here = EPI == kEpiGeluUp ? RB / 2 : RB;
  for (int b = 0; b < IT * RB * 16; b += T) {
    const int idx = b + t;
    const int rr = idx >> 4, j = idx & 15;  // rr = k * RB + r
    float v = 0.f;
    if (rr < IT * RB) {
      if (GC) {
#pragma unroll
        for (int g = j; g < GC; g += 16) v += part[rr * GC + g];
      } else {
        for (int g = j; g < G; g += 16) v += part[rr * G + g];
      }
    }
    v = team_sum<16>(v);
    if (j == 0 && rr < IT * RB) {
      if (EPI == kEpiGeluUp) {
        rs[rr] = v;
      } else {
        const int k = rr / RB, r = rr - k * RB;
        const int rg = blockIdx.x + k * (int)gridDim.x;
        int o0;
        const FusedSeg &S = seg_for<EPI>(A, rg, rows_here, &o0);
        const int row = o0 + r;
        if (rg < ngroups && row < S.N)
          S.y[row] = EPI == kEpiGeluMul ? gelu_tanh(v) * A.mul[row] : v;
      }
    }
  }
  if (EPI == kEpiGeluUp) {
    __syncthreads();
    for (int e = t; e < IT * rows_here; e += T) {
      const int k = e / rows_here, r = e - k * rows_here;
      const int rg = blockIdx.x + k * (int)gridDim.x;
      const int row = rg * rows_here + r;
      if (rg < ngroups && row < A.seg[0].N)
        A.seg[0].y[row] = gelu_tanh(rs[k * RB + r]) * rs[k * RB + rows_here + r];
    }
  }
}

// Row split of a fused launch at in_dim 1536 (48 groups per row): 16 lanes per
// output row, lane c taking groups c, c + 16 and c + 32, as in
// w4_gemv_r16_kernel.  A block of W waves owns row groups of 4 W rows, IT of
// them as in fused_gemv_kernel.  The prologue and staging are the flat
// kernel's; after the staging barrier every lane reads its groups' x pairs
// into registers and each row sum is a 16-lane DPP reduction: no LDS
// partials and no barrier after the weights land.  The group partials and
// their order are the flat kernel's, so the outputs are bit-identical.  (No
// gelu(gate) * up epilogue: gate/up keeps the flat split.)
template <int EPI>
__device__ __forceinline__ const FusedSeg &r16_row(const FusedArgs &A, int rg, int team, int W,
                                                   int *o) {
  int o0;
  const FusedSeg &S = seg_for<EPI>(A, rg, 4 * W, &o0);
  *o = o0 + team;
  return S;
}

template <int W, int IT, int PRO, int EPI>
__global__ __launch_bounds__(64 * W) void fused_r16_kernel(FusedArgs A, int ngroups) {
  static_assert(EPI != kEpiGeluUp, "gate/up takes the flat split");
  constexpr int J = 3, G = 16 * J, nch = 4 * G;
  constexpr int PW = (nch + 63) / 64 < W ? (nch + 63) / 64 : W;  // prologue waves
  constexpr int XI = (nch + 64 * PW - 1) / (64 * PW);
  __shared__ uint4 hi[4 * G], lo[4 * G];
  __shared__ float sx[G], red[32];
  const int t = threadIdx.x, c16 = t & 15, team = t >> 4;
  const bool pro = (t >> 6) < PW;  // uniform per wave

  // 1. activation chunks, issued before the weight stream
  ProIn<XI, PRO> in;
  pro_load<XI, PRO>(A, t, 64 * PW, nch, pro, in);

  // 2. the lane's groups of its row in every row group (groups past the last
  // re-read it, rows past N the last row; neither is stored)
  uint4 q[IT][J];
  uint32_t s[IT][J];
#pragma unroll
  for (int k = 0; k < IT; ++k) {
    const int rg = blockIdx.x + k * (int)gridDim.x;
    int o;
    const FusedSeg &S = r16_row<EPI>(A, rg < ngroups ? rg : ngroups - 1, team, W, &o);
    const int rr = o < S.N ? o : S.N - 1;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const size_t it = (size_t)rr * G + c16 + 16 * j;
      q[k][j] = ld_nt(&S.wq[it]);
      s[k][j] = ld_nt_u16(&S.ws[it]);
    }
  }

  // 3-4. prologue and x staging; keep the weight arithmetic below its barriers
  __builtin_amdgcn_sched_barrier(0);
  pro_stage<XI, PRO>(A, in, t, 64 * PW, nch, PW, pro, G, hi, lo, sx, red);

  // 5. the lane's x groups into registers, all reads issued before any weight use
  uint4 xh[J][4], xl[J][4];
  float sxr[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int g = c16 + 16 * j;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      xh[j][c] = hi[c * G + g];
      xl[j][c] = lo[c * G + g];
    }
    sxr[j] = sx[g];
  }
  __builtin_amdgcn_sched_barrier(0);

  // 6. per row group: group partials, the 16-lane row sum, the epilogue
  uint32_t mask = 0x000F000Fu;
  asm volatile("" : "+v"(mask));  // keep the mask in a VGPR: lets v_and_or_b32 take the magic
#pragma unroll
  for (int k = 0; k < IT; ++k) {
    float v = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      uint32_t pr[4][4];
      group_pairs(q[k][j], mask, pr);
      float d0 = 0.f, d1 = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t p0 = pr[c][0], p1 = pr[c][1], p2 = pr[c][2], p3 = pr[c][3];
        const uint4 xp = xh[j][c];
        const uint4 xq = xl[j][c];
        d0 = dot2_bf16(xp.x, p0, d0);
        d1 = dot2_bf16(xp.y, p1, d1);
        d0 = dot2_bf16(xp.z, p2, d0);
        d1 = dot2_bf16(xp.w, p3, d1);
        d0 = dot2_bf16(xq.x, p0, d0);
        d1 = dot2_bf16(xq.y, p1, d1);
        d0 = dot2_bf16(xq.z, p2, d0);
        d1 = dot2_bf16(xq.w, p3, d1);
      }
      float pj = bf16_to_f32(s[k][j]) * ((d0 + d1) - sxr[j]);
      asm volatile("" : "+v"(pj));  // rounded on its own (no FMA into the row sum)
      v += pj;
    }
    v = team_sum<16>(v);
    const int rg = blockIdx.x + k * (int)gridDim.x;
    int o;
    const FusedSeg &S = r16_row<EPI>(A, rg < ngroups ? rg : ngroups - 1, team, W, &o);
    if (c16 == 0 && rg < ngroups && o < S.N)
      S.y[o] = EPI == kEpiGeluMul ? gelu_tanh(v) * A.mul[o] : v;
  }
}

// LDS of a fused launch: x hi/lo pairs, group sums, IT * RB rows of partials
// and row sums, the reduction scratch.
size_t fused_lds(int G, int RB, int IT) {
  return (size_t)G * 4 * 16 * 2 + (size_t)G * 4 + (size_t)IT * RB * G * 4 + (size_t)IT * RB * 4 +
         32 * 4;
}

template <int GC, int TC, int IPL, int IT, int PRO, int EPI>
int launch_fused_it(const FusedArgs &a, const Gemv1Plan &p, int ngroups) {
  const int blocks = (ngroups + IT - 1) / IT;
  const size_t lds = fused_lds(GC ? GC : a.K / 32, p.RB, IT);
  if (lds > 64 * 1024) return fail(G4_E_ARG, "fused GEMV: %zu bytes of LDS", lds);
  hipLaunchKernelGGL((fused_gemv_kernel<GC, TC, IPL, IT, PRO, EPI>), dim3(blocks), dim3(p.T), lds,
                     stream(), a, p.RB, ngroups);
  G4_LAUNCH_CHECK("fused_gemv_kernel");
  return G4_OK;
}

// Row groups per block: one per block while they fit one wave of blocks on
// the CUs, else more per block, up to 3 (measured: more loads per block
// delay the blocks' activation loads behind their weight stream).
template <int GC, int TC, int IPL, int PRO, int EPI>
int launch_fused_i(const FusedArgs &a, const Gemv1Plan &p, int ngroups) {
  constexpr int kMaxIt = IPL <= 2 ? 3 : 2;
  const int cap = cu_count() > 0 ? cu_count() : 256;
  int it = (ngroups + cap - 1) / cap;
  it = it < 1 ? 1 : it > kMaxIt ? kMaxIt : it;
  switch (it) {
    case 1: return launch_fused_it<GC, TC, IPL, 1, PRO, EPI>(a, p, ngroups);
    case 2: return launch_fused_it<GC, TC, IPL, 2, PRO, EPI>(a, p, ngroups);
    default: return launch_fused_it<GC, TC, IPL, kMaxIt, PRO, EPI>(a, p, ngroups);
  }
}

// Rows per block: 16 (8 when there are fewer than 2048 rows), one 16-byte
// group per thread (measured best for the Gemma-4-E2B shapes with cold
// weights: gate/up 6144 and 12288, q/k/v, the PLE gate).
bool plan_fused(int G, int total_rows, Gemv1Plan *p) {
  const int want = total_rows >= 2048 ? 16 : 8;
  for (int RB = want; RB <= 256; RB *= 2)
    for (int ipl = 1; ipl <= 4; ++ipl) {
      const long items = (long)RB * G;
      if (items % ipl || (items / ipl) % 64 || items / ipl > 1024) continue;
      p->T = (int)(items / ipl);
      p->IPL = ipl;
      p->RB = RB;
      p->lds = fused_lds(G, RB, 3);
      return p->lds <= 64 * 1024;
    }
  return false;
}

template <int W, int IT, int PRO, int EPI>
int launch_fused_r16_it(const FusedArgs &a, int groups) {
  hipLaunchKernelGGL((fused_r16_kernel<W, IT, PRO, EPI>), dim3((groups + IT - 1) / IT),
                     dim3(64 * W), 0, stream(), a, groups);
  G4_LAUNCH_CHECK("fused_r16_kernel");
  return G4_OK;
}

// Row groups of 4 W rows; up to 3 per block once they outnumber the CUs, as
// in launch_fused_i.
template <int W, int PRO, int EPI>
int launch_fused_r16(FusedArgs a) {
  int groups = 0;
  for (int i = 0; i < a.nseg; ++i) {
    a.seg[i].block0 = groups;
    groups += (a.seg[i].N + 4 * W - 1) / (4 * W);
  }
  const int cap = cu_count() > 0 ? cu_count() : 256;
  int it = (groups + cap - 1) / cap;
  it = it < 1 ? 1 : it > 3 ? 3 : it;
  switch (it) {
    case 1: return launch_fused_r16_it<W, 1, PRO, EPI>(a, groups);
    case 2: return launch_fused_r16_it<W, 2, PRO, EPI>(a, groups);
    default: return launch_fused_r16_it<W, 3, PRO, EPI>(a, groups);
  }
}

template <int PRO, int EPI>
int launch_fused(FusedArgs a) {
  const int G = a.K / 32;
  // The PLE gate (256 rows at in_dim 1536) takes the row split with 12 rows
  // per block: E2B decode 1.253 ms/token against 1.260 with the flat split.
  // q/k/v and gate/up keep the flat split, whose 12-wave blocks give each
  // lane one group (the row split's three groups per lane measured 1.265).
  if constexpr (EPI == kEpiGeluMul) {
    if (a.K == 1536) return launch_fused_r16<3, PRO, EPI>(a);
  }
  int total_rows = 0;
  for (int i = 0; i < a.nseg; ++i) total_rows += a.seg[i].N;
  Gemv1Plan p;
  if (a.K % 32 != 0 || !plan_fused(G, total_rows, &p))
    return fail(G4_E_ARG, "fused GEMV: no plan for in_dim %d", a.K);
  if (4 * G > p.T * p.IPL)
    return fail(G4_E_ARG, "fused GEMV: in_dim %d needs more threads than the plan has", a.K);
  const int rows_per_group = EPI == kEpiGeluUp ? p.RB / 2 : p.RB;
  int groups = 0;
  if (EPI == kEpiGeluUp) {
    a.seg[0].block0 = 0;
    groups = (a.seg[0].N + rows_per_group - 1) / rows_per_group;
  } else {
    for (int i = 0; i < a.nseg; ++i) {
      a.seg[i].block0 = groups;
      groups += (a.seg[i].N + rows_per_group - 1) / rows_per_group;
    }
  }
  if (G == 48) {  // the E2B hidden size 1536
    if (p.T == 384 && p.IPL == 1) return launch_fused_i<48, 384, 1, PRO, EPI>(a, p, groups);
    if (p.T == 768 && p.IPL == 1) return launch_fused_i<48, 768, 1, PRO, EPI>(a, p, groups);
  }
  switch (p.IPL) {
    case 1: return launch_fused_i<0, 0, 1, PRO, EPI>(a, p, groups);
    case 2: return launch_fused_i<0, 0, 2, PRO, EPI>(a, p, groups);
    case 3: return launch_fused_i<0, 0, 3, PRO, EPI>(a, p, groups);
    default: return launch_fused_i<0, 0, 4, PRO, EPI>(a, p, groups);
  }
}

FusedSeg seg_of(const g4_w4 *w, float *y) {
  FusedSeg s;
  s.wq = w->packed;
  s.ws = w->scales;
  s.y = y;
  s.N = w->N;
  s.block0 = 0;
  return s;
}

// ---- q/k norm-RoPE, k/v cache append, v norm: one launch --------------------
// Blocks [0, heads) rotate the q heads; block heads writes k and block
// heads + 1 writes v (RMS norm without scale) at position *pos of the caches.
__global__ __launch_bounds__(256) void rope_qkv_kernel(
    const float *__restrict__ qraw, const float *__restrict__ kraw,
    const float *__restrict__ vraw, int heads, int hd, const int *__restrict__ pos_dev,
    const float *__restrict__ qnorm, const float *__restrict__ knorm, int rope_angles,
    float base, float eps, float *__restrict__ q, float *__restrict__ kc,
    float *__restrict__ vc) {
  __shared__ float red[4];
  const int b = blockIdx.x, t = threadIdx.x, half = hd >> 1;
  const int pos = *pos_dev;
  const bool is_v = b == heads + 1;
  const float *x = b < heads ? qraw + (size_t)b * hd : b == heads ? kraw : vraw;
  float a = 0.f, c = 0.f;
  if (t < half) {
    a = x[t];
    c = x[t + half];
  }
  float ss = a * a + c * c;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  if ((t & 63) == 0) red[t >> 6] = ss;
  __syncthreads();
  ss = red[0] + red[1] + red[2] + red[3];
  const float inv = 1.f / sqrtf(ss / (float)hd + eps);
  if (t >= half) return;
  if (is_v) {
    float *vo = vc + (size_t)pos * hd;
    vo[t] = a * inv;
    vo[t + half] = c * inv;
    return;
  }
  const float *sc = b < heads ? qnorm : knorm;
  const float an = a * inv * sc[t], cn = c * inv * sc[t + half];
  float sn = 0.f, cs = 1.f;
  if (t < rope_angles) {
    const float ex = 2.f * (float)t / (float)hd;
    const float theta = (float)pos / powf(base, ex);
    sn = sinf(theta);
    cs = cosf(theta);
  }
  float *yo = b < heads ? q + (size_t)b * hd : kc + (size_t)pos * hd;
  yo[t] = an * cs - cn * sn;
  yo[t + half] = cn * cs + an * sn;
}

// ---- token start: the scaled embedding row and the RoPE tables -------------
// Block 0 writes y = bf16 row(ids[0]) * scale (NaN for an id out of range);
// block 1 + j fills table j with (cos, sin) of theta = pos / base^(2t/hd) for
// t < angles at the current position, the angles of NORM_ROPE_SHADER
// (gpu-runtime.js:1175-1202), so the attention kernels do no pow/sin/cos.
__global__ __launch_bounds__(256) void token_start_kernel(const uint16_t *__restrict__ E,
                                                          int vocab, int width,
                                                          const int *__restrict__ ids,
                                                          float scale, float *__restrict__ y,
                                                          const int *__restrict__ pos_dev,
                                                          RopeSlots slots,
                                                          float2 *__restrict__ tab) {
  const int b = blockIdx.x;
  if (b == 0) {
    const int id = ids[0];
    const bool ok = id >= 0 && id < vocab;
    const uint16_t *row = E + (size_t)(ok ? id : 0) * width;
    constexpr int U = 8;
    for (int b0 = threadIdx.x; b0 < width; b0 += 256 * U) {
      uint16_t v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = b0 + 256 * u;
        v[u] = row[i < width ? i : width - 1];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = b0 + 256 * u;
        if (i < width) y[i] = ok ? bf16_to_f32(v[u]) * scale : __int_as_float(0x7fc00000);
      }
    }
    return;
  }
  const int j = b - 1;
  const int pos = *pos_dev;
  const int hd = slots.hd[j];
  for (int t = threadIdx.x; t < slots.angles[j]; t += 256) {
    const float ex = 2.f * (float)t / (float)hd;
    const float theta = (float)pos / powf(slots.base[j], ex);
    tab[j * kRopeTable + t] = make_float2(cosf(theta), sinf(theta));
  }
}

// ---- decode attention in one launch ------------------------------------------
// The q/k RMS norm and RoPE and the v norm (NORM_ROPE_SHADER), the append of
// k and v at position pos of the cache (KVCache.append), attention of the one
// query over the visible keys (QK, SOFTMAX and ATTN_OUT shaders,
// gpu-runtime.js:1204-1248) and the merge of the key splits.
//
// Grid: H * S blocks, block h * S + s = head h, split s of the visible keys
// [lo, pos] (S a multiple of 8: the blocks of one split share an XCD and
// its L2 copy of the k/v rows).  Block = 4 waves; wave w takes keys
// k0 + w, k0 + w + 4, ...  A wave holds a whole head: lane l keeps dims
// [l*DH, l*DH + DH) and their RoPE partners [hd/2 + l*DH, ...), so the norms
// are wave reductions and the rotation stays in the lane.  Every wave
// normalises and rotates q itself; the wave whose keys include pos also
// builds the new k and v (block h = 0 writes them to the cache).
// Each block writes (max, sum, unnormalised output) of its keys; the last
// block of a head to finish (a device-scope counter, reset by that block)
// merges the S partials into ctx.
struct AttnRopeArgs {
  const float *qraw, *kraw, *vraw;  // [H, hd], [hd], [hd]
  const float *qnorm, *knorm;       // [hd]
  const float2 *rope;               // (cos, sin) at the current position, [angles]
  float *kc, *vc;                   // caches [max_seq, hd]
  float *part;                      // [H][S][hd + 2]
  int *count;                       // [H * kCountStride], zero between launches
  float *ctx;                       // [H, hd]
  const int *pos_dev;
  int H, S, angles, own, sliding, window;
  float eps;
};

template <int DH>
__device__ __forceinline__ void load_halves(const float *p, int lane, float (&a)[DH],
                                            float (&b)[DH]) {
  constexpr int HALF = 64 * DH;
  if constexpr (DH == 4) {
    const float4 x = *reinterpret_cast<const float4 *>(p + lane * 4);
    const float4 z = *reinterpret_cast<const float4 *>(p + HALF + lane * 4);
    a[0] = x.x; a[1] = x.y; a[2] = x.z; a[3] = x.w;
    b[0] = z.x; b[1] = z.y; b[2] = z.z; b[3] = z.w;
  } else if constexpr (DH == 2) {
    const float2 x = *reinterpret_cast<const float2 *>(p + lane * 2);
    const float2 z = *reinterpret_cast<const float2 *>(p + HALF + lane * 2);
    a[0] = x.x; a[1] = x.y;
    b[0] = z.x; b[1] = z.y;
  } else {
    a[0] = p[lane];
    b[0] = p[HALF + lane];
  }
}

// Device-coherent buffer accesses (cache policy SC1): they bypass the L2
// state that is private to one XCD, so data handed between blocks on
// different XCDs needs no L2 writeback or invalidate.
constexpr int kSc1 = 16;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(float *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(p, 0, bytes, 0x00020000);
}

template <int N>
__device__ __forceinline__ void ld_coherent(__amdgpu_buffer_rsrc_t r, int off, float *v) {
  if constexpr (N == 4) {
    const u32x4v x = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSc1);
    v[0] = __uint_as_float(x.x); v[1] = __uint_as_float(x.y);
    v[2] = __uint_as_float(x.z); v[3] = __uint_as_float(x.w);
  } else if constexpr (N == 2) {
    const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kSc1);
    v[0] = __uint_as_float(x.x); v[1] = __uint_as_float(x.y);
  } else {
    v[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kSc1));
  }
}

__device__ __forceinline__ void st_coherent4(__amdgpu_buffer_rsrc_t r, int off, float a, float b,
                                             float c, float d) {
  const u32x4v x = {__float_as_uint(a), __float_as_uint(b), __float_as_uint(c), __float_as_uint(d)};
  __builtin_amdgcn_raw_buffer_store_b128(x, r, off, 0, kSc1);
}

template <int DH>
__device__ __forceinline__ void store_halves(float *p, int lane, const float (&a)[DH],
                                             const float (&b)[DH]) {
  constexpr int HALF = 64 * DH;
#pragma unroll
  for (int j = 0; j < DH; ++j) {
    p[lane * DH + j] = a[j];
    p[HALF + lane * DH + j] = b[j];
  }
}

// The norm weights and RoPE factors of one lane (dims lane * DH + j and
// their partners hd/2 + ...), loaded once at kernel start.
template <int DH>
struct NormRope {
  float sa[DH], sb[DH];
  float2 r[DH];
};

template <int DH, bool SCALE, bool ROPE>
__device__ __forceinline__ void load_norm_rope(NormRope<DH> &n, const float *scale,
                                               const float2 *rope, int angles, int lane) {
  constexpr int HALF = 64 * DH;
#pragma unroll
  for (int j = 0; j < DH; ++j) {
    const int t = lane * DH + j;
    if (SCALE) {
      n.sa[j] = scale[t];
      n.sb[j] = scale[HALF + t];
    }
    if (ROPE) n.r[j] = rope[t < angles ? t : (angles > 0 ? angles - 1 : 0)];
  }
}

// x = rms(x) * scale (SCALE), then (ROPE) the rotation of the pairs
// (t, t + hd/2) for t < angles: the arithmetic of rope_qkv_kernel, on
// factors loaded beforehand.
template <int DH, bool SCALE, bool ROPE>
__device__ __forceinline__ void norm_rope_wave(float (&a)[DH], float (&b)[DH],
                                               const NormRope<DH> &n, int angles, float eps,
                                               int lane) {
  constexpr int HALF = 64 * DH;
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < DH; ++j) ss += a[j] * a[j] + b[j] * b[j];
  const float inv = 1.f / sqrtf(wave_sum(ss) / (float)(2 * HALF) + eps);
#pragma unroll
  for (int j = 0; j < DH; ++j) {
    const int t = lane * DH + j;
    const float an = SCALE ? a[j] * inv * n.sa[j] : a[j] * inv;
    const float bn = SCALE ? b[j] * inv * n.sb[j] : b[j] * inv;
    if (ROPE) {
      const bool rot = t < angles;
      a[j] = rot ? an * n.r[j].x - bn * n.r[j].y : an;
      b[j] = rot ? bn * n.r[j].x + an * n.r[j].y : bn;
    } else {
      a[j] = an;
      b[j] = bn;
    }
  }
}

// SMAX: the largest split count S this instantiation merges (4 waves x SMAX/4).
template <int DH, int SMAX>
__global__ __launch_bounds__(256) void attn_rope_dec_kernel(AttnRopeArgs A) {
  constexpr int HALF = 64 * DH, HD = 2 * HALF;
  constexpr int KC = DH == 4 ? 4 : 8;  // keys per wave whose loads are in flight together
  __shared__ float wm[4], wl[4];
  __shared__ float wo[4][HD];
  __shared__ int last_sh;
  const int h = blockIdx.x / A.S, s = blockIdx.x - h * A.S;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  // Only the key range needs the position (a scalar load).  q and its norm
  // weights and RoPE factors (a table of the current position) go out first,
  // so that the q norm runs while the k/v rows are in flight; the wave that
  // builds the new key loads its k/v row and norm weights before its k/v rows.
  const int pos = *A.pos_dev;
  float qa[DH], qb[DH], na[DH], nb[DH], va[DH], vb[DH];
  load_halves<DH>(A.qraw + (size_t)h * HD, lane, qa, qb);
  NormRope<DH> qn, kn;
  load_norm_rope<DH, true, true>(qn, A.qnorm, A.rope, A.angles, lane);
  int lo = A.sliding ? pos - A.window + 1 : 0;
  lo = lo > 0 ? lo : 0;
  const int kps = (pos - lo + A.S) / A.S;  // ceil((pos - lo + 1) / S)
  const int k0 = lo + s * kps;
  const int k1 = k0 + kps < pos + 1 ? k0 + kps : pos + 1;  // [k0, k1), maybe empty
  // the new key at pos (own-KV layers): built by the wave that owns it
  const bool has_new = A.own && k0 <= pos && pos < k1 && ((pos - k0) & 3) == wave;
  if (has_new) {
    load_halves<DH>(A.kraw, lane, na, nb);
    load_halves<DH>(A.vraw, lane, va, vb);
    load_norm_rope<DH, true, false>(kn, A.knorm, nullptr, 0, lane);
#pragma unroll
    for (int j = 0; j < DH; ++j) kn.r[j] = qn.r[j];
  }

  // k/v rows of the wave's first KC keys (clamped to valid rows; keys past k1
  // are not used)
  float ka[KC][DH], kb[KC][DH], xa[KC][DH], xb[KC][DH];
  int base = k0 + wave;
  auto load_chunk = [&](int b0) {
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      int key = b0 + 4 * c;
      key = key < k1 ? key : k1 - 1;
      load_halves<DH>(A.kc + (size_t)key * HD, lane, ka[c], kb[c]);
      load_halves<DH>(A.vc + (size_t)key * HD, lane, xa[c], xb[c]);
    }
  };
  load_chunk(base);

  norm_rope_wave<DH, true, true>(qa, qb, qn, A.angles, A.eps, lane);

  if (has_new) {
    norm_rope_wave<DH, true, true>(na, nb, kn, A.angles, A.eps, lane);
    norm_rope_wave<DH, false, false>(va, vb, kn, 0, A.eps, lane);
    if (h == 0) {
      store_halves<DH>(A.kc + (size_t)pos * HD, lane, na, nb);
      store_halves<DH>(A.vc + (size_t)pos * HD, lane, va, vb);
    }
  }

  float m = -1e30f, l = 0.f, oa[DH], ob[DH];
#pragma unroll
  for (int j = 0; j < DH; ++j) oa[j] = ob[j] = 0.f;
  for (;;) {  // one chunk of up to KC keys per pass (an empty chunk changes nothing)
    float d[KC];
    float mc = m;
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      const int key = base + 4 * c;
      if (has_new && key == pos) {
#pragma unroll
        for (int j = 0; j < DH; ++j) {
          ka[c][j] = na[j]; kb[c][j] = nb[j];
          xa[c][j] = va[j]; xb[c][j] = vb[j];
        }
      }
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < DH; ++j) acc = fmaf(qb[j], kb[c][j], fmaf(qa[j], ka[c][j], acc));
      d[c] = wave_sum(acc);
      if (key < k1) mc = fmaxf(mc, d[c]);
    }
    const float corr = expf(m - mc);
    l *= corr;
#pragma unroll
    for (int j = 0; j < DH; ++j) {
      oa[j] *= corr;
      ob[j] *= corr;
    }
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      const int key = base + 4 * c;
      if (key >= k1) break;  // wave-uniform; the clamped rows are not used
      const float p = expf(d[c] - mc);
      l += p;
#pragma unroll
      for (int j = 0; j < DH; ++j) {
        oa[j] = fmaf(p, xa[c][j], oa[j]);
        ob[j] = fmaf(p, xb[c][j], ob[j]);
      }
    }
    m = mc;
    base += 4 * KC;
    if (base >= k1) break;
    load_chunk(base);
  }

  // merge the 4 waves, write the block's partial
  if (lane == 0) {
    wm[wave] = m;
    wl[wave] = l;
  }
#pragma unroll
  for (int j = 0; j < DH; ++j) {
    wo[wave][lane * DH + j] = oa[j];
    wo[wave][HALF + lane * DH + j] = ob[j];
  }
  __syncthreads();
  const float M = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
  const float e0 = expf(wm[0] - M), e1 = expf(wm[1] - M), e2 = expf(wm[2] - M),
              e3 = expf(wm[3] - M);
  // The partials cross XCDs (whose L2s are not coherent with each other):
  // they are written and read with device-coherent accesses, so that no L2
  // writeback or invalidate (a fence) is needed around the counter.
  // Partial of split s: [max, sum, 0, 0, output[HD]] (stride HD + 4 floats).
  constexpr int stride = HD + 4;
  const __amdgpu_buffer_rsrc_t pr =
      coherent_rsrc(A.part + (size_t)h * A.S * stride, (uint32_t)(A.S * stride * 4));
  const int pbase = s * stride * 4;
  if (t < HD / 4) {
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int dd = 4 * t + j;
      v[j] = wo[0][dd] * e0 + wo[1][dd] * e1 + wo[2][dd] * e2 + wo[3][dd] * e3;
    }
    st_coherent4(pr, pbase + 16 + 16 * t, v[0], v[1], v[2], v[3]);
  } else if (t == HD / 4) {
    st_coherent4(pr, pbase, M, wl[0] * e0 + wl[1] * e1 + wl[2] * e2 + wl[3] * e3, 0.f, 0.f);
  }

  // the last block of head h merges the S partials
  __builtin_amdgcn_s_waitcnt(0);  // this wave's coherent stores are performed
  __syncthreads();
  if (t == 0)
    last_sh = __hip_atomic_fetch_add(&A.count[h * kCountStride], 1, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT) == A.S - 1;
  __syncthreads();
  if (!last_sh) return;
  // wave w merges splits w, w + 4, ... (up to SMAX / 4 each, all loads in
  // flight together; lanes hold the dims as above), then the 4 waves merge
  // in LDS
  constexpr int SW = SMAX / 4;  // splits per wave
  float pm[SW], pl[SW], pa[SW][DH], pb[SW][DH];
#pragma unroll
  for (int i = 0; i < SW; ++i) {
    int j = wave + 4 * i;
    j = j < A.S ? j : A.S - 1;
    const int pj = j * stride * 4;
    float ml[2];
    ld_coherent<2>(pr, pj, ml);
    pm[i] = ml[0];
    pl[i] = ml[1];
    ld_coherent<DH>(pr, pj + 16 + 4 * lane * DH, pa[i]);
    ld_coherent<DH>(pr, pj + 16 + 4 * (HALF + lane * DH), pb[i]);
  }
  float mw = -1e30f;
#pragma unroll
  for (int i = 0; i < SW; ++i) mw = fmaxf(mw, wave + 4 * i < A.S ? pm[i] : -1e30f);
  float lw = 0.f;
#pragma unroll
  for (int j = 0; j < DH; ++j) oa[j] = ob[j] = 0.f;
#pragma unroll
  for (int i = 0; i < SW; ++i) {
    // splits past S re-read split S - 1 and weigh 0: no load waits in a branch
    const float w = wave + 4 * i < A.S ? expf(pm[i] - mw) : 0.f;
    lw = fmaf(w, pl[i], lw);
#pragma unroll
    for (int j = 0; j < DH; ++j) {
      oa[j] = fmaf(w, pa[i][j], oa[j]);
      ob[j] = fmaf(w, pb[i][j], ob[j]);
    }
  }
  if (lane == 0) {  // wm/wl/wo were last read before the barriers above
    wm[wave] = mw;
    wl[wave] = lw;
  }
#pragma unroll
  for (int j = 0; j < DH; ++j) {
    wo[wave][lane * DH + j] = oa[j];
    wo[wave][HALF + lane * DH + j] = ob[j];
  }
  __syncthreads();
  {
    const float Mx = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
    const float f0 = expf(wm[0] - Mx), f1 = expf(wm[1] - Mx), f2 = expf(wm[2] - Mx),
                f3 = expf(wm[3] - Mx);
    const float L = wl[0] * f0 + wl[1] * f1 + wl[2] * f2 + wl[3] * f3;
    for (int dd = t; dd < HD; dd += 256)
      A.ctx[(size_t)h * HD + dd] =
          (wo[0][dd] * f0 + wo[1][dd] * f1 + wo[2][dd] * f2 + wo[3][dd] * f3) / L;
  }
  if (t == 0) A.count[h * kCountStride] = 0;
}

// ---- standalone chain r = (h + rms(a) * w1) * c; x = rms(r) * w2 ------------
// One block per row; writes r (if r_out) and x (if x_out; without x_out, r_out
// is required and w2 is not read).  a is the sum of a_parts planes a_stride
// floats apart, added in order (a GEMM's K slices).
__global__ __launch_bounds__(256) void norm_chain_kernel(const float *__restrict__ a,
                                                         int a_parts, size_t a_stride,
                                                         const float *__restrict__ h,
                                                         const float *__restrict__ w1,
                                                         const float *__restrict__ w2, float c,
                                                         float eps, int width,
                                                         float *__restrict__ r_out,
                                                         float *__restrict__ x_out) {
  __shared__ float red[16];
  const size_t off = (size_t)blockIdx.x * width;
  constexpr int U = 8;
  if (width <= 256 * U) {
    // every load first (indices past width re-read the last element and are
    // left out of the sums and stores)
    float av[U], hv[U], w1v[U], w2v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int i = threadIdx.x + 256 * u;
      i = i < width ? i : width - 1;
      av[u] = a[off + i];
      for (int s = 1; s < a_parts; ++s) av[u] += a[s * a_stride + off + i];
      hv[u] = h[off + i];
      w1v[u] = w1[i];
      w2v[u] = x_out ? w2[i] : 0.f;
    }
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (threadIdx.x + 256 * u < width) ss += av[u] * av[u];
    const float inv1 = 1.f / sqrtf(fblock_sum(ss, red, 4) / (float)width + eps);
    float r[U], ss2 = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      r[u] = (hv[u] + av[u] * inv1 * w1v[u]) * c;
      if (threadIdx.x + 256 * u < width) ss2 += r[u] * r[u];
    }
    if (!x_out) {  // the residual alone
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (threadIdx.x + 256 * u < width) r_out[off + threadIdx.x + 256 * u] = r[u];
      return;
    }
    const float inv2 = 1.f / sqrtf(fblock_sum(ss2, red + 4, 4) / (float)width + eps);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = threadIdx.x + 256 * u;
      if (i < width) {
        if (r_out) r_out[off + i] = r[u];
        x_out[off + i] = r[u] * inv2 * w2v[u];
      }
    }
    return;
  }
  auto a_at = [&](int i) {
    float v = a[off + i];
    for (int s = 1; s < a_parts; ++s) v += a[s * a_stride + off + i];
    return v;
  };
  float ss = 0.f;
  for (int i = threadIdx.x; i < width; i += 256) ss += a_at(i) * a_at(i);
  const float inv1 = 1.f / sqrtf(fblock_sum(ss, red, 4) / (float)width + eps);
  float ss2 = 0.f;
  for (int i = threadIdx.x; i < width; i += 256) {
    const float r = (h[off + i] + a_at(i) * inv1 * w1[i]) * c;
    if (r_out) r_out[off + i] = r;
    ss2 += r * r;
  }
  if (!x_out) return;
  const float inv2 = 1.f / sqrtf(fblock_sum(ss2, red, 4) / (float)width + eps);
  for (int i = threadIdx.x; i < width; i += 256) {
    const float r = (h[off + i] + a_at(i) * inv1 * w1[i]) * c;
    x_out[off + i] = r * inv2 * w2[i];
  }
}

// Block maximum; all threads get it.  red: >= 4 floats, not reused by the
// next call before a barrier.
__device__ __forceinline__ float fblock_max(float v, float *red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}


// norm_chain_kernel's chain for a row of up to 2048 values (a multiple of 8)
// with the prefill GEMM's x pre-pass of its output fused in: the GEMM input
// (x = rms(r) * w2, or r itself without w2) leaves as x' for the GEMM that
// follows - per row the exponent xe (max |x * 2^-xe| in [2^13, 2^14), 0 for
// an all-zero or non-finite row), per 8-value chunk c the FP16 pairs (0,4)
// (1,5) (2,6) (3,7) of x * 2^-xe (hi) and of the rounding remainders (lo) at
// xt[c * Mp + row] and xt[(width / 8 + c) * Mp + row].  r_out and x_out (FP32)
// are optional.
//
// One wave per row, one row per block: lane l holds whole chunks l, l + 64,
// ... (up to 4), so the norms and the maximum are wave reductions (no
// barrier) and each chunk is converted where it was loaded.  Blocks are
// dealt to the 8 XCDs round-robin; rows go to them in runs of Mp / 8, so the
// 8 rows that share each 128-byte line of xt[c][m] are written through one
// XCD's L2.  Grid: Mp blocks of 64 threads (Mp a multiple of 32); rows past
// `rows` write zero chunks.
// CPL: chunks per lane, ceil(width / 512) (up to kChainCpl: width <= 2048), so
// no lane loads a chunk past the row.
constexpr int kChainCpl = 4;
template <int CPL>
__global__ __launch_bounds__(64) void norm_chain_xprep_kernel(
    const float *__restrict__ a, int a_parts, size_t a_stride, const float *__restrict__ h,
    const float *__restrict__ w1, const float *__restrict__ w2, float c, float eps, int width,
    int rows, float *__restrict__ r_out, float *__restrict__ x_out, uint4 *__restrict__ xt,
    int *__restrict__ xe, int Mp) {
  const int lane = threadIdx.x & 63;
  // (4-row blocks left half of the CUs idle at 512 rows and gave each busy
  // CU four rows of loads: E2B prefill of 512 tokens 9.69-9.72 -> 9.63-9.66 ms)
  const int row = (blockIdx.x & 7) * (Mp >> 3) + (blockIdx.x >> 3);
  const int nch = width >> 3;
  const size_t lo_plane = (size_t)nch * Mp;
  if (row >= rows) {
    for (int ch = lane; ch < nch; ch += 64) {
      xt[(size_t)ch * Mp + row] = make_uint4(0u, 0u, 0u, 0u);
      xt[lo_plane + (size_t)ch * Mp + row] = make_uint4(0u, 0u, 0u, 0u);
    }
    return;
  }
  const size_t off = (size_t)row * width;
  // every load first (chunks past the row re-read chunk 0 and are left out)
  float av[CPL][8], hv[CPL][8], w1v[CPL][8], w2v[CPL][8];
#pragma unroll
  for (int u = 0; u < CPL; ++u) {
    int ch = lane + 64 * u;
    ch = ch < nch ? ch : 0;
    load8(a + off, ch, av[u]);
    load8(h + off, ch, hv[u]);
    load8(w1, ch, w1v[u]);
    if (w2) load8(w2, ch, w2v[u]);
  }
  // the other partial planes, added in order, two at a time: both planes'
  // loads go out together (past a_parts plane sp0 is re-read), so a pair
  // costs one memory round trip instead of two.  (E2B prefill of 512
  // tokens: 9.80 -> 9.60 ms; four at a time, 256 registers and one wave per
  // SIMD, 9.64 ms.)
  for (int sp0 = 1; sp0 < a_parts; sp0 += 2) {
    float t[2][CPL][8];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int sp = sp0 + b < a_parts ? sp0 + b : sp0;
#pragma unroll
      for (int u = 0; u < CPL; ++u) {
        int ch = lane + 64 * u;
        ch = ch < nch ? ch : 0;
        load8(a + sp * a_stride + off, ch, t[b][u]);
      }
    }
#pragma unroll
    for (int b = 0; b < 2; ++b)
      if (sp0 + b < a_parts)
#pragma unroll
        for (int u = 0; u < CPL; ++u)
#pragma unroll
          for (int q = 0; q < 8; ++q) av[u][q] += t[b][u][q];
  }
  float ss = 0.f;
#pragma unroll
  for (int u = 0; u < CPL; ++u)
    if (lane + 64 * u < nch)
#pragma unroll
      for (int q = 0; q < 8; ++q) ss += av[u][q] * av[u][q];
  const float inv1 = 1.f / sqrtf(wave_sum(ss) / (float)width + eps);
  float r[CPL][8], ss2 = 0.f;
#pragma unroll
  for (int u = 0; u < CPL; ++u)
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      r[u][q] = (hv[u][q] + av[u][q] * inv1 * w1v[u][q]) * c;
      if (lane + 64 * u < nch) ss2 += r[u][q] * r[u][q];
    }
  float xv[CPL][8];
  if (w2) {
    const float inv2 = 1.f / sqrtf(wave_sum(ss2) / (float)width + eps);
#pragma unroll
    for (int u = 0; u < CPL; ++u)
#pragma unroll
      for (int q = 0; q < 8; ++q) xv[u][q] = r[u][q] * inv2 * w2v[u][q];
  } else {
#pragma unroll
    for (int u = 0; u < CPL; ++u)
#pragma unroll
      for (int q = 0; q < 8; ++q) xv[u][q] = r[u][q];
  }
  float mx = 0.f;
#pragma unroll
  for (int u = 0; u < CPL; ++u) {
    const int ch = lane + 64 * u;
    if (ch >= nch) continue;
    float4 *ro = r_out ? reinterpret_cast<float4 *>(r_out + off) + 2 * ch : nullptr;
    float4 *xo = x_out ? reinterpret_cast<float4 *>(x_out + off) + 2 * ch : nullptr;
    if (ro) {
      ro[0] = make_float4(r[u][0], r[u][1], r[u][2], r[u][3]);
      ro[1] = make_float4(r[u][4], r[u][5], r[u][6], r[u][7]);
    }
    if (xo) {
      xo[0] = make_float4(xv[u][0], xv[u][1], xv[u][2], xv[u][3]);
      xo[1] = make_float4(xv[u][4], xv[u][5], xv[u][6], xv[u][7]);
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) mx = fmaxf(mx, fabsf(xv[u][q]));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  const int e = mx > 0.f && mx <= 3.4e38f ? ilogbf(mx) - 13 : 0;
  if (lane == 0) xe[row] = e;
#pragma unroll
  for (int u = 0; u < CPL; ++u) {
    const int ch = lane + 64 * u;
    if (ch >= nch) continue;
    _Float16 hh[8], ll[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float sv = ldexpf(xv[u][q], -e);
      hh[q] = (_Float16)sv;
      ll[q] = (_Float16)(sv - (float)hh[q]);
    }
    xt[(size_t)ch * Mp + row] = make_uint4(half2_bits(hh[0], hh[4]), half2_bits(hh[1], hh[5]),
                                           half2_bits(hh[2], hh[6]), half2_bits(hh[3], hh[7]));
    xt[lo_plane + (size_t)ch * Mp + row] =
        make_uint4(half2_bits(ll[0], ll[4]), half2_bits(ll[1], ll[5]), half2_bits(ll[2], ll[6]),
                   half2_bits(ll[3], ll[7]));
  }
}

// The PLE gate's product gelu(gate) * ple (gelu_ple_kernel) with the PLE
// projection GEMM's x pre-pass fused in, written as in norm_chain_xprep_kernel
// (exponent per row, FP16 hi/lo chunks at xt[c * Mp + row] and
// xt[(width / 8 + c) * Mp + row]); y (FP32) is optional.  The gate arrives
// as the gate GEMM's K slices, `parts` planes pstride floats apart, added in
// slice order as gemm_splitk_sum_kernel adds them, so y and x' equal those
// of the three kernels this replaces.  One wave per row and one row per
// block (rows to the XCDs in runs of Mp / 8); lane l owns chunk l, so width
// is at most 512.  Rows past `rows` write zero chunks.
constexpr int kPleMaxParts = 8;
__global__ __launch_bounds__(64) void gelu_ple_xprep_kernel(
    const float *__restrict__ gate, int parts, size_t pstride, const float *__restrict__ ple,
    int layer, int layers, int width, int rows, float *__restrict__ y, uint4 *__restrict__ xt,
    int *__restrict__ xe, int Mp) {
  const int lane = threadIdx.x;
  const int row = (blockIdx.x & 7) * (Mp >> 3) + (blockIdx.x >> 3);
  const int nch = width >> 3;
  const size_t lo_plane = (size_t)nch * Mp;
  if (row >= rows) {
    if (lane < nch) {
      xt[(size_t)lane * Mp + row] = make_uint4(0u, 0u, 0u, 0u);
      xt[lo_plane + (size_t)lane * Mp + row] = make_uint4(0u, 0u, 0u, 0u);
    }
    return;
  }
  const bool live = lane < nch;
  const int ch = live ? lane : 0;  // idle lanes re-read chunk 0 and are left out
  const size_t off = (size_t)row * width;
  // every load first: the slices (past `parts`, slice 0 again) and the ple row
  float g[kPleMaxParts][8], pv[8];
#pragma unroll
  for (int sp = 0; sp < kPleMaxParts; ++sp)
    load8(gate + (size_t)(sp < parts ? sp : 0) * pstride + off, ch, g[sp]);
  load8(ple + ((size_t)row * layers + layer) * width, ch, pv);
#pragma unroll
  for (int sp = 1; sp < kPleMaxParts; ++sp)
    if (sp < parts)
#pragma unroll
      for (int q = 0; q < 8; ++q) g[0][q] += g[sp][q];
  float v[8], mx = 0.f;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    v[q] = gelu_tanh(g[0][q]) * pv[q];
    mx = fmaxf(mx, live ? fabsf(v[q]) : 0.f);
  }
  if (y && live) {
    float4 *yo = reinterpret_cast<float4 *>(y + off) + 2 * ch;
    yo[0] = make_float4(v[0], v[1], v[2], v[3]);
    yo[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  const int e = mx > 0.f && mx <= 3.4e38f ? ilogbf(mx) - 13 : 0;
  if (lane == 0) xe[row] = e;
  if (!live) return;
  _Float16 hh[8], ll[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const float sv = ldexpf(v[q], -e);
    hh[q] = (_Float16)sv;
    ll[q] = (_Float16)(sv - (float)hh[q]);
  }
  xt[(size_t)ch * Mp + row] = make_uint4(half2_bits(hh[0], hh[4]), half2_bits(hh[1], hh[5]),
                                         half2_bits(hh[2], hh[6]), half2_bits(hh[3], hh[7]));
  xt[lo_plane + (size_t)ch * Mp + row] =
      make_uint4(half2_bits(ll[0], ll[4]), half2_bits(ll[1], ll[5]), half2_bits(ll[2], ll[6]),
                 half2_bits(ll[3], ll[7]));
}

}  // namespace

// ---- launchers used by the engine --------------------------------------------

// y_i = W_i . rms(a) * w1 for up to three weights sharing the input (q, k, v).
int fused_norm_linear(const float *a, const float *w1, float eps, const g4_w4 *const *w,
                      float *const *y, int n) {
  FusedArgs f = {};
  f.nseg = n;
  for (int i = 0; i < n; ++i) f.seg[i] = seg_of(w[i], y[i]);
  f.a = a;
  f.w1 = w1;
  f.eps = eps;
  f.K = w[0]->K;
  return launch_fused<kProNorm, kEpiNone>(f);
}

// r = (h + rms(a) * w1) * c (written to r_out); y_i = W_i . rms(r) * w2.
int fused_res_norm_linear(const float *a, const float *h, const float *w1, float c,
                          const float *w2, float eps, float *r_out, const g4_w4 *const *w,
                          float *const *y, int n) {
  FusedArgs f = {};
  f.nseg = n;
  for (int i = 0; i < n; ++i) f.seg[i] = seg_of(w[i], y[i]);
  f.a = a;
  f.h = h;
  f.w1 = w1;
  f.w2 = w2;
  f.c = c;
  f.eps = eps;
  f.r_out = r_out;
  f.K = w[0]->K;
  return launch_fused<kProResNorm, kEpiNone>(f);
}

// r = (h + rms(a) * w1) * c; x = rms(r) * w2; act = gelu(Wg . x) * (Wu . x).
int fused_res_norm_gate_up(const float *a, const float *h, const float *w1, float c,
                           const float *w2, float eps, float *r_out, const g4_w4 *gate,
                           const g4_w4 *up, float *act) {
  FusedArgs f = {};
  f.nseg = 2;
  f.seg[0] = seg_of(gate, act);
  f.seg[1] = seg_of(up, act);
  f.a = a;
  f.h = h;
  f.w1 = w1;
  f.w2 = w2;
  f.c = c;
  f.eps = eps;
  f.r_out = r_out;
  f.K = gate->K;
  return launch_fused<kProResNorm, kEpiGeluUp>(f);
}

// r = h + rms(a) * w1 (written to r_out); y = gelu(W . r) * mul.  a is the
// sum of a_parts vectors of W's input width, added in order.
int fused_res_linear_gelu_mul(const float *a, int a_parts, const float *h, const float *w1,
                              float eps, float *r_out, const g4_w4 *w, const float *mul,
                              float *y) {
  if (a_parts < 1 || a_parts > kMaxParts)
    return fail(G4_E_ARG, "fused PLE gate: %d partial inputs (1..%d)", a_parts, kMaxParts);
  FusedArgs f = {};
  f.nseg = 1;
  f.seg[0] = seg_of(w, y);
  f.a = a;
  f.a_parts = a_parts;
  f.h = h;
  f.w1 = w1;
  f.c = 1.f;
  f.eps = eps;
  f.r_out = r_out;
  f.mul = mul;
  f.K = w->K;
  return launch_fused<kProRes, kEpiGeluMul>(f);
}

int launch_rope_qkv(const float *qraw, const float *kraw, const float *vraw, int heads, int hd,
                    const int *pos_dev, const float *qnorm, const float *knorm, int rope_angles,
                    float base, float eps, float *q, float *kc, float *vc, bool own_kv) {
  if (hd > 512 || hd % 2) return fail(G4_E_ARG, "rope_qkv: head_dim %d", hd);
  hipLaunchKernelGGL(rope_qkv_kernel, dim3(heads + (own_kv ? 2 : 0)), dim3(256), 0, stream(),
                     qraw, kraw, vraw, heads, hd, pos_dev, qnorm, knorm, rope_angles, base, eps,
                     q, kc, vc);
  G4_LAUNCH_CHECK("rope_qkv_kernel");
  return G4_OK;
}

int launch_token_start(const uint16_t *E, int vocab, int width, const int *ids_dev, float scale,
                       float *y, const int *pos_dev, const RopeSlots &slots, float2 *tab) {
  if (slots.n < 0 || slots.n > kRopeSlots) return fail(G4_E_ARG, "token start: %d RoPE tables", slots.n);
  for (int j = 0; j < slots.n; ++j)
    if (slots.angles[j] > kRopeTable) return fail(G4_E_ARG, "token start: %d RoPE angles", slots.angles[j]);
  hipLaunchKernelGGL(token_start_kernel, dim3(1 + slots.n), dim3(256), 0, stream(), E, vocab,
                     width, ids_dev, scale, y, pos_dev, slots, tab);
  G4_LAUNCH_CHECK("token_start_kernel");
  return G4_OK;
}

// About 32 keys per block, in multiples of 8 splits, 8 to 32: past 32 splits
// the last block's merge (more than 8 partials per wave) costs more than the
// longer key loops save (hd 512 at 1000 keys: 7.7 us at 32 splits, 10.4 at 64).
int attn_rope_splits(int max_keylen, bool sliding, int window) {
  const int span = sliding && window < max_keylen ? window : max_keylen;
  int S = (span + 31) / 32;
  S = (S + 7) / 8 * 8;
  return S < 8 ? 8 : S > 32 ? 32 : S;
}

bool attn_rope_supported(int hd) { return hd == 128 || hd == 256 || hd == 512; }

int launch_attn_rope_dec(const float *qraw, const float *kraw, const float *vraw, int heads,
                         int hd, const int *pos_dev, const float *qnorm, const float *knorm,
                         const float2 *rope, int angles, float eps, float *kc, float *vc,
                         bool own_kv, bool sliding, int window, int max_keylen, float *part,
                         size_t part_floats, int *count, float *ctx) {
  AttnRopeArgs a;
  a.qraw = qraw;
  a.kraw = kraw;
  a.vraw = vraw;
  a.qnorm = qnorm;
  a.knorm = knorm;
  a.rope = rope;
  a.kc = kc;
  a.vc = vc;
  a.part = part;
  a.count = count;
  a.ctx = ctx;
  a.pos_dev = pos_dev;
  a.H = heads;
  a.S = attn_rope_splits(max_keylen, sliding, window);
  a.angles = angles;
  a.own = own_kv ? 1 : 0;
  a.sliding = sliding ? 1 : 0;
  a.window = window;
  a.eps = eps;
  if ((size_t)heads * a.S * ((size_t)hd + 4) > part_floats)
    return fail(G4_E_ARG, "decode attention: split scratch too small");
  if (angles > hd / 2 || angles > kRopeTable) return fail(G4_E_ARG, "decode attention: %d angles", angles);
  const dim3 grid(heads * a.S);
#define G4_ATTN(DH)                                                                       \
  do {                                                                                    \
    if (a.S <= 8)                                                                         \
      hipLaunchKernelGGL((attn_rope_dec_kernel<DH, 8>), grid, dim3(256), 0, stream(), a);  \
    else if (a.S <= 16)                                                                   \
      hipLaunchKernelGGL((attn_rope_dec_kernel<DH, 16>), grid, dim3(256), 0, stream(), a); \
    else                                                                                  \
      hipLaunchKernelGGL((attn_rope_dec_kernel<DH, 32>), grid, dim3(256), 0, stream(), a); \
  } while (0)
  switch (hd) {
    case 128: G4_ATTN(1); break;
    case 256: G4_ATTN(2); break;
    case 512: G4_ATTN(4); break;
    default: return fail(G4_E_ARG, "decode attention: head_dim %d", hd);
  }
#undef G4_ATTN
  G4_LAUNCH_CHECK("attn_rope_dec_kernel");
  return G4_OK;
}

int launch_norm_chain(const float *a, const float *h, const float *w1, const float *w2, float c,
                      float eps, int rows, int width, float *r_out, float *x_out, int a_parts,
                      size_t a_stride) {
  if (rows == 0) return G4_OK;
  hipLaunchKernelGGL(norm_chain_kernel, dim3(rows), dim3(256), 0, stream(), a, a_parts, a_stride,
                     h, w1, w2, c, eps, width, r_out, x_out);
  G4_LAUNCH_CHECK("norm_chain_kernel");
  return G4_OK;
}

int launch_norm_chain_xprep(const float *a, int a_parts, size_t a_stride, const float *h,
                            const float *w1, const float *w2, float c, float eps, int rows,
                            int width, float *r_out, float *x_out, void *xt, int *xe, int Mp) {
  if (width > 64 * kChainCpl * 8 || width % 8 || rows > Mp || Mp % 32)
    return fail(G4_E_ARG, "norm chain with x pre-pass: width %d (<= 2048, multiple of 8), "
                "rows %d <= %d (a multiple of 32)", width, rows, Mp);
  const int cpl = (width / 8 + 63) / 64;
  auto kernel = cpl == 1   ? norm_chain_xprep_kernel<1>
                : cpl == 2 ? norm_chain_xprep_kernel<2>
                : cpl == 3 ? norm_chain_xprep_kernel<3>
                           : norm_chain_xprep_kernel<4>;
  hipLaunchKernelGGL(kernel, dim3(Mp), dim3(64), 0, stream(), a, a_parts, a_stride, h, w1, w2, c,
                     eps, width, rows, r_out, x_out, static_cast<uint4 *>(xt), xe, Mp);
  G4_LAUNCH_CHECK("norm_chain_xprep_kernel");
  return G4_OK;
}

bool gelu_ple_xprep_fits(int width, int parts) {
  return width % 8 == 0 && width > 0 && width <= 512 && parts >= 1 && parts <= kPleMaxParts;
}

int launch_gelu_ple_xprep(const float *gate, int parts, size_t pstride, const float *ple,
                          int layer, int layers, int width, int rows, float *y, void *xt,
                          int *xe, int Mp) {
  if (!gelu_ple_xprep_fits(width, parts) || rows > Mp || Mp % 32)
    return fail(G4_E_ARG, "gelu·ple with x pre-pass: width %d (<= 512, multiple of 8), %d "
                "gate slices (<= %d), rows %d <= %d (a multiple of 32)", width, parts,
                kPleMaxParts, rows, Mp);
  hipLaunchKernelGGL(gelu_ple_xprep_kernel, dim3(Mp), dim3(64), 0, stream(), gate, parts,
                     pstride, ple, layer, layers, width, rows, y, static_cast<uint4 *>(xt), xe,
                     Mp);
  G4_LAUNCH_CHECK("gelu_ple_xprep_kernel");
  return G4_OK;
}

}  // namespace g4
