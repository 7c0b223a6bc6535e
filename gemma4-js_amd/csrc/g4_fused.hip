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
    s[i] = ws[idx];
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
  const int wave = t >> 6, lane = t & 63;
  const int pw = ((nch + 63) >> 6) < nwaves ? ((nch + 63) >> 6) : nwaves;
  const bool pro = wave < pw;  // uniform per wave
  const int cstride = 64 * pw;
  constexpr int XI = (GC && TC) ? (4 * GC + 63) / 64 <= TC / 64 ? 1 : (4 * GC + TC - 1) / TC : IPL;

  // 1. activation chunks, issued before the weight stream
  float av[XI][8], hv[XI][8], w1v[XI][8], w2v[XI][8];
  if (pro) {
#pragma unroll
    for (int i = 0; i < XI; ++i) {
      const int ct = t + i * cstride;
      const int cc = ct < nch ? ct : nch - 1;
      load8(A.a, cc, av[i]);
      if (PRO != kProNone) load8(A.w1, cc, w1v[i]);
      if (PRO == kProRes || PRO == kProResNorm) load8(A.h, cc, hv[i]);
      if (PRO == kProResNorm) load8(A.w2, cc, w2v[i]);
    }
  }

  // 2. weights of all the block's row groups (groups past the last re-read it
  // and store nothing; rows past N re-read the last group)
  uint4 q[IT][IPL];
  uint32_t s[IT][IPL];
#pragma unroll
  for (int k = 0; k < IT; ++k) {
    const int rg = blockIdx.x + k * (int)gridDim.x;
    load_rows<IPL, EPI>(A, rg < ngroups ? rg : ngroups - 1, G, RB, T, t, q[k], s[k]);
  }

  // 3. prologue
  constexpr int CH = 2;  // FP32 activations: hi and lo
  uint4 *hi = lds;
  uint4 *lo = lds + 4 * G;
  float *sx = reinterpret_cast<float *>(lds + 4 * G * CH);
  float *part = sx + G;              // [IT * RB][G]
  float *rs = part + IT * RB * G;    // row sums [IT * RB] (kEpiGeluUp)
  float *red = rs + IT * RB;         // 2 x 16 wave sums
  // Everything element-wise stays inside `if (pro)`; the reductions are
  // called by every wave.
  float xv[XI][8];
  if (PRO == kProNone) {
    if (pro) {
#pragma unroll
      for (int i = 0; i < XI; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[i][e] = av[i][e];
    }
  } else {
    float ss = 0.f;
    if (pro) {
#pragma unroll
      for (int i = 0; i < XI; ++i)
        if (t + i * cstride < nch)
#pragma unroll
          for (int e = 0; e < 8; ++e) ss += av[i][e] * av[i][e];
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
          for (int e = 0; e < 8; ++e) xv[i][e] = av[i][e] * inv1 * w1v[i][e];
      } else {
#pragma unroll
        for (int i = 0; i < XI; ++i)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            r[i][e] = (hv[i][e] + av[i][e] * inv1 * w1v[i][e]) * A.c;
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
          for (int e = 0; e < 8; ++e) xv[i][e] = r[i][e] * inv2 * w2v[i][e];
      }
    }
  }

  // 4. stage x: hi/lo bf16 pairs per chunk, 136 * group sum
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

  // 5. one partial per group, for every row group of the block
  uint32_t mask = 0x000F000Fu;
  asm volatile("" : "+v"(mask));  // keep the mask in a VGPR: lets v_and_or_b32 take the magic
#pragma unroll
  for (int k = 0; k < IT; ++k)
#pragma unroll
    for (int i = 0; i < IPL; ++i) {
      const int li = t + i * T;
      const int g = li % G;
      const uint32_t wd[4] = {q[k][i].x, q[k][i].y, q[k][i].z, q[k][i].w};
      float d0 = 0.f, d1 = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t p0 = (wd[c] & mask) | kPairMagic;
        const uint32_t p1 = ((wd[c] >> 4) & mask) | kPairMagic;
        const uint32_t p2 = ((wd[c] >> 8) & mask) | kPairMagic;
        const uint32_t p3 = ((wd[c] >> 12) & mask) | kPairMagic;
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

template <int PRO, int EPI>
int launch_fused(FusedArgs a) {
  const int G = a.K / 32;
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

// ---- standalone chain r = (h + rms(a) * w1) * c; x = rms(r) * w2 ------------
// One block per row; writes r (if r_out) and x.
__global__ __launch_bounds__(256) void norm_chain_kernel(const float *__restrict__ a,
                                                         const float *__restrict__ h,
                                                         const float *__restrict__ w1,
                                                         const float *__restrict__ w2, float c,
                                                         float eps, int width,
                                                         float *__restrict__ r_out,
                                                         float *__restrict__ x_out) {
  __shared__ float red[16];
  const size_t off = (size_t)blockIdx.x * width;
  float ss = 0.f;
  for (int i = threadIdx.x; i < width; i += 256) ss += a[off + i] * a[off + i];
  const float inv1 = 1.f / sqrtf(fblock_sum(ss, red, 4) / (float)width + eps);
  float ss2 = 0.f;
  for (int i = threadIdx.x; i < width; i += 256) {
    const float r = (h[off + i] + a[off + i] * inv1 * w1[i]) * c;
    if (r_out) r_out[off + i] = r;
    ss2 += r * r;
  }
  const float inv2 = 1.f / sqrtf(fblock_sum(ss2, red, 4) / (float)width + eps);
  for (int i = threadIdx.x; i < width; i += 256) {
    const float r = (h[off + i] + a[off + i] * inv1 * w1[i]) * c;
    x_out[off + i] = r * inv2 * w2[i];
  }
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

// r = h + rms(a) * w1 (written to r_out); y = gelu(W . r) * mul.
int fused_res_linear_gelu_mul(const float *a, const float *h, const float *w1, float eps,
                              float *r_out, const g4_w4 *w, const float *mul, float *y) {
  FusedArgs f = {};
  f.nseg = 1;
  f.seg[0] = seg_of(w, y);
  f.a = a;
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

int launch_norm_chain(const float *a, const float *h, const float *w1, const float *w2, float c,
                      float eps, int rows, int width, float *r_out, float *x_out) {
  if (rows == 0) return G4_OK;
  hipLaunchKernelGGL(norm_chain_kernel, dim3(rows), dim3(256), 0, stream(), a, h, w1, w2, c, eps,
                     width, r_out, x_out);
  G4_LAUNCH_CHECK("norm_chain_kernel");
  return G4_OK;
}

}  // namespace g4
