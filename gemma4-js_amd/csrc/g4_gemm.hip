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
//   W' = q * s * 2^shift[n]   (exact FP16; shift set at load, one per tensor
//                              unless its rows' scales differ by more than 2^12)
//   x' = x * 2^-e[m]          (per row; max |x'| in [2^13, 2^14))
// and writes y = acc * 2^(e[m] - shift[n]), an exact power-of-two rescale.
// Output rows of any relative magnitude are exact; within a row, a group
// whose scale is more than 2^26 below the row's largest may lose bits (each
// of its products then errs by at most 2^-26 of the row's largest one).
// BF16 activations are exact in FP16 after the rescale (8 significant bits;
// only values 2^28 below the row maximum lose bits).  FP32 activations are
// split as x' = hi + lo (two FP16 values, ~22 bits) and take two MFMAs.
//
// Pre-pass.  Per row it finds e[m] and writes x' as FP16 chunks
// of 8 values in "pair order": chunk (x0..x7) is stored as (x0,x4)(x1,x5)
// (x2,x6)(x3,x7), the order in which ((w >> 4t) & 0x000F000F) | 0x64006400
// unpacks a packed word into FP16 pairs (1024 + n_t, 1024 + n_t+4).  The
// MFMA only needs A and B to share one k order inside each 8-wide chunk, so
// no lane shuffles are needed.  The chunks are laid out chunk-major,
// xt[c][m] (16 bytes each, m padded to a multiple of 128), so the main
// kernel's tile loads read whole contiguous runs of rows.
//
// Main kernel: a 256-thread block (2 x 2 waves) computes a (32 TM) x (32 TN)
// output tile, each wave (16 TM) x (16 TN) as TM x TN MFMA tiles of 16 x 16.
// K advances KS groups (32 KS values) per stage through double-buffered LDS:
// while the MFMAs of stage s run, the loads of stage s + 1 are in flight in
// registers; afterwards they are stored to the other buffer, the weights
// dequantized on the way:
//   pair = ((w >> 4t) & 0x000F000F) | 0x64006400     (1024 + n, exact)
//   pair = (pair - 1032) * s'                        (v_pk_add/mul_f16, exact)
// LDS layout [chunk c][row] (16 B each) so the 16 lanes that read one MFMA
// operand touch consecutive addresses.
#include <math.h>

#include "g4_gemv.h"
#include "g4_internal.h"

namespace {

using namespace g4;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));


constexpr int kThreads = 256;
constexpr int kRowPad = 128;   // x' rows are padded to a multiple of the largest BM

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

// Row exponents: one wave per row.  e[m]: max |x[m]| * 2^-e in [2^13, 2^14);
// all-zero or non-finite rows keep e = 0.  Grid: ceil(M / 4) blocks.
template <bool F32X>
__global__ __launch_bounds__(kThreads) void gemm_xexp_kernel(const void *__restrict__ x, int M,
                                                             int K, int *__restrict__ xe) {
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (m >= M) return;
  const int nch = K >> 3;
  float mx = 0.f;
  // U chunks per lane per pass with every load issued first (chunks past the
  // row's end re-read its last chunk, which does not change the max)
  constexpr int U = 8;
  for (int c0 = lane; c0 < nch; c0 += 64 * U) {
    float v[U][8];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + 64 * u;
      load8<F32X>(x, (size_t)m * nch + (c < nch ? c : nch - 1), v[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[u][e]));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  int e = 0;
  if (mx > 0.f && mx <= 3.4e38f) e = ilogbf(mx) - 13;
  if (lane == 0) xe[m] = e;
}

// x' = x * 2^-e[m] as FP16 chunks in pair order, transposed to xt[c][m]
// through LDS: a block converts a tile of 64 rows x 16 chunks, reading 256
// contiguous bytes per row and writing 1 KB contiguous per chunk.  Rows
// M <= m < Mp are written as zeros.  For FP32 x the low halves go to
// xt[K/8 + c][m].  Grid: (Mp / 64, ceil(K / 128)).
constexpr int kPrepTileM = 64, kPrepTileC = 16;
template <bool F32X>
__global__ __launch_bounds__(kThreads) void gemm_xprep_kernel(const void *__restrict__ x,
                                                              const int *__restrict__ xe, int M,
                                                              int Mp, int K,
                                                              uint4 *__restrict__ xt) {
  __shared__ uint4 hs[kPrepTileC][kPrepTileM + 1];
  __shared__ uint4 ls[F32X ? kPrepTileC : 1][kPrepTileM + 1];
  const int nch = K >> 3;
  const int m0 = blockIdx.x * kPrepTileM, c0 = blockIdx.y * kPrepTileC;
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < kPrepTileM * kPrepTileC / kThreads; ++i) {
    const int idx = t + i * kThreads;
    const int r = idx / kPrepTileC, cc = idx % kPrepTileC;
    const int m = m0 + r, c = c0 + cc;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int e = 0;
    if (m < M && c < nch) {
      load8<F32X>(x, (size_t)m * nch + c, v);
      e = xe[m];
    }
    _Float16 h[8], l[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float s = ldexpf(v[j], -e);
      h[j] = (_Float16)s;
      if (F32X) l[j] = (_Float16)(s - (float)h[j]);
    }
    hs[cc][r] = make_uint4(h2bits(h[0], h[4]), h2bits(h[1], h[5]), h2bits(h[2], h[6]),
                           h2bits(h[3], h[7]));
    if (F32X)
      ls[cc][r] = make_uint4(h2bits(l[0], l[4]), h2bits(l[1], l[5]), h2bits(l[2], l[6]),
                             h2bits(l[3], l[7]));
  }
  __syncthreads();
  const size_t lo_plane = (size_t)nch * Mp;
#pragma unroll
  for (int i = 0; i < kPrepTileM * kPrepTileC / kThreads; ++i) {
    const int idx = t + i * kThreads;
    const int cc = idx / kPrepTileM, r = idx % kPrepTileM;
    const int c = c0 + cc;
    if (c >= nch) continue;
    const size_t o = (size_t)c * Mp + m0 + r;
    xt[o] = hs[cc][r];
    if (F32X) xt[lo_plane + o] = ls[cc][r];
  }
}

// Both pre-pass steps in one launch, for rows that fit a block's registers:
// a block owns kRowsFused = 4 whole rows, one wave (kPrepTpr = 64 threads)
// per row, and thread (r, j) holds chunks j, j + 64, ... (up to CPT) of row
// r.  Each row is read once: its maximum comes from a wave reduction, then
// the chunks are converted as in gemm_xprep_kernel and leave through an LDS
// tile [chunk][4 rows], so every wave store writes 64 contiguous bytes per
// chunk.  Rows M <= m < Mp are written as zeros.  Grid: Mp / 4.  (8 rows of
// 32 threads, half the blocks with twice the chunks per thread, took
// 12.76 / 6.28 us at M 2048 and K 6144 / 1536 against 9.80 / 5.88.)
constexpr int kRowsFused = 4, kPrepTpr = 64;
template <bool F32X, int CPT>
__global__ __launch_bounds__(kThreads) void gemm_xprep_fused_kernel(const void *__restrict__ x,
                                                                    int M, int Mp, int K,
                                                                    int *__restrict__ xe,
                                                                    uint4 *__restrict__ xt) {
  static_assert(kRowsFused * kPrepTpr == kThreads, "one wave per row");
  constexpr int NCH = kPrepTpr * CPT;  // chunk capacity of a row
  __shared__ uint4 hs[NCH][kRowsFused];
  __shared__ uint4 ls[F32X ? NCH : 1][kRowsFused];
  const int nch = K >> 3;
  const int t = threadIdx.x, r = t / kPrepTpr, j = t % kPrepTpr;
  const int m = blockIdx.x * kRowsFused + r;
  const bool row_live = m < M;
  // raw chunks: 16 bytes (BF16) or 32 bytes (FP32) each
  constexpr int W = F32X ? 2 : 1;
  uint4 raw[CPT][W];
  const uint4 *src = static_cast<const uint4 *>(x);
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = j + kPrepTpr * i;
    // every load issued first; chunks past the row re-read its first chunk
    // and rows past M re-read row 0 (both are left out below)
    const size_t cc = (size_t)(row_live ? m : 0) * nch + (c < nch ? c : 0);
#pragma unroll
    for (int w = 0; w < W; ++w) raw[i][w] = src[W * cc + w];
  }
  auto unpack = [&](int i, float (&v)[8]) {
    if (F32X) {
      const uint32_t u[8] = {raw[i][0].x, raw[i][0].y, raw[i][0].z, raw[i][0].w,
                             raw[i][W - 1].x, raw[i][W - 1].y, raw[i][W - 1].z, raw[i][W - 1].w};
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = __uint_as_float(u[q]);
    } else {
      const uint32_t u[4] = {raw[i][0].x, raw[i][0].y, raw[i][0].z, raw[i][0].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v[2 * q] = bf16_to_f32(u[q] & 0xffffu);
        v[2 * q + 1] = bf16_to_f32(u[q] >> 16);
      }
    }
  };
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    float v[8];
    unpack(i, v);
    if (j + kPrepTpr * i < nch)
#pragma unroll
      for (int q = 0; q < 8; ++q) mx = fmaxf(mx, fabsf(v[q]));
  }
#pragma unroll
  for (int o = kPrepTpr / 2; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kPrepTpr));
  int e = 0;
  if (row_live && mx > 0.f && mx <= 3.4e38f) e = ilogbf(mx) - 13;
  if (j == 0 && row_live) xe[m] = e;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = j + kPrepTpr * i;
    if (c >= nch) continue;
    float v[8];
    unpack(i, v);
    _Float16 h[8], l[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float sv = row_live ? ldexpf(v[q], -e) : 0.f;
      h[q] = (_Float16)sv;
      if (F32X) l[q] = (_Float16)(sv - (float)h[q]);
    }
    hs[c][r] = make_uint4(h2bits(h[0], h[4]), h2bits(h[1], h[5]), h2bits(h[2], h[6]),
                          h2bits(h[3], h[7]));
    if (F32X)
      ls[c][r] = make_uint4(h2bits(l[0], l[4]), h2bits(l[1], l[5]), h2bits(l[2], l[6]),
                            h2bits(l[3], l[7]));
  }
  __syncthreads();
  const size_t lo_plane = (size_t)nch * Mp;
  const int m0 = blockIdx.x * kRowsFused;
  for (int idx = t; idx < nch * kRowsFused; idx += kThreads) {
    const int c = idx / kRowsFused, rr = idx % kRowsFused;
    const size_t o = (size_t)c * Mp + m0 + rr;
    xt[o] = hs[c][rr];
    if (F32X) xt[lo_plane + o] = ls[c][rr];
  }
}

// Chunks per thread of the fused pre-pass for K, or 0 when the rows do not
// fit (then the two-kernel pre-pass runs).
int fused_prep_cpt(int K, bool f32x) {
  const int need = (K / 8 + kPrepTpr - 1) / kPrepTpr;
  const int caps[] = {2, 4, 8, 12, 16, 24, 32};
  for (int c : caps)
    if (need <= c && (!f32x || c <= 16)) return c;
  return 0;
}

// ---- main kernel -------------------------------------------------------------

__device__ __forceinline__ f16x8 as_f16x8(u32x4 u) { return __builtin_bit_cast(f16x8, u); }

__device__ __forceinline__ uint32_t deq_pair(uint32_t w, int t, f16x2 s2) {
  const uint32_t u = ((w >> (4 * t)) & 0x000F000Fu) | 0x64006400u;
  f16x2 h = __builtin_bit_cast(f16x2, u);
  const f16x2 off = {(_Float16)1032.f, (_Float16)1032.f};
  h = (h - off) * s2;
  return __builtin_bit_cast(uint32_t, h);
}

// Requires Mp a multiple of BM and (K / 32) a multiple of KS * gridDim.y (the
// launcher checks both); FLAT requires the stage count of a slice a multiple
// of an even P.
//
// Split K: with gridDim.y > 1, block row blockIdx.y covers stages
// [y * S, y * S + S) of the input dimension and writes its FP32 partial
// products (already rescaled) to part + y * pstride + poff[weight], rows < M
// only; the slices are then added in order by gemm_splitk_sum_kernel (one
// weight), or by the caller (several weights side by side in each plane).
// Weights of one input dimension over the same x' in one launch: the n tiles
// of weight i are t0[i] .. t0[i + 1] - 1 of the grid's tile axis.
//
// glu: weights 0 and 1 are gate and up of one width N; n tile j covers
// columns [j BN/2, (j + 1) BN/2) of both (gate in the first half of the tile,
// up in the second), and the block writes y[0] = gelu(gate) * up (FP32).
constexpr int kMaxGemmSegs = 3;
struct GemmSegs {
  const u32x4 *wq[kMaxGemmSegs];
  const uint16_t *ws[kMaxGemmSegs];
  // stage-major tile copies (g4_w4::tiles), read by the packed-weight kernel
  const u32x4 *tw[kMaxGemmSegs];
  void *y[kMaxGemmSegs];
  // per-row power-of-two shifts (g4_w4::rshift), or null: shift[] for the tensor
  const int16_t *rs[kMaxGemmSegs];
  int N[kMaxGemmSegs], shift[kMaxGemmSegs];
  int t0[kMaxGemmSegs + 1];
  int n, glu;
  // K split: weight i's planes start at part + poff[i] (rows x N[i] floats in
  // each plane of pstride floats)
  size_t poff[kMaxGemmSegs];
};

template <int TM, int TN, int NX, int KS, int P, bool FLAT>
__global__ __launch_bounds__(kThreads, 2) void w4_gemm_kernel(
    const u32x4 *__restrict__ xt, const int *__restrict__ xe, GemmSegs SG, int y_bf16, int M,
    int Mp, int K, int xcd_map, float *__restrict__ part, size_t pstride) {
  constexpr int BM = 32 * TM, BN = 32 * TN;
  constexpr int KC = 4 * KS;              // 16-byte chunks per row per stage
  constexpr int AE = BM * KC / kThreads;  // x' chunks per thread per stage (per plane)
  constexpr int BG = BN * KS;             // weight groups per stage
  constexpr int BE = (BG + kThreads - 1) / kThreads;
  static_assert(BM * KC % kThreads == 0, "A tile must split evenly over the block");
  // idle B entries (BG not a multiple of the block) store into a pad row
  constexpr int BNP = BG % kThreads ? BN + 1 : BN;
  __shared__ u32x4 As[2][NX][KC][BM];
  __shared__ u32x4 Bs[2][KC][BNP];

  const int G = K >> 5;
  const int S = G / KS / (int)gridDim.y;  // stages of this block's slice of K
  const int st0_slice = (int)blockIdx.y * S;
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // block -> (m tile, n tile); with xcd_map, all n tiles of one m band run on
  // one XCD (blocks are dealt to the 8 XCDs round-robin), so its L2 holds
  // that band of x' for every one of them.
  const bool glu = SG.glu != 0;
  constexpr int HALF = BN / 2;  // glu: gate and up columns per tile
  const int nn = glu ? (SG.N[0] + HALF - 1) / HALF : SG.t0[SG.n];
  int mt, ntile;
  if (xcd_map) {
    const int b = blockIdx.x, xcd = b & 7, j = b >> 3;
    mt = xcd + 8 * (j / nn);
    ntile = j - (j / nn) * nn;
  } else {
    mt = blockIdx.x / nn;
    ntile = blockIdx.x - mt * nn;
  }
  const int si = glu ? 0 : SG.n > 2 && ntile >= SG.t0[2] ? 2 : SG.n > 1 && ntile >= SG.t0[1] ? 1 : 0;
  const u32x4 *__restrict__ wq = SG.wq[si];
  const uint16_t *__restrict__ ws = SG.ws[si];
  void *__restrict__ y = SG.y[si];
  const int N = SG.N[si], shift = SG.shift[si];
  const int16_t *__restrict__ rsh = SG.rs[si];
  const int m0 = mt * BM, n0 = glu ? ntile * HALF : (ntile - SG.t0[si]) * BN;

  // A: entry i of this thread is chunk a_c[i] of tile row a_row[i]
  const size_t a_stage = (size_t)KC * Mp;  // xt entries per stage
  const size_t lo_plane = (size_t)(K >> 3) * Mp;
  int a_row[AE], a_c[AE];
  const u32x4 *a_src[AE];
#pragma unroll
  for (int i = 0; i < AE; ++i) {
    const int idx = t + i * kThreads;
    a_c[i] = idx / BM;
    a_row[i] = idx % BM;
    a_src[i] = xt + (size_t)(st0_slice * KC + a_c[i]) * Mp + m0 + a_row[i];
  }
  // B: entry i is group b_kk[i] of the stage for tile row b_row[i]
  int b_row[BE], b_kk[BE];
  // Scales: with an even KS, one aligned 32-bit load brings the scales of
  // groups kk & ~1 and kk | 1 (G is even then); the half is picked at store.
  constexpr int SW = KS % 2 == 0 ? 2 : 1;  // scales per scale load
  const u32x4 *b_src[BE];
  const uint16_t *s_src[BE];
  int b_shift[BE];
#pragma unroll
  for (int i = 0; i < BE; ++i) {
    const int idx = t + i * kThreads;
    const bool live = idx < BG;  // idle entries load group 0 of row n0 into the pad row
    b_row[i] = live ? idx / KS : BN;
    b_kk[i] = live ? idx % KS : 0;
    const int up = glu && live && b_row[i] >= HALF;  // glu: the tile's up half
    const int rn = live ? b_row[i] - up * HALF : 0;
    const int gn = n0 + rn < N ? n0 + rn : N - 1;
    b_src[i] = (up ? SG.wq[1] : wq) + (size_t)gn * G + st0_slice * KS + b_kk[i];
    s_src[i] = (up ? SG.ws[1] : ws) + (size_t)gn * G + st0_slice * KS + (b_kk[i] & ~(SW - 1));
    const int16_t *rsi = up ? SG.rs[1] : rsh;
    b_shift[i] = rsi ? rsi[gn] : up ? SG.shift[1] : shift;
  }

  // Ring of P register slots: stage j is loaded into slot j % P, P - 1
  // stages ahead of the MFMAs that use it.  Loads past the last stage re-read
  // it (in bounds, never used), so every step issues the same loads.
  u32x4 ra[P][NX][AE];
  u32x4 rb[P][BE];
  uint32_t rs[P][BE];
  auto fetch = [&](int st, int slot) {
    const int sc = st < S ? st : S - 1;
#pragma unroll
    for (int i = 0; i < AE; ++i) {
      ra[slot][0][i] = a_src[i][sc * a_stage];
      if (NX == 2) ra[slot][NX - 1][i] = a_src[i][lo_plane + sc * a_stage];
    }
#pragma unroll
    for (int i = 0; i < BE; ++i) {
      rb[slot][i] = b_src[i][sc * KS];
      if (SW == 2)
        rs[slot][i] = *reinterpret_cast<const uint32_t *>(s_src[i] + sc * KS);
      else
        rs[slot][i] = s_src[i][sc * KS];
    }
  };
  auto store = [&](int slot, int buf) {
#pragma unroll
    for (int x = 0; x < NX; ++x)
#pragma unroll
      for (int i = 0; i < AE; ++i) As[buf][x][a_c[i]][a_row[i]] = ra[slot][x][i];
#pragma unroll
    for (int i = 0; i < BE; ++i) {
      const uint32_t sbits = SW == 2 && (b_kk[i] & 1) ? rs[slot][i] >> 16 : rs[slot][i] & 0xffffu;
      const _Float16 sh = (_Float16)ldexpf(bf16_to_f32(sbits), b_shift[i]);
      const f16x2 s2 = {sh, sh};
      const u32x4 w = rb[slot][i];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        Bs[buf][4 * b_kk[i] + j][b_row[i]] =
            (u32x4){deq_pair(w[j], 0, s2), deq_pair(w[j], 1, s2), deq_pair(w[j], 2, s2),
                    deq_pair(w[j], 3, s2)};
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  const int lr = lane & 15, lc = lane >> 4;  // operand row within a 16-tile, k chunk
  auto compute = [&](int buf) {
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      f16x8 bop[TN];
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bop[j] = as_f16x8(Bs[buf][4 * kk + lc][wn * 16 * TN + j * 16 + lr]);
#pragma unroll
      for (int x = 0; x < NX; ++x)
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const f16x8 aop = as_f16x8(As[buf][x][4 * kk + lc][wm * 16 * TM + i * 16 + lr]);
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop[j], acc[i][j], 0, 0, 0);
        }
    }
  };

#pragma unroll
  for (int s = 0; s < P - 1; ++s) fetch(s, s);
  store(0, 0);
  __syncthreads();
  if constexpr (FLAT) {
    // Each step is one branch-free scheduling region: unrolled by an even P,
    // the ring slot and the LDS buffer of every step are constants, and the
    // step after the last stores a re-read stage into the idle buffer.  The
    // group barriers interleave the MFMAs with the next operands' LDS reads,
    // the global loads, the dequant VALU and the LDS writes of the next stage.
    constexpr int NM = TM * TN * NX * KS;   // MFMAs per step
    constexpr int NR = (TM * NX + TN) * KS; // LDS operand reads
    constexpr int NW = AE * NX + 4 * BE;    // LDS writes
    for (int st0 = 0; st0 < S; st0 += P) {
#pragma unroll
      for (int s = 0; s < P; ++s) {
        fetch(st0 + s + P - 1, (s + P - 1) % P);
        compute(s & 1);
        store((s + 1) % P, (s + 1) & 1);
        __builtin_amdgcn_sched_group_barrier(0x020, AE * NX + 2 * BE, 0);  // global loads
        __builtin_amdgcn_sched_group_barrier(0x100, TM * NX + TN, 0);      // LDS reads, first k
#pragma unroll
        for (int k = 0; k < NM; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          if (k < NR - (TM * NX + TN)) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // VALU
          if (k >= NM - NW) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
        }
        __syncthreads();
      }
    }
  } else {
  // unrolled by P, so the ring slot of every step is a constant
  for (int st0 = 0; st0 < S; st0 += P) {
#pragma unroll
    for (int s = 0; s < P; ++s) {
      const int st = st0 + s;
      if (st >= S) break;
      fetch(st + P - 1, (s + P - 1) % P);  // the slot of stage st - 1, already in LDS
      compute(st & 1);
      if (st + 1 < S) store((s + 1) % P, (st + 1) & 1);
      __syncthreads();
    }
  }
  }

  // Every row exponent and column shift is read, and every accumulator
  // rescaled, before the first output store: vmcnt counts stores too, so a
  // wait for a load issued (or first used) among the stores would also wait
  // for the stores before it, one store at a time.
  {
    int ev[TM][4], csh[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 16 * TM + i * 16 + 4 * lc + r;
        ev[i][r] = xe[m < M ? m : M - 1];
      }
    // this lane's output columns (glu: columns n0 + j * 16 + lr of up for wn = 1,
    // of gate for wn = 0)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = glu ? n0 + j * 16 + lr : n0 + wn * 16 * TN + j * 16 + lr;
      const int seg = glu ? (wn == 1 ? 1 : 0) : si;
      const int16_t *r = SG.rs[seg];
      csh[j] = r ? r[n < N ? n : N - 1] : SG.shift[seg];
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][r] = ldexpf(acc[i][j][r], ev[i][r] - csh[j]);
  }

  // epilogue: lane holds rows 4*lc + r (r = 0..3) of column lr of each tile;
  // one branch-free copy per output type
  auto epilogue = [&](auto *out) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 16 * TM + i * 16 + 4 * lc + r;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = n0 + wn * 16 * TN + j * 16 + lr;
          if (n >= N) continue;
          const float v = acc[i][j][r];
          if constexpr (sizeof(*out) == 2)
            out[(size_t)m * N + n] = (uint16_t)f32_to_bf16_rne(v);
          else
            out[(size_t)m * N + n] = v;
        }
      }
    }
  };
  if (glu) {
    // waves wn = 1 hold the up values of the positions waves wn = 0 hold the
    // gate values of (same lane and register): they pass them through the
    // A tile's LDS, free after the last stage's barrier
    constexpr int NE = TM * TN * 4;  // accumulator floats per lane
    static_assert(2 * NE * 64 * sizeof(float) <= sizeof(As), "up values must fit the A tile");
    float *upv = reinterpret_cast<float *>(&As[0][0][0][0]);
    if (wn == 1) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            upv[(wm * NE + (i * TN + j) * 4 + r) * 64 + lane] = acc[i][j][r];
    }
    __syncthreads();
    if (wn == 0) {
      float *out = static_cast<float *>(y);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm * 16 * TM + i * 16 + 4 * lc + r;
          if (m >= M) continue;
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const int n = n0 + j * 16 + lr;
            if (n >= N) continue;
            const float g = acc[i][j][r];
            out[(size_t)m * N + n] = gelu_tanh(g) * upv[(wm * NE + (i * TN + j) * 4 + r) * 64 + lane];
          }
        }
      }
    }
  } else if (gridDim.y > 1)
    epilogue(part + blockIdx.y * pstride + SG.poff[si]);
  else if (y_bf16)
    epilogue(static_cast<uint16_t *>(y));
  else
    epilogue(static_cast<float *>(y));
}

// ---- main kernel, packed weights per wave --------------------------------------
//
// The same product, laid out so that every weight is used by one wave only
// and stays packed (4 bits) until that wave's registers.  The 4 waves of a
// block sit side by side in N: wave w computes rows [m0, m0 + BM)
// (BM = 16 TMW) times TNW tiles of 16 columns.  A stage is 64 values of K (2
// groups, 8 x' chunks).  Every operand of a stage reaches LDS by direct
// global -> LDS loads, two stages ahead, into one of three buffers:
//   x'      64 consecutive rows of one chunk per wave instruction;
//   weights per wave, the stage's 576-byte blocks of its TNW tiles from the
//           weight's stage-major tile copy (g4_w4::tiles): 512 bytes of
//           words, in the order the lanes read them (lane l's two words at
//           8 l, so the 64 lanes' 8-byte reads hit every bank once), and the
//           16 rows' scale pairs, 16 bytes per lane, so words and scales of
//           3 tiles take 2 load instructions.
// From the row-major arrays each word or scale load instruction touched 32-48
// cache lines, and those loads, not the MFMAs, held the main loop (M 2048 N
// 6144 K 1536: 51.1 -> 44.5 us with the same addresses made contiguous).
// Lane (c = lane % 16, q = lane / 16) then reads words 2q and 2q + 1 of the
// stage's 8 words of row c (both in group q / 2, one scale) and dequantizes
// them; MFMA step j (0, 1) takes word j as its B operand and x' chunk 2q + j
// of row m as its A operand, so A and B agree on the k order inside every
// lane's 8 values.  Only the waits for these loads order the main loop: the
// compiler's own waits for register loads cannot follow a ring across the
// loop's back edge and would wait for every load in flight.
//
// glu: TNW is even and a wave's tiles TNW/2 .. TNW-1 are the up columns of
// its gate tiles 0 .. TNW/2-1, so gelu(gate) * up needs no exchange.
// P: stages (LDS buffers) in the ring; MINB: blocks per CU the registers are
// sized for (1: up to 512 per lane, accumulators in AGPRs).
template <int TMW, int TNW, int NX, int P, int MINB>
__global__ __launch_bounds__(kThreads, MINB) void w4_gemm_rb_kernel(
    const u32x4 *__restrict__ xt, const int *__restrict__ xe, GemmSegs SG, int y_bf16, int M,
    int Mp, int K, int xcd_map, float *__restrict__ part, size_t pstride) {
  constexpr int BM = 16 * TMW;
  constexpr int KC = 8;                 // x' chunks per stage
  constexpr int AW = KC * BM / 64 / 4;  // x' wave loads per wave, per plane
  constexpr int TU = 36;                    // 16-byte units of a tile's stage block
  constexpr int WU = TNW * TU;              // units of a wave's stage stream
  constexpr int NB = (WU + 63) / 64;        // weight wave loads per wave
  static_assert(BM % 64 == 0 && AW >= 1, "A rows must come in runs of 64");
  static_assert(WU >= 64, "a wave's weight stream fills at least one load");
  // load d covers units w0(d) .. + 63: the last one ends at the stream's end,
  // overlapping the one before (those units are written twice, with the same
  // bytes), so the LDS region is the stream itself
  auto w0 = [](int d) { return 64 * d < WU - 64 ? 64 * d : WU - 64; };
  struct Stage {
    u32x4 a[NX][KC][BM];
    u32x4 w[4][WU];  // per wave: its tiles' stage blocks, TU units each
  };
  // one LDS object: the stage ring and the block's row exponents (loaded
  // with the first stages).  A second __shared__ array makes the compiler
  // wait for every direct load in flight before each LDS read of the ring.
  struct Smem {
    Stage st[P];
    int xe[BM];
  };
  __shared__ Smem smem;
  Stage *const st_lds = smem.st;
  int *const xe_lds = smem.xe;

  const int G = K >> 5;
  const int S = G / 2 / (int)gridDim.y;  // stages of this block's slice of K
  const int st0_slice = (int)blockIdx.y * S;
  const int t = threadIdx.x;
  // wave index in a scalar register: the LDS destinations of the direct loads
  // are then scalar arithmetic (no readfirstlane per load)
  const int lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lr = lane & 15, lq = lane >> 4;

  const bool glu = SG.glu != 0;
  // columns per block: 64 TNW, or 32 TNW gate (+ the same up) columns with glu
  const int bn = glu ? 32 * TNW : 64 * TNW;
  const int nn = glu ? (SG.N[0] + bn - 1) / bn : SG.t0[SG.n];
  int mt, ntile;
  if (xcd_map) {
    const int b = blockIdx.x, xcd = b & 7, j = b >> 3;
    mt = xcd + 8 * (j / nn);
    ntile = j - (j / nn) * nn;
  } else {
    mt = blockIdx.x / nn;
    ntile = blockIdx.x - mt * nn;
  }
  const int si = glu ? 0 : SG.n > 2 && ntile >= SG.t0[2] ? 2 : SG.n > 1 && ntile >= SG.t0[1] ? 1 : 0;
  const int N = SG.N[si];
  const int m0 = mt * BM;
  // this wave's first output column; tile jj covers columns col(jj) .. + 15
  const int wc0 = glu ? ntile * bn + wave * 8 * TNW : (ntile - SG.t0[si]) * bn + wave * 16 * TNW;
  auto col = [&](int jj) { return wc0 + 16 * (glu && jj >= TNW / 2 ? jj - TNW / 2 : jj); };
  // the weight of tile jj, and its row for tile row r (rows past N re-read the last)
  auto seg_of = [&](int jj) { return glu ? (jj >= TNW / 2 ? 1 : 0) : si; };
  auto row_of = [&](int jj, int r) {
    const int gn = col(jj) + r, Nw = SG.N[seg_of(jj)];
    return gn < Nw ? gn : Nw - 1;
  };

  // sources of this lane's loads at stage 0 of the slice (tiles past TNW
  // re-read tile 0 into an unread part of the buffer)
  const size_t a_stage = (size_t)KC * Mp;
  const size_t lo_plane = (size_t)(K >> 3) * Mp;
  // x' sources: a uniform base (this slice's first stage, this block's rows)
  // plus a 32-bit per-lane byte offset, so the loads take a scalar base and
  // the stage advance is scalar arithmetic
  const u32x4 *a_base = xt + (size_t)(st0_slice * KC) * Mp + m0;
  uint32_t a_off[AW];
  int a_c[AW], a_r[AW];
#pragma unroll
  for (int i = 0; i < AW; ++i) {
    const int u = wave * AW + i;
    a_c[i] = u / (BM / 64);
    a_r[i] = 64 * (u % (BM / 64));
    a_off[i] = (uint32_t)((a_c[i] * Mp + a_r[i] + lane) * 16);
  }
  // weight words and scales from the stage-major tile copies: unit u of the
  // wave's stream is unit u % TU of tile u / TU's block; tiles past N (a
  // ragged last block) read the last tile.  The stage stride is the same for
  // every tile of a block (gate and up share N).
  const int Tn = (SG.N[seg_of(0)] + 15) >> 4;
  const size_t w_stage = (size_t)Tn * TU;
  const u32x4 *w_src[NB];
#pragma unroll
  for (int d = 0; d < NB; ++d) {
    const int u = w0(d) + lane;
    const int jj = u / TU, e = u - jj * TU;
    int tile = col(jj) >> 4;
    tile = tile < Tn ? tile : Tn - 1;
    w_src[d] = SG.tw[seg_of(jj)] + ((size_t)st0_slice * Tn + tile) * TU + e;
  }
  int b_shift[TNW];
#pragma unroll
  for (int jj = 0; jj < TNW; ++jj) {
    const int seg = seg_of(jj);
    b_shift[jj] = SG.rs[seg] ? SG.rs[seg][row_of(jj, lr)] : SG.shift[seg];
  }

  typedef __attribute__((address_space(3))) void *lds_ptr;
  auto issue = [&](int stg, int slot) {
    const int sc = stg < S ? stg : S - 1;  // past the last stage: re-read it, never used
    Stage &L = st_lds[slot];
#pragma unroll
    for (int x = 0; x < NX; ++x)
#pragma unroll
      for (int i = 0; i < AW; ++i)
        __builtin_amdgcn_global_load_lds(
            (const void *)(reinterpret_cast<const char *>(a_base + (x ? lo_plane : 0) + sc * a_stage) +
                           a_off[i]),
            (lds_ptr)&L.a[x][a_c[i]][a_r[i]], 16, 0, 0);
#pragma unroll
    for (int d = 0; d < NB; ++d)
      __builtin_amdgcn_global_load_lds((const void *)(w_src[d] + sc * w_stage),
                                       (lds_ptr)&L.w[wave][w0(d)], 16, 0, 0);
  };

  f32x4 acc[TMW][TNW];
#pragma unroll
  for (int i = 0; i < TMW; ++i)
#pragma unroll
    for (int j = 0; j < TNW; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  uint32_t mask = 0x000F000Fu;
  asm volatile("" : "+v"(mask));  // keep the mask in a VGPR: lets v_and_or_b32 take the magic
  auto deq = [&](uint32_t w, int sh, f16x2 s2) {
    const uint32_t u = ((w >> (4 * sh)) & mask) | 0x64006400u;
    f16x2 h = __builtin_bit_cast(f16x2, u);
    const f16x2 off = {(_Float16)1032.f, (_Float16)1032.f};
    h = (h - off) * s2;
    return __builtin_bit_cast(uint32_t, h);
  };
  // One stage: every LDS read is issued before the first use, and step 1's
  // operands (A reads, B dequant) are prepared while step 0's MFMAs run.
  auto compute = [&](int slot) {
    const Stage &L = st_lds[slot];
    u32x2 wds[TNW];
    uint32_t sp[TNW];
    const char *wb = reinterpret_cast<const char *>(&L.w[wave][0]);
#pragma unroll
    for (int jj = 0; jj < TNW; ++jj) {
      wds[jj] = *reinterpret_cast<const u32x2 *>(wb + jj * TU * 16 + 8 * lane);
      sp[jj] = *reinterpret_cast<const uint32_t *>(wb + jj * TU * 16 + 512 + 4 * lr);
    }
    f16x8 a0[NX][TMW], a1[NX][TMW];
#pragma unroll
    for (int x = 0; x < NX; ++x)
#pragma unroll
      for (int i = 0; i < TMW; ++i) a0[x][i] = as_f16x8(L.a[x][2 * lq][i * 16 + lr]);
    f16x2 s2[TNW];
#pragma unroll
    for (int jj = 0; jj < TNW; ++jj) {
      const uint32_t sb = (lq >> 1) ? sp[jj] >> 16 : sp[jj] & 0xffffu;
      const _Float16 sh = (_Float16)ldexpf(bf16_to_f32(sb), b_shift[jj]);
      s2[jj] = (f16x2){sh, sh};
    }
    // the nibbles of both words at shifts 4, 8, 12 from three 64-bit shifts
    // (the low word's top bits then come from the high word and fall outside
    // the mask)
    uint32_t sh_lo[TNW][4], sh_hi[TNW][4];
#pragma unroll
    for (int jj = 0; jj < TNW; ++jj) {
      const uint64_t u = ((uint64_t)wds[jj][1] << 32) | wds[jj][0];
      uint64_t s4, s8, s12;
      asm("v_lshrrev_b64 %0, 4, %1" : "=v"(s4) : "v"(u));
      asm("v_lshrrev_b64 %0, 8, %1" : "=v"(s8) : "v"(u));
      asm("v_lshrrev_b64 %0, 12, %1" : "=v"(s12) : "v"(u));
      sh_lo[jj][0] = wds[jj][0];
      sh_lo[jj][1] = (uint32_t)s4;
      sh_lo[jj][2] = (uint32_t)s8;
      sh_lo[jj][3] = (uint32_t)s12;
      sh_hi[jj][0] = wds[jj][1];
      sh_hi[jj][1] = (uint32_t)(s4 >> 32);
      sh_hi[jj][2] = (uint32_t)(s8 >> 32);
      sh_hi[jj][3] = (uint32_t)(s12 >> 32);
    }
    auto deq8 = [&](const uint32_t (&w)[4], f16x2 sc) {
      return as_f16x8((u32x4){deq(w[0], 0, sc), deq(w[1], 0, sc), deq(w[2], 0, sc), deq(w[3], 0, sc)});
    };
    f16x8 b0[TNW], b1[TNW];
#pragma unroll
    for (int jj = 0; jj < TNW; ++jj) b0[jj] = deq8(sh_lo[jj], s2[jj]);
#pragma unroll
    for (int x = 0; x < NX; ++x)
#pragma unroll
      for (int i = 0; i < TMW; ++i) a1[x][i] = as_f16x8(L.a[x][2 * lq + 1][i * 16 + lr]);
#pragma unroll
    for (int jj = 0; jj < TNW; ++jj) b1[jj] = deq8(sh_hi[jj], s2[jj]);
#pragma unroll
    for (int x = 0; x < NX; ++x)
#pragma unroll
      for (int i = 0; i < TMW; ++i)
#pragma unroll
        for (int jj = 0; jj < TNW; ++jj)
          acc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0[x][i], b0[jj], acc[i][jj], 0, 0, 0);
#pragma unroll
    for (int x = 0; x < NX; ++x)
#pragma unroll
      for (int i = 0; i < TMW; ++i)
#pragma unroll
        for (int jj = 0; jj < TNW; ++jj)
          acc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1[x][i], b1[jj], acc[i][jj], 0, 0, 0);
    // the order above, as scheduling groups: this stage's loads, every LDS
    // read of step 0, the scales and step 0's dequant, step 1's A reads, then
    // step 0's MFMAs with step 1's dequant between them, then step 1's MFMAs
    constexpr int NM = NX * TMW * TNW;  // MFMAs per step
    __builtin_amdgcn_sched_group_barrier(0x020, NX * AW + NB, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * TNW + NX * TMW, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, 20 * TNW, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, NX * TMW, 0);
#pragma unroll
    for (int k = 0; k < NM; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, (12 * TNW + NM - 1) / NM, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);
  };

  // Loads of one issue, per thread: they retire in order, so waiting until at
  // most one issue is outstanding completes the one before it.  The wait and
  // the barrier are one asm statement with a memory clobber: __syncthreads()
  // would add a workgroup release, which waits for every load in flight (the
  // direct-LDS loads count as LDS writes), the next stage's included.
  constexpr int NI = NX * AW + NB;
  constexpr int NW = (P - 2) * NI;  // loads that may stay in flight: stages st + 2 .. st + P - 1
  static_assert(NW < 64, "vmcnt is 6 bits");
  // the row exponents first (older than every stage load, so each wait below
  // completes them too): the epilogue then reads them from LDS instead of
  // waiting on a global load after the main loop
  if (wave < BM / 64) {
    const int m = m0 + wave * 64 + lane;
    __builtin_amdgcn_global_load_lds((const void *)(xe + (m < M ? m : M - 1)),
                                     (lds_ptr)&xe_lds[wave * 64], 4, 0, 0);
  }
#pragma unroll
  for (int q = 0; q < P - 1; ++q) issue(q, q);
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(NW) : "memory");
  for (int st0 = 0; st0 < S; st0 += P) {
#pragma unroll
    for (int s = 0; s < P; ++s) {
      const int stg = st0 + s;
      if (stg >= S) break;
      issue(stg + P - 1, (s + P - 1) % P);  // the buffer of stage stg - 1, free after its barrier
      compute(s);
      // stage stg + 1 has landed (this wave's loads; after the barrier,
      // everyone's), and no wave still reads stage stg's buffer; nothing
      // (the MFMAs included) moves across
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(NW) : "memory");
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // the re-reads issued past the last stage land before the block may end
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // rescale before the first store (vmcnt counts stores too)
  {
    int ev[TMW][4];
#pragma unroll
    for (int i = 0; i < TMW; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ev[i][r] = xe_lds[i * 16 + 4 * lq + r];
      }
#pragma unroll
    for (int i = 0; i < TMW; ++i)
#pragma unroll
      for (int j = 0; j < TNW; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][r] = ldexpf(acc[i][j][r], ev[i][r] - b_shift[j]);
  }

  if (glu) {
    float *out = static_cast<float *>(SG.y[0]);
#pragma unroll
    for (int i = 0; i < TMW; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + i * 16 + 4 * lq + r;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < TNW / 2; ++j) {
          const int n = col(j) + lr;
          if (n >= N) continue;
          out[(size_t)m * N + n] = gelu_tanh(acc[i][j][r]) * acc[i][j + TNW / 2][r];
        }
      }
    }
    return;
  }
  auto epilogue = [&](auto *out) {
#pragma unroll
    for (int i = 0; i < TMW; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + i * 16 + 4 * lq + r;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < TNW; ++j) {
          const int n = col(j) + lr;
          if (n >= N) continue;
          const float v = acc[i][j][r];
          if constexpr (sizeof(*out) == 2)
            out[(size_t)m * N + n] = (uint16_t)f32_to_bf16_rne(v);
          else
            out[(size_t)m * N + n] = v;
        }
      }
    }
  };
  if (gridDim.y > 1)
    epilogue(part + blockIdx.y * pstride + SG.poff[si]);
  else if (y_bf16)
    epilogue(static_cast<uint16_t *>(SG.y[si]));
  else
    epilogue(static_cast<float *>(SG.y[si]));
}

// y[i] = sum of part[s * pstride + i] over the slices s in order, as FP32 or
// BF16.  VEC: four outputs per thread (n a multiple of 4, y 16-byte aligned).
template <bool VEC>
__global__ __launch_bounds__(kThreads) void gemm_splitk_sum_kernel(const float *__restrict__ part,
                                                                   int slices, size_t pstride,
                                                                   size_t n, void *__restrict__ y,
                                                                   int y_bf16) {
  const size_t i = ((size_t)blockIdx.x * kThreads + threadIdx.x) * (VEC ? 4 : 1);
  if (i >= n) return;
  if (VEC) {
    f32x4 v = *reinterpret_cast<const f32x4 *>(part + i);
    for (int s = 1; s < slices; ++s) v += *reinterpret_cast<const f32x4 *>(part + s * pstride + i);
    if (y_bf16) {
      const uint32_t lo = f32_to_bf16_rne(v[0]) | (f32_to_bf16_rne(v[1]) << 16);
      const uint32_t hi = f32_to_bf16_rne(v[2]) | (f32_to_bf16_rne(v[3]) << 16);
      *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(y) + i) = make_uint2(lo, hi);
    } else {
      *reinterpret_cast<f32x4 *>(static_cast<float *>(y) + i) = v;
    }
  } else {
    float v = part[i];
    for (int s = 1; s < slices; ++s) v += part[s * pstride + i];
    if (y_bf16)
      static_cast<uint16_t *>(y)[i] = (uint16_t)f32_to_bf16_rne(v);
    else
      static_cast<float *>(y)[i] = v;
  }
}

// Floats between consecutive split-K partial planes of rows x N outputs.
size_t splitk_pstride(int rows, int N) { return ((size_t)rows * N + 63) & ~size_t(63); }
// The same for the weights of one launch, side by side in each plane.
size_t splitk_pstride(const g4_w4 *const *w, int nw, int rows) {
  size_t n = 0;
  for (int i = 0; i < nw; ++i) n += (size_t)rows * w[i]->N;
  return (n + 63) & ~size_t(63);
}

// n weights (1..kMaxGemmSegs) of one input dimension, y[i] receiving weight
// i's output; a K split (slices > 1) that is summed here takes one weight,
// one left to the caller (sum false) any number.
template <int TM, int TN, int NX, int KS, int P>
int launch_gemm(const g4_w4 *const *w, int nw, const uint4 *xt, const int *xe, int rows, int Mp,
                void *const *ys, bool y_bf16, float *part, int slices, bool sum, bool glu) {
  constexpr int BM = 32 * TM, BN = 32 * TN;
  if (Mp % BM != 0 || w[0]->G % (KS * slices) != 0 || (slices > 1 && nw != 1 && sum))
    return fail(G4_E_ARG, "w4_gemm: tile %dx%d (KS %d, %d slices) does not fit rows %d, K %d",
                BM, BN, KS, slices, rows, w[0]->K);
  GemmSegs sg{};
  sg.n = nw;
  for (int i = 0; i < nw; ++i) {
    sg.wq[i] = reinterpret_cast<const u32x4 *>(w[i]->packed);
    sg.ws[i] = w[i]->scales;
    sg.y[i] = ys[i];
    sg.N[i] = w[i]->N;
    sg.rs[i] = w[i]->row_shift ? w[i]->rshift : nullptr;
    sg.shift[i] = w[i]->shift;
    sg.t0[i + 1] = sg.t0[i] + (w[i]->N + BN - 1) / BN;
  }
  sg.glu = glu;
  const int nm = (rows + BM - 1) / BM;
  const int nn = glu ? (w[0]->N + BN / 2 - 1) / (BN / 2) : sg.t0[nw];
  const int xcd_map = nm % 8 == 0;
  const bool flat = P % 2 == 0 && (w[0]->G / KS / slices) % P == 0;
  size_t pstride = 0;
  for (int i = 0; i < nw; ++i) {
    sg.poff[i] = pstride;
    pstride += (size_t)rows * w[i]->N;
  }
  pstride = (pstride + 63) & ~size_t(63);
  auto kernel = flat ? w4_gemm_kernel<TM, TN, NX, KS, P, true> : w4_gemm_kernel<TM, TN, NX, KS, P, false>;
  hipLaunchKernelGGL(kernel, dim3(nm * nn, slices), dim3(kThreads), 0, stream(),
                     reinterpret_cast<const u32x4 *>(xt), xe, sg, (int)y_bf16, rows, Mp,
                     w[0]->K, xcd_map, part, pstride);
  G4_LAUNCH_CHECK("w4_gemm_kernel");
  if (slices > 1 && sum) {
    void *y = ys[0];
    const size_t n = (size_t)rows * w[0]->N;
    const bool vec = n % 4 == 0 && (reinterpret_cast<uintptr_t>(y) & 15u) == 0;
    const size_t threads = vec ? n / 4 : n;
    const dim3 grid((unsigned)((threads + kThreads - 1) / kThreads));
    if (vec)
      hipLaunchKernelGGL(gemm_splitk_sum_kernel<true>, grid, dim3(kThreads), 0, stream(), part,
                         slices, pstride, n, y, (int)y_bf16);
    else
      hipLaunchKernelGGL(gemm_splitk_sum_kernel<false>, grid, dim3(kThreads), 0, stream(), part,
                         slices, pstride, n, y, (int)y_bf16);
    G4_LAUNCH_CHECK("gemm_splitk_sum_kernel");
  }
  return G4_OK;
}

// The registers-B kernel: BM = 16 TMW rows by BN = 64 TNW columns per block,
// stages of 64 values of K.
template <int TMW, int TNW, int NX, int P, int MINB>
int launch_gemm_rb(const g4_w4 *const *w, int nw, const uint4 *xt, const int *xe, int rows,
                   int Mp, void *const *ys, bool y_bf16, float *part, int slices, bool sum,
                   bool glu) {
  constexpr int BM = 16 * TMW;
  const int BN = glu ? 32 * TNW : 64 * TNW;  // output columns per block
  if (Mp % BM != 0 || w[0]->G % (2 * slices) != 0 || (slices > 1 && nw != 1 && sum) ||
      (glu && TNW % 2 != 0))
    return fail(G4_E_ARG, "w4_gemm: tile %dx%d (%d slices) does not fit rows %d, K %d", BM, BN,
                slices, rows, w[0]->K);
  GemmSegs sg{};
  sg.n = nw;
  for (int i = 0; i < nw; ++i) {
    if (!w[i]->tiles)
      return fail(G4_E_ARG, "w4_gemm: no tile copy of a weight with odd group count %d",
                  w[i]->G);
    sg.wq[i] = reinterpret_cast<const u32x4 *>(w[i]->packed);
    sg.ws[i] = w[i]->scales;
    sg.tw[i] = reinterpret_cast<const u32x4 *>(w[i]->tiles);
    sg.y[i] = ys[i];
    sg.N[i] = w[i]->N;
    sg.rs[i] = w[i]->row_shift ? w[i]->rshift : nullptr;
    sg.shift[i] = w[i]->shift;
    sg.t0[i + 1] = sg.t0[i] + (w[i]->N + BN - 1) / BN;
  }
  sg.glu = glu;
  const int nm = (rows + BM - 1) / BM;
  const int nn = glu ? (w[0]->N + BN - 1) / BN : sg.t0[nw];
  const int xcd_map = nm % 8 == 0;
  size_t pstride = 0;
  for (int i = 0; i < nw; ++i) {
    sg.poff[i] = pstride;
    pstride += (size_t)rows * w[i]->N;
  }
  pstride = (pstride + 63) & ~size_t(63);
  hipLaunchKernelGGL((w4_gemm_rb_kernel<TMW, TNW, NX, P, MINB>), dim3(nm * nn, slices), dim3(kThreads),
                     0, stream(), reinterpret_cast<const u32x4 *>(xt), xe, sg, (int)y_bf16, rows,
                     Mp, w[0]->K, xcd_map, part, pstride);
  G4_LAUNCH_CHECK("w4_gemm_rb_kernel");
  if (slices > 1 && sum) {
    void *y = ys[0];
    const size_t n = (size_t)rows * w[0]->N;
    const bool vec = n % 4 == 0 && (reinterpret_cast<uintptr_t>(y) & 15u) == 0;
    const size_t threads = vec ? n / 4 : n;
    const dim3 grid((unsigned)((threads + kThreads - 1) / kThreads));
    if (vec)
      hipLaunchKernelGGL(gemm_splitk_sum_kernel<true>, grid, dim3(kThreads), 0, stream(), part,
                         slices, pstride, n, y, (int)y_bf16);
    else
      hipLaunchKernelGGL(gemm_splitk_sum_kernel<false>, grid, dim3(kThreads), 0, stream(), part,
                         slices, pstride, n, y, (int)y_bf16);
    G4_LAUNCH_CHECK("gemm_splitk_sum_kernel");
  }
  return G4_OK;
}

// Tile and K split of one prefill GEMM.  Tile: the largest (128 x 128, BF16
// x) unless that leaves CUs idle or a ragged last wave; then 128 x 96 or 64 x 96
// tiles when those fill whole rounds of the CUs (e.g. M 2048, N 1536 -> 256
// tiles of 128 x 96), then 64 x 128 and 64 x 64.  Two groups per stage unless
// the group count is odd.
//
// K split (partial planes added by gemm_splitk_sum_kernel): a grid of fewer
// 64 x 64 tiles than CUs (the E2B prefill's 1536-wide outputs at 512 rows:
// 192 tiles) takes 64 x 96 (or 64 x 64) tiles and splits K into slices of at
// least 16 stages, up to two blocks per CU; a grid below a quarter of the
// CUs takes slices of 6 or more stages, up to one block per CU.  One round of
// 128 x 96 tiles over a long K (M 2048, N 1536, K 6144) splits in two.
// Measured at M 512 with FP32 x: N 1536 at K 6144 / 12288 / 2048 37 / 61 /
// 21 us instead of 70 / 127 / 25; N 256 at K 1536 10.6 instead of 18.
struct GemmPlan {
  int tm, tn, ks, slices;
  int rb;  // the registers-B kernel (tm, tn, ks unused)
};
constexpr int kMaxSplitK = 8;

// multi_split: a K split may take several weights (their planes are left to
// the caller, not summed).
GemmPlan plan_gemm(const g4_w4 *const *w, int nw, int rows, bool f32x, bool multi_split = false) {
  const int cus = cu_count() > 0 ? cu_count() : 256;
  if (w[0]->G % 2 != 0) return {2, 2, 1, 1};
  bool tiled = true;  // the packed-weight kernel reads every weight's tile copy
  for (int i = 0; i < nw; ++i) tiled = tiled && w[i]->tiles != nullptr;
  const int S = w[0]->G / 2;
  auto blocks = [&](int bm, int bn) {
    long tiles = 0;
    for (int i = 0; i < nw; ++i) tiles += (w[i]->N + bn - 1) / bn;
    return (long)((rows + bm - 1) / bm) * tiles;
  };
  bool n96 = true;
  for (int i = 0; i < nw; ++i) n96 = n96 && w[i]->N % 96 == 0;
  const int split_ok = nw == 1 || multi_split;  // summed K splits take one weight
  {
    // registers-B tiles: 128 x 192 (BF16 x) or 64 x 192 (FP32 x), split K
    // into slices of at least 8 stages while that keeps the grid within two
    // blocks per CU
    const long b = blocks(f32x ? 64 : 128, 192);
    if (tiled && b >= cus) return {0, 0, 0, 1, 1};
    if (tiled && split_ok) {
      int slices = 1;
      for (int k = 2; k <= kMaxSplitK; ++k)
        if (S % k == 0 && S / k >= 8 && b * k <= 2L * cus) slices = k;
      if (b * slices >= cus) return {0, 0, 0, slices, 1};
    }
  }
  // FP32 x holds two planes of x' in LDS: 128-row tiles then fit one block
  // per CU, and 64-row tiles run faster (M 512, N 6144: 33 vs 45 us)
  if (!f32x && blocks(128, 128) >= 2L * cus) return {4, 4, 2, 1};
  if (!f32x && n96 && blocks(128, 96) % cus == 0)
    return {4, 3, 2, split_ok && blocks(128, 96) == cus && S % 2 == 0 && S / 2 >= 16 ? 2 : 1};
  if (n96 && blocks(64, 96) % cus == 0) return {2, 3, 2, 1};
  if (blocks(64, 128) >= cus) return {2, 4, 2, 1};
  if (blocks(64, 64) >= cus || !split_ok) return {2, 2, 2, 1};
  const long b = n96 ? blocks(64, 96) : blocks(64, 64);
  int slices = 1;
  for (int k = 2; k <= kMaxSplitK; ++k)
    if (S % k == 0 && S / k >= 16 && b * k <= 2L * cus) slices = k;
  if (slices == 1 && b * 4 < cus)
    for (int k = 2; k <= kMaxSplitK; ++k)
      if (S % k == 0 && S / k >= 6 && b * k <= cus) slices = k;
  return {2, n96 ? 3 : 2, 2, slices};
}

template <int NX>
int launch_planned(const GemmPlan &pl, const g4_w4 *const *w, int nw, const uint4 *xt,
                   const int *xe, int rows, int Mp, void *const *y, bool y_bf16, float *part,
                   bool sum, bool glu) {
  constexpr int P = 4;
  const int sl = pl.slices;
  if (pl.rb) {
    // two blocks per CU, 3 stages; 128 x 192 tiles (64 x 192 with FP32 x,
    // whose two x' planes double the LDS per row), gate/up 64 x (128 + 128)
    if (glu)
      return launch_gemm_rb<4, 4, NX, 3, 2>(w, nw, xt, xe, rows, Mp, y, y_bf16, part, sl, sum,
                                            glu);
    return launch_gemm_rb<NX == 1 ? 8 : 4, 3, NX, 3, 2>(w, nw, xt, xe, rows, Mp, y, y_bf16, part,
                                                       sl, sum, glu);
  }
#define G4_GEMM_TILE(TM, TN, KS) \
  return launch_gemm<TM, TN, NX, KS, P>(w, nw, xt, xe, rows, Mp, y, y_bf16, part, sl, sum, glu)
  if (pl.ks == 1) G4_GEMM_TILE(2, 2, 1);
  if (pl.tm == 4 && pl.tn == 4) G4_GEMM_TILE(4, 4, 2);
  if constexpr (NX == 1) {
    if (pl.tm == 4 && pl.tn == 3) G4_GEMM_TILE(4, 3, 2);
  }
  if (pl.tn == 3) G4_GEMM_TILE(2, 3, 2);
  if (pl.tn == 4) G4_GEMM_TILE(2, 4, 2);
  G4_GEMM_TILE(2, 2, 2);
#undef G4_GEMM_TILE
}

// x' (and its low half), the row exponents and the K-slice planes, reused by
// every later call; g_ws_x: x' and exponents written by the producer of x.
Workspace g_ws, g_ws_x;

}  // namespace

namespace g4 {

// keep: when set and the plan splits K, the partial planes are left for the
// caller to add (keep->parts, ->n, ->stride) instead of summed into y.
// The GEMM scratch for one call: x' planes, row exponents and K-slice planes.
struct GemmScratch {
  GemmPlan plan;
  int Mp;
  uint4 *xt;
  int *xe;
  float *part;
};

// prepped: x' and the exponents live in their own scratch (g_ws_x), written
// by the producer of x while the GEMM scratch may still hold the producer's
// inputs (its K-slice planes).
// Rows padded to the tile height, and the byte offsets of the exponents and
// of the end of x' + exponents in a scratch buffer.
void xprep_layout(int K, int rows, bool f32x, int *Mp, size_t *eoff, size_t *xend) {
  *Mp = (rows + kRowPad - 1) / kRowPad * kRowPad;
  const size_t xt_bytes = (size_t)*Mp * K * 2 * (f32x ? 2 : 1);  // FP16 x' (hi [+ lo])
  *eoff = (xt_bytes + 255) & ~size_t(255);
  *xend = *eoff + (size_t)rows * 4;
}

int gemm_scratch(const g4_w4 *const *w, int nw, bool f32x, int rows, bool prepped,
                 GemmScratch *sc, const ExtScratch *ext, bool multi_split = false) {
  const g4_w4 *w0 = w[0];
  size_t eoff, xend;
  xprep_layout(w0->K, rows, f32x, &sc->Mp, &eoff, &xend);
  const size_t poff = prepped ? 0 : (xend + 255) & ~size_t(255);
  sc->plan = plan_gemm(w, nw, rows, f32x, multi_split);
  const size_t part_bytes =
      sc->plan.slices > 1 ? sc->plan.slices * splitk_pstride(w, nw, rows) * 4 : 0;
  void *ws = nullptr, *wx = nullptr;
  if (ext) {
    // one region: x', exponents, then the K-slice planes (x is never prepared here)
    if (prepped) return fail(G4_E_ARG, "%s: a prepared x needs the library scratch", ext->who);
    if (poff + part_bytes > ext->bytes)
      return fail(G4_E_ARG,
                  "%s: %d rows of in_dim %d (%s x) into out_dim %d need %zu bytes of scratch; "
                  "the static scratch holds %zu",
                  ext->who, rows, w0->K, f32x ? "FP32" : "BF16", w0->N, poff + part_bytes,
                  ext->bytes);
    sc->xt = static_cast<uint4 *>(ext->mem);
    sc->xe = reinterpret_cast<int *>(static_cast<char *>(ext->mem) + eoff);
    sc->part = reinterpret_cast<float *>(static_cast<char *>(ext->mem) + poff);
    return G4_OK;
  }
  if (poff + part_bytes > 0)
    if (int rc = g_ws.get(poff + part_bytes, &ws, "g4_w4_linear (prefill)")) return rc;
  if (prepped) {
    if (int rc = g_ws_x.get(xend, &wx, "g4_w4_linear (prefill, prepared x)")) return rc;
  } else {
    wx = ws;
  }
  sc->xt = static_cast<uint4 *>(wx);
  sc->xe = reinterpret_cast<int *>(static_cast<char *>(wx) + eoff);
  sc->part = reinterpret_cast<float *>(static_cast<char *>(ws) + poff);
  return G4_OK;
}

// x == nullptr: x' and the row exponents are already in the scratch
// (written by the producer after w4_gemm_prepare).
static int gemm_run(const g4_w4 *const *w, int nw, const void *x, bool f32x, int rows,
                    void *const *y, bool y_bf16, GemmParts *keep, bool glu = false,
                    const ExtScratch *ext = nullptr) {
  // weights whose joint grid still leaves CUs idle run one by one (each may
  // then split K); not with x' prepared, whose scratch is sized for the joint call
  const int cus = cu_count() > 0 ? cu_count() : 256;
  long tiles64 = 0;
  for (int i = 0; i < nw; ++i) tiles64 += (long)((rows + 63) / 64) * ((w[i]->N + 63) / 64);
  if (nw > 1 && tiles64 < cus && !glu && x && !keep) {
    for (int i = 0; i < nw; ++i)
      if (int rc = gemm_run(w + i, 1, x, f32x, rows, y + i, y_bf16, nullptr)) return rc;
    return G4_OK;
  }
  const g4_w4 *w0 = w[0];
  GemmScratch sc;
  if (int rc = gemm_scratch(w, nw, f32x, rows, !x, &sc, ext, keep && nw > 1)) return rc;
  const GemmPlan plan = sc.plan;
  const int Mp = sc.Mp;
  uint4 *xt = sc.xt;
  int *xe = sc.xe;
  float *part = sc.part;
  const bool sum = !keep || plan.slices == 1;
  if (keep) {  // one entry per weight, planes side by side
    size_t off = 0;
    for (int i = 0; i < nw; ++i) {
      keep[i].parts = sum ? static_cast<const float *>(y[i]) : part + off;
      keep[i].n = sum ? 1 : plan.slices;
      keep[i].stride = splitk_pstride(w, nw, rows);
      off += (size_t)rows * w[i]->N;
    }
  }
  if (!x)
    return f32x ? launch_planned<2>(plan, w, nw, xt, xe, rows, Mp, y, y_bf16, part, sum, glu)
                : launch_planned<1>(plan, w, nw, xt, xe, rows, Mp, y, y_bf16, part, sum, glu);
  const int cpt = fused_prep_cpt(w0->K, f32x);
  if (cpt) {
    const dim3 fgrid(Mp / kRowsFused);
#define G4_PREP_FUSED(F, C)                                                                   \
  hipLaunchKernelGGL((gemm_xprep_fused_kernel<F, C>), fgrid, dim3(kThreads), 0, stream(), x, \
                     rows, Mp, w0->K, xe, xt)
    if (f32x) {
      switch (cpt) {
        case 2: G4_PREP_FUSED(true, 2); break;
        case 4: G4_PREP_FUSED(true, 4); break;
        case 8: G4_PREP_FUSED(true, 8); break;
        case 12: G4_PREP_FUSED(true, 12); break;
        default: G4_PREP_FUSED(true, 16); break;
      }
    } else {
      switch (cpt) {
        case 2: G4_PREP_FUSED(false, 2); break;
        case 4: G4_PREP_FUSED(false, 4); break;
        case 8: G4_PREP_FUSED(false, 8); break;
        case 12: G4_PREP_FUSED(false, 12); break;
        case 16: G4_PREP_FUSED(false, 16); break;
        case 24: G4_PREP_FUSED(false, 24); break;
        default: G4_PREP_FUSED(false, 32); break;
      }
    }
#undef G4_PREP_FUSED
    G4_LAUNCH_CHECK("gemm_xprep_fused_kernel");
    return f32x ? launch_planned<2>(plan, w, nw, xt, xe, rows, Mp, y, y_bf16, part, sum, glu)
                : launch_planned<1>(plan, w, nw, xt, xe, rows, Mp, y, y_bf16, part, sum, glu);
  }
  const dim3 egrid((rows + kThreads / 64 - 1) / (kThreads / 64));
  const dim3 pgrid(Mp / kPrepTileM, (w0->K / 8 + kPrepTileC - 1) / kPrepTileC);
  if (f32x) {
    hipLaunchKernelGGL(gemm_xexp_kernel<true>, egrid, dim3(kThreads), 0, stream(), x, rows, w0->K,
                       xe);
    hipLaunchKernelGGL(gemm_xprep_kernel<true>, pgrid, dim3(kThreads), 0, stream(), x, xe, rows,
                       Mp, w0->K, xt);
  } else {
    hipLaunchKernelGGL(gemm_xexp_kernel<false>, egrid, dim3(kThreads), 0, stream(), x, rows,
                       w0->K, xe);
    hipLaunchKernelGGL(gemm_xprep_kernel<false>, pgrid, dim3(kThreads), 0, stream(), x, xe, rows,
                       Mp, w0->K, xt);
  }
  G4_LAUNCH_CHECK("gemm_xprep_kernel");
  return f32x ? launch_planned<2>(plan, w, nw, xt, xe, rows, Mp, y, y_bf16, part, sum, glu)
              : launch_planned<1>(plan, w, nw, xt, xe, rows, Mp, y, y_bf16, part, sum, glu);
}

int w4_gemm_multi(const g4_w4 *const *w, int nw, const void *x, bool f32x, int rows,
                  void *const *y, bool y_bf16) {
  return gemm_run(w, nw, x, f32x, rows, y, y_bf16, nullptr);
}

int w4_gemm(const g4_w4 *w, const void *x, bool f32x, int rows, void *y, bool y_bf16) {
  return gemm_run(&w, 1, x, f32x, rows, &y, y_bf16, nullptr);
}

int w4_gemm_ext(const g4_w4 *w, const void *x, bool f32x, int rows, void *y, bool y_bf16,
                const ExtScratch &ext) {
  return gemm_run(&w, 1, x, f32x, rows, &y, y_bf16, nullptr, false, &ext);
}

int w4_gemm_glu(const g4_w4 *gate, const g4_w4 *up, const float *x, int rows, float *act) {
  if (gate->N != up->N || gate->K != up->K)
    return fail(G4_E_ARG, "w4_gemm_glu: gate [%d, %d] and up [%d, %d] differ", gate->N, gate->K,
                up->N, up->K);
  const g4_w4 *w[2] = {gate, up};
  void *y[2] = {act, nullptr};
  return gemm_run(w, 2, x, true, rows, y, false, nullptr, true);
}

int w4_gemm_prepare(const g4_w4 *const *w, int nw, int rows, GemmXPrep *out) {
  // only the x' scratch: the GEMM scratch may still hold the producer's
  // inputs, and is sized by the GEMM call itself
  (void)nw;
  size_t eoff, xend;
  xprep_layout(w[0]->K, rows, true, &out->Mp, &eoff, &xend);
  void *wx = nullptr;
  if (int rc = g_ws_x.get(xend, &wx, "g4_w4_linear (prefill, prepared x)")) return rc;
  out->xt = static_cast<uint4 *>(wx);
  out->xe = reinterpret_cast<int *>(static_cast<char *>(wx) + eoff);
  return G4_OK;
}

int w4_gemm_multi_parts(const g4_w4 *const *w, int nw, const float *x, int rows,
                        float *const *y, GemmParts *out) {
  if (nw < 1 || nw > kMaxGemmSegs) return fail(G4_E_ARG, "w4_gemm_multi_parts: %d weights", nw);
  void *ys[kMaxGemmSegs];
  for (int i = 0; i < nw; ++i) {
    if (w[i]->K != w[0]->K)
      return fail(G4_E_ARG, "w4_gemm_multi_parts: in_dim %d and %d differ", w[0]->K, w[i]->K);
    ys[i] = y[i];
  }
  return gemm_run(w, nw, x, true, rows, ys, false, out);
}

int w4_gemm_parts(const g4_w4 *w, const float *x, int rows, float *y, GemmParts *out) {
  void *yv = y;
  return gemm_run(&w, 1, x, true, rows, &yv, false, out);
}

}  // namespace g4

// ---- allocation-free linear ------------------------------------------------
// The GEMM scratch of g4_w4_linear_noalloc: one static array per device,
// allocated with the code object when the library loads on a device and held
// until the process ends.  Host code must not pass `scratch` itself to a
// kernel (in host code the name is a host-side stand-in, not a device
// address): static_scratch_init looks up each device's address once, with
// that device current, and every launch takes that address.
constexpr size_t kStaticScratchBytes = size_t(64) << 20;
constexpr int kMaxScratchDevices = 64;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {
void *g_static_scratch[kMaxScratchDevices];
}  // namespace

namespace g4 {

int static_scratch_init(int device) {
  if (device < 0 || device >= kMaxScratchDevices)
    return fail(G4_E_ARG, "static scratch: device %d beyond %d", device, kMaxScratchDevices);
  if (g_static_scratch[device]) return G4_OK;
  void *p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p)
    return fail(G4_E_HIP, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
  g_static_scratch[device] = p;
  return G4_OK;
}

}  // namespace g4

G4_API int g4_w4_linear_noalloc(const g4_w4 *w, const void *x, int x_dtype, int rows, void *y,
                                int y_dtype) {
  G4_CHECK_INIT();
  void *mem = g_static_scratch[current_device()];
  if (!mem) return fail(G4_E_STATE, "g4_w4_linear_noalloc: static scratch not set up");
  const ExtScratch ext{mem, kStaticScratchBytes, "g4_w4_linear_noalloc"};
  const int rc = w4_linear_impl(w, x, x_dtype, rows, y, y_dtype, &ext, "g4_w4_linear_noalloc");
  return rc ? rc : ok();
}
