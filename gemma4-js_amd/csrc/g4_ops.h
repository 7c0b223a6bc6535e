// Launchers of the GPUOps kernels (g4_ops.hip) and of the fused head/argmax
// (g4_head.hip), shared by the C ABI and the model engine.  They enqueue on
// the library stream and do no operand checking: callers validate first.
#pragma once

#include <stddef.h>
#include <stdint.h>

struct g4_w4;

namespace g4 {

int launch_rms(const float *x, int rows, int width, const float *scale, float eps, float *y,
               const int *pos_dev);
int launch_add_scale(const float *a, const float *b, size_t n, float s, float *y);
int launch_scale(const float *a, size_t n, float s, float *y);
int launch_gelu_mul(const float *gate, const float *up, size_t n, float *y);
int launch_gelu_ple(const float *gate, const float *ple, int rows, int layer, int width,
                    int layers, float *y);
// x may be the sum of `parts` (<= 8) planes pstride floats apart (a GEMM's K
// slices), added in plane order.
int launch_norm_rope(const float *x, int rows, int heads, int hd, int pos0, const int *pos_dev,
                     const float *scale, int rope_angles, float base, float eps, float *y,
                     bool at_pos, int parts = 1, size_t pstride = 0);
// A prefill layer's q norm + RoPE, k norm + RoPE into the cache at
// *pos_dev + row, and v's RMS norm (no weights) into the cache, in one
// launch.  q, k and v are each the sum of qparts planes qpstride floats apart
// (the K slices of one GEMM launch; head dim at most 512).
int launch_norm_rope_qkv(const float *q, int qparts, size_t qpstride, const float *k,
                         const float *v, int rows, int heads, int hd, const int *pos_dev,
                         const float *qscale, const float *kscale, int rope_angles, float base,
                         float eps, float *qy, float *kc, float *vc);
// Floats of split scratch that launch_attention needs for up to max_keylen keys.
size_t attention_part_floats(int qrows, int heads, int hd, int max_keylen, int kpw);
// With xt, xe, Mp (w4_gemm_prepare of the GEMM that takes the [qrows, heads
// * hd] output) and x_done: where the matrix-core kernel runs and its 16-row
// blocks hold whole query rows (heads divides 16), the output leaves as that
// GEMM's x' instead of through `out`, and *x_done is set.
int launch_attention(const float *q, const float *k, const float *v, int qrows, int heads,
                     int hd, int keylen, int qpos0, const int *pos_dev, int max_keylen,
                     bool sliding, int window, int kpw, float *part, float *out,
                     void *xt = nullptr, int *xe = nullptr, int Mp = 0, bool *x_done = nullptr);
int launch_ple_mix(const float *proj, float pre_scale, const float *norm_scale,
                   const float *token_ple, int rows, int width, int layers, float eps,
                   float ple_scale, float out_scale, float *y);
int launch_embed(const uint16_t *E, int vocab, int width, const int *ids_dev, int n, float scale,
                 float *y);

// Fused one-token kernels (g4_fused.hip).  Inputs and r_out must not alias.
int fused_norm_linear(const float *a, const float *w1, float eps, const g4_w4 *const *w,
                      float *const *y, int n);
int fused_res_norm_linear(const float *a, const float *h, const float *w1, float c,
                          const float *w2, float eps, float *r_out, const g4_w4 *const *w,
                          float *const *y, int n);
int fused_res_norm_gate_up(const float *a, const float *h, const float *w1, float c,
                           const float *w2, float eps, float *r_out, const g4_w4 *gate,
                           const g4_w4 *up, float *act);
int fused_res_linear_gelu_mul(const float *a, int a_parts, const float *h, const float *w1,
                              float eps, float *r_out, const g4_w4 *w, const float *mul,
                              float *y);
int launch_rope_qkv(const float *qraw, const float *kraw, const float *vraw, int heads, int hd,
                    const int *pos_dev, const float *qnorm, const float *knorm, int rope_angles,
                    float base, float eps, float *q, float *kc, float *vc, bool own_kv);
// r = (h + rms(a) * w1) * c; x = rms(r) * w2 (x_out optional), a the sum of
// a_parts planes a_stride floats apart.
int launch_norm_chain(const float *a, const float *h, const float *w1, const float *w2, float c,
                      float eps, int rows, int width, float *r_out, float *x_out,
                      int a_parts = 1, size_t a_stride = 0);
// The same chain writing its GEMM input (x, or r without w2) as the prefill
// GEMM's x' (xt, xe, Mp from w4_gemm_prepare); r_out / x_out optional.
int launch_norm_chain_xprep(const float *a, int a_parts, size_t a_stride, const float *h,
                            const float *w1, const float *w2, float c, float eps, int rows,
                            int width, float *r_out, float *x_out, void *xt, int *xe, int Mp);
// y = gelu(gate) * ple[:, layer] (launch_gelu_ple) written as the next prefill
// GEMM's x' (xt, xe, Mp from w4_gemm_prepare), the gate the sum of `parts`
// K-slice planes pstride floats apart; y optional.  Fits: width <= 512, a
// multiple of 8, at most 8 planes.
bool gelu_ple_xprep_fits(int width, int parts);
int launch_gelu_ple_xprep(const float *gate, int parts, size_t pstride, const float *ple,
                          int layer, int layers, int width, int rows, float *y, void *xt,
                          int *xe, int Mp);

// RoPE (cos, sin) tables of the current position for up to kRopeSlots
// (base, head_dim, angles) variants, kRopeTable entries each.
constexpr int kRopeSlots = 4, kRopeTable = 256;
struct RopeSlots {
  float base[kRopeSlots];
  int hd[kRopeSlots], angles[kRopeSlots];
  int n;
};
// The decode step's first kernel: y = embedding row of ids[0] * scale, and
// the RoPE tables at *pos_dev.
int launch_token_start(const uint16_t *E, int vocab, int width, const int *ids_dev, float scale,
                       float *y, const int *pos_dev, const RopeSlots &slots, float2 *tab);
// One-query attention with the q/k norm + RoPE, the k/v cache append at
// *pos_dev and the split merge in one launch (head_dim 128, 256 or 512).
// count: heads * kCountStride ints (one 128-byte line per head), zero before
// the first launch (each launch leaves them 0).
constexpr int kCountStride = 32;
bool attn_rope_supported(int hd);
int attn_rope_splits(int max_keylen, bool sliding, int window);
int launch_attn_rope_dec(const float *qraw, const float *kraw, const float *vraw, int heads,
                         int hd, const int *pos_dev, const float *qnorm, const float *knorm,
                         const float2 *rope, int angles, float eps, float *kc, float *vc,
                         bool own_kv, bool sliding, int window, int max_keylen, float *part,
                         size_t part_floats, int *count, float *ctx);

// Head partials for the device argmax: per block (max value, first index).
size_t head_argmax_blocks(int rows);
int launch_bf16_head(const float *x, const uint16_t *E, int rows, int K, float *out, float scale,
                     float softcap, float2 *partials);
int launch_argmax_partials(const float2 *partials, int nparts, int *out_idx);
int launch_argmax(const float *x, int n, float2 *partials, int *out_idx);
size_t argmax_blocks(int n);

}  // namespace g4
