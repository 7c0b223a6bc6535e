// Decoder engine: Gemma4WebGPU (custom-webgpu/gemma4-webgpu.js:139-502) on the
// HIP kernels of this library.  The forward pass is the reference's op
// sequence (encodeLayer 215-301, forward 303-402, logits 404-431, greedy
// 441-481) with one MI355X-first change: the token position and the next
// token live in device memory.  Kernels read the position from there, and
// the last kernel of a step (argmax over the head partials) writes the next
// token and advances the position, so one recorded decode step (a HIP graph)
// is replayed for every generated token without a host round trip.
//
// Weights are borrowed (g4_w4 / g4_ple handles and the BF16 embedding stay
// owned by the caller); norm vectors are copied in.  Activation buffers and
// KV caches are allocated once, sized for max_seq positions.
#include <math.h>
#include <string.h>

#include <vector>

#include "g4_internal.h"
#include "g4_ops.h"

namespace {

using namespace g4;

constexpr int kNorms = 7;  // input, post_attn, pre_ffw, post_ffw, post_ple, q, k
constexpr int kProjs = 9;  // q, k, v, o, gate, up, down, ple_gate, ple_proj
// The one-token down projection is split over input slices of this width,
// at most this many (the PLE gate prologue adds the partial sums).
constexpr int kDownSlice = 1536, kDownMaxSlices = 8;

struct Layer {
  int hd = 0, inter = 0, full = 0, kv_src = -1, rope_angles = 0;
  int rope_slot = -1;  // RoPE table of the one-launch decode attention, -1: the op-by-op path
  float rope_base = 0.f;
  const g4_w4 *w[kProjs] = {};
  float *norm[kNorms] = {};
  float skip = 1.f;
  float *kc = nullptr, *vc = nullptr;  // own caches [max_seq, hd]
};

// One split attention pass needs this many keys per split (decode: small
// splits over many blocks; prefill: larger ones).
int kpw_for(int rows) { return rows <= 4 ? 4 : 64; }

// Final argmax reduction + advance: ids[0] = token, gen[pos + rows] = token,
// pos += rows.  One block.
__global__ __launch_bounds__(1024) void advance_kernel(const float2 *__restrict__ partials,
                                                       int nparts, int rows, int *__restrict__ ids,
                                                       int *__restrict__ pos,
                                                       int *__restrict__ gen, int gen_cap) {
  __shared__ float sv[16];
  __shared__ int si[16];
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  // U partials per thread per pass, all loads in flight together; indices
  // past the end re-read the last partial, which cannot change the result
  constexpr int U = 8;
  for (int b0 = threadIdx.x; b0 < nparts; b0 += 1024 * U) {
    float2 p[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = b0 + u * 1024;
      p[u] = partials[i < nparts ? i : nparts - 1];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float v = p[u].x;
      const int ix = __float_as_int(p[u].y);
      if (v > bv || (v == bv && ix < bi)) {
        bv = v;
        bi = ix;
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = bv;
    si[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 16; ++w)
      if (sv[w] > bv || (sv[w] == bv && si[w] < bi)) {
        bv = sv[w];
        bi = si[w];
      }
    const int tok = bi == 0x7fffffff ? -1 : bi;
    const int p = *pos + rows;
    ids[0] = tok;
    if (p < gen_cap) gen[p] = tok;
    *pos = p;
  }
}

}  // namespace

struct g4_gemma {
  g4_gemma_config cfg;
  std::vector<Layer> L;
  const g4_w4 *top = nullptr;
  float *ple_norm = nullptr, *final_norm = nullptr;
  const uint16_t *E = nullptr;
  const g4_ple *ple = nullptr;
  const uint16_t *ple_dense = nullptr;  // BF16 [vocab, layers * ple_dim], when no W4 table
  int max_rows = 0, hd_max = 0, inter_max = 0, ple_total = 0;
  int cache_len = 0;  // host mirror of the KV length (KVCache.length)
  // device state
  int *ids = nullptr, *pos = nullptr, *gen = nullptr;
  float *h[2] = {}, *pre = nullptr, *qraw = nullptr, *q = nullptr, *kraw = nullptr,
        *vraw = nullptr, *ctx = nullptr, *attn = nullptr, *ares = nullptr, *pf = nullptr,
        *gate = nullptr, *up = nullptr, *act = nullptr, *down = nullptr, *downp = nullptr,
        *fres = nullptr, *pg = nullptr, *pm = nullptr, *pp = nullptr, *tokple = nullptr,
        *proj = nullptr, *perlayer = nullptr, *last = nullptr, *logits = nullptr,
        *part = nullptr;
  float2 *hpart = nullptr;
  size_t part_floats = 0;
  RopeSlots rope_slots = {};
  float2 *rope_tab = nullptr;  // [kRopeSlots][kRopeTable] at the current position
  int *attn_count = nullptr;   // [heads * kCountStride] split counters of the decode attention
  std::vector<void *> allocs;
  g4_cmdbuf *step = nullptr;  // recorded one-token decode step
};

namespace {

int galloc(g4_gemma *m, size_t bytes, void **p) {
  int rc = device_alloc(bytes, p);
  if (!rc) m->allocs.push_back(*p);
  return rc;
}

template <typename T>
int galloc_n(g4_gemma *m, size_t n, T **p) {
  return galloc(m, n * sizeof(T), reinterpret_cast<void **>(p));
}

void drop_step(g4_gemma *m) {
  if (m->step) {
    g4_cmdbuf_free(m->step);
    m->step = nullptr;
  }
}

int check_ready(const g4_gemma *m) {
  const g4_gemma_config &c = m->cfg;
  if (!m->top || !m->ple_norm || !m->final_norm || !m->E || (!m->ple && !m->ple_dense))
    return fail(G4_E_STATE, "g4_gemma: top-level weights are not set (embedding, PLE table, "
                            "per-layer projection, PLE norm, final norm)");
  for (int i = 0; i < c.layers; ++i) {
    const Layer &l = m->L[i];
    for (int p = 0; p < kProjs; ++p) {
      const bool needed = !((p == G4_PROJ_K || p == G4_PROJ_V) && l.kv_src >= 0);
      if (needed && !l.w[p])
        return fail(G4_E_STATE, "g4_gemma: layer %d projection %d is not set", i, p);
    }
    for (int n = 0; n < kNorms; ++n) {
      const bool needed = !(n == G4_NORM_K && l.kv_src >= 0);
      if (needed && !l.norm[n])
        return fail(G4_E_STATE, "g4_gemma: layer %d norm %d is not set", i, n);
    }
  }
  return G4_OK;
}

// The token rows of the per-layer embeddings into m->tokple (FP32): gathered
// and dequantized from the W4 table (reader.pleRowsToGpu), or, for a
// checkpoint with a dense BF16 embed_tokens_per_layer, its rows widened
// (bf16Rows + uploadF32; gemma4-webgpu.js:198-215).
int token_ple(g4_gemma *m, int rows) {
  const g4_gemma_config &c = m->cfg;
  if (m->ple) return g4_ple_gather_dev(m->ple, m->ids, rows, m->tokple, G4_F32);
  return launch_embed(m->ple_dense, c.vocab, c.layers * c.ple_dim, m->ids, rows, 1.f, m->tokple);
}

// One token (a decode step) on the fused kernels: per layer q/k/v GEMV with
// the norm chain of the previous layer's end in its prologue, one RoPE/cache
// kernel, attention, o GEMV, gate/up GEMV with the post-attention chain in its
// prologue and gelu(gate) * up in its epilogue, down GEMV, PLE gate GEMV with
// the post-FFW residual in its prologue and gelu * PLE in its epilogue, PLE
// projection GEMV: 9 launches instead of the reference's 20-24 dispatches.
int run_token(g4_gemma *m, bool graph) {
  const g4_gemma_config &c = m->cfg;
  const int H = c.hidden, P = c.ple_dim, NL = c.layers;
  const float eps = c.eps;
  int rc;
  if ((rc = launch_token_start(m->E, c.vocab, H, m->ids, (float)sqrt((double)H), m->h[0], m->pos,
                               m->rope_slots, m->rope_tab)))
    return rc;
  if ((rc = token_ple(m, 1))) return rc;
  if ((rc = g4_w4_linear(m->top, m->h[0], G4_F32, 1, m->proj, G4_F32))) return rc;
  // ops.scale(proj, 1/sqrt(hidden)) happens inside the PLE mix
  if ((rc = launch_ple_mix(m->proj, (float)(1.0 / sqrt((double)H)), m->ple_norm, m->tokple, 1,
                           P, NL, 1e-6f, 16.f, 0.7071067811865476f, m->perlayer)))
    return rc;
  const int keylen_host = m->cache_len + 1;
  const int max_keylen = graph ? c.max_seq : keylen_host;
  float *hid = m->h[0];
  for (int i = 0; i < NL; ++i) {
    const Layer &l = m->L[i];
    const bool own = l.kv_src < 0;
    const g4_w4 *w[3] = {l.w[G4_PROJ_Q], l.w[G4_PROJ_K], l.w[G4_PROJ_V]};
    float *y[3] = {m->qraw, m->kraw, m->vraw};
    const int nseg = own ? 3 : 1;
    if (i == 0) {
      rc = fused_norm_linear(hid, l.norm[G4_NORM_INPUT], eps, w, y, nseg);
    } else {
      // the previous layer's output (fres + rms(pp) * w) * skip is this layer's hidden
      const Layer &p = m->L[i - 1];
      float *next = m->h[i & 1];
      rc = fused_res_norm_linear(m->pp, m->fres, p.norm[G4_NORM_POST_PLE], p.skip,
                                 l.norm[G4_NORM_INPUT], eps, next, w, y, nseg);
      hid = next;
    }
    if (rc) return rc;
    const Layer &src = own ? l : m->L[l.kv_src];
    if (l.rope_slot >= 0) {
      // norm + RoPE, cache append, attention and split merge in one launch
      rc = launch_attn_rope_dec(m->qraw, m->kraw, m->vraw, c.heads, l.hd, m->pos,
                                l.norm[G4_NORM_Q], l.norm[G4_NORM_K],
                                m->rope_tab + (size_t)l.rope_slot * kRopeTable, l.rope_angles,
                                eps, src.kc, src.vc, own, !l.full, c.window, max_keylen,
                                m->part, m->part_floats, m->attn_count, m->ctx);
      if (rc) return rc;
    } else {
      if ((rc = launch_rope_qkv(m->qraw, m->kraw, m->vraw, c.heads, l.hd, m->pos,
                                l.norm[G4_NORM_Q], l.norm[G4_NORM_K], l.rope_angles,
                                l.rope_base, eps, m->q, l.kc, l.vc, own)))
        return rc;
      if ((rc = launch_attention(m->q, src.kc, src.vc, 1, c.heads, l.hd, keylen_host, 0, m->pos,
                                 max_keylen, !l.full, c.window, kpw_for(1), m->part, m->ctx)))
        return rc;
    }
    if ((rc = g4_w4_linear(l.w[G4_PROJ_O], m->ctx, G4_F32, 1, m->attn, G4_F32))) return rc;
    if ((rc = fused_res_norm_gate_up(m->attn, hid, l.norm[G4_NORM_POST_ATTN], 1.f,
                                     l.norm[G4_NORM_PRE_FFW], eps, m->ares, l.w[G4_PROJ_GATE],
                                     l.w[G4_PROJ_UP], m->act)))
      return rc;
    // down: split over 1536-wide input slices (per-slice partial sums that the
    // PLE gate's prologue adds) when the input is 2..8 slices long
    const g4_w4 *wd = l.w[G4_PROJ_DOWN];
    int parts = 0;
    if (wd->K % kDownSlice == 0 && wd->K / kDownSlice <= kDownMaxSlices) {
      parts = launch_gemv1_split(wd, m->act, m->downp);
      if (parts < 0) return -parts;
    }
    if (parts == 0) {
      if ((rc = g4_w4_linear(wd, m->act, G4_F32, 1, m->down, G4_F32))) return rc;
      parts = 1;
    }
    if ((rc = fused_res_linear_gelu_mul(parts > 1 ? m->downp : m->down, parts, m->ares,
                                        l.norm[G4_NORM_POST_FFW], eps, m->fres,
                                        l.w[G4_PROJ_PLE_GATE], m->perlayer + (size_t)i * P,
                                        m->pm)))
      return rc;
    if ((rc = g4_w4_linear(l.w[G4_PROJ_PLE_PROJ], m->pm, G4_F32, 1, m->pp, G4_F32))) return rc;
  }
  // last layer's output, then the final norm (gemma4-webgpu.js:394-400)
  const Layer &last = m->L[NL - 1];
  return launch_norm_chain(m->pp, m->fres, last.norm[G4_NORM_POST_PLE], m->final_norm, last.skip,
                           eps, 1, H, nullptr, m->last);
}

// y = x . W^T for prefill rows (FP32), a GEMM's K slices left unsummed for a
// consumer that adds them; the GEMV path (up to kMaxGemvRows rows) writes y.
int linear_parts(const g4_w4 *w, const float *x, int rows, float *y, GemmParts *p) {
  if (rows > kMaxGemvRows) return w4_gemm_parts(w, x, rows, y, p);
  *p = {y, 1, 0};
  return g4_w4_linear(w, x, G4_F32, rows, y, G4_F32);
}

// Enqueue the forward of `rows` tokens whose ids are in m->ids and whose first
// position is *m->pos; leaves the final-norm last row in m->last.
// The diagnostic read-outs of forward(ids, pos, {diagnostic: true})
// (gemma4-webgpu.js:311-397): device buffers, each optional.
struct Diag {
  float *top_hidden = nullptr;  // [rows, hidden]: the scaled embedding rows
  float *top_ple = nullptr;     // [rows, layers * ple_dim]: pleMix's per-layer inputs
  float *layers = nullptr;      // [layers, rows, hidden]: every layer's output rows
  int stage_layer = -1;         // the layer whose encodeLayer stages go to `stages`
  float *stages = nullptr;      // the stages at the offsets of diag_stage_offsets
  size_t off[G4_STAGES + 1] = {};
};

// Floats of each encodeLayer stage of `layer` at `rows` rows (the reference's
// probe counts, gemma4-webgpu.js:224-309; the k/v stages of a shared-KV layer
// are empty) and their offsets in a stage buffer.
void diag_stage_offsets(const g4_gemma *m, int layer, int rows, size_t *off) {
  const g4_gemma_config &c = m->cfg;
  const Layer &l = m->L[layer];
  const size_t R = (size_t)rows, H = c.hidden, QD = (size_t)c.heads * l.hd;
  const size_t kv = l.kv_src < 0 ? R * l.hd : 0;
  const size_t n[G4_STAGES] = {R * H, R * QD, R * QD, kv, kv, kv, kv, R * QD, R * H, R * H,
                               R * H, R * H, R * l.inter, R * l.inter, R * l.inter, R * H, R * H,
                               R * H, R * c.ple_dim, R * c.ple_dim, R * H, R * H, R * H};
  off[0] = 0;
  for (int i = 0; i < G4_STAGES; ++i) off[i + 1] = off[i] + n[i];
}

int run_layers(g4_gemma *m, int rows, bool graph, const Diag *dg = nullptr) {
  if (rows == 1 && !dg) return run_token(m, graph);
  const g4_gemma_config &c = m->cfg;
  const int H = c.hidden, P = c.ple_dim, NL = c.layers;
  const float eps = c.eps;
  int rc;
  auto cp = [&](float *dst, const float *src, size_t n) -> int {
    const hipError_t e =
        hipMemcpyAsync(dst, src, n * 4, hipMemcpyDeviceToDevice, stream());
    return e == hipSuccess ? G4_OK : fail(G4_E_HIP, "diagnostic copy: %s", hipGetErrorString(e));
  };
  // Top level (gemma4-webgpu.js:316-323): scaled embedding, PLE rows,
  // per-layer projection, pleMix.
  if ((rc = launch_embed(m->E, c.vocab, H, m->ids, rows, (float)sqrt((double)H), m->h[0])))
    return rc;
  if ((rc = token_ple(m, rows))) return rc;
  if ((rc = g4_w4_linear(m->top, m->h[0], G4_F32, rows, m->proj, G4_F32))) return rc;
  if ((rc = launch_ple_mix(m->proj, (float)(1.0 / sqrt((double)H)), m->ple_norm, m->tokple,
                           rows, P, NL, 1e-6f, 16.f, 0.7071067811865476f, m->perlayer)))
    return rc;
  if (dg && dg->top_hidden && (rc = cp(dg->top_hidden, m->h[0], (size_t)rows * H))) return rc;
  if (dg && dg->top_ple && (rc = cp(dg->top_ple, m->perlayer, (size_t)rows * NL * P))) return rc;

  const int keylen_host = m->cache_len + rows;  // prefill calls know it; graphs read *pos
  const int max_keylen = graph ? c.max_seq : keylen_host;
  const int kpw = kpw_for(rows);
  int cur = 0;
  // Each norm -> residual add -> norm run of encodeLayer is one norm_chain
  // launch: post-attention norm + residual + pre-FFN norm; post-FFN norm +
  // residual; post-PLE norm + residual + layer scalar + the next layer's
  // input norm (so only layer 0 runs its input norm alone).
  //
  // With the GEMM path (more than kMaxGemvRows rows) the chains whose output
  // feeds a GEMM (q/k/v, gate/up, PLE gate) also write it as the GEMM's x'
  // (launch_norm_chain_xprep after w4_gemm_prepare), so those GEMMs skip
  // their x pre-pass.
  // (the diagnostic forward keeps every stage as its own buffer)
  const bool gemm = rows > kMaxGemvRows && !dg;
  if ((rc = launch_rms(m->h[0], rows, H, m->L[0].norm[G4_NORM_INPUT], eps, m->pre, nullptr)))
    return rc;
  bool pre_prepped = false;  // x' of m->pre already in the GEMM's prepared scratch
  for (int i = 0; i < NL; ++i) {
    const Layer &l = m->L[i];
    float *hid = m->h[cur], *out = m->h[cur ^ 1];
    // this layer's stage buffer (diagnostic forward), or null
    float *sb = dg && dg->stages && i == dg->stage_layer ? dg->stages : nullptr;
    auto stage = [&](int st, const float *src) -> int {
      const size_t n = dg->off[st + 1] - dg->off[st];
      return n ? cp(sb + dg->off[st], src, n) : G4_OK;
    };
    // encodeLayer (gemma4-webgpu.js:215-301); m->pre holds rms(hid) * input norm
    // q, and k/v for a layer with its own cache, from one pre-pass and launch
    const g4_w4 *qkv[3] = {l.w[G4_PROJ_Q], l.w[G4_PROJ_K], l.w[G4_PROJ_V]};
    void *qkv_out[3] = {m->qraw, m->kraw, m->vraw};
    const int nqkv = l.kv_src < 0 ? 3 : 1;
    GemmParts qp = {m->qraw, 1, 0};
    const float *kin = m->kraw, *vin = m->vraw;
    if (pre_prepped && nqkv == 1) {  // q alone: its K slices go to the q norm unsummed
      rc = w4_gemm_parts(qkv[0], nullptr, rows, m->qraw, &qp);
    } else if (pre_prepped) {
      // q, k and v in one launch that may split K: the q/k/v norms add the slices
      float *outs[3] = {m->qraw, m->kraw, m->vraw};
      GemmParts p3[3];
      rc = w4_gemm_multi_parts(qkv, 3, nullptr, rows, outs, p3);
      qp = p3[0];
      kin = p3[1].parts;
      vin = p3[2].parts;
    } else
      rc = g4_w4_linear_multi(qkv, nqkv, m->pre, G4_F32, rows, qkv_out, G4_F32);
    if (rc) return rc;
    if (sb && ((rc = stage(G4_STAGE_PRE_ATTENTION, m->pre)) || (rc = stage(G4_STAGE_Q_RAW, m->qraw))))
      return rc;
    if (l.kv_src < 0) {
      // q, and KVCache.append: k/v rows go straight to positions pos .. pos + rows - 1
      if ((rc = launch_norm_rope_qkv(qp.parts, qp.n, qp.stride, kin, vin, rows, c.heads,
                                     l.hd, m->pos, l.norm[G4_NORM_Q], l.norm[G4_NORM_K],
                                     l.rope_angles, l.rope_base, eps, m->q, l.kc, l.vc)))
        return rc;
    } else if ((rc = launch_norm_rope(qp.parts, rows, c.heads, l.hd, 0, m->pos,
                                      l.norm[G4_NORM_Q], l.rope_angles, l.rope_base, eps, m->q,
                                      false, qp.n, qp.stride))) {
      return rc;
    }
    if (sb && (rc = stage(G4_STAGE_Q_NORM_ROPE, m->q))) return rc;
    const Layer &src = l.kv_src >= 0 ? m->L[l.kv_src] : l;
    if (l.kv_src < 0) {
      if (sb) {
        const size_t at = (size_t)m->cache_len * l.hd;  // the appended rows
        if ((rc = stage(G4_STAGE_K_RAW, m->kraw)) || (rc = stage(G4_STAGE_V_RAW, m->vraw)) ||
            (rc = stage(G4_STAGE_K_NORM_ROPE, l.kc + at)) || (rc = stage(G4_STAGE_V_NORM, l.vc + at)))
          return rc;
      }
    }
    // with the GEMM path, attention may write the o projection's x' itself
    const g4_w4 *ow = l.w[G4_PROJ_O];
    GemmXPrep oxp = {nullptr, nullptr, 0};
    bool o_prepped = false;
    if (gemm && (rc = w4_gemm_prepare(&ow, 1, rows, &oxp))) return rc;
    if ((rc = launch_attention(m->q, src.kc, src.vc, rows, c.heads, l.hd, keylen_host, 0, m->pos,
                               max_keylen, !l.full, c.window, kpw, m->part, m->ctx, oxp.xt,
                               oxp.xe, oxp.Mp, gemm ? &o_prepped : nullptr)))
      return rc;
    if (sb && (rc = stage(G4_STAGE_ATTENTION_CONTEXT, m->ctx))) return rc;
    GemmParts op;
    if (dg) {  // the projection whole (no K slices left for the chain to add)
      if ((rc = g4_w4_linear(ow, m->ctx, G4_F32, rows, m->attn, G4_F32))) return rc;
      op = {m->attn, 1, 0};
    } else if (o_prepped) {
      if ((rc = w4_gemm_parts(ow, nullptr, rows, m->attn, &op))) return rc;
    } else if ((rc = linear_parts(ow, m->ctx, rows, m->attn, &op))) {
      return rc;
    }
    if (sb) {
      float *pan = sb + dg->off[G4_STAGE_POST_ATTENTION_NORM];
      if ((rc = stage(G4_STAGE_ATTENTION_OUTPUT, m->attn)) ||
          (rc = launch_rms(m->attn, rows, H, l.norm[G4_NORM_POST_ATTN], eps, pan, nullptr)))
        return rc;
    }
    const g4_w4 *gu[2] = {l.w[G4_PROJ_GATE], l.w[G4_PROJ_UP]};
    if (gemm) {  // gate, up and gelu(gate) * up in one GEMM launch on the chain's x'
      GemmXPrep xp;
      if ((rc = w4_gemm_prepare(gu, 2, rows, &xp))) return rc;
      if ((rc = launch_norm_chain_xprep(op.parts, op.n, op.stride, hid,
                                        l.norm[G4_NORM_POST_ATTN], l.norm[G4_NORM_PRE_FFW], 1.f,
                                        eps, rows, H, m->ares, nullptr, xp.xt, xp.xe, xp.Mp)))
        return rc;
      if ((rc = w4_gemm_glu(gu[0], gu[1], nullptr, rows, m->act))) return rc;
    } else {
      if ((rc = launch_norm_chain(op.parts, hid, l.norm[G4_NORM_POST_ATTN],
                                  l.norm[G4_NORM_PRE_FFW], 1.f, eps, rows, H, m->ares, m->pf,
                                  op.n, op.stride)))
        return rc;
      void *gu_out[2] = {m->gate, m->up};
      if ((rc = g4_w4_linear_multi(gu, 2, m->pf, G4_F32, rows, gu_out, G4_F32))) return rc;
      if ((rc = launch_gelu_mul(m->gate, m->up, (size_t)rows * l.inter, m->act))) return rc;
    }
    if (sb && ((rc = stage(G4_STAGE_ATTENTION_RESIDUAL, m->ares)) ||
               (rc = stage(G4_STAGE_PRE_FFW, m->pf)) || (rc = stage(G4_STAGE_MLP_GATE, m->gate)) ||
               (rc = stage(G4_STAGE_MLP_UP, m->up)) || (rc = stage(G4_STAGE_MLP_ACTIVATED, m->act))))
      return rc;
    GemmParts dp;
    if (dg) {
      if ((rc = g4_w4_linear(l.w[G4_PROJ_DOWN], m->act, G4_F32, rows, m->down, G4_F32))) return rc;
      dp = {m->down, 1, 0};
    } else if ((rc = linear_parts(l.w[G4_PROJ_DOWN], m->act, rows, m->down, &dp))) {
      return rc;
    }
    if (sb) {
      float *pfn = sb + dg->off[G4_STAGE_POST_FFW_NORM];
      if ((rc = stage(G4_STAGE_FFW_OUTPUT, m->down)) ||
          (rc = launch_rms(m->down, rows, H, l.norm[G4_NORM_POST_FFW], eps, pfn, nullptr)))
        return rc;
    }
    const g4_w4 *pgw = l.w[G4_PROJ_PLE_GATE], *ppw = l.w[G4_PROJ_PLE_PROJ];
    bool ple_done = false;
    if (gemm) {  // the residual itself is the PLE gate's input
      GemmXPrep xp;
      if ((rc = w4_gemm_prepare(&pgw, 1, rows, &xp))) return rc;
      if ((rc = launch_norm_chain_xprep(dp.parts, dp.n, dp.stride, m->ares,
                                        l.norm[G4_NORM_POST_FFW], nullptr, 1.f, eps, rows, H,
                                        m->fres, nullptr, xp.xt, xp.xe, xp.Mp)))
        return rc;
      if (!gelu_ple_xprep_fits(P, 1)) {
        if ((rc = w4_gemm(pgw, nullptr, true, rows, m->pg, false))) return rc;
      } else {
        // the gate's K slices (at most 8) go unsummed to gelu·ple, which writes
        // the PLE projection's x': the slice sum and the projection's pre-pass
        // are skipped
        GemmParts gp;
        GemmXPrep pxp;
        if ((rc = w4_gemm_parts(pgw, nullptr, rows, m->pg, &gp)) ||
            (rc = w4_gemm_prepare(&ppw, 1, rows, &pxp)) ||
            (rc = launch_gelu_ple_xprep(gp.parts, gp.n, gp.stride, m->perlayer, i, NL, P, rows,
                                        m->pm, pxp.xt, pxp.xe, pxp.Mp)) ||
            (rc = w4_gemm(ppw, nullptr, true, rows, m->pp, false)))
          return rc;
        ple_done = true;
      }
    } else {
      if ((rc = launch_norm_chain(dp.parts, m->ares, l.norm[G4_NORM_POST_FFW], nullptr, 1.f, eps,
                                  rows, H, m->fres, nullptr, dp.n, dp.stride)))
        return rc;
      if ((rc = g4_w4_linear(pgw, m->fres, G4_F32, rows, m->pg, G4_F32))) return rc;
    }
    if (!ple_done) {
      if ((rc = launch_gelu_ple(m->pg, m->perlayer, rows, i, P, NL, m->pm))) return rc;
      if ((rc = g4_w4_linear(ppw, m->pm, G4_F32, rows, m->pp, G4_F32))) return rc;
    }
    if (sb) {
      float *pln = sb + dg->off[G4_STAGE_PLE_NORMALIZED];
      if ((rc = stage(G4_STAGE_FFW_RESIDUAL, m->fres)) || (rc = stage(G4_STAGE_PLE_GATE, m->pg)) ||
          (rc = stage(G4_STAGE_PLE_MODULATED, m->pm)) ||
          (rc = stage(G4_STAGE_PLE_PROJECTED, m->pp)) ||
          (rc = launch_rms(m->pp, rows, H, l.norm[G4_NORM_POST_PLE], eps, pln, nullptr)))
        return rc;
    }
    const bool last = i + 1 == NL;
    pre_prepped = gemm && !last;
    if (pre_prepped) {  // the next layer's q/k/v input, as that GEMM's x'
      const Layer &nx = m->L[i + 1];
      const g4_w4 *nq = nx.w[G4_PROJ_Q];
      GemmXPrep xp;
      if ((rc = w4_gemm_prepare(&nq, 1, rows, &xp))) return rc;
      if ((rc = launch_norm_chain_xprep(m->pp, 1, 0, m->fres, l.norm[G4_NORM_POST_PLE],
                                        nx.norm[G4_NORM_INPUT], l.skip, eps, rows, H, out,
                                        nullptr, xp.xt, xp.xe, xp.Mp)))
        return rc;
    } else if ((rc = launch_norm_chain(m->pp, m->fres, l.norm[G4_NORM_POST_PLE],
                                       last ? nullptr : m->L[i + 1].norm[G4_NORM_INPUT], l.skip,
                                       eps, rows, H, out, last ? nullptr : m->pre))) {
      return rc;
    }
    if (sb && (rc = stage(G4_STAGE_OUTPUT, out))) return rc;
    if (dg && dg->layers && (rc = cp(dg->layers + (size_t)i * rows * H, out, (size_t)rows * H)))
      return rc;
    cur ^= 1;
  }
  // final norm of the last row (gemma4-webgpu.js:394-400)
  return launch_rms(m->h[cur] + (size_t)(rows - 1) * H, 1, H, m->final_norm, eps, m->last,
                    nullptr);
}

// Head over the whole vocabulary with per-block argmax partials, then the
// advance kernel (token -> ids[0], gen[pos + rows]; pos += rows).
int run_head(g4_gemma *m, int rows) {
  const g4_gemma_config &c = m->cfg;
  int rc = launch_bf16_head(m->last, m->E, c.vocab, c.hidden, m->logits, 1.f, c.softcap,
                            m->hpart);
  if (rc) return rc;
  const int nparts = (int)head_argmax_blocks(c.vocab);
  hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1024), 0, stream(), m->hpart, nparts, rows,
                     m->ids, m->pos, m->gen, c.max_seq + 1);
  G4_LAUNCH_CHECK("advance_kernel");
  return G4_OK;
}

int stage_ids(g4_gemma *m, const int32_t *ids, int n, int start_pos) {
  const g4_gemma_config &c = m->cfg;
  if (n <= 0) return fail(G4_E_ARG, "g4_gemma: token count must be positive, got %d", n);
  if (n > m->max_rows) return fail(G4_E_ARG, "g4_gemma: %d tokens exceed max_seq %d", n, m->max_rows);
  // KVCache.append checks (gemma4-webgpu.js:128-130)
  if (start_pos != m->cache_len)
    return fail(G4_E_ARG, "KV append position %d != cache length %d", start_pos, m->cache_len);
  if (start_pos + n > c.max_seq)
    return fail(G4_E_RANGE, "KV cache capacity %d exceeded", c.max_seq);
  for (int i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= c.vocab)
      return fail(G4_E_RANGE, "token id %d out of range [0, %d)", ids[i], c.vocab);
  G4_HIP_TRY(hipMemcpyAsync(m->ids, ids, (size_t)n * 4, hipMemcpyHostToDevice, stream()));
  G4_HIP_TRY(hipMemcpyAsync(m->pos, &start_pos, 4, hipMemcpyHostToDevice, stream()));
  // the host buffers above may be pageable stack/heap memory: wait for the copies
  G4_HIP_TRY(hipStreamSynchronize(stream()));
  return G4_OK;
}

int upload_f32(g4_gemma *m, float **dst, const float *src, int n) {
  if (!src) return fail(G4_E_ARG, "g4_gemma: null norm vector");
  if (!*dst) {
    int rc = galloc_n(m, (size_t)n, dst);
    if (rc) return rc;
  }
  G4_HIP_TRY(hipMemcpyAsync(*dst, src, (size_t)n * 4, hipMemcpyHostToDevice, stream()));
  G4_HIP_TRY(hipStreamSynchronize(stream()));
  return G4_OK;
}

}  // namespace

// ---- C ABI ---------------------------------------------------------------------

G4_API int g4_gemma_e2b_config(int max_seq, g4_gemma_config *c) {
  if (!c) return fail(G4_E_ARG, "g4_gemma_e2b_config: null config");
  memset(c, 0, sizeof *c);
  // gemma4-webgpu.js:12 (HIDDEN, PLE, LAYERS, HEADS) and spec(i) (65-77)
  c->hidden = 1536;
  c->heads = 8;
  c->ple_dim = 256;
  c->vocab = 262144;
  c->layers = 35;
  c->max_seq = max_seq;
  c->window = 512;
  c->eps = 1e-6f;
  c->softcap = 30.f;
  for (int i = 0; i < 35; ++i) {
    const bool full = (i + 1) % 5 == 0;
    c->head_dim[i] = full ? 512 : 256;
    c->intermediate[i] = i < 15 ? 6144 : 12288;
    c->full[i] = full ? 1 : 0;
    // layers >= 15 read the cache of layer 13 (sliding) or 14 (full)
    c->kv_source[i] = i < 15 ? -1 : (full ? 14 : 13);
    c->rope_base[i] = full ? 1000000.f : 10000.f;
    c->rope_prop[i] = full ? 0.25f : 1.f;
  }
  return ok();
}

// The prefill's norm chains hold one hidden row per block (2048 values).
constexpr int kMaxHidden = 2048;

G4_API int g4_gemma_create(const g4_gemma_config *cfg, g4_gemma **out) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (!cfg || !out) return fail(G4_E_ARG, "g4_gemma_create: null argument");
  *out = nullptr;
  const g4_gemma_config &c = *cfg;
  if (c.layers <= 0 || c.layers > G4_GEMMA_MAX_LAYERS || c.hidden <= 0 || c.hidden % 32 != 0 ||
      c.hidden > kMaxHidden || c.heads <= 0 || c.heads > 8 || c.ple_dim <= 0 ||
      c.ple_dim % 32 != 0 || c.vocab <= 0 || c.max_seq <= 0 || c.window <= 0)
    return fail(G4_E_ARG,
                "g4_gemma_create: bad config (layers %d <= %d, hidden %d multiple of 32 <= "
                "2048, heads %d <= 8, ple_dim %d multiple of 32, vocab %d, max_seq %d)",
                c.layers, G4_GEMMA_MAX_LAYERS, c.hidden, c.heads, c.ple_dim, c.vocab, c.max_seq);
  for (int i = 0; i < c.layers; ++i) {
    const int hd = c.head_dim[i];
    if (hd != 64 && hd != 128 && hd != 256 && hd != 512)
      return fail(G4_E_ARG, "g4_gemma_create: layer %d head_dim %d (64, 128, 256 or 512)", i, hd);
    if (c.intermediate[i] <= 0 || c.intermediate[i] % 32 != 0)
      return fail(G4_E_ARG, "g4_gemma_create: layer %d intermediate %d", i, c.intermediate[i]);
    const int s = c.kv_source[i];
    if (s >= i || s < -1 || (s >= 0 && (c.kv_source[s] != -1 || c.head_dim[s] != hd)))
      return fail(G4_E_ARG,
                  "g4_gemma_create: layer %d kv_source %d must be an earlier layer with its own "
                  "cache and the same head_dim",
                  i, s);
    if (c.rope_prop[i] < 0.f || c.rope_prop[i] > 1.f || !(c.rope_base[i] > 0.f))
      return fail(G4_E_ARG, "g4_gemma_create: layer %d rope base %g / proportion %g", i,
                  c.rope_base[i], c.rope_prop[i]);
  }
  g4_gemma *m = new g4_gemma();
  m->cfg = c;
  m->L.resize(c.layers);
  m->max_rows = c.max_seq;
  m->ple_total = c.layers * c.ple_dim;
  for (int i = 0; i < c.layers; ++i) {
    Layer &l = m->L[i];
    l.hd = c.head_dim[i];
    l.inter = c.intermediate[i];
    l.full = c.full[i];
    l.kv_src = c.kv_source[i];
    l.rope_base = c.rope_base[i];
    // normRope passes floor(ropeProp * hd / 2) (gpu-runtime.js:1352)
    l.rope_angles = (int)floorf(c.rope_prop[i] * (float)l.hd / 2.f);
    if (l.hd > m->hd_max) m->hd_max = l.hd;
    if (l.inter > m->inter_max) m->inter_max = l.inter;
    // one RoPE table per distinct (base, head_dim, angles) of the layers the
    // one-launch decode attention serves
    if (attn_rope_supported(l.hd) && l.rope_angles <= kRopeTable) {
      RopeSlots &rs = m->rope_slots;
      for (int j = 0; j < rs.n; ++j)
        if (rs.base[j] == l.rope_base && rs.hd[j] == l.hd && rs.angles[j] == l.rope_angles)
          l.rope_slot = j;
      if (l.rope_slot < 0 && rs.n < kRopeSlots) {
        rs.base[rs.n] = l.rope_base;
        rs.hd[rs.n] = l.hd;
        rs.angles[rs.n] = l.rope_angles;
        l.rope_slot = rs.n++;
      }
    }
  }
  const size_t R = (size_t)m->max_rows, H = c.hidden;
  const size_t QD = (size_t)c.heads * m->hd_max;
  int rc = G4_OK;
  auto A = [&](float **p, size_t n) {
    if (!rc) rc = galloc_n(m, n, p);
  };
  if (!rc) rc = galloc_n(m, R, &m->ids);
  if (!rc) rc = galloc_n(m, 1, &m->pos);
  if (!rc) rc = galloc_n(m, (size_t)c.max_seq + 1, &m->gen);
  A(&m->h[0], R * H);
  A(&m->h[1], R * H);
  A(&m->pre, R * H);
  A(&m->qraw, R * QD);
  A(&m->q, R * QD);
  A(&m->kraw, R * m->hd_max);
  A(&m->vraw, R * m->hd_max);
  A(&m->ctx, R * QD);
  A(&m->attn, R * H);
  A(&m->ares, R * H);
  A(&m->pf, R * H);
  A(&m->gate, R * m->inter_max);
  A(&m->up, R * m->inter_max);
  A(&m->act, R * m->inter_max);
  A(&m->down, R * H);
  A(&m->downp, (size_t)kDownMaxSlices * H);
  A(&m->fres, R * H);
  A(&m->pg, R * c.ple_dim);
  A(&m->pm, R * c.ple_dim);
  A(&m->pp, R * H);
  A(&m->tokple, R * m->ple_total);
  A(&m->proj, R * m->ple_total);
  A(&m->perlayer, R * m->ple_total);
  A(&m->last, H);
  A(&m->logits, (size_t)c.vocab);
  {
    const int small = m->max_rows < 4 ? m->max_rows : 4;  // row counts that use kpw_for(1)
    const size_t a = attention_part_floats(small, c.heads, m->hd_max, c.max_seq, kpw_for(1));
    const size_t b = attention_part_floats(m->max_rows, c.heads, m->hd_max, c.max_seq,
                                           kpw_for(m->max_rows));
    // and the one-launch decode attention's partials: heads x splits x (hd + 4)
    const size_t d = (size_t)c.heads * attn_rope_splits(c.max_seq, false, c.window) *
                     ((size_t)m->hd_max + 4);
    m->part_floats = a > b ? a : b;
    if (d > m->part_floats) m->part_floats = d;
    A(&m->part, m->part_floats);
  }
  if (!rc) rc = galloc_n(m, head_argmax_blocks(c.vocab), &m->hpart);
  if (!rc) rc = galloc_n(m, (size_t)kRopeSlots * kRopeTable, &m->rope_tab);
  if (!rc) rc = galloc_n(m, (size_t)c.heads * kCountStride, &m->attn_count);  // zero-filled

  for (int i = 0; i < c.layers && !rc; ++i) {
    Layer &l = m->L[i];
    if (l.kv_src < 0) {
      A(&l.kc, (size_t)c.max_seq * l.hd);
      A(&l.vc, (size_t)c.max_seq * l.hd);
    }
  }
  if (rc) {
    for (void *p : m->allocs) device_free(p);
    delete m;
    return rc;
  }
  *out = m;
  return ok();
}

G4_API int g4_gemma_free(g4_gemma *m) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (!m) return ok();
  drop_step(m);
  int rc = G4_OK;
  for (void *p : m->allocs) {
    int r = device_free(p);
    if (r && !rc) rc = r;
  }
  delete m;
  return rc ? rc : ok();
}

G4_API int g4_gemma_set_linear(g4_gemma *m, int layer, int which, const g4_w4 *w) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (!m || !w) return fail(G4_E_ARG, "g4_gemma_set_linear: null argument");
  const g4_gemma_config &c = m->cfg;
  int N = 0, K = 0;
  g4_w4_info(w, &N, &K, nullptr, nullptr);
  if (layer == -1) {
    if (which != G4_PROJ_TOP)
      return fail(G4_E_ARG, "g4_gemma_set_linear: layer -1 takes G4_PROJ_TOP only");
    if (N != c.layers * c.ple_dim || K != c.hidden)
      return fail(G4_E_ARG, "per_layer_model_projection must be [%d, %d], got [%d, %d]",
                  c.layers * c.ple_dim, c.hidden, N, K);
    m->top = w;
    drop_step(m);
    return ok();
  }
  if (layer < 0 || layer >= c.layers || which < 0 || which >= kProjs)
    return fail(G4_E_ARG, "g4_gemma_set_linear: layer %d / projection %d out of range", layer,
                which);
  Layer &l = m->L[layer];
  if ((which == G4_PROJ_K || which == G4_PROJ_V) && l.kv_src >= 0)
    return fail(G4_E_ARG, "g4_gemma_set_linear: layer %d shares layer %d's KV (no k/v proj)",
                layer, l.kv_src);
  const int H = c.hidden, QD = c.heads * l.hd, P = c.ple_dim;
  static const char *names[kProjs] = {"q_proj", "k_proj", "v_proj", "o_proj", "gate_proj",
                                      "up_proj", "down_proj", "per_layer_input_gate",
                                      "per_layer_projection"};
  const int want[kProjs][2] = {{QD, H}, {l.hd, H}, {l.hd, H}, {H, QD}, {l.inter, H},
                               {l.inter, H}, {H, l.inter}, {P, H}, {H, P}};
  if (N != want[which][0] || K != want[which][1])
    return fail(G4_E_ARG, "layer %d %s must be [%d, %d], got [%d, %d]", layer, names[which],
                want[which][0], want[which][1], N, K);
  l.w[which] = w;
  drop_step(m);
  return ok();
}

G4_API int g4_gemma_set_norm(g4_gemma *m, int layer, int which, const float *v, int n) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (!m) return fail(G4_E_ARG, "g4_gemma_set_norm: null model");
  const g4_gemma_config &c = m->cfg;
  if (layer == -1) {
    if (which == G4_NORM_PLE_PROJECTION) {
      if (n != c.ple_dim) return fail(G4_E_ARG, "per_layer_projection_norm needs %d values", c.ple_dim);
      return upload_f32(m, &m->ple_norm, v, n) ?: ok();
    }
    if (which == G4_NORM_FINAL) {
      if (n != c.hidden) return fail(G4_E_ARG, "final norm needs %d values", c.hidden);
      return upload_f32(m, &m->final_norm, v, n) ?: ok();
    }
    return fail(G4_E_ARG, "g4_gemma_set_norm: layer -1 takes the PLE projection or final norm");
  }
  if (layer < 0 || layer >= c.layers || which < 0 || which >= kNorms)
    return fail(G4_E_ARG, "g4_gemma_set_norm: layer %d / norm %d out of range", layer, which);
  Layer &l = m->L[layer];
  if (which == G4_NORM_K && l.kv_src >= 0)
    return fail(G4_E_ARG, "g4_gemma_set_norm: layer %d has no k_norm (shared KV)", layer);
  const int want = (which == G4_NORM_Q || which == G4_NORM_K) ? l.hd : c.hidden;
  if (n != want)
    return fail(G4_E_ARG, "layer %d norm %d needs %d values, got %d", layer, which, want, n);
  return upload_f32(m, &l.norm[which], v, n) ?: ok();
}

G4_API int g4_gemma_set_layer_scalar(g4_gemma *m, int layer, float s) {
  if (!m || layer < 0 || layer >= m->cfg.layers)
    return fail(G4_E_ARG, "g4_gemma_set_layer_scalar: bad layer %d", layer);
  m->L[layer].skip = s;
  drop_step(m);
  return ok();
}

G4_API int g4_gemma_set_embedding(g4_gemma *m, const void *E_dev) {
  G4_CHECK_INIT();
  if (!m) return fail(G4_E_ARG, "g4_gemma_set_embedding: null model");
  int rc = check_device_range(E_dev, (size_t)m->cfg.vocab * m->cfg.hidden * 2,
                              "g4_gemma_set_embedding E");
  if (rc) return rc;
  if ((reinterpret_cast<uintptr_t>(E_dev) & 15u) != 0)
    return fail(G4_E_ARG, "g4_gemma_set_embedding: E must be 16-byte aligned");
  m->E = static_cast<const uint16_t *>(E_dev);
  drop_step(m);
  return ok();
}

G4_API int g4_gemma_set_ple(g4_gemma *m, const g4_ple *t) {
  if (!m || !t) return fail(G4_E_ARG, "g4_gemma_set_ple: null argument");
  int vocab = 0, width = 0;
  ple_geometry(t, &vocab, &width);
  // the table must cover the vocabulary with layers * ple_dim columns
  if (vocab < m->cfg.vocab || width != m->cfg.layers * m->cfg.ple_dim)
    return fail(G4_E_ARG, "g4_gemma_set_ple: table [%d, %d] does not match vocab %d x %d",
                vocab, width, m->cfg.vocab, m->cfg.layers * m->cfg.ple_dim);
  m->ple = t;
  m->ple_dense = nullptr;
  drop_step(m);
  return ok();
}

G4_API int g4_gemma_set_ple_dense(g4_gemma *m, const void *rows_dev) {
  G4_CHECK_INIT();
  if (!m) return fail(G4_E_ARG, "g4_gemma_set_ple_dense: null model");
  const g4_gemma_config &c = m->cfg;
  int rc = check_device_range(rows_dev, (size_t)c.vocab * c.layers * c.ple_dim * 2,
                              "g4_gemma_set_ple_dense rows");
  if (rc) return rc;
  m->ple_dense = static_cast<const uint16_t *>(rows_dev);
  m->ple = nullptr;
  drop_step(m);
  return ok();
}

G4_API int g4_gemma_reset(g4_gemma *m) {
  if (!m) return fail(G4_E_ARG, "g4_gemma_reset: null model");
  m->cache_len = 0;  // resetCache (gemma4-webgpu.js:191-194)
  return ok();
}

G4_API int g4_gemma_cache_length(const g4_gemma *m, int *len) {
  if (!m || !len) return fail(G4_E_ARG, "g4_gemma_cache_length: null argument");
  *len = m->cache_len;
  return ok();
}

G4_API int g4_gemma_last_hidden(g4_gemma *m, float *last_hidden) {
  G4_CHECK_INIT();
  if (!m || !last_hidden) return fail(G4_E_ARG, "g4_gemma_last_hidden: null argument");
  if (m->cache_len == 0) return fail(G4_E_STATE, "g4_gemma_last_hidden: no token has run");
  int rc = check_device_range(last_hidden, (size_t)m->cfg.hidden * 4, "g4_gemma_last_hidden");
  if (rc) return rc;
  G4_HIP_TRY(hipMemcpyAsync(last_hidden, m->last, (size_t)m->cfg.hidden * 4,
                            hipMemcpyDeviceToDevice, stream()));
  return ok();
}

G4_API int g4_gemma_forward(g4_gemma *m, const int32_t *ids, int n, int start_pos,
                            float *last_hidden) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (!m || !ids) return fail(G4_E_ARG, "g4_gemma_forward: null argument");
  int rc = check_ready(m);
  if (!rc && last_hidden) rc = check_device_range(last_hidden, (size_t)m->cfg.hidden * 4,
                                                  "g4_gemma_forward last_hidden");
  if (!rc) rc = stage_ids(m, ids, n, start_pos);
  if (!rc) rc = run_layers(m, n, false);
  if (rc) return rc;
  m->cache_len += n;
  if (last_hidden)
    G4_HIP_TRY(hipMemcpyAsync(last_hidden, m->last, (size_t)m->cfg.hidden * 4,
                              hipMemcpyDeviceToDevice, stream()));
  return ok();
}

G4_API int g4_gemma_diag_stages(const g4_gemma *m, int layer, int n, size_t *offsets) {
  if (!m || !offsets) return fail(G4_E_ARG, "g4_gemma_diag_stages: null argument");
  if (layer < 0 || layer >= m->cfg.layers || n <= 0)
    return fail(G4_E_ARG, "g4_gemma_diag_stages: layer %d / %d rows out of range", layer, n);
  diag_stage_offsets(m, layer, n, offsets);
  return ok();
}

G4_API int g4_gemma_forward_diag(g4_gemma *m, const int32_t *ids, int n, int start_pos,
                                 float *last_hidden, float *top_hidden, float *top_ple,
                                 float *layer_hidden, int stage_layer, float *stages) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (!m || !ids) return fail(G4_E_ARG, "g4_gemma_forward_diag: null argument");
  const g4_gemma_config &c = m->cfg;
  Diag dg;
  dg.top_hidden = top_hidden;
  dg.top_ple = top_ple;
  dg.layers = layer_hidden;
  dg.stages = stages;
  dg.stage_layer = stages ? stage_layer : -1;
  int rc = check_ready(m);
  if (!rc && n <= 0) rc = fail(G4_E_ARG, "g4_gemma: token count must be positive, got %d", n);
  if (!rc && stages && (stage_layer < 0 || stage_layer >= c.layers))
    rc = fail(G4_E_ARG, "g4_gemma_forward_diag: stage layer %d out of range", stage_layer);
  if (!rc && stages) diag_stage_offsets(m, stage_layer, n, dg.off);
  const size_t R = n > 0 ? (size_t)n : 0, H = c.hidden;
  if (!rc && last_hidden) rc = check_device_range(last_hidden, H * 4, "forward_diag last_hidden");
  if (!rc && top_hidden) rc = check_device_range(top_hidden, R * H * 4, "forward_diag top_hidden");
  if (!rc && top_ple)
    rc = check_device_range(top_ple, R * c.layers * c.ple_dim * 4, "forward_diag top_ple");
  if (!rc && layer_hidden)
    rc = check_device_range(layer_hidden, (size_t)c.layers * R * H * 4,
                            "forward_diag layer_hidden");
  if (!rc && stages) rc = check_device_range(stages, dg.off[G4_STAGES] * 4, "forward_diag stages");
  if (!rc) rc = stage_ids(m, ids, n, start_pos);
  if (!rc) rc = run_layers(m, n, false, &dg);
  if (rc) return rc;
  m->cache_len += n;
  if (last_hidden)
    G4_HIP_TRY(hipMemcpyAsync(last_hidden, m->last, H * 4, hipMemcpyDeviceToDevice, stream()));
  return ok();
}

G4_API int g4_gemma_logits(g4_gemma *m, const float *last_hidden, float *logits) {
  G4_CHECK_INIT();
  if (!m || !last_hidden || !logits) return fail(G4_E_ARG, "g4_gemma_logits: null argument");
  if (!m->E) return fail(G4_E_STATE, "g4_gemma_logits: embedding not set");
  const g4_gemma_config &c = m->cfg;
  int rc = check_device_range(last_hidden, (size_t)c.hidden * 4, "g4_gemma_logits last_hidden");
  if (!rc) rc = check_device_range(logits, (size_t)c.vocab * 4, "g4_gemma_logits logits");
  if (!rc)
    rc = launch_bf16_head(last_hidden, m->E, c.vocab, c.hidden, logits, 1.f, c.softcap, nullptr);
  return rc ? rc : ok();
}

G4_API int g4_gemma_greedy(g4_gemma *m, const int32_t *ids, int n, int start_pos,
                           int32_t *next_token, float *logits) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (!m || !ids || !next_token) return fail(G4_E_ARG, "g4_gemma_greedy: null argument");
  int rc = check_ready(m);
  if (!rc && logits)
    rc = check_device_range(logits, (size_t)m->cfg.vocab * 4, "g4_gemma_greedy logits");
  if (!rc) rc = stage_ids(m, ids, n, start_pos);
  if (!rc) rc = run_layers(m, n, false);
  if (!rc) rc = run_head(m, n);
  if (rc) return rc;
  m->cache_len += n;
  if (logits)
    G4_HIP_TRY(hipMemcpyAsync(logits, m->logits, (size_t)m->cfg.vocab * 4,
                              hipMemcpyDeviceToDevice, stream()));
  int32_t tok = -1;
  G4_HIP_TRY(hipMemcpyAsync(&tok, m->ids, 4, hipMemcpyDeviceToHost, stream()));
  G4_HIP_TRY(hipStreamSynchronize(stream()));
  if (tok < 0) return fail(G4_E_STATE, "topK(): no finite logits.");
  *next_token = tok;
  return ok();
}

G4_API int g4_gemma_decode(g4_gemma *m, int steps, int32_t *tokens) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (!m || steps < 0) return fail(G4_E_ARG, "g4_gemma_decode: bad argument");
  if (steps == 0) return ok();
  int rc = check_ready(m);
  if (rc) return rc;
  if (m->cache_len == 0)
    return fail(G4_E_STATE, "g4_gemma_decode: run g4_gemma_greedy on a prompt first");
  if (m->cache_len + steps > m->cfg.max_seq)
    return fail(G4_E_RANGE, "KV cache capacity %d exceeded", m->cfg.max_seq);
  if (!m->step) {
    // record one token: ids[0] and *pos come from the previous step's advance
    if ((rc = g4_encoder_begin())) return rc;
    rc = run_layers(m, 1, true);
    if (!rc) rc = run_head(m, 1);
    g4_cmdbuf *cb = nullptr;
    const int rc2 = g4_encoder_finish(&cb);
    if (rc) {
      if (cb) g4_cmdbuf_free(cb);
      return rc;
    }
    if (rc2) return rc2;
    m->step = cb;
  }
  const int first = m->cache_len;
  for (int s = 0; s < steps; ++s) {
    rc = g4_submit(m->step);
    if (rc) return rc;
  }
  m->cache_len += steps;
  if (tokens) {
    // gen[p] holds the token chosen for position p; step s fills first + 1 + s
    G4_HIP_TRY(hipMemcpyAsync(tokens, m->gen + first + 1, (size_t)steps * 4,
                              hipMemcpyDeviceToHost, stream()));
    G4_HIP_TRY(hipStreamSynchronize(stream()));
    for (int s = 0; s < steps; ++s)
      if (tokens[s] < 0) return fail(G4_E_STATE, "topK(): no finite logits.");
  }
  return ok();
}
