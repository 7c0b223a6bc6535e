"""CPU restatement of the decoder-layer ops and the forward pass of
custom-webgpu (gpu-runtime.js shaders, gemma4-webgpu.js Gemma4WebGPU).

TEST INFRASTRUCTURE, NOT PRODUCT CODE: imported only by tests/ (and by
__graft_entry__.smoke() / bench.py's CPU leg, to check results against);
nothing in the product path calls it.

Arithmetic is float64 on float32 inputs: a higher-precision version of the
FP32 shaders, used with a stated tolerance.  The exceptions follow the
shader's float32 steps where they decide the result: the RoPE angle
(float32 pow and divide, NORM_ROPE_SHADER) and the embedding scale (one
float32 multiply of an exact bf16 value).

Pinning (tests/test_oracle_layers.py): closed forms and invariants for each
op (constant-vector RMS, GELU values and limits, RoPE at position 0 and as a
rotation, single-key and uniform attention, masks against brute force,
pleMix with zero inputs).  The model forward is pinned by a closed form and
two invariants: one token through a layer of selection-matrix projections
equals an element-by-element restatement of encodeLayer (planted mistakes -
gelu(up) * gate, swapped norms, the layer scalar on one term, another
layer's PLE slice - each fail it); with every projection zero each layer only
scales the residual stream by its skip scalar (a dropped residual add fails
it); and a sequence fed whole equals the same sequence fed in parts
(positions, causal mask, KV append and KV sharing).  DequantModel is pinned
against Model.
"""
import numpy as np

import g4oracle

F64 = np.float64


def rms(x, width, scale=None, eps=1e-6):
    """RMS_SHADER (gpu-runtime.js:1104-1118): x * inverseSqrt(mean(x^2) + eps) * scale."""
    x = np.asarray(x, dtype=np.float32).reshape(-1, width).astype(F64)
    inv = 1.0 / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps)
    y = x * inv
    if scale is not None:
        y = y * np.asarray(scale, dtype=np.float32).astype(F64)[None, :]
    return y.astype(np.float32)


def add_scale(a, b, s):
    """ADD_SCALE_SHADER (gpu-runtime.js:1120-1128): (a + b) * scale."""
    return ((np.asarray(a, np.float32).astype(F64) + np.asarray(b, np.float32)) * np.float32(s)).astype(np.float32)


def scale(a, s):
    """SCALE_SHADER (gpu-runtime.js:1130-1137)."""
    return (np.asarray(a, np.float32).astype(F64) * np.float32(s)).astype(np.float32)


def gelu_tanh(x):
    """GELU of GELU_MUL_SHADER (gpu-runtime.js:1148-1155), tanh argument clamped to +-10."""
    x = np.asarray(x, dtype=np.float32).astype(F64)
    c = 0.7978845608028654
    z = c * (x + 0.044715 * x * x * x)
    t = np.tanh(np.clip(z, -10.0, 10.0))
    return 0.5 * x * (1.0 + t)


def gelu_mul(gate, up):
    """GELU_MUL_SHADER: gelu(gate) * up."""
    return (gelu_tanh(gate) * np.asarray(up, np.float32)).astype(np.float32)


def gelu_ple(gate, ple, rows, layer, width=256, layers=35):
    """GELU_PLE_SHADER (gpu-runtime.js:1159-1173): gelu(gate[r,d]) * ple[r, layer, d]."""
    g = np.asarray(gate, np.float32).reshape(rows, width)
    p = np.asarray(ple, np.float32).reshape(rows, layers, width)[:, layer, :]
    return (gelu_tanh(g) * p).astype(np.float32)


def rope_theta(pos, pair, hd, base):
    """The shader's angle in float32: f32(pos) / pow(base, 2*pair/hd)."""
    ex = np.float32(2.0) * np.float32(pair) / np.float32(hd)
    return np.float32(pos) / np.power(np.float32(base), ex, dtype=np.float32)


def norm_rope(x, rows, heads, hd, pos0, scale_, rope_angles, base, eps=1e-6):
    """NORM_ROPE_SHADER (gpu-runtime.js:1175-1202): per (row, head) RMS norm
    times scale, then rotate-half RoPE of the first rope_angles pairs."""
    x = np.asarray(x, np.float32).reshape(rows, heads, hd).astype(F64)
    s = np.asarray(scale_, np.float32).astype(F64)
    inv = 1.0 / np.sqrt((x * x).mean(axis=2, keepdims=True) + eps)
    n = x * inv * s[None, None, :]
    half = hd // 2
    a, b = n[..., :half], n[..., half:]
    y = np.empty_like(n)
    cs = np.ones((rows, half))
    sn = np.zeros((rows, half))
    for r in range(rows):
        for p in range(min(rope_angles, half)):
            th = float(rope_theta(pos0 + r, p, hd, base))
            cs[r, p], sn[r, p] = np.cos(th), np.sin(th)
    y[..., :half] = a * cs[:, None, :] - b * sn[:, None, :]
    y[..., half:] = b * cs[:, None, :] + a * sn[:, None, :]
    return y.reshape(rows, heads * hd).astype(np.float32)


def attention(q, k, v, qrows, heads, hd, keylen, qpos0, sliding, window):
    """GPUOps.attention (gpu-runtime.js:1357-1365): QK_SHADER (1204-1221) with its
    mask (key <= qpos, and key + window > qpos when sliding; masked logit
    -1e30), SOFTMAX_SHADER (1223-1234), ATTN_OUT_SHADER (1236-1248)."""
    q = np.asarray(q, np.float32).reshape(qrows, heads, hd).astype(F64)
    k = np.asarray(k, np.float32).reshape(-1, hd)[:keylen].astype(F64)
    v = np.asarray(v, np.float32).reshape(-1, hd)[:keylen].astype(F64)
    logits = np.einsum("rhd,kd->rhk", q, k)
    key = np.arange(keylen)[None, :]
    qp = (qpos0 + np.arange(qrows))[:, None]
    valid = key <= qp
    if sliding:
        valid = valid & (key + window > qp)
    logits = np.where(valid[:, None, :], logits, -1e30)
    mx = logits.max(axis=2, keepdims=True)
    e = np.exp(logits - mx)
    p = e / e.sum(axis=2, keepdims=True)
    out = np.einsum("rhk,kd->rhd", p, v)
    return out.reshape(qrows, heads * hd).astype(np.float32)


def ple_mix(proj, norm_scale, token_ple, rows, width=256, layers=35):
    """PLE_MIX_SHADER (gpu-runtime.js:1250-1263): per 256-chunk RMS (eps 1e-6)
    times norm scale, plus token PLE * 16, times 1/sqrt(2)."""
    p = np.asarray(proj, np.float32).reshape(rows * layers, width).astype(F64)
    t = np.asarray(token_ple, np.float32).reshape(rows * layers, width).astype(F64)
    s = np.asarray(norm_scale, np.float32).astype(F64)
    inv = 1.0 / np.sqrt((p * p).mean(axis=1, keepdims=True) + 1e-6)
    y = (p * inv * s[None, :] + t * 16.0) * 0.7071067811865476
    return y.reshape(rows, layers * width).astype(np.float32)


def embed(E_bits, ids, scale_):
    """bf16Rows(embed_tokens, ids) then ops.scale (gemma4-webgpu.js:198-215, 318):
    an exact bf16 -> f32 widening and one float32 multiply."""
    sel = np.asarray(E_bits, np.uint16)[np.asarray(ids)]
    rows = g4oracle.bf16_to_f32_array(sel).reshape(sel.shape)
    return (rows.astype(np.float32) * np.float32(scale_)).astype(np.float32)


# ---- model ---------------------------------------------------------------------

def e2b_spec(i):
    """spec(i) (gemma4-webgpu.js:65-77)."""
    full = (i + 1) % 5 == 0
    return dict(full=full, head_dim=512 if full else 256, intermediate=6144 if i < 15 else 12288,
                shared=i >= 15, store_shared=i in (13, 14),
                rope_base=1e6 if full else 1e4, rope_prop=0.25 if full else 1.0)


class Model:
    """Gemma4WebGPU.forward/logits/greedy (gemma4-webgpu.js:215-481) over host
    weights.  `layers` is a list of dicts: head_dim, intermediate, full,
    kv_source (-1 own, else earlier layer index), rope_base, rope_prop,
    linear {q,k,v,o,gate,up,down,ple_gate,ple_proj: (packed, scales_bf16)},
    norm {input,post_attn,pre_ffw,post_ffw,post_ple,q,k}, skip."""

    def __init__(self, hidden, heads, ple_dim, vocab, layers, E_bits, ple_rows, top, ple_norm,
                 final_norm, window=512, softcap=30.0, eps=1e-6):
        self.hidden, self.heads, self.ple_dim, self.vocab = hidden, heads, ple_dim, vocab
        self.layers, self.E_bits, self.ple_rows, self.top = layers, E_bits, ple_rows, top
        self.ple_norm, self.final_norm = ple_norm, final_norm
        self.window, self.softcap, self.eps = window, softcap, eps
        self.reset()

    def reset(self):
        self.k = {}
        self.v = {}
        self.length = 0

    def _w4(self, lin, x):
        packed, scales = lin
        return g4oracle.w4_linear_f64(np.asarray(x, np.float32), packed, scales)

    def forward(self, ids, start_pos, probes=None, probe_layer=1):
        """forward; with a dict `probes`, also the diagnostic read-outs of
        forward(..., {diagnostic: true}) (gemma4-webgpu.js:311-397): "top
        hidden", "top PLE", "layer i" (each layer's output) and, for layer
        probe_layer, every encodeLayer stage under its probe name (224-309)."""
        ids = np.asarray(ids)
        rows, H, P, NL = len(ids), self.hidden, self.ple_dim, len(self.layers)
        if start_pos != self.length:
            raise ValueError("KV append position %d != cache length %d" % (start_pos, self.length))
        hidden = embed(self.E_bits, ids, np.float32(np.sqrt(H)))
        proj = self._w4(self.top, hidden)
        projs = scale(proj, np.float32(1.0 / np.sqrt(H)))
        tokple = self.ple_rows(ids)
        perlayer = ple_mix(projs, self.ple_norm, tokple, rows, P, NL)
        if probes is not None:
            probes["top hidden"], probes["top PLE"] = hidden, perlayer
        for i, L in enumerate(self.layers):
            st = {}  # this layer's stages
            hd, heads = L["head_dim"], self.heads
            angles = int(np.floor(np.float32(L["rope_prop"]) * hd / 2))
            pre = st["preAttention"] = rms(hidden, H, L["norm"]["input"], self.eps)
            st["qRaw"] = self._w4(L["linear"]["q"], pre)
            q = st["qNormRoPE"] = norm_rope(st["qRaw"], rows, heads, hd, start_pos,
                                            L["norm"]["q"], angles, L["rope_base"], self.eps)
            src = i if L["kv_source"] < 0 else L["kv_source"]
            if L["kv_source"] < 0:
                st["kRaw"] = self._w4(L["linear"]["k"], pre)
                st["vRaw"] = self._w4(L["linear"]["v"], pre)
                k = st["kNormRoPE"] = norm_rope(st["kRaw"], rows, 1, hd, start_pos,
                                                L["norm"]["k"], angles, L["rope_base"], self.eps)
                v = st["vNorm"] = rms(st["vRaw"], hd, None, self.eps)
                self.k[i] = np.concatenate([self.k.get(i, np.zeros((0, hd), np.float32)), k])
                self.v[i] = np.concatenate([self.v.get(i, np.zeros((0, hd), np.float32)), v])
            keylen = start_pos + rows
            ctx = st["attentionContext"] = attention(q, self.k[src], self.v[src], rows, heads, hd,
                                                     keylen, start_pos, not L["full"], self.window)
            st["attentionOutput"] = self._w4(L["linear"]["o"], ctx)
            an = st["postAttentionNorm"] = rms(st["attentionOutput"], H, L["norm"]["post_attn"],
                                               self.eps)
            ares = st["attentionResidual"] = add_scale(hidden, an, 1.0)
            pf = st["preFfw"] = rms(ares, H, L["norm"]["pre_ffw"], self.eps)
            st["mlpGate"] = self._w4(L["linear"]["gate"], pf)
            st["mlpUp"] = self._w4(L["linear"]["up"], pf)
            act = st["mlpActivated"] = gelu_mul(st["mlpGate"], st["mlpUp"])
            st["ffwOutput"] = self._w4(L["linear"]["down"], act)
            fn = st["postFfwNorm"] = rms(st["ffwOutput"], H, L["norm"]["post_ffw"], self.eps)
            fres = st["ffwResidual"] = add_scale(ares, fn, 1.0)
            st["pleGate"] = self._w4(L["linear"]["ple_gate"], fres)
            pm = st["pleModulated"] = gelu_ple(st["pleGate"], perlayer, rows, i, P, NL)
            st["pleProjected"] = self._w4(L["linear"]["ple_proj"], pm)
            pn = st["pleNormalized"] = rms(st["pleProjected"], H, L["norm"]["post_ple"], self.eps)
            hidden = st["output"] = add_scale(fres, pn, L["skip"])
            if probes is not None:
                probes["layer %d" % i] = hidden
                if i == probe_layer:
                    probes["stages"] = st
        self.length += rows
        return rms(hidden[-1:], H, self.final_norm, self.eps)[0]

    def logits(self, last):
        return g4oracle.bf16_head(last, self.E_bits, 1.0, self.softcap)

    def greedy(self, ids, start_pos):
        lg = self.logits(self.forward(ids, start_pos))
        top_ids, _ = g4oracle.topk(lg, 10)
        return int(top_ids[0]), lg


class DequantModel(Model):
    """Model whose W4 projections dequantize each weight once to float64
    (q * widened bf16 scale, exact) and multiply with numpy's float64 matmul:
    the same product as g4o_w4_linear_f64 in another summation order, fast
    enough for the E2B widths (hidden 1536, hundreds of rows).  Pinned against
    Model by tests/test_oracle_layers.py."""

    def __init__(self, *a, **kw):
        super().__init__(*a, **kw)
        self._deq = {}

    def _w4(self, lin, x):
        packed, scales = lin
        key = id(packed)
        w = self._deq.get(key)
        if w is None:
            p = np.asarray(packed).view(np.uint32)
            n, kw = p.shape
            shifts = np.arange(8, dtype=np.uint32) * np.uint32(4)
            q = (((p[:, :, None] >> shifts) & np.uint32(15)).astype(np.int8) - 8).reshape(n, kw * 8)
            s = g4oracle.bf16_to_f32_array(np.asarray(scales).view(np.uint16)).reshape(n, -1)
            w = q.astype(F64) * np.repeat(s.astype(F64), 32, axis=1)
            self._deq[key] = (packed, w)  # keep `packed` alive so its id stays unique
        else:
            w = w[1]
        return np.asarray(x, np.float32).astype(F64) @ w.T
