"""Pins the decoder-layer oracle (oracle/layer_oracle.py) with closed forms,
invariants and brute force, so a dropped term, a wrong sign or a swapped
index in the restatement fails here before results are checked against it."""
import math

import numpy as np
import pytest

import layer_oracle as lo


def test_rms_constant_vector_closed_form():
    # x = c everywhere: y = c / sqrt(c^2 + eps) * scale
    c, w, eps = 3.0, 64, 1e-6
    s = np.linspace(0.5, 2.0, w).astype(np.float32)
    y = lo.rms(np.full((2, w), c, np.float32), w, s, eps)
    want = c / math.sqrt(c * c + eps) * s
    np.testing.assert_allclose(y[0], want, rtol=1e-6)
    np.testing.assert_allclose(y[1], want, rtol=1e-6)


def test_rms_unit_mean_square_and_no_scale():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 100)).astype(np.float32) * 7
    y = lo.rms(x, 100, None, 0.0).astype(np.float64)
    np.testing.assert_allclose((y * y).mean(axis=1), 1.0, rtol=1e-6)
    # direction is kept: y is a positive multiple of x
    assert np.all(np.sign(y) == np.sign(x))


def test_add_scale_and_scale():
    a = np.array([1, -2, 3.5], np.float32)
    b = np.array([0.5, 2, -1], np.float32)
    np.testing.assert_array_equal(lo.add_scale(a, b, 2.0), np.array([3, 0, 5], np.float32))
    np.testing.assert_array_equal(lo.scale(a, -0.5), np.array([-0.5, 1, -1.75], np.float32))


def test_gelu_known_values_and_limits():
    # tanh-form GELU: gelu(0) = 0, gelu(1) = 0.5 * (1 + tanh(0.79788456 * 1.044715))
    g = lo.gelu_tanh(np.array([0.0, 1.0, -1.0, 20.0, -20.0], np.float32))
    t1 = math.tanh(0.7978845608028654 * 1.044715)
    np.testing.assert_allclose(g[:3], [0.0, 0.5 * (1 + t1), -0.5 * (1 - t1)], rtol=1e-12)
    # the clamp at |z| = 10 leaves the asymptotes: x and 0
    np.testing.assert_allclose(g[3], 20.0 * 0.5 * (1 + math.tanh(10.0)), rtol=1e-12)
    assert abs(g[4]) < 1e-6
    # gelu(x) - gelu(-x) = x (odd part of 0.5 x (1 + tanh))
    x = np.linspace(-3, 3, 13).astype(np.float32)
    np.testing.assert_allclose(lo.gelu_tanh(x) - lo.gelu_tanh(-x), x, atol=1e-7)


def test_gelu_mul_and_gelu_ple_index_layer_and_width():
    rows, width, layers = 2, 4, 3
    gate = np.arange(rows * width, dtype=np.float32).reshape(rows, width) / 4
    ple = np.arange(rows * layers * width, dtype=np.float32).reshape(rows, layers, width)
    y = lo.gelu_ple(gate, ple, rows, 1, width, layers)
    want = lo.gelu_tanh(gate) * ple[:, 1, :]
    np.testing.assert_allclose(y, want, rtol=1e-6)
    np.testing.assert_allclose(lo.gelu_mul(gate, 2 * np.ones_like(gate)), 2 * lo.gelu_tanh(gate),
                               rtol=1e-6)


def test_norm_rope_position_zero_is_plain_norm():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((1, 2 * 8)).astype(np.float32)
    s = rng.uniform(0.5, 1.5, 8).astype(np.float32)
    y = lo.norm_rope(x, 1, 2, 8, 0, s, 4, 10000.0)
    np.testing.assert_allclose(y.reshape(2, 8), lo.rms(x.reshape(2, 8), 8, s), rtol=1e-6)


def test_norm_rope_rotation_known_angle_and_norm():
    # hd 4, pair 0 at position 1 rotates by exactly 1 rad; pair 1 by 1/base^(1/2)
    x = np.array([[1.0, 2.0, 3.0, 4.0]], np.float32)
    s = np.ones(4, np.float32)
    base = 100.0
    y = lo.norm_rope(x, 1, 1, 4, 1, s, 2, base, eps=0.0)[0].astype(np.float64)
    n = x[0] / math.sqrt((x[0] ** 2).mean())
    th0, th1 = 1.0, float(np.float32(1.0) / np.float32(math.sqrt(base)))
    want = [n[0] * math.cos(th0) - n[2] * math.sin(th0), n[1] * math.cos(th1) - n[3] * math.sin(th1),
            n[2] * math.cos(th0) + n[0] * math.sin(th0), n[3] * math.cos(th1) + n[1] * math.sin(th1)]
    np.testing.assert_allclose(y, want, rtol=1e-6)
    # pairs beyond rope_angles are not rotated
    y1 = lo.norm_rope(x, 1, 1, 4, 5, s, 1, base, eps=0.0)[0]
    np.testing.assert_allclose([y1[1], y1[3]], [n[1], n[3]], rtol=1e-6)


def test_norm_rope_rows_advance_position():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 16)).astype(np.float32)
    s = np.ones(16, np.float32)
    y = lo.norm_rope(x, 3, 1, 16, 7, s, 8, 10000.0)
    for r in range(3):
        np.testing.assert_allclose(y[r], lo.norm_rope(x[r:r + 1], 1, 1, 16, 7 + r, s, 8, 10000.0)[0],
                                   rtol=1e-7)


def test_attention_single_visible_key_returns_its_value():
    rng = np.random.default_rng(4)
    hd, heads = 8, 2
    k = rng.standard_normal((5, hd)).astype(np.float32)
    v = rng.standard_normal((5, hd)).astype(np.float32)
    q = rng.standard_normal((1, heads * hd)).astype(np.float32)
    # query at position 0 sees only key 0
    y = lo.attention(q, k, v, 1, heads, hd, 1, 0, False, 512)
    np.testing.assert_allclose(y.reshape(heads, hd), np.stack([v[0], v[0]]), rtol=1e-6)


def test_attention_uniform_logits_average_visible_values():
    rng = np.random.default_rng(5)
    hd, heads = 4, 1
    k = rng.standard_normal((10, hd)).astype(np.float32)
    v = rng.standard_normal((10, hd)).astype(np.float32)
    q = np.zeros((2, hd), np.float32)  # all logits 0
    # query rows at positions 8 and 9, sliding window 3: keys 6..8 and 7..9
    y = lo.attention(q, k, v, 2, heads, hd, 10, 8, True, 3)
    np.testing.assert_allclose(y[0], v[6:9].mean(axis=0), rtol=1e-6)
    np.testing.assert_allclose(y[1], v[7:10].mean(axis=0), rtol=1e-6)
    # global: all keys up to the position
    y = lo.attention(q, k, v, 2, heads, hd, 10, 8, False, 3)
    np.testing.assert_allclose(y[0], v[:9].mean(axis=0), rtol=1e-6)


def test_attention_matches_brute_force_loops():
    rng = np.random.default_rng(6)
    qrows, heads, hd, keylen, qpos0, window = 3, 2, 4, 7, 4, 2
    q = rng.standard_normal((qrows, heads * hd)).astype(np.float32)
    k = rng.standard_normal((keylen, hd)).astype(np.float32)
    v = rng.standard_normal((keylen, hd)).astype(np.float32)
    for sliding in (False, True):
        y = lo.attention(q, k, v, qrows, heads, hd, keylen, qpos0, sliding, window)
        for r in range(qrows):
            qp = qpos0 + r
            for h in range(heads):
                qv = q[r, h * hd:(h + 1) * hd].astype(np.float64)
                logits = []
                for key in range(keylen):
                    ok = key <= qp and (not sliding or key + window > qp)
                    logits.append(float(qv @ k[key]) if ok else -1e30)
                m = max(logits)
                e = [math.exp(t - m) for t in logits]
                out = sum(ei * v[i].astype(np.float64) for i, ei in enumerate(e)) / sum(e)
                np.testing.assert_allclose(y[r, h * hd:(h + 1) * hd], out, rtol=1e-6, atol=1e-7)


def test_ple_mix_closed_forms():
    rows, width, layers = 1, 8, 2
    s = np.linspace(1, 2, width).astype(np.float32)
    tok = np.arange(rows * layers * width, dtype=np.float32).reshape(rows, layers * width) / 10
    # zero projection: the token rows alone, times 16 / sqrt(2)
    y = lo.ple_mix(np.zeros_like(tok), s, tok, rows, width, layers)
    np.testing.assert_allclose(y, tok * 16 / math.sqrt(2), rtol=1e-6)
    # constant projection c, zero token rows: c / sqrt(c^2 + 1e-6) * s / sqrt(2)
    c = 2.0
    y = lo.ple_mix(np.full_like(tok, c), s, np.zeros_like(tok), rows, width, layers)
    want = np.tile(c / math.sqrt(c * c + 1e-6) * s / math.sqrt(2), layers)
    np.testing.assert_allclose(y[0], want, rtol=1e-6)


def test_embed_is_exact_bf16_times_scale():
    E = np.array([[0x3F80, 0xC000], [0x4040, 0x0000]], np.uint16)  # 1, -2, 3, 0
    y = lo.embed(E, [1, 0], np.float32(math.sqrt(1536)))
    s = np.float32(math.sqrt(1536))
    np.testing.assert_array_equal(y, np.array([[3 * s, 0], [s, -2 * s]], np.float32))


def test_e2b_spec_schedule():
    full = [i for i in range(35) if lo.e2b_spec(i)["full"]]
    assert full == [4, 9, 14, 19, 24, 29, 34]
    assert lo.e2b_spec(14)["head_dim"] == 512 and lo.e2b_spec(13)["head_dim"] == 256
    assert [lo.e2b_spec(i)["intermediate"] for i in (14, 15)] == [6144, 12288]
    assert not lo.e2b_spec(14)["shared"] and lo.e2b_spec(15)["shared"]
    assert lo.e2b_spec(13)["store_shared"] and lo.e2b_spec(14)["store_shared"]


@pytest.mark.parametrize("plant", [None, "no_window"])
def test_attention_window_planted_mistake_is_caught(plant):
    # A restatement that forgets the sliding window must disagree with the
    # uniform-logit closed form; this guards the check itself.
    rng = np.random.default_rng(7)
    k = rng.standard_normal((6, 2)).astype(np.float32)
    v = rng.standard_normal((6, 2)).astype(np.float32)
    q = np.zeros((1, 2), np.float32)
    y = lo.attention(q, k, v, 1, 1, 2, 6, 5, plant is None, 2)
    want = v[4:6].mean(axis=0)
    if plant is None:
        np.testing.assert_allclose(y[0], want, rtol=1e-6)
    else:
        assert not np.allclose(y[0], want, rtol=1e-3)


# ---------------------------------------------------------------------------
# Model-level pins (Model.forward composes the ops above in the order of
# gemma4-webgpu.js encodeLayer 215-301 / forward 303-402).

def _tiny_layers(rng, H, heads, P, zero):
    import synthetic as syn
    spec = [dict(head_dim=16, full=0, kv_source=-1, intermediate=32, rope_base=1e4, rope_prop=1.0),
            dict(head_dim=32, full=1, kv_source=-1, intermediate=32, rope_base=1e6, rope_prop=0.25),
            dict(head_dim=16, full=0, kv_source=0, intermediate=64, rope_base=1e4, rope_prop=1.0)]
    layers, seed = [], 100
    for L in spec:
        hd, inter = L["head_dim"], L["intermediate"]
        shapes = dict(q=(heads * hd, H), o=(H, heads * hd), gate=(inter, H), up=(inter, H),
                      down=(H, inter), ple_gate=(P, H), ple_proj=(H, P))
        if L["kv_source"] < 0:
            shapes.update(k=(hd, H), v=(hd, H))
        lin = {}
        for name, (n, k) in shapes.items():
            seed += 1
            if zero:  # q = 0 everywhere: every projection outputs exactly 0
                lin[name] = (syn.pack_w4(np.zeros((n, k), np.int8)),
                             syn.bf16_rne(np.ones((n, k // 32), np.float32)))
            else:
                packed, scales, _ = syn.w4_weights(seed, n, k, 0.1)
                lin[name] = (packed, scales)
        norm = {n: rng.uniform(0.8, 1.2, H).astype(np.float32)
                for n in ("input", "post_attn", "pre_ffw", "post_ffw", "post_ple")}
        norm["q"] = rng.uniform(0.8, 1.2, hd).astype(np.float32)
        norm["k"] = rng.uniform(0.8, 1.2, hd).astype(np.float32)
        layers.append(dict(L, linear=lin, norm=norm, skip=float(rng.uniform(0.5, 2.0))))
    return layers


def _tiny_model(seed, zero=False, window=4):
    import synthetic as syn
    H, heads, P, V = 64, 2, 32, 32
    rng = np.random.default_rng(seed)
    E = syn.bf16_rne(rng.standard_normal((V, H), dtype=np.float32))
    layers = _tiny_layers(rng, H, heads, P, zero)
    NL = len(layers)
    ple = rng.standard_normal((V, NL * P)).astype(np.float32)
    top = syn.w4_weights(seed + 1, NL * P, H, 0.1)[:2]
    m = lo.Model(H, heads, P, V, layers, E, lambda ids: ple[np.asarray(ids)], top,
                 rng.uniform(0.8, 1.2, P).astype(np.float32),
                 rng.uniform(0.8, 1.2, H).astype(np.float32), window=window)
    return m, E


def test_model_zero_projections_leave_the_residual_stream():
    # Every projection 0: attention, MLP and PLE branches add exactly 0, so
    # each layer maps hidden -> hidden * skip and the output is the final norm
    # of the scaled embedding row.  A dropped residual add fails this.
    m, E = _tiny_model(3, zero=True)
    ids = [5, 17, 2, 30]
    got = m.forward(ids, 0)
    skip = np.prod([L["skip"] for L in m.layers])
    h = lo.embed(E, ids, np.float32(math.sqrt(m.hidden))).astype(np.float64)[-1:] * skip
    want = lo.rms(h.astype(np.float32), m.hidden, m.final_norm)[0]
    np.testing.assert_allclose(got, want, rtol=1e-6)


def test_model_zero_projections_planted_residual_drop_is_caught(monkeypatch):
    m, E = _tiny_model(3, zero=True)
    real = lo.add_scale
    monkeypatch.setattr(lo, "add_scale", lambda a, b, s: real(np.zeros_like(a), b, s))
    got = m.forward([5, 17, 2, 30], 0)
    h = lo.embed(E, [30], np.float32(math.sqrt(m.hidden)))
    want = lo.rms(h, m.hidden, m.final_norm)[0]
    assert not np.allclose(got, want, rtol=1e-3)


@pytest.mark.parametrize("split", [1, 3, 6])
def test_model_prefill_equals_incremental_forward(split):
    # Causal masking, the sliding window (4 < 9 tokens), KV sharing and the
    # position offsets of a later call: a sequence fed whole and fed in two
    # parts (then one token at a time) must give the same last hidden state.
    ids = [3, 9, 27, 1, 14, 22, 8, 31, 0]
    m, _ = _tiny_model(4)
    whole = m.forward(ids, 0)
    m.reset()
    m.forward(ids[:split], 0)
    for p in range(split, len(ids)):
        part = m.forward(ids[p:p + 1], p)
    np.testing.assert_allclose(part, whole, rtol=1e-9, atol=1e-12)
    assert m.length == len(ids)


def test_model_rejects_wrong_append_position():
    m, _ = _tiny_model(5)
    m.forward([1, 2], 0)
    with pytest.raises(ValueError, match="KV append position 1 != cache length 2"):
        m.forward([3], 1)


# ---- the layer composition in closed form, with planted mistakes -----------------
#
# One token at position 0 through one layer whose W4 projections are selection
# matrices: row o of a projection holds a single nonzero q = m[o] at input
# column c[o] with scale s (powers of two), so y[o] = x[c[o]] * m[o] * s
# exactly.  q and k are zero, so the one visible key gets softmax weight 1 and
# the attention context is the normalised v row.  The expected output follows
# encodeLayer (gemma4-webgpu.js:224-309) and the top-level PLE mix (317-321)
# written out element by element below, with the shaders' formulas taken from
# gpu-runtime.js (RMS 1104-1118, GELU 1139-1173, PLE mix 1250-1263); no oracle
# function is called to build it.

CF_H, CF_P, CF_V = 64, 32, 4


def _selection(n, k, cols, mult, scale_bits):
    import synthetic as syn
    q = np.zeros((n, k), np.int8)
    q[np.arange(n), cols] = mult
    return syn.pack_w4(q), np.full((n, k // 32), scale_bits, np.uint16)


def _cf_setup(seed=7, skip=1.7):
    import synthetic as syn
    H, P, V = CF_H, CF_P, CF_V
    rng = np.random.default_rng(seed)
    E = syn.bf16_rne(rng.uniform(-1, 1, (V, H)).astype(np.float32))
    tok_ple = rng.standard_normal((V, P)).astype(np.float32)
    sels = {}
    spec = dict(q=(H, H), k=(H, H), v=(H, H), o=(H, H), gate=(H, H), up=(H, H), down=(H, H),
                ple_gate=(P, H), ple_proj=(H, P))
    for name, (n, k) in spec.items():
        cols = rng.integers(0, k, n)
        mult = np.zeros(n, np.int8) if name in ("q", "k") else rng.integers(1, 8, n).astype(np.int8)
        sels[name] = (cols, mult)
    # scales 2^-2 (0x3E80) for gate/up so the GELU sees moderate arguments, else 1
    scale_bits = {n: (0x3E80 if n in ("gate", "up") else 0x3F80) for n in spec}
    lin = {n: _selection(spec[n][0], spec[n][1], sels[n][0], sels[n][1], scale_bits[n])
           for n in spec}
    top_cols, top_mult = rng.integers(0, H, P), rng.integers(1, 8, P).astype(np.int8)
    top = _selection(P, H, top_cols, top_mult, 0x3F80)
    names = ("input", "post_attn", "pre_ffw", "post_ffw", "post_ple")
    norm = {n: rng.uniform(0.5, 1.5, H).astype(np.float32) for n in names}
    norm["q"] = rng.uniform(0.5, 1.5, H).astype(np.float32)
    norm["k"] = rng.uniform(0.5, 1.5, H).astype(np.float32)
    layer = dict(head_dim=H, intermediate=H, full=0, kv_source=-1, rope_base=1e4, rope_prop=1.0,
                 linear=lin, norm=norm, skip=skip)
    ple_norm = rng.uniform(0.5, 1.5, P).astype(np.float32)
    final = rng.uniform(0.5, 1.5, H).astype(np.float32)
    parts = dict(E=E, tok_ple=tok_ple, sels=sels, scale={n: 0.25 if n in ("gate", "up") else 1.0
                                                         for n in spec},
                 top=(top_cols, top_mult), norm=norm, ple_norm=ple_norm, final=final, skip=skip)
    return layer, top, parts


def _cf_model(layer, top, parts):
    return lo.Model(CF_H, 1, CF_P, CF_V, [layer], parts["E"],
                    lambda ids: parts["tok_ple"][np.asarray(ids)], top, parts["ple_norm"],
                    parts["final"])


def _cf_expected(parts, tok):
    """The layer for one token at position 0, element by element in float64."""
    H = CF_H
    f = np.float64

    def rmsn(x, w=None):  # RMS_SHADER: x * inverseSqrt(mean(x*x) + 1e-6) * w
        y = x / math.sqrt(float(np.mean(x * x)) + 1e-6)
        return y if w is None else y * w.astype(f)

    def gelu(x):  # GELU_MUL_SHADER / GELU_PLE_SHADER, tanh argument clamped
        z = 0.7978845608028654 * (x + 0.044715 * x ** 3)
        return 0.5 * x * (1.0 + np.tanh(np.clip(z, -10, 10)))

    def sel(name, x):
        cols, mult = parts["sels"][name]
        return x[cols] * mult.astype(f) * parts["scale"][name]

    nrm = parts["norm"]
    e = (parts["E"][tok].astype(np.uint32) << 16).view(np.float32).astype(f)
    h = e * 8.0                                   # scale(embed, sqrt(64))
    tc, tm = parts["top"]
    proj = h[tc] * tm.astype(f) * 0.125           # scale(w4(top, hidden), 1/sqrt(64))
    per = (rmsn(proj, parts["ple_norm"]) + parts["tok_ple"][tok].astype(f) * 16.0) \
        / math.sqrt(2.0)                          # PLE_MIX_SHADER
    pre = rmsn(h, nrm["input"])
    ctx = rmsn(sel("v", pre))                     # one visible key: context = vNorm row
    an = rmsn(sel("o", ctx), nrm["post_attn"])
    ares = h + an
    pf = rmsn(ares, nrm["pre_ffw"])
    act = gelu(sel("gate", pf)) * sel("up", pf)
    fres = ares + rmsn(sel("down", act), nrm["post_ffw"])
    pm = gelu(sel("ple_gate", fres)) * per
    pn = rmsn(sel("ple_proj", pm), nrm["post_ple"])
    out = (fres + pn) * parts["skip"]
    return rmsn(out, parts["final"])


def test_layer_composition_matches_closed_form():
    layer, top, parts = _cf_setup()
    for tok in range(CF_V):
        m = _cf_model(layer, top, parts)
        got = m.forward([tok], 0)
        np.testing.assert_allclose(got, _cf_expected(parts, tok), rtol=2e-5, atol=1e-6)


def _cf_error(layer, top, parts):
    errs = []
    for tok in range(CF_V):
        got = _cf_model(layer, top, parts).forward([tok], 0).astype(np.float64)
        want = _cf_expected(parts, tok)
        errs.append(np.linalg.norm(got - want) / np.linalg.norm(want))
    return max(errs)


def test_layer_composition_planted_gelu_operand_swap_is_caught(monkeypatch):
    layer, top, parts = _cf_setup()
    assert _cf_error(layer, top, parts) < 1e-5
    real = lo.gelu_mul
    monkeypatch.setattr(lo, "gelu_mul", lambda gate, up: real(up, gate))  # gelu(up) * gate
    assert _cf_error(layer, top, parts) > 1e-2


def test_layer_composition_planted_norm_swap_is_caught():
    layer, top, parts = _cf_setup()
    swapped = dict(layer, norm=dict(layer["norm"], post_attn=layer["norm"]["pre_ffw"],
                                    pre_ffw=layer["norm"]["post_attn"]))
    assert _cf_error(swapped, top, parts) > 1e-2
    swapped = dict(layer, norm=dict(layer["norm"], post_ffw=layer["norm"]["post_ple"],
                                    post_ple=layer["norm"]["post_ffw"]))
    assert _cf_error(swapped, top, parts) > 1e-2


@pytest.mark.parametrize("plant", ["skip_on_pn", "skip_on_fres"])
def test_layer_composition_planted_skip_placement_is_caught(monkeypatch, plant):
    # out = (fres + pn) * skip; a skip on one term only changes the direction
    # of out, which the final RMS norm keeps
    layer, top, parts = _cf_setup()
    real = lo.add_scale

    def wrong(a, b, s):
        if s == 1.0:
            return real(a, b, s)
        if plant == "skip_on_pn":
            return real(a, lo.scale(b, s), 1.0)
        return real(lo.scale(a, s), b, 1.0)

    monkeypatch.setattr(lo, "add_scale", wrong)
    assert _cf_error(layer, top, parts) > 1e-2


def test_layer_composition_planted_ple_layer_index_is_caught(monkeypatch):
    # a two-layer model reading layer 0's PLE slice at layer 1 differs from
    # the same model reading its own slice
    layer, top, parts = _cf_setup()
    H, P = CF_H, CF_P
    rng = np.random.default_rng(9)
    tok_ple2 = rng.standard_normal((CF_V, 2 * P)).astype(np.float32)
    top2 = _selection(2 * P, H, rng.integers(0, H, 2 * P),
                      rng.integers(1, 8, 2 * P).astype(np.int8), 0x3F80)

    def run():
        m = lo.Model(H, 1, P, CF_V, [layer, dict(layer, skip=0.9)], parts["E"],
                     lambda ids: tok_ple2[np.asarray(ids)], top2, parts["ple_norm"],
                     parts["final"])
        return m.forward([1], 0)

    good = run()
    real = lo.gelu_ple
    monkeypatch.setattr(lo, "gelu_ple", lambda g, p, rows, layer_i, w, nl: real(g, p, rows, 0, w, nl))
    bad = run()
    assert np.linalg.norm(bad - good) / np.linalg.norm(good) > 1e-2


def test_dequant_model_equals_model():
    # the float64 dequantize-once product used for the E2B-width GPU checks
    # equals the scalar float64 oracle product up to summation order
    m, _ = _tiny_model(6)
    d = lo.DequantModel(m.hidden, m.heads, m.ple_dim, m.vocab, m.layers, m.E_bits, m.ple_rows,
                        m.top, m.ple_norm, m.final_norm, window=m.window)
    ids = [3, 9, 27, 1, 14, 22]
    a = m.forward(ids, 0)
    b = d.forward(ids, 0)
    np.testing.assert_allclose(b, a, rtol=1e-6, atol=1e-7)
    a2, b2 = m.forward([5], 6), d.forward([5], 6)
    np.testing.assert_allclose(b2, a2, rtol=1e-6, atol=1e-7)
    assert len(d._deq) > 0
