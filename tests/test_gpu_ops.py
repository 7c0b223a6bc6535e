"""GPU parity of the decoder-layer ops (rms, addScale, scale, geluMul, geluPle,
normRope, attention, pleMix, embedding rows, argmax) against the oracle.

Tolerances: the kernels compute in FP32 with tree-shaped reductions; the
oracle in float64.  Element-wise ops are checked to a few FP32 ulps, the
normalisations to rtol 1e-5, attention to rtol 2e-5.  RoPE angles carry the
float32 pow/divide of the shader (theta = pos / base^(2p/hd)): one ulp of
pow moves theta by ~pos * 2^-23, so normRope allows that much times |y|.
Embedding rows and argmax are bit-exact / index-exact."""
import math

import numpy as np
import pytest

import layer_oracle as lo
import synthetic as syn

pytestmark = pytest.mark.gpu


def dev(g4, a):
    return g4.Buffer.from_array(np.ascontiguousarray(a))


def out(g4, n, dtype=np.float32):
    return g4.Buffer(int(n) * np.dtype(dtype).itemsize)


def assert_gelu_close(got, want, x, other):
    # 0.5 * x * (1 + tanh(z)) cancels for x << 0 in FP32 (as in the shader):
    # allow a few FP32 ulps of |x * other| on top of the relative bound.
    bound = 1e-6 + 2e-6 * np.abs(want) + 4 * 1.2e-7 * np.abs(x * other)
    assert np.all(np.abs(got - want) <= bound)


def rel_err(got, want):
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    return np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)


@pytest.mark.parametrize("rows,width,with_scale", [(1, 1536, True), (7, 1536, True),
                                                   (3, 256, False), (2, 512, False),
                                                   (5, 100, True)])
def test_rms(g4, rows, width, with_scale):
    rng = np.random.default_rng([rows, width])
    x = (rng.standard_normal((rows, width)) * 5).astype(np.float32)
    s = rng.uniform(0.5, 1.5, width).astype(np.float32)
    y = out(g4, rows * width)
    g4.rms(dev(g4, x), rows, width, dev(g4, s) if with_scale else None, y)
    want = lo.rms(x, width, s if with_scale else None)
    np.testing.assert_allclose(y.download(np.float32).reshape(rows, width), want, rtol=1e-5,
                               atol=1e-6)


def test_elementwise_ops(g4):
    rng = np.random.default_rng(9)
    n = 100003  # ragged: not a multiple of the block
    a = rng.standard_normal(n).astype(np.float32) * 4
    b = rng.standard_normal(n).astype(np.float32) * 4
    y = out(g4, n)
    g4.add_scale(dev(g4, a), dev(g4, b), n, 0.75, y)
    np.testing.assert_array_equal(y.download(np.float32), ((a + b) * np.float32(0.75)))
    g4.scale(dev(g4, a), n, 1 / math.sqrt(1536), y)
    np.testing.assert_array_equal(y.download(np.float32), a * np.float32(1 / math.sqrt(1536)))
    g4.gelu_mul(dev(g4, a), dev(g4, b), n, y)
    assert_gelu_close(y.download(np.float32), lo.gelu_mul(a, b), a, b)


def test_gelu_ple(g4):
    rng = np.random.default_rng(10)
    rows, width, layers = 3, 256, 35
    gate = rng.standard_normal((rows, width)).astype(np.float32) * 3
    ple = rng.standard_normal((rows, layers * width)).astype(np.float32)
    y = out(g4, rows * width)
    for layer in (0, 17, 34):
        g4.gelu_ple(dev(g4, gate), dev(g4, ple), rows, layer, width, layers, y)
        assert_gelu_close(y.download(np.float32).reshape(rows, width),
                          lo.gelu_ple(gate, ple, rows, layer, width, layers), gate,
                          ple.reshape(rows, layers, width)[:, layer, :])


@pytest.mark.parametrize("rows,heads,hd,pos0,prop,base", [
    (1, 8, 256, 0, 1.0, 1e4), (1, 8, 256, 37, 1.0, 1e4), (3, 8, 512, 5, 0.25, 1e6),
    (2, 1, 256, 700, 1.0, 1e4), (1, 1, 512, 767, 0.25, 1e6), (4, 2, 64, 3, 0.5, 100.0),
    (2, 3, 130, 9, 1.0, 1e4), (1, 2, 384, 11, 0.5, 1e6)])  # 65 / 192 pairs: 2 / 4 waves
def test_norm_rope(g4, rows, heads, hd, pos0, prop, base):
    rng = np.random.default_rng([rows, heads, hd, pos0])
    x = rng.standard_normal((rows, heads * hd)).astype(np.float32) * 2
    s = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    angles = int(math.floor(prop * hd / 2))
    y = out(g4, rows * heads * hd)
    g4.norm_rope(dev(g4, x), rows, heads, hd, pos0, dev(g4, s), angles, base, y)
    got = y.download(np.float32).reshape(rows, heads * hd)
    want = lo.norm_rope(x, rows, heads, hd, pos0, s, angles, base)
    # theta = pos / pow(base, 2p/hd) in float32: a one-ulp difference of pow
    # between libraries moves theta by ~pos * 2^-23, the output by that times |y|
    atol = 2e-6 + 2 * (pos0 + rows) * 1.2e-7 * float(np.abs(want).max())
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=atol)


@pytest.mark.parametrize("qrows,heads,hd,keylen,sliding,window", [
    (1, 8, 256, 1, True, 512), (1, 8, 256, 37, True, 512), (1, 8, 512, 600, False, 512),
    (1, 8, 256, 700, True, 512), (1, 8, 256, 700, True, 100), (5, 8, 256, 40, True, 16),
    (64, 8, 512, 64, False, 512), (33, 2, 128, 80, True, 20), (3, 1, 64, 9, False, 512),
    # a prompt: 512 rows over 512 keys (the matrix-core kernel, 256 row tiles)
    (512, 8, 256, 512, True, 512), (96, 8, 512, 300, False, 512), (40, 3, 64, 57, True, 11),
    # a few rows over a long cache: the key-split kernel
    (2, 8, 256, 700, True, 512), (3, 8, 512, 900, False, 512),
    # longer caches under the matrix-core kernel: windows that start past key
    # 0, three heads (row tiles across positions), one head over a short
    # window, one key past a multiple of 128
    (200, 8, 512, 1000, True, 512), (129, 3, 128, 385, False, 512),
    (257, 1, 64, 257, True, 100), (64, 8, 256, 129, False, 512),
    # head dim 512 (dim-split kernel, two key groups): one key tile (the
    # second group's only step fully masked), three heads under a 7-key
    # window cutting through tiles, one head over an odd tile count
    (5, 8, 512, 9, False, 512), (17, 3, 512, 33, True, 7), (31, 1, 512, 47, False, 512)])
def test_attention(g4, qrows, heads, hd, keylen, sliding, window):
    rng = np.random.default_rng([qrows, heads, hd, keylen, window])
    q = rng.standard_normal((qrows, heads * hd)).astype(np.float32) * 0.2
    k = rng.standard_normal((keylen, hd)).astype(np.float32)
    v = rng.standard_normal((keylen, hd)).astype(np.float32)
    qpos0 = keylen - qrows
    y = out(g4, qrows * heads * hd)
    g4.attention(dev(g4, q), dev(g4, k), dev(g4, v), qrows, heads, hd, keylen, qpos0, sliding,
                 window, y)
    got = y.download(np.float32).reshape(qrows, heads * hd)
    want = lo.attention(q, k, v, qrows, heads, hd, keylen, qpos0, sliding, window)
    check_attention(got, want, fp32_attention(q, k, v, qrows, heads, hd, keylen, qpos0, sliding,
                                              window))


@pytest.mark.parametrize("seed", range(24))
def test_attention_random_shapes(g4, seed):
    # Seeded random row counts, head counts and dims, cache lengths and
    # sliding windows: whichever kernel the shape selects (one row, key
    # split, matrix-core rows with or without the key-tile prefetch).
    rng = np.random.default_rng(4000 + seed)
    qrows = int(rng.choice([1, 2, 3, 5, 16, 17, 40, 64, 100, 200]))
    heads = int(rng.choice([1, 2, 3, 4, 8]))
    hd = int(rng.choice([64, 128, 256, 512]))
    keylen = qrows + int(rng.integers(0, 700 - qrows))
    sliding = bool(rng.integers(0, 2))
    window = int(rng.integers(1, 600))
    q = rng.standard_normal((qrows, heads * hd)).astype(np.float32) * 0.2
    k = rng.standard_normal((keylen, hd)).astype(np.float32)
    v = rng.standard_normal((keylen, hd)).astype(np.float32)
    qpos0 = keylen - qrows
    y = out(g4, qrows * heads * hd)
    g4.attention(dev(g4, q), dev(g4, k), dev(g4, v), qrows, heads, hd, keylen, qpos0, sliding,
                 window, y)
    got = y.download(np.float32).reshape(qrows, heads * hd)
    want = lo.attention(q, k, v, qrows, heads, hd, keylen, qpos0, sliding, window)
    check_attention(got, want, fp32_attention(q, k, v, qrows, heads, hd, keylen, qpos0, sliding,
                                              window))


def fp32_attention(q, k, v, qrows, heads, hd, keylen, qpos0, sliding, window):
    """The same attention evaluated plainly in float32 (numpy): the yardstick
    for FP32 rounding against the float64 oracle."""
    q = np.asarray(q, np.float32).reshape(qrows, heads, hd)
    k = np.asarray(k, np.float32)[:keylen]
    v = np.asarray(v, np.float32)[:keylen]
    lg = np.einsum("rhd,kd->rhk", q, k, dtype=np.float32)
    key = np.arange(keylen)[None, :]
    qp = (qpos0 + np.arange(qrows))[:, None]
    valid = key <= qp
    if sliding:
        valid &= key + window > qp
    lg = np.where(valid[:, None, :], lg, np.float32(-1e30))
    e = np.exp(lg - lg.max(axis=2, keepdims=True)).astype(np.float32)
    p = (e / e.sum(axis=2, keepdims=True)).astype(np.float32)
    return np.einsum("rhk,kd->rhd", p, v, dtype=np.float32).reshape(qrows, heads * hd)


def check_attention(got, want, plain):
    # An output is a convex combination of N(0,1) value rows computed in FP32;
    # against the float64 oracle its error is rounding of order keys * 2^-24 *
    # sum p|v|, whatever the summation order.  Bounds: every element within
    # 1e-5 absolute (or 2e-5 relative), and the mean error within 3x that of a
    # plain float32 evaluation of the same inputs; a mistake in the masks or
    # the indexing moves whole rows far beyond both.
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=1e-5)
    err = float(np.abs(got.astype(np.float64) - want).mean())
    ref = float(np.abs(plain.astype(np.float64) - want).mean())
    assert err <= 3 * ref + 1e-8, (err, ref)


def test_attention_cache_longer_than_keylen(g4):
    # the KV buffers hold max_seq rows; only the first keylen are read
    hd, heads, keylen, cap = 256, 8, 10, 64
    rng = np.random.default_rng(11)
    q = rng.standard_normal((1, heads * hd)).astype(np.float32)
    k = np.full((cap, hd), np.nan, np.float32)
    v = np.full((cap, hd), np.nan, np.float32)
    k[:keylen] = rng.standard_normal((keylen, hd))
    v[:keylen] = rng.standard_normal((keylen, hd))
    y = out(g4, heads * hd)
    g4.attention(dev(g4, q), dev(g4, k), dev(g4, v), 1, heads, hd, keylen, keylen - 1, True, 512, y)
    got = y.download(np.float32)
    assert np.all(np.isfinite(got))
    np.testing.assert_allclose(got, lo.attention(q, k, v, 1, heads, hd, keylen, keylen - 1, True,
                                                 512)[0], rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("qrows", [7, 40])
def test_attention_rows_cache_longer_than_keylen(g4, qrows):
    # many query rows (the matrix-core kernel): cache rows past keylen are NaN
    # and must never be read, whatever the tile overhang
    hd, heads, keylen, cap = 128, 8, 45, 96
    rng = np.random.default_rng(qrows)
    q = rng.standard_normal((qrows, heads * hd)).astype(np.float32) * 0.3
    k = np.full((cap, hd), np.nan, np.float32)
    v = np.full((cap, hd), np.nan, np.float32)
    k[:keylen] = rng.standard_normal((keylen, hd))
    v[:keylen] = rng.standard_normal((keylen, hd))
    qpos0 = keylen - qrows
    y = out(g4, qrows * heads * hd)
    g4.attention(dev(g4, q), dev(g4, k), dev(g4, v), qrows, heads, hd, keylen, qpos0, True, 16, y)
    got = y.download(np.float32).reshape(qrows, heads * hd)
    assert np.all(np.isfinite(got))
    want = lo.attention(q, k[:keylen], v[:keylen], qrows, heads, hd, keylen, qpos0, True, 16)
    check_attention(got, want, fp32_attention(q, k, v, qrows, heads, hd, keylen, qpos0, True, 16))


def test_ple_mix(g4):
    rng = np.random.default_rng(12)
    rows, width, layers = 4, 256, 35
    proj = rng.standard_normal((rows, layers * width)).astype(np.float32) * 0.3
    tok = rng.standard_normal((rows, layers * width)).astype(np.float32) * 0.05
    s = rng.uniform(0.5, 1.5, width).astype(np.float32)
    y = out(g4, rows * layers * width)
    g4.ple_mix(dev(g4, proj), dev(g4, s), dev(g4, tok), rows, width, layers, y)
    np.testing.assert_allclose(y.download(np.float32).reshape(rows, -1),
                               lo.ple_mix(proj, s, tok, rows, width, layers), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("rows,width", [(40, 256), (33, 300)])
def test_ple_mix_many_chunks_match_oracle_and_one_row_calls(g4, rows, width):
    # rows x 35 layers >= 1024 chunks take one wave per chunk; each one-row
    # call (35 chunks) takes one block per chunk.  Both add the squares in
    # the same order, so the rows must agree bit for bit.
    layers = 35
    rng = np.random.default_rng(14)
    proj = rng.standard_normal((rows, layers * width)).astype(np.float32) * 0.3
    tok = rng.standard_normal((rows, layers * width)).astype(np.float32) * 0.05
    s = rng.uniform(0.5, 1.5, width).astype(np.float32)
    sd = dev(g4, s)
    y = out(g4, rows * layers * width)
    g4.ple_mix(dev(g4, proj), sd, dev(g4, tok), rows, width, layers, y)
    got = y.download(np.float32).reshape(rows, -1)
    np.testing.assert_allclose(got, lo.ple_mix(proj, s, tok, rows, width, layers),
                               rtol=1e-5, atol=1e-6)
    for r in (0, rows // 2, rows - 1):
        y1 = out(g4, layers * width)
        g4.ple_mix(dev(g4, proj[r:r + 1]), sd, dev(g4, tok[r:r + 1]), 1, width, layers, y1)
        np.testing.assert_array_equal(y1.download(np.float32), got[r])


def test_embed_bit_exact_and_bad_id(g4):
    vocab, width = 5000, 1536
    rng = np.random.default_rng(13)
    E = syn.bf16_rne(rng.standard_normal((vocab, width), dtype=np.float32) * np.float32(0.05))
    ids = np.array([0, 4999, 17, 17, 2500], np.int32)
    s = math.sqrt(1536)
    y = out(g4, len(ids) * width)
    Eb = dev(g4, E)
    g4.embed(Eb, vocab, width, dev(g4, ids), len(ids), s, y)
    np.testing.assert_array_equal(y.download(np.float32).reshape(len(ids), width),
                                  lo.embed(E, ids, np.float32(s)))
    bad = np.array([3, -1, vocab], np.int32)
    y2 = out(g4, 3 * width)
    g4.embed(Eb, vocab, width, dev(g4, bad), 3, s, y2)
    got = y2.download(np.float32).reshape(3, width)
    np.testing.assert_array_equal(got[0], lo.embed(E, [3], np.float32(s))[0])
    assert np.all(np.isnan(got[1])) and np.all(np.isnan(got[2]))


@pytest.mark.parametrize("n", [1, 5, 4096, 4097, 262144])
def test_argmax_first_index_of_max_skipping_nonfinite(g4, oracle, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    if n > 10:
        x[n // 3] = x.max() + 1
        x[n - 2] = x[n // 3]  # a tie: the first index wins
        x[n // 5] = np.inf    # skipped like topK's isFinite check
        x[n // 7] = np.nan
    o = out(g4, 1, np.int32)
    g4.argmax(dev(g4, x), n, o)
    got = int(o.download(np.int32)[0])
    assert got == int(oracle.topk(x, 1)[0][0])


def test_argmax_no_finite_value(g4):
    x = np.array([np.nan, np.inf, -np.inf], np.float32)
    o = out(g4, 1, np.int32)
    g4.argmax(dev(g4, x), 3, o)
    assert int(o.download(np.int32)[0]) == -1


def test_op_argument_errors(g4):
    x = out(g4, 16)
    with pytest.raises(g4.G4Error) as e:
        g4.rms(x, 2, 16, None, x)  # 32 floats do not fit a 16-float buffer
    assert e.value.code == 2
    with pytest.raises(g4.G4Error) as e:
        g4.attention(x, x, x, 1, 9, 64, 1, 0, False, 512, x)  # heads > 8
    assert e.value.code == 1
    with pytest.raises(g4.G4Error) as e:
        g4.norm_rope(x, 1, 1, 16, 0, x, 9, 1e4, x)  # rope_angles > hd / 2
    assert e.value.code == 1
