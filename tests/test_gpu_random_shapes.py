"""Seeded random shapes through the W4 linear, dequant and PLE entry points.

A linear case draws a row count (the GEMV sizes 1-4 and the GEMM sizes
above), an output width that is rarely a tile multiple, an input width (a
multiple of the 32-value group), an activation dtype and an output dtype, and
checks the result against the binary64 product x . dequant(W)^T (max
relative L2 error per row); BF16 outputs must be the round-to-nearest-even of
the FP32 outputs of the same call.  Dequant and PLE cases draw shapes, row
ranges, table geometry and ids, and must match the oracle bit for bit.
"""
import numpy as np
import pytest

import synthetic as syn

pytestmark = pytest.mark.gpu

ROWS = [1, 2, 3, 4, 5, 8, 33, 100, 257]


def dense(q, scales):
    return q.astype(np.float64) * np.repeat(syn.bf16_to_f32(scales).astype(np.float64), 32, axis=1)


def rel_l2_rows(y, ref):
    num = np.linalg.norm(np.asarray(y, np.float64) - ref, axis=-1)
    den = np.maximum(np.linalg.norm(ref, axis=-1), 1e-300)
    return float((num / den).max())


def draw(seed):
    rng = np.random.default_rng(1000 + seed)
    rows = int(rng.choice(ROWS))
    n = int(rng.integers(1, 700))
    k = 32 * int(rng.integers(1, 129))  # 32 .. 4096
    f32x = bool(rng.integers(0, 2))
    return rng, rows, n, k, f32x


def activations(g4, rng, rows, k, f32x):
    x = rng.standard_normal((rows, k)).astype(np.float32)
    if f32x:
        return g4.Buffer.from_array(x), x, g4.F32
    bits = syn.bf16_rne(x)
    return g4.Buffer.from_array(bits), syn.bf16_to_f32(bits).reshape(rows, k), g4.BF16


@pytest.mark.parametrize("seed", range(48))
def test_random_linear(g4, seed):
    rng, rows, n, k, f32x = draw(seed)
    packed, scales, q = syn.w4_weights(500 + seed, n, k)
    lin = g4.W4Linear(packed, scales)
    xb, x, xd = activations(g4, rng, rows, k, f32x)
    y32 = g4.Buffer(rows * n * 4)
    y16 = g4.Buffer(rows * n * 2)
    lin.linear(xb.ptr, xd, rows, y32.ptr, g4.F32)
    lin.linear(xb.ptr, xd, rows, y16.ptr, g4.BF16)
    got = y32.download(np.float32).reshape(rows, n)
    ref = x.astype(np.float64) @ dense(q, scales).T
    assert rel_l2_rows(got, ref) <= 1e-4, (rows, n, k, f32x)
    assert np.array_equal(y16.download(np.uint16).reshape(rows, n),
                          syn.bf16_rne(got).reshape(rows, n)), (rows, n, k, f32x)


@pytest.mark.parametrize("k", [16384, 32768])
@pytest.mark.parametrize("rows", [1, 3, 40])
@pytest.mark.parametrize("f32x", [False, True])
def test_long_in_dim_linear(g4, k, rows, f32x):
    # in_dims whose activation row no longer fits the GEMVs' LDS staging
    # (32768 BF16, 16384 and 32768 FP32) take the GEMM at every row count;
    # the reference's GPUOps.w4 takes any inDim
    rng = np.random.default_rng([k, rows, f32x])
    n = 300
    packed, scales, q = syn.w4_weights(k + rows, n, k)
    lin = g4.W4Linear(packed, scales)
    xb, x, xd = activations(g4, rng, rows, k, f32x)
    y32 = g4.Buffer(rows * n * 4)
    lin.linear(xb.ptr, xd, rows, y32.ptr, g4.F32)
    ref = x.astype(np.float64) @ dense(q, scales).T
    assert rel_l2_rows(y32.download(np.float32).reshape(rows, n), ref) <= 1e-4
    ys = [g4.Buffer(rows * w * 4) for w in (64, 200)]
    lins = [g4.W4Linear(*syn.w4_weights(k + w, w, k)[:2]) for w in (64, 200)]
    g4.W4Linear.linear_multi(lins, xb.ptr, xd, rows, [b.ptr for b in ys], g4.F32)
    for w, lw, yb in zip((64, 200), lins, ys):
        _, sc, qq = syn.w4_weights(k + w, w, k)
        r = x.astype(np.float64) @ dense(qq, sc).T
        assert rel_l2_rows(yb.download(np.float32).reshape(rows, w), r) <= 1e-4


@pytest.mark.parametrize("seed", range(16))
def test_random_linear_multi(g4, seed):
    rng, rows, _, k, f32x = draw(100 + seed)
    widths = [int(v) for v in rng.integers(1, 700, size=int(rng.integers(2, 4)))]
    lins, refs = [], []
    xb, x, xd = activations(g4, rng, rows, k, f32x)
    for i, n in enumerate(widths):
        packed, scales, q = syn.w4_weights(600 + 4 * seed + i, n, k)
        lins.append(g4.W4Linear(packed, scales))
        refs.append(x.astype(np.float64) @ dense(q, scales).T)
    ys = [g4.Buffer(rows * n * 4) for n in widths]
    g4.W4Linear.linear_multi(lins, xb.ptr, xd, rows, [y.ptr for y in ys], g4.F32)
    for y, n, ref in zip(ys, widths, refs):
        got = y.download(np.float32).reshape(rows, n)
        assert rel_l2_rows(got, ref) <= 1e-4, (rows, widths, k, f32x)


@pytest.mark.parametrize("seed", range(8))
def test_random_ple_geometry(g4, oracle, seed):
    # Random table geometry (vocab, width, rows per shard, a short last
    # shard) and ids with the edges: rows bit-exact against the oracle's
    # readRows restatement, BF16 the round-to-nearest-even of FP32.
    rng = np.random.default_rng(2000 + seed)
    width = 32 * int(rng.integers(1, 129))
    rps = 8 * int(rng.integers(1, 65))
    vocab = int(rng.integers(1, 5000))
    shards = syn.ple_table(300 + seed, vocab, width, rps, threads=4)
    t = g4.PleTable(vocab, width, 32, rps)
    for i, s in enumerate(shards):
        t.upload_shard(i, s)
    host = np.concatenate(shards)
    ids = rng.integers(0, vocab, size=int(rng.integers(1, 300))).astype(np.int32)
    ids[: min(3, len(ids))] = [0, vocab - 1, min(rps, vocab - 1)][: min(3, len(ids))]
    want = oracle.ple_gather(host, vocab, width, rps, ids)
    out = g4.Buffer(len(ids) * width * 4)
    t.gather(ids, out.ptr, g4.F32)
    assert np.array_equal(out.download(np.uint32).reshape(-1), want.view(np.uint32).reshape(-1))
    out16 = g4.Buffer(len(ids) * width * 2)
    t.gather(ids, out16.ptr, g4.BF16)
    assert np.array_equal(out16.download(np.uint16).reshape(-1), oracle.f32_to_bf16_array(want))
    t.free()


@pytest.mark.parametrize("seed", range(8))
def test_random_dequant(g4, oracle, seed):
    # dequantizeOfficialW4A16Rows over random shapes and row ranges, bit-exact.
    rng = np.random.default_rng(3000 + seed)
    n, k = int(rng.integers(1, 600)), 32 * int(rng.integers(1, 129))
    packed, scales, _ = syn.w4_weights(700 + seed, n, k)
    lin = g4.W4Linear(packed, scales)
    r0 = int(rng.integers(0, n))
    rc = int(rng.integers(0, n - r0 + 1))
    want_rc, want = oracle.w4_dequant_rows(packed, syn.bf16_to_f32(scales), n, k, r0, rc)
    assert want_rc == 0
    if rc == 0:
        return
    out = g4.Buffer(rc * k * 4)
    lin.dequant(r0, rc, out.ptr, g4.F32)
    assert np.array_equal(out.download(np.uint32).reshape(-1), want.view(np.uint32).reshape(-1))
