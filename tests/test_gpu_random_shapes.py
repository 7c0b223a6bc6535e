"""Seeded random shapes through the W4 linear entry points.

Each case draws a row count (the GEMV sizes 1-4 and the GEMM sizes above),
an output width that is rarely a tile multiple, an input width (a multiple
of the 32-value group), an activation dtype and an output dtype, and checks
the result against the binary64 product x . dequant(W)^T (max relative L2
error per row).  BF16 outputs must be the round-to-nearest-even of the FP32
outputs of the same call.
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


@pytest.mark.parametrize("seed", range(24))
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


@pytest.mark.parametrize("seed", range(8))
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
