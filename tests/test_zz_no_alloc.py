"""g4_w4_linear_noalloc, the allocation-free linear, against g4_w4_linear.

It runs g4_w4_linear's kernels with their GEMM scratch in a static device
array, so its outputs must equal g4_w4_linear's bit for bit (and be within
the 1e-3 contract of the binary64 product).  Two calls in a row, the second
with a smaller input, check that the shared array's leftover contents from
the first call do not leak into the second; a recording replayed several
times checks it under graph capture, where allocation is impossible."""
import numpy as np
import pytest

import synthetic as syn

pytestmark = pytest.mark.gpu


def dense(q, scales):
    return q.astype(np.float64) * np.repeat(syn.bf16_to_f32(scales).astype(np.float64), 32, axis=1)


def rel_l2_rows(y, ref):
    num = np.linalg.norm(np.asarray(y, np.float64) - ref, axis=-1)
    return float((num / np.maximum(np.linalg.norm(ref, axis=-1), 1e-300)).max())


def case(g4, seed, rows, n, k, f32x):
    packed, scales, q = syn.w4_weights(seed, n, k)
    lin = g4.W4Linear(packed, scales)
    bits, x = syn.activations(seed, rows, k)
    xb = g4.Buffer.from_array(x if f32x else bits)
    return lin, xb, x, q, scales, (g4.F32 if f32x else g4.BF16)


def both(g4, lin, xb, xd, rows, yd):
    ye = 4 if yd == g4.F32 else 2
    a, b = g4.Buffer(rows * lin.out_dim * ye), g4.Buffer(rows * lin.out_dim * ye)
    lin.linear(xb.ptr, xd, rows, a.ptr, yd)
    lin.linear_noalloc(xb.ptr, xd, rows, b.ptr, yd)
    dt = np.uint32 if yd == g4.F32 else np.uint16
    return a.download(dt), b.download(dt)


@pytest.mark.parametrize("first,second", [
    # (rows, out_dim, in_dim, FP32 x): the prefill shapes, then a smaller call
    ((2048, 6144, 1536, False), (100, 1536, 6144, True)),   # second splits K
    ((512, 1536, 12288, True), (40, 300, 2048, False)),
    ((300, 2048, 1536, True), (3, 6144, 1536, False)),     # second is a GEMV
])
def test_noalloc_equals_linear_on_two_calls(g4, first, second):
    for i, (rows, n, k, f32x) in enumerate((first, second)):
        lin, xb, x, q, scales, xd = case(g4, 70 + i, rows, n, k, f32x)
        for yd in (g4.F32, g4.BF16):
            a, b = both(g4, lin, xb, xd, rows, yd)
            assert np.array_equal(a, b), (rows, n, k, f32x, yd)
        got = g4.Buffer(rows * n * 4)
        lin.linear_noalloc(xb.ptr, xd, rows, got.ptr, g4.F32)
        ref = x.astype(np.float64) @ dense(q, scales).T
        assert rel_l2_rows(got.download(np.float32).reshape(rows, n), ref) < 1e-3


def test_noalloc_recorded_and_replayed(g4):
    # recorded into a command buffer: no scratch sizing call comes first
    lin, xb, x, q, scales, xd = case(g4, 81, 700, 2560, 2048, True)
    want = g4.Buffer(700 * 2560 * 4)
    lin.linear(xb.ptr, xd, 700, want.ptr, g4.F32)
    y = g4.Buffer(700 * 2560 * 4)
    with g4.Encoder() as enc:
        lin.linear_noalloc(xb.ptr, xd, 700, y.ptr, g4.F32)
    for _ in range(3):
        y.upload(np.zeros(700 * 2560, np.float32))
        enc.cmdbuf.submit()
        assert np.array_equal(y.download(np.uint32), want.download(np.uint32))
    enc.cmdbuf.free()


def test_noalloc_refuses_more_than_its_scratch(g4):
    lin, xb, _, _, _, _ = case(g4, 90, 8, 64, 4096, True)
    x_big = g4.Buffer(4096 * 4096 * 4)
    y = g4.Buffer(4096 * 64 * 4)
    with pytest.raises(g4.G4Error) as e:
        lin.linear_noalloc(x_big.ptr, g4.F32, 4096, y.ptr, g4.F32)
    assert e.value.code == g4.G4_E_ARG
    assert "bytes of scratch" in str(e.value) and "67108864" in str(e.value)
    # the failed call launched nothing and left the entry point usable
    y8 = g4.Buffer(8 * 64 * 4)
    lin.linear_noalloc(xb.ptr, g4.F32, 8, y8.ptr, g4.F32)
    assert np.all(np.isfinite(y8.download(np.float32)))
