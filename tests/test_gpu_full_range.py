"""The formats' whole nibble range through every kernel, against the oracle.

The W4 format stores q = nibble - 8, so nibble 0 is q = -8
(official-w4a16.js:15-19; the shader's `i32(...) - 8`, gpu-runtime.js:1096),
and the PLE format stores two's-complement nibbles, so nibble 8 is q = -8
(ple-w4-shard-reader.js:92; the shader's signed4, gpu-runtime.js:234-235).
The benchmark distributions stop at |q| <= 7, so these tests draw q uniform
over all of [-8, 7] with q = -8 in every 32-wide group, and run the device
dequant (bit-exact), the decode GEMVs at 1-4 rows, the prefill GEMM at the
M2048 shapes, the several-weight launches, the allocation-free linear and
the PLE gather (bit-exact) on them.  Linear outputs must be within relative
L2 1e-3 of the oracle's FP32 dequant-then-matMul and of the binary64
product (and, as everywhere, far inside it).

The packed-weight GEMM's per-output-row power-of-two shift (taken when the
rows' largest scales spread beyond 2^12) is checked here at the M2048 shape
the planner runs that kernel on, with BF16 and FP32 activations.
"""
import numpy as np
import pytest

import synthetic as syn

pytestmark = pytest.mark.gpu

TOL = 1e-3


def rel_l2_rows(y, ref):
    y = np.asarray(y, dtype=np.float64).reshape(ref.shape)
    num = np.linalg.norm(y - ref, axis=-1)
    den = np.maximum(np.linalg.norm(ref, axis=-1), 1e-300)
    return float((num / den).max())


def dense(q, scales):
    return q.astype(np.float64) * np.repeat(syn.bf16_to_f32(scales).astype(np.float64), 32, axis=1)


def full_weights(seed, n, k):
    packed, scales, q = syn.w4_weights(seed, n, k, full_range=True)
    # the generator's own promise: all 16 stored nibbles, nibble 0 in every group
    nib = (q.astype(np.int16) + 8).reshape(n, k // 32, 32)
    assert (nib == 0).any(axis=2).all()
    assert set(np.unique(nib).tolist()) == set(range(16))
    assert np.array_equal(syn.unpack_w4(packed), q)
    return packed, scales, q


def x_buffer(g4, bits, x, xd):
    return g4.Buffer.from_array(bits if xd == g4.BF16 else x.astype(np.float32))


def linear(g4, lin, xb, xd, rows, yd=0, noalloc=False):
    ye = 4 if yd == g4.F32 else 2
    yb = g4.Buffer(rows * lin.out_dim * ye)
    (lin.linear_noalloc if noalloc else lin.linear)(xb.ptr, xd, rows, yb.ptr, yd)
    return yb.download(np.float32 if yd == g4.F32 else np.uint16).reshape(rows, lin.out_dim)


def test_synthetic_full_range_generators():
    # CPU-side promise of the PLE generator (the W4 one is checked per use)
    data = syn.ple_shard(5, 0, 64, 512, full_range=True)
    packed = data[:64 * 256].reshape(64, 256)
    nib = np.stack([packed & 15, packed >> 4], axis=-1).reshape(64, 512)
    assert set(np.unique(nib).tolist()) == set(range(16))
    assert (nib.reshape(64, 16, 32) == 8).any(axis=2).all()


@pytest.mark.parametrize("n,k", [(256, 1536), (96, 256), (130, 6144)])
def test_dequant_full_range_bit_exact(g4, oracle, n, k):
    packed, scales, q = full_weights(500 + n, n, k)
    lin = g4.W4Linear(packed, scales)
    out = g4.Buffer(n * k * 4)
    lin.dequant(0, n, out.ptr, g4.F32)
    got = out.download(np.float32).reshape(n, k)
    rc, want = oracle.w4_dequant_rows(packed, syn.bf16_to_f32(scales), n, k, 0, n)
    assert rc == 0
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # every q = -8 element came out as -8 * its group's scale
    s = np.repeat(syn.bf16_to_f32(scales).reshape(n, k // 32), 32, axis=1)
    assert np.array_equal(got[q == -8], (-8.0 * s[q == -8]).astype(np.float32))
    outb = g4.Buffer(n * k * 2)
    lin.dequant(0, n, outb.ptr, g4.BF16)
    assert np.array_equal(outb.download(np.uint16).reshape(n, k),
                          oracle.f32_to_bf16_array(want).reshape(n, k))


# (out_dim, in_dim): the row-split GEMV (K 1536, 2048), the flat split (K 256,
# 6144) and a K 12288 flat split with more than one x chunk per lane
GEMV_SHAPES = [(6144, 1536), (2048, 2048), (1536, 256), (1536, 6144), (256, 12288)]


@pytest.mark.parametrize("x_dtype_name", ["bf16", "f32"])
@pytest.mark.parametrize("n,k", GEMV_SHAPES)
def test_gemv_full_range_rows_1_to_4(g4, oracle, n, k, x_dtype_name):
    packed, scales, q = full_weights(510 + k, n, k)
    lin = g4.W4Linear(packed, scales)
    w = dense(q, scales)
    xd = g4.BF16 if x_dtype_name == "bf16" else g4.F32
    for rows in (1, 2, 3, 4):
        bits, x = syn.activations(520 + rows, rows, k)
        if xd == g4.F32:  # full FP32 mantissas: the hi + lo split path
            x = np.random.default_rng(rows).standard_normal((rows, k)).astype(np.float32)
        y = linear(g4, lin, x_buffer(g4, bits, x, xd), xd, rows)
        ref64 = x.astype(np.float64) @ w.T
        ref32 = oracle.w4_linear(x, packed, scales).astype(np.float64)
        assert rel_l2_rows(y, ref32) <= TOL, rows
        assert rel_l2_rows(y, ref64) < 1e-4, rows


@pytest.mark.parametrize("x_dtype_name", ["bf16", "f32"])
@pytest.mark.parametrize("n,k", [(6144, 1536), (1536, 6144)])
def test_gemm_m2048_full_range(g4, oracle, n, k, x_dtype_name):
    packed, scales, q = full_weights(530 + n, n, k)
    lin = g4.W4Linear(packed, scales)
    xd = g4.BF16 if x_dtype_name == "bf16" else g4.F32
    bits, x = syn.activations(531, 2048, k)
    if xd == g4.F32:
        x = np.random.default_rng(532).standard_normal((2048, k)).astype(np.float32)
    xb = x_buffer(g4, bits, x, xd)
    y = linear(g4, lin, xb, xd, 2048)
    ref = x.astype(np.float64) @ dense(q, scales).T
    assert rel_l2_rows(y, ref) <= (TOL if xd == g4.BF16 else 1e-5)
    sample = np.array([0, 1, 1000, 2047])
    assert rel_l2_rows(y[sample], oracle.w4_linear(x[sample], packed, scales).astype(np.float64)) <= TOL
    # the allocation-free entry point runs the same kernels: identical bits,
    # or (BF16 x at K 6144: x' and four K-slice planes, 75.5 MB) a refusal
    # of a call beyond its 64 MiB
    try:
        z = linear(g4, lin, xb, xd, 2048, noalloc=True)
    except g4.G4Error as e:
        assert (k, xd) == (6144, g4.BF16)
        assert e.code == g4.G4_E_ARG and "static scratch" in str(e)
    else:
        assert np.array_equal(z.view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("rows", [1, 512])
def test_linear_multi_full_range(g4, rows):
    k = 1536
    shapes = (2048, 256, 256)
    bits, x = syn.activations(540, rows, k)
    if rows > 1:
        x = np.random.default_rng(541).standard_normal((rows, k)).astype(np.float32)
    xd = g4.BF16 if rows == 1 else g4.F32
    xb = x_buffer(g4, bits, x, xd)
    lins, refs = [], []
    for i, n in enumerate(shapes):
        packed, scales, q = full_weights(542 + i, n, k)
        lins.append(g4.W4Linear(packed, scales))
        refs.append(x.astype(np.float64) @ dense(q, scales).T)
    ys = [g4.Buffer(rows * n * 4) for n in shapes]
    g4.W4Linear.linear_multi(lins, xb.ptr, xd, rows, [y.ptr for y in ys], g4.F32)
    for lin, y, ref in zip(lins, ys, refs):
        got = y.download(np.float32).reshape(rows, lin.out_dim)
        assert rel_l2_rows(got, ref) <= (1e-4 if rows == 1 else 1e-5)
        if rows == 1:  # one-row launches run the single-weight body: identical bits
            assert np.array_equal(got, linear(g4, lin, xb, xd, rows))


@pytest.mark.parametrize("rows,n,k,f32x", [(700, 1536, 6144, True), (3, 6144, 1536, False)])
def test_noalloc_full_range(g4, rows, n, k, f32x):
    packed, scales, q = full_weights(550 + rows, n, k)
    lin = g4.W4Linear(packed, scales)
    bits, x = syn.activations(551, rows, k)
    xd = g4.F32 if f32x else g4.BF16
    xb = x_buffer(g4, bits, x, xd)
    for yd in (g4.F32, g4.BF16):
        a = linear(g4, lin, xb, xd, rows, yd)
        b = linear(g4, lin, xb, xd, rows, yd, noalloc=True)
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    ref = x.astype(np.float64) @ dense(q, scales).T
    assert rel_l2_rows(linear(g4, lin, xb, xd, rows, noalloc=True), ref) <= TOL


def test_device_fill_full_range_kinds(g4, oracle):
    # the device generator's full-range kinds cover all 16 nibbles, and a
    # weight loaded from them dequantizes bit-exactly like the oracle
    n, k = 512, 2048
    pk = g4.Buffer(n * k // 2)
    sc = g4.Buffer(n * (k // 32) * 2)
    g4.fill_random(pk, n * k // 8, g4.RAND_W4_PACKED_FULL, 91)
    g4.fill_random(sc, n * (k // 32), g4.RAND_BF16_ABS_NORMAL, 92, 0.02)
    packed = pk.download(np.uint32).reshape(n, k // 8)
    scales = sc.download(np.uint16).reshape(n, k // 32)
    nib = (packed[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15
    counts = np.bincount(nib.reshape(-1), minlength=16)
    assert counts.min() > 0.9 * nib.size / 16 and counts.max() < 1.1 * nib.size / 16
    lin = g4.W4Linear(packed, scales)
    out = g4.Buffer(n * k * 4)
    lin.dequant(0, n, out.ptr, g4.F32)
    rc, want = oracle.w4_dequant_rows(packed, syn.bf16_to_f32(scales), n, k, 0, n)
    assert rc == 0
    assert np.array_equal(out.download(np.float32).view(np.uint32), want.reshape(-1).view(np.uint32))
    pb = g4.Buffer(1 << 16)
    g4.fill_random(pb, 1 << 16, g4.RAND_PLE_PACKED_FULL, 93)
    b = pb.download(np.uint8)
    counts = np.bincount(np.concatenate([b & 15, b >> 4]), minlength=16)
    assert counts.min() > 0.9 * 2 * b.size / 16 and counts.max() < 1.1 * 2 * b.size / 16


VOCAB, WIDTH, RPS = 10000, 8960, 4096


@pytest.fixture(scope="module")
def full_table(g4):
    shards = syn.ple_table(77, VOCAB, WIDTH, RPS, threads=8, full_range=True)
    t = g4.PleTable(VOCAB, WIDTH, 32, RPS)
    for i, s in enumerate(shards):
        t.upload_shard(i, s)
    host = np.concatenate(shards)
    yield t, host
    t.free()


@pytest.mark.parametrize("n", [1, 127, 300, 2048])
def test_ple_gather_full_range_bit_exact(g4, oracle, full_table, n):
    # 1 and 127 ids take the element kernel, 300 and 2048 the row kernel
    t, host = full_table
    ids = syn.token_ids(60 + n, n, VOCAB)
    if n > 4:
        ids[:4] = [0, VOCAB - 1, RPS - 1, RPS]
    want = oracle.ple_gather(host, VOCAB, WIDTH, RPS, ids)
    for dt in (g4.F32, g4.BF16):
        out = g4.Buffer(n * WIDTH * (4 if dt == g4.F32 else 2))
        t.gather(ids, out.ptr, dt)
        if dt == g4.F32:
            got = out.download(np.float32).reshape(n, WIDTH)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        else:
            got = out.download(np.uint16)
            assert np.array_equal(got, oracle.f32_to_bf16_array(want))


def test_ple_gather_full_range_minus_eight_values(g4, oracle, full_table):
    # the q = -8 elements of a gathered row are exactly -8 * scale
    t, host = full_table
    tid = 4097  # shard 1, local row 1
    shard1 = host[RPS * (WIDTH // 2 + WIDTH // 16):]
    packed = shard1[(tid - RPS) * (WIDTH // 2):(tid - RPS + 1) * (WIDTH // 2)]
    sc_off = min(RPS, VOCAB - RPS) * (WIDTH // 2)  # shard 1's packed block, then its scales
    scales = shard1[sc_off + (tid - RPS) * (WIDTH // 16):sc_off + (tid - RPS + 1) * (WIDTH // 16)]
    scales = syn.bf16_to_f32(scales.view("<u2"))
    nib = np.stack([packed & 15, packed >> 4], axis=-1).reshape(WIDTH)
    out = g4.Buffer(WIDTH * 4)
    t.gather(np.array([tid], np.int32), out.ptr, g4.F32)
    got = out.download(np.float32)
    s = np.repeat(scales, 32)
    assert (nib == 8).sum() >= WIDTH // 32
    assert np.array_equal(got[nib == 8], (-8.0 * s[nib == 8]).astype(np.float32))
    assert np.array_equal(got.view(np.uint32),
                          oracle.ple_gather(host, VOCAB, WIDTH, RPS, [tid])[0].view(np.uint32))


@pytest.mark.parametrize("x_dtype_name", ["bf16", "f32"])
def test_gemm_rb_row_shift_m2048(g4, x_dtype_name):
    # M2048 N6144 K1536 is planned on the packed-weight GEMM.  Scales by output
    # row spread over 2^-30 .. 2^0 (far beyond 2^12), so that kernel runs with
    # a power-of-two shift per output row; rows of any relative magnitude keep
    # every bit, and each row is checked against the binary64 product.
    n, k, rows = 6144, 1536, 2048
    G = k // 32
    rng = np.random.default_rng(2048)
    q = rng.integers(-8, 8, size=(n, k), dtype=np.int8)
    ex = (-30.0 * np.arange(n) / (n - 1))[:, None] - rng.uniform(0, 1, (n, G))
    scales = syn.bf16_rne(np.exp2(ex).astype(np.float32))
    lin = g4.W4Linear(syn.pack_w4(q), scales)
    xd = g4.BF16 if x_dtype_name == "bf16" else g4.F32
    bits, x = syn.activations(2049, rows, k)
    if xd == g4.F32:
        x = rng.standard_normal((rows, k)).astype(np.float32)
    y = linear(g4, lin, x_buffer(g4, bits, x, xd), xd, rows)
    w = dense(q, scales)
    # per output column (= weight row) relative error over all 2048 rows
    ref = x.astype(np.float64) @ w.T
    err = np.linalg.norm(y.astype(np.float64) - ref, axis=0) / np.linalg.norm(ref, axis=0)
    assert err.max() < 1e-5, (x_dtype_name, int(err.argmax()), float(err.max()))
