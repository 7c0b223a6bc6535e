"""GPU parity of the W4A16 linear entry points against the oracle.

Bar: dequantized weights bit-exact (FP32) and bit-exact to round-to-nearest-
even of the exact value (BF16); matmul outputs within max-over-rows relative
L2 error 1e-3 of the reference's FP32 dequant-then-matMul (the oracle), and
of the binary64 product.
"""
import ctypes

import numpy as np
import pytest

import synthetic as syn

pytestmark = pytest.mark.gpu

TOL = 1e-3  # max relative L2 error per output row

# (out_dim, in_dim) of every W4A16 projection of Gemma-4-E2B
# (gemma4-webgpu.js:65-95 layer schedule; hidden 1536).
E2B_SHAPES = {
    "q_sliding": (2048, 1536), "kv_sliding": (256, 1536), "o_sliding": (1536, 2048),
    "gate_up_l0_14": (6144, 1536), "down_l0_14": (1536, 6144),
    "q_full": (4096, 1536), "kv_full": (512, 1536), "o_full": (1536, 4096),
    "gate_up_l15_34": (12288, 1536), "down_l15_34": (1536, 12288),
    "ple_gate": (256, 1536), "ple_proj": (1536, 256), "top_proj": (8960, 1536),
}


def rel_l2_rows(y, ref):
    y = np.asarray(y, dtype=np.float64).reshape(ref.shape)
    num = np.linalg.norm(y - ref, axis=-1)
    den = np.maximum(np.linalg.norm(ref, axis=-1), 1e-300)
    return float((num / den).max())


def dense(q, scales):
    return q.astype(np.float64) * np.repeat(syn.bf16_to_f32(scales).astype(np.float64), 32, axis=1)


def run_linear(g4, lin, x_bits, x_f32, rows, x_dtype, y_dtype=0):
    if x_dtype == g4.BF16:
        xb = g4.Buffer.from_array(x_bits)
    else:
        xb = g4.Buffer.from_array(x_f32.astype(np.float32))
    ye = 4 if y_dtype == g4.F32 else 2
    yb = g4.Buffer(rows * lin.out_dim * ye)
    lin.linear(xb.ptr, x_dtype, rows, yb.ptr, y_dtype)
    out = yb.download(np.float32 if y_dtype == g4.F32 else np.uint16)
    return out.reshape(rows, lin.out_dim)


def test_dequant_bit_exact(g4, oracle):
    for seed, (n, k) in enumerate([(256, 1536), (96, 256), (130, 6144)]):
        packed, scales, q = syn.w4_weights(100 + seed, n, k)
        lin = g4.W4Linear(packed, scales)
        out = g4.Buffer(n * k * 4)
        lin.dequant(0, n, out.ptr, g4.F32)
        got = out.download(np.float32).reshape(n, k)
        rc, want = oracle.w4_dequant_rows(packed, syn.bf16_to_f32(scales), n, k, 0, n)
        assert rc == 0
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        # a sub-range, as BF16 (roundFloat32ToBF16 of the exact value)
        r0, rc_ = n // 3, n // 2
        outb = g4.Buffer(rc_ * k * 2)
        lin.dequant(r0, rc_, outb.ptr, g4.BF16)
        gotb = outb.download(np.uint16).reshape(rc_, k)
        assert np.array_equal(gotb, oracle.f32_to_bf16_array(want[r0:r0 + rc_]).reshape(rc_, k))


def test_gemv_config0_against_oracle(g4, oracle):
    # M=1, K=1536, N=6144, BF16 activations, FP32 accumulate.
    packed, scales, q = syn.w4_weights(0, 6144, 1536)
    x_bits, x = syn.activations(0, 1, 1536)
    lin = g4.W4Linear(packed, scales)
    y_bf = run_linear(g4, lin, x_bits, x, 1, g4.BF16)
    y_f32 = run_linear(g4, lin, x_bits, x, 1, g4.F32)
    # the same values in either input dtype give the same arithmetic
    assert np.array_equal(y_bf, y_f32)
    ref32 = oracle.w4_linear(x, packed, scales)
    ref64 = oracle.w4_linear_f64(x, packed, scales)
    assert rel_l2_rows(y_bf, ref32.astype(np.float64)) <= TOL
    assert rel_l2_rows(y_bf, ref64) <= TOL
    # and far inside it
    assert rel_l2_rows(y_bf, ref64) < 1e-4


@pytest.mark.parametrize("name", sorted(E2B_SHAPES))
def test_gemv_e2b_shapes(g4, name):
    n, k = E2B_SHAPES[name]
    packed, scales, q = syn.w4_weights(len(name), n, k)
    x_bits, x = syn.activations(len(name), 1, k)
    lin = g4.W4Linear(packed, scales)
    y = run_linear(g4, lin, x_bits, x, 1, g4.BF16)
    ref = x.astype(np.float64) @ dense(q, scales).T
    assert rel_l2_rows(y, ref) <= TOL


@pytest.mark.parametrize("rows", [2, 3, 4, 5, 7, 9])
def test_linear_few_rows(g4, oracle, rows):
    packed, scales, q = syn.w4_weights(rows, 2048, 1536)
    x_bits, x = syn.activations(rows, rows, 1536)
    lin = g4.W4Linear(packed, scales)
    y = run_linear(g4, lin, x_bits, x, rows, g4.F32)
    ref = oracle.w4_linear(x, packed, scales).astype(np.float64)
    assert rel_l2_rows(y, ref) <= TOL
    ref64 = x.astype(np.float64) @ dense(q, scales).T
    assert rel_l2_rows(y, ref64) < 1e-4


def test_one_hot_input_returns_a_weight_column_exactly(g4):
    n, k = 640, 1536
    packed, scales, q = syn.w4_weights(77, n, k)
    lin = g4.W4Linear(packed, scales)
    w = (q.astype(np.float32) * np.repeat(syn.bf16_to_f32(scales).reshape(n, k // 32), 32, axis=1))
    for col in (0, 31, 32, 700, k - 1):
        x = np.zeros((1, k), dtype=np.float32)
        x[0, col] = 1.0
        y = run_linear(g4, lin, None, x, 1, g4.F32)
        assert np.array_equal(y[0], w[:, col])


def test_bf16_output_is_rne_of_fp32_output(g4, oracle):
    packed, scales, q = syn.w4_weights(5, 1536, 2048)
    x_bits, x = syn.activations(5, 1, 2048)
    lin = g4.W4Linear(packed, scales)
    y32 = run_linear(g4, lin, x_bits, x, 1, g4.BF16, g4.F32)
    y16 = run_linear(g4, lin, x_bits, x, 1, g4.BF16, g4.BF16)
    assert np.array_equal(y16.reshape(-1), oracle.f32_to_bf16_array(y32))


def test_prefill_gemm_config3(g4, oracle):
    # M=2048 tokens at both prefill shapes; checked against the binary64
    # product everywhere and the FP32 oracle on a sample of rows.
    for (n, k) in [(6144, 1536), (1536, 6144)]:
        packed, scales, q = syn.w4_weights(3, n, k)
        x_bits, x = syn.activations(3, 2048, k)
        lin = g4.W4Linear(packed, scales)
        y = run_linear(g4, lin, x_bits, x, 2048, g4.BF16)
        ref = x.astype(np.float64) @ dense(q, scales).T
        assert rel_l2_rows(y, ref) <= TOL
        sample = np.array([0, 1, 777, 2047])
        ref32 = oracle.w4_linear(x[sample], packed, scales).astype(np.float64)
        assert rel_l2_rows(y[sample], ref32) <= TOL


@pytest.mark.parametrize("x_dtype_name", ["f32", "bf16"])
@pytest.mark.parametrize("k", [256, 320, 96])
def test_gemm_ragged_shapes_and_activation_ranges(g4, x_dtype_name, k):
    # Rows and columns that are not tile multiples, and activation rows far
    # outside FP16's range (1e5..1e-7 scale factors): the per-row power-of-two
    # rescale must keep every row inside the tolerance.  K 256 runs the
    # unrolled branch-free stage loop (8 groups: 4 stages of 2), K 320 (5
    # stages) and K 96 (3 groups, one per stage) the general one.
    n, m = 200, 130
    packed, scales, q = syn.w4_weights(9, n, k)
    rng = np.random.default_rng(9)
    x = rng.standard_normal((m, k)).astype(np.float32)
    factors = np.array([1e5, 3e4, 1.0, 1e-3, 1e-7, 7.0] * 22, dtype=np.float32)[:m]
    x *= factors[:, None]
    x[5] = 0.0  # an all-zero row
    x_bits = syn.bf16_rne(x)
    if x_dtype_name == "bf16":
        x = syn.bf16_to_f32(x_bits).reshape(m, k)
    lin = g4.W4Linear(packed, scales)
    y = run_linear(g4, lin, x_bits, x, m, g4.BF16 if x_dtype_name == "bf16" else g4.F32)
    ref = x.astype(np.float64) @ dense(q, scales).T
    nz = np.ones(m, bool)
    nz[5] = False
    assert rel_l2_rows(y[nz], ref[nz]) <= TOL
    assert np.all(y[5] == 0.0)


@pytest.mark.parametrize("rows,n,k", [(512, 1536, 6144), (512, 1536, 12288), (512, 1536, 2048),
                                        (512, 256, 1536), (300, 1536, 6144)])
def test_gemm_split_k_prefill_shapes(g4, rows, n, k):
    # The E2B prefill's 1536- and 256-wide outputs at 512 rows leave most CUs
    # idle as whole tiles, so K is split into partial planes that are added in
    # slice order (slices of 16+ stages; of 6 for N 256, the general loop).
    # FP32 activations, as the model feeds them, against the binary64 product:
    # hi + lo halves keep the error near FP32 rounding.
    packed, scales, q = syn.w4_weights(21, n, k)
    x = np.random.default_rng(21).standard_normal((rows, k)).astype(np.float32)
    lin = g4.W4Linear(packed, scales)
    y = run_linear(g4, lin, None, x, rows, g4.F32)
    ref = x.astype(np.float64) @ dense(q, scales).T
    assert rel_l2_rows(y, ref) <= 1e-5
    yb = run_linear(g4, lin, None, x, rows, g4.F32, g4.BF16)
    assert np.array_equal(yb, syn.bf16_rne(y).reshape(rows, n))


@pytest.mark.parametrize("rows,n,k,x_dtype_name", [(1900, 6100, 1536, "bf16"),
                                                   (1800, 1500, 6144, "bf16"),
                                                   (2100, 6144, 1536, "bf16"),
                                                   (1000, 6100, 1536, "f32"),
                                                   (700, 1500, 6144, "f32")])
def test_gemm_large_ragged(g4, rows, n, k, x_dtype_name):
    # Prefill-sized GEMMs off the tile grid: rows that are not a multiple of
    # the 128-row (BF16 x) or 64-row (FP32 x, two x' planes) tile, a ragged
    # last column tile (the weight's tile copy repeats its last row there), a
    # K split (N 1500) and grids of more than two rounds of the CUs; BF16
    # output is the RNE of the FP32 output.
    packed, scales, q = syn.w4_weights(31, n, k)
    x_bits, x = syn.activations(31, rows, k)
    if x_dtype_name == "f32":
        x = np.random.default_rng(31).standard_normal((rows, k)).astype(np.float32)
    xd = g4.BF16 if x_dtype_name == "bf16" else g4.F32
    lin = g4.W4Linear(packed, scales)
    y = run_linear(g4, lin, x_bits, x, rows, xd)
    ref = x.astype(np.float64) @ dense(q, scales).T
    assert rel_l2_rows(y, ref) <= (TOL if x_dtype_name == "bf16" else 1e-5)
    yb = run_linear(g4, lin, x_bits, x, rows, xd, g4.BF16)
    assert np.array_equal(yb, syn.bf16_rne(y).reshape(rows, n))


def test_gemm_matches_gemv_path(g4):
    # Rows 1..4 take the streaming GEMV, more rows the MFMA GEMM: the row a
    # caller computes must not depend on how many rows come with it.
    packed, scales, q = syn.w4_weights(13, 1536, 2048)
    x_bits, x = syn.activations(13, 40, 2048)
    lin = g4.W4Linear(packed, scales)
    big = run_linear(g4, lin, x_bits, x, 40, g4.BF16)
    ref = x.astype(np.float64) @ dense(q, scales).T
    for r in (0, 17, 39):
        one = run_linear(g4, lin, x_bits[r:r + 1], x[r:r + 1], 1, g4.BF16)
        assert rel_l2_rows(one, ref[r:r + 1]) < 1e-4
        assert rel_l2_rows(big[r:r + 1], ref[r:r + 1]) < 1e-4


@pytest.mark.parametrize("layout", ["by_row", "by_group"])
@pytest.mark.parametrize("x_dtype_name", ["bf16", "f32"])
def test_scales_spanning_2e40_stay_exact(g4, layout, x_dtype_name):
    # One tensor whose group scales span 2^-40 .. 2^0: by output row (each
    # row's scales within a factor 2 of 2^-40 r / (N - 1)), or independently
    # per group inside every row.  The prefill GEMM runs on FP16 operands with
    # a power-of-two shift per output row, so rows of any relative magnitude
    # keep every bit; inside a row only groups 2^26 below its largest may lose
    # bits, a negligible share of that row's output.  GEMV rows (1, 3) and
    # GEMM rows (64) must all stay within 1e-5 of the binary64 product.
    n, k = 384, 2048
    G = k // 32
    rng = np.random.default_rng([40, layout == "by_row"])
    q = rng.integers(-7, 8, size=(n, k), dtype=np.int8)
    if layout == "by_row":
        ex = (-40.0 * np.arange(n) / (n - 1))[:, None] - rng.uniform(0, 1, (n, G))
    else:
        ex = rng.uniform(-40, 0, (n, G))
    scales = syn.bf16_rne(np.exp2(ex).astype(np.float32))
    lin = g4.W4Linear(syn.pack_w4(q), scales)
    w = dense(q, scales)
    xd = g4.BF16 if x_dtype_name == "bf16" else g4.F32
    for rows in (1, 3, 64):
        bits, x = syn.activations(41 + rows, rows, k)
        y = run_linear(g4, lin, bits, x, rows, xd)
        assert rel_l2_rows(y, x.astype(np.float64) @ w.T) < 1e-5, (layout, rows)


def test_recording_survives_scratch_growth(g4):
    # A GEMM-path linear recorded into a command buffer holds the library's
    # scratch address.  A later, larger eager call grows the scratch; the old
    # block must not be handed out again while the recording exists, so a
    # replay still computes the recorded call and touches no newer buffer.
    n, k, rows, big = 256, 2048, 16, 16384
    packed, scales, _ = syn.w4_weights(31, n, k)
    lin = g4.W4Linear(packed, scales)
    _, x = syn.activations(31, rows, k)
    xb = g4.Buffer.from_array(x)
    y_ref, y_rec = g4.Buffer(rows * n * 4), g4.Buffer(rows * n * 4)
    lin.linear(xb.ptr, g4.F32, rows, y_ref.ptr, g4.F32)
    with g4.Encoder() as enc:
        lin.linear(xb.ptr, g4.F32, rows, y_rec.ptr, g4.F32)
    cb = enc.cmdbuf
    xbig = g4.Buffer(big * k * 4)
    xbig.upload(np.tile(x, (big // rows, 1)))
    ybig = g4.Buffer(big * n * 4)
    lin.linear(xbig.ptr, g4.F32, big, ybig.ptr, g4.F32)  # grows the scratch
    pattern = np.full(1 << 20, 0x5A5A5A5A, np.uint32)
    probes = []
    for size in (1 << 16, 1 << 20, 1 << 22, 1 << 24, 1 << 25):
        b = g4.Buffer(size)
        b.upload(np.resize(pattern, size // 4))
        probes.append(b)
    for _ in range(3):
        cb.submit()
    got = y_rec.download(np.float32)
    assert np.array_equal(got.view(np.uint32), y_ref.download(np.float32).view(np.uint32))
    for b in probes:
        assert np.all(b.download(np.uint32) == 0x5A5A5A5A)
    # the large call tiles differently; its rows agree to FP32 rounding
    ybig_rows = ybig.download(np.float32).reshape(big, n)[:rows].astype(np.float64)
    assert rel_l2_rows(ybig_rows, y_ref.download(np.float32).reshape(rows, n).astype(np.float64)) < 1e-5
    cb.free()


def test_errors_are_reported_not_faulted(g4):
    packed, scales, _ = syn.w4_weights(1, 256, 512)
    lin = g4.W4Linear(packed, scales)
    x = g4.Buffer(512 * 4)
    y_small = g4.Buffer(255 * 4)
    with pytest.raises(g4.G4Error) as e:
        lin.linear(x.ptr, g4.F32, 1, y_small.ptr, g4.F32)
    assert e.value.code == g4.G4_E_RANGE
    with pytest.raises(g4.G4Error) as e:
        lin.linear(x.ptr, g4.F32, 2, g4.Buffer(512 * 4).ptr, g4.F32)  # x too short for 2 rows
    assert e.value.code == g4.G4_E_RANGE
    with pytest.raises(g4.G4Error) as e:
        lin.linear(x.ptr, 7, 1, y_small.ptr, g4.F32)
    assert e.value.code == g4.G4_E_ARG
    with pytest.raises(g4.G4Error) as e:
        g4.W4Linear(np.zeros((4, 5), np.uint32), np.zeros((4, 1), np.uint16))  # K=40
    assert "divisible by groupSize" in str(e.value)
    with pytest.raises(g4.G4Error) as e:
        lin.dequant(200, 100, g4.Buffer(100 * 512 * 4).ptr)
    assert e.value.code == g4.G4_E_RANGE


# Weights sharing one input, as q/k/v and gate/up do (and ragged and generic-plan shapes).
MULTI_SHAPES = {
    "qkv_sliding": ((2048, 1536), (256, 1536), (256, 1536)),
    "gate_up": ((6144, 1536), (6144, 1536)),
    "ragged_k2048": ((100, 2048), (36, 2048), (1536, 2048)),
    "ragged_k256": ((260, 256), (12, 256)),
}


@pytest.mark.parametrize("x_dtype_name", ["bf16", "f32"])
@pytest.mark.parametrize("name", sorted(MULTI_SHAPES))
def test_linear_multi_matches_single_launches(g4, oracle, name, x_dtype_name):
    shapes = MULTI_SHAPES[name]
    k = shapes[0][1]
    x_dtype = g4.BF16 if x_dtype_name == "bf16" else g4.F32
    x_bits, x = syn.activations(7, 1, k)
    lins, refs = [], []
    for i, (n, _) in enumerate(shapes):
        packed, scales, _ = syn.w4_weights(300 + i, n, k)
        lins.append(g4.W4Linear(packed, scales))
        refs.append(np.asarray(oracle.w4_linear(x, packed, scales), np.float64).reshape(1, n))
    xb = g4.Buffer.from_array(x_bits if x_dtype == g4.BF16 else x.astype(np.float32))
    for y_dtype in (g4.F32, g4.BF16):
        ye, dt = (4, np.float32) if y_dtype == g4.F32 else (2, np.uint16)
        ys = [g4.Buffer(lin.out_dim * ye) for lin in lins]
        g4.W4Linear.linear_multi(lins, xb.ptr, x_dtype, 1, [y.ptr for y in ys], y_dtype)
        for lin, y, ref in zip(lins, ys, refs):
            got = y.download(dt)
            single = g4.Buffer(lin.out_dim * ye)
            lin.linear(xb.ptr, x_dtype, 1, single.ptr, y_dtype)
            # every row runs the single-weight kernel body: identical bits
            assert np.array_equal(got, single.download(dt))
            if y_dtype == g4.F32:
                assert rel_l2_rows(got.reshape(1, -1), ref) <= TOL


@pytest.mark.parametrize("rows", [3, 64])
def test_linear_multi_several_rows(g4, oracle, rows):
    k = 1536
    x_bits, x = syn.activations(8, rows, k)
    xb = g4.Buffer.from_array(x_bits)
    lins, refs = [], []
    for i, n in enumerate((512, 96)):
        packed, scales, _ = syn.w4_weights(310 + i, n, k)
        lins.append(g4.W4Linear(packed, scales))
        refs.append(np.asarray(oracle.w4_linear(x, packed, scales), np.float64).reshape(rows, n))
    ys = [g4.Buffer(rows * lin.out_dim * 4) for lin in lins]
    g4.W4Linear.linear_multi(lins, xb.ptr, g4.BF16, rows, [y.ptr for y in ys], g4.F32)
    for lin, y, ref in zip(lins, ys, refs):
        got = y.download(np.float32).reshape(rows, lin.out_dim)
        assert np.array_equal(got, run_linear(g4, lin, x_bits, x, rows, g4.BF16))
        assert rel_l2_rows(got, ref) <= TOL


@pytest.mark.parametrize("shapes", [((2048, 1536), (256, 1536), (256, 1536)),
                                    ((6144, 1536), (6144, 1536)),
                                    ((1000, 2048), (70, 2048))])
def test_linear_multi_prefill_gemm(g4, shapes):
    # 512 FP32 rows, as the model's prefill: one x pre-pass and one GEMM launch
    # over the weights' tiles; each output against the binary64 product, and
    # the same weight run alone (its own plan: tile, K split) agrees within the
    # same bound.
    rows, k = 512, shapes[0][1]
    x = np.random.default_rng(31).standard_normal((rows, k)).astype(np.float32)
    xb = g4.Buffer.from_array(x)
    lins, refs = [], []
    for i, (n, _) in enumerate(shapes):
        packed, scales, q = syn.w4_weights(330 + i, n, k)
        lins.append(g4.W4Linear(packed, scales))
        refs.append(x.astype(np.float64) @ dense(q, scales).T)
    ys = [g4.Buffer(rows * lin.out_dim * 4) for lin in lins]
    g4.W4Linear.linear_multi(lins, xb.ptr, g4.F32, rows, [y.ptr for y in ys], g4.F32)
    for lin, y, ref in zip(lins, ys, refs):
        got = y.download(np.float32).reshape(rows, lin.out_dim)
        assert rel_l2_rows(got, ref) <= 1e-5
    if shapes[0][0] == 2048:
        alone = run_linear(g4, lins[0], None, x, rows, g4.F32)
        assert rel_l2_rows(ys[0].download(np.float32).reshape(rows, 2048), alone) <= 1e-5


@pytest.mark.parametrize("rows", [5, 200, 512])
def test_linear_multi_gemm_bf16_out_ragged(g4, rows):
    # BF16 x and BF16 y through the several-weight GEMM: ragged widths (not
    # tile multiples), a joint grid that fills the GPU (512 rows) or not (5,
    # 200 rows: each weight alone); every output is the RNE of the FP32 one.
    k = 1024
    x_bits, x = syn.activations(41, rows, k)
    xb = g4.Buffer.from_array(x_bits)
    lins, refs = [], []
    for i, n in enumerate((1000, 100, 36)):
        packed, scales, q = syn.w4_weights(340 + i, n, k)
        lins.append(g4.W4Linear(packed, scales))
        refs.append(x.astype(np.float64) @ dense(q, scales).T)
    y32 = [g4.Buffer(rows * lin.out_dim * 4) for lin in lins]
    y16 = [g4.Buffer(rows * lin.out_dim * 2) for lin in lins]
    g4.W4Linear.linear_multi(lins, xb.ptr, g4.BF16, rows, [y.ptr for y in y32], g4.F32)
    g4.W4Linear.linear_multi(lins, xb.ptr, g4.BF16, rows, [y.ptr for y in y16], g4.BF16)
    for lin, a, b, ref in zip(lins, y32, y16, refs):
        got = a.download(np.float32).reshape(rows, lin.out_dim)
        assert rel_l2_rows(got, ref) <= 1e-4
        assert np.array_equal(b.download(np.uint16).reshape(rows, lin.out_dim),
                              syn.bf16_rne(got).reshape(rows, lin.out_dim))


def test_linear_multi_errors(g4):
    a = g4.W4Linear(*syn.w4_weights(320, 64, 512)[:2])
    b = g4.W4Linear(*syn.w4_weights(321, 64, 256)[:2])
    x = g4.Buffer(512 * 4)
    ys = [g4.Buffer(64 * 4) for _ in range(4)]
    with pytest.raises(g4.G4Error) as e:  # different input dims
        g4.W4Linear.linear_multi([a, b], x.ptr, g4.F32, 1, [y.ptr for y in ys[:2]])
    assert e.value.code == g4.G4_E_ARG
    with pytest.raises(g4.G4Error) as e:  # more than three weights
        g4.W4Linear.linear_multi([a] * 4, x.ptr, g4.F32, 1, [y.ptr for y in ys])
    assert e.value.code == g4.G4_E_ARG
    short = g4.Buffer(63 * 4)
    with pytest.raises(g4.G4Error) as e:  # second output too short
        g4.W4Linear.linear_multi([a, a], x.ptr, g4.F32, 1, [ys[0].ptr, short.ptr])
    assert e.value.code == g4.G4_E_RANGE


@pytest.mark.parametrize("rows,n,k", [(2048, 6144, 1536), (512, 1536, 6144), (1, 6144, 1536)])
def test_weight_without_gemm_tiles(g4, rows, n, k):
    # g4_w4_load_opts(G4_W4_NO_GEMM_TILES): a decode-only weight holds no tile
    # copy (about half the device bytes); a prefill call on it takes the
    # row-major MFMA kernel, the decode GEMV is unchanged (identical bits)
    packed, scales, q = syn.w4_weights(61, n, k)
    a = g4.W4Linear(packed, scales)
    b = g4.W4Linear(packed, scales, gemm_tiles=False)
    assert b.info()["device_bytes"] < 0.6 * a.info()["device_bytes"]
    x = np.random.default_rng(61).standard_normal((rows, k)).astype(np.float32)
    xb = g4.Buffer.from_array(x)
    ya = run_linear(g4, a, None, x, rows, g4.F32)
    yb = run_linear(g4, b, None, x, rows, g4.F32)
    ref = x.astype(np.float64) @ dense(q, scales).T
    assert rel_l2_rows(yb, ref) <= 1e-5
    if rows == 1:
        assert np.array_equal(ya, yb)
    h = ctypes.c_void_p()
    with pytest.raises(g4.G4Error) as e:  # an unknown flag
        g4.check(g4.lib().g4_w4_load_opts(packed.ctypes.data, scales.ctypes.data, n, k, 32, 8,
                                          ctypes.byref(h)))
    assert e.value.code == g4.G4_E_ARG and not h.value


@pytest.mark.parametrize("n,k,xd", [(6144, 1536, "bf16"), (2048, 1536, "f32"), (1536, 2048, "bf16")])
def test_gemv_stamps_same_output_and_ordered_stamps(g4, n, k, xd):
    # g4_w4_gemv_stamps runs the row-split decode GEMV with clock stamps: its
    # output must be the plain launch's, bit for bit, and every wave's five
    # stamps must be set and in order (start <= staged <= barrier <= weights
    # landed <= store issued)
    packed, scales, _ = syn.w4_weights(61, n, k, full_range=True)
    lin = g4.W4Linear(packed, scales, gemm_tiles=False)
    x_bits, x_f32 = syn.activations(62, 1, k)
    dt = g4.BF16 if xd == "bf16" else g4.F32
    xb = g4.Buffer.from_array(x_bits if xd == "bf16" else x_f32.astype(np.float32))
    y0, y1 = g4.Buffer(n * 4), g4.Buffer(n * 4)
    lin.linear(xb.ptr, dt, 1, y0.ptr, g4.F32)
    waves = lin.stamp_waves()
    assert n <= 4 * waves < n + 16  # 4 rows per wave, blocks of 2 or 4 waves
    st = g4.Buffer(waves * 5 * 8)
    assert lin.gemv_stamps(xb.ptr, dt, y1.ptr, st.ptr) == waves
    g4.sync()
    assert np.array_equal(y0.download(np.uint32), y1.download(np.uint32))
    s = st.download(np.uint64).reshape(waves, 5).astype(np.int64)
    assert (s > 0).all()
    assert (np.diff(s, axis=1) >= 0).all()
    # one launch spans microseconds, not seconds (100 MHz clock)
    assert s[:, 4].max() - s[:, 0].min() < 100_000
    lin.free()


def test_gemv_stamps_refuses_other_widths(g4):
    packed, scales, _ = syn.w4_weights(63, 256, 256)
    lin = g4.W4Linear(packed, scales, gemm_tiles=False)
    with pytest.raises(g4.G4Error) as e:
        lin.stamp_waves()
    assert "row split" in str(e.value)
    lin.free()


@pytest.mark.parametrize("k", [4096, 6144, 12288])
@pytest.mark.parametrize("n", [1, 7, 1001])
def test_wide_rows_ragged_out_dim(g4, oracle, n, k):
    # the 64-lane row split (in_dim 4096, 6144, and 12288 with BF16 x) with
    # out_dim not a multiple of its 8-row blocks: the last block's rows past
    # out_dim re-read row out_dim - 1 and store nothing; both x dtypes, and
    # the several-weight launch gives the single launch's bits
    packed, scales, q = syn.w4_weights(400 + n, n, k, full_range=True)
    p2, s2, _ = syn.w4_weights(401 + n, 9, k)
    lin, lin2 = g4.W4Linear(packed, scales, gemm_tiles=False), g4.W4Linear(p2, s2, gemm_tiles=False)
    x_bits, x = syn.activations(402, 1, k)
    ref = np.asarray(oracle.w4_linear(x, packed, scales), np.float64).reshape(1, n)
    for dt in (g4.BF16, g4.F32):
        xb = g4.Buffer.from_array(x_bits if dt == g4.BF16 else x.astype(np.float32))
        guard = g4.Buffer((n + 64) * 4)
        guard.upload(np.full(n + 64, 7.0, np.float32))
        lin.linear(xb.ptr, dt, 1, guard.ptr, g4.F32)
        out = guard.download(np.float32)
        assert (out[n:] == 7.0).all()  # nothing written past out_dim
        assert rel_l2_rows(out[:n].reshape(1, n), ref) <= TOL
        ya, yb = g4.Buffer(n * 4), g4.Buffer(9 * 4)
        g4.W4Linear.linear_multi([lin, lin2], xb.ptr, dt, 1, [ya.ptr, yb.ptr], g4.F32)
        assert np.array_equal(ya.download(np.uint32), out[:n].view(np.uint32))
    lin.free()
    lin2.free()
