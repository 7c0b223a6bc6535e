"""Pins the CPU oracle (oracle/g4_oracle.c) before anything is compared to it.

The reference has no tests, golden vectors or fixtures for this path, so each
oracle function is pinned by what the mathematics or an independent library
fixes: exhaustive tables, literal known answers derived from the reference's
documented formats, numpy/torch routines, and the reference manifest's shard
table (tests/golden/ple_w4_layout.json).  Each check is chosen so that a
plausible slip (nibble order, sign convention, transposed operand, wrong
block size, off-by-one offsets) fails it.
"""
import json
import math
import os

import numpy as np
import pytest

import synthetic as syn

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ---- nibble decoding --------------------------------------------------------

def test_w4_nibble_table(oracle):
    # compressed-tensors offset binary: stored 0..15 -> logical -8..7
    # (official-w4a16.js:15-19 comment)
    expected = [-8, -7, -6, -5, -4, -3, -2, -1, 0, 1, 2, 3, 4, 5, 6, 7]
    assert [oracle.w4_nibble(n) for n in range(16)] == expected
    # only the low nibble matters
    assert [oracle.w4_nibble(n | 0xF0) for n in range(16)] == expected


def test_ple_nibble_table(oracle):
    # two's-complement nibble (manifest signed_encoding "two_complement_nibble")
    expected = [0, 1, 2, 3, 4, 5, 6, 7, -8, -7, -6, -5, -4, -3, -2, -1]
    assert [oracle.ple_nibble(n) for n in range(16)] == expected
    # independent derivation: sign-extend the nibble through an int8 shift
    for n in range(16):
        assert oracle.ple_nibble(n) == int(np.int8(np.uint8(n << 4).view(np.int8)) >> 4)


# ---- bf16 conversions --------------------------------------------------------

def test_bf16_to_f32_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint32)
    want = (bits << 16).view(np.float32)
    got = oracle.bf16_to_f32_array(bits.astype(np.uint16))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    finite = np.isfinite(want)
    assert all(oracle.bf16_to_f32(int(b)) == float(w) for b, w in
               zip(bits[finite][::97], want[finite][::97]))


def test_f32_to_bf16_known_answers(oracle):
    cases = {
        0x3F800000: 0x3F80,  # 1.0
        0x3F808000: 0x3F80,  # halfway, even neighbour below
        0x3F818000: 0x3F82,  # halfway, even neighbour above
        0x3F808001: 0x3F81,  # just above halfway
        0x3F807FFF: 0x3F80,  # just below halfway
        0x7F7FFFFF: 0x7F80,  # max finite rounds to +inf
        0x80000000: 0x8000,  # -0
        0x00000001: 0x0000,  # smallest subnormal rounds to +0
    }
    for f_bits, b in cases.items():
        v = np.array([f_bits], dtype=np.uint32).view(np.float32)[0]
        assert oracle.f32_to_bf16(float(v)) == b, hex(f_bits)


def test_f32_to_bf16_matches_torch(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(7)
    v = np.concatenate([rng.standard_normal(3000).astype(np.float32),
                        (rng.standard_normal(1000) * 1e30).astype(np.float32),
                        (rng.standard_normal(1000) * 1e-30).astype(np.float32)])
    want = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = oracle.f32_to_bf16_array(v)
    assert np.array_equal(got, want)
    assert np.array_equal(syn.bf16_rne(v), want)


# ---- W4 dequant ----------------------------------------------------------------

def test_w4_dequant_known_answer(oracle):
    # One row, K = 32 (one group, four words).  Word 0x76543210 holds nibbles
    # 0..7 low-first -> logical -8..-1; 0xFEDCBA98 holds 8..15 -> 0..7.
    packed = np.array([[0x76543210, 0xFEDCBA98, 0x00000000, 0xFFFFFFFF]], dtype=np.uint32)
    scale = np.array([[2.0]], dtype=np.float32)
    rc, w = oracle.w4_dequant_rows(packed, scale, 1, 32, 0, 1)
    assert rc == 0
    want = [2.0 * v for v in list(range(-8, 0)) + list(range(0, 8)) + [-8] * 8 + [7] * 8]
    assert w.reshape(-1).tolist() == want
    # the synthetic packer agrees with the layout
    assert syn.pack_w4(np.array([list(range(-8, 0))]))[0, 0] == 0x76543210


def test_w4_dequant_validation(oracle):
    p = np.zeros((4, 4), dtype=np.uint32)
    s = np.ones((4, 1), dtype=np.float32)
    assert oracle.w4_dequant_rows(p, s, 4, 36, 0, 1)[0] == 1  # inDim % 8
    assert oracle.w4_dequant_rows(p, s, 4, 32, 0, 1, group=24)[0] == 2  # inDim % groupSize
    assert oracle.w4_dequant_rows(p[:3], s, 4, 32, 0, 1)[0] == 3  # packed length
    assert oracle.w4_dequant_rows(p, s[:3], 4, 32, 0, 1)[0] == 4  # scale length
    assert oracle.w4_dequant_rows(p, s, 4, 32, 0, 4)[0] == 0


def test_w4_dequant_against_known_q(oracle):
    # q is drawn first, then packed: dequant must return q * s exactly.
    packed, scales, q = syn.w4_weights(3, 40, 256)
    s = syn.bf16_to_f32(scales).reshape(40, 8)
    rc, w = oracle.w4_dequant_rows(packed, s, 40, 256, 5, 30)
    assert rc == 0
    want = q[5:35].astype(np.float32) * np.repeat(s[5:35], 32, axis=1)
    assert np.array_equal(w, want)
    assert np.array_equal(syn.unpack_w4(packed), q)


# ---- W4 linear ------------------------------------------------------------------

def test_w4_linear_one_hot_is_a_column(oracle):
    packed, scales, q = syn.w4_weights(11, 96, 128)
    s = syn.bf16_to_f32(scales).reshape(96, 4)
    for k in (0, 31, 32, 77, 127):
        x = np.zeros((1, 128), dtype=np.float32)
        x[0, k] = 1.0
        y = oracle.w4_linear(x, packed, scales)
        assert np.array_equal(y[0], q[:, k].astype(np.float32) * s[:, k // 32])


def test_w4_linear_integer_exact(oracle):
    # scale 1.0 (bf16 0x3F80) and small integer x: every partial sum is an
    # integer far below 2^24, so FP32 must equal exact integer arithmetic.
    rng = np.random.default_rng(5)
    q = rng.integers(-8, 8, size=(70, 192))
    packed = syn.pack_w4(q)
    scales = np.full((70, 6), 0x3F80, dtype=np.uint16)
    x = rng.integers(-4, 5, size=(3, 192))
    y = oracle.w4_linear(x.astype(np.float32), packed, scales)
    assert np.array_equal(y, (x @ q.T).astype(np.float32))


def test_w4_linear_tfjs_block_rounding(oracle):
    # tfjs-backend-cpu adds a binary64 partial sum into the float32 result
    # once per 48-wide k block.  Block 0 sums to 2^24 + 1, which float32
    # rounds to 2^24 (ties to even); block 1 adds 1 and rounds back to 2^24.
    # A single binary64 accumulator would give 2^24 + 2 (exact in float32),
    # and a 64-wide block would too.
    K = 96
    q = np.zeros((1, K), dtype=np.int64)
    q[0, 0], q[0, 1], q[0, 48] = 2, 1, 1
    packed = syn.pack_w4(q)
    scales = np.full((1, K // 32), 0x3F80, dtype=np.uint16)
    x = np.zeros((1, K), dtype=np.float32)
    x[0, 0], x[0, 1], x[0, 48] = 2.0 ** 23, 1.0, 1.0
    assert oracle.w4_linear(x, packed, scales)[0, 0] == np.float32(2.0 ** 24)
    assert oracle.w4_linear_f64(x, packed, scales)[0, 0] == 2.0 ** 24 + 2


def test_w4_linear_chunking_does_not_change_values(oracle):
    packed, scales, _ = syn.w4_weights(9, 300, 256)
    _, x = syn.activations(9, 2, 256)
    a = oracle.w4_linear(x, packed, scales, chunk=256)
    b = oracle.w4_linear(x, packed, scales, chunk=37)
    assert np.array_equal(a, b)


def test_w4_linear_threads_bit_identical(oracle):
    # the all-core CPU leg: chunks over threads, each element's sequence
    # unchanged, so the bits equal the single-threaded oracle's
    packed, scales, _ = syn.w4_weights(13, 1000, 1536)
    _, x = syn.activations(13, 3, 1536)
    a = oracle.w4_linear(x, packed, scales)
    for t in (1, 3, 0):
        b = oracle.w4_linear_mt(x, packed, scales, threads=t)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _run_js_leg(tmp_path, x, packed, scales):
    import shutil
    import subprocess
    node = shutil.which("node")
    if node is None:
        pytest.skip("node is not installed")
    m, k = x.shape
    n = packed.shape[0]
    paths = [str(tmp_path / f) for f in ("p.bin", "s.bin", "x.bin", "y.bin")]
    np.ascontiguousarray(packed).view(np.int32).tofile(paths[0])
    np.ascontiguousarray(scales).view(np.uint16).tofile(paths[1])
    np.ascontiguousarray(x, dtype=np.float32).tofile(paths[2])
    script = os.path.join(os.path.dirname(GOLDEN), "..", "oracle", "w4_linear_cpu.js")
    p = subprocess.run([node, script, str(m), str(k), str(n)] + paths + ["0"],
                       stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=120)
    assert p.returncode == 0, p.stderr
    assert json.loads(p.stdout.strip().splitlines()[-1])["calls"] >= 1
    return np.fromfile(paths[3], dtype=np.float32).reshape(m, n)


def test_js_cpu_leg_matches_c_oracle(oracle, tmp_path):
    # the single-threaded JavaScript leg restates the same dequant and
    # 48-blocked matMul: identical bits, ragged chunk and k-block tails included
    packed, scales, _ = syn.w4_weights(14, 300, 1568)
    _, x = syn.activations(14, 2, 1568)
    got = _run_js_leg(tmp_path, x, packed, scales)
    want = oracle.w4_linear(x, packed, scales)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_js_cpu_leg_block_rounding(oracle, tmp_path):
    # the 2^24 known answer of test_w4_linear_tfjs_block_rounding, in JS
    K = 96
    q = np.zeros((1, K), dtype=np.int64)
    q[0, 0], q[0, 1], q[0, 48] = 2, 1, 1
    packed = syn.pack_w4(q)
    scales = np.full((1, K // 32), 0x3F80, dtype=np.uint16)
    x = np.zeros((1, K), dtype=np.float32)
    x[0, 0], x[0, 1], x[0, 48] = 2.0 ** 23, 1.0, 1.0
    assert _run_js_leg(tmp_path, x, packed, scales)[0, 0] == np.float32(2.0 ** 24)


def test_js_ple_rows_leg_matches_c_oracle(oracle, tmp_path):
    # the JS restatement of readRows' per-row loop (the CPU baseline beside
    # the PLE gather) on rows holding every nibble value, nibble 8 (-8) in
    # every group: identical bits to the C oracle's gather
    import shutil
    import subprocess
    node = shutil.which("node")
    if node is None:
        pytest.skip("node is not installed")
    vocab, width, rps = 9000, 512, 4096
    table = np.concatenate(syn.ple_table(3, vocab, width, rps, threads=2, full_range=True))
    ids = np.array([0, 4095, 4096, 8999, 17, 17], dtype=np.int32)
    recs = []
    for t in ids:
        po, so = oracle.ple_row_offsets(vocab, width, rps, int(t) // rps, int(t) % rps)
        recs += [table[po:po + width // 2], table[so:so + width // 16]]
    rp, op = str(tmp_path / "rows.bin"), str(tmp_path / "out.bin")
    np.concatenate(recs).tofile(rp)
    script = os.path.join(os.path.dirname(GOLDEN), "..", "oracle", "ple_rows_cpu.js")
    p = subprocess.run([node, script, str(ids.size), str(width), rp, op, "0"],
                       stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=120)
    assert p.returncode == 0, p.stderr
    got = np.fromfile(op, dtype=np.float32).reshape(ids.size, width)
    want = oracle.ple_gather(table, vocab, width, rps, ids)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_ple_gather_mt_matches_single_thread(oracle):
    vocab, width, rps = 9000, 512, 4096
    table = np.concatenate(syn.ple_table(4, vocab, width, rps, threads=2, full_range=True))
    ids = syn.token_ids(5, 700, vocab)
    want = oracle.ple_gather(table, vocab, width, rps, ids)
    for t in (1, 3, 0):
        got = oracle.ple_gather_mt(table, vocab, width, rps, ids, threads=t)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    with pytest.raises(IndexError):
        oracle.ple_gather_mt(table, vocab, width, rps, np.array([1, vocab], np.int32))


def test_w4_linear_f64_matches_numpy(oracle):
    packed, scales, q = syn.w4_weights(21, 512, 1536)
    _, x = syn.activations(21, 2, 1536)
    w = q.astype(np.float64) * np.repeat(syn.bf16_to_f32(scales).astype(np.float64), 32, axis=1)
    want = x.astype(np.float64) @ w.T
    got = oracle.w4_linear_f64(x, packed, scales)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
    f32 = oracle.w4_linear(x, packed, scales)
    rel = np.linalg.norm(f32 - want, axis=1) / np.linalg.norm(want, axis=1)
    assert rel.max() < 1e-6


def test_w4_linear_config0_shape(oracle):
    # M=1, K=1536, N=6144: the oracle itself sits far inside the 1e-3 budget.
    packed, scales, q = syn.w4_weights(1, 6144, 1536)
    _, x = syn.activations(1, 1, 1536)
    y = oracle.w4_linear(x, packed, scales)
    w = q.astype(np.float64) * np.repeat(syn.bf16_to_f32(scales).astype(np.float64), 32, axis=1)
    ref = x.astype(np.float64) @ w.T
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 1e-6


# ---- PLE --------------------------------------------------------------------------

def test_ple_dequant_every_byte(oracle):
    # Element 2b is the low nibble of byte b, element 2b+1 the high nibble.
    row = np.arange(256, dtype=np.uint8).repeat(1)  # 256 bytes = 512 elements
    scales = np.full(16, 0x3F80, dtype=np.uint16)  # 1.0
    out = oracle.ple_dequant_row(row, scales, 512)
    lo = (row.astype(np.uint8) << 4).view(np.int8) >> 4
    hi = row.view(np.int8) >> 4
    assert np.array_equal(out[0::2], lo.astype(np.float32))
    assert np.array_equal(out[1::2], hi.astype(np.float32))


def test_ple_dequant_scale_per_group(oracle):
    row = np.full(64, 0x11, dtype=np.uint8)  # every element +1
    scales = syn.bf16_rne(np.array([0.5, -3.0, 0.125, 96.0], dtype=np.float32))
    out = oracle.ple_dequant_row(row, scales, 128)
    assert np.array_equal(out, np.repeat(np.array([0.5, -3.0, 0.125, 96.0], np.float32), 32))


def _layout():
    with open(os.path.join(GOLDEN, "ple_w4_layout.json")) as f:
        return json.load(f)


def test_ple_layout_matches_reference_manifest(oracle):
    m = _layout()
    vocab, width = m["vocab_size"], m["width"]
    rps = m["layout"]["rows_per_shard"]
    assert m["layout"]["packed_row_bytes"] == width // 2
    assert m["layout"]["scale_row_bytes"] == (width // 32) * 2
    assert m["total_bytes"] == m["packed_bytes"] + m["scale_bytes"]
    base = 0
    for s in m["shards"]:
        rows = s["row_end"] - s["row_start"]
        po, so = oracle.ple_row_offsets(vocab, width, rps, s["index"], 0)
        assert po - base == s["packed_offset"]
        assert so - base == s["scales_offset"]
        assert s["bytes"] == s["packed_bytes"] + s["scales_bytes"]
        po_last, so_last = oracle.ple_row_offsets(vocab, width, rps, s["index"], rows - 1)
        assert po_last - base + width // 2 == s["packed_bytes"]
        assert so_last - base + (width // 32) * 2 == s["bytes"]
        assert oracle.ple_locate(s["row_start"], vocab, rps) == (s["index"], 0)
        assert oracle.ple_locate(s["row_end"] - 1, vocab, rps) == (s["index"], rows - 1)
        base += s["bytes"]
    assert base == m["total_bytes"]
    for tid in m["verification_rows"]:
        shard, local = oracle.ple_locate(tid, vocab, rps)
        assert m["shards"][shard]["row_start"] + local == tid
    assert oracle.ple_locate(-1, vocab, rps) is None
    assert oracle.ple_locate(vocab, vocab, rps) is None


def test_ple_gather_partial_last_shard(oracle):
    # vocab not a multiple of rows_per_shard: the last shard is short and its
    # scales block starts earlier (rows * packed_row).
    vocab, width, rps = 700, 256, 256
    shards, qs, ss = [], [], []
    for si in range(3):
        rows = min(rps, vocab - si * rps)
        rng = np.random.default_rng(si)
        q = rng.integers(-7, 8, size=(rows, width))
        s = syn.bf16_rne(np.abs(rng.standard_normal((rows, width // 32)).astype(np.float32)))
        shards.append(np.concatenate([syn.pack_ple(q).reshape(-1),
                                      s.astype("<u2").view(np.uint8).reshape(-1)]))
        qs.append(q)
        ss.append(s)
    table = np.concatenate(shards)
    q_all = np.concatenate(qs)
    s_all = syn.bf16_to_f32(np.concatenate(ss)).reshape(vocab, width // 32)
    ids = np.array([0, 255, 256, 511, 512, 699, 699, 3, 600], dtype=np.int32)
    out = oracle.ple_gather(table, vocab, width, rps, ids)
    want = q_all[ids].astype(np.float32) * np.repeat(s_all[ids], 32, axis=1)
    assert np.array_equal(out, want)
    with pytest.raises(IndexError):
        oracle.ple_gather(table, vocab, width, rps, np.array([1, 700], dtype=np.int32))


def test_ple_quantizer_properties(oracle):
    rng = np.random.default_rng(17)
    x = syn.bf16_to_f32(syn.bf16_rne(rng.standard_normal((6, 256)).astype(np.float32) * 0.3))
    x = x.reshape(6, 256).copy()
    x[2, :32] = 0.0  # an all-zero group
    packed, scales = oracle.ple_quantize_rows(x)
    s = syn.bf16_to_f32(scales).reshape(6, 8)
    # scale = bf16(maxabs / 7), 1.0 for the zero group
    maxabs = np.abs(x.reshape(6, 8, 32)).max(axis=2)
    want_s = np.where(maxabs == 0, np.float32(1.0), maxabs / np.float32(7)).astype(np.float32)
    assert np.array_equal(scales, syn.bf16_rne(want_s))
    # decode through the independent byte decoder and check the error bound
    deq = np.stack([oracle.ple_dequant_row(packed[i], scales[i], 256) for i in range(6)])
    q = deq / np.repeat(s, 32, axis=1)
    assert np.array_equal(q, np.round(q)) and np.abs(q).max() <= 7
    err = np.abs(deq - x)
    assert np.all(err <= np.repeat(s, 32, axis=1) * 0.5 + np.abs(x) * 2.0 ** -7)


def test_ple_quantizer_divides_by_the_stored_bf16_scale(oracle):
    # tools/build_ple_w4_full.py:54-56 quantizes against the STORED BF16
    # scale.  Every group's FP32 seventh of its maximum differs from its BF16
    # rounding, and most elements lie between the two scales' rounding
    # boundaries, so a divisor of maxabs / 7 in FP32 gives other codes there.
    # The codes must equal the brute-force nearest k * s_bf16 (ties to even),
    # found without division or rint.
    import quantizer_cases as qc
    rows, width = 64, 1024
    _, x, differs = qc.divisor_rows(23, rows, width)
    packed, scales = oracle.ple_quantize_rows(x)
    maxabs = np.abs(x.reshape(rows, width // 32, 32)).max(axis=2)
    assert np.array_equal(scales, syn.bf16_rne((maxabs / np.float32(7)).astype(np.float32)))
    s_stored = syn.bf16_to_f32(scales).reshape(rows, width // 32)
    assert differs.sum() > x.size // 16  # about 13% of the elements
    assert np.array_equal(qc.codes_of(packed), qc.best_codes(x, s_stored))


def test_ple_quantizer_brute_force_codes_on_random_rows(oracle):
    # the same brute-force characterisation on ordinary rows (normal values,
    # zero groups), where the divisor rarely matters
    import quantizer_cases as qc
    rng = np.random.default_rng(29)
    x = syn.bf16_to_f32(syn.bf16_rne(rng.standard_normal((32, 512)).astype(np.float32) * 0.2))
    x = x.reshape(32, 512).copy()
    x[4, 64:96] = 0.0
    packed, scales = oracle.ple_quantize_rows(x)
    s = syn.bf16_to_f32(scales).reshape(32, 16)
    assert np.array_equal(qc.codes_of(packed), qc.best_codes(x, s))


def test_ple_quantizer_rounds_half_to_even(oracle):
    x = np.zeros((1, 32), dtype=np.float32)
    x[0, :5] = [7.0, 2.5, 3.5, -2.5, 0.5]  # maxabs 7 -> scale exactly 1.0
    packed, scales = oracle.ple_quantize_rows(x)
    assert scales[0, 0] == 0x3F80
    out = oracle.ple_dequant_row(packed[0], scales[0], 32)
    assert out[:5].tolist() == [7.0, 2.0, 4.0, -2.0, 0.0]


# ---- head and top-k ------------------------------------------------------------------

def test_bf16_head_matches_float64(oracle):
    rng = np.random.default_rng(4)
    E = syn.bf16_rne(rng.standard_normal((300, 1536)).astype(np.float32) * 0.05)
    x = rng.standard_normal(1536).astype(np.float32)
    got = oracle.bf16_head(x, E.reshape(300, 1536))
    raw = syn.bf16_to_f32(E).reshape(300, 1536).astype(np.float64) @ x.astype(np.float64)
    want = 30.0 * np.tanh(raw / 30.0)
    assert np.allclose(got, want, rtol=2e-5, atol=2e-5)
    raw_only = oracle.bf16_head(x, E.reshape(300, 1536), softcap=0.0)
    assert np.allclose(raw_only, raw, rtol=2e-5, atol=2e-5)


def test_bf16_head_one_hot_softcap(oracle):
    E = syn.bf16_rne(np.array([[0.0, 45.0], [-90.0, 1.0], [3.0, 0.0]], dtype=np.float32))
    out = oracle.bf16_head(np.array([1.0, 0.0], np.float32), E)
    assert np.allclose(out, [0.0, 30 * math.tanh(-3.0), 30 * math.tanh(0.1)], rtol=1e-6, atol=0)


def test_topk_matches_lexsort(oracle):
    rng = np.random.default_rng(8)
    for trial in range(20):
        n = int(rng.integers(1, 400))
        v = rng.integers(-5, 6, size=n).astype(np.float32)  # many ties
        v[rng.random(n) < 0.05] = np.nan
        v[rng.random(n) < 0.03] = np.inf
        k = int(rng.integers(1, 15))
        ids, vals = oracle.topk(v, k)
        fin = np.where(np.isfinite(v))[0]
        order = fin[np.lexsort((fin, -v[fin]))][:k]
        assert ids.tolist() == order.tolist()
        assert np.array_equal(vals, v[order])
    assert oracle.topk(np.array([np.nan, np.inf], np.float32), 3)[0].size == 0
