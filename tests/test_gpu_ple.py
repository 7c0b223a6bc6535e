"""GPU parity of the PLE W4 gather-dequant: bit-exact against the oracle.

The full [262144, 8960] table (64 shards, 1.32 GB) is generated once per
session in the builder's shard layout, uploaded shard by shard, and every
gathered row is compared bit for bit with the oracle's readRows restatement;
BF16 rows must equal round-to-nearest-even of the oracle's FP32 rows.
"""
import numpy as np
import pytest

import synthetic as syn

pytestmark = pytest.mark.gpu

VOCAB, WIDTH, RPS = 262144, 8960, 4096


@pytest.fixture(scope="module")
def table(g4):
    shards = syn.ple_table(2024, VOCAB, WIDTH, RPS, threads=16)
    t = g4.PleTable(VOCAB, WIDTH, 32, RPS)
    assert t.num_shards == 64
    for i, s in enumerate(shards):
        assert s.nbytes == t.shard_bytes(i) == 20643840
        t.upload_shard(i, s)
    host = np.concatenate(shards)
    del shards
    yield t, host
    t.free()


def gather(g4, t, ids, dtype):
    out = g4.Buffer(len(ids) * WIDTH * (4 if dtype == g4.F32 else 2))
    t.gather(ids, out.ptr, dtype)
    return out.download(np.float32 if dtype == g4.F32 else np.uint16).reshape(len(ids), WIDTH)


def test_gather_2048_ids_fp32_and_bf16(g4, oracle, table):
    t, host = table
    ids = syn.token_ids(1, 2048, VOCAB)
    ids[:6] = [0, VOCAB - 1, RPS - 1, RPS, 5 * RPS + 17, 0]  # edges and a duplicate
    want = oracle.ple_gather(host, VOCAB, WIDTH, RPS, ids)
    got = gather(g4, t, ids, g4.F32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got16 = gather(g4, t, ids, g4.BF16)
    assert np.array_equal(got16.reshape(-1), oracle.f32_to_bf16_array(want))


def test_gather_single_id(g4, oracle, table):
    t, host = table
    for tid in (0, 1, 123456, VOCAB - 1):
        ids = np.array([tid], dtype=np.int32)
        want = oracle.ple_gather(host, VOCAB, WIDTH, RPS, ids)
        got = gather(g4, t, ids, g4.F32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_gather_values_are_in_the_quantized_range(g4, table):
    t, host = table
    got = gather(g4, t, syn.token_ids(3, 64, VOCAB), g4.F32)
    assert np.isfinite(got).all()
    assert np.abs(got).max() <= 7 * 0.05 * 6  # |q| <= 7, scale = bf16(|N|*0.05)


def test_out_of_range_host_id_throws_before_launch(g4, table):
    t, _ = table
    out = g4.Buffer(3 * WIDTH * 4)
    sentinel = np.full(3 * WIDTH, 7.0, dtype=np.float32)
    out.upload(sentinel)
    for bad in (-1, VOCAB):
        with pytest.raises(g4.G4Error) as e:
            t.gather(np.array([5, bad, 6], dtype=np.int32), out.ptr, g4.F32)
        assert e.value.code == g4.G4_E_RANGE
        assert "PLE token id out of range" in str(e.value)
    assert np.array_equal(out.download(np.float32), sentinel)


def test_device_ids_out_of_range_give_nan_rows(g4, oracle, table):
    t, host = table
    ids = np.array([10, -3, 262143, VOCAB + 5, 77], dtype=np.int32)
    dev = g4.Buffer.from_array(ids)
    out = g4.Buffer(ids.size * WIDTH * 4)
    t.gather_dev(dev.ptr, ids.size, out.ptr, g4.F32)
    got = out.download(np.float32).reshape(ids.size, WIDTH)
    ok = np.array([0, 2, 4])
    want = oracle.ple_gather(host, VOCAB, WIDTH, RPS, ids[ok])
    assert np.array_equal(got[ok].view(np.uint32), want.view(np.uint32))
    assert np.isnan(got[[1, 3]]).all()


@pytest.mark.parametrize("n", [127, 128, 129, 700, 1023, 1024, 1500])
def test_gather_counts_across_kernel_choices(g4, oracle, table, n):
    # 128 ids and more take the one-block-per-row kernel (512 threads for FP32;
    # BF16: 512 below 1024 ids, 128 from there on); 127 the element kernel
    t, host = table
    ids = syn.token_ids(40 + n, n, VOCAB)
    ids[:7] = [0, VOCAB - 1, RPS - 1, RPS, 63 * RPS, 5 * RPS + 17, 0]
    ids[-1] = ids[3]
    want = oracle.ple_gather(host, VOCAB, WIDTH, RPS, ids)
    got = gather(g4, t, ids, g4.F32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got16 = gather(g4, t, ids, g4.BF16)
    assert np.array_equal(got16.reshape(-1), oracle.f32_to_bf16_array(want))


def test_row_kernel_bad_device_ids_and_short_last_shard(g4, oracle):
    # 300 ids (the one-block-per-row kernel) over a table whose last shard is
    # short, with device ids outside [0, vocab) that must give NaN rows
    vocab, rps, width = 9000, 4096, 8960
    shards = syn.ple_table(11, vocab, width, rps, threads=4)
    t = g4.PleTable(vocab, width, 32, rps)
    for i, s in enumerate(shards):
        t.upload_shard(i, s)
    host = np.concatenate(shards)
    ids = syn.token_ids(12, 300, vocab)
    ids[:4] = [8192, 8999, 4095, 0]
    bad = np.array([5, 77, 150, 299])
    ids[bad] = [-1, vocab, -(2 ** 31), 2 ** 31 - 1]
    for dtype in (g4.F32, g4.BF16):
        dev = g4.Buffer.from_array(ids)
        out = g4.Buffer(ids.size * width * (4 if dtype == g4.F32 else 2))
        t.gather_dev(dev.ptr, ids.size, out.ptr, dtype)
        ok = np.setdiff1d(np.arange(ids.size), bad)
        want = oracle.ple_gather(host, vocab, width, rps, ids[ok])
        if dtype == g4.F32:
            got = out.download(np.float32).reshape(ids.size, width)
            assert np.array_equal(got[ok].view(np.uint32), want.view(np.uint32))
            assert np.isnan(got[bad]).all()
        else:
            got = out.download(np.uint16).reshape(ids.size, width)
            assert np.array_equal(got[ok].reshape(-1), oracle.f32_to_bf16_array(want))
            assert (got[bad] == 0x7fc0).all()  # bf16 of the quiet NaN
    t.free()


def test_short_last_shard(g4, oracle):
    # vocab not a multiple of rows_per_shard: the last shard's scales block
    # starts after its own (shorter) packed block.
    vocab, rps, width = 9000, 4096, 8960
    shards = syn.ple_table(7, vocab, width, rps, threads=4)
    t = g4.PleTable(vocab, width, 32, rps)
    assert t.num_shards == 3 and t.shard_bytes(2) == (9000 - 8192) * 5040
    for i, s in enumerate(shards):
        t.upload_shard(i, s)
    host = np.concatenate(shards)
    ids = np.array([8192, 8999, 8500, 4095, 0], dtype=np.int32)
    got = gather(g4, t, ids, g4.F32)
    want = oracle.ple_gather(host, vocab, width, rps, ids)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    with pytest.raises(g4.G4Error):
        t.upload_shard(2, shards[1])  # wrong size for the short shard
    t.free()


# ---- the builder's quantizer on the device ---------------------------------------

def quantizer_rows(seed, rows, width):
    """BF16 rows with the builder's edge cases: all-zero and negative-zero
    groups, groups whose values sit exactly halfway between two steps (ties
    to even), and groups of tiny and huge magnitude."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, width), dtype=np.float32) * np.float32(0.05)
    x[::97, :32] = 0.0
    x[5::101, 32:64] = -0.0
    ties = np.array([7, 0.5, 1.5, 2.5, 3.5, 4.5, 5.5, 6.5, -0.5, -1.5, -2.5, -3.5, -4.5, -5.5,
                     -6.5, -7] * 2, np.float32)
    for j, r in enumerate(range(3, rows, 53)):
        x[r, 64:96] = ties * np.float32(2.0 ** (j % 40 - 20))  # maxabs 7 * 2^k: scale 2^k
    x[7::89, 96:128] *= np.float32(1e-30)
    x[11::83, 128:160] *= np.float32(1e30)
    bits = syn.bf16_rne(x)
    return bits, syn.bf16_to_f32(bits).reshape(rows, width)


def test_quantize_rows_matches_builder_bit_exact(g4, oracle):
    # quantize_batch + one shard's layout (tools/build_ple_w4_full.py:48-60,
    # 130-170) on 4096 rows of the table's width, against the oracle's bytes
    rows = 4096
    bits, x = quantizer_rows(5, rows, WIDTH)
    src = g4.Buffer.from_array(bits)
    shard = g4.Buffer(rows * (WIDTH // 2 + WIDTH // 16))
    g4.ple_quantize_rows(src, rows, WIDTH, shard)
    got = shard.download(np.uint8)
    packed, scales = oracle.ple_quantize_rows(x)
    want = np.concatenate([packed.reshape(-1), scales.astype("<u2").view(np.uint8).reshape(-1)])
    assert got.size == want.size
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, (bad[:8], got[bad[:8]], want[bad[:8]])
    # the tie rows decode to the even neighbours
    deq = oracle.ple_dequant_row(packed[3], scales[3], WIDTH)[64:96] * np.float32(2.0 ** 20)
    assert deq[:8].tolist() == [7.0, 0.0, 2.0, 2.0, 4.0, 4.0, 6.0, 6.0]  # row 3: scale 2^-20


def test_quantize_rows_divides_by_the_stored_scale(g4, oracle):
    # rows whose elements lie between the stored-BF16-scale and FP32-scale
    # rounding boundaries (tools/build_ple_w4_full.py:54-56): the device codes
    # must be the brute-force nearest k * s_bf16 (ties to even), and equal the
    # oracle's bytes
    import quantizer_cases as qc
    rows = 64
    bits, x, differs = qc.divisor_rows(31, rows, WIDTH)
    src = g4.Buffer.from_array(bits)
    shard = g4.Buffer(rows * (WIDTH // 2 + WIDTH // 16))
    g4.ple_quantize_rows(src, rows, WIDTH, shard)
    got = shard.download(np.uint8)
    packed = got[:rows * WIDTH // 2].reshape(rows, WIDTH // 2)
    scales = got[rows * WIDTH // 2:].view("<u2").reshape(rows, WIDTH // 32)
    assert differs.sum() > x.size // 16
    s = syn.bf16_to_f32(scales).reshape(rows, WIDTH // 32)
    assert np.array_equal(qc.codes_of(packed), qc.best_codes(x, s))
    want_p, want_s = oracle.ple_quantize_rows(x)
    assert np.array_equal(packed, want_p) and np.array_equal(scales, want_s)


def test_quantize_table_in_place_then_gather(g4, oracle):
    # a dense [5000, 8960] BF16 table quantized shard by shard in place (the
    # last shard short), then gathered: bit-exact against the oracle's shards
    vocab = 5000
    bits, x = quantizer_rows(6, vocab, WIDTH)
    dense = g4.Buffer.from_array(bits)
    t = g4.PleTable(vocab, WIDTH, 32, RPS)
    t.quantize_from(dense)
    shards = []
    for s in range(t.num_shards):
        packed, scales = oracle.ple_quantize_rows(x[s * RPS:(s + 1) * RPS])
        shards.append(np.concatenate([packed.reshape(-1),
                                      scales.astype("<u2").view(np.uint8).reshape(-1)]))
        assert shards[-1].nbytes == t.shard_bytes(s)
    ids = np.concatenate([np.arange(0, vocab, 7), [RPS - 1, RPS, vocab - 1]]).astype(np.int32)
    got = gather(g4, t, ids, g4.F32)
    want = oracle.ple_gather(np.concatenate(shards), vocab, WIDTH, RPS, ids)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    t.free()


def test_quantize_rejects_bad_geometry(g4):
    src = g4.Buffer(64 * 48 * 2)
    out = g4.Buffer(64 * 48)
    with pytest.raises(g4.G4Error) as e:
        g4.ple_quantize_rows(src, 64, 48, out)  # width not a multiple of 32
    assert e.value.code == g4.G4_E_ARG
    with pytest.raises(g4.G4Error) as e:
        g4.ple_quantize_rows(src, 64, 64, out)  # src too short for 64 x 64
    assert e.value.code == g4.G4_E_RANGE
