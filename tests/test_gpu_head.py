"""GPU parity of the tied BF16 LM head (GEMV + 30*tanh(x/30) softcap)."""
import numpy as np
import pytest

import synthetic as syn

pytestmark = pytest.mark.gpu


def test_head_full_vocab(g4, oracle):
    vocab, k = 262144, 1536
    rng = np.random.default_rng(12)
    E = syn.bf16_rne(rng.standard_normal((vocab, k), dtype=np.float32) * np.float32(0.03))
    h = rng.standard_normal(k).astype(np.float32) * np.float32(2.0)
    Eb = g4.Buffer.from_array(E)
    hb = g4.Buffer.from_array(h)
    out = g4.Buffer(vocab * 4)
    g4.bf16_head(hb.ptr, Eb.ptr, vocab, k, out.ptr, 1.0, 30.0)
    got = out.download(np.float32)
    want = oracle.bf16_head(h, E, 1.0, 30.0)
    assert np.allclose(got, want, rtol=1e-4, atol=1e-4)
    # the largest logits agree, so greedy decoding picks the same token
    assert oracle.topk(got, 10)[0][0] == oracle.topk(want, 10)[0][0]


def test_head_chunks_write_at_their_offset(g4, oracle):
    # headChunk writes rows [start, start+rows) of the logits buffer
    # (gemma4-webgpu.js:417-419): pass the offset pointer.
    k, rows = 1536, 5000
    rng = np.random.default_rng(3)
    E = syn.bf16_rne(rng.standard_normal((rows, k), dtype=np.float32) * np.float32(0.05))
    h = rng.standard_normal(k).astype(np.float32)
    Eb = g4.Buffer.from_array(E)
    hb = g4.Buffer.from_array(h)
    out = g4.Buffer(rows * 4)
    for start in range(0, rows, 4096):
        n = min(4096, rows - start)
        g4.bf16_head(hb.ptr, Eb.at(start * k * 2), n, k, out.at(start * 4), 1.0, 30.0)
    got = out.download(np.float32)
    want = oracle.bf16_head(h, E, 1.0, 30.0)
    assert np.allclose(got, want, rtol=1e-4, atol=1e-4)


def test_head_no_softcap_and_scale(g4, oracle):
    k, rows = 256, 333
    rng = np.random.default_rng(4)
    E = syn.bf16_rne(rng.standard_normal((rows, k), dtype=np.float32))
    h = rng.standard_normal(k).astype(np.float32)
    Eb, hb, out = g4.Buffer.from_array(E), g4.Buffer.from_array(h), g4.Buffer(rows * 4)
    g4.bf16_head(hb.ptr, Eb.ptr, rows, k, out.ptr, 0.5, 0.0)
    want = oracle.bf16_head(h, E, 0.5, 0.0)
    assert np.allclose(out.download(np.float32), want, rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("seed", range(16))
def test_head_random_shapes(g4, oracle, seed):
    # Seeded random row counts (ragged against the kernel's 8-row groups and
    # blocks) and input widths (multiples of 8 up to 4096), with and without
    # the softcap.
    rng = np.random.default_rng(5000 + seed)
    rows = int(rng.integers(1, 3000))
    k = 8 * int(rng.integers(1, 513))
    scale, softcap = (1.0, 30.0) if seed % 2 == 0 else (0.5, 0.0)
    E = syn.bf16_rne(rng.standard_normal((rows, k), dtype=np.float32) * np.float32(0.05))
    h = rng.standard_normal(k).astype(np.float32)
    Eb, hb, out = g4.Buffer.from_array(E), g4.Buffer.from_array(h), g4.Buffer(rows * 4)
    g4.bf16_head(hb.ptr, Eb.ptr, rows, k, out.ptr, scale, softcap)
    got = out.download(np.float32)
    want = oracle.bf16_head(h, E, scale, softcap)
    assert np.allclose(got, want, rtol=1e-4, atol=1e-4), (rows, k)
