"""Seeded synthetic inputs in the checkpoint's own byte formats.

The model weights are not available offline, so benchmarks and tests feed the
kernels seeded data with the distributions of the measured workloads:

* W4A16 linear: q uniform integer in [-7, 7], stored as the offset nibble q+8,
  8 per little-endian u32 along K, low nibble first (compressed-tensors,
  official-w4a16.js:1-19); per-group (32 along K) scales bf16(|N(0,1)|*0.02).
  With full_range, q is uniform over the format's whole [-8, 7] (stored
  nibbles 0..15; official-w4a16.js:15-19) and every group holds q = -8
  (nibble 0) at least once.
* activations: bf16(N(0,1)), handed to the kernels as bf16 bits or as the
  exactly equal FP32 values.
* PLE table: q uniform integer in [-7, 7] as two's-complement nibbles, two per
  byte, low nibble first; scales bf16(|N(0,1)|*0.05) per 32-column group; each
  shard laid out packed block then scales block as the builder writes it
  (tools/build_ple_w4_full.py:130-170).  With full_range, q is uniform over
  [-8, 7] (all 16 nibbles; nibble 8 is -8, ple-w4-shard-reader.js:92) and
  every group holds nibble 8 at least once.
* token ids: uniform in [0, vocab).

bf16 conversion is round-to-nearest-even (official-w4a16.js:34-48).
"""
import numpy as np


def bf16_rne(a):
    """float32 array -> bf16 bits (uint16), round to nearest even."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    return ((u + np.uint32(0x7FFF) + lsb) >> np.uint32(16)).astype(np.uint16)


def bf16_to_f32(bits):
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def pack_w4(q):
    """int array [N, K] in [-8, 7] -> u32 [N, K/8] offset nibbles, low first."""
    q = np.asarray(q)
    n, k = q.shape
    nib = (q.astype(np.int32) + 8).astype(np.uint32).reshape(n, k // 8, 8)
    shifts = (np.arange(8, dtype=np.uint32) * np.uint32(4))
    return np.bitwise_or.reduce(nib << shifts, axis=2).astype(np.uint32)


def unpack_w4(packed):
    """u32 [N, K/8] -> int8 [N, K] logical values (nibble - 8)."""
    p = np.asarray(packed, dtype=np.uint32)
    n, kw = p.shape
    shifts = (np.arange(8, dtype=np.uint32) * np.uint32(4))
    nib = (p[:, :, None] >> shifts) & np.uint32(15)
    return (nib.astype(np.int16) - 8).astype(np.int8).reshape(n, kw * 8)


def _force_in_every_group(rng, q, value, group=32):
    """Set one random element of every `group`-wide group of q to `value`."""
    r, w = q.shape
    g = w // group
    pos = rng.integers(0, group, size=(r, g)) + np.arange(g) * group
    q[np.arange(r)[:, None], pos] = value
    return q


def w4_weights(seed, n, k, scale_mult=0.02, full_range=False):
    """(packed u32 [n, k/8], scales bf16 bits [n, k/32], q int8 [n, k])."""
    rng = np.random.default_rng([seed, n, k, 0x57 if not full_range else 0x58])
    if full_range:
        q = _force_in_every_group(rng, rng.integers(-8, 8, size=(n, k), dtype=np.int8), -8)
    else:
        q = rng.integers(-7, 8, size=(n, k), dtype=np.int8)
    s = np.abs(rng.standard_normal((n, k // 32), dtype=np.float32)) * np.float32(scale_mult)
    return pack_w4(q), bf16_rne(s), q


def activations(seed, m, k):
    """(bf16 bits [m, k], the same values as float32)."""
    rng = np.random.default_rng([seed, m, k, 0xA5])
    bits = bf16_rne(rng.standard_normal((m, k), dtype=np.float32))
    return bits, bf16_to_f32(bits).reshape(m, k)


def pack_ple(q):
    """int array [R, W] in [-8, 7] -> u8 [R, W/2] two's-complement, low first."""
    nib = (np.asarray(q).astype(np.int16) & 15).astype(np.uint8)
    return (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)


# Byte value for a uniformly drawn pair index p in [0, 225): low nibble
# q0 = p % 15 - 7, high nibble q1 = p // 15 - 7, both two's complement.
_PAIR = np.arange(225)
_PLE_PAIR_LUT = ((((_PAIR % 15) - 7) & 15) | ((((_PAIR // 15) - 7) & 15) << 4)).astype(np.uint8)


def ple_shard(seed, shard, rows, width=8960, scale_mult=0.05, full_range=False):
    """One shard file's bytes (packed block then scales block) as uint8.

    Each byte holds two independent q uniform in [-7, 7] (a pair drawn
    uniformly from the 225 combinations), or with full_range two q uniform in
    [-8, 7] (a uniform byte) with q = -8 in every 32-column group."""
    rng = np.random.default_rng([seed, shard, width, 0x91 if not full_range else 0x92])
    if full_range:
        q = rng.integers(-8, 8, size=(rows, width), dtype=np.int8)
        packed = pack_ple(_force_in_every_group(rng, q, -8))
    else:
        packed = _PLE_PAIR_LUT[rng.integers(0, 225, size=(rows, width // 2), dtype=np.uint8)]
    s = np.abs(rng.standard_normal((rows, width // 32), dtype=np.float32)) * np.float32(scale_mult)
    scales = bf16_rne(s).astype("<u2")
    return np.concatenate([packed.reshape(-1), scales.view(np.uint8).reshape(-1)])


def ple_table(seed, vocab=262144, width=8960, rows_per_shard=4096, threads=8, full_range=False):
    """All shard files of a table, generated in parallel: list of uint8 arrays."""
    from concurrent.futures import ThreadPoolExecutor
    nshards = (vocab + rows_per_shard - 1) // rows_per_shard

    def one(si):
        rows = min(rows_per_shard, vocab - si * rows_per_shard)
        return ple_shard(seed, si, rows, width, full_range=full_range)

    with ThreadPoolExecutor(max(1, threads)) as ex:
        return list(ex.map(one, range(nshards)))


def token_ids(seed, n, vocab):
    rng = np.random.default_rng([seed, n, vocab, 0x1D])
    return rng.integers(0, vocab, size=n, dtype=np.int32)
