"""Rows that pin the PLE quantizer's divisor, and a brute-force check of codes.

quantize_batch (tools/build_ple_w4_full.py:48-60) takes s = maxabs / 7 in
FP32, stores it as BF16 (round to nearest even) and quantizes against the
STORED scale: q = clip(rint(x / s_bf16), -7, 7) ("matching runtime
behavior", :54-56).  A restatement that divided by the FP32 scale instead
would agree on most inputs, because the two scales differ by at most 2^-9
relative.  These rows make the difference visible: every group's maximum M
has bf16(M / 7) != M / 7, and most other elements are BF16 values that lie
strictly between the two scales' rounding boundaries (k + 1/2) * s_bf16 and
(k + 1/2) * s_f32, so the two divisors give different codes there.

best_codes() characterises the expected codes without division or rint: the
k in [-7, 7] minimising |k * s - x|, ties to the even k, evaluated exactly in
binary64 (k * s and x - k * s are exact there for BF16 x and s).  Elements
whose quotient x / s lies within 2^-20 of a half-integer without being one
are avoided, so that FP32 division followed by rint (the reference's steps)
and the exact argmin cannot disagree.
"""
import numpy as np

import synthetic as syn


def _bf16(v):
    return syn.bf16_to_f32(syn.bf16_rne(np.asarray(v, np.float32))).reshape(np.shape(v))


def _ambiguous(x, s):
    t = np.asarray(x, np.float64) / np.asarray(s, np.float64)
    h = t - np.floor(t) - 0.5
    return (h != 0) & (np.abs(h) < 2.0 ** -20 * np.maximum(np.abs(t), 1.0))


def divisor_rows(seed, rows, width):
    """(bf16 bits [rows, width], the same values as FP32, mask of the
    elements where the FP32 divisor would give a different code)."""
    rng = np.random.default_rng(seed)
    G = width // 32
    # group maxima: BF16 values whose FP32 seventh is not a BF16 value
    M = _bf16(np.abs(rng.standard_normal((rows, G))).astype(np.float32) * np.float32(0.05) + 1e-3)
    s_f = (M / np.float32(7)).astype(np.float32)
    s_st = _bf16(s_f)
    for _ in range(8):
        same = s_st == s_f
        if not same.any():
            break
        M[same] = _bf16(M[same] * np.float32(1.0 + 2.0 ** -7))
        s_f = (M / np.float32(7)).astype(np.float32)
        s_st = _bf16(s_f)
    M[s_st == s_f] = np.float32(0.625)  # 0.625 / 7 is not a BF16 value
    s_f = (M / np.float32(7)).astype(np.float32)
    s_st = _bf16(s_f)
    assert (s_st != s_f).all()
    sf = np.repeat(s_f, 32, axis=1).astype(np.float64)
    ss = np.repeat(s_st, 32, axis=1).astype(np.float64)
    # candidates between the boundaries (k + 1/2) * s_bf16 and (k + 1/2) * s_f32
    k = rng.integers(0, 7, size=(rows, width)).astype(np.float64)
    sign = np.where(rng.integers(0, 2, size=(rows, width)) == 1, 1.0, -1.0)
    b_st, b_f = (k + 0.5) * ss, (k + 0.5) * sf
    lo, hi = np.minimum(b_st, b_f), np.maximum(b_st, b_f)
    mid = _bf16(((lo + hi) / 2).astype(np.float32)).astype(np.float64)
    bits = syn.bf16_rne(mid.astype(np.float32)).reshape(rows, width)
    x = mid.copy()
    ok = (x > lo) & (x < hi)
    for step in (-1, 1):  # the BF16 neighbours of the rounded midpoint
        cand = syn.bf16_to_f32((bits.astype(np.int32) + step).astype(np.uint16)).reshape(rows, width)
        cand = cand.astype(np.float64)
        take = ~ok & (cand > lo) & (cand < hi)
        x[take] = cand[take]
        ok |= take
    # the rest: uniform in (-M, M), BF16, avoiding near-ties
    rest = _bf16((rng.uniform(-1, 1, (rows, width)) * np.repeat(M, 32, axis=1)).astype(np.float32))
    x = np.where(ok, sign * x, rest.astype(np.float64))
    x[_ambiguous(x, ss) | _ambiguous(x, sf)] = 0.0
    # element 0 of every group carries the maximum (either sign)
    first = np.arange(G) * 32
    x[:, first] = np.where(rng.integers(0, 2, size=(rows, G)) == 1, 1.0, -1.0) * M
    x32 = x.astype(np.float32)
    assert np.array_equal(_bf16(x32), x32)
    assert np.array_equal(np.abs(x32).reshape(rows, G, 32).max(axis=2), M)
    xbits = syn.bf16_rne(x32).reshape(rows, width)
    differs = best_codes(x32, s_st) != best_codes(x32, s_f)
    return xbits, x32, differs


def best_codes(x, s):
    """The k in [-7, 7] minimising |k * s - x| (ties to even k) per element;
    x [rows, width], s [rows, width / 32] per-group scales (binary64-exact)."""
    x = np.asarray(x, np.float64)
    rows, width = x.shape
    s = np.repeat(np.asarray(s, np.float64).reshape(rows, width // 32), 32, axis=1)
    ks = np.arange(-7, 8, dtype=np.float64)
    err = np.abs(ks[None, None, :] * s[..., None] - x[..., None])
    best = err.min(axis=2, keepdims=True)
    cand = err == best
    # among the minimisers prefer an even k (there are at most two)
    even = cand & (ks[None, None, :] % 2 == 0)
    pick = np.where(even.any(axis=2, keepdims=True), even, cand)
    return (ks[np.argmax(pick, axis=2)]).astype(np.int8)


def codes_of(packed):
    """Two's-complement nibbles of packed bytes [rows, width/2] as int8 q."""
    p = np.asarray(packed, np.uint8)
    nib = np.stack([p & 15, p >> 4], axis=-1).reshape(p.shape[0], -1).astype(np.int16)
    return np.where(nib >= 8, nib - 16, nib).astype(np.int8)
