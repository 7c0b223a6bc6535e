"""ctypes front end of the C oracle (g4_oracle.c).

TEST INFRASTRUCTURE, NOT PRODUCT CODE: imported only by tests/, by
__graft_entry__.smoke() and by bench.py's CPU-baseline leg, always to check
results against; nothing in the product path calls it.

Build recipe (also run by __graft_entry__.build()):
    gcc -O2 -std=c99 -fPIC -shared -fopenmp -ffp-contract=off oracle/g4_oracle.c -lm \
        -o oracle/_build/libg4oracle.so
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "g4_oracle.c")
LIB_PATH = os.path.join(HERE, "_build", "libg4oracle.so")

_c = ctypes
_p = _c.c_void_p
_i = _c.c_int
_z = _c.c_size_t

_SIGS = {
    "g4o_bf16_to_f32": (_c.c_float, [_c.c_uint16]),
    "g4o_f32_to_bf16": (_c.c_uint16, [_c.c_float]),
    "g4o_bf16_to_f32_array": (None, [_p, _z, _p]),
    "g4o_f32_to_bf16_array": (None, [_p, _z, _p]),
    "g4o_w4_nibble": (_i, [_c.c_uint32]),
    "g4o_ple_nibble": (_i, [_c.c_uint32]),
    "g4o_w4_dequant_rows": (_i, [_p, _z, _p, _z, _i, _i, _i, _i, _i, _p]),
    "g4o_w4_linear": (_i, [_p, _i, _p, _p, _i, _i, _i, _i, _p]),
    "g4o_w4_linear_f64": (_i, [_p, _i, _p, _p, _i, _i, _i, _p]),
    "g4o_w4_linear_mt": (_i, [_p, _i, _p, _p, _i, _i, _i, _i, _p, _i]),
    "g4o_omp_threads": (_i, [_i]),
    "g4o_ple_dequant_row": (None, [_p, _p, _i, _p]),
    "g4o_ple_locate": (_i, [_c.c_longlong, _i, _i, _c.POINTER(_i), _c.POINTER(_i)]),
    "g4o_ple_row_offsets": (None, [_i, _i, _i, _i, _i, _c.POINTER(_z), _c.POINTER(_z)]),
    "g4o_ple_gather": (_i, [_p, _i, _i, _i, _p, _i, _p]),
    "g4o_ple_gather_mt": (_i, [_p, _i, _i, _i, _p, _i, _p, _i]),
    "g4o_ple_quantize_rows": (None, [_p, _i, _i, _p, _p]),
    "g4o_bf16_head": (None, [_p, _p, _i, _i, _c.c_float, _c.c_float, _p]),
    "g4o_topk": (_i, [_p, _i, _i, _p, _p]),
}


def build(force=False):
    if force or not os.path.exists(LIB_PATH) or os.path.getmtime(LIB_PATH) < os.path.getmtime(SRC):
        os.makedirs(os.path.dirname(LIB_PATH), exist_ok=True)
        tmp = LIB_PATH + ".tmp"
        subprocess.run(["gcc", "-O2", "-std=c99", "-Wall", "-fPIC", "-shared", "-fopenmp",
                        "-ffp-contract=off", SRC, "-lm", "-o", tmp], check=True)
        os.replace(tmp, LIB_PATH)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data


def bf16_to_f32(bits):
    return lib().g4o_bf16_to_f32(int(bits))


def f32_to_bf16(v):
    return lib().g4o_f32_to_bf16(float(v))


def bf16_to_f32_array(bits):
    bits = np.ascontiguousarray(bits, dtype=np.uint16).reshape(-1)
    out = np.empty(bits.size, dtype=np.float32)
    lib().g4o_bf16_to_f32_array(_ptr(bits), bits.size, _ptr(out))
    return out


def f32_to_bf16_array(v):
    v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1)
    out = np.empty(v.size, dtype=np.uint16)
    lib().g4o_f32_to_bf16_array(_ptr(v), v.size, _ptr(out))
    return out


def w4_nibble(n):
    return lib().g4o_w4_nibble(int(n))


def ple_nibble(n):
    return lib().g4o_ple_nibble(int(n))


def w4_dequant_rows(packed, scales_f32, out_dim, in_dim, row_start, row_count, group=32):
    """Returns (status, FP32 [row_count, in_dim])."""
    packed = np.ascontiguousarray(packed).view(np.int32).reshape(-1)
    scales_f32 = np.ascontiguousarray(scales_f32, dtype=np.float32).reshape(-1)
    out = np.zeros((max(row_count, 0), in_dim), dtype=np.float32)
    rc = lib().g4o_w4_dequant_rows(_ptr(packed), packed.size, _ptr(scales_f32), scales_f32.size,
                                   out_dim, in_dim, row_start, row_count, group, _ptr(out))
    return rc, out


def w4_linear(x, packed, scales_bf16, group=32, chunk=256):
    """FP32 TF.js-semantics linear: x [M, K] f32 -> y [M, N] f32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    packed = np.ascontiguousarray(packed).view(np.int32)
    scales_bf16 = np.ascontiguousarray(scales_bf16).view(np.uint16)
    m, k = x.shape
    n = packed.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    rc = lib().g4o_w4_linear(_ptr(x), m, _ptr(packed), _ptr(scales_bf16), n, k, group, chunk, _ptr(y))
    if rc:
        raise ValueError("g4o_w4_linear failed with %d" % rc)
    return y


def w4_linear_mt(x, packed, scales_bf16, threads=0, group=32, chunk=256):
    """w4_linear with the output chunks over `threads` OpenMP threads (0: all);
    bit-identical to w4_linear."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    packed = np.ascontiguousarray(packed).view(np.int32)
    scales_bf16 = np.ascontiguousarray(scales_bf16).view(np.uint16)
    m, k = x.shape
    n = packed.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    rc = lib().g4o_w4_linear_mt(_ptr(x), m, _ptr(packed), _ptr(scales_bf16), n, k, group, chunk,
                                _ptr(y), int(threads))
    if rc:
        raise ValueError("g4o_w4_linear_mt failed with %d" % rc)
    return y


def omp_threads(threads=0):
    return lib().g4o_omp_threads(int(threads))


def w4_linear_f64(x, packed, scales_bf16, group=32):
    x = np.ascontiguousarray(x, dtype=np.float32)
    packed = np.ascontiguousarray(packed).view(np.int32)
    scales_bf16 = np.ascontiguousarray(scales_bf16).view(np.uint16)
    m, k = x.shape
    n = packed.shape[0]
    y = np.empty((m, n), dtype=np.float64)
    rc = lib().g4o_w4_linear_f64(_ptr(x), m, _ptr(packed), _ptr(scales_bf16), n, k, group, _ptr(y))
    if rc:
        raise ValueError("g4o_w4_linear_f64 failed with %d" % rc)
    return y


def ple_dequant_row(packed_row, scale_bits, width):
    packed_row = np.ascontiguousarray(packed_row, dtype=np.uint8)
    scale_bits = np.ascontiguousarray(scale_bits, dtype=np.uint16)
    out = np.empty(width, dtype=np.float32)
    lib().g4o_ple_dequant_row(_ptr(packed_row), _ptr(scale_bits), width, _ptr(out))
    return out


def ple_locate(token_id, vocab, rows_per_shard=4096):
    s, l = _i(), _i()
    rc = lib().g4o_ple_locate(int(token_id), vocab, rows_per_shard, ctypes.byref(s), ctypes.byref(l))
    return None if rc else (s.value, l.value)


def ple_row_offsets(vocab, width, rows_per_shard, shard, local_row):
    po, so = _z(), _z()
    lib().g4o_ple_row_offsets(vocab, width, rows_per_shard, shard, local_row,
                              ctypes.byref(po), ctypes.byref(so))
    return po.value, so.value


def ple_gather(table, vocab, width, rows_per_shard, ids):
    """table: uint8 concatenation of the shard files; returns FP32 [n, width]."""
    table = np.ascontiguousarray(table, dtype=np.uint8)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    out = np.empty((ids.size, width), dtype=np.float32)
    rc = lib().g4o_ple_gather(_ptr(table), vocab, width, rows_per_shard, _ptr(ids), ids.size, _ptr(out))
    if rc:
        raise IndexError("PLE token out of range at position %d" % (-1 - rc))
    return out


def ple_gather_mt(table, vocab, width, rows_per_shard, ids, threads=0):
    """ple_gather with the ids over `threads` OpenMP threads (0: all); the same output."""
    table = np.ascontiguousarray(table, dtype=np.uint8)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    out = np.empty((ids.size, width), dtype=np.float32)
    rc = lib().g4o_ple_gather_mt(_ptr(table), vocab, width, rows_per_shard, _ptr(ids), ids.size,
                                 _ptr(out), int(threads))
    if rc:
        raise IndexError("PLE token out of range at position %d" % (-1 - rc))
    return out


def ple_quantize_rows(rows):
    rows = np.ascontiguousarray(rows, dtype=np.float32)
    b, w = rows.shape
    packed = np.empty((b, w // 2), dtype=np.uint8)
    scales = np.empty((b, w // 32), dtype=np.uint16)
    lib().g4o_ple_quantize_rows(_ptr(rows), b, w, _ptr(packed), _ptr(scales))
    return packed, scales


def bf16_head(x, E_bits, scale=1.0, softcap=30.0):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    E_bits = np.ascontiguousarray(E_bits).view(np.uint16)
    rows, k = E_bits.shape
    out = np.empty(rows, dtype=np.float32)
    lib().g4o_bf16_head(_ptr(x), _ptr(E_bits), rows, k, scale, softcap, _ptr(out))
    return out


def topk(logits, k=10):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    ids = np.zeros(max(k, 1), dtype=np.int32)
    vals = np.zeros(max(k, 1), dtype=np.float32)
    n = lib().g4o_topk(_ptr(logits), logits.size, k, _ptr(ids), _ptr(vals))
    return ids[:n].copy(), vals[:n].copy()
