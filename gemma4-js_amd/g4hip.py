"""ctypes binding of libg4hip (include/g4hip.h) for the Python tests and benchmark.

The Node addon (node/g4_napi.cc) is the reference-facing binding; this module
is the same C ABI seen from Python.  It never computes anything itself: if
libg4hip.so is missing it raises, it does not fall back to a CPU path.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libg4hip.so")

F32 = 0
BF16 = 1

G4_OK = 0
G4_E_ARG = 1
G4_E_RANGE = 2
G4_E_STATE = 3
G4_E_HIP = 4
G4_E_NOMEM = 5

_c = ctypes
_vp = _c.c_void_p
_int = _c.c_int
_sz = _c.c_size_t

# name -> (restype, argtypes); mirrors include/g4hip.h
SIGNATURES = {
    "g4_init": (_int, [_int]),
    "g4_last_error": (_c.c_char_p, []),
    "g4_device_info": (_int, [_c.c_char_p, _sz, _c.POINTER(_int), _c.POINTER(_sz), _c.POINTER(_int)]),
    "g4_alloc": (_int, [_sz, _c.POINTER(_vp)]),
    "g4_free": (_int, [_vp]),
    "g4_upload": (_int, [_vp, _sz, _vp, _sz]),
    "g4_download": (_int, [_vp, _sz, _vp, _sz]),
    "g4_copy": (_int, [_vp, _sz, _vp, _sz, _sz]),
    "g4_sync": (_int, []),
    "g4_stream": (_vp, []),
    "g4_encoder_begin": (_int, []),
    "g4_encoder_finish": (_int, [_c.POINTER(_vp)]),
    "g4_submit": (_int, [_vp]),
    "g4_cmdbuf_free": (_int, [_vp]),
    "g4_event_create": (_int, [_c.POINTER(_vp)]),
    "g4_event_record": (_int, [_vp]),
    "g4_event_elapsed_ms": (_int, [_vp, _vp, _c.POINTER(_c.c_float)]),
    "g4_event_destroy": (_int, [_vp]),
    "g4_w4_load": (_int, [_vp, _vp, _int, _int, _int, _c.POINTER(_vp)]),
    "g4_w4_free": (_int, [_vp]),
    "g4_w4_info": (_int, [_vp, _c.POINTER(_int), _c.POINTER(_int), _c.POINTER(_int), _c.POINTER(_sz)]),
    "g4_w4_linear": (_int, [_vp, _vp, _int, _int, _vp, _int]),
    "g4_w4_linear_multi": (_int, [_c.POINTER(_vp), _int, _vp, _int, _int, _c.POINTER(_vp), _int]),
    "g4_w4_linear_noalloc": (_int, [_vp, _vp, _int, _int, _vp, _int]),
    "g4_w4_gemv_stamps": (_int, [_vp, _vp, _int, _vp, _int, _vp, _c.POINTER(_int)]),
    "g4_w4_dequant": (_int, [_vp, _int, _int, _vp, _int]),
    "g4_ple_create": (_int, [_int, _int, _int, _int, _c.POINTER(_vp)]),
    "g4_ple_upload_shard": (_int, [_vp, _int, _vp, _sz]),
    "g4_ple_shard_bytes": (_int, [_vp, _int, _c.POINTER(_int), _c.POINTER(_sz)]),
    "g4_ple_free": (_int, [_vp]),
    "g4_ple_quantize_rows": (_int, [_vp, _int, _int, _vp]),
    "g4_ple_quantize_table": (_int, [_vp, _vp]),
    "g4_ple_gather": (_int, [_vp, _vp, _int, _vp, _int]),
    "g4_ple_gather_dev": (_int, [_vp, _vp, _int, _vp, _int]),
    "g4_bf16_head": (_int, [_vp, _vp, _int, _int, _vp, _c.c_float, _c.c_float]),
    "g4_rms": (_int, [_vp, _int, _int, _vp, _c.c_float, _vp]),
    "g4_add_scale": (_int, [_vp, _vp, _sz, _c.c_float, _vp]),
    "g4_scale": (_int, [_vp, _sz, _c.c_float, _vp]),
    "g4_gelu_mul": (_int, [_vp, _vp, _sz, _vp]),
    "g4_gelu_ple": (_int, [_vp, _vp, _int, _int, _int, _int, _vp]),
    "g4_norm_rope": (_int, [_vp, _int, _int, _int, _int, _vp, _int, _c.c_float, _c.c_float, _vp]),
    "g4_attention": (_int, [_vp, _vp, _vp, _int, _int, _int, _int, _int, _int, _int, _vp]),
    "g4_ple_mix": (_int, [_vp, _vp, _vp, _int, _int, _int, _vp]),
    "g4_embed": (_int, [_vp, _int, _int, _vp, _int, _c.c_float, _vp]),
    "g4_argmax": (_int, [_vp, _int, _vp]),
    "g4_w4_load_dev": (_int, [_vp, _vp, _int, _int, _int, _c.POINTER(_vp)]),
    "g4_w4_load_opts": (_int, [_vp, _vp, _int, _int, _int, _int, _c.POINTER(_vp)]),
    "g4_ple_upload_shard_dev": (_int, [_vp, _int, _vp, _sz]),
    "g4_fill_random": (_int, [_vp, _sz, _int, _c.c_uint64, _c.c_float]),
    "g4_gemma_e2b_config": (_int, [_int, _vp]),
    "g4_gemma_create": (_int, [_vp, _c.POINTER(_vp)]),
    "g4_gemma_free": (_int, [_vp]),
    "g4_gemma_set_linear": (_int, [_vp, _int, _int, _vp]),
    "g4_gemma_set_norm": (_int, [_vp, _int, _int, _vp, _int]),
    "g4_gemma_set_layer_scalar": (_int, [_vp, _int, _c.c_float]),
    "g4_gemma_set_embedding": (_int, [_vp, _vp]),
    "g4_gemma_set_ple": (_int, [_vp, _vp]),
    "g4_gemma_set_ple_dense": (_int, [_vp, _vp]),
    "g4_gemma_reset": (_int, [_vp]),
    "g4_gemma_cache_length": (_int, [_vp, _c.POINTER(_int)]),
    "g4_gemma_forward": (_int, [_vp, _vp, _int, _int, _vp]),
    "g4_gemma_logits": (_int, [_vp, _vp, _vp]),
    "g4_gemma_greedy": (_int, [_vp, _vp, _int, _int, _c.POINTER(_c.c_int32), _vp]),
    "g4_gemma_decode": (_int, [_vp, _int, _vp]),
    "g4_gemma_last_hidden": (_int, [_vp, _vp]),
    "g4_gemma_forward_diag": (_int, [_vp, _vp, _int, _int, _vp, _vp, _vp, _vp, _int, _vp]),
    "g4_gemma_diag_stages": (_int, [_vp, _int, _int, _c.POINTER(_sz)]),
}

# g4_fill_random kinds
(RAND_W4_PACKED, RAND_PLE_PACKED, RAND_BF16_ABS_NORMAL, RAND_BF16_NORMAL, RAND_F32_NORMAL,
 RAND_W4_PACKED_FULL, RAND_PLE_PACKED_FULL) = range(7)
# g4_gemma projections and norms
PROJ = dict(q=0, k=1, v=2, o=3, gate=4, up=5, down=6, ple_gate=7, ple_proj=8, top=9)
NORM = dict(input=0, post_attn=1, pre_ffw=2, post_ffw=3, post_ple=4, q=5, k=6,
            ple_projection=7, final=8)
GEMMA_MAX_LAYERS = 64
# g4_gemma_forward_diag stages, encodeLayer's probe names (gemma4-webgpu.js:224-309)
STAGE_NAMES = ["preAttention", "qRaw", "qNormRoPE", "kRaw", "vRaw", "kNormRoPE", "vNorm",
               "attentionContext", "attentionOutput", "postAttentionNorm", "attentionResidual",
               "preFfw", "mlpGate", "mlpUp", "mlpActivated", "ffwOutput", "postFfwNorm",
               "ffwResidual", "pleGate", "pleModulated", "pleProjected", "pleNormalized",
               "output"]
STAGES = len(STAGE_NAMES)


class GemmaConfig(_c.Structure):
    _fields_ = [("hidden", _int), ("heads", _int), ("ple_dim", _int), ("vocab", _int),
                ("layers", _int), ("max_seq", _int), ("window", _int), ("eps", _c.c_float),
                ("softcap", _c.c_float),
                ("head_dim", _int * GEMMA_MAX_LAYERS), ("intermediate", _int * GEMMA_MAX_LAYERS),
                ("full", _int * GEMMA_MAX_LAYERS), ("kv_source", _int * GEMMA_MAX_LAYERS),
                ("rope_base", _c.c_float * GEMMA_MAX_LAYERS),
                ("rope_prop", _c.c_float * GEMMA_MAX_LAYERS)]


class G4Error(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("[g4 status %d] %s" % (code, msg))
        self.code = code


_lib = None


def lib(path=LIB_PATH):
    """Load libg4hip.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise FileNotFoundError(
                "%s is missing: build it with `python3 gemma4-js_amd/build.py` "
                "(there is no CPU fallback)" % path)
        L = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc):
    if rc != G4_OK:
        raise G4Error(rc, lib().g4_last_error().decode(errors="replace"))


def init(device=0):
    check(lib().g4_init(device))


def device_info():
    name = ctypes.create_string_buffer(256)
    cu, hbm, clk = _int(), _sz(), _int()
    check(lib().g4_device_info(name, 256, ctypes.byref(cu), ctypes.byref(hbm), ctypes.byref(clk)))
    return {"name": name.value.decode(), "cu_count": cu.value, "hbm_bytes": hbm.value,
            "clock_khz": clk.value}


def sync():
    check(lib().g4_sync())


class Buffer:
    """A device buffer from g4_alloc (createBuffer)."""

    def __init__(self, nbytes):
        p = _vp()
        check(lib().g4_alloc(int(nbytes), ctypes.byref(p)))
        self.ptr = p.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a, offset=0):
        a = np.ascontiguousarray(a)
        check(lib().g4_upload(self.ptr, int(offset), a.ctypes.data, a.nbytes))

    def download(self, dtype, count=None, offset=0):
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(int(count), dtype=dtype)
        check(lib().g4_download(self.ptr, int(offset), out.ctypes.data, out.nbytes))
        return out

    def at(self, offset):
        """Device address `offset` bytes into the buffer."""
        return self.ptr + int(offset)

    def free(self):
        if self.ptr:
            check(lib().g4_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.g4_free(self.ptr)
        except Exception:
            pass


class CommandBuffer:
    """A finished command encoder (captured HIP graph); submit() replays it."""

    def __init__(self, ptr):
        self.ptr = ptr

    def submit(self):
        check(lib().g4_submit(self.ptr))

    def free(self):
        if self.ptr:
            check(lib().g4_cmdbuf_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.g4_cmdbuf_free(self.ptr)
        except Exception:
            pass


class Encoder:
    """`with Encoder() as enc:` records the launches made inside the block."""

    def __enter__(self):
        check(lib().g4_encoder_begin())
        self.cmdbuf = None
        return self

    def __exit__(self, et, ev, tb):
        p = _vp()
        rc = lib().g4_encoder_finish(ctypes.byref(p))
        if et is None:
            check(rc)
            self.cmdbuf = CommandBuffer(p.value)
        return False


class Event:
    def __init__(self):
        p = _vp()
        check(lib().g4_event_create(ctypes.byref(p)))
        self.ptr = p.value

    def record(self):
        check(lib().g4_event_record(self.ptr))

    def elapsed_ms(self, stop):
        ms = _c.c_float()
        check(lib().g4_event_elapsed_ms(self.ptr, stop.ptr, ctypes.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.g4_event_destroy(self.ptr)
        except Exception:
            pass


# g4_w4_load_opts flags
W4_SRC_DEVICE, W4_NO_GEMM_TILES = 1, 2


class W4Linear:
    """GPUW4Linear: compressed-tensors W4A16 weights resident on the device.
    gemm_tiles=False skips the prefill GEMM's tile copy (decode-only weights)."""

    def __init__(self, packed, scales, group=32, gemm_tiles=True):
        packed = np.ascontiguousarray(packed).view(np.uint32)
        scales = np.ascontiguousarray(scales).view(np.uint16)
        if packed.ndim != 2 or scales.ndim != 2:
            raise ValueError("packed and scales must be rank-2")
        self.out_dim = packed.shape[0]
        self.in_dim = packed.shape[1] * 8
        self.group = group
        h = _vp()
        if gemm_tiles:
            check(lib().g4_w4_load(packed.ctypes.data, scales.ctypes.data, self.out_dim,
                                   self.in_dim, group, ctypes.byref(h)))
        else:
            check(lib().g4_w4_load_opts(packed.ctypes.data, scales.ctypes.data, self.out_dim,
                                        self.in_dim, group, W4_NO_GEMM_TILES, ctypes.byref(h)))
        self.h = h.value

    @classmethod
    def _from_handle(cls, h, out_dim, in_dim, group=32):
        self = cls.__new__(cls)
        self.h, self.out_dim, self.in_dim, self.group = h, out_dim, in_dim, group
        return self

    def info(self):
        n, k, g, b = _int(), _int(), _int(), _sz()
        check(lib().g4_w4_info(self.h, ctypes.byref(n), ctypes.byref(k), ctypes.byref(g),
                               ctypes.byref(b)))
        return {"out_dim": n.value, "in_dim": k.value, "group": g.value, "device_bytes": b.value}

    def linear(self, x_ptr, x_dtype, rows, y_ptr, y_dtype=F32):
        check(lib().g4_w4_linear(self.h, x_ptr, x_dtype, rows, y_ptr, y_dtype))

    def stamp_waves(self):
        """Waves of the row-split decode GEMV launch (g4_w4_gemv_stamps size query)."""
        n = _c.c_int()
        check(lib().g4_w4_gemv_stamps(self.h, None, BF16, None, F32, None, _c.byref(n)))
        return n.value

    def gemv_stamps(self, x_ptr, x_dtype, y_ptr, stamps_ptr, y_dtype=F32):
        """g4_w4_gemv_stamps: one row through the row-split GEMV, 5 clock stamps
        per wave into stamps_ptr (device, stamp_waves() * 5 uint64)."""
        n = _c.c_int()
        check(lib().g4_w4_gemv_stamps(self.h, x_ptr, x_dtype, y_ptr, y_dtype, stamps_ptr,
                                      _c.byref(n)))
        return n.value

    def linear_noalloc(self, x_ptr, x_dtype, rows, y_ptr, y_dtype=F32):
        """g4_w4_linear_noalloc: the same linear on the library's static scratch."""
        check(lib().g4_w4_linear_noalloc(self.h, x_ptr, x_dtype, rows, y_ptr, y_dtype))

    @staticmethod
    def linear_multi(linears, x_ptr, x_dtype, rows, y_ptrs, y_dtype=F32):
        """g4_w4_linear_multi: every linear of `linears` (same in_dim) over
        one x; y_ptrs[i] receives linears[i]'s output."""
        n = len(linears)
        if len(y_ptrs) != n:
            raise ValueError("one output per linear")
        ws = (_vp * n)(*[w.h for w in linears])
        ys = (_vp * n)(*y_ptrs)
        check(lib().g4_w4_linear_multi(ws, n, x_ptr, x_dtype, rows, ys, y_dtype))

    def dequant(self, row_start, row_count, out_ptr, out_dtype=F32):
        check(lib().g4_w4_dequant(self.h, row_start, row_count, out_ptr, out_dtype))

    def free(self):
        if self.h:
            check(lib().g4_w4_free(self.h))
            self.h = None

    def __del__(self):
        try:
            if self.h and _lib is not None:
                _lib.g4_w4_free(self.h)
        except Exception:
            pass


class PleTable:
    """W4PleShardBundle with the whole table resident on the device."""

    def __init__(self, vocab, width=8960, group=32, rows_per_shard=4096):
        h = _vp()
        check(lib().g4_ple_create(vocab, width, group, rows_per_shard, ctypes.byref(h)))
        self.h = h.value
        self.vocab, self.width, self.rows_per_shard = vocab, width, rows_per_shard
        ns = _int()
        check(lib().g4_ple_shard_bytes(self.h, 0, ctypes.byref(ns), None))
        self.num_shards = ns.value

    def shard_bytes(self, shard):
        b = _sz()
        check(lib().g4_ple_shard_bytes(self.h, shard, None, ctypes.byref(b)))
        return b.value

    def upload_shard(self, shard, data):
        data = np.frombuffer(data, dtype=np.uint8) if isinstance(data, (bytes, bytearray)) \
            else np.ascontiguousarray(data).view(np.uint8)
        check(lib().g4_ple_upload_shard(self.h, shard, data.ctypes.data, data.nbytes))

    def quantize_from(self, dense):
        """g4_ple_quantize_table: build every shard from dense BF16 rows [vocab, width]
        (a Buffer or device pointer)."""
        check(lib().g4_ple_quantize_table(self.h, _f(dense)))

    def gather(self, ids, out_ptr, out_dtype=F32):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        check(lib().g4_ple_gather(self.h, ids.ctypes.data, ids.size, out_ptr, out_dtype))

    def gather_dev(self, ids_ptr, n, out_ptr, out_dtype=F32):
        check(lib().g4_ple_gather_dev(self.h, ids_ptr, n, out_ptr, out_dtype))

    def free(self):
        if self.h:
            check(lib().g4_ple_free(self.h))
            self.h = None

    def __del__(self):
        try:
            if self.h and _lib is not None:
                _lib.g4_ple_free(self.h)
        except Exception:
            pass


def ple_quantize_rows(rows_bf16, nrows, width, shard):
    """g4_ple_quantize_rows: one shard file's bytes from BF16 rows on the device."""
    check(lib().g4_ple_quantize_rows(_f(rows_bf16), nrows, width, _f(shard)))


def bf16_head(x_ptr, E_ptr, rows, in_dim, out_ptr, scale=1.0, softcap=30.0):
    check(lib().g4_bf16_head(x_ptr, E_ptr, rows, in_dim, out_ptr, scale, softcap))


def _f(p):
    return p if p is None or isinstance(p, int) else p.ptr


def rms(x, rows, width, scale, y, eps=1e-6):
    check(lib().g4_rms(_f(x), rows, width, _f(scale), eps, _f(y)))


def add_scale(a, b, n, s, y):
    check(lib().g4_add_scale(_f(a), _f(b), n, s, _f(y)))


def scale(a, n, s, y):
    check(lib().g4_scale(_f(a), n, s, _f(y)))


def gelu_mul(gate, up, n, y):
    check(lib().g4_gelu_mul(_f(gate), _f(up), n, _f(y)))


def gelu_ple(gate, ple, rows, layer, width, layers, y):
    check(lib().g4_gelu_ple(_f(gate), _f(ple), rows, layer, width, layers, _f(y)))


def norm_rope(x, rows, heads, hd, pos0, scale_, rope_angles, base, y, eps=1e-6):
    check(lib().g4_norm_rope(_f(x), rows, heads, hd, pos0, _f(scale_), rope_angles, base, eps,
                             _f(y)))


def attention(q, k, v, qrows, heads, hd, keylen, qpos0, sliding, window, y):
    check(lib().g4_attention(_f(q), _f(k), _f(v), qrows, heads, hd, keylen, qpos0,
                             1 if sliding else 0, window, _f(y)))


def ple_mix(proj, norm_scale, token_ple, rows, width, layers, y):
    check(lib().g4_ple_mix(_f(proj), _f(norm_scale), _f(token_ple), rows, width, layers, _f(y)))


def embed(E, vocab, width, ids, n, s, y):
    check(lib().g4_embed(_f(E), vocab, width, _f(ids), n, s, _f(y)))


def argmax(x, n, out):
    check(lib().g4_argmax(_f(x), n, _f(out)))


def fill_random(buf, count, kind, seed, sigma=1.0):
    check(lib().g4_fill_random(_f(buf), count, kind, seed, sigma))


def w4_random(n, k, seed, scale_sigma=0.02, keep_host=False):
    """A W4Linear of random weights generated on the device (q uniform in
    [-7, 7], scales bf16 |N(0,1)| * sigma).  keep_host: also return the
    generated bytes, (packed uint32 [n, k/8], scales uint16 [n, k/32])."""
    packed = Buffer(n * k // 2)
    scales = Buffer(n * (k // 32) * 2)
    fill_random(packed, n * k // 8, RAND_W4_PACKED, seed)
    fill_random(scales, n * (k // 32), RAND_BF16_ABS_NORMAL, seed ^ 0x5CA1E, scale_sigma)
    h = _vp()
    check(lib().g4_w4_load_dev(packed.ptr, scales.ptr, n, k, 32, ctypes.byref(h)))
    host = None
    if keep_host:
        host = (packed.download(np.uint32).reshape(n, k // 8),
                scales.download(np.uint16).reshape(n, k // 32))
    packed.free()
    scales.free()
    lin = W4Linear._from_handle(h.value, n, k)
    return (lin, host) if keep_host else lin


def e2b_config(max_seq):
    c = GemmaConfig()
    check(lib().g4_gemma_e2b_config(max_seq, ctypes.byref(c)))
    return c


class Gemma:
    """Gemma4WebGPU on the device engine (g4_gemma_*)."""

    def __init__(self, cfg):
        h = _vp()
        check(lib().g4_gemma_create(ctypes.byref(cfg), ctypes.byref(h)))
        self.h = h.value
        self.cfg = cfg
        self._keep = []  # borrowed handles must outlive the model

    def set_linear(self, layer, which, w):
        check(lib().g4_gemma_set_linear(self.h, layer, PROJ[which], w.h))
        self._keep.append(w)

    def set_norm(self, layer, which, v):
        v = np.ascontiguousarray(v, dtype=np.float32)
        check(lib().g4_gemma_set_norm(self.h, layer, NORM[which], v.ctypes.data, v.size))

    def set_layer_scalar(self, layer, s):
        check(lib().g4_gemma_set_layer_scalar(self.h, layer, s))

    def set_embedding(self, E):
        check(lib().g4_gemma_set_embedding(self.h, _f(E)))
        self._keep.append(E)

    def set_ple(self, t):
        check(lib().g4_gemma_set_ple(self.h, t.h))
        self._keep.append(t)

    def set_ple_dense(self, rows):
        """Dense BF16 per-layer embeddings [vocab, layers * ple_dim] (a Buffer)."""
        check(lib().g4_gemma_set_ple_dense(self.h, rows.ptr))
        self._keep.append(rows)

    def reset(self):
        check(lib().g4_gemma_reset(self.h))

    def cache_length(self):
        n = _int()
        check(lib().g4_gemma_cache_length(self.h, ctypes.byref(n)))
        return n.value

    def forward(self, ids, start_pos, last_hidden=None):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        check(lib().g4_gemma_forward(self.h, ids.ctypes.data, ids.size, start_pos,
                                     _f(last_hidden)))

    def forward_diag(self, ids, start_pos, last_hidden=None, top_hidden=None, top_ple=None,
                     layer_hidden=None, stage_layer=-1, stages=None):
        """forward(tokenIds, startPos, {diagnostic: true}) read-outs into the
        given device buffers (g4_gemma_forward_diag)."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        check(lib().g4_gemma_forward_diag(self.h, ids.ctypes.data, ids.size, start_pos,
                                          _f(last_hidden), _f(top_hidden), _f(top_ple),
                                          _f(layer_hidden), stage_layer, _f(stages)))

    def diag_stages(self, layer, rows):
        """Float offsets of layer's G4_STAGE_* buffers at `rows` rows."""
        off = (_sz * (STAGES + 1))()
        check(lib().g4_gemma_diag_stages(self.h, layer, rows, off))
        return list(off)

    def logits(self, last_hidden, out):
        check(lib().g4_gemma_logits(self.h, _f(last_hidden), _f(out)))

    def greedy(self, ids, start_pos, logits=None):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        tok = ctypes.c_int32()
        check(lib().g4_gemma_greedy(self.h, ids.ctypes.data, ids.size, start_pos,
                                    ctypes.byref(tok), _f(logits)))
        return tok.value

    def last_hidden(self, out):
        """The final-norm hidden state of the last token run, into `out` (a Buffer)."""
        check(lib().g4_gemma_last_hidden(self.h, _f(out)))

    def decode(self, steps, want_tokens=True):
        out = np.zeros(max(steps, 1), dtype=np.int32)
        check(lib().g4_gemma_decode(self.h, steps, out.ctypes.data if want_tokens else None))
        return out[:steps] if want_tokens else None

    def free(self):
        if self.h:
            check(lib().g4_gemma_free(self.h))
            self.h = None

    def __del__(self):
        try:
            if self.h and _lib is not None:
                _lib.g4_gemma_free(self.h)
        except Exception:
            pass


def exported_symbols():
    return sorted(SIGNATURES)
