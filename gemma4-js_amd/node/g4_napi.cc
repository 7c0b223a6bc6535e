// N-API binding of libg4hip (include/g4hip.h) for Node.
//
// This is the native half of the bridge that replaces the WebGPU buffer and
// dispatch layer of custom-webgpu/gpu-runtime.js: device buffers become
// DeviceBuffer objects, GPUW4Linear weights become W4Weight objects, the PLE
// shard bundle becomes a PleTable, and every non-zero status from the C ABI is
// thrown as a JS Error carrying g4_last_error() - the reference's own error
// convention (synchronous throws for shape/range/capacity errors).
//
// Only plain pointers and sizes cross into the C ABI.  Objects own their
// native handle; destroy() releases it and a finalizer is the backstop.
#include <node_api.h>

#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "g4hip.h"

namespace {

#define NAPI_CALL(env, call)                                                   \
  do {                                                                         \
    napi_status s_ = (call);                                                   \
    if (s_ != napi_ok) {                                                       \
      const napi_extended_error_info *info_ = nullptr;                         \
      napi_get_last_error_info((env), &info_);                                 \
      bool pending_ = false;                                                   \
      napi_is_exception_pending((env), &pending_);                             \
      if (!pending_)                                                           \
        napi_throw_error((env), nullptr,                                       \
                         info_ && info_->error_message ? info_->error_message  \
                                                       : "N-API call failed"); \
      return nullptr;                                                          \
    }                                                                          \
  } while (0)

// Throws the C ABI's error and returns nullptr from the calling function.
#define G4_CALL(env, call)                                      \
  do {                                                          \
    int rc_ = (call);                                           \
    if (rc_ != G4_OK) {                                         \
      char code_[32];                                           \
      snprintf(code_, sizeof code_, "G4_STATUS_%d", rc_);       \
      napi_throw_error((env), code_, g4_last_error());          \
      return nullptr;                                           \
    }                                                           \
  } while (0)

napi_value undefined(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

bool get_args(napi_env env, napi_callback_info info, size_t want, napi_value *argv,
              napi_value *self, void **data = nullptr) {
  size_t argc = want;
  if (napi_get_cb_info(env, info, &argc, argv, self, data) != napi_ok) return false;
  for (size_t i = argc; i < want; ++i) napi_get_undefined(env, &argv[i]);
  return true;
}

// True when v was made by the class whose constructor `ctor` refers to.
bool is_instance(napi_env env, napi_value v, napi_ref ctor) {
  bool ok = false;
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (!ctor || t != napi_object) return false;
  napi_value c;
  napi_get_reference_value(env, ctor, &c);
  napi_instanceof(env, v, c, &ok);
  return ok;
}

napi_ref g_devbuf_ctor = nullptr, g_w4_ctor = nullptr, g_ple_ctor = nullptr,
         g_cmd_ctor = nullptr, g_engine_ctor = nullptr;

bool to_i64(napi_env env, napi_value v, int64_t *out, const char *what) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t != napi_number) {
    char msg[128];
    snprintf(msg, sizeof msg, "%s must be a number", what);
    napi_throw_type_error(env, nullptr, msg);
    return false;
  }
  double d;
  napi_get_value_double(env, v, &d);
  if (d != (double)(int64_t)d) {
    char msg[128];
    snprintf(msg, sizeof msg, "%s must be an integer", what);
    napi_throw_range_error(env, nullptr, msg);
    return false;
  }
  *out = (int64_t)d;
  return true;
}

// An integer argument that the C ABI takes as int: outside the int32 range it
// throws a RangeError instead of wrapping around in the cast.
bool to_int(napi_env env, napi_value v, int64_t *out, const char *what) {
  if (!to_i64(env, v, out, what)) return false;
  if (*out < INT32_MIN || *out > INT32_MAX) {
    char msg[128];
    snprintf(msg, sizeof msg, "%s is out of the int range", what);
    napi_throw_range_error(env, nullptr, msg);
    return false;
  }
  return true;
}

bool to_f64(napi_env env, napi_value v, double *out, const char *what) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t != napi_number) {
    char msg[128];
    snprintf(msg, sizeof msg, "%s must be a number", what);
    napi_throw_type_error(env, nullptr, msg);
    return false;
  }
  napi_get_value_double(env, v, out);
  return true;
}

// Bytes of an ArrayBuffer, TypedArray, DataView or Buffer.
bool host_bytes(napi_env env, napi_value v, void **data, size_t *len, const char *what) {
  bool is;
  napi_is_typedarray(env, v, &is);
  if (is) {
    napi_typedarray_type type;
    size_t n, off;
    napi_value ab;
    void *p;
    napi_get_typedarray_info(env, v, &type, &n, &p, &ab, &off);
    size_t el = 1;
    switch (type) {
      case napi_int16_array: case napi_uint16_array: el = 2; break;
      case napi_int32_array: case napi_uint32_array: case napi_float32_array: el = 4; break;
      case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: el = 8; break;
      default: el = 1;
    }
    *data = p;
    *len = n * el;
    return true;
  }
  napi_is_dataview(env, v, &is);
  if (is) {
    napi_value ab;
    size_t off;
    napi_get_dataview_info(env, v, len, data, &ab, &off);
    return true;
  }
  napi_is_arraybuffer(env, v, &is);
  if (is) {
    napi_get_arraybuffer_info(env, v, data, len);
    return true;
  }
  char msg[128];
  snprintf(msg, sizeof msg, "%s must be an ArrayBuffer or a typed array", what);
  napi_throw_type_error(env, nullptr, msg);
  return false;
}

// ---- DeviceBuffer ------------------------------------------------------------

struct DevBuf {
  void *ptr;
  size_t size;
};

void devbuf_finalize(napi_env, void *data, void *) {
  DevBuf *b = static_cast<DevBuf *>(data);
  if (b->ptr) g4_free(b->ptr);
  delete b;
}

DevBuf *unwrap_buf(napi_env env, napi_value v, const char *what) {
  void *p = nullptr;
  if (!is_instance(env, v, g_devbuf_ctor) || napi_unwrap(env, v, &p) != napi_ok || !p) {
    char msg[128];
    snprintf(msg, sizeof msg, "%s must be a DeviceBuffer", what);
    napi_throw_type_error(env, nullptr, msg);
    return nullptr;
  }
  DevBuf *b = static_cast<DevBuf *>(p);
  if (!b->ptr) {
    char msg[128];
    snprintf(msg, sizeof msg, "%s was destroyed", what);
    napi_throw_error(env, nullptr, msg);
    return nullptr;
  }
  return b;
}

// Device address of byte `off` of a buffer; throws if off > size.
bool buf_at(napi_env env, napi_value v, napi_value off_v, const char *what, void **out) {
  DevBuf *b = unwrap_buf(env, v, what);
  if (!b) return false;
  int64_t off = 0;
  napi_valuetype t;
  napi_typeof(env, off_v, &t);
  if (t != napi_undefined && !to_i64(env, off_v, &off, what)) return false;
  if (off < 0 || (size_t)off > b->size) {
    char msg[160];
    snprintf(msg, sizeof msg, "%s: byte offset %lld outside the %zu-byte buffer", what,
             (long long)off, b->size);
    napi_throw_range_error(env, nullptr, msg);
    return false;
  }
  *out = static_cast<char *>(b->ptr) + off;
  return true;
}

// A DeviceBuffer argument as a device pointer (whole buffer), or null.
bool dev(napi_env env, napi_value v, const char *what, void **out) {
  napi_value no_offset;
  napi_get_undefined(env, &no_offset);
  return buf_at(env, v, no_offset, what, out);
}

bool dev_or_null(napi_env env, napi_value v, const char *what, void **out) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_null || t == napi_undefined) {
    *out = nullptr;
    return true;
  }
  return dev(env, v, what, out);
}

// new DeviceBuffer(size)  - createBuffer (gpu-runtime.js:8-12)
napi_value DevBuf_new(napi_env env, napi_callback_info info) {
  napi_value argv[1], self;
  if (!get_args(env, info, 1, argv, &self)) return nullptr;
  int64_t size;
  if (!to_i64(env, argv[0], &size, "size")) return nullptr;
  if (size < 0) {
    napi_throw_range_error(env, nullptr, "size must be >= 0");
    return nullptr;
  }
  void *p = nullptr;
  G4_CALL(env, g4_alloc((size_t)size, &p));
  DevBuf *b = new DevBuf{p, size < 4 ? 4 : ((size_t)size + 3) & ~size_t(3)};
  if (napi_wrap(env, self, b, devbuf_finalize, nullptr, nullptr) != napi_ok) {
    g4_free(p);
    delete b;
    napi_throw_error(env, nullptr, "napi_wrap failed");
    return nullptr;
  }
  return self;
}

napi_value DevBuf_size(napi_env env, napi_callback_info info) {
  napi_value self;
  if (!get_args(env, info, 0, nullptr, &self)) return nullptr;
  void *p;
  NAPI_CALL(env, napi_unwrap(env, self, &p));
  napi_value r;
  NAPI_CALL(env, napi_create_double(env, (double)static_cast<DevBuf *>(p)->size, &r));
  return r;
}

// buffer.destroy()
napi_value DevBuf_destroy(napi_env env, napi_callback_info info) {
  napi_value self;
  if (!get_args(env, info, 0, nullptr, &self)) return nullptr;
  void *p;
  NAPI_CALL(env, napi_unwrap(env, self, &p));
  DevBuf *b = static_cast<DevBuf *>(p);
  if (b->ptr) {
    void *q = b->ptr;
    b->ptr = nullptr;
    G4_CALL(env, g4_free(q));
  }
  return undefined(env);
}

// buffer.write(bytes, byteOffset = 0)  - queue.writeBuffer
napi_value DevBuf_write(napi_env env, napi_callback_info info) {
  napi_value argv[2], self;
  if (!get_args(env, info, 2, argv, &self)) return nullptr;
  void *dst;
  if (!buf_at(env, self, argv[1], "buffer", &dst)) return nullptr;
  void *src;
  size_t n;
  if (!host_bytes(env, argv[0], &src, &n, "data")) return nullptr;
  G4_CALL(env, g4_upload(dst, 0, src, n));
  return undefined(env);
}

// buffer.read(byteOffset, byteLength) -> ArrayBuffer  (waits for the queue)
napi_value DevBuf_read(napi_env env, napi_callback_info info) {
  napi_value argv[2], self;
  if (!get_args(env, info, 2, argv, &self)) return nullptr;
  void *src;
  if (!buf_at(env, self, argv[0], "buffer", &src)) return nullptr;
  int64_t n;
  if (!to_i64(env, argv[1], &n, "byteLength")) return nullptr;
  if (n < 0) {
    napi_throw_range_error(env, nullptr, "byteLength must be >= 0");
    return nullptr;
  }
  void *data;
  napi_value ab;
  NAPI_CALL(env, napi_create_arraybuffer(env, (size_t)n, &data, &ab));
  G4_CALL(env, g4_download(src, 0, data, (size_t)n));
  return ab;
}

// ---- W4Weight (GPUW4Linear) ----------------------------------------------------

struct W4 {
  g4_w4 *h;
  int out_dim, in_dim, group;
};

void w4_finalize(napi_env, void *data, void *) {
  W4 *w = static_cast<W4 *>(data);
  if (w->h) g4_w4_free(w->h);
  delete w;
}

W4 *unwrap_w4(napi_env env, napi_value self) {
  void *p = nullptr;
  if (!is_instance(env, self, g_w4_ctor) || napi_unwrap(env, self, &p) != napi_ok || !p) {
    napi_throw_type_error(env, nullptr, "not a W4Weight");
    return nullptr;
  }
  W4 *w = static_cast<W4 *>(p);
  if (!w->h) {
    napi_throw_error(env, nullptr, "W4Weight was disposed");
    return nullptr;
  }
  return w;
}

// new W4Weight(packedBytes, scaleBytes, outDim, inDim, groupSize): host bytes
// (ArrayBuffer / typed arrays), or two DeviceBuffers already holding the same
// layouts on the device.
napi_value W4_new(napi_env env, napi_callback_info info) {
  napi_value argv[5], self;
  if (!get_args(env, info, 5, argv, &self)) return nullptr;
  int64_t out_dim, in_dim, group;
  if (!to_int(env, argv[2], &out_dim, "outDim") || !to_int(env, argv[3], &in_dim, "inDim") ||
      !to_int(env, argv[4], &group, "groupSize"))
    return nullptr;
  if (is_instance(env, argv[0], g_devbuf_ctor)) {
    void *pk, *sc;
    if (!dev(env, argv[0], "packed", &pk) || !dev(env, argv[1], "scales", &sc)) return nullptr;
    g4_w4 *h = nullptr;
    G4_CALL(env, g4_w4_load_dev(pk, sc, (int)out_dim, (int)in_dim, (int)group, &h));
    W4 *w = new W4{h, (int)out_dim, (int)in_dim, (int)group};
    if (napi_wrap(env, self, w, w4_finalize, nullptr, nullptr) != napi_ok) {
      g4_w4_free(h);
      delete w;
      napi_throw_error(env, nullptr, "napi_wrap failed");
      return nullptr;
    }
    return self;
  }
  void *pk, *sc;
  size_t npk, nsc;
  if (!host_bytes(env, argv[0], &pk, &npk, "packed")) return nullptr;
  if (!host_bytes(env, argv[1], &sc, &nsc, "scales")) return nullptr;
  if (out_dim <= 0 || in_dim <= 0 || group <= 0 || in_dim % 8 || in_dim % group) {
    // the C ABI reports the precise message
  } else if (npk != (size_t)(out_dim * (in_dim / 8) * 4)) {
    napi_throw_error(env, nullptr, "packed weight length mismatch");
    return nullptr;
  } else if (nsc != (size_t)(out_dim * (in_dim / group) * 2)) {
    napi_throw_error(env, nullptr, "scale length mismatch");
    return nullptr;
  }
  g4_w4 *h = nullptr;
  G4_CALL(env, g4_w4_load(pk, sc, (int)out_dim, (int)in_dim, (int)group, &h));
  W4 *w = new W4{h, (int)out_dim, (int)in_dim, (int)group};
  if (napi_wrap(env, self, w, w4_finalize, nullptr, nullptr) != napi_ok) {
    g4_w4_free(h);
    delete w;
    napi_throw_error(env, nullptr, "napi_wrap failed");
    return nullptr;
  }
  return self;
}

// w.linear(x, xDtype, rows, y, yDtype, xByteOffset = 0, yByteOffset = 0)
napi_value W4_linear(napi_env env, napi_callback_info info) {
  napi_value argv[7], self;
  if (!get_args(env, info, 7, argv, &self)) return nullptr;
  W4 *w = unwrap_w4(env, self);
  if (!w) return nullptr;
  void *x, *y;
  if (!buf_at(env, argv[0], argv[5], "x", &x)) return nullptr;
  if (!buf_at(env, argv[3], argv[6], "y", &y)) return nullptr;
  int64_t xd, rows, yd;
  if (!to_int(env, argv[1], &xd, "xDtype") || !to_int(env, argv[2], &rows, "rows") ||
      !to_int(env, argv[4], &yd, "yDtype"))
    return nullptr;
  G4_CALL(env, g4_w4_linear(w->h, x, (int)xd, (int)rows, y, (int)yd));
  return undefined(env);
}

// linearMulti([w...], x, xDtype, rows, [y...], yDtype): g4_w4_linear_multi,
// every weight over the same x, y[i] receiving weight i's output.
napi_value F_linearMulti(napi_env env, napi_callback_info info) {
  napi_value argv[6];
  if (!get_args(env, info, 6, argv, nullptr)) return nullptr;
  bool wa = false, ya = false;
  napi_is_array(env, argv[0], &wa);
  napi_is_array(env, argv[4], &ya);
  if (!wa || !ya) {
    napi_throw_type_error(env, nullptr, "linearMulti: weights and outputs must be arrays");
    return nullptr;
  }
  uint32_t n = 0, ny = 0;
  napi_get_array_length(env, argv[0], &n);
  napi_get_array_length(env, argv[4], &ny);
  if (n != ny || n == 0 || n > 3) {
    napi_throw_range_error(env, nullptr,
                           "linearMulti: 1..3 weights and one output buffer per weight");
    return nullptr;
  }
  const g4_w4 *ws[3];
  void *ys[3];
  for (uint32_t i = 0; i < n; ++i) {
    napi_value e;
    napi_get_element(env, argv[0], i, &e);
    W4 *w = unwrap_w4(env, e);
    if (!w) return nullptr;
    ws[i] = w->h;
    napi_get_element(env, argv[4], i, &e);
    if (!dev(env, e, "y", &ys[i])) return nullptr;
  }
  void *x;
  if (!dev(env, argv[1], "x", &x)) return nullptr;
  int64_t xd, rows, yd;
  if (!to_int(env, argv[2], &xd, "xDtype") || !to_int(env, argv[3], &rows, "rows") ||
      !to_int(env, argv[5], &yd, "yDtype"))
    return nullptr;
  G4_CALL(env, g4_w4_linear_multi(ws, (int)n, x, (int)xd, (int)rows, ys, (int)yd));
  return undefined(env);
}

// w.dequant(rowStart, rowCount, out, dtype, outByteOffset = 0)
napi_value W4_dequant(napi_env env, napi_callback_info info) {
  napi_value argv[5], self;
  if (!get_args(env, info, 5, argv, &self)) return nullptr;
  W4 *w = unwrap_w4(env, self);
  if (!w) return nullptr;
  int64_t r0, rc, dt;
  if (!to_int(env, argv[0], &r0, "rowStart") || !to_int(env, argv[1], &rc, "rowCount") ||
      !to_int(env, argv[3], &dt, "dtype"))
    return nullptr;
  void *out;
  if (!buf_at(env, argv[2], argv[4], "out", &out)) return nullptr;
  G4_CALL(env, g4_w4_dequant(w->h, (int)r0, (int)rc, out, (int)dt));
  return undefined(env);
}

napi_value W4_dispose(napi_env env, napi_callback_info info) {
  napi_value self;
  if (!get_args(env, info, 0, nullptr, &self)) return nullptr;
  void *p;
  NAPI_CALL(env, napi_unwrap(env, self, &p));
  W4 *w = static_cast<W4 *>(p);
  if (w->h) {
    g4_w4 *h = w->h;
    w->h = nullptr;
    G4_CALL(env, g4_w4_free(h));
  }
  return undefined(env);
}

napi_value W4_info(napi_env env, napi_callback_info info) {
  napi_value self;
  if (!get_args(env, info, 0, nullptr, &self)) return nullptr;
  W4 *w = unwrap_w4(env, self);
  if (!w) return nullptr;
  int n, k, g;
  size_t bytes;
  G4_CALL(env, g4_w4_info(w->h, &n, &k, &g, &bytes));
  napi_value o, v;
  NAPI_CALL(env, napi_create_object(env, &o));
  napi_create_int32(env, n, &v);
  napi_set_named_property(env, o, "outDim", v);
  napi_create_int32(env, k, &v);
  napi_set_named_property(env, o, "inDim", v);
  napi_create_int32(env, g, &v);
  napi_set_named_property(env, o, "groupSize", v);
  napi_create_double(env, (double)bytes, &v);
  napi_set_named_property(env, o, "deviceBytes", v);
  return o;
}

// ---- PleTable -----------------------------------------------------------------

struct Ple {
  g4_ple *h;
};

void ple_finalize(napi_env, void *data, void *) {
  Ple *t = static_cast<Ple *>(data);
  if (t->h) g4_ple_free(t->h);
  delete t;
}

Ple *unwrap_ple(napi_env env, napi_value self) {
  void *p = nullptr;
  if (!is_instance(env, self, g_ple_ctor) || napi_unwrap(env, self, &p) != napi_ok || !p) {
    napi_throw_type_error(env, nullptr, "not a PleTable");
    return nullptr;
  }
  Ple *t = static_cast<Ple *>(p);
  if (!t->h) {
    napi_throw_error(env, nullptr, "PleTable was disposed");
    return nullptr;
  }
  return t;
}

// new PleTable(vocab, width, groupSize, rowsPerShard)
napi_value Ple_new(napi_env env, napi_callback_info info) {
  napi_value argv[4], self;
  if (!get_args(env, info, 4, argv, &self)) return nullptr;
  int64_t vocab, width, group, rps;
  if (!to_int(env, argv[0], &vocab, "vocab") || !to_int(env, argv[1], &width, "width") ||
      !to_int(env, argv[2], &group, "groupSize") || !to_int(env, argv[3], &rps, "rowsPerShard"))
    return nullptr;
  g4_ple *h = nullptr;
  G4_CALL(env, g4_ple_create((int)vocab, (int)width, (int)group, (int)rps, &h));
  Ple *t = new Ple{h};
  if (napi_wrap(env, self, t, ple_finalize, nullptr, nullptr) != napi_ok) {
    g4_ple_free(h);
    delete t;
    napi_throw_error(env, nullptr, "napi_wrap failed");
    return nullptr;
  }
  return self;
}

// t.shardBytes(i) -> number
napi_value Ple_shardBytes(napi_env env, napi_callback_info info) {
  napi_value argv[1], self;
  if (!get_args(env, info, 1, argv, &self)) return nullptr;
  Ple *t = unwrap_ple(env, self);
  if (!t) return nullptr;
  int64_t i;
  if (!to_int(env, argv[0], &i, "shard")) return nullptr;
  size_t bytes;
  int ns;
  G4_CALL(env, g4_ple_shard_bytes(t->h, (int)i, &ns, &bytes));
  napi_value r;
  NAPI_CALL(env, napi_create_double(env, (double)bytes, &r));
  return r;
}

// t.uploadShard(i, bytes)
napi_value Ple_uploadShard(napi_env env, napi_callback_info info) {
  napi_value argv[2], self;
  if (!get_args(env, info, 2, argv, &self)) return nullptr;
  Ple *t = unwrap_ple(env, self);
  if (!t) return nullptr;
  int64_t i;
  if (!to_int(env, argv[0], &i, "shard")) return nullptr;
  void *p;
  size_t n;
  if (is_instance(env, argv[1], g_devbuf_ctor)) {  // the shard's bytes on the device
    DevBuf *b = unwrap_buf(env, argv[1], "shard bytes");
    if (!b) return nullptr;
    size_t want = 0;
    int nshards = 0;
    G4_CALL(env, g4_ple_shard_bytes(t->h, (int)i, &nshards, &want));
    if (want > b->size) {
      napi_throw_range_error(env, nullptr, "shard bytes: the DeviceBuffer is smaller than the shard");
      return nullptr;
    }
    G4_CALL(env, g4_ple_upload_shard_dev(t->h, (int)i, b->ptr, want));
    return undefined(env);
  }
  if (!host_bytes(env, argv[1], &p, &n, "shard bytes")) return nullptr;
  G4_CALL(env, g4_ple_upload_shard(t->h, (int)i, p, n));
  return undefined(env);
}

// t.gather(idsInt32Array, out, dtype, outByteOffset = 0)
napi_value Ple_gather(napi_env env, napi_callback_info info) {
  napi_value argv[4], self;
  if (!get_args(env, info, 4, argv, &self)) return nullptr;
  Ple *t = unwrap_ple(env, self);
  if (!t) return nullptr;
  bool is;
  napi_is_typedarray(env, argv[0], &is);
  napi_typedarray_type type = napi_uint8_array;
  size_t n = 0;
  void *ids = nullptr;
  if (is) {
    napi_value ab;
    size_t off;
    napi_get_typedarray_info(env, argv[0], &type, &n, &ids, &ab, &off);
  }
  if (!is || type != napi_int32_array) {
    napi_throw_type_error(env, nullptr, "ids must be an Int32Array");
    return nullptr;
  }
  void *out;
  if (!buf_at(env, argv[1], argv[3], "out", &out)) return nullptr;
  int64_t dt;
  if (!to_int(env, argv[2], &dt, "dtype")) return nullptr;
  G4_CALL(env, g4_ple_gather(t->h, static_cast<const int32_t *>(ids), (int)n, out, (int)dt));
  return undefined(env);
}

// t.gatherDev(idsBuffer, n, out, dtype, idsByteOffset = 0, outByteOffset = 0)
napi_value Ple_gatherDev(napi_env env, napi_callback_info info) {
  napi_value argv[6], self;
  if (!get_args(env, info, 6, argv, &self)) return nullptr;
  Ple *t = unwrap_ple(env, self);
  if (!t) return nullptr;
  void *ids, *out;
  if (!buf_at(env, argv[0], argv[4], "ids", &ids)) return nullptr;
  if (!buf_at(env, argv[2], argv[5], "out", &out)) return nullptr;
  int64_t n, dt;
  if (!to_int(env, argv[1], &n, "n") || !to_int(env, argv[3], &dt, "dtype")) return nullptr;
  G4_CALL(env, g4_ple_gather_dev(t->h, static_cast<const int32_t *>(ids), (int)n, out, (int)dt));
  return undefined(env);
}

napi_value Ple_dispose(napi_env env, napi_callback_info info) {
  napi_value self;
  if (!get_args(env, info, 0, nullptr, &self)) return nullptr;
  void *p;
  NAPI_CALL(env, napi_unwrap(env, self, &p));
  Ple *t = static_cast<Ple *>(p);
  if (t->h) {
    g4_ple *h = t->h;
    t->h = nullptr;
    G4_CALL(env, g4_ple_free(h));
  }
  return undefined(env);
}

// ---- CommandBuffer (a finished encoder) ----------------------------------------------

struct Cmd {
  g4_cmdbuf *h;
};

void cmd_finalize(napi_env, void *data, void *) {
  Cmd *c = static_cast<Cmd *>(data);
  if (c->h) g4_cmdbuf_free(c->h);
  delete c;
}

napi_value Cmd_new(napi_env env, napi_callback_info info) {
  napi_value self;
  if (!get_args(env, info, 0, nullptr, &self)) return nullptr;
  Cmd *c = new Cmd{nullptr};
  if (napi_wrap(env, self, c, cmd_finalize, nullptr, nullptr) != napi_ok) {
    delete c;
    napi_throw_error(env, nullptr, "napi_wrap failed");
    return nullptr;
  }
  return self;
}

napi_value Cmd_submit(napi_env env, napi_callback_info info) {
  napi_value self;
  if (!get_args(env, info, 0, nullptr, &self)) return nullptr;
  void *p = nullptr;
  if (!is_instance(env, self, g_cmd_ctor) || napi_unwrap(env, self, &p) != napi_ok || !p) {
    napi_throw_type_error(env, nullptr, "not a CommandBuffer");
    return nullptr;
  }
  Cmd *c = static_cast<Cmd *>(p);
  if (!c->h) {
    napi_throw_error(env, nullptr, "CommandBuffer is empty or destroyed");
    return nullptr;
  }
  G4_CALL(env, g4_submit(c->h));
  return undefined(env);
}

napi_value Cmd_destroy(napi_env env, napi_callback_info info) {
  napi_value self;
  if (!get_args(env, info, 0, nullptr, &self)) return nullptr;
  void *p = nullptr;
  if (!is_instance(env, self, g_cmd_ctor) || napi_unwrap(env, self, &p) != napi_ok || !p) {
    napi_throw_type_error(env, nullptr, "not a CommandBuffer");
    return nullptr;
  }
  Cmd *c = static_cast<Cmd *>(p);
  if (c->h) {
    g4_cmdbuf *h = c->h;
    c->h = nullptr;
    G4_CALL(env, g4_cmdbuf_free(h));
  }
  return undefined(env);
}

// ---- free functions ------------------------------------------------------------

napi_value F_init(napi_env env, napi_callback_info info) {
  napi_value argv[1], self;
  if (!get_args(env, info, 1, argv, &self)) return nullptr;
  int64_t dev = 0;
  napi_valuetype t;
  napi_typeof(env, argv[0], &t);
  if (t != napi_undefined && !to_int(env, argv[0], &dev, "device")) return nullptr;
  G4_CALL(env, g4_init((int)dev));
  return undefined(env);
}

napi_value F_deviceInfo(napi_env env, napi_callback_info) {
  char name[256];
  int cu, clk;
  size_t hbm;
  G4_CALL(env, g4_device_info(name, sizeof name, &cu, &hbm, &clk));
  napi_value o, v;
  NAPI_CALL(env, napi_create_object(env, &o));
  napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &v);
  napi_set_named_property(env, o, "name", v);
  napi_create_int32(env, cu, &v);
  napi_set_named_property(env, o, "cuCount", v);
  napi_create_double(env, (double)hbm, &v);
  napi_set_named_property(env, o, "hbmBytes", v);
  napi_create_int32(env, clk, &v);
  napi_set_named_property(env, o, "clockKHz", v);
  return o;
}

napi_value F_sync(napi_env env, napi_callback_info) {
  G4_CALL(env, g4_sync());
  return undefined(env);
}

// copy(dst, dstOffset, src, srcOffset, byteLength)  - copyBufferToBuffer
napi_value F_copy(napi_env env, napi_callback_info info) {
  napi_value argv[5], self;
  if (!get_args(env, info, 5, argv, &self)) return nullptr;
  void *dst, *src;
  if (!buf_at(env, argv[0], argv[1], "dst", &dst)) return nullptr;
  if (!buf_at(env, argv[2], argv[3], "src", &src)) return nullptr;
  int64_t n;
  if (!to_i64(env, argv[4], &n, "byteLength")) return nullptr;
  if (n < 0) {
    napi_throw_range_error(env, nullptr, "byteLength must be >= 0");
    return nullptr;
  }
  G4_CALL(env, g4_copy(dst, 0, src, 0, (size_t)n));
  return undefined(env);
}

// bf16Head(x, E, rows, inDim, out, scale, softcap, eByteOffset = 0, outByteOffset = 0)
napi_value F_bf16Head(napi_env env, napi_callback_info info) {
  napi_value argv[9], self;
  if (!get_args(env, info, 9, argv, &self)) return nullptr;
  void *x, *E, *out;
  napi_value zero;
  napi_create_int32(env, 0, &zero);
  if (!buf_at(env, argv[0], zero, "x", &x)) return nullptr;
  if (!buf_at(env, argv[1], argv[7], "E", &E)) return nullptr;
  if (!buf_at(env, argv[4], argv[8], "out", &out)) return nullptr;
  int64_t rows, k;
  double scale, softcap;
  if (!to_int(env, argv[2], &rows, "rows") || !to_int(env, argv[3], &k, "inDim") ||
      !to_f64(env, argv[5], &scale, "scale") || !to_f64(env, argv[6], &softcap, "softcap"))
    return nullptr;
  G4_CALL(env, g4_bf16_head(static_cast<const float *>(x), E, (int)rows, (int)k,
                            static_cast<float *>(out), (float)scale, (float)softcap));
  return undefined(env);
}

napi_value F_encoderBegin(napi_env env, napi_callback_info) {
  G4_CALL(env, g4_encoder_begin());
  return undefined(env);
}

// encoderFinish() -> CommandBuffer
napi_value F_encoderFinish(napi_env env, napi_callback_info) {
  g4_cmdbuf *h = nullptr;
  G4_CALL(env, g4_encoder_finish(&h));
  napi_value ctor, obj;
  NAPI_CALL(env, napi_get_reference_value(env, g_cmd_ctor, &ctor));
  NAPI_CALL(env, napi_new_instance(env, ctor, 0, nullptr, &obj));
  void *p;
  NAPI_CALL(env, napi_unwrap(env, obj, &p));
  static_cast<Cmd *>(p)->h = h;
  return obj;
}

// timeMs(fn): runs fn() between two stream events and returns the GPU ms.
napi_value F_timeMs(napi_env env, napi_callback_info info) {
  napi_value argv[1], self;
  if (!get_args(env, info, 1, argv, &self)) return nullptr;
  void *a = nullptr, *b = nullptr;
  G4_CALL(env, g4_event_create(&a));
  int rc = g4_event_create(&b);
  if (rc) {
    g4_event_destroy(a);
    G4_CALL(env, rc);
  }
  napi_value r = nullptr;
  float ms = 0.f;
  rc = g4_event_record(a);
  if (!rc) {
    napi_value global, res;
    napi_get_global(env, &global);
    if (napi_call_function(env, global, argv[0], 0, nullptr, &res) != napi_ok) {
      g4_event_destroy(a);
      g4_event_destroy(b);
      return nullptr;  // the JS exception propagates
    }
    rc = g4_event_record(b);
  }
  if (!rc) rc = g4_event_elapsed_ms(a, b, &ms);
  g4_event_destroy(a);
  g4_event_destroy(b);
  G4_CALL(env, rc);
  NAPI_CALL(env, napi_create_double(env, ms, &r));
  return r;
}

// ---- remaining GPUOps (gpu-runtime.js:1325-1369) ----------------------------------
// Each takes DeviceBuffers (whole-buffer pointers) and plain numbers and
// enqueues one C-ABI op; the JS GPUOps allocates the outputs.

bool ints(napi_env env, napi_value *argv, const int *idx, int64_t *out, int n,
          const char *const *names) {
  for (int i = 0; i < n; ++i)
    if (!to_int(env, argv[idx[i]], &out[i], names[i])) return false;
  return true;
}

// rms(x, rows, width, scale | null, eps, y)
napi_value F_rms(napi_env env, napi_callback_info info) {
  napi_value a[6], self;
  if (!get_args(env, info, 6, a, &self)) return nullptr;
  void *x, *sc, *y;
  int64_t rows, width;
  double eps;
  if (!dev(env, a[0], "x", &x) || !to_int(env, a[1], &rows, "rows") ||
      !to_int(env, a[2], &width, "width") || !dev_or_null(env, a[3], "scale", &sc) ||
      !to_f64(env, a[4], &eps, "eps") || !dev(env, a[5], "y", &y))
    return nullptr;
  G4_CALL(env, g4_rms((const float *)x, (int)rows, (int)width, (const float *)sc, (float)eps,
                      (float *)y));
  return undefined(env);
}

// addScale(a, b, n, scale, y)
napi_value F_addScale(napi_env env, napi_callback_info info) {
  napi_value a[5], self;
  if (!get_args(env, info, 5, a, &self)) return nullptr;
  void *x, *z, *y;
  int64_t n;
  double s;
  if (!dev(env, a[0], "a", &x) || !dev(env, a[1], "b", &z) || !to_i64(env, a[2], &n, "n") ||
      !to_f64(env, a[3], &s, "scale") || !dev(env, a[4], "y", &y))
    return nullptr;
  G4_CALL(env, g4_add_scale((const float *)x, (const float *)z, (size_t)n, (float)s, (float *)y));
  return undefined(env);
}

// scale(a, n, s, y)
napi_value F_scale(napi_env env, napi_callback_info info) {
  napi_value a[4], self;
  if (!get_args(env, info, 4, a, &self)) return nullptr;
  void *x, *y;
  int64_t n;
  double s;
  if (!dev(env, a[0], "a", &x) || !to_i64(env, a[1], &n, "n") ||
      !to_f64(env, a[2], &s, "scale") || !dev(env, a[3], "y", &y))
    return nullptr;
  G4_CALL(env, g4_scale((const float *)x, (size_t)n, (float)s, (float *)y));
  return undefined(env);
}

// geluMul(gate, up, n, y)
napi_value F_geluMul(napi_env env, napi_callback_info info) {
  napi_value a[4], self;
  if (!get_args(env, info, 4, a, &self)) return nullptr;
  void *g, *u, *y;
  int64_t n;
  if (!dev(env, a[0], "gate", &g) || !dev(env, a[1], "up", &u) || !to_i64(env, a[2], &n, "n") ||
      !dev(env, a[3], "y", &y))
    return nullptr;
  G4_CALL(env, g4_gelu_mul((const float *)g, (const float *)u, (size_t)n, (float *)y));
  return undefined(env);
}

// geluPle(gate, ple, rows, layer, width, layers, y)
napi_value F_geluPle(napi_env env, napi_callback_info info) {
  napi_value a[7], self;
  if (!get_args(env, info, 7, a, &self)) return nullptr;
  void *g, *p, *y;
  int64_t v[4];
  static const int idx[4] = {2, 3, 4, 5};
  static const char *const names[4] = {"rows", "layer", "width", "layers"};
  if (!dev(env, a[0], "gate", &g) || !dev(env, a[1], "ple", &p) || !ints(env, a, idx, v, 4, names) ||
      !dev(env, a[6], "y", &y))
    return nullptr;
  G4_CALL(env, g4_gelu_ple((const float *)g, (const float *)p, (int)v[0], (int)v[1], (int)v[2],
                           (int)v[3], (float *)y));
  return undefined(env);
}

// normRope(x, rows, heads, hd, pos0, scale, ropeAngles, base, eps, y)
napi_value F_normRope(napi_env env, napi_callback_info info) {
  napi_value a[10], self;
  if (!get_args(env, info, 10, a, &self)) return nullptr;
  void *x, *sc, *y;
  int64_t v[4], angles;
  double base, eps;
  static const int idx[4] = {1, 2, 3, 4};
  static const char *const names[4] = {"rows", "heads", "hd", "pos0"};
  if (!dev(env, a[0], "x", &x) || !ints(env, a, idx, v, 4, names) ||
      !dev(env, a[5], "scale", &sc) || !to_int(env, a[6], &angles, "ropeAngles") ||
      !to_f64(env, a[7], &base, "base") || !to_f64(env, a[8], &eps, "eps") ||
      !dev(env, a[9], "y", &y))
    return nullptr;
  G4_CALL(env, g4_norm_rope((const float *)x, (int)v[0], (int)v[1], (int)v[2], (int)v[3],
                            (const float *)sc, (int)angles, (float)base, (float)eps, (float *)y));
  return undefined(env);
}

// attention(q, k, v, qrows, heads, hd, keylen, qpos0, sliding, window, y)
napi_value F_attention(napi_env env, napi_callback_info info) {
  napi_value a[11], self;
  if (!get_args(env, info, 11, a, &self)) return nullptr;
  void *q, *k, *vv, *y;
  int64_t v[7];
  static const int idx[7] = {3, 4, 5, 6, 7, 8, 9};
  static const char *const names[7] = {"qrows", "heads", "hd", "keylen", "qpos0", "sliding",
                                       "window"};
  if (!dev(env, a[0], "q", &q) || !dev(env, a[1], "k", &k) || !dev(env, a[2], "v", &vv) ||
      !ints(env, a, idx, v, 7, names) || !dev(env, a[10], "y", &y))
    return nullptr;
  G4_CALL(env, g4_attention((const float *)q, (const float *)k, (const float *)vv, (int)v[0],
                            (int)v[1], (int)v[2], (int)v[3], (int)v[4], (int)v[5], (int)v[6],
                            (float *)y));
  return undefined(env);
}

// pleMix(proj, normScale, tokenPle, rows, width, layers, y)
napi_value F_pleMix(napi_env env, napi_callback_info info) {
  napi_value a[7], self;
  if (!get_args(env, info, 7, a, &self)) return nullptr;
  void *p, *ns, *tp, *y;
  int64_t v[3];
  static const int idx[3] = {3, 4, 5};
  static const char *const names[3] = {"rows", "width", "layers"};
  if (!dev(env, a[0], "proj", &p) || !dev(env, a[1], "normScale", &ns) ||
      !dev(env, a[2], "tokenPle", &tp) || !ints(env, a, idx, v, 3, names) ||
      !dev(env, a[6], "y", &y))
    return nullptr;
  G4_CALL(env, g4_ple_mix((const float *)p, (const float *)ns, (const float *)tp, (int)v[0],
                          (int)v[1], (int)v[2], (float *)y));
  return undefined(env);
}

// fillRandom(buffer, count, kind, seed, sigma = 1, byteOffset = 0): device-side
// synthetic data (g4_fill_random kinds)
napi_value F_fillRandom(napi_env env, napi_callback_info info) {
  napi_value a[6], self;
  if (!get_args(env, info, 6, a, &self)) return nullptr;
  void *p;
  int64_t count, kind, seed;
  double sigma = 1.0;
  napi_valuetype t;
  if (!buf_at(env, a[0], a[5], "buffer", &p) || !to_i64(env, a[1], &count, "count") ||
      !to_int(env, a[2], &kind, "kind") || !to_i64(env, a[3], &seed, "seed"))
    return nullptr;
  napi_typeof(env, a[4], &t);
  if (t != napi_undefined && !to_f64(env, a[4], &sigma, "sigma")) return nullptr;
  if (count < 0 || seed < 0) {
    napi_throw_range_error(env, nullptr, "fillRandom: count and seed must be non-negative");
    return nullptr;
  }
  G4_CALL(env, g4_fill_random(p, (size_t)count, (int)kind, (uint64_t)seed, (float)sigma));
  return undefined(env);
}

// argmax(x, n, out): out[0] = first index of the largest finite x, or -1
napi_value F_argmax(napi_env env, napi_callback_info info) {
  napi_value a[3], self;
  if (!get_args(env, info, 3, a, &self)) return nullptr;
  void *x, *o;
  int64_t n;
  if (!dev(env, a[0], "x", &x) || !to_int(env, a[1], &n, "n") || !dev(env, a[2], "out", &o))
    return nullptr;
  G4_CALL(env, g4_argmax((const float *)x, (int)n, (int32_t *)o));
  return undefined(env);
}

// ---- GemmaEngine (g4_gemma_*) ---------------------------------------------------
// The native decoder engine behind Gemma4WebGPU's load/forward/logits/greedy
// surface (gemma4-webgpu.js:139-481), plus decode(steps) on a recorded step.
// The engine borrows the W4Weight / PleTable / DeviceBuffer objects it is
// given; the JS object holds references to them so they outlive it.

struct Engine {
  g4_gemma *h;
};

void engine_finalize(napi_env, void *data, void *) {
  Engine *e = static_cast<Engine *>(data);
  if (e->h) g4_gemma_free(e->h);
  delete e;
}

Engine *unwrap_engine(napi_env env, napi_value self) {
  void *p = nullptr;
  if (!is_instance(env, self, g_engine_ctor) || napi_unwrap(env, self, &p) != napi_ok || !p) {
    napi_throw_type_error(env, nullptr, "not a GemmaEngine");
    return nullptr;
  }
  Engine *e = static_cast<Engine *>(p);
  if (!e->h) {
    napi_throw_error(env, nullptr, "GemmaEngine was disposed");
    return nullptr;
  }
  return e;
}

bool get_prop(napi_env env, napi_value obj, const char *name, napi_value *out) {
  bool has = false;
  napi_has_named_property(env, obj, name, &has);
  if (!has) {
    char msg[128];
    snprintf(msg, sizeof msg, "config.%s is missing", name);
    napi_throw_type_error(env, nullptr, msg);
    return false;
  }
  return napi_get_named_property(env, obj, name, out) == napi_ok;
}

bool prop_int(napi_env env, napi_value obj, const char *name, int *out) {
  napi_value v;
  int64_t x;
  if (!get_prop(env, obj, name, &v) || !to_i64(env, v, &x, name)) return false;
  if (x < INT32_MIN || x > INT32_MAX) {
    napi_throw_range_error(env, nullptr, "config value out of int range");
    return false;
  }
  *out = (int)x;
  return true;
}

bool prop_float(napi_env env, napi_value obj, const char *name, float *out) {
  napi_value v;
  double x;
  if (!get_prop(env, obj, name, &v) || !to_f64(env, v, &x, name)) return false;
  *out = (float)x;
  return true;
}

// Token ids from an Array of numbers or an Int32Array / Uint32Array.
bool id_list(napi_env env, napi_value v, std::vector<int32_t> *ids) {
  bool is = false;
  napi_is_typedarray(env, v, &is);
  if (is) {
    napi_typedarray_type type;
    size_t n, off;
    napi_value ab;
    void *p;
    napi_get_typedarray_info(env, v, &type, &n, &p, &ab, &off);
    if (type != napi_int32_array && type != napi_uint32_array) {
      napi_throw_type_error(env, nullptr, "token ids must be an Array, Int32Array or Uint32Array");
      return false;
    }
    const int32_t *q = static_cast<const int32_t *>(p);
    ids->assign(q, q + n);
    return true;
  }
  napi_is_array(env, v, &is);
  if (!is) {
    napi_throw_type_error(env, nullptr, "token ids must be an Array, Int32Array or Uint32Array");
    return false;
  }
  uint32_t n = 0;
  napi_get_array_length(env, v, &n);
  ids->resize(n);
  for (uint32_t i = 0; i < n; ++i) {
    napi_value x;
    int64_t id;
    napi_get_element(env, v, i, &x);
    if (!to_i64(env, x, &id, "token id")) return false;
    if (id < INT32_MIN || id > INT32_MAX) {
      napi_throw_range_error(env, nullptr, "token id out of int range");
      return false;
    }
    (*ids)[i] = (int32_t)id;
  }
  return true;
}

napi_value config_object(napi_env env, const g4_gemma_config &c) {
  napi_value o, v, layers;
  NAPI_CALL(env, napi_create_object(env, &o));
#define SET_NUM(key, val)                                \
  NAPI_CALL(env, napi_create_double(env, (double)(val), &v)); \
  NAPI_CALL(env, napi_set_named_property(env, o, key, v));
  SET_NUM("hidden", c.hidden);
  SET_NUM("heads", c.heads);
  SET_NUM("pleDim", c.ple_dim);
  SET_NUM("vocab", c.vocab);
  SET_NUM("maxSeq", c.max_seq);
  SET_NUM("window", c.window);
  SET_NUM("eps", c.eps);
  SET_NUM("softcap", c.softcap);
#undef SET_NUM
  NAPI_CALL(env, napi_create_array_with_length(env, c.layers, &layers));
  for (int i = 0; i < c.layers; ++i) {
    napi_value L;
    NAPI_CALL(env, napi_create_object(env, &L));
#define SET_L(key, val)                                  \
  NAPI_CALL(env, napi_create_double(env, (double)(val), &v)); \
  NAPI_CALL(env, napi_set_named_property(env, L, key, v));
    SET_L("headDim", c.head_dim[i]);
    SET_L("intermediate", c.intermediate[i]);
    SET_L("full", c.full[i]);
    SET_L("kvSource", c.kv_source[i]);
    SET_L("ropeBase", c.rope_base[i]);
    SET_L("ropeProp", c.rope_prop[i]);
#undef SET_L
    NAPI_CALL(env, napi_set_element(env, layers, i, L));
  }
  NAPI_CALL(env, napi_set_named_property(env, o, "layers", layers));
  return o;
}

// e2bConfig(maxSeq) -> the Gemma-4-E2B geometry (gemma4-webgpu.js:12, 65-77)
napi_value F_e2bConfig(napi_env env, napi_callback_info info) {
  napi_value a[1], self;
  if (!get_args(env, info, 1, a, &self)) return nullptr;
  int64_t max_seq;
  if (!to_int(env, a[0], &max_seq, "maxSeq")) return nullptr;
  g4_gemma_config c;
  G4_CALL(env, g4_gemma_e2b_config((int)max_seq, &c));
  return config_object(env, c);
}

// new GemmaEngine({hidden, heads, pleDim, vocab, maxSeq, window, eps, softcap,
//                  layers: [{headDim, intermediate, full, kvSource, ropeBase, ropeProp}]})
napi_value Engine_new(napi_env env, napi_callback_info info) {
  napi_value a[1], self;
  if (!get_args(env, info, 1, a, &self)) return nullptr;
  napi_valuetype t;
  napi_typeof(env, a[0], &t);
  if (t != napi_object) {
    napi_throw_type_error(env, nullptr, "GemmaEngine needs a config object");
    return nullptr;
  }
  g4_gemma_config c;
  memset(&c, 0, sizeof c);
  if (!prop_int(env, a[0], "hidden", &c.hidden) || !prop_int(env, a[0], "heads", &c.heads) ||
      !prop_int(env, a[0], "pleDim", &c.ple_dim) || !prop_int(env, a[0], "vocab", &c.vocab) ||
      !prop_int(env, a[0], "maxSeq", &c.max_seq) || !prop_int(env, a[0], "window", &c.window) ||
      !prop_float(env, a[0], "eps", &c.eps) || !prop_float(env, a[0], "softcap", &c.softcap))
    return nullptr;
  napi_value layers;
  bool is_array = false;
  if (!get_prop(env, a[0], "layers", &layers)) return nullptr;
  napi_is_array(env, layers, &is_array);
  uint32_t n = 0;
  if (is_array) napi_get_array_length(env, layers, &n);
  if (!is_array || n == 0 || n > G4_GEMMA_MAX_LAYERS) {
    napi_throw_range_error(env, nullptr, "config.layers must be an array of 1-64 layer specs");
    return nullptr;
  }
  c.layers = (int)n;
  for (uint32_t i = 0; i < n; ++i) {
    napi_value L;
    napi_get_element(env, layers, i, &L);
    if (!prop_int(env, L, "headDim", &c.head_dim[i]) ||
        !prop_int(env, L, "intermediate", &c.intermediate[i]) ||
        !prop_int(env, L, "full", &c.full[i]) || !prop_int(env, L, "kvSource", &c.kv_source[i]) ||
        !prop_float(env, L, "ropeBase", &c.rope_base[i]) ||
        !prop_float(env, L, "ropeProp", &c.rope_prop[i]))
      return nullptr;
  }
  g4_gemma *h = nullptr;
  G4_CALL(env, g4_gemma_create(&c, &h));
  Engine *e = new Engine{h};
  if (napi_wrap(env, self, e, engine_finalize, nullptr, nullptr) != napi_ok) {
    g4_gemma_free(h);
    delete e;
    napi_throw_error(env, nullptr, "napi_wrap failed");
    return nullptr;
  }
  return self;
}

// e.setLinear(layer, which, w4Weight)   (layer -1: the per-layer model projection)
napi_value Engine_setLinear(napi_env env, napi_callback_info info) {
  napi_value a[3], self;
  if (!get_args(env, info, 3, a, &self)) return nullptr;
  Engine *e = unwrap_engine(env, self);
  int64_t layer, which;
  if (!e || !to_int(env, a[0], &layer, "layer") || !to_int(env, a[1], &which, "which"))
    return nullptr;
  W4 *w = unwrap_w4(env, a[2]);
  if (!w) return nullptr;
  G4_CALL(env, g4_gemma_set_linear(e->h, (int)layer, (int)which, w->h));
  return undefined(env);
}

// e.setNorm(layer, which, Float32Array)
napi_value Engine_setNorm(napi_env env, napi_callback_info info) {
  napi_value a[3], self;
  if (!get_args(env, info, 3, a, &self)) return nullptr;
  Engine *e = unwrap_engine(env, self);
  int64_t layer, which;
  if (!e || !to_int(env, a[0], &layer, "layer") || !to_int(env, a[1], &which, "which"))
    return nullptr;
  bool is = false;
  napi_is_typedarray(env, a[2], &is);
  napi_typedarray_type type = napi_int8_array;
  size_t n = 0, off;
  void *p = nullptr;
  napi_value ab;
  if (is) napi_get_typedarray_info(env, a[2], &type, &n, &p, &ab, &off);
  if (!is || type != napi_float32_array) {
    napi_throw_type_error(env, nullptr, "norm weights must be a Float32Array");
    return nullptr;
  }
  G4_CALL(env, g4_gemma_set_norm(e->h, (int)layer, (int)which, static_cast<const float *>(p),
                                 (int)n));
  return undefined(env);
}

// e.setLayerScalar(layer, s)
napi_value Engine_setLayerScalar(napi_env env, napi_callback_info info) {
  napi_value a[2], self;
  if (!get_args(env, info, 2, a, &self)) return nullptr;
  Engine *e = unwrap_engine(env, self);
  int64_t layer;
  double s;
  if (!e || !to_int(env, a[0], &layer, "layer") || !to_f64(env, a[1], &s, "scalar"))
    return nullptr;
  G4_CALL(env, g4_gemma_set_layer_scalar(e->h, (int)layer, (float)s));
  return undefined(env);
}

// e.setEmbedding(deviceBuffer)   BF16 [vocab, hidden]
napi_value Engine_setEmbedding(napi_env env, napi_callback_info info) {
  napi_value a[1], self;
  if (!get_args(env, info, 1, a, &self)) return nullptr;
  Engine *e = unwrap_engine(env, self);
  void *p;
  if (!e || !dev(env, a[0], "embedding", &p)) return nullptr;
  G4_CALL(env, g4_gemma_set_embedding(e->h, p));
  return undefined(env);
}

// e.setPle(pleTable)
napi_value Engine_setPle(napi_env env, napi_callback_info info) {
  napi_value a[1], self;
  if (!get_args(env, info, 1, a, &self)) return nullptr;
  Engine *e = unwrap_engine(env, self);
  if (!e) return nullptr;
  Ple *t = unwrap_ple(env, a[0]);
  if (!t) return nullptr;
  G4_CALL(env, g4_gemma_set_ple(e->h, t->h));
  return undefined(env);
}

// e.setPleDense(deviceBuffer)   BF16 [vocab, layers * pleDim]
napi_value Engine_setPleDense(napi_env env, napi_callback_info info) {
  napi_value a[1], self;
  if (!get_args(env, info, 1, a, &self)) return nullptr;
  Engine *e = unwrap_engine(env, self);
  void *p;
  if (!e || !dev(env, a[0], "per-layer embeddings", &p)) return nullptr;
  G4_CALL(env, g4_gemma_set_ple_dense(e->h, p));
  return undefined(env);
}

napi_value Engine_reset(napi_env env, napi_callback_info info) {
  napi_value self;
  if (!get_args(env, info, 0, nullptr, &self)) return nullptr;
  Engine *e = unwrap_engine(env, self);
  if (!e) return nullptr;
  G4_CALL(env, g4_gemma_reset(e->h));
  return undefined(env);
}

napi_value Engine_cacheLength(napi_env env, napi_callback_info info) {
  napi_value self, v;
  if (!get_args(env, info, 0, nullptr, &self)) return nullptr;
  Engine *e = unwrap_engine(env, self);
  if (!e) return nullptr;
  int len = 0;
  G4_CALL(env, g4_gemma_cache_length(e->h, &len));
  NAPI_CALL(env, napi_create_int32(env, len, &v));
  return v;
}

// e.forward(ids, startPos, lastHidden?)   lastHidden: DeviceBuffer of hidden floats
napi_value Engine_forward(napi_env env, napi_callback_info info) {
  napi_value a[3], self;
  if (!get_args(env, info, 3, a, &self)) return nullptr;
  Engine *e = unwrap_engine(env, self);
  std::vector<int32_t> ids;
  int64_t start;
  void *out;
  if (!e || !id_list(env, a[0], &ids) || !to_int(env, a[1], &start, "startPos") ||
      !dev_or_null(env, a[2], "lastHidden", &out))
    return nullptr;
  if (ids.empty()) {
    napi_throw_range_error(env, nullptr, "forward needs at least one token id");
    return nullptr;
  }
  G4_CALL(env, g4_gemma_forward(e->h, ids.data(), (int)ids.size(), (int)start,
                                static_cast<float *>(out)));
  return undefined(env);
}

// e.forwardDiag(ids, startPos, lastHidden?, topHidden?, topPle?, layerHidden?,
//               stageLayer, stages?)   the buffers DeviceBuffers or null
napi_value Engine_forwardDiag(napi_env env, napi_callback_info info) {
  napi_value a[8], self;
  if (!get_args(env, info, 8, a, &self)) return nullptr;
  Engine *e = unwrap_engine(env, self);
  std::vector<int32_t> ids;
  int64_t start, stage_layer;
  void *last, *top, *ple, *layers, *stages;
  if (!e || !id_list(env, a[0], &ids) || !to_int(env, a[1], &start, "startPos") ||
      !dev_or_null(env, a[2], "lastHidden", &last) || !dev_or_null(env, a[3], "topHidden", &top) ||
      !dev_or_null(env, a[4], "topPle", &ple) || !dev_or_null(env, a[5], "layerHidden", &layers) ||
      !to_int(env, a[6], &stage_layer, "stageLayer") || !dev_or_null(env, a[7], "stages", &stages))
    return nullptr;
  if (ids.empty()) {
    napi_throw_range_error(env, nullptr, "forward needs at least one token id");
    return nullptr;
  }
  G4_CALL(env, g4_gemma_forward_diag(e->h, ids.data(), (int)ids.size(), (int)start,
                                     static_cast<float *>(last), static_cast<float *>(top),
                                     static_cast<float *>(ple), static_cast<float *>(layers),
                                     (int)stage_layer, static_cast<float *>(stages)));
  return undefined(env);
}

// e.diagStages(layer, rows) -> [offsets] (G4_STAGES + 1 float offsets)
napi_value Engine_diagStages(napi_env env, napi_callback_info info) {
  napi_value a[2], self, arr;
  if (!get_args(env, info, 2, a, &self)) return nullptr;
  Engine *e = unwrap_engine(env, self);
  int64_t layer, rows;
  if (!e || !to_int(env, a[0], &layer, "layer") || !to_int(env, a[1], &rows, "rows"))
    return nullptr;
  size_t off[G4_STAGES + 1];
  G4_CALL(env, g4_gemma_diag_stages(e->h, (int)layer, (int)rows, off));
  napi_create_array_with_length(env, G4_STAGES + 1, &arr);
  for (int i = 0; i <= G4_STAGES; ++i) {
    napi_value v;
    napi_create_double(env, (double)off[i], &v);
    napi_set_element(env, arr, i, v);
  }
  return arr;
}

// e.logits(lastHidden, logits)   both DeviceBuffers
napi_value Engine_logits(napi_env env, napi_callback_info info) {
  napi_value a[2], self;
  if (!get_args(env, info, 2, a, &self)) return nullptr;
  Engine *e = unwrap_engine(env, self);
  void *h, *l;
  if (!e || !dev(env, a[0], "lastHidden", &h) || !dev(env, a[1], "logits", &l)) return nullptr;
  G4_CALL(env, g4_gemma_logits(e->h, static_cast<const float *>(h), static_cast<float *>(l)));
  return undefined(env);
}

// e.greedy(ids, startPos, logits?) -> next token id
napi_value Engine_greedy(napi_env env, napi_callback_info info) {
  napi_value a[3], self, v;
  if (!get_args(env, info, 3, a, &self)) return nullptr;
  Engine *e = unwrap_engine(env, self);
  std::vector<int32_t> ids;
  int64_t start;
  void *lg;
  if (!e || !id_list(env, a[0], &ids) || !to_int(env, a[1], &start, "startPos") ||
      !dev_or_null(env, a[2], "logits", &lg))
    return nullptr;
  if (ids.empty()) {
    napi_throw_range_error(env, nullptr, "greedy needs at least one token id");
    return nullptr;
  }
  int32_t tok = -1;
  G4_CALL(env, g4_gemma_greedy(e->h, ids.data(), (int)ids.size(), (int)start, &tok,
                               static_cast<float *>(lg)));
  NAPI_CALL(env, napi_create_int32(env, tok, &v));
  return v;
}

// e.decode(steps) -> Int32Array of the next `steps` greedy tokens
napi_value Engine_decode(napi_env env, napi_callback_info info) {
  napi_value a[1], self;
  if (!get_args(env, info, 1, a, &self)) return nullptr;
  Engine *e = unwrap_engine(env, self);
  int64_t steps;
  if (!e || !to_i64(env, a[0], &steps, "steps")) return nullptr;
  if (steps < 0 || steps > INT32_MAX / 4) {
    napi_throw_range_error(env, nullptr, "steps must be a non-negative count");
    return nullptr;
  }
  napi_value ab, arr;
  void *data = nullptr;
  NAPI_CALL(env, napi_create_arraybuffer(env, (size_t)steps * 4, &data, &ab));
  G4_CALL(env, g4_gemma_decode(e->h, (int)steps, static_cast<int32_t *>(data)));
  NAPI_CALL(env, napi_create_typedarray(env, napi_int32_array, (size_t)steps, ab, 0, &arr));
  return arr;
}

napi_value Engine_dispose(napi_env env, napi_callback_info info) {
  napi_value self;
  if (!get_args(env, info, 0, nullptr, &self)) return nullptr;
  void *p = nullptr;
  if (!is_instance(env, self, g_engine_ctor) || napi_unwrap(env, self, &p) != napi_ok || !p) {
    napi_throw_type_error(env, nullptr, "not a GemmaEngine");
    return nullptr;
  }
  Engine *e = static_cast<Engine *>(p);
  if (e->h) {
    g4_gemma *h = e->h;
    e->h = nullptr;
    G4_CALL(env, g4_gemma_free(h));
  }
  return undefined(env);
}

napi_value define_class(napi_env env, napi_value exports, const char *name, napi_callback ctor,
                        const napi_property_descriptor *props, size_t nprops, napi_ref *ref) {
  napi_value cls;
  NAPI_CALL(env, napi_define_class(env, name, NAPI_AUTO_LENGTH, ctor, nullptr, nprops, props, &cls));
  NAPI_CALL(env, napi_create_reference(env, cls, 1, ref));
  NAPI_CALL(env, napi_set_named_property(env, exports, name, cls));
  return cls;
}

#define METHOD(name, fn) {name, nullptr, fn, nullptr, nullptr, nullptr, napi_default, nullptr}
#define GETTER(name, fn) {name, nullptr, nullptr, fn, nullptr, nullptr, napi_default, nullptr}

napi_value Init(napi_env env, napi_value exports) {
  const napi_property_descriptor buf_props[] = {
      GETTER("size", DevBuf_size), METHOD("destroy", DevBuf_destroy),
      METHOD("write", DevBuf_write), METHOD("read", DevBuf_read)};
  if (!define_class(env, exports, "DeviceBuffer", DevBuf_new, buf_props, 4, &g_devbuf_ctor))
    return nullptr;
  const napi_property_descriptor w4_props[] = {
      METHOD("linear", W4_linear), METHOD("dequant", W4_dequant), METHOD("dispose", W4_dispose),
      METHOD("info", W4_info)};
  if (!define_class(env, exports, "W4Weight", W4_new, w4_props, 4, &g_w4_ctor)) return nullptr;
  const napi_property_descriptor ple_props[] = {
      METHOD("shardBytes", Ple_shardBytes), METHOD("uploadShard", Ple_uploadShard),
      METHOD("gather", Ple_gather), METHOD("gatherDev", Ple_gatherDev),
      METHOD("dispose", Ple_dispose)};
  if (!define_class(env, exports, "PleTable", Ple_new, ple_props, 5, &g_ple_ctor)) return nullptr;
  const napi_property_descriptor cmd_props[] = {METHOD("submit", Cmd_submit),
                                                METHOD("destroy", Cmd_destroy)};
  if (!define_class(env, exports, "CommandBuffer", Cmd_new, cmd_props, 2, &g_cmd_ctor))
    return nullptr;
  const napi_property_descriptor engine_props[] = {
      METHOD("setLinear", Engine_setLinear), METHOD("setNorm", Engine_setNorm),
      METHOD("setLayerScalar", Engine_setLayerScalar), METHOD("setEmbedding", Engine_setEmbedding),
      METHOD("setPle", Engine_setPle), METHOD("setPleDense", Engine_setPleDense),
      METHOD("reset", Engine_reset), METHOD("cacheLength", Engine_cacheLength),
      METHOD("forward", Engine_forward), METHOD("forwardDiag", Engine_forwardDiag),
      METHOD("diagStages", Engine_diagStages), METHOD("logits", Engine_logits),
      METHOD("greedy", Engine_greedy), METHOD("decode", Engine_decode),
      METHOD("dispose", Engine_dispose)};
  if (!define_class(env, exports, "GemmaEngine", Engine_new, engine_props,
                    sizeof engine_props / sizeof engine_props[0], &g_engine_ctor))
    return nullptr;
  const napi_property_descriptor fns[] = {
      METHOD("init", F_init), METHOD("deviceInfo", F_deviceInfo), METHOD("sync", F_sync),
      METHOD("copy", F_copy), METHOD("bf16Head", F_bf16Head), METHOD("linearMulti", F_linearMulti),
      METHOD("encoderBegin", F_encoderBegin), METHOD("encoderFinish", F_encoderFinish),
      METHOD("timeMs", F_timeMs), METHOD("rms", F_rms), METHOD("addScale", F_addScale),
      METHOD("scale", F_scale), METHOD("geluMul", F_geluMul), METHOD("geluPle", F_geluPle),
      METHOD("normRope", F_normRope), METHOD("attention", F_attention),
      METHOD("pleMix", F_pleMix), METHOD("argmax", F_argmax), METHOD("e2bConfig", F_e2bConfig), METHOD("fillRandom", F_fillRandom)};
  NAPI_CALL(env, napi_define_properties(env, exports, sizeof fns / sizeof fns[0], fns));
  napi_value v;
  napi_create_int32(env, G4_F32, &v);
  napi_set_named_property(env, exports, "F32", v);
  napi_create_int32(env, G4_BF16, &v);
  napi_set_named_property(env, exports, "BF16", v);
  const struct { const char *name; int value; } kinds[] = {
      {"RAND_W4_PACKED", G4_RAND_W4_PACKED}, {"RAND_PLE_PACKED", G4_RAND_PLE_PACKED},
      {"RAND_BF16_ABS_NORMAL", G4_RAND_BF16_ABS_NORMAL},
      {"RAND_BF16_NORMAL", G4_RAND_BF16_NORMAL}, {"RAND_F32_NORMAL", G4_RAND_F32_NORMAL},
      {"RAND_W4_PACKED_FULL", G4_RAND_W4_PACKED_FULL},
      {"RAND_PLE_PACKED_FULL", G4_RAND_PLE_PACKED_FULL}};
  for (const auto &k : kinds) {
    napi_create_int32(env, k.value, &v);
    napi_set_named_property(env, exports, k.name, v);
  }
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
