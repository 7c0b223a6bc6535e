// Device, queue and buffer layer: the HIP replacement of gpu-runtime.js:6-38
// (createBuffer / uploadBytes / uploadF32 / uploadU32 / readF32) and of the
// WebGPU queue that orders every dispatch.
//
// One stream per process, created at g4_init with the default priority, plays
// the role of device.queue: every upload, copy and kernel is enqueued on it,
// so work runs in submission order as in the reference.
#include <map>
#include <mutex>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "g4_internal.h"

namespace g4 {
namespace {

thread_local char g_err[1024] = "";
hipStream_t g_stream = nullptr;
bool g_encoding = false;
// Recordings alive (g4_encoder_finish .. g4_cmdbuf_free), and the scratch
// blocks a Workspace outgrew while any of them was alive: a recording holds
// the scratch address it was made with, so those blocks stay allocated until
// the last recording is freed.
int g_live_cmdbufs = 0;
std::vector<void *> g_retired;
int g_device = -1;
int g_cu_count = 0;

// Live device allocations: base -> requested size (align4).  Used to
// bounds-check operands before a kernel is launched.
std::mutex g_mu;
std::map<uintptr_t, size_t> g_allocs;

// Caching allocator.  The reference creates a buffer per op output and
// destroys it right after submit (gemma4-webgpu.js:216-301, 357-381); doing a
// hipMalloc/hipFree per op would serialise the queue.  Because every use of
// device memory is ordered on the one library stream, a block freed after its
// last use was enqueued can serve a later allocation at once: the stream runs
// the old reader before the new writer.  Blocks are kept per capacity class.
std::map<uintptr_t, size_t> g_capacity;    // live and cached block -> capacity
std::multimap<size_t, void *> g_free;      // capacity -> cached block
size_t g_cached_bytes = 0;
constexpr size_t kCacheLimit = size_t(16) << 30;

size_t capacity_class(size_t n) {
  if (n <= (size_t(64) << 10)) {
    size_t c = 256;
    while (c < n) c <<= 1;
    return c;
  }
  const size_t g = size_t(64) << 10;
  return (n + g - 1) / g * g;
}

// Gives every cached block back to HIP (after the stream is idle).
int release_cache_locked() {
  if (g_free.empty()) return G4_OK;
  hipError_t e = hipStreamSynchronize(g_stream);
  if (e != hipSuccess) return fail(G4_E_HIP, "hipStreamSynchronize: %s", hipGetErrorString(e));
  for (auto &kv : g_free) {
    g_capacity.erase(reinterpret_cast<uintptr_t>(kv.second));
    (void)hipFree(kv.second);
  }
  g_free.clear();
  g_cached_bytes = 0;
  return G4_OK;
}

}  // namespace

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return G4_OK;
}

hipStream_t stream() { return g_stream; }
bool initialised() { return g_stream != nullptr; }
bool encoding() { return g_encoding; }
int current_device() { return g_device; }
int cu_count() { return g_cu_count; }

int check_device_range(const void *p, size_t bytes, const char *what) {
  if (p == nullptr) return fail(G4_E_ARG, "%s: null device pointer", what);
  uintptr_t a = reinterpret_cast<uintptr_t>(p);
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_allocs.upper_bound(a);
    if (it != g_allocs.begin()) {
      --it;
      if (a >= it->first && a < it->first + it->second) {
        if (bytes > it->first + it->second - a)
          return fail(G4_E_RANGE,
                      "%s: %zu bytes at offset %zu overrun its %zu-byte buffer",
                      what, bytes, (size_t)(a - it->first), it->second);
        return G4_OK;
      }
    }
    auto ct = g_capacity.upper_bound(a);
    if (ct != g_capacity.begin()) {
      --ct;
      if (a < ct->first + ct->second)
        return fail(G4_E_STATE, "%s: %p points into a buffer that was freed", what, p);
    }
  }
  // Not one of ours: ask the HIP runtime for the allocation's extent.
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p) != hipSuccess ||
      base == nullptr) {
    (void)hipGetLastError();
    return fail(G4_E_RANGE, "%s: %p is not a device allocation", what, p);
  }
  size_t off = (size_t)(a - reinterpret_cast<uintptr_t>(base));
  if (bytes > size - off)
    return fail(G4_E_RANGE, "%s: %zu bytes at offset %zu overrun its %zu-byte buffer",
                what, bytes, off, size);
  return G4_OK;
}

int device_alloc(size_t bytes, void **p) {
  if (!p) return fail(G4_E_ARG, "device_alloc: null output pointer");
  size_t n = bytes < 4 ? 4 : (bytes + 3) & ~size_t(3);  // align4 (gpu-runtime.js:7)
  const size_t cap = capacity_class(n);
  void *d = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_free.find(cap);
    if (it != g_free.end()) {
      d = it->second;
      g_free.erase(it);
      g_cached_bytes -= cap;
    }
  }
  if (!d) {
    hipError_t e = hipMalloc(&d, cap);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      // retry once with the cache given back
      std::lock_guard<std::mutex> lk(g_mu);
      int rc = release_cache_locked();
      if (rc) return rc;
      e = hipMalloc(&d, cap);
      if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(G4_E_NOMEM, "hipMalloc(%zu) failed: %s", cap, hipGetErrorString(e));
      }
    }
    std::lock_guard<std::mutex> lk(g_mu);
    g_capacity[reinterpret_cast<uintptr_t>(d)] = cap;
  }
  // WebGPU buffers start zeroed; stream-ordered after any earlier user.
  hipError_t e = hipMemsetAsync(d, 0, n, g_stream);
  if (e != hipSuccess) {
    std::lock_guard<std::mutex> lk(g_mu);
    g_free.emplace(cap, d);
    g_cached_bytes += cap;
    return fail(G4_E_HIP, "hipMemsetAsync failed: %s", hipGetErrorString(e));
  }
  {
    std::lock_guard<std::mutex> lk(g_mu);
    g_allocs[reinterpret_cast<uintptr_t>(d)] = n;
  }
  *p = d;
  return G4_OK;
}

int device_free(void *p) {
  if (!p) return G4_OK;
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_allocs.find(reinterpret_cast<uintptr_t>(p));
  if (it == g_allocs.end())
    return fail(G4_E_ARG, "g4_free: %p was not allocated by g4_alloc", p);
  g_allocs.erase(it);
  // Stream-ordered reuse: work already queued that reads the block runs
  // before any later writer (WebGPU's destroy() likewise waits for submitted
  // work).  Past the cache limit the cached blocks go back to HIP.
  const size_t cap = g_capacity[reinterpret_cast<uintptr_t>(p)];
  g_free.emplace(cap, p);
  g_cached_bytes += cap;
  if (g_cached_bytes > kCacheLimit) return release_cache_locked();
  return G4_OK;
}

int Workspace::get(size_t need, void **p, const char *who) {
  if (need <= bytes) {
    if (g_encoding) captured = true;
    *p = mem;
    return G4_OK;
  }
  if (g_encoding)
    return fail(G4_E_STATE,
                "%s: scratch must grow to %zu bytes; make one call of this size outside a "
                "command encoder first", who, need);
  if (mem) {
    // only a block that a recording may hold must outlive the recordings
    if (captured && g_live_cmdbufs > 0) {
      g_retired.push_back(mem);
    } else {
      int rc = device_free(mem);
      if (rc) return rc;
    }
    mem = nullptr;
    bytes = 0;
    captured = false;
  }
  int rc = device_alloc(need, &mem);
  if (rc) return rc;
  bytes = need;
  *p = mem;
  return G4_OK;
}

}  // namespace g4

using namespace g4;

G4_API const char *g4_last_error(void) { return g4::g_err; }

G4_API int g4_init(int device) {
  if (g_stream) {
    if (device == g_device) return ok();
    return fail(G4_E_STATE, "g4_init: already initialised on device %d", g_device);
  }
  int n = 0;
  G4_HIP_TRY(hipGetDeviceCount(&n));
  if (device < 0 || device >= n)
    return fail(G4_E_ARG, "g4_init: device %d out of range (%d visible)", device, n);
  G4_HIP_TRY(hipSetDevice(device));
  hipDeviceProp_t prop;
  G4_HIP_TRY(hipGetDeviceProperties(&prop, device));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(G4_E_STATE, "g4_init: device %d is %s; this library is built for gfx950",
                device, prop.gcnArchName);
  g_cu_count = prop.multiProcessorCount;
  if (int rc = static_scratch_init(device)) return rc;
  hipStream_t s = nullptr;
  G4_HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  g_stream = s;
  g_device = device;
  return ok();
}

G4_API int g4_device_info(char *name, size_t name_len, int *cu, size_t *hbm,
                          int *clock_khz) {
  G4_CHECK_INIT();
  hipDeviceProp_t prop;
  G4_HIP_TRY(hipGetDeviceProperties(&prop, g_device));
  if (name && name_len) {
    snprintf(name, name_len, "%s (%s)", prop.name, prop.gcnArchName);
  }
  if (cu) *cu = prop.multiProcessorCount;
  if (hbm) *hbm = prop.totalGlobalMem;
  if (clock_khz) *clock_khz = prop.clockRate;
  return ok();
}

G4_API int g4_alloc(size_t bytes, void **dptr) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  int rc = device_alloc(bytes, dptr);
  return rc ? rc : ok();
}

G4_API int g4_free(void *dptr) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  int rc = device_free(dptr);
  return rc ? rc : ok();
}

G4_API int g4_upload(void *dst, size_t dst_off, const void *src, size_t n) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (n == 0) return ok();
  if (!src) return fail(G4_E_ARG, "g4_upload: null host pointer");
  int rc = check_device_range(static_cast<char *>(dst) + dst_off, n, "g4_upload dst");
  if (rc) return rc;
  // Pageable host memory: hipMemcpyAsync stages it, so `src` is free to reuse
  // on return (queue.writeBuffer semantics).
  G4_HIP_TRY(hipMemcpyAsync(static_cast<char *>(dst) + dst_off, src, n,
                            hipMemcpyHostToDevice, g_stream));
  G4_HIP_TRY(hipStreamSynchronize(g_stream));
  return ok();
}

G4_API int g4_download(const void *src, size_t src_off, void *dst, size_t n) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (n == 0) return ok();
  if (!dst) return fail(G4_E_ARG, "g4_download: null host pointer");
  int rc = check_device_range(static_cast<const char *>(src) + src_off, n,
                              "g4_download src");
  if (rc) return rc;
  G4_HIP_TRY(hipMemcpyAsync(dst, static_cast<const char *>(src) + src_off, n,
                            hipMemcpyDeviceToHost, g_stream));
  G4_HIP_TRY(hipStreamSynchronize(g_stream));
  return ok();
}

G4_API int g4_copy(void *dst, size_t dst_off, const void *src, size_t src_off,
                   size_t n) {
  G4_CHECK_INIT();
  if (n == 0) return ok();
  int rc = check_device_range(static_cast<char *>(dst) + dst_off, n, "g4_copy dst");
  if (rc) return rc;
  rc = check_device_range(static_cast<const char *>(src) + src_off, n, "g4_copy src");
  if (rc) return rc;
  G4_HIP_TRY(hipMemcpyAsync(static_cast<char *>(dst) + dst_off,
                            static_cast<const char *>(src) + src_off, n,
                            hipMemcpyDeviceToDevice, g_stream));
  return ok();
}

G4_API int g4_sync(void) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  G4_HIP_TRY(hipStreamSynchronize(g_stream));
  return ok();
}

G4_API void *g4_stream(void) { return g_stream; }

G4_API int g4_event_create(void **ev) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (!ev) return fail(G4_E_ARG, "g4_event_create: null output");
  hipEvent_t e;
  G4_HIP_TRY(hipEventCreate(&e));
  *ev = e;
  return ok();
}

G4_API int g4_event_record(void *ev) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  G4_HIP_TRY(hipEventRecord(static_cast<hipEvent_t>(ev), g_stream));
  return ok();
}

G4_API int g4_event_elapsed_ms(void *start, void *stop, float *ms) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (!ms) return fail(G4_E_ARG, "g4_event_elapsed_ms: null output");
  G4_HIP_TRY(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
  G4_HIP_TRY(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                 static_cast<hipEvent_t>(stop)));
  return ok();
}

G4_API int g4_event_destroy(void *ev) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  G4_HIP_TRY(hipEventDestroy(static_cast<hipEvent_t>(ev)));
  return ok();
}

// ---- command encoders: stream capture into a HIP graph ---------------------

struct g4_cmdbuf {
  hipGraph_t graph;
  hipGraphExec_t exec;
};

G4_API int g4_encoder_begin(void) {
  G4_CHECK_INIT();
  if (g_encoding) return fail(G4_E_STATE, "g4_encoder_begin: an encoder is already open");
  G4_HIP_TRY(hipStreamBeginCapture(g_stream, hipStreamCaptureModeRelaxed));
  g_encoding = true;
  return ok();
}

G4_API int g4_encoder_finish(g4_cmdbuf **out) {
  G4_CHECK_INIT();
  if (!g_encoding) return fail(G4_E_STATE, "g4_encoder_finish: no open encoder");
  g_encoding = false;
  hipGraph_t graph = nullptr;
  G4_HIP_TRY(hipStreamEndCapture(g_stream, &graph));
  if (!out) {
    (void)hipGraphDestroy(graph);
    return fail(G4_E_ARG, "g4_encoder_finish: null output");
  }
  hipGraphExec_t exec = nullptr;
  hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(graph);
    return fail(G4_E_HIP, "hipGraphInstantiate failed: %s", hipGetErrorString(e));
  }
  *out = new g4_cmdbuf{graph, exec};
  ++g_live_cmdbufs;
  return ok();
}

G4_API int g4_submit(const g4_cmdbuf *cb) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (!cb) return fail(G4_E_ARG, "g4_submit: null command buffer");
  G4_HIP_TRY(hipGraphLaunch(cb->exec, g_stream));
  return ok();
}

G4_API int g4_cmdbuf_free(g4_cmdbuf *cb) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (!cb) return ok();
  G4_HIP_TRY(hipStreamSynchronize(g_stream));
  (void)hipGraphExecDestroy(cb->exec);
  (void)hipGraphDestroy(cb->graph);
  delete cb;
  if (--g_live_cmdbufs == 0) {
    int first = G4_OK;
    for (void *p : g_retired) {
      const int rc = device_free(p);
      if (rc && !first) first = rc;
    }
    g_retired.clear();  // even after a failed free: no pointer is freed twice
    if (first) return first;
  }
  return ok();
}
