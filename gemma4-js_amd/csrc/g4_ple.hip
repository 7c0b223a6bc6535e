// Per-layer-embedding (PLE) W4 gather-dequant: the gfx950 replacement of
// W4PleShardBundle.rowsToGpu + the PLE dequant shader
// (custom-webgpu/gpu-runtime.js:190-256, 413-527).
//
// The reference gathers the rows of the requested token ids on the CPU (two
// File.slice reads per id), uploads them and dequantizes on the GPU.  Here
// the whole table stays resident in HBM (1.32 GB for [262144, 8960]) in the
// exact byte layout of the builder's shards (tools/build_ple_w4_full.py:
// 130-170), and the gather runs on the device:
//
//   shard s = id / rows_per_shard, local row = id - s * rows_per_shard
//   packed  at shard_base + local * (width/2)                 (low nibble first,
//                                                              two's complement)
//   scales  at shard_base + rows_in_shard * (width/2) + local * (width/32 * 2)
//
// Element i of a row is nibble (i & 1) of byte i >> 1, i.e. bits 4k..4k+3 of
// the little-endian 32-bit word holding elements 8w..8w+7 - the same order as
// the W4 linear weights; only the signed decoding differs (q = n >= 8 ? n - 16
// : n, ple-w4-shard-reader.js:89-96), which equals (n ^ 8) - 8.
#include <string.h>

#include "g4_internal.h"

struct g4_ple {
  int vocab, width, group, rows_per_shard, num_shards;
  size_t packed_row, scale_row, full_shard_bytes, total_bytes;
  uint8_t *table;
  int32_t *ids_dev;     // device staging for host ids
  int32_t *ids_host;    // pinned staging for host ids
  int ids_cap;
  hipEvent_t ids_done;  // last copy out of ids_host has finished
};

namespace {

using namespace g4;

// One thread per 32 bytes of output: EPT consecutive elements of one row (8
// for FP32, 16 for BF16), loaded as one 32- or 64-bit word of packed nibbles
// and one scale (the EPT elements lie in one 32-element group), stored as two
// 16-byte chunks.  Measured at 2048 ids: 17.4 vs 20.1 us (FP32) and 11.6 vs
// 13.5 us (BF16) for one 16-byte chunk per thread; four chunks per thread
// (stores 64 bytes apart across the lanes) took 52.7 us.  The table is only
// read (1.32 GB, far beyond the caches); the output is written once.
template <bool BF16OUT>
__global__ __launch_bounds__(256) void ple_gather_kernel(
    const uint8_t *__restrict__ table, const int32_t *__restrict__ ids, int n,
    void *__restrict__ out, int vocab, int width, int rows_per_shard, size_t packed_row,
    size_t scale_row, size_t full_shard_bytes) {
  constexpr int EPT = BF16OUT ? 16 : 8;
  constexpr int NW = EPT / 8;  // packed words per thread
  const int per_row = width / EPT;
  const size_t item = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= (size_t)n * per_row) return;
  const int j = (int)(item / per_row);
  const int e0 = (int)(item - (size_t)j * per_row) * EPT;  // first element
  const int id = ids[j];
  float v[EPT];
  if (id < 0 || id >= vocab) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) v[i] = __uint_as_float(0x7fc00000u);
  } else {
    const int shard = id / rows_per_shard;
    const int local = id - shard * rows_per_shard;
    const int left = vocab - shard * rows_per_shard;
    const int rows_in_shard = left < rows_per_shard ? left : rows_per_shard;
    const uint8_t *base = table + (size_t)shard * full_shard_bytes;
    const uint8_t *prow = base + (size_t)local * packed_row;
    uint32_t w[NW];
    if constexpr (NW == 1) {
      w[0] = *reinterpret_cast<const uint32_t *>(prow + e0 / 2);
    } else {
      const uint2 x = *reinterpret_cast<const uint2 *>(prow + e0 / 2);
      w[0] = x.x;
      w[1] = x.y;
    }
    const uint16_t sb = reinterpret_cast<const uint16_t *>(
        base + (size_t)rows_in_shard * packed_row + (size_t)local * scale_row)[e0 / 32];
    const float s = bf16_to_f32(sb);
#pragma unroll
    for (int k = 0; k < NW; ++k) {
      // two's-complement nibbles -> offset binary: n ^ 8 = q + 8
      const uint32_t ww = w[k] ^ 0x88888888u;
#pragma unroll
      for (int i = 0; i < 8; ++i) v[8 * k + i] = (float)((int)((ww >> (4 * i)) & 15u) - 8) * s;
    }
  }
  const size_t o = (size_t)j * width + e0;
  // streaming stores: the output is written once and not read back here
  if (BF16OUT) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      u32x4 p;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        p[q] = f32_to_bf16_rne(v[8 * k + 2 * q]) | (f32_to_bf16_rne(v[8 * k + 2 * q + 1]) << 16);
      __builtin_nontemporal_store(p, reinterpret_cast<u32x4 *>(static_cast<uint16_t *>(out) + o) + k);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const u32x4 p = {__float_as_uint(v[4 * k]), __float_as_uint(v[4 * k + 1]),
                       __float_as_uint(v[4 * k + 2]), __float_as_uint(v[4 * k + 3])};
      __builtin_nontemporal_store(p, reinterpret_cast<u32x4 *>(static_cast<float *>(out) + o) + k);
    }
  }
}

// Rows of width 8960 (the only PLE geometry gpu-runtime.js:449-458 accepts) at
// 128 ids and more: one block per id.  The row's 4480 packed bytes and 560 scale
// bytes travel global -> LDS directly (16-byte `global_load_lds_dwordx4`, no
// registers), then the block writes the row's output with 16 bytes per lane per
// store, so each wave store instruction covers 1 KB of consecutive output.  The
// values are those of ple_gather_kernel, bit for bit.  Measured at 2048 ids (cold
// table, 16 id sets in rotation): FP32 17.8 -> 14.5 us with 512 threads, BF16
// 11.4 -> 9.0 us with 128 threads (9.6 with 256, 10.2 with 512); below 128 ids
// the element-per-thread kernel is as fast or faster (1 id: 2.7 against 2.8 us).
constexpr int kRowWidth = 8960;

template <bool BF16OUT, int T>
__global__ __launch_bounds__(T) void ple_gather_row_kernel(
    const uint8_t *__restrict__ table, const int32_t *__restrict__ ids, void *__restrict__ out,
    int vocab, int rows_per_shard, size_t full_shard_bytes) {
  constexpr int PR = kRowWidth / 2, SR = kRowWidth / 16;  // packed and scale bytes per row
  constexpr int C = (PR + SR) / 16, P16 = PR / 16;        // 16-byte chunks: all, packed
  constexpr int LC = (C + T - 1) / T;                     // chunks loaded per thread
  constexpr int EPC = BF16OUT ? 8 : 4;                    // elements per 16-byte output chunk
  constexpr int OC = kRowWidth / EPC;                     // output chunks per row
  constexpr int SC = (OC + T - 1) / T;                    // output chunks per thread
  static_assert(PR % 16 == 0 && SR % 16 == 0, "row blocks must be 16-byte multiples");
  // every wave's destination base stays inside the array, lanes past C load nothing
  __shared__ uint4 row[LC * T];
  typedef __attribute__((address_space(3))) void *lds_ptr;
  const int t = threadIdx.x, wave = t >> 6;
  const int j = blockIdx.x;
  const int id = __builtin_amdgcn_readfirstlane(ids[j]);
  const bool valid = id >= 0 && id < vocab;
  if (valid) {
    const int shard = id / rows_per_shard;
    const int local = id - shard * rows_per_shard;
    const int left = vocab - shard * rows_per_shard;
    const int rows_in_shard = left < rows_per_shard ? left : rows_per_shard;
    const uint8_t *base = table + (size_t)shard * full_shard_bytes;
    const uint8_t *prow = base + (size_t)local * PR;
    const uint8_t *srow = base + (size_t)rows_in_shard * PR + (size_t)local * SR;
#pragma unroll
    for (int k = 0; k < LC; ++k) {
      const int c = t + T * k;
      if (c < C)  // lane l of the wave lands at the wave's base + 16 l
        __builtin_amdgcn_global_load_lds(
            (const void *)(c < P16 ? prow + 16 * c : srow + 16 * (c - P16)),
            (lds_ptr)&row[T * k + 64 * wave], 16, 0, 0);
    }
  }
  // the direct loads count in vmcnt only; the barrier makes every wave's chunks visible
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  const uint8_t *L = reinterpret_cast<const uint8_t *>(row);
  u32x4 *dst = reinterpret_cast<u32x4 *>(static_cast<uint8_t *>(out) +
                                         (size_t)j * kRowWidth * (BF16OUT ? 2 : 4));
#pragma unroll
  for (int k = 0; k < SC; ++k) {
    const int i = t + T * k;
    if (i < OC) {
      const int e0 = i * EPC;
      const float s = bf16_to_f32(*reinterpret_cast<const uint16_t *>(L + PR + (e0 >> 5) * 2));
      // two's-complement nibbles -> offset binary: n ^ 8 = q + 8
      const uint32_t ww =
          EPC == 4 ? (uint32_t)(*reinterpret_cast<const uint16_t *>(L + (e0 >> 1))) ^ 0x8888u
                   : *reinterpret_cast<const uint32_t *>(L + (e0 >> 1)) ^ 0x88888888u;
      float v[EPC];
#pragma unroll
      for (int q = 0; q < EPC; ++q)
        v[q] = valid ? (float)((int)((ww >> (4 * q)) & 15u) - 8) * s : __uint_as_float(0x7fc00000u);
      u32x4 p;
      if (BF16OUT) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          p[q] = f32_to_bf16_rne(v[2 * q]) | (f32_to_bf16_rne(v[2 * q + 1]) << 16);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) p[q] = __float_as_uint(v[q]);
      }
      __builtin_nontemporal_store(p, dst + i);
    }
  }
}

template <bool BF16OUT, int T>
int launch_gather_rows(const g4_ple *t, const int32_t *ids_dev, int n, void *out) {
  hipLaunchKernelGGL((ple_gather_row_kernel<BF16OUT, T>), dim3(n), dim3(T), 0, stream(), t->table,
                     ids_dev, out, t->vocab, t->rows_per_shard, t->full_shard_bytes);
  G4_LAUNCH_CHECK("ple_gather_row_kernel");
  return G4_OK;
}

int launch_gather(const g4_ple *t, const int32_t *ids_dev, int n, void *out, int out_dtype) {
  const bool bf = out_dtype == G4_BF16;
  if (t->width == kRowWidth && t->group == 32 && n >= 128) {
    if (!bf) return launch_gather_rows<false, 512>(t, ids_dev, n, out);
    return n >= 1024 ? launch_gather_rows<true, 128>(t, ids_dev, n, out)
                     : launch_gather_rows<true, 512>(t, ids_dev, n, out);
  }
  const size_t items = (size_t)n * (t->width / (bf ? 16 : 8));
  const unsigned blocks = (unsigned)((items + 255) / 256);
  if (bf)
    hipLaunchKernelGGL(ple_gather_kernel<true>, dim3(blocks), dim3(256), 0, stream(), t->table,
                       ids_dev, n, out, t->vocab, t->width, t->rows_per_shard, t->packed_row,
                       t->scale_row, t->full_shard_bytes);
  else
    hipLaunchKernelGGL(ple_gather_kernel<false>, dim3(blocks), dim3(256), 0, stream(), t->table,
                       ids_dev, n, out, t->vocab, t->width, t->rows_per_shard, t->packed_row,
                       t->scale_row, t->full_shard_bytes);
  G4_LAUNCH_CHECK("ple_gather_kernel");
  return G4_OK;
}

// quantize_batch of the builder (tools/build_ple_w4_full.py:48-60), one
// thread per 32-column group: s = bf16_rne(maxabs / 7) (1.0 for an all-zero
// group, the float32 division of numpy), q = clip(rint(x / s_bf16), -7, 7)
// with round half to even, stored as two's-complement nibbles, low nibble
// first.  Row r goes to shard r / rows_per_shard of a table of `vocab` rows,
// each shard its packed block then its scales block (130-170).  The 64 input
// bytes of a group are four 16-byte loads; its 16 packed bytes one store.
__global__ __launch_bounds__(256) void ple_quantize_kernel(
    const uint4 *__restrict__ src, int vocab, int width, int rows_per_shard, size_t packed_row,
    size_t scale_row, size_t full_shard_bytes, uint8_t *__restrict__ table) {
  const int G = width / 32;
  const size_t item = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= (size_t)vocab * G) return;
  const int r = (int)(item / G);
  const int g = (int)(item - (size_t)r * G);
  const uint4 *p = src + item * 4;  // 32 bf16 = 4 x 16 bytes
  float x[32];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const uint4 v = p[c];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[8 * c + 2 * k] = __uint_as_float(w[k] << 16);
      x[8 * c + 2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
    }
  }
  float maxabs = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) maxabs = fmaxf(maxabs, fabsf(x[i]));
  const float sc = maxabs == 0.f ? 1.f : maxabs / 7.f;  // IEEE division, as numpy's float32
  const uint32_t sbits = f32_to_bf16_rne(sc);
  const float stored = bf16_to_f32(sbits);
  uint32_t packed[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const float q = fminf(fmaxf(rintf(x[i] / stored), -7.f), 7.f);
    packed[i >> 3] |= ((uint32_t)(int)q & 15u) << (4 * (i & 7));
  }
  const int shard = r / rows_per_shard;
  const int local = r - shard * rows_per_shard;
  const int left = vocab - shard * rows_per_shard;
  const int rows_in_shard = left < rows_per_shard ? left : rows_per_shard;
  uint8_t *base = table + (size_t)shard * full_shard_bytes;
  *reinterpret_cast<uint4 *>(base + (size_t)local * packed_row + (size_t)g * 16) =
      make_uint4(packed[0], packed[1], packed[2], packed[3]);
  reinterpret_cast<uint16_t *>(base + (size_t)rows_in_shard * packed_row +
                               (size_t)local * scale_row)[g] = (uint16_t)sbits;
}

int launch_quantize(const void *src, int vocab, int width, int rows_per_shard,
                    size_t full_shard_bytes, uint8_t *table) {
  const size_t items = (size_t)vocab * (width / 32);
  hipLaunchKernelGGL(ple_quantize_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0,
                     stream(), static_cast<const uint4 *>(src), vocab, width, rows_per_shard,
                     (size_t)width / 2, (size_t)(width / 32) * 2, full_shard_bytes, table);
  G4_LAUNCH_CHECK("ple_quantize_kernel");
  return G4_OK;
}

int check_out(const g4_ple *t, int n, void *out, int out_dtype) {
  if (out_dtype != G4_F32 && out_dtype != G4_BF16)
    return fail(G4_E_ARG, "PLE gather: bad out dtype %d", out_dtype);
  if ((reinterpret_cast<uintptr_t>(out) & 15u) != 0)
    return fail(G4_E_ARG, "PLE gather: out must be 16-byte aligned");
  return check_device_range(out, (size_t)n * t->width * (out_dtype == G4_F32 ? 4 : 2),
                            "PLE gather out");
}

}  // namespace

G4_API int g4_ple_create(int vocab, int width, int group, int rows_per_shard,
                         g4_ple **out) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (!out) return fail(G4_E_ARG, "g4_ple_create: null output handle");
  *out = nullptr;
  if (vocab <= 0 || rows_per_shard <= 0)
    return fail(G4_E_ARG, "g4_ple_create: bad vocab %d / rows_per_shard %d", vocab,
                rows_per_shard);
  // gpu-runtime.js:449-458 accepts width 8960 and group 32 only; the kernel
  // needs width to be a multiple of the 32-column group.
  if (group != 32 || width <= 0 || width % 32 != 0)
    return fail(G4_E_ARG, "PLE shard manifest has unexpected geometry/layout.");
  g4_ple *t = new g4_ple();
  t->vocab = vocab;
  t->width = width;
  t->group = group;
  t->rows_per_shard = rows_per_shard;
  t->num_shards = (vocab + rows_per_shard - 1) / rows_per_shard;
  t->packed_row = (size_t)width / 2;
  t->scale_row = (size_t)(width / group) * 2;
  t->full_shard_bytes = (size_t)rows_per_shard * (t->packed_row + t->scale_row);
  t->total_bytes = (size_t)vocab * (t->packed_row + t->scale_row);
  // Every shard must start 16-byte aligned for the kernel's 128-bit loads
  // (true for the distribution: 4096 rows x 5040 bytes).
  if (t->full_shard_bytes % 16 != 0) {
    delete t;
    return fail(G4_E_ARG, "g4_ple_create: shard size %d x %d bytes is not a multiple of 16",
                rows_per_shard, width / 2 + (width / 32) * 2);
  }
  int rc = device_alloc(t->total_bytes, reinterpret_cast<void **>(&t->table));
  if (rc) {
    delete t;
    return rc;
  }
  hipError_t e = hipEventCreateWithFlags(&t->ids_done, hipEventDisableTiming);
  if (e != hipSuccess) {
    device_free(t->table);
    delete t;
    return fail(G4_E_HIP, "hipEventCreate failed: %s", hipGetErrorString(e));
  }
  *out = t;
  return ok();
}

G4_API int g4_ple_shard_bytes(const g4_ple *t, int shard, int *num_shards, size_t *bytes) {
  if (!t) return fail(G4_E_ARG, "g4_ple_shard_bytes: null handle");
  if (num_shards) *num_shards = t->num_shards;
  if (shard < 0 || shard >= t->num_shards)
    return fail(G4_E_RANGE, "PLE shard %d outside [0, %d)", shard, t->num_shards);
  const int left = t->vocab - shard * t->rows_per_shard;
  const int rows = left < t->rows_per_shard ? left : t->rows_per_shard;
  if (bytes) *bytes = (size_t)rows * (t->packed_row + t->scale_row);
  return ok();
}

G4_API int g4_ple_upload_shard(g4_ple *t, int shard, const void *bytes, size_t n) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  size_t want = 0;
  int rc = g4_ple_shard_bytes(t, shard, nullptr, &want);
  if (rc) return rc;
  if (!bytes) return fail(G4_E_ARG, "g4_ple_upload_shard: null data");
  if (n != want)
    return fail(G4_E_ARG, "PLE shard %d has %zu bytes, expected %zu", shard, n, want);
  G4_HIP_TRY(hipMemcpyAsync(t->table + (size_t)shard * t->full_shard_bytes, bytes, n,
                            hipMemcpyHostToDevice, stream()));
  G4_HIP_TRY(hipStreamSynchronize(stream()));
  return ok();
}

namespace g4 {
void ple_geometry(const g4_ple *t, int *vocab, int *width) {
  *vocab = t->vocab;
  *width = t->width;
}
}  // namespace g4

G4_API int g4_ple_upload_shard_dev(g4_ple *t, int shard, const void *bytes_dev, size_t n) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  size_t want = 0;
  int rc = g4_ple_shard_bytes(t, shard, nullptr, &want);
  if (rc) return rc;
  if (n != want)
    return fail(G4_E_ARG, "PLE shard %d has %zu bytes, expected %zu", shard, n, want);
  rc = check_device_range(bytes_dev, n, "g4_ple_upload_shard_dev bytes");
  if (rc) return rc;
  G4_HIP_TRY(hipMemcpyAsync(t->table + (size_t)shard * t->full_shard_bytes, bytes_dev, n,
                            hipMemcpyDeviceToDevice, stream()));
  return ok();
}

G4_API int g4_ple_free(g4_ple *t) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  if (!t) return ok();
  int rc = device_free(t->table);
  if (t->ids_dev) device_free(t->ids_dev);
  if (t->ids_host) {
    (void)hipEventSynchronize(t->ids_done);
    (void)hipHostFree(t->ids_host);
  }
  (void)hipEventDestroy(t->ids_done);
  delete t;
  return rc ? rc : ok();
}

G4_API int g4_ple_gather(const g4_ple *tc, const int32_t *ids, int n, void *out,
                         int out_dtype) {
  G4_CHECK_INIT();
  G4_CHECK_NOT_ENCODING();
  g4_ple *t = const_cast<g4_ple *>(tc);
  if (!t) return fail(G4_E_ARG, "g4_ple_gather: null handle");
  if (n < 0) return fail(G4_E_ARG, "g4_ple_gather: negative id count");
  if (n == 0) return ok();
  if (!ids) return fail(G4_E_ARG, "g4_ple_gather: null ids");
  // _location (gpu-runtime.js:463-485): every id must be an integer in range.
  for (int j = 0; j < n; ++j)
    if (ids[j] < 0 || ids[j] >= t->vocab)
      return fail(G4_E_RANGE, "PLE token id out of range: %d", ids[j]);
  int rc = check_out(t, n, out, out_dtype);
  if (rc) return rc;
  if (n > t->ids_cap) {
    G4_HIP_TRY(hipStreamSynchronize(stream()));
    if (t->ids_dev) device_free(t->ids_dev);
    if (t->ids_host) (void)hipHostFree(t->ids_host);
    t->ids_dev = nullptr;
    t->ids_host = nullptr;
    t->ids_cap = 0;
    int cap = n < 4096 ? 4096 : n;
    rc = device_alloc((size_t)cap * 4, reinterpret_cast<void **>(&t->ids_dev));
    if (rc) return rc;
    G4_HIP_TRY(hipHostMalloc(reinterpret_cast<void **>(&t->ids_host), (size_t)cap * 4,
                             hipHostMallocDefault));
    t->ids_cap = cap;
  } else {
    // The previous gather may still be copying out of the pinned buffer.
    G4_HIP_TRY(hipEventSynchronize(t->ids_done));
  }
  memcpy(t->ids_host, ids, (size_t)n * 4);
  G4_HIP_TRY(hipMemcpyAsync(t->ids_dev, t->ids_host, (size_t)n * 4, hipMemcpyHostToDevice,
                            stream()));
  G4_HIP_TRY(hipEventRecord(t->ids_done, stream()));
  rc = launch_gather(t, t->ids_dev, n, out, out_dtype);
  return rc ? rc : ok();
}

G4_API int g4_ple_gather_dev(const g4_ple *t, const int32_t *ids_dev, int n, void *out,
                             int out_dtype) {
  G4_CHECK_INIT();
  if (!t) return fail(G4_E_ARG, "g4_ple_gather_dev: null handle");
  if (n < 0) return fail(G4_E_ARG, "g4_ple_gather_dev: negative id count");
  if (n == 0) return ok();
  int rc = check_device_range(ids_dev, (size_t)n * 4, "g4_ple_gather_dev ids");
  if (rc) return rc;
  rc = check_out(t, n, out, out_dtype);
  if (rc) return rc;
  rc = launch_gather(t, ids_dev, n, out, out_dtype);
  return rc ? rc : ok();
}

G4_API int g4_ple_quantize_rows(const void *rows_bf16, int rows, int width, void *shard_dev) {
  G4_CHECK_INIT();
  if (rows < 0 || width <= 0 || width % 32 != 0)
    return fail(G4_E_ARG, "g4_ple_quantize_rows: %d rows of width %d (a multiple of 32)", rows,
                width);
  if (rows == 0) return ok();
  if ((reinterpret_cast<uintptr_t>(rows_bf16) & 15u) || (reinterpret_cast<uintptr_t>(shard_dev) & 15u))
    return fail(G4_E_ARG, "g4_ple_quantize_rows: rows and shard must be 16-byte aligned");
  const size_t packed_row = (size_t)width / 2, scale_row = (size_t)(width / 32) * 2;
  int rc = check_device_range(rows_bf16, (size_t)rows * width * 2, "g4_ple_quantize_rows rows");
  if (!rc)
    rc = check_device_range(shard_dev, (size_t)rows * (packed_row + scale_row),
                            "g4_ple_quantize_rows shard");
  if (!rc) rc = launch_quantize(rows_bf16, rows, width, rows, 0, static_cast<uint8_t *>(shard_dev));
  return rc ? rc : ok();
}

G4_API int g4_ple_quantize_table(g4_ple *t, const void *dense_bf16) {
  G4_CHECK_INIT();
  if (!t) return fail(G4_E_ARG, "g4_ple_quantize_table: null table");
  if (reinterpret_cast<uintptr_t>(dense_bf16) & 15u)
    return fail(G4_E_ARG, "g4_ple_quantize_table: rows must be 16-byte aligned");
  int rc = check_device_range(dense_bf16, (size_t)t->vocab * t->width * 2,
                              "g4_ple_quantize_table rows");
  if (!rc)
    rc = launch_quantize(dense_bf16, t->vocab, t->width, t->rows_per_shard, t->full_shard_bytes,
                         t->table);
  return rc ? rc : ok();
}
