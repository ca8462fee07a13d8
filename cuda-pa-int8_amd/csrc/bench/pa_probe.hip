// Streaming probes: the practical HBM read rate of the MI355X for a plain
// contiguous sweep and for chunks in an arbitrary order (the access pattern
// of a block-permuted paged cache), and the practical rate of a contiguous
// stream that writes one byte for every two it reads (the INT8 write
// kernel's ratio).  Measurement helpers for bench.py's roofline context,
// built into their own library (libpa_bench_probe.so, declared in
// pa_probe.h); not part of the decode path or its C ABI.
//
// The read probes keep several independent 16-byte loads per lane in flight
// and fold every loaded word into a checksum, so the compiler can neither
// narrow nor drop a load.  They load with the non-temporal hint, as the
// decode kernels' V loads do; the read+write probe also stores with the
// write kernel's non-temporal policy.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pa_device.hpp"
#include "pa_probe.h"

namespace {

constexpr int kProbeThreads = 256;
constexpr int kUnroll = 4;   // independent 16-B loads per lane per step

__device__ __forceinline__ uint32_t fold(uint4 v) { return v.x ^ v.y ^ v.z ^ v.w; }
__device__ __forceinline__ uint4 ld(const uint4* p) { return pa::load_stream<uint4>(p); }

__global__ void __launch_bounds__(kProbeThreads)
probe_read_contiguous(const uint4* __restrict__ p, size_t n16, uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  const size_t step = (size_t)gridDim.x * kProbeThreads * kUnroll;
  size_t i = (size_t)blockIdx.x * kProbeThreads * kUnroll + threadIdx.x;
  for (; i + (kUnroll - 1) * kProbeThreads < n16; i += step) {
    uint4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = ld(p + i + u * kProbeThreads);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= fold(v[u]);
  }
  for (int u = 0; u < kUnroll; ++u)   // ragged end of the sweep
    if (i + u * kProbeThreads < n16) acc ^= fold(ld(p + i + u * kProbeThreads));
  if (acc == 0x9E3779B9u) sink[0] = acc;   // keeps the loads live; practically never taken
}

// Each wave reads 4 KB per step (4 loads per lane): one 4 KB piece of a chunk,
// or, for chunks below 4 KB, several chunks at once.  chunk_bytes is a
// multiple of 1 KB that divides 4 KB or is a multiple of 4 KB.
__global__ void __launch_bounds__(kProbeThreads)
probe_read_chunks(const uint4* __restrict__ p, const int32_t* __restrict__ order, int32_t nchunk,
                  int32_t total, int32_t c16, uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  const int wave = (blockIdx.x * kProbeThreads + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  const int nw = (gridDim.x * kProbeThreads) >> 6;
  if (c16 >= 64 * kUnroll) {
    for (int b = wave; b < nchunk; b += nw) {
      const int32_t c = order[b];
      if ((uint32_t)c >= (uint32_t)total) continue;
      const uint4* q = p + (size_t)c * c16 + lane;
      for (int j = 0; j < c16; j += 64 * kUnroll) {
        uint4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) v[u] = ld(q + j + 64 * u);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) acc ^= fold(v[u]);
      }
    }
  } else {
    const int per = 64 * kUnroll / c16;   // chunks per 4 KB step (2 or 4)
    for (int b0 = wave * per; b0 < nchunk; b0 += nw * per) {
      uint4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int e = 64 * u + lane;          // 16-B element of this step
        const int b = b0 + e / c16;
        const int32_t c = b < nchunk ? order[b] : -1;
        v[u] = (uint32_t)c < (uint32_t)total ? ld(p + (size_t)c * c16 + e % c16) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) acc ^= fold(v[u]);
    }
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

// Reads 16 B and writes 8 B (a fold of them) per lane and element, 4
// elements per lane in flight: the read and written streams are contiguous.
__global__ void __launch_bounds__(kProbeThreads)
probe_read_write(const uint4* __restrict__ p, size_t n16, void* dst) {
  const auto out = __builtin_amdgcn_make_buffer_rsrc(dst, 0, (int)(uint32_t)(n16 * 8), 0x00020000);
  const size_t step = (size_t)gridDim.x * kProbeThreads * kUnroll;
  size_t i = (size_t)blockIdx.x * kProbeThreads * kUnroll + threadIdx.x;
  typedef uint32_t u2v_t __attribute__((ext_vector_type(2)));
  constexpr int kStorePolicy = 2;   // non-temporal, as the write kernel's tile stores
  for (; i + (kUnroll - 1) * kProbeThreads < n16; i += step) {
    uint4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = ld(p + i + u * kProbeThreads);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      __builtin_amdgcn_raw_buffer_store_b64((u2v_t){v[u].x ^ v[u].z, v[u].y ^ v[u].w}, out,
                                            (uint32_t)((i + u * kProbeThreads) * 8), 0,
                                            kStorePolicy);
  }
  for (int u = 0; u < kUnroll; ++u) {   // ragged end of the sweep
    const size_t e = i + u * kProbeThreads;
    if (e < n16) {
      const uint4 w = ld(p + e);
      __builtin_amdgcn_raw_buffer_store_b64((u2v_t){w.x ^ w.z, w.y ^ w.w}, out, (uint32_t)(e * 8),
                                            0, kStorePolicy);
    }
  }
}

}  // namespace

extern "C" {

pa_status_t pa_probe_read_contiguous(const void* src, size_t bytes, uint32_t* sink, int32_t grid,
                                     pa_stream_t stream) {
  if (!src || !sink) return PA_ERR_NULL_POINTER;
  if (grid < 1 || reinterpret_cast<uintptr_t>(src) % 16 != 0) return PA_ERR_BAD_SHAPE;
  probe_read_contiguous<<<grid, kProbeThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<const uint4*>(src), bytes / 16, sink);
  return hipGetLastError() == hipSuccess ? PA_OK : PA_ERR_LAUNCH;
}

pa_status_t pa_probe_read_chunks(const void* src, size_t bytes, const int32_t* order,
                                 int32_t num_chunks, int32_t chunk_bytes, uint32_t* sink,
                                 int32_t grid, pa_stream_t stream) {
  if (!src || !order || !sink) return PA_ERR_NULL_POINTER;
  const bool small = chunk_bytes == 1024 || chunk_bytes == 2048;
  if (grid < 1 || (!small && (chunk_bytes < 4096 || chunk_bytes % 4096 != 0)) ||
      num_chunks < 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0)
    return PA_ERR_BAD_SHAPE;
  const size_t total = bytes / (size_t)chunk_bytes;
  if (total > (size_t)INT32_MAX) return PA_ERR_BAD_SHAPE;
  probe_read_chunks<<<grid, kProbeThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<const uint4*>(src), order, num_chunks, (int32_t)total, chunk_bytes / 16, sink);
  return hipGetLastError() == hipSuccess ? PA_OK : PA_ERR_LAUNCH;
}

pa_status_t pa_probe_read_write(const void* src, size_t read_bytes, void* dst, int32_t grid,
                               pa_stream_t stream) {
  if (!src || !dst) return PA_ERR_NULL_POINTER;
  const size_t n16 = read_bytes / 16;
  if (grid < 1 || reinterpret_cast<uintptr_t>(src) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(dst) % 8 != 0 || n16 * 8 > 0xFFFFFFFFull)
    return PA_ERR_BAD_SHAPE;
  probe_read_write<<<grid, kProbeThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<const uint4*>(src), n16, dst);
  return hipGetLastError() == hipSuccess ? PA_OK : PA_ERR_LAUNCH;
}

}  // extern "C"
