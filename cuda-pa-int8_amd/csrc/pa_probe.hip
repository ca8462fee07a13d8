// Streaming-read probes: the practical HBM read rate of the MI355X for a
// plain contiguous sweep and for chunks in an arbitrary order (the access
// pattern of a block-permuted paged cache).  Measurement helpers for
// bench.py's roofline context; not part of the decode path.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pa_mi355x.h"

namespace {

__global__ void __launch_bounds__(256)
probe_read_contiguous(const uint4* __restrict__ p, size_t n16, uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
    const uint4 v = p[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;   // keeps the loads live; practically never taken
}

// One wave reads one chunk (chunk_bytes, a multiple of 4 KB) per step.
__global__ void __launch_bounds__(256)
probe_read_chunks(const uint4* __restrict__ p, const int32_t* __restrict__ order, int32_t nchunk,
                  int32_t total, int32_t c16, uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  const int nw = (gridDim.x * blockDim.x) >> 6;
  for (int b = wave; b < nchunk; b += nw) {
    const int32_t c = order[b];
    if ((uint32_t)c >= (uint32_t)total) continue;
    const uint4* q = p + (size_t)c * c16;
    for (int j = lane; j < c16; j += 64) {
      const uint4 v = q[j];
      acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

}  // namespace

extern "C" {

pa_status_t pa_probe_read_contiguous(const void* src, size_t bytes, uint32_t* sink, int32_t grid,
                                     pa_stream_t stream) {
  if (!src || !sink) return PA_ERR_NULL_POINTER;
  if (grid < 1 || reinterpret_cast<uintptr_t>(src) % 16 != 0) return PA_ERR_BAD_SHAPE;
  probe_read_contiguous<<<grid, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<const uint4*>(src), bytes / 16, sink);
  return hipGetLastError() == hipSuccess ? PA_OK : PA_ERR_LAUNCH;
}

pa_status_t pa_probe_read_chunks(const void* src, size_t bytes, const int32_t* order,
                                 int32_t num_chunks, int32_t chunk_bytes, uint32_t* sink,
                                 int32_t grid, pa_stream_t stream) {
  if (!src || !order || !sink) return PA_ERR_NULL_POINTER;
  if (grid < 1 || chunk_bytes < 4096 || chunk_bytes % 4096 != 0 || num_chunks < 0 ||
      reinterpret_cast<uintptr_t>(src) % 16 != 0)
    return PA_ERR_BAD_SHAPE;
  const size_t total = bytes / (size_t)chunk_bytes;
  if (total > (size_t)INT32_MAX) return PA_ERR_BAD_SHAPE;
  probe_read_chunks<<<grid, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<const uint4*>(src), order, num_chunks, (int32_t)total, chunk_bytes / 16, sink);
  return hipGetLastError() == hipSuccess ? PA_OK : PA_ERR_LAUNCH;
}

}  // extern "C"
