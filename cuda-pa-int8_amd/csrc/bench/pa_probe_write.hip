// Exact-address-stream probe of the INT8 quantize + paged-cache write
// (reshape_and_cache_int8: fp16 input, per-token scales, head_dim 128): the
// same launch (grid, jobs, waves), the same input loads and the same K, V and
// scale stores as the write kernel, from the same kernel template
// (quant_write_kernel of pa_quant_kernel.hpp) instantiated with PROBE, which
// stores each input element's high byte and a scale of 1 instead of the
// quantized values.  Its time is the memory system's for exactly the write
// kernel's address stream: the ceiling the write kernel is measured against.
// It overwrites the caches it is given.  Measurement helper of
// libpa_bench_probe.so (declared in pa_probe.h).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "pa_internal.hpp"
#include "pa_probe.h"
#include "pa_quant_kernel.hpp"

extern "C" pa_status_t pa_probe_quant_write(const void* key, const void* value, int64_t kts,
                                            int64_t khs, int64_t vts, int64_t vhs,
                                            const int64_t* slot_mapping, int32_t num_tokens,
                                            int32_t num_kv_heads, void* k_cache, void* v_cache,
                                            float* k_scales, float* v_scales, int32_t num_blocks,
                                            int32_t block_size, pa_stream_t stream) {
  constexpr int D = 128;
  if (!key || !value || !slot_mapping || !k_cache || !v_cache || !k_scales || !v_scales)
    return PA_ERR_NULL_POINTER;
  if (block_size < 16 || block_size > 128 || (block_size & (block_size - 1)) != 0)
    return PA_ERR_BAD_BLOCK_SIZE;
  if (num_tokens < 1 || num_kv_heads < 1 || num_blocks < 1) return PA_ERR_BAD_SHAPE;
  const int64_t strides[4] = {kts, khs, vts, vhs};
  for (int64_t s : strides)
    if (s < 0 || s % 8 != 0) return PA_ERR_BAD_SHAPE;
  const void* ptrs[4] = {key, value, k_cache, v_cache};
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return PA_ERR_BAD_SHAPE;
  // the grid of the write kernel's launcher
  const int tiles = (num_tokens + 15) / 16;
  const int njobs = tiles * num_kv_heads * 2;
  const int want = (njobs + pa::kQuantWaves - 1) / pa::kQuantWaves;
  const int grid = std::min(want, pa::resident_groups<D, false, false, true>());
  pa::quant_write_kernel<D, false, false, true>
      <<<grid, pa::kQuantWaves * pa::kWave, 0, reinterpret_cast<hipStream_t>(stream)>>>(
          static_cast<const uint16_t*>(key), static_cast<const uint16_t*>(value), kts, khs, vts,
          vhs, slot_mapping, num_tokens, num_kv_heads, static_cast<int8_t*>(k_cache),
          static_cast<int8_t*>(v_cache), k_scales, v_scales, num_blocks, block_size,
          __builtin_ctz((unsigned)block_size), njobs, nullptr, nullptr);
  return hipGetLastError() == hipSuccess ? PA_OK : PA_ERR_LAUNCH;
}
