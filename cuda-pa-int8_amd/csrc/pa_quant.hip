// Launchers of the per-token / per-tensor INT8 quantize + paged-cache write
// (the kernel and its semantics are in pa_quant_kernel.hpp).
#include <algorithm>

#include "pa_internal.hpp"
#include "pa_quant_kernel.hpp"

namespace pa {

template <int D, bool STATIC, bool BF>
static hipError_t launch_quant_d(const QuantLaunch& l) {
  const int tiles = (l.num_tokens + 15) / 16;
  const int njobs = tiles * l.num_kv_heads * 2;
  const int want = (njobs + kQuantWaves - 1) / kQuantWaves;
  const int grid = std::min(want, resident_groups<D, STATIC, BF>());
  quant_write_kernel<D, STATIC, BF><<<grid, kQuantWaves * kWave, 0, l.stream>>>(
      static_cast<const uint16_t*>(l.key), static_cast<const uint16_t*>(l.value), l.key_token_stride,
      l.key_head_stride, l.value_token_stride, l.value_head_stride, l.slot_mapping, l.num_tokens,
      l.num_kv_heads, static_cast<int8_t*>(l.k_cache), static_cast<int8_t*>(l.v_cache),
      l.k_scales, l.v_scales, l.num_blocks, l.block_size, __builtin_ctz((unsigned)l.block_size),
      njobs, l.k_scale_in, l.v_scale_in);
  return hipGetLastError();
}

template <bool STATIC, bool BF>
static hipError_t launch_quant(const QuantLaunch& l) {
  switch (l.head_dim) {
#define PA_CASE(D) \
  case D: return launch_quant_d<D, STATIC, BF>(l);
    PA_FOR_EACH_HEAD_DIM(PA_CASE)
#undef PA_CASE
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_quant_write_i8(const QuantLaunch& l) {
  if (l.bf16_input)
    return (l.k_scale_in != nullptr) ? launch_quant<true, true>(l) : launch_quant<false, true>(l);
  return (l.k_scale_in != nullptr) ? launch_quant<true, false>(l) : launch_quant<false, false>(l);
}

}  // namespace pa
