// The decode entry point that allocates nothing (pa_paged_decode_attn_noalloc).
//
// Its counters and split partials live in `scratch`, a file-scope device
// array of PA_NOALLOC_SCRATCH_BYTES, one copy per GPU, loaded with the
// library's code object and kept until the process ends.  In host code the
// name `scratch` is only a host-side stand-in: the device address of each
// GPU's copy comes from hipGetSymbolAddress, taken once per device with that
// device current, and only that address is handed to kernels.  Layout: the
// first PA_NOALLOC_COUNTER_BYTES are the counters (a fixed region, so the
// partials of one shape never cover the counters of another), the rest is
// the workspace.  Each call zeroes the counter bytes it uses with a fill
// kernel (no memset node, so a HIP graph may capture the call) before the
// decode; the decode leaves them zero as well.
#include <hip/hip_runtime.h>

#include <mutex>

#include "pa_internal.hpp"
#include "pa_mi355x.h"

namespace {

static_assert(PA_NOALLOC_SCRATCH_BYTES % 256 == 0 && PA_NOALLOC_COUNTER_BYTES % 256 == 0,
              "scratch regions keep 256-byte alignment");

static __device__ __align__(256) uint8_t scratch[PA_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's `scratch`, looked up on the first
// call on that device.
pa_status_t scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return PA_ERR_LAUNCH;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr)
      return PA_ERR_LAUNCH;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return PA_OK;
}

}  // namespace

extern "C" pa_status_t pa_paged_decode_attn_noalloc(
    pa_decode_kind_t kind, void* out, const void* q, const void* k_cache, const void* v_cache,
    const float* k_scales, const float* v_scales, const int32_t* block_table,
    const int32_t* context_lens, float scale, int32_t block_size, int32_t num_seqs,
    int32_t num_heads, int32_t head_dim, int32_t num_kv_heads, int32_t num_blocks, int32_t x,
    int32_t max_blocks_per_seq, int32_t max_context_len, int32_t partition_tokens,
    pa_stream_t stream) {
  const bool int8 = kind == PA_DECODE_WARP_I8 || kind == PA_DECODE_SPLITK_I8;
  const pa::DecodeCall c{kind,          out,           q,           k_cache,
                         v_cache,       int8 ? k_scales : nullptr,  int8 ? v_scales : nullptr,
                         block_table,   context_lens,  scale,       block_size,
                         num_seqs,      num_heads,     head_dim,    num_kv_heads,
                         num_blocks,    x,             max_blocks_per_seq,
                         max_context_len, partition_tokens};
  constexpr size_t kWorkspaceBytes = PA_NOALLOC_SCRATCH_BYTES - PA_NOALLOC_COUNTER_BYTES;
  size_t counter_bytes = 0, ws_bytes = 0;
  pa_status_t st = pa::decode_sizes_capped(c, kWorkspaceBytes, &counter_bytes, &ws_bytes);
  if (st != PA_OK || num_seqs == 0) return st;
  if (counter_bytes > PA_NOALLOC_COUNTER_BYTES) return PA_ERR_SCRATCH_LIMIT;
  void* base = nullptr;
  if ((st = scratch_address(&base)) != PA_OK) return st;
  uint8_t* counters = static_cast<uint8_t*>(base);
  uint8_t* workspace = counters + PA_NOALLOC_COUNTER_BYTES;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (pa::launch_fill_zero(counters, counter_bytes, s) != hipSuccess) return PA_ERR_LAUNCH;
  return pa::decode_launch_capped(c, counters, PA_NOALLOC_COUNTER_BYTES, workspace,
                                  kWorkspaceBytes, s);
}
