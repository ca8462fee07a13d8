// FP16 paged-cache write (gfx950): no quantization, only the placement.
//
// Semantics of PagedKVCache.prefill / decode_append for the "fp16" variant
// (benchmarks/int8_bridge/paged_cache.py:116-130,148-150) and of the fp16
// builder (tests/paged_decode_attn.py:85-99):
//   k_cache[blk, h, :, off, :] = k[t, h].view(D/8, 8)
//   v_cache[blk, h, :, off]    = v[t, h]
// with slot_mapping[t] = blk * block_size + off (vLLM's reshape_and_cache
// convention); a slot outside the pool skips the token.
//
// A job is (16 consecutive input tokens, kv head, K or V), one wave each,
// grid-stride over the jobs.  Lane l owns token l & 15 and the dim groups
// (l >> 4) + 4j (8 dims, one 16-B load).  K leaves as one 16-B store per
// (token, dim group).  V is transposed through LDS when the 16 tokens fill 16
// consecutive slots starting at a multiple of 16 inside one block (prefill),
// so each V row of 16 tokens leaves as two 16-B stores; otherwise each element
// is stored on its own (decode append, scattered slots).
#include <algorithm>

#include "pa_device.hpp"
#include "pa_internal.hpp"

namespace pa {

constexpr int kWriteWaves = 4;

template <int D>
__global__ void __launch_bounds__(kWriteWaves * kWave)
cache_write_f16_kernel(const half_t* __restrict__ key, const half_t* __restrict__ value,
                       int64_t kts, int64_t khs, int64_t vts, int64_t vhs,
                       const int64_t* __restrict__ slots, int num_tokens, int num_kv_heads,
                       half_t* __restrict__ kc, half_t* __restrict__ vc, int num_blocks, int bs,
                       int bs_log2, int njobs) {
  static_assert(D % 8 == 0, "head_dim must be a multiple of 8");
  constexpr int DG = D / 8;            // 8-dim groups of a row
  constexpr int JQ = (DG + 3) / 4;     // 16-B groups per lane: dim groups (l >> 4) + 4j
  // (with head_dim % 32 != 0 the last j is a group only for lanes with
  // (l >> 4) + 4j < DG; the others load the row's last group, in bounds, and
  // store nothing)
  __shared__ __attribute__((aligned(16))) half_t tile[kWriteWaves][D * 16];

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int i = lane & 15, qq = lane >> 4;
  const int64_t pool = (int64_t)num_blocks * bs;
  const int nw = gridDim.x * kWriteWaves;

  for (int job = blockIdx.x * kWriteWaves + w; job < njobs; job += nw) {
    const int is_v = job & 1;
    const int th = job >> 1;
    const int h = th % num_kv_heads;
    const int t0 = (th / num_kv_heads) * 16;
    const int tok = t0 + i;
    const bool tv = tok < num_tokens;
    const int tc = tv ? tok : num_tokens - 1;
    const half_t* src = is_v ? value + (int64_t)tc * vts + (int64_t)h * vhs
                             : key + (int64_t)tc * kts + (int64_t)h * khs;
    uint4 x[JQ];
#pragma unroll
    for (int j = 0; j < JQ; ++j)
      x[j] = *reinterpret_cast<const uint4*>(src + (qq + 4 * j < DG ? qq + 4 * j : DG - 1) * 8);
    const int64_t slot = tv ? slots[tc] : -1;
    const bool sok = slot >= 0 && slot < pool;
    // block_size is a power of two: shifts instead of a 64-bit division
    const int64_t blk = sok ? (slot >> bs_log2) : 0;
    const int off = sok ? (int)(slot & (bs - 1)) : 0;
    const int64_t bh = blk * num_kv_heads + h;

    if (!is_v) {
#pragma unroll
      for (int j = 0; j < JQ; ++j) {
        const int o = qq + 4 * j;
        if (sok && o < DG) *reinterpret_cast<uint4*>(kc + ((bh * DG + o) * bs + off) * 8) = x[j];
      }
      continue;
    }
    // V: 16 tokens in one aligned 16-slot run of a block go through LDS.
    const int64_t slot0 = (int64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(slot & 0xFFFFFFFF)) |
                          ((int64_t)__builtin_amdgcn_readfirstlane((int)(slot >> 32)) << 32);
    const bool mine = tv && slot == slot0 + i;
    const bool vfast = (bs % 16 == 0) && (t0 + 16 <= num_tokens) && slot0 >= 0 &&
                       (slot0 & 15) == 0 && slot0 + 16 <= pool &&
                       __builtin_amdgcn_ballot_w64(!mine) == 0;
    if (vfast) {
#pragma unroll
      for (int j = 0; j < JQ; ++j) {
        const int o = qq + 4 * j;
        if (o >= DG) continue;
        const uint32_t wv[4] = {x[j].x, x[j].y, x[j].z, x[j].w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          tile[w][(o * 8 + e) * 16 + i] =
              __builtin_bit_cast(half_t, (uint16_t)(wv[e >> 1] >> (16 * (e & 1))));
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int64_t blk0 = slot0 >> bs_log2;
      const int off0 = (int)(slot0 & (bs - 1));
      const int64_t bh0 = blk0 * num_kv_heads + h;
      // Row rr of the tile (16 tokens of dim rr, 32 B) leaves as two 16-B halves.
#pragma unroll
      for (int c = lane; c < 2 * D; c += kWave) {
        const int rr = c >> 1, hf = c & 1;
        const uint4 row = *reinterpret_cast<const uint4*>(&tile[w][rr * 16 + 8 * hf]);
        *reinterpret_cast<uint4*>(vc + (bh0 * D + rr) * bs + off0 + 8 * hf) = row;
      }
      // The tile is rewritten by this wave's next job only after every lane
      // has read its rows.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    } else if (sok) {
#pragma unroll
      for (int j = 0; j < JQ; ++j) {
        const int o = qq + 4 * j;
        if (o >= DG) continue;
        const uint32_t wv[4] = {x[j].x, x[j].y, x[j].z, x[j].w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          vc[(bh * D + o * 8 + e) * bs + off] =
              __builtin_bit_cast(half_t, (uint16_t)(wv[e >> 1] >> (16 * (e & 1))));
      }
    }
  }
}

template <int D>
static hipError_t launch_write_d(const CacheWriteLaunch& l) {
  const int tiles = (l.num_tokens + 15) / 16;
  const int njobs = tiles * l.num_kv_heads * 2;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  const int want = (njobs + kWriteWaves - 1) / kWriteWaves;
  const int grid = std::min(want, cus * 8);
  cache_write_f16_kernel<D><<<grid, kWriteWaves * kWave, 0, l.stream>>>(
      static_cast<const half_t*>(l.key), static_cast<const half_t*>(l.value), l.key_token_stride,
      l.key_head_stride, l.value_token_stride, l.value_head_stride, l.slot_mapping, l.num_tokens,
      l.num_kv_heads, static_cast<half_t*>(l.k_cache), static_cast<half_t*>(l.v_cache),
      l.num_blocks, l.block_size, __builtin_ctz((unsigned)l.block_size), njobs);
  return hipGetLastError();
}

hipError_t launch_cache_write_f16(const CacheWriteLaunch& l) {
  switch (l.head_dim) {
#define PA_CASE(D) \
  case D: return launch_write_d<D>(l);
    PA_FOR_EACH_HEAD_DIM(PA_CASE)
#undef PA_CASE
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pa
