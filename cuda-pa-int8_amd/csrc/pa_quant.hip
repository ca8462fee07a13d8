// Per-token INT8 quantize + paged-cache write (gfx950).
//
// Semantics (bit-exact with the reference's torch code):
//   quantize_per_token, tests/paged_decode_attn.py:106-112
//     amax  = max_d |x_d|                 (in fp16, exact)
//     scale = fp32(fp16(max(amax, 1e-8) / 127))   (fp16 division rounded once)
//     q_d   = int8(clamp(rne(fp32(x_d) / scale), -127, 127)), NaN -> 0
//   placement, tests/paged_decode_attn.py:190-197 and
//   benchmarks/int8_bridge/paged_cache.py:145-154
//     k_cache[blk, h, :, off, :] = q.view(D/8, 8)
//     v_cache[blk, h, :, off]    = q
//     scales[blk, h, off]        = scale,   with slot = blk * block_size + off.
//
// One wave handles one job = (16 consecutive input tokens, kv head, K or V).
// Lane l owns token l&15 and the dim groups (l>>4) + 4j (8 dims each, one
// 16-B load).  amax is combined over the 4 lanes of a token with permlane
// swaps.  K rows go out as 8-B stores per (token, dim group).  V is
// transposed through LDS when the 16 tokens fill 16 consecutive, 16-aligned
// slots (prefill), so each V row leaves as one 16-B store; otherwise it is
// written byte by byte (decode append, scattered slots).
#include <math.h>

#include "pa_device.hpp"
#include "pa_internal.hpp"

namespace pa {

constexpr int kQuantWaves = 4;

__device__ __forceinline__ uint32_t quant_pair_bytes(uint32_t h2bits, float s, int& b0, int& b1) {
  const half2_t h = __builtin_bit_cast(half2_t, h2bits);
  float r0 = __builtin_rintf((float)h.x / s);
  float r1 = __builtin_rintf((float)h.y / s);
  r0 = (r0 != r0) ? 0.f : fminf(fmaxf(r0, -127.f), 127.f);
  r1 = (r1 != r1) ? 0.f : fminf(fmaxf(r1, -127.f), 127.f);
  b0 = (int)r0;
  b1 = (int)r1;
  return ((uint32_t)(b0 & 0xFF)) | ((uint32_t)(b1 & 0xFF) << 8);
}

template <int D>
__global__ void __launch_bounds__(kQuantWaves * kWave)
quant_write_kernel(const half_t* __restrict__ key, const half_t* __restrict__ value, int64_t kts,
                   int64_t khs, int64_t vts, int64_t vhs, const int64_t* __restrict__ slots,
                   int num_tokens, int num_kv_heads, int8_t* __restrict__ kc,
                   int8_t* __restrict__ vc, float* __restrict__ ksc, float* __restrict__ vsc,
                   int num_blocks, int bs, int njobs) {
  constexpr int JQ = D / 32;   // 16-B groups per lane
  __shared__ __attribute__((aligned(16))) uint8_t tile[kQuantWaves][D * 16];

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int job = blockIdx.x * kQuantWaves + w;
  if (job >= njobs) return;
  const int is_v = job & 1;
  const int th = job >> 1;
  const int h = th % num_kv_heads;
  const int t0 = (th / num_kv_heads) * 16;
  const int i = lane & 15, qq = lane >> 4;
  const int tok = t0 + i;
  const bool tv = tok < num_tokens;
  const int64_t pool = (int64_t)num_blocks * bs;
  const int64_t slot = tv ? slots[tok] : -1;
  const bool sok = slot >= 0 && slot < pool;

  const half_t* src = is_v ? value + (int64_t)(tv ? tok : 0) * vts + (int64_t)h * vhs
                           : key + (int64_t)(tv ? tok : 0) * kts + (int64_t)h * khs;
  uint4 x[JQ];
#pragma unroll
  for (int j = 0; j < JQ; ++j) {
    x[j] = tv ? *reinterpret_cast<const uint4*>(src + (qq + 4 * j) * 8) : make_uint4(0, 0, 0, 0);
  }

  // amax over the token's D values as fp16 magnitude bits (ordered like the values;
  // a NaN input gives NaN bits above +inf, so the scale becomes NaN as in torch).
  uint32_t am = 0;
#pragma unroll
  for (int j = 0; j < JQ; ++j) {
    const uint32_t wv[4] = {x[j].x, x[j].y, x[j].z, x[j].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t lo = wv[k] & 0x7FFFu, hi = (wv[k] >> 16) & 0x7FFFu;
      am = am > lo ? am : lo;
      am = am > hi ? am : hi;
    }
  }
  am = rows_umax(am);
  const float amax = (float)__builtin_bit_cast(half_t, (uint16_t)am);
  const float a = (amax < 1e-8f) ? 1e-8f : amax;      // clamp_min, NaN-preserving
  const float s = (float)(half_t)(a / 127.0f);        // fp16 division, RNE

  // quantize: 8 bytes per dim group
  uint2 qv[JQ];
  int qb[JQ][8];
#pragma unroll
  for (int j = 0; j < JQ; ++j) {
    const uint32_t wv[4] = {x[j].x, x[j].y, x[j].z, x[j].w};
    uint32_t pk[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) pk[k] = quant_pair_bytes(wv[k], s, qb[j][2 * k], qb[j][2 * k + 1]);
    qv[j].x = pk[0] | (pk[1] << 16);
    qv[j].y = pk[2] | (pk[3] << 16);
  }

  const int64_t blk = sok ? slot / bs : 0;
  const int off = sok ? (int)(slot - blk * bs) : 0;
  const int64_t bh = blk * num_kv_heads + h;   // (block, kv_head) row

  if (!is_v) {
    if (sok) {
#pragma unroll
      for (int j = 0; j < JQ; ++j) {
        const int o = qq + 4 * j;
        *reinterpret_cast<uint2*>(kc + ((bh * (D / 8) + o) * bs + off) * 8) = qv[j];
      }
      if (qq == 0) ksc[bh * bs + off] = s;
    }
    return;
  }

  // V: 16 tokens filling one aligned 16-slot run of a block -> LDS transpose.
  const int64_t slot0 = __builtin_amdgcn_readfirstlane((int)(slot & 0xFFFFFFFF)) |
                        ((int64_t)__builtin_amdgcn_readfirstlane((int)(slot >> 32)) << 32);
  const bool mine = tv && slot == slot0 + i;
  const bool fast = (t0 + 16 <= num_tokens) && slot0 >= 0 && (slot0 & 15) == 0 &&
                    slot0 + 16 <= pool && __builtin_amdgcn_ballot_w64(!mine) == 0;
  if (fast) {
#pragma unroll
    for (int j = 0; j < JQ; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) tile[w][((qq + 4 * j) * 8 + e) * 16 + i] = (uint8_t)qb[j][e];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int64_t blk0 = slot0 / bs;
    const int off0 = (int)(slot0 - blk0 * bs);
    const int64_t bh0 = blk0 * num_kv_heads + h;
#pragma unroll
    for (int r = lane; r < D; r += kWave) {
      const uint4 row = *reinterpret_cast<const uint4*>(&tile[w][r * 16]);
      *reinterpret_cast<uint4*>(vc + (bh0 * D + r) * bs + off0) = row;
    }
  } else if (sok) {
#pragma unroll
    for (int j = 0; j < JQ; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) vc[(bh * D + (qq + 4 * j) * 8 + e) * bs + off] = (int8_t)qb[j][e];
  }
  if (sok && qq == 0) vsc[bh * bs + off] = s;
}

template <int D>
static hipError_t launch_quant_d(const QuantLaunch& l) {
  const int tiles = (l.num_tokens + 15) / 16;
  const int njobs = tiles * l.num_kv_heads * 2;
  const int grid = (njobs + kQuantWaves - 1) / kQuantWaves;
  quant_write_kernel<D><<<grid, kQuantWaves * kWave, 0, l.stream>>>(
      static_cast<const half_t*>(l.key), static_cast<const half_t*>(l.value), l.key_token_stride,
      l.key_head_stride, l.value_token_stride, l.value_head_stride, l.slot_mapping, l.num_tokens,
      l.num_kv_heads, static_cast<int8_t*>(l.k_cache), static_cast<int8_t*>(l.v_cache),
      l.k_scales, l.v_scales, l.num_blocks, l.block_size, njobs);
  return hipGetLastError();
}

hipError_t launch_quant_write_i8(const QuantLaunch& l) {
  switch (l.head_dim) {
    case 64: return launch_quant_d<64>(l);
    case 128: return launch_quant_d<128>(l);
    case 256: return launch_quant_d<256>(l);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pa
