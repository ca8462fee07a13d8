// Per-token INT8 quantize + paged-cache write (gfx950).
//
// Semantics (bit-exact with the reference's torch code):
//   quantize_per_token, tests/paged_decode_attn.py:106-112
//     amax  = max_d |x_d|                 (in the input type, exact)
//     scale = fp32(t(max(amax, t(1e-8)) / 127))   (t = fp16 or bf16, the input
//                                                  type; the division rounded once)
//     q_d   = int8(clamp(rne(fp32(x_d) / scale), -127, 127)), NaN -> 0
//   placement, tests/paged_decode_attn.py:190-197 and
//   benchmarks/int8_bridge/paged_cache.py:145-154
//     k_cache[blk, h, :, off, :] = q.view(D/8, 8)
//     v_cache[blk, h, :, off]    = q
//     scales[blk, h, off]        = scale,   with slot = blk * block_size + off.
//   per-tensor mode (PagedKVCache "int8_per_tensor",
//   benchmarks/int8_bridge/paged_cache.py:99-106,140-142): the caller passes
//   one fp32 scale for all of K and one for all of V (device pointers), and
//     q_d = int8(clamp(rne(fp32(x_d) / scale), -127, 127)), scale stored per slot.
//
// A job is (16 consecutive input tokens, kv head, K or V).  The grid holds as
// many work-groups as the GPU keeps resident; each wave loops over jobs with a
// grid stride and keeps the inputs of its next two jobs in flight while it
// quantizes the current one.  Lane l owns token l&15 and the dim groups
// (l>>4) + 4j (8 dims each, one 16-B load).  amax is combined over the 4
// lanes of a token with permlane swaps.  Quantizing multiplies by the IEEE
// reciprocal of the scale; an element whose product lies too close to a
// rounding tie (or is not finite) is redone with the IEEE division, so every
// byte equals the reference's.  K rows go out as 8-B stores per (token, dim
// group).  V is transposed through LDS when the 16 tokens fill 16
// consecutive, 16-aligned slots (prefill), so each V row leaves as one 16-B
// store; otherwise it is written byte by byte (decode append, scattered
// slots).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>

#include "pa_device.hpp"
#include "pa_internal.hpp"

namespace pa {

constexpr int kQuantWaves = 4;

typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

// The fast path multiplies by r, the hardware reciprocal of s (within 1 ulp
// of 1/s), instead of dividing.  With |x / s| < 128:
//   |fl(x * r) - x / s| <= 128 * (2^-23 + 2^-24) ~ 2.3e-5   (r, then the product)
//   |fl(x / s) - x / s| <= 2^-18 ~ 3.8e-6                    (the reference's quotient)
// so a product farther than 2.7e-5 from every half-integer rounds to the same
// integer as the IEEE quotient the reference computes.  The guard keeps a margin.
constexpr float kTieGuard = 4.0e-5f;
constexpr float kRoundMagic = 12582912.0f;   // 1.5 * 2^23: y + magic rounds y to an integer (RNE)
// fp16(a / 127) == fp16(fl(a * fl(1/127))) for every fp16 value a and for the
// clamp value 1e-8: a / 127 is never an fp16 rounding midpoint and stays more
// than 2^-18 (relative) away from one, beyond the 2^-23 error of the product
// (checked exhaustively on the CPU).
constexpr float kInv127 = 1.0f / 127.0f;

// The two elements of a 32-bit word of fp16 (BF false) or bf16 (BF true)
// input, widened to fp32 (exactly).
template <bool BF>
__device__ __forceinline__ void widen2(uint32_t w, float& lo, float& hi) {
  if constexpr (BF) {
    lo = __builtin_bit_cast(float, w << 16);
    hi = __builtin_bit_cast(float, w & 0xFFFF0000u);
  } else {
    const half2_t h = __builtin_bit_cast(half2_t, w);
    lo = (float)h.x;
    hi = (float)h.y;
  }
}

// fp32 -> bf16 -> fp32, round to nearest even; a NaN stays a (quiet) NaN.
__device__ __forceinline__ float round_bf16(float f) {
  const uint32_t b = __builtin_bit_cast(uint32_t, f);
  const uint32_t r = (f != f) ? ((b >> 16) | 0x40u) : ((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
  return __builtin_bit_cast(float, r << 16);
}

// Exact path: rne(x / s) with IEEE division, clamped to [-127, 127], NaN -> 0.
__device__ __forceinline__ uint32_t quant_exact_byte(float x, float s) {
  float r = __builtin_rintf(x / s);
  r = (r != r) ? 0.f : fminf(fmaxf(r, -127.f), 127.f);
  return (uint32_t)((int)r) & 0xFFu;
}

// Quantizes the 8 fp16 values of one 16-B group to 8 bytes with the
// reciprocal.  `slow` is set when some element's product lies within
// kTieGuard of a half-integer: the fast byte is then not provably the
// reference's and the caller redoes the group exactly.  With a normal fp16
// scale, |x / s| <= 127 * (1 + 2^-11) < 127.5 for every element of the row, so
// no range check is needed, and the inputs are finite (a NaN or inf in the row
// makes the scale non-normal, which takes the exact path): the largest
// distance to an integer over the group decides with one comparison.
template <bool BF>
__device__ __forceinline__ uint2 quant_group_fast(uint4 xv, float r, bool& slow) {
  const uint32_t wv[4] = {xv.x, xv.y, xv.z, xv.w};
  uint32_t bytes[8];
  float dmax = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float xs[2];
    widen2<BF>(wv[k], xs[0], xs[1]);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float y = xs[e] * r;
      dmax = fmaxf(dmax, __builtin_fabsf(y - __builtin_rintf(y)));
      bytes[2 * k + e] = __builtin_bit_cast(uint32_t, y + kRoundMagic);   // low byte = rne(y) mod 256
    }
  }
  slow = slow || !(dmax < 0.5f - kTieGuard);
  uint2 out;
  out.x = __builtin_amdgcn_perm(__builtin_amdgcn_perm(bytes[3], bytes[2], 0x0c0c0400u),
                                __builtin_amdgcn_perm(bytes[1], bytes[0], 0x0c0c0400u), 0x05040100u);
  out.y = __builtin_amdgcn_perm(__builtin_amdgcn_perm(bytes[7], bytes[6], 0x0c0c0400u),
                                __builtin_amdgcn_perm(bytes[5], bytes[4], 0x0c0c0400u), 0x05040100u);
  return out;
}

// The same with a scale given by the caller (per-tensor mode), where the
// quotient can exceed the int8 range: a product of magnitude >= 127 gives
// +-127 (the IEEE quotient then exceeds 126.5, the reciprocal being a normal
// number, so it rounds to >= 127 and clamps there); the rest lies below 127
// and rounds as above.
template <bool BF>
__device__ __forceinline__ uint2 quant_group_fast_sat(uint4 xv, float r, bool& slow) {
  const uint32_t wv[4] = {xv.x, xv.y, xv.z, xv.w};
  uint32_t bytes[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float xs[2];
    widen2<BF>(wv[k], xs[0], xs[1]);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float y = xs[e] * r;
      const bool sat = __builtin_fabsf(y) >= 127.f;
      slow = slow || (!sat && !(__builtin_fabsf(y - __builtin_rintf(y)) < 0.5f - kTieGuard));
      bytes[2 * k + e] = sat ? (y > 0.f ? 0x7Fu : 0x81u)
                             : __builtin_bit_cast(uint32_t, y + kRoundMagic);
    }
  }
  uint2 out;
  out.x = __builtin_amdgcn_perm(__builtin_amdgcn_perm(bytes[3], bytes[2], 0x0c0c0400u),
                                __builtin_amdgcn_perm(bytes[1], bytes[0], 0x0c0c0400u), 0x05040100u);
  out.y = __builtin_amdgcn_perm(__builtin_amdgcn_perm(bytes[7], bytes[6], 0x0c0c0400u),
                                __builtin_amdgcn_perm(bytes[5], bytes[4], 0x0c0c0400u), 0x05040100u);
  return out;
}

// The exact path for one 16-B group.
template <bool BF>
__device__ __forceinline__ uint2 quant_group_exact(uint4 xv, float s) {
  const uint32_t wv[4] = {xv.x, xv.y, xv.z, xv.w};
  uint32_t b[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float lo, hi;
    widen2<BF>(wv[k], lo, hi);
    b[2 * k] = quant_exact_byte(lo, s);
    b[2 * k + 1] = quant_exact_byte(hi, s);
  }
  return make_uint2(b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24),
                    b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24));
}

// Cache policy of the cache-tile stores (buffer store aux bits): nt, the
// streaming policy; the tiles are not read again by this kernel.  Measured on
// MI355X on the config-3 write (524,288 tokens x 2 heads, inputs read
// non-temporally) with two destination caches in turn, so that no call
// rewrites lines the previous call left in the Infinity Cache: nt 166-167 us,
// sc1 (write-through) 170 us, no hint 178 us.  (Rewriting one destination
// favours sc1 and plain stores, whose lines that cache absorbs: 158 us.)
constexpr int kTileStorePolicy = 2;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, (int)bytes, 0x00020000);
}

// The 16-B input groups of one job for one lane, and the lane's token slot.
// Lane quarter qq owns the dim groups qq + 4j; with head_dim % 32 != 0 the
// last j holds a group only for qq + 4j < D / 8 (the others load the row's
// last group, in bounds, and ignore it).
template <int D>
struct QuantJob {
  static constexpr int DG = D / 8;          // 8-dim groups of a row
  static constexpr int JQ = (DG + 3) / 4;   // 16-B groups per lane
  uint4 x[JQ];
  int64_t slot;
};

// STATIC: every K element is quantized with *k_scale_in and every V element
// with *v_scale_in (the per-tensor mode), instead of its token's own scale.
// BF: the inputs are bf16 (bit patterns) instead of fp16.
// PROBE (the benchmark's write-stream probe, not a write op): the same jobs,
// loads and stores, with the quantization replaced by the high byte of each
// input element and the scale by 1, so that its time is the memory system's
// for exactly this kernel's address stream.
template <int D, bool STATIC, bool BF, bool PROBE = false>
__global__ void __launch_bounds__(kQuantWaves * kWave)
quant_write_kernel(const uint16_t* __restrict__ key, const uint16_t* __restrict__ value, int64_t kts,
                   int64_t khs, int64_t vts, int64_t vhs, const int64_t* __restrict__ slots,
                   int num_tokens, int num_kv_heads, int8_t* __restrict__ kc,
                   int8_t* __restrict__ vc, float* __restrict__ ksc, float* __restrict__ vsc,
                   int num_blocks, int bs, int bs_log2, int njobs, const float* __restrict__ k_scale_in,
                   const float* __restrict__ v_scale_in) {
  static_assert(D % 8 == 0, "head_dim must be a multiple of 8");
  constexpr int JQ = QuantJob<D>::JQ;
  constexpr int DG = QuantJob<D>::DG;
  __shared__ __attribute__((aligned(16))) uint8_t tile[kQuantWaves][D * 16];

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int i = lane & 15, qq = lane >> 4;
  const int64_t pool = (int64_t)num_blocks * bs;
  const int nw = gridDim.x * kQuantWaves;
  int job = blockIdx.x * kQuantWaves + w;
  if (job >= njobs) return;

  // Loads are unconditional (a token past the end reads the last token and is
  // never stored), so the compiler's wait for one job never covers the loads
  // of the jobs issued after it.
  auto load = [&](int jb, QuantJob<D>& J) {
    const int is_v = jb & 1;
    const int th = jb >> 1;
    const int h = th % num_kv_heads;
    const int tok = (th / num_kv_heads) * 16 + i;
    const int tc = tok < num_tokens ? tok : num_tokens - 1;
    J.slot = slots[tc];
    const uint16_t* src = is_v ? value + (int64_t)tc * vts + (int64_t)h * vhs
                               : key + (int64_t)tc * kts + (int64_t)h * khs;
#pragma unroll
    for (int j = 0; j < JQ; ++j) {
      const int o = qq + 4 * j < DG ? qq + 4 * j : DG - 1;
      J.x[j] = load_stream<uint4>(src + o * 8);   // read once
    }
  };

  // Two jobs stay in flight ahead of the one being quantized.  A prefetch
  // past the end reloads the current job, so every load in the loop is
  // unconditional (those lines are cached).  The three job buffers keep their
  // registers and rotate roles over a 3-way unrolled loop: copying a buffer
  // whose loads are still in flight would make the compiler wait for them.
  QuantJob<D> b0, b1, b2;
  load(job, b0);
  load(job + nw < njobs ? job + nw : job, b1);
  auto step = [&](const QuantJob<D>& cur, QuantJob<D>& pf) {
    const int nxt = job + nw;
    const int nxt2 = job + 2 * nw;
    load(nxt2 < njobs ? nxt2 : job, pf);   // past the end: reload this job (cached)
    __builtin_amdgcn_sched_barrier(0);
    const int is_v = job & 1;
    const int th = job >> 1;
    const int h = th % num_kv_heads;
    const int t0 = (th / num_kv_heads) * 16;
    const bool tv = t0 + i < num_tokens;
    const int64_t slot = tv ? cur.slot : -1;
    const bool sok = slot >= 0 && slot < pool;

    float s;
    bool s_normal;
    if constexpr (PROBE) {
      s = 1.f;
      s_normal = true;
    } else if constexpr (STATIC) {
      s = is_v ? v_scale_in[0] : k_scale_in[0];
      // The saturating fast path needs a normal, finite reciprocal.
      const float rr = 1.0f / s;
      s_normal = rr >= 1.17549435e-38f && rr <= 3.40282347e+38f;
    } else {
      // amax over the token's D values as fp16 / bf16 magnitude bits (ordered
      // like the values; a NaN input gives NaN bits above +inf, so the scale
      // becomes NaN as in torch).
      u16x2_t am2 = {0, 0};
#pragma unroll
      for (int j = 0; j < JQ; ++j) {
        if (qq + 4 * j >= DG) continue;   // a padding group (duplicate of the last one)
        const uint32_t wv[4] = {cur.x[j].x, cur.x[j].y, cur.x[j].z, cur.x[j].w};
#pragma unroll
        for (int k = 0; k < 4; ++k)
          am2 = __builtin_elementwise_max(am2, __builtin_bit_cast(u16x2_t, wv[k] & 0x7FFF7FFFu));
      }
      uint32_t am = am2[0] > am2[1] ? am2[0] : am2[1];
      am = rows_umax(am);
      if constexpr (BF) {
        // bf16: amax and clamp_min(bf16(1e-8)) are exact in fp32; the quotient
        // is the IEEE one rounded to bf16 (one rounding, as torch's).
        const float amax = __builtin_bit_cast(float, am << 16);
        const float lo = __builtin_bit_cast(float, 0x322C0000u);   // bf16(1e-8), RNE
        const float a = (amax < lo) ? lo : amax;             // clamp_min, NaN-preserving
        s = round_bf16(a / 127.f);
        // bf16 keeps fp32's exponent range: only NaN / inf leave the fast path
        // (a normal bf16 scale keeps |x / s| <= 127 (1 + 2^-8) < 127.5).
        s_normal = s >= 1.17549435e-38f && s <= 3.38953139e+38f;
      } else {
        const float amax = (float)__builtin_bit_cast(half_t, (uint16_t)am);
        const float a = (amax < 1e-8f) ? 1e-8f : amax;      // clamp_min, NaN-preserving
        s = (float)(half_t)(a * kInv127);                   // == fp16(a / 127), RNE
        // A scale that is not a normal fp16 number (zero, subnormal, NaN, inf)
        // sends the token's elements to the exact path.
        s_normal = s >= 6.103515625e-05f && s <= 65504.0f;
      }
    }
    // Per-token scales are normal fp16 numbers on the fast path, so the
    // hardware reciprocal is finite and within the guard's error budget; a
    // caller's scale (per-tensor mode) takes the IEEE reciprocal.
    const float r = STATIC ? 1.0f / s : __builtin_amdgcn_rcpf(s);

    // block_size is a power of two: shifts instead of a 64-bit division
    const int64_t blk = sok ? (slot >> bs_log2) : 0;
    const int off = sok ? (int)(slot & (bs - 1)) : 0;
    const int64_t bh = blk * num_kv_heads + h;   // (block, kv_head) row

    // 16 tokens filling one aligned 16-slot run of a block (prefill): K rows
    // and V rows then lie in one (block, kv head) tile each, stored through a
    // buffer resource over that tile; V is transposed through LDS and leaves
    // as 16-B rows.
    const int64_t slot0 = (int64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(slot & 0xFFFFFFFF)) |
                          ((int64_t)__builtin_amdgcn_readfirstlane((int)(slot >> 32)) << 32);
    const bool mine = tv && slot == slot0 + i;
    const bool run16 = (t0 + 16 <= num_tokens) && slot0 >= 0 && (slot0 & 15) == 0 &&
                       slot0 + 16 <= pool && __builtin_amdgcn_ballot_w64(!mine) == 0;
    const bool vfast = is_v && run16;
    const int64_t bh0 = (slot0 >> bs_log2) * num_kv_heads + h;   // the run's tile (run16)
    const int off0 = (int)(slot0 & (bs - 1));
    const uint32_t tile_bytes = (uint32_t)(D * bs);
    const auto ktile = tile_rsrc(kc + bh0 * D * bs, tile_bytes);

    // One 16-B group at a time: quantize, fix rare elements exactly, store.
#pragma unroll
    for (int j = 0; j < JQ; ++j) {
      if (qq + 4 * j >= DG) continue;   // padding group: nothing to write
      bool slow = !s_normal;
      uint2 qj;
      if constexpr (PROBE) {
        const uint4 x = cur.x[j];
        qj = make_uint2(__builtin_amdgcn_perm(x.y, x.x, 0x07050301u),
                        __builtin_amdgcn_perm(x.w, x.z, 0x07050301u));
      } else {
        qj = STATIC ? quant_group_fast_sat<BF>(cur.x[j], r, slow)
                    : quant_group_fast<BF>(cur.x[j], r, slow);
        if (__builtin_amdgcn_ballot_w64(slow) != 0) {
          if (slow) qj = quant_group_exact<BF>(cur.x[j], s);   // rare: the reference's division
        }
      }
      const int o = qq + 4 * j;   // dim group: dims 8o .. 8o+7
      if (!is_v) {
        if (run16) {
          typedef uint32_t u2v_t __attribute__((ext_vector_type(2)));
          __builtin_amdgcn_raw_buffer_store_b64((u2v_t){qj.x, qj.y}, ktile, (o * bs + off) * 8, 0,
                                                kTileStorePolicy);
        } else if (sok) {
          *reinterpret_cast<uint2*>(kc + ((bh * (D / 8) + o) * bs + off) * 8) = qj;
        }
      } else if (vfast) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          tile[w][(o * 8 + e) * 16 + i] = (uint8_t)((e < 4 ? qj.x : qj.y) >> (8 * (e & 3)));
      } else if (sok) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          vc[(bh * D + o * 8 + e) * bs + off] = (int8_t)((e < 4 ? qj.x : qj.y) >> (8 * (e & 3)));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (vfast) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const auto vtile = tile_rsrc(vc + bh0 * D * bs, tile_bytes);
#pragma unroll
      for (int rr = lane; rr < D; rr += kWave) {
        typedef uint32_t u4v_t __attribute__((ext_vector_type(4)));
        const u4v_t row = *reinterpret_cast<const u4v_t*>(&tile[w][rr * 16]);
        __builtin_amdgcn_raw_buffer_store_b128(row, vtile, rr * bs + off0, 0, kTileStorePolicy);
      }
      // The tile is rewritten by this wave's next job only after every lane
      // has read its rows.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (sok && qq == 0) (is_v ? vsc : ksc)[bh * bs + off] = s;

    job = nxt;
  };
  // Whole rounds of three steps run without an exit test inside them: an exit
  // in the middle of a round would give the compiler's wait-count analysis a
  // path from a step with loads in flight to the loop head, and a full wait
  // there.  The last 0-2 jobs follow the loop.
  const int total = (njobs - job + nw - 1) / nw;   // jobs of this wave, >= 1
  int k = 0;
  for (; k + 3 <= total; k += 3) {
    step(b0, b2);
    step(b1, b0);
    step(b2, b1);
  }
  if (k < total) step(b0, b2);
  if (k + 1 < total) step(b1, b0);
}

// Work-groups the GPU holds at once for this kernel: the grid-stride loop is
// sized to them so that no group starts after the others have finished.
template <int D, bool STATIC, bool BF, bool PROBE = false>
int resident_groups() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256 * 4;
  if (cache[dev] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, quant_write_kernel<D, STATIC, BF, PROBE>,
                                                     kQuantWaves * kWave, 0) != hipSuccess ||
        per_cu <= 0)
      per_cu = 4;
    cache[dev] = cus * per_cu;
  }
  return cache[dev];
}

}  // namespace pa
