// Device helpers for the gfx950 paged-attention kernels.
//
// Wave64 cross-lane reductions use DPP inside a 16-lane row and the gfx950
// permlane swaps across rows, so every lane ends with the same value and no
// LDS round trip is needed.  Dot products over fp16 pairs use v_dot2 (two
// fp16 products accumulated into fp32), which replaces the reference's
// per-element fp32 FMAs (kernels/paged_attention_common.cuh:98-138).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pa {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

__device__ __forceinline__ uint32_t fbits(float v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ float bitsf(uint32_t v) { return __builtin_bit_cast(float, v); }

// fp32 += a.lo*b.lo + a.hi*b.hi with a, b packed fp16 pairs.
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b), c,
                                false);
}

// Row-local DPP move (all rows and banks enabled, every source lane valid).
// No lane keeps the destination's old value, so none is supplied (an
// explicit one, update_dpp's first operand, costs a move per call).  Call it
// with every lane active: a lane whose source lane is inactive would read an
// undefined value.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return bitsf((uint32_t)__builtin_amdgcn_mov_dpp((int)fbits(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}

// DPP controls used below.
constexpr int kQuadXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;  // lane i <- 7-i within each 8 lanes
constexpr int kRowMirror = 0x140;      // lane i <- 15-i within each 16 lanes

// Combine across rows: after the call, op(v[row 2k], v[row 2k+1]) in rows 2k and 2k+1.
template <class Op>
__device__ __forceinline__ float cross_row16(float v, Op op) {
  auto r = __builtin_amdgcn_permlane16_swap(fbits(v), fbits(v), false, false);
  return op(bitsf(r[0]), bitsf(r[1]));
}
// Combine the two 32-lane halves.
template <class Op>
__device__ __forceinline__ float cross_half32(float v, Op op) {
  auto r = __builtin_amdgcn_permlane32_swap(fbits(v), fbits(v), false, false);
  return op(bitsf(r[0]), bitsf(r[1]));
}

struct OpMax {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct OpSum {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};

// Full-wave reduction; every lane receives the same bits (each combining
// step is commutative, so mirrored lanes compute identical values).
// Must be called with all 64 lanes active.
template <class Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
  v = op(v, dpp_mov<kQuadXor1>(v));
  v = op(v, dpp_mov<kQuadXor2>(v));
  v = op(v, dpp_mov<kRowHalfMirror>(v));
  v = op(v, dpp_mov<kRowMirror>(v));
  v = cross_row16(v, op);
  v = cross_half32(v, op);
  return v;
}
__device__ __forceinline__ float wave_max(float v) { return wave_reduce(v, OpMax()); }
__device__ __forceinline__ float wave_sum(float v) { return wave_reduce(v, OpSum()); }

// Sum of lane pairs (l, l^1): both lanes get the sum.
__device__ __forceinline__ float pair_sum(float v) { return v + dpp_mov<kQuadXor1>(v); }

// Unsigned max over lanes that share l & 15 (the four 16-lane rows).
__device__ __forceinline__ uint32_t rows_umax(uint32_t v) {
  auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = r[0] > r[1] ? r[0] : r[1];
  auto s = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return s[0] > s[1] ? s[0] : s[1];
}

// int8x4 -> two packed fp16 pairs holding 1152 + value, exactly.
// Flipping the sign bit maps a signed byte b to the unsigned byte b + 128;
// placing it under the fp16 exponent byte 0x64 gives the fp16 number
// 1024 + (b + 128).  Bytes 0,1 go to the first pair, bytes 2,3 to the second.
__device__ __forceinline__ void i8x4_to_biased_h2(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const uint32_t u = w ^ 0x80808080u;
  lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
  hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
}

// A load of data that is read once (cache tiles, inputs of the write
// kernels): the non-temporal hint keeps it from being retained in the caches.
// On MI355X it raised the decode kernels' streaming rate from about 5.9 to
// 6.4 TB/s (FP16, config 3 and config 4 shapes).
template <typename T>
__device__ __forceinline__ T load_stream(const void* p) {
  static_assert(sizeof(T) == 16 || sizeof(T) == 8, "16- or 8-byte loads");
  typedef uint32_t v4_t __attribute__((ext_vector_type(4)));
  typedef uint32_t v2_t __attribute__((ext_vector_type(2)));
  if constexpr (sizeof(T) == 16) {
    return __builtin_bit_cast(T, __builtin_nontemporal_load(reinterpret_cast<const v4_t*>(p)));
  } else {
    return __builtin_bit_cast(T, __builtin_nontemporal_load(reinterpret_cast<const v2_t*>(p)));
  }
}

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  half2_t h = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(uint32_t, h);
}

}  // namespace pa
